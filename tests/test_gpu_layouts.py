"""KV layouts beyond the reference's contiguous [B, Hkv, N, D]: the token-major
[B, N, Hkv, D] layout FlashInfer uses (flashinfer_looptimed.py:63-65) and paged
caches (NHD pages, HND pages as a strided view), for fp16, int8 and int4, with
ragged sequence lengths; and bf16 caches (no counterpart in the reference) in
every layout. Checked against the float64 oracle at max-abs 2e-3;
the token-major layout also bit for bit against the contiguous entry point,
since only addresses differ."""

import numpy as np
import pytest
import torch

import oracle
import fqkv_decode as fq

pytestmark = pytest.mark.gpu

TOL = 2e-3


def draw(g, *shape):
    return torch.randn(*shape, generator=g, dtype=torch.float32)


def maxerr(out, ref):
    return float(np.abs(out.float().cpu().numpy().astype(np.float64) - ref).max())


def quantize(fmt, X):
    if fmt == "int8":
        q, s = fq.quantize_int8_per_token(X.cuda())
        return q, s, oracle.dequant_int8(q.cpu().numpy(), s.cpu().numpy())
    q, s = fq.quantize_int4_per_token(X.cuda())
    return q, s, oracle.dequant_int4(q.cpu().numpy(), s.cpu().numpy())


@pytest.mark.parametrize("B,Hq,Hkv,N,D", [(2, 32, 8, 1000, 128), (1, 32, 8, 16384, 64), (3, 8, 8, 17, 128)])
def test_nhd_fp16_equals_contiguous(B, Hq, Hkv, N, D):
    g = torch.Generator().manual_seed(50)
    q, K, V = draw(g, B, Hq, D).half(), draw(g, B, Hkv, N, D).half(), draw(g, B, Hkv, N, D).half()
    a = fq.decode_attn_gqa(q.cuda(), K.cuda(), V.cuda(), 8)
    b = fq.decode_attn_gqa_nhd(q.cuda(), K.permute(0, 2, 1, 3).contiguous().cuda(),
                               V.permute(0, 2, 1, 3).contiguous().cuda(), 8)
    assert torch.equal(a, b)
    assert maxerr(b, oracle.gqa_attention(q.numpy(), K.numpy(), V.numpy())) <= TOL


@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_nhd_quantized(fmt):
    g = torch.Generator().manual_seed(51)
    B, Hq, Hkv, N, D = 2, 16, 4, 777, 128
    q = draw(g, B, Hq, D).half()
    Kq, Ks, Kf = quantize(fmt, draw(g, B, N, Hkv, D))
    Vq, Vs, Vf = quantize(fmt, draw(g, B, N, Hkv, D))
    out = fq.decode_attn_gqa_nhd(q.cuda(), Kq, Vq, 8, Ks, Vs)
    ref = oracle.gqa_attention(q.numpy(), Kf.transpose(0, 2, 1, 3), Vf.transpose(0, 2, 1, 3))
    assert maxerr(out, ref) <= TOL


@pytest.mark.parametrize("B", [8, 2])
def test_nhd_int4_head_grouping_equals_contiguous(B):
    """Token-major int4 rows are 64 bytes, so KV heads h and h ^ 1 share each 128-byte line
    and the launcher renumbers the work items to put such heads on one XCD. At B 8 (64 rows,
    4 splits, groups interleaved with their splits) and B 2 (16 rows, 16 splits, split-major
    order) the renumbering is not the identity; it changes only which workgroup computes what,
    so the output must equal the contiguous layout's bit for bit, and the oracle."""
    g = torch.Generator().manual_seed(52 + B)
    Hq, Hkv, N, D = 32, 8, 2000, 128
    q = draw(g, B, Hq, D).half()
    Kq, Ks, Kf = quantize("int4", draw(g, B, N, Hkv, D))
    Vq, Vs, Vf = quantize("int4", draw(g, B, N, Hkv, D))
    out = fq.decode_attn_gqa_nhd(q.cuda(), Kq, Vq, 8, Ks, Vs)
    hm = lambda t: t.transpose(1, 2).contiguous()  # [B, N, Hkv, ...] -> [B, Hkv, N, ...]
    ref_c = fq.decode_attn_gqa_int4(q.cuda(), hm(Kq), hm(Vq), hm(Ks), hm(Vs), 8)
    assert torch.equal(out, ref_c)
    ref = oracle.gqa_attention(q.numpy(), Kf.transpose(0, 2, 1, 3), Vf.transpose(0, 2, 1, 3))
    assert maxerr(out, ref) <= TOL


def paged_cache(g, lens, Hkv, D, page, fmt, hnd=False, spare=3):
    """Scatter per-sequence K/V into pages at shuffled page ids; returns the
    device pages (NHD views), page table, lengths and the float64 per-sequence caches."""
    npages = [(L + page - 1) // page for L in lens]
    P = sum(npages) + spare
    ids = torch.randperm(P, generator=g)
    max_pages = max(npages)
    table = torch.full((len(lens), max_pages), -1, dtype=torch.int32)
    k = 0
    for b, n in enumerate(npages):
        table[b, :n] = ids[k:k + n].to(torch.int32)
        k += n
    X = draw(g, 2, P, page, Hkv, D)  # raw K and V pages, NHD
    if fmt in ("fp16", "bf16"):
        dt = torch.float16 if fmt == "fp16" else torch.bfloat16
        Kp, Vp = X[0].to(dt), X[1].to(dt)
        Kf, Vf = Kp.float().numpy(), Vp.float().numpy()
        Ks = Vs = None
    else:
        Kp, Ks, Kf = quantize(fmt, X[0])
        Vp, Vs, Vf = quantize(fmt, X[1])
        Kp, Vp, Ks, Vs = Kp.cpu(), Vp.cpu(), Ks.cpu(), Vs.cpu()
    seqs = []
    for b, L in enumerate(lens):
        t = np.arange(L)
        pid = table[b, t // page].numpy()
        pos = t % page
        seqs.append((Kf[pid, pos].transpose(1, 0, 2), Vf[pid, pos].transpose(1, 0, 2)))  # [Hkv, L, D]
    if hnd:  # store pages head-major, hand the kernel the NHD view
        Kp = Kp.permute(0, 2, 1, 3).contiguous().cuda().permute(0, 2, 1, 3)
        Vp = Vp.permute(0, 2, 1, 3).contiguous().cuda().permute(0, 2, 1, 3)
        if Ks is not None:
            Ks = Ks.permute(0, 2, 1).contiguous().cuda().permute(0, 2, 1)
            Vs = Vs.permute(0, 2, 1).contiguous().cuda().permute(0, 2, 1)
    else:
        Kp, Vp = Kp.cuda(), Vp.cuda()
        if Ks is not None:
            Ks, Vs = Ks.cuda(), Vs.cuda()
    return Kp, Vp, Ks, Vs, table.cuda(), torch.tensor(lens, dtype=torch.int32).cuda(), seqs


@pytest.mark.parametrize("fmt", ["fp16", "bf16", "int8", "int4"])
@pytest.mark.parametrize("page,hnd", [(16, False), (64, True), (256, False)])
def test_paged(fmt, page, hnd):
    g = torch.Generator().manual_seed(52)
    lens = [1, 15, 16, 17, 300, 3000]
    Hq, Hkv, D = 32, 8, 128
    Kp, Vp, Ks, Vs, table, sl, seqs = paged_cache(g, lens, Hkv, D, page, fmt, hnd)
    q = draw(g, len(lens), Hq, D).half()
    out = fq.decode_attn_gqa_paged(q.cuda(), Kp, Vp, table, sl, max(lens), 8, Ks, Vs)
    for b, (Kb, Vb) in enumerate(seqs):
        ref = oracle.gqa_attention(q.numpy()[b:b + 1], Kb[None], Vb[None])[0]
        assert maxerr(out[b], ref) <= TOL, (b, lens[b])


@pytest.mark.parametrize("fmt", ["int8", "int4"])
@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (40, 5)])
def test_paged_quant_group_widths(fmt, Hq, Hkv):
    """Paged int8/int4 caches at one query head per KV head (four tiles share the
    score columns) and at G = 5 (head group of 8, two tiles share them): the
    per-tile scale descriptors are picked per lane."""
    g = torch.Generator().manual_seed(54)
    lens = [5, 16, 33, 700]
    D = 128
    Kp, Vp, Ks, Vs, table, sl, seqs = paged_cache(g, lens, Hkv, D, 32, fmt)
    q = draw(g, len(lens), Hq, D).half()
    out = fq.decode_attn_gqa_paged(q.cuda(), Kp, Vp, table, sl, max(lens), 4, Ks, Vs)
    for b, (Kb, Vb) in enumerate(seqs):
        ref = oracle.gqa_attention(q.numpy()[b:b + 1], Kb[None], Vb[None])[0]
        assert maxerr(out[b], ref) <= TOL, (b, lens[b])


def test_paged_d64_long_and_split():
    """One long sequence (internal split over many pages) and D = 64."""
    g = torch.Generator().manual_seed(53)
    lens = [20000]
    Kp, Vp, Ks, Vs, table, sl, seqs = paged_cache(g, lens, 8, 64, 32, "fp16")
    q = draw(g, 1, 32, 64).half()
    out = fq.decode_attn_gqa_paged(q.cuda(), Kp, Vp, table, sl, 20000, 4)
    ref = oracle.gqa_attention(q.numpy(), seqs[0][0][None], seqs[0][1][None])
    assert maxerr(out, ref) <= TOL


def test_layout_entry_points_reject_bad_input():
    q = torch.zeros(1, 8, 128, dtype=torch.float16, device="cuda")
    Kp = torch.zeros(4, 24, 2, 128, dtype=torch.float16, device="cuda")
    table = torch.zeros(1, 4, dtype=torch.int32, device="cuda")
    sl = torch.ones(1, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="page_size"):
        fq.decode_attn_gqa_paged(q, Kp, Kp, table, sl, 16, 8)
    with pytest.raises(RuntimeError, match="^shape"):
        fq.decode_attn_gqa_paged(q, Kp[:, :16], Kp[:, :16], table.long(), sl, 16, 8)
    Ki = torch.zeros(1, 16, 2, 128, dtype=torch.int8, device="cuda")
    with pytest.raises(RuntimeError, match="^int8"):
        fq.decode_attn_gqa_nhd(q, Ki, Ki, 8)


@pytest.mark.parametrize("fmt", ["fp16", "int8", "int4"])
@pytest.mark.parametrize("D", [64, 128])
def test_strided_view_of_a_larger_cache_equals_contiguous(fmt, D):
    """decode_attn_gqa_strided on the filled part of a preallocated [B, Hkv, capacity, D]
    cache gives the bytes of the contiguous entry point on a copy of that part."""
    g = torch.Generator().manual_seed(52)
    B, Hq, Hkv, N, cap = 2, 16, 4, 1234, 2048
    q = draw(g, B, Hq, D).half().cuda()
    if fmt == "fp16":
        Kc, Vc = draw(g, B, Hkv, cap, D).half().cuda(), draw(g, B, Hkv, cap, D).half().cuda()
        K, V = Kc[:, :, :N], Vc[:, :, :N]
        a = fq.decode_attn_gqa(q, K.contiguous(), V.contiguous(), 8)
        b = fq.decode_attn_gqa_strided(q, K, V, 8)
    else:
        Kc, Ksc, _ = quantize(fmt, draw(g, B, Hkv, cap, D))
        Vc, Vsc, _ = quantize(fmt, draw(g, B, Hkv, cap, D))
        K, V, Ks, Vs = Kc[:, :, :N], Vc[:, :, :N], Ksc[:, :, :N], Vsc[:, :, :N]
        f = fq.decode_attn_gqa_int8 if fmt == "int8" else fq.decode_attn_gqa_int4
        a = f(q, K.contiguous(), V.contiguous(), Ks.contiguous(), Vs.contiguous(), 8)
        b = fq.decode_attn_gqa_strided(q, K, V, 8, Ks, Vs)
    assert torch.equal(a, b)


def test_strided_token_major_view_equals_nhd():
    g = torch.Generator().manual_seed(53)
    B, Hq, Hkv, N, D = 2, 32, 8, 700, 128
    q = draw(g, B, Hq, D).half().cuda()
    K, V = draw(g, B, N, Hkv, D).half().cuda(), draw(g, B, N, Hkv, D).half().cuda()
    a = fq.decode_attn_gqa_nhd(q, K, V, 8)
    b = fq.decode_attn_gqa_strided(q, K.transpose(1, 2), V.transpose(1, 2), 8)
    assert torch.equal(a, b)


def test_strided_rejects_bad_views():
    q = torch.zeros(1, 4, 64, dtype=torch.float16, device="cuda")
    K = torch.zeros(1, 2, 40, 64, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="^contig"):
        fq.decode_attn_gqa_strided(q, K[..., ::2].expand(1, 2, 40, 32), K[..., ::2].expand(1, 2, 40, 32), 8)
    with pytest.raises(RuntimeError, match="^shape"):
        fq.decode_attn_gqa_strided(q, K, K[:, :, :30], 8)
    with pytest.raises(RuntimeError, match="strides"):  # token stride not a multiple of 16 bytes
        Kb = torch.zeros(1, 2, 40, 68, dtype=torch.float16, device="cuda")[..., :64]
        fq.decode_attn_gqa_strided(q, Kb, Kb, 8)


@pytest.mark.parametrize("fmt", ["fp16", "bf16", "int8", "int4"])
@pytest.mark.parametrize("lens", [[0, 5, 0, 300], [0, 20000, 0]])
def test_paged_empty_sequences_give_zeros(fmt, lens):
    """A batch slot with seq_len 0 (continuous batching) has no keys: its output
    is defined as zeros, in the single-pass and in the split path alike, and
    its neighbours are unaffected."""
    g = torch.Generator().manual_seed(56)
    Hq, Hkv, D = 32, 8, 128
    Kp, Vp, Ks, Vs, table, sl, seqs = paged_cache(g, lens, Hkv, D, 32, fmt)
    q = draw(g, len(lens), Hq, D).half()
    out = fq.decode_attn_gqa_paged(q.cuda(), Kp, Vp, table, sl, max(lens), 8, Ks, Vs)
    for b, (Kb, Vb) in enumerate(seqs):
        if lens[b] == 0:
            assert torch.equal(out[b].cpu(), torch.zeros(Hq, D, dtype=torch.float16)), b
        else:
            ref = oracle.gqa_attention(q.numpy()[b:b + 1], Kb[None], Vb[None])[0]
            assert maxerr(out[b], ref) <= TOL, (b, lens[b])


# ------------------------------------------------------------------ bf16 ----

@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("G", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("N", [1, 100, 3000, 20000])
def test_bf16_strided_against_the_oracle(N, G, D):
    """bf16 K and V through decode_attn_gqa_strided (a view of a larger cache) at every head-group
    width, from one token to the internally split 20000: the matrix-core products take the query
    and the weights as bf16 pairs, so the output is as close to the float64 oracle on the bf16
    values as the fp16 path's is."""
    g = torch.Generator().manual_seed(57 + N + G + D)
    B, Hkv = 2, 2
    Hq = G * Hkv
    q = draw(g, B, Hq, D).half()
    Kc, Vc = draw(g, B, Hkv, N + 7, D).bfloat16(), draw(g, B, Hkv, N + 7, D).bfloat16()
    K, V = Kc[:, :, :N], Vc[:, :, :N]
    out = fq.decode_attn_gqa_strided(q.cuda(), Kc.cuda()[:, :, :N], Vc.cuda()[:, :, :N], 8)
    ref = oracle.gqa_attention(q.numpy(), K.float().numpy(), V.float().numpy())
    assert maxerr(out, ref) <= TOL


def test_bf16_nhd_equals_strided_and_the_oracle():
    g = torch.Generator().manual_seed(58)
    B, Hq, Hkv, N, D = 2, 32, 8, 1500, 128
    q = draw(g, B, Hq, D).half()
    K, V = draw(g, B, N, Hkv, D).bfloat16(), draw(g, B, N, Hkv, D).bfloat16()
    a = fq.decode_attn_gqa_nhd(q.cuda(), K.cuda(), V.cuda(), 8)
    b = fq.decode_attn_gqa_strided(q.cuda(), K.cuda().transpose(1, 2), V.cuda().transpose(1, 2), 8)
    assert torch.equal(a, b)
    ref = oracle.gqa_attention(q.numpy(), K.float().numpy().transpose(0, 2, 1, 3),
                               V.float().numpy().transpose(0, 2, 1, 3))
    assert maxerr(a, ref) <= TOL


def test_bf16_keys_beyond_the_fp16_range():
    """Keys outside fp16's range (elements up to ~1e5, and ~1e-6, below fp16's normal range) are
    exact in bf16 and must neither overflow nor lose precision in the products: a score of ~2e5
    picks one token for head 0, the other heads weigh every token almost alike."""
    g = torch.Generator().manual_seed(59)
    B, Hq, Hkv, N, D = 1, 4, 1, 64, 64
    q = draw(g, B, Hq, D).half()
    K = (draw(g, B, Hkv, N, D) * 1e-6).bfloat16()
    V = (draw(g, B, Hkv, N, D) * 1e-3).bfloat16()
    K[0, 0, 9] = (q[0, 0].float() * 3e4).bfloat16()  # elements past fp16's 65504; a dot of ~2e6 for head 0
    out = fq.decode_attn_gqa_strided(q.cuda(), K.cuda(), V.cuda(), 8)
    ref = oracle.gqa_attention(q.numpy(), K.float().numpy(), V.float().numpy())
    assert np.isfinite(out.float().cpu().numpy()).all()
    assert maxerr(out, ref) <= 1e-5


@pytest.mark.parametrize("N,D,S", [(16384, 128, 32), (100, 64, 7), (3, 128, 8)])
def test_bf16_split_k_with_caller_scratch(N, D, S):
    """gqa_sk_fast_bf16: the reference's split-K call (caller-owned scratch) with bf16 K and V,
    against the oracle; fp16 K and V are refused."""
    g = torch.Generator().manual_seed(60 + N)
    Hq, Hkv = 32, 8
    q = draw(g, Hq, D).half()
    K, V = draw(g, Hkv, N, D).bfloat16(), draw(g, Hkv, N, D).bfloat16()
    mp, lp = torch.empty(Hq, S, device="cuda"), torch.empty(Hq, S, device="cuda")
    op = torch.empty(Hq, S, D, device="cuda")
    o = torch.empty(Hq, D, dtype=torch.float16, device="cuda")
    fq.gqa_sk_fast_bf16(q.cuda(), K.cuda(), V.cuda(), mp, lp, op, o, S, 8, 8)
    Kf, Vf = K.float().numpy(), V.float().numpy()
    assert maxerr(o, oracle.gqa_attention(q.numpy()[None], Kf[None], Vf[None])[0]) <= TOL
    with pytest.raises(RuntimeError, match="^bf16"):
        fq.gqa_sk_fast_bf16(q.cuda(), K.half().cuda(), V.half().cuda(), mp, lp, op, o, S, 8, 8)
