"""The on-GPU per-token KV quantizers (fqkv_quantize_kv) against the oracle's
restatement of the reference quantizers (tests/test_kernels.py:32-34,
nb:292-299): bytes and fp16 scales identical, for fp16 and fp32 inputs, both
head dims, random rows and hand-built edge rows (round-half-even ties,
all-zero rows, fp16 scale underflow, +-0, single spikes), then the quantized
cache through the decode kernels."""

import numpy as np
import pytest
import torch

import oracle
import fqkv_decode as fq
from fqkv_decode import quant

pytestmark = pytest.mark.gpu

TOL = 2e-3


def draw(g, *shape):
    return torch.randn(*shape, generator=g, dtype=torch.float32)


def edge_rows(D, dtype):
    rows = []
    r = np.zeros(D, np.float32)
    rows.append(r.copy())                                   # all zero
    r = np.zeros(D, np.float32); r[0] = 127.0; r[1:8] = [2.5, -2.5, 3.5, -0.5, 0.5, 1.5, -1.5]
    rows.append(r)                                          # s = 1: exact .5 ties
    r = np.zeros(D, np.float32); r[0] = 7.0; r[1:6] = [2.5, -3.5, 0.5, 6.5, -6.5]
    rows.append(r)                                          # int4 ties at s = 1
    r = np.zeros(D, np.float32); r[5] = -3.0
    rows.append(r)                                          # single spike
    r = np.full(D, 1e-7, np.float32); r[3] = -2e-7
    rows.append(r)                                          # tiny: fp16 scale underflows to 0
    r = np.zeros(D, np.float32); r[0] = -0.0; r[1] = 60000.0 if dtype == np.float16 else 3.0e5 / 7.0
    rows.append(r)                                          # -0 and a huge value
    r = np.linspace(-1, 1, D).astype(np.float32)
    rows.append(r)
    return np.stack(rows).astype(dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_gpu_quantizer_bit_exact(dtype, D, fmt):
    g = torch.Generator().manual_seed(30)
    X = torch.randn(3, 1000, D, generator=g).to(dtype)
    X = torch.cat([X.reshape(-1, D), torch.from_numpy(edge_rows(D, X.numpy().dtype))]).contiguous()
    if fmt == "int8":
        q, s = fq.quantize_int8_per_token(X.cuda())
        oq, os_ = oracle.quant_int8_per_token(X.numpy())
    else:
        q, s = fq.quantize_int4_per_token(X.cuda())
        oq, os_ = oracle.quant_int4_per_token(X.numpy())
    assert q.shape == oq.shape and s.shape == os_.shape
    np.testing.assert_array_equal(q.cpu().numpy(), oq)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint16), os_.view(np.uint16))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_gpu_quantizer_matches_pytorch_expressions_on_gpu(dtype):
    """Same bytes as the package's PyTorch quantizers evaluated on the same device."""
    g = torch.Generator().manual_seed(31)
    X = torch.randn(4, 8, 333, 128, generator=g).to(dtype).cuda()
    q, s = fq.quantize_int8_per_token(X)
    tq, ts = quant.quant_int8_per_token(X)
    assert torch.equal(q, tq) and torch.equal(s.view(torch.int16), ts.view(torch.int16))
    P, s4 = fq.quantize_int4_per_token(X)
    tP, ts4 = quant.quant_int4_per_token(X)
    assert torch.equal(P, tP) and torch.equal(s4.view(torch.int16), ts4.view(torch.int16))


@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_gpu_quantized_cache_decodes(fmt):
    """Quantize K/V on the GPU, decode with the int8 / int4 kernels: within 2e-3
    of the float64 oracle on the dequantised cache."""
    g = torch.Generator().manual_seed(32)
    B, N, D = 16, 2048, 128
    q = torch.randn(B, D, generator=g).half()
    K, V = torch.randn(B, N, D, generator=g), torch.randn(B, N, D, generator=g)
    f = fq.quantize_int8_per_token if fmt == "int8" else fq.quantize_int4_per_token
    Kq, Ks = f(K.cuda())
    Vq, Vs = f(V.cuda())
    if fmt == "int8":
        out = fq.decode_attn_int8_mw(q.cuda(), Kq, Vq, Ks, Vs, 8)
        Kf = oracle.dequant_int8(Kq.cpu().numpy(), Ks.cpu().numpy())
        Vf = oracle.dequant_int8(Vq.cpu().numpy(), Vs.cpu().numpy())
    else:
        out = fq.decode_attn_int4(q.cuda(), Kq, Vq, Ks, Vs, 8)
        Kf = oracle.dequant_int4(Kq.cpu().numpy(), Ks.cpu().numpy())
        Vf = oracle.dequant_int4(Vq.cpu().numpy(), Vs.cpu().numpy())
    ref = oracle.attention(q.numpy(), Kf, Vf)
    assert float(np.abs(out.float().cpu().numpy() - ref).max()) <= TOL


def test_gpu_quantizer_rejects_bad_input():
    with pytest.raises(RuntimeError, match="^D:"):
        fq.quantize_int8_per_token(torch.zeros(4, 96, device="cuda"))
    with pytest.raises(RuntimeError, match="^fp16:"):
        fq.quantize_int4_per_token(torch.zeros(4, 64, device="cuda", dtype=torch.float64))
    with pytest.raises(RuntimeError, match="^contig:"):
        fq.quantize_int8_per_token(torch.zeros(64, 4, device="cuda").t())


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_gpu_quantize_append_writes_only_its_slots(dtype, D, fmt):
    """quantize_kv_append_ puts the quantizer's bytes and scales of the new K and V
    tokens at positions pos .. pos+n-1 of every cache row and leaves the rest alone."""
    B, H, cap = 2, 3, 40
    g = torch.Generator().manual_seed(60)
    width, qdt = (D, torch.int8) if fmt == "int8" else (D // 2, torch.uint8)
    Kc = torch.full((B, H, cap, width), 0x55, dtype=qdt, device="cuda")
    Vc = torch.full_like(Kc, 0x33)
    Ksc = torch.full((B, H, cap), 7.0, dtype=torch.float16, device="cuda")
    Vsc = torch.full_like(Ksc, 9.0)
    qfn = fq.quantize_int8_per_token if fmt == "int8" else fq.quantize_int4_per_token
    pos = 0
    for n in (5, 1, 1, 17):
        Kn = (torch.randn(B, H, n, D, generator=g) * 3).to(dtype).cuda()
        Vn = (torch.randn(B, H, n, D, generator=g) * 3).to(dtype).cuda()
        if n == 17:
            Kn[0, 0, 0] = torch.from_numpy(edge_rows(D, np.float16 if dtype == torch.float16 else np.float32)[1])
        before = [t.clone() for t in (Kc, Vc, Ksc, Vsc)]
        fq.quantize_kv_append_(Kn, Vn, Kc, Vc, Ksc, Vsc, pos)
        for got, old, (q, s) in ((Kc, before[0], qfn(Kn)), (Vc, before[1], qfn(Vn))):
            assert torch.equal(got[:, :, pos:pos + n], q)
            assert torch.equal(got[:, :, :pos], old[:, :, :pos]) and torch.equal(got[:, :, pos + n:], old[:, :, pos + n:])
        for got, old, (q, s) in ((Ksc, before[2], qfn(Kn)), (Vsc, before[3], qfn(Vn))):
            assert torch.equal(got[:, :, pos:pos + n], s)
            assert torch.equal(got[:, :, :pos], old[:, :, :pos]) and torch.equal(got[:, :, pos + n:], old[:, :, pos + n:])
        pos += n
    with pytest.raises(RuntimeError, match="pos"):
        fq.quantize_kv_append_(Kn[:, :, :1].contiguous(), Vn[:, :, :1].contiguous(), Kc, Vc, Ksc, Vsc, cap)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_gpu_quantize_append_at_device_positions(dtype, D, fmt):
    """quantize_kv_append_at_ writes sequence b's new tokens at pos[b] (an int32 tensor read on the
    GPU): the caches equal quantize_kv_append_ called per sequence at that position. Sequences whose
    tokens would not fit in [0, capacity) (pos < 0, pos + n > capacity) are left untouched, and the
    same call replayed from a captured graph follows the positions as they change."""
    B, H, cap = 5, 3, 40
    g = torch.Generator().manual_seed(64)
    width, qdt = (D, torch.int8) if fmt == "int8" else (D // 2, torch.uint8)

    def caches():
        Kc = torch.full((B, H, cap, width), 0x55, dtype=qdt, device="cuda")
        Ksc = torch.full((B, H, cap), 7.0, dtype=torch.float16, device="cuda")
        return [Kc, torch.full_like(Kc, 0x33), Ksc, torch.full_like(Ksc, 9.0)]

    for n, positions in ((4, [0, 7, 36, 37, -1]), (1, [39, 0, 40, 12, -7]), (17, [23, 3, 24, 0, 2**31 - 1])):
        Kn = (torch.randn(B, H, n, D, generator=g) * 3).to(dtype).cuda()
        Vn = (torch.randn(B, H, n, D, generator=g) * 3).to(dtype).cuda()
        got, want = caches(), caches()
        pos = torch.tensor(positions, dtype=torch.int32, device="cuda")
        fq.quantize_kv_append_at_(Kn, Vn, *got, pos)
        for b, p in enumerate(positions):
            if 0 <= p <= cap - n:
                per_seq = [t[b:b + 1] for t in want]
                fq.quantize_kv_append_(Kn[b:b + 1].contiguous(), Vn[b:b + 1].contiguous(), *per_seq, p)
        for x, y in zip(got, want):
            assert torch.equal(x, y)

    # captured: each replay appends one token where pos points, then the graph-free add moves pos on
    Kn = (torch.randn(B, H, 1, D, generator=g) * 3).to(dtype).cuda()
    Vn = (torch.randn(B, H, 1, D, generator=g) * 3).to(dtype).cuda()
    got, want = caches(), caches()
    pos = torch.tensor([0, 5, 10, 38, 39], dtype=torch.int32, device="cuda")
    start = pos.clone()
    fq.quantize_kv_append_at_(Kn, Vn, *got, pos)  # first call outside the capture loads the kernel
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fq.quantize_kv_append_at_(Kn, Vn, *got, pos)
    for step in range(3):
        pos.copy_(start + step)
        graph.replay()
        torch.cuda.synchronize()
    for step in range(3):
        for b, p in enumerate((start + step).tolist()):
            if p <= cap - 1:
                fq.quantize_kv_append_(Kn[b:b + 1].contiguous(), Vn[b:b + 1].contiguous(), *[t[b:b + 1] for t in want],
                                       p)
    for x, y in zip(got, want):
        assert torch.equal(x, y)
    with pytest.raises(RuntimeError, match="^shape: pos"):
        fq.quantize_kv_append_at_(Kn, Vn, *got, pos[:4])
    with pytest.raises(RuntimeError, match="^shape: pos"):
        fq.quantize_kv_append_at_(Kn, Vn, *got, pos.long())


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_gpu_quantizers_take_bf16_rows(fmt, D):
    """bf16 rows (a bf16 model's keys and values) widen exactly to fp32, so every quantizer form
    writes the bytes the fp32 quantizer writes for x.float(): bulk, append at host and device
    positions, and into pages by slot."""
    g = torch.Generator().manual_seed(67)
    qfn = fq.quantize_int8_per_token if fmt == "int8" else fq.quantize_int4_per_token
    X = (torch.randn(3, 37, D, generator=g) * 5).bfloat16().cuda()
    X[0, 0] = 0.0  # an all-zero row
    X[1, 2, 5] = 3.0e38  # beyond fp16's range: exact in bf16 and fp32
    for got, want in zip(qfn(X), qfn(X.float())):
        assert torch.equal(got, want)
    B, H, cap, n = 2, 3, 20, 4
    width, qdt = (D, torch.int8) if fmt == "int8" else (D // 2, torch.uint8)
    Kn = (torch.randn(B, H, n, D, generator=g) * 3).bfloat16().cuda()
    Vn = (torch.randn(B, H, n, D, generator=g) * 3).bfloat16().cuda()
    for at in (False, True):
        a = [torch.zeros(B, H, cap, width, dtype=qdt, device="cuda") for _ in range(2)] + \
            [torch.zeros(B, H, cap, dtype=torch.float16, device="cuda") for _ in range(2)]
        b = [t.clone() for t in a]
        if at:
            pos = torch.tensor([3, 9], dtype=torch.int32, device="cuda")
            fq.quantize_kv_append_at_(Kn, Vn, *a, pos)
            fq.quantize_kv_append_at_(Kn.float(), Vn.float(), *b, pos)
        else:
            fq.quantize_kv_append_(Kn, Vn, *a, 5)
            fq.quantize_kv_append_(Kn.float(), Vn.float(), *b, 5)
        for x, y in zip(a, b):
            assert torch.equal(x, y)
    Kt, Vt = Kn.flatten(0, 2).view(-1, 1, D).expand(-1, H, D).contiguous(), Vn.flatten(0, 2).view(-1, 1, D).expand(-1, H, D).contiguous()
    slots = torch.randperm(64, generator=g)[:Kt.shape[0]].to(torch.int32).cuda()
    pa, pb = page_views(4, 16, H, width, qdt, "hnd"), page_views(4, 16, H, width, qdt, "hnd")
    fq.quantize_kv_to_pages_(Kt, Vt, slots, *pa)
    fq.quantize_kv_to_pages_(Kt.float(), Vt.float(), slots, *pb)
    for x, y in zip(pa, pb):
        assert torch.equal(x, y)


def page_views(P, page, H, width, qdt, layout):
    """Sentinel-filled pages [P, page, H, width] and scale pages [P, page, H] as the decode entry point
    takes them: NHD storage as is, HND storage ([P, H, page, .]) through a permuted view."""
    def codes(fill):
        if layout == "nhd":
            return torch.full((P, page, H, width), fill, dtype=qdt, device="cuda")
        return torch.full((P, H, page, width), fill, dtype=qdt, device="cuda").permute(0, 2, 1, 3)

    def scales(fill):
        if layout == "nhd":
            return torch.full((P, page, H), fill, dtype=torch.float16, device="cuda")
        return torch.full((P, H, page), fill, dtype=torch.float16, device="cuda").permute(0, 2, 1)

    return codes(0x55), codes(0x33), scales(7.0), scales(9.0)


@pytest.mark.parametrize("layout", ["nhd", "hnd"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_gpu_quantize_to_pages(fmt, D, dtype, layout):
    """quantize_kv_to_pages_ writes token t's K and V codes and scales (the quantizer's bytes) at
    slot_mapping[t] of token-major or head-major pages and nothing else; slots -1 and past the last
    page are skipped."""
    P, page, H, T = 6, 16, 2, 40
    g = torch.Generator().manual_seed(65)
    width, qdt = (D, torch.int8) if fmt == "int8" else (D // 2, torch.uint8)
    Kn = (torch.randn(T, H, D, generator=g) * 3).to(dtype).cuda()
    Vn = (torch.randn(T, H, D, generator=g) * 3).to(dtype).cuda()
    slots = torch.randperm(P * page, generator=g)[:T].to(torch.int32)
    slots[3], slots[11], slots[20] = -1, -7, P * page  # padding tokens and a slot past the pages
    slots[29] = 2 ** 31 - 1
    pages = page_views(P, page, H, width, qdt, layout)
    want = [t.clone() for t in pages]
    fq.quantize_kv_to_pages_(Kn, Vn, slots.cuda(), *pages)
    qfn = fq.quantize_int8_per_token if fmt == "int8" else fq.quantize_int4_per_token
    (kq, ks), (vq, vs) = qfn(Kn), qfn(Vn)
    ok = (slots >= 0) & (slots < P * page)
    pg, off = (slots[ok] // page).long().cuda(), (slots[ok] % page).long().cuda()
    sel = ok.nonzero().flatten().cuda()
    for w, x in zip(want, (kq, vq, ks, vs)):
        w[pg, off] = x[sel]
    for got, w in zip(pages, want):
        assert torch.equal(got, w)
    with pytest.raises(RuntimeError, match="^shape: slot_mapping"):
        fq.quantize_kv_to_pages_(Kn, Vn, slots.cuda().long(), *pages)
    with pytest.raises(RuntimeError, match="^shape: pages"):
        fq.quantize_kv_to_pages_(Kn[:, :1].contiguous(), Vn[:, :1].contiguous(), slots.cuda(), *pages)


@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_gpu_pages_filled_by_the_quantizer_decode_like_the_oracle(fmt):
    """A serving-style round trip: three ragged sequences (37, 16, 50 tokens) written into shuffled
    head-major pages of 16 tokens through their slot mapping, then decode_attn_gqa_paged over
    those pages against the float64 oracle on the dequantized tokens of each sequence."""
    B, Hq, Hkv, D, page = 3, 8, 2, 128, 16
    lens = [37, 16, 50]
    g = torch.Generator().manual_seed(66)
    npg = [-(-n // page) for n in lens]
    P = sum(npg) + 2
    perm = torch.randperm(P, generator=g).tolist()
    table = torch.zeros(B, max(npg), dtype=torch.int32)
    slot_list, K_list, V_list = [], [], []
    used = 0
    for b, n in enumerate(lens):
        ids = perm[used:used + npg[b]]
        used += npg[b]
        table[b, :npg[b]] = torch.tensor(ids, dtype=torch.int32)
        slot_list += [ids[t // page] * page + t % page for t in range(n)]
        K_list.append(draw(g, n, Hkv, D))
        V_list.append(draw(g, n, Hkv, D))
    Kn, Vn = torch.cat(K_list).half().cuda(), torch.cat(V_list).half().cuda()
    width, qdt = (D, torch.int8) if fmt == "int8" else (D // 2, torch.uint8)
    Kp, Vp, Ks, Vs = page_views(P, page, Hkv, width, qdt, "hnd")
    fq.quantize_kv_to_pages_(Kn, Vn, torch.tensor(slot_list, dtype=torch.int32).cuda(), Kp, Vp, Ks, Vs)
    q = draw(g, B, Hq, D).half()
    out = fq.decode_attn_gqa_paged(q.cuda(), Kp, Vp, table.cuda(), torch.tensor(lens, dtype=torch.int32).cuda(),
                                   max(lens), 8, Ks, Vs)
    deq = quant.dequant_int8 if fmt == "int8" else quant.dequant_int4
    qfn = fq.quantize_int8_per_token if fmt == "int8" else fq.quantize_int4_per_token
    start = 0
    for b, n in enumerate(lens):
        (kq, ks), (vq, vs) = qfn(Kn[start:start + n]), qfn(Vn[start:start + n])
        Kf = deq(kq, ks).permute(1, 0, 2).cpu().double().numpy()  # [Hkv, n, D]
        Vf = deq(vq, vs).permute(1, 0, 2).cpu().double().numpy()
        ref = oracle.gqa_attention(q[b:b + 1].numpy(), Kf[None], Vf[None])[0]
        assert float(np.abs(out[b].float().cpu().numpy().astype(np.float64) - ref).max()) <= TOL
        start += n


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_reference_quantizer_expressions_on_gpu_match_oracle(dtype, fmt):
    """The reference quantizes with PyTorch expressions on its device tensors,
    written with a division by the Python scalar 127.0 or 7.0
    (tests/test_kernels.py:32-34, nb:292-299). Those expressions, evaluated as
    written on this GPU's PyTorch, give exactly the oracle's bytes and fp16
    scales; the oracle rounds the scale as max|x| * fp32(1/qmax), the form
    PyTorch's division by a scalar takes."""
    qmax = 127 if fmt == "int8" else 7
    D = 128
    g = torch.Generator().manual_seed(31)
    X = torch.randn(2, 4000, D, generator=g).to(dtype)
    X = torch.cat([X.reshape(-1, D), torch.from_numpy(edge_rows(D, X.numpy().dtype))]).contiguous()
    Xd = X.cuda()
    a = Xd.abs().amax(-1, keepdim=True)
    s = (a / float(qmax)).clamp(min=1e-8)
    qv = torch.clamp(torch.round(Xd / s), -qmax, qmax).to(torch.int8)
    if fmt == "int4":
        qv = qv.view(qv.shape[0], D // 2, 2)
        qv = ((qv[..., 0] & 0xF) | ((qv[..., 1] & 0xF) << 4)).to(torch.uint8)
        oq, os_ = oracle.quant_int4_per_token(X.numpy())
    else:
        oq, os_ = oracle.quant_int8_per_token(X.numpy())
    np.testing.assert_array_equal(qv.cpu().numpy(), oq)
    np.testing.assert_array_equal(s.squeeze(-1).half().cpu().numpy().view(np.uint16), os_.view(np.uint16))
