"""fp8 e4m3 KV caches (no counterpart in the reference; needs an MI355X).

The format is OCP fp8 e4m3 codes with fp16 per-token scales, value = code *
scale, defined by the oracle's quant_fp8_per_token (fp32 expressions, round to
nearest even; pinned against torch's float8_e4m3fn conversions on the CPU).
Here: the GPU quantizer's bytes equal the oracle's for fp32, fp16 and bf16
rows in every form (bulk, append, append at device positions, pages), and
decode over fp8 caches -- MHA, GQA at every group width, split-K, the internal
split, strided and paged layouts -- is within max-abs 2e-3 of the float64
oracle over the dequantized cache.
"""

import numpy as np
import pytest
import torch

import oracle
import fqkv_decode as fq

pytestmark = pytest.mark.gpu

TOL = 2e-3
DEV = "cuda"


def draw(g, *shape):
    return torch.randn(*shape, generator=g, dtype=torch.float32)


def maxerr(out, ref):
    return float(np.abs(out.float().cpu().numpy().astype(np.float64) - ref).max())


def codes(t):
    return t.view(torch.uint8).cpu().numpy()


def quantize(X):
    """GPU quantizer on X, with the float64 dequantized values from the oracle's decode of its codes."""
    q, s = fq.quantize_fp8_per_token(X.to(DEV))
    return q, s, oracle.dequant_fp8(codes(q), s.cpu().numpy()).astype(np.float64)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 128])
def test_quantizer_bytes_equal_the_oracle(dtype, D):
    g = torch.Generator().manual_seed(80)
    X = (draw(g, 5, 301, D) * 4).to(dtype)
    X[0, 0] = 0.0                      # all-zero row: codes 0, scale fp16(1e-8)
    X[0, 1, :7] = -0.0                 # -0 is stored as +0
    X[1, 2, 0] = 448.0                 # a row whose maximum is exactly 448
    X[1, 3, :] = 1e-3                  # a constant row
    X[2, 4, 9] = -60000.0              # one spike: everything else rounds small
    q, s = fq.quantize_fp8_per_token(X.to(DEV))
    assert q.dtype == torch.float8_e4m3fn and s.dtype == torch.float16
    oq, os_ = oracle.quant_fp8_per_token(X.float().numpy())
    np.testing.assert_array_equal(codes(q), oq)
    np.testing.assert_array_equal(s.cpu().numpy(), os_)


@pytest.mark.parametrize("D", [64, 128])
def test_append_forms_write_the_quantizer_bytes(D):
    g = torch.Generator().manual_seed(81)
    B, H, cap, n = 2, 3, 40, 5
    Kn, Vn = draw(g, B, H, n, D).half().to(DEV), draw(g, B, H, n, D).half().to(DEV)
    (kq, ks), (vq, vs) = fq.quantize_fp8_per_token(Kn), fq.quantize_fp8_per_token(Vn)

    def caches():
        c = lambda: torch.zeros(B, H, cap, D, dtype=torch.uint8, device=DEV).view(torch.float8_e4m3fn)
        sc = lambda: torch.zeros(B, H, cap, dtype=torch.float16, device=DEV)
        return [c(), c(), sc(), sc()]

    a = caches()
    fq.quantize_kv_append_(Kn, Vn, *a, 7)
    for got, want in ((a[0], kq), (a[1], vq)):
        assert np.array_equal(codes(got[:, :, 7:7 + n]), codes(want))
        assert not codes(got[:, :, :7]).any() and not codes(got[:, :, 7 + n:]).any()
    assert torch.equal(a[2][:, :, 7:7 + n], ks) and torch.equal(a[3][:, :, 7:7 + n], vs)
    b = caches()
    pos = torch.tensor([2, 30], dtype=torch.int32, device=DEV)
    fq.quantize_kv_append_at_(Kn, Vn, *b, pos)
    for i, p in enumerate((2, 30)):
        assert np.array_equal(codes(b[0][i, :, p:p + n]), codes(kq[i]))
        assert torch.equal(b[3][i, :, p:p + n], vs[i])
    # pages: token t of [T, H, D] rows to slot t * 3 of head-major pages of 16
    T = 20
    Kt, Vt = draw(g, T, H, D).bfloat16().to(DEV), draw(g, T, H, D).bfloat16().to(DEV)
    P, page = 4, 16
    hnd = lambda: torch.zeros(P, H, page, D, dtype=torch.uint8, device=DEV).view(torch.float8_e4m3fn).permute(0, 2, 1, 3)
    Kp, Vp = hnd(), hnd()
    Ksp = torch.zeros(P, H, page, dtype=torch.float16, device=DEV).permute(0, 2, 1)
    Vsp = torch.zeros(P, H, page, dtype=torch.float16, device=DEV).permute(0, 2, 1)
    slots = torch.arange(T, dtype=torch.int32, device=DEV) * 3
    fq.quantize_kv_to_pages_(Kt, Vt, slots, Kp, Vp, Ksp, Vsp)
    tq, ts = fq.quantize_fp8_per_token(Kt)
    sl = slots.long()
    assert np.array_equal(Kp.view(torch.uint8)[sl // page, sl % page].cpu().numpy(), codes(tq))
    assert torch.equal(Ksp[sl // page, sl % page], ts)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 8), (32, 8), (64, 8), (128, 8), (48, 8)])
@pytest.mark.parametrize("N", [1, 100, 3000])
def test_gqa_against_the_oracle(N, Hq, Hkv, D):
    g = torch.Generator().manual_seed(82 + N + Hq + D)
    B = 2
    q = draw(g, B, Hq, D).half()
    Kq, Ks, Kf = quantize(draw(g, B, Hkv, N, D) * 3)
    Vq, Vs, Vf = quantize(draw(g, B, Hkv, N, D))
    out = fq.decode_attn_gqa_fp8(q.to(DEV), Kq, Vq, Ks, Vs, 8)
    assert maxerr(out, oracle.gqa_attention(q.numpy(), Kf, Vf)) <= TOL


@pytest.mark.parametrize("B,N,D", [(1, 20000, 128), (3, 5000, 64), (64, 300, 128)])
def test_mha_and_the_internal_split(B, N, D):
    """One query head per KV head (MHA), from one long row (split internally over the CUs) to many
    short ones."""
    g = torch.Generator().manual_seed(83)
    q = draw(g, B, 1, D).half()
    Kq, Ks, Kf = quantize(draw(g, B, 1, N, D))
    Vq, Vs, Vf = quantize(draw(g, B, 1, N, D))
    out = fq.decode_attn_gqa_fp8(q.to(DEV), Kq, Vq, Ks, Vs, 8)
    assert maxerr(out, oracle.gqa_attention(q.numpy(), Kf, Vf)) <= TOL


@pytest.mark.parametrize("N,D,S", [(16384, 128, 32), (4096, 64, 16), (100, 128, 7), (3, 64, 8)])
def test_split_k_against_the_oracle(N, D, S):
    g = torch.Generator().manual_seed(84)
    Hq, Hkv = 32, 8
    q = draw(g, Hq, D).half()
    Kq, Ks, Kf = quantize(draw(g, Hkv, N, D))
    Vq, Vs, Vf = quantize(draw(g, Hkv, N, D))
    mp, lp = torch.empty(Hq, S, device=DEV), torch.empty(Hq, S, device=DEV)
    op = torch.empty(Hq, S, D, device=DEV)
    o = torch.empty(Hq, D, dtype=torch.float16, device=DEV)
    fq.gqa_sk_fast_fp8(q.to(DEV), Kq, Vq, Ks, Vs, mp, lp, op, o, S, 8, 8)
    ref = oracle.gqa_attention(q.numpy()[None], Kf[None], Vf[None])[0]
    assert maxerr(o, ref) <= TOL


def test_strided_and_paged_layouts():
    """The filled part of a larger fp8 cache through decode_attn_gqa_strided equals the contiguous
    entry point bit for bit; head-major pages at shuffled ids through decode_attn_gqa_paged match
    the oracle for ragged lengths."""
    g = torch.Generator().manual_seed(85)
    B, Hq, Hkv, N, cap, D = 2, 32, 8, 1000, 1536, 128
    q = draw(g, B, Hq, D).half().to(DEV)
    Kc, Ksc, _ = quantize(draw(g, B, Hkv, cap, D))
    Vc, Vsc, _ = quantize(draw(g, B, Hkv, cap, D))
    a = fq.decode_attn_gqa_fp8(q, Kc[:, :, :N].contiguous(), Vc[:, :, :N].contiguous(), Ksc[:, :, :N].contiguous(),
                               Vsc[:, :, :N].contiguous(), 8)
    b = fq.decode_attn_gqa_strided(q, Kc[:, :, :N], Vc[:, :, :N], 8, Ksc[:, :, :N], Vsc[:, :, :N])
    assert torch.equal(a, b)
    lens, page = [1, 17, 700], 32
    npg = [-(-n // page) for n in lens]
    P = sum(npg) + 2
    perm = torch.randperm(P, generator=g)
    table = torch.full((3, max(npg)), -1, dtype=torch.int32)
    k = 0
    for i, n in enumerate(npg):
        table[i, :n] = perm[k:k + n].to(torch.int32)
        k += n
    Kp, Ksp, Kpf = quantize(draw(g, P, Hkv, page, D))  # head-major storage
    Vp, Vsp, Vpf = quantize(draw(g, P, Hkv, page, D))
    q3 = draw(g, 3, Hq, D).half()
    out = fq.decode_attn_gqa_paged(q3.to(DEV), Kp.permute(0, 2, 1, 3), Vp.permute(0, 2, 1, 3), table.to(DEV),
                                   torch.tensor(lens, dtype=torch.int32, device=DEV), max(lens), 8,
                                   Ksp.permute(0, 2, 1), Vsp.permute(0, 2, 1))
    for i, n in enumerate(lens):
        t = np.arange(n)
        pid = table[i, t // page].numpy()
        Kb = Kpf[pid, :, t % page].transpose(1, 0, 2)  # [Hkv, n, D]
        Vb = Vpf[pid, :, t % page].transpose(1, 0, 2)
        ref = oracle.gqa_attention(q3.numpy()[i:i + 1], Kb[None], Vb[None])[0]
        assert maxerr(out[i], ref) <= TOL, (i, n)


def test_entry_points_reject_other_dtypes():
    q = torch.zeros(1, 8, 128, dtype=torch.float16, device=DEV)
    K = torch.zeros(1, 8, 16, 128, dtype=torch.int8, device=DEV)
    s = torch.zeros(1, 8, 16, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError, match="^fp8"):
        fq.decode_attn_gqa_fp8(q, K, K, s, s, 8)


@pytest.mark.parametrize("D,B", [(64, 8), (64, 2), (128, 8)])
def test_token_major_layout(D, B):
    """Token-major [B, N, Hkv, D] fp8 caches: at D 64 a token's row is 64 bytes, so neighbouring
    KV heads share 128-byte lines and the launcher's head grouping renumbers the work items; the
    output equals the head-major layout's bit for bit, and the oracle."""
    g = torch.Generator().manual_seed(86 + D + B)
    Hq, Hkv, N = 32, 8, 2000
    q = draw(g, B, Hq, D).half()
    Kq, Ks, Kf = quantize(draw(g, B, N, Hkv, D))
    Vq, Vs, Vf = quantize(draw(g, B, N, Hkv, D))
    out = fq.decode_attn_gqa_nhd(q.to(DEV), Kq, Vq, 8, Ks, Vs)
    hm = lambda t: t.transpose(1, 2).contiguous()
    ref_c = fq.decode_attn_gqa_fp8(q.to(DEV), hm(Kq.view(torch.uint8)).view(torch.float8_e4m3fn),
                                   hm(Vq.view(torch.uint8)).view(torch.float8_e4m3fn), hm(Ks), hm(Vs), 8)
    assert torch.equal(out, ref_c)
    assert maxerr(out, oracle.gqa_attention(q.numpy(), Kf.transpose(0, 2, 1, 3), Vf.transpose(0, 2, 1, 3))) <= TOL
