"""Quantized GQA and split-K decode (int8 / int4 KV with per-token fp16
scales and a GQA head mapping): the combinations the reference does not have
(its int8/int4 kernels are MHA only, decode_attn_int8_mw.cu:52-64 and
decode_attn_int4.cu:47-57; its GQA and split-K kernels fp16 only,
decode_attn_gqa.cu:56-68 and decode_attn_gqa_sk_fast.cu:95-112). Checked
against the float64 oracle on the exactly dequantised cache at max-abs 2e-3,
the split scratch against the oracle's per-split partials."""

import numpy as np
import pytest
import torch

import oracle
import fqkv_decode as fq

pytestmark = pytest.mark.gpu

TOL = 2e-3


def draw(g, *shape):
    return torch.randn(*shape, generator=g, dtype=torch.float32)


def quantized(fmt, X):
    """Quantize on the GPU; return (bytes, scales) on the GPU and the float32 dequantised cache on the CPU."""
    if fmt == "int8":
        q, s = fq.quantize_int8_per_token(X.cuda())
        return q, s, oracle.dequant_int8(q.cpu().numpy(), s.cpu().numpy())
    P, s = fq.quantize_int4_per_token(X.cuda())
    return P, s, oracle.dequant_int4(P.cpu().numpy(), s.cpu().numpy())


def maxerr(out, ref):
    return float(np.abs(out.float().cpu().numpy().astype(np.float64) - ref).max())


@pytest.mark.parametrize("fmt", ["int8", "int4"])
@pytest.mark.parametrize("B,Hq,Hkv,N,D,W", [(2, 32, 8, 1000, 128, 8), (1, 16, 1, 4096, 64, 4),
                                            (3, 8, 8, 77, 128, 2), (1, 32, 8, 512, 64, 8)])
def test_gqa_quantized(fmt, B, Hq, Hkv, N, D, W):
    g = torch.Generator().manual_seed(40)
    q = draw(g, B, Hq, D).half()
    Kq, Ks, Kf = quantized(fmt, draw(g, B, Hkv, N, D))
    Vq, Vs, Vf = quantized(fmt, draw(g, B, Hkv, N, D))
    f = fq.decode_attn_gqa_int8 if fmt == "int8" else fq.decode_attn_gqa_int4
    out = f(q.cuda(), Kq, Vq, Ks, Vs, W)
    assert out.shape == (B, Hq, D) and out.dtype == torch.float16
    assert maxerr(out, oracle.gqa_attention(q.numpy(), Kf, Vf)) <= TOL


@pytest.mark.parametrize("fmt", ["int8", "int4"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("Hq,Hkv", [(32, 32), (32, 16), (24, 8), (40, 5), (7, 1), (48, 3)])
def test_gqa_quantized_group_sizes(fmt, D, Hq, Hkv):
    """Every head-group width of the kernel over quantized caches: groups of 1, 2
    and 4 heads (four tiles share the 16 score columns), 8 (two tiles) and 16
    (one), full and partial (G = 3, 5, 7 leave columns without a head)."""
    B, N = 2, 333
    g = torch.Generator().manual_seed(43)
    q = draw(g, B, Hq, D).half()
    Kq, Ks, Kf = quantized(fmt, draw(g, B, Hkv, N, D))
    Vq, Vs, Vf = quantized(fmt, draw(g, B, Hkv, N, D))
    f = fq.decode_attn_gqa_int8 if fmt == "int8" else fq.decode_attn_gqa_int4
    out = f(q.cuda(), Kq, Vq, Ks, Vs, 4)
    assert maxerr(out, oracle.gqa_attention(q.numpy(), Kf, Vf)) <= TOL


@pytest.mark.parametrize("fmt", ["int8", "int4"])
@pytest.mark.parametrize("Hq,Hkv,N,D,S,W", [(32, 8, 16384, 128, 32, 8), (8, 2, 100, 64, 7, 4),
                                            (4, 4, 3, 128, 8, 8), (64, 4, 5000, 128, 16, 8),
                                            (16, 8, 2000, 128, 16, 8), (40, 5, 1500, 64, 12, 4)])
def test_gqa_sk_fast_quantized(fmt, Hq, Hkv, N, D, S, W, merge_mode):
    g = torch.Generator().manual_seed(41)
    q = draw(g, Hq, D).half()
    Kq, Ks, Kf = quantized(fmt, draw(g, Hkv, N, D))
    Vq, Vs, Vf = quantized(fmt, draw(g, Hkv, N, D))
    mp = torch.empty(Hq, S, device="cuda")
    lp = torch.empty(Hq, S, device="cuda")
    op = torch.empty(Hq, S, D, device="cuda")
    o = torch.empty(Hq, D, device="cuda", dtype=torch.float16)
    f = fq.gqa_sk_fast_int8 if fmt == "int8" else fq.gqa_sk_fast_int4
    f(q.cuda(), Kq, Vq, Ks, Vs, mp, lp, op, o, S, W, 8)
    assert maxerr(o, oracle.gqa_attention(q.numpy()[None], Kf[None], Vf[None])[0]) <= TOL
    m, l, acc = oracle.split_partials(q.numpy(), Kf, Vf, S)
    assert np.array_equal(np.isneginf(mp.cpu().numpy()), np.isneginf(m))
    np.testing.assert_allclose(lp.cpu().numpy(), l, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(op.cpu().numpy(), acc, rtol=1e-4, atol=2e-4)


@pytest.mark.parametrize("N", [1, 17, 100, 127, 128, 129, 255, 257, 383, 1000])
@pytest.mark.parametrize("W", [2, 4, 8])
def test_int4_d64_single_head_ragged_passes(N, W):
    """int4 at D = 64 with one query head per work item loads 8 tiles (128 tokens)
    per wave pass: token counts on both sides of a pass and of a whole round of
    waves, against the oracle."""
    g = torch.Generator().manual_seed(43 + N)
    B, D = 3, 64
    q = draw(g, B, D).half()
    Kq, Ks, Kf = quantized("int4", draw(g, B, N, D))
    Vq, Vs, Vf = quantized("int4", draw(g, B, N, D))
    out = fq.decode_attn_int4(q.cuda(), Kq, Vq, Ks, Vs, W)
    assert maxerr(out, oracle.attention(q.numpy(), Kf, Vf)) <= TOL


@pytest.mark.parametrize("N,S,W", [(100, 3, 8), (257, 2, 4), (1000, 7, 8), (4095, 16, 8), (129, 1, 2),
                                   (2048, 32, 4)])
def test_int4_d64_single_head_split_k_ragged(N, S, W, merge_mode):
    """Split-K over int4 at D = 64 with one query head per KV head (8-tile passes):
    splits that end inside a pass, output and scratch against the oracle."""
    g = torch.Generator().manual_seed(47 + N)
    H, D = 4, 64
    q = draw(g, H, D).half()
    Kq, Ks, Kf = quantized("int4", draw(g, H, N, D))
    Vq, Vs, Vf = quantized("int4", draw(g, H, N, D))
    mp = torch.empty(H, S, device="cuda")
    lp = torch.empty(H, S, device="cuda")
    op = torch.empty(H, S, D, device="cuda")
    o = torch.empty(H, D, device="cuda", dtype=torch.float16)
    fq.gqa_sk_fast_int4(q.cuda(), Kq, Vq, Ks, Vs, mp, lp, op, o, S, W, 8)
    assert maxerr(o, oracle.gqa_attention(q.numpy()[None], Kf[None], Vf[None])[0]) <= TOL
    m, l, acc = oracle.split_partials(q.numpy(), Kf, Vf, S)
    assert np.array_equal(np.isneginf(mp.cpu().numpy()), np.isneginf(m))
    np.testing.assert_allclose(lp.cpu().numpy(), l, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(op.cpu().numpy(), acc, rtol=1e-4, atol=2e-4)


def test_gqa_quantized_matches_mha_kernel_on_expanded_cache():
    """GQA int8 = the reference-style MHA int8 kernel on repeat_kv-expanded K/V and scales."""
    g = torch.Generator().manual_seed(42)
    B, Hq, Hkv, N, D = 2, 32, 8, 777, 128
    G = Hq // Hkv
    q = draw(g, B, Hq, D).half().cuda()
    Kq, Ks, _ = quantized("int8", draw(g, B, Hkv, N, D))
    Vq, Vs, _ = quantized("int8", draw(g, B, Hkv, N, D))
    a = fq.decode_attn_gqa_int8(q, Kq, Vq, Ks, Vs, 8).float()
    ex = lambda t: t.repeat_interleave(G, 1).reshape(B * Hq, *t.shape[2:]).contiguous()
    b = fq.decode_attn_int8_mw(q.reshape(B * Hq, D), ex(Kq), ex(Vq), ex(Ks), ex(Vs), 8).float()
    assert float((a.reshape(B * Hq, D) - b).abs().max()) <= TOL


def test_quantized_entry_points_reject_bad_input():
    g = torch.Generator().manual_seed(43)
    q = draw(g, 1, 8, 128).half().cuda()
    K = torch.zeros(1, 2, 16, 128, dtype=torch.int8, device="cuda")
    s = torch.ones(1, 2, 16, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="^packed uint8"):
        fq.decode_attn_gqa_int4(q, K, K, s, s, 8)
    with pytest.raises(RuntimeError, match="^shape"):
        fq.decode_attn_gqa_int8(q, K, K, s[:, :1], s[:, :1], 8)
    with pytest.raises(RuntimeError, match="^heads"):
        fq.decode_attn_gqa_int8(draw(g, 1, 7, 128).half().cuda(), K, K, s, s, 8)


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("N,S,W", [(17, 1, 8), (100, 3, 8), (257, 8, 4), (1000, 16, 8), (2047, 32, 8),
                                   (4100, 32, 8), (16383, 32, 8), (129, 2, 2)])
def test_one_pass_waves_transposed_tokens_ragged(fmt, D, N, S, W, merge_mode):
    """int8 / fp8 waves of one pass (two-tile passes, and one four-tile pass with
    the deferred query preparation) score their tiles in a transposed token order
    and take V as loaded: splits and rows that end inside a tile, output and
    split scratch against the oracle, for grouped (Hq 32 / Hkv 8) heads."""
    g = torch.Generator().manual_seed(53 + N + D)
    Hq, Hkv = 32, 8
    q = draw(g, Hq, D).half()
    if fmt == "int8":
        Kq, Ks, Kf = quantized("int8", draw(g, Hkv, N, D))
        Vq, Vs, Vf = quantized("int8", draw(g, Hkv, N, D))
        f = fq.gqa_sk_fast_int8
    else:
        Kq, Ks = fq.quantize_fp8_per_token(draw(g, Hkv, N, D).cuda())
        Vq, Vs = fq.quantize_fp8_per_token(draw(g, Hkv, N, D).cuda())
        codes = lambda t: t.view(torch.uint8).cpu().numpy()
        Kf = oracle.dequant_fp8(codes(Kq), Ks.cpu().numpy())
        Vf = oracle.dequant_fp8(codes(Vq), Vs.cpu().numpy())
        f = fq.gqa_sk_fast_fp8
    mp = torch.empty(Hq, S, device="cuda")
    lp = torch.empty(Hq, S, device="cuda")
    op = torch.empty(Hq, S, D, device="cuda")
    o = torch.empty(Hq, D, device="cuda", dtype=torch.float16)
    f(q.cuda(), Kq, Vq, Ks, Vs, mp, lp, op, o, S, W, 8)
    assert maxerr(o, oracle.gqa_attention(q.numpy()[None], Kf[None], Vf[None])[0]) <= TOL
    if S > 1:
        m, l, acc = oracle.split_partials(q.numpy(), Kf, Vf, S)
        assert np.array_equal(np.isneginf(mp.cpu().numpy()), np.isneginf(m))
        np.testing.assert_allclose(lp.cpu().numpy(), l, rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(op.cpu().numpy(), acc, rtol=1e-4, atol=2e-4)
