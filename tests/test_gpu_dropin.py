"""The reference's own acceptance checks, run through the drop-in path (needs an MI355X).

The reference's test file builds each kernel with torch.utils.cpp_extension.load and
accepts a result that is allclose to PyTorch attention at atol 2e-2 (int8: 3e-2 against
attention over the dequantized cache) for the shapes of tests/test_kernels.py:18,26,41,59.
Here the modules come from fqkv_decode.load with the reference's own arguments, and the
same shapes and tolerances are checked, so a caller's test suite can switch by changing
its import. The comparison attention is computed in float32 (the oracle-based tests hold
the kernels to 2e-3 against float64; this file checks the calling convention end to end).
"""

import pytest
import torch
import torch.nn.functional as F

import fqkv_decode
from fqkv_decode import quant

pytestmark = pytest.mark.gpu

DEV = "cuda"


def modules():
    """The four modules the reference's test fixture loads (tests/test_kernels.py:8-11)."""
    kw = dict(extra_cuda_cflags=["-O3"], verbose=False)
    return {n: fqkv_decode.load(name="t_" + n, sources=["kernels/%s.cu" % f], **kw)
            for n, f in (("fp16", "decode_attn_fp16_mw"), ("int8", "decode_attn_int8_mw"),
                         ("int4", "decode_attn_int4"), ("gqa", "decode_attn_gqa"))}


def attention(q, K, V):
    """softmax(q K^T / sqrt(D)) V per row in float32: q [R, D], K / V [R, N, D]."""
    R, N, D = K.shape
    out = F.scaled_dot_product_attention(q.float().view(R, 1, 1, D), K.float().view(R, 1, N, D).contiguous(),
                                         V.float().view(R, 1, N, D).contiguous())
    return out.view(R, D)


def randn(*shape):
    return torch.randn(*shape, dtype=torch.float16, device=DEV)


@pytest.mark.parametrize("B,N,W", [(1, 1024, 8), (8, 2048, 4), (256, 4096, 8)])
def test_reference_fp16(B, N, W):
    torch.manual_seed(0)
    q, K, V = randn(B, 64), randn(B, N, 64), randn(B, N, 64)
    out = modules()["fp16"].decode_attn_fp16_mw(q, K, V, W)
    assert torch.allclose(out.float(), attention(q, K, V), atol=2e-2)


@pytest.mark.parametrize("B,N,W", [(1, 1024, 8), (8, 2048, 4)])
def test_reference_int8(B, N, W):
    torch.manual_seed(0)
    q, K, V = randn(B, 64), randn(B, N, 64), randn(B, N, 64)
    (Kq, Ks), (Vq, Vs) = quant.quant_int8_per_token(K), quant.quant_int8_per_token(V)
    out = modules()["int8"].decode_attn_int8_mw(q, Kq, Vq, Ks, Vs, W)
    ref = attention(q, quant.dequant_int8(Kq, Ks).half(), quant.dequant_int8(Vq, Vs).half())
    assert torch.allclose(out.float(), ref, atol=3e-2)


@pytest.mark.parametrize("B,N,W", [(1, 1024, 8), (16, 4096, 8)])
def test_reference_gqa(B, N, W):
    torch.manual_seed(0)
    Hq, Hkv, D = 32, 8, 64
    q, K, V = randn(B, Hq, D), randn(B, Hkv, N, D), randn(B, Hkv, N, D)
    out = modules()["gqa"].decode_attn_gqa(q, K, V, W)
    G = Hq // Hkv
    ref = attention(q.reshape(B * Hq, D), K.repeat_interleave(G, 1).reshape(B * Hq, N, D),
                    V.repeat_interleave(G, 1).reshape(B * Hq, N, D)).view(B, Hq, D)
    assert torch.allclose(out.float(), ref, atol=2e-2)


# the split-K cases include N < S, N = 1 and S not dividing N (empty splits)
@pytest.mark.parametrize("N,D,S,W,CW", [(1024, 64, 8, 8, 4), (4096, 128, 16, 8, 4), (16384, 64, 64, 8, 8),
                                        (3, 128, 8, 4, 4), (1, 64, 4, 2, 4), (100, 64, 7, 4, 4)])
def test_reference_gqa_sk_fast(N, D, S, W, CW):
    m = fqkv_decode.load(name="t_gsk", sources=["kernels/decode_attn_gqa_sk_fast.cu"], extra_cuda_cflags=["-O3"],
                         verbose=False)
    torch.manual_seed(0)
    Hq, Hkv = 32, 8
    q, K, V = randn(Hq, D), randn(Hkv, N, D), randn(Hkv, N, D)
    mp = torch.empty(Hq, S, device=DEV)
    lp = torch.empty(Hq, S, device=DEV)
    op = torch.empty(Hq, S, D, device=DEV)
    out = torch.empty(Hq, D, dtype=torch.float16, device=DEV)
    m.gqa_sk_fast(q, K, V, mp, lp, op, out, S, W, CW)
    G = Hq // Hkv
    ref = attention(q, K.repeat_interleave(G, 0), V.repeat_interleave(G, 0))
    assert torch.allclose(out.float(), ref, atol=2e-2)


def test_reference_int4_gate():
    """The notebook's int4 check at its shape (D 64, per-token int4 K and V)."""
    torch.manual_seed(0)
    B, N = 8, 2048
    q, K, V = randn(B, 64), randn(B, N, 64), randn(B, N, 64)
    (Kp, Ks), (Vp, Vs) = quant.quant_int4_per_token(K), quant.quant_int4_per_token(V)
    out = modules()["int4"].decode_attn_int4(q, Kp, Vp, Ks, Vs, 8)
    ref = attention(q, quant.dequant_int4(Kp, Ks).half(), quant.dequant_int4(Vp, Vs).half())
    assert torch.allclose(out.float(), ref, atol=3e-2)
