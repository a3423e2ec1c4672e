"""GPU parity at the exact benchmark configurations (needs an MI355X).

* MHA over fp16 / int8 / int4 KV at B in {8, 256, 2048}, N = 4096, D = 128
  (the precision benchmark; the reference's own is benchmarks/standalone_quant.json
  at D = 64).
* GQA split-K, 32 query / 8 KV heads, batch 1, over the N sweep
  {512, 1K, 2K, 4K, 8K, 16K, 32K} at D = 64 and 128 (flashinfer_looptimed.py's grid).
* GQA split-K at batch 8, N = 32768, D = 128, with the batch folded into the
  heads: q [256, 128], K, V [64, 32768, 128].

Rows (MHA) and KV rows (GQA) are independent, so a seeded sample of 16 of them
(first and last included) is checked against the float64 oracle, and the whole
output against fp32 softmax(q K^T / sqrt(D)) V computed with PyTorch on the
GPU; both at the 2e-3 max-abs bar. The int8 / int4 caches come from the GPU
quantizer kernels, whose bytes are pinned against the oracle elsewhere
(tests/test_gpu_quant.py); the references dequantise those same bytes.
"""

import math

import numpy as np
import pytest
import torch

import oracle
import fqkv_decode as fq

pytestmark = pytest.mark.gpu

TOL = 2e-3
DEV = "cuda"


def sample_rows(n, k=16, seed=0):
    """k distinct row indices in [0, n): first, last and a seeded spread."""
    if n <= k:
        return list(range(n))
    rng = np.random.default_rng(seed)
    mid = rng.choice(np.arange(1, n - 1), size=k - 2, replace=False)
    return sorted({0, n - 1, *mid.tolist()})


def ref_fp32(q, Kf, Vf, chunk=128):
    """fp32 softmax(q K^T / sqrt(D)) V on the GPU, q [B, D], K/V [B, N, D] fp32, in row chunks."""
    B, D = q.shape
    out = torch.empty(B, D, device=DEV)
    for b0 in range(0, B, chunk):
        k = Kf[b0:b0 + chunk].contiguous()
        v = Vf[b0:b0 + chunk].contiguous()
        s = torch.bmm(k, q[b0:b0 + chunk].float().unsqueeze(2)).squeeze(2) / math.sqrt(D)
        out[b0:b0 + chunk] = torch.bmm(torch.softmax(s, dim=1).unsqueeze(1), v).squeeze(1)
    return out


def check(out, ref_full, ref_rows, rows):
    """Whole output vs the fp32 GPU reference, sampled rows vs the float64 oracle."""
    err_full = float((out.float() - ref_full).abs().max())
    assert err_full <= TOL, err_full
    got = out[rows].float().cpu().numpy().astype(np.float64)
    err_rows = float(np.abs(got - ref_rows).max())
    assert err_rows <= TOL, err_rows


@pytest.mark.parametrize("fmt", ["fp16", "int8", "int4"])
@pytest.mark.parametrize("B", [8, 256, 2048])
def test_mha_precision_benchmark_shapes(fmt, B):
    N, D, W = 4096, 128, 8
    g = torch.Generator(device=DEV).manual_seed(B)
    q = torch.randn(B, D, device=DEV, generator=g).half()
    rows = sample_rows(B, seed=B)
    if fmt == "fp16":
        K = torch.randn(B, N, D, device=DEV, generator=g).half()
        V = torch.randn(B, N, D, device=DEV, generator=g).half()
        out = fq.decode_attn_fp16_mw(q, K, V, W)
        ref_full = torch.empty(B, D, device=DEV)
        for b0 in range(0, B, 256):
            ref_full[b0:b0 + 256] = ref_fp32(q[b0:b0 + 256], K[b0:b0 + 256].float(), V[b0:b0 + 256].float())
        Kr, Vr = K[rows].float().cpu().numpy(), V[rows].float().cpu().numpy()
    else:
        quantize = fq.quantize_int8_per_token if fmt == "int8" else fq.quantize_int4_per_token
        Kq, Ks = quantize(torch.randn(B, N, D, device=DEV, generator=g))
        Vq, Vs = quantize(torch.randn(B, N, D, device=DEV, generator=g))
        if fmt == "int8":
            out = fq.decode_attn_int8_mw(q, Kq, Vq, Ks, Vs, W)
            deq = oracle.dequant_int8
            deq_gpu = lambda x, s: x.float() * s.float()[..., None]
        else:
            out = fq.decode_attn_int4(q, Kq, Vq, Ks, Vs, W)
            deq = oracle.dequant_int4
            from fqkv_decode import quant
            deq_gpu = quant.dequant_int4
        ref_full = torch.empty(B, D, device=DEV)
        for b0 in range(0, B, 256):
            sl = slice(b0, b0 + 256)
            ref_full[sl] = ref_fp32(q[sl], deq_gpu(Kq[sl], Ks[sl]), deq_gpu(Vq[sl], Vs[sl]))
        Kr = deq(Kq[rows].cpu().numpy(), Ks[rows].cpu().numpy())
        Vr = deq(Vq[rows].cpu().numpy(), Vs[rows].cpu().numpy())
    assert out.shape == (B, D) and out.dtype == torch.float16
    ref_rows = oracle.attention(q[rows].cpu().numpy(), Kr, Vr)
    check(out, ref_full, ref_rows, rows)


def run_sk(q, K, V, S, W, CW=8):
    Hq, D = q.shape
    mp = torch.empty(Hq, S, device=DEV)
    lp = torch.empty(Hq, S, device=DEV)
    op = torch.empty(Hq, S, D, device=DEV)
    o = torch.empty(Hq, D, dtype=torch.float16, device=DEV)
    fq.gqa_sk_fast(q, K, V, mp, lp, op, o, S, W, CW)
    return o


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("N", [512, 1024, 2048, 4096, 8192, 16384, 32768])
def test_gqa_split_k_n_sweep(N, D, merge_mode):
    """Batch 1, Hq 32 / Hkv 8: every head against the float64 oracle, at the
    benchmark's split counts (16 and 32) and both W the sweep uses."""
    Hq, Hkv = 32, 8
    g = torch.Generator().manual_seed(N + D)
    q = torch.randn(Hq, D, generator=g).half()
    K = torch.randn(Hkv, N, D, generator=g).half()
    V = torch.randn(Hkv, N, D, generator=g).half()
    ref = oracle.gqa_attention(q.numpy()[None], K.numpy()[None], V.numpy()[None])[0]
    qd, Kd, Vd = q.to(DEV), K.to(DEV), V.to(DEV)
    for S in (16, 32):
        for W in (4, 8):
            o = run_sk(qd, Kd, Vd, S, W)
            err = float(np.abs(o.float().cpu().numpy().astype(np.float64) - ref).max())
            assert err <= TOL, (S, W, err)


@pytest.mark.parametrize("S,W", [(4, 8), (8, 8), (16, 4)])
def test_gqa_split_k_batch8_n32k(S, W, merge_mode):
    """q [256, 128], K, V [64, 32768, 128] (1.07 GB of KV): 16 sampled KV rows
    (their 64 query heads) against the float64 oracle, all 256 heads against
    fp32 PyTorch on the GPU."""
    B, Hq, Hkv, N, D = 8, 32, 8, 32768, 128
    G = Hq // Hkv
    g = torch.Generator(device=DEV).manual_seed(32768)
    q = torch.randn(B * Hq, D, device=DEV, generator=g).half()
    K = torch.randn(B * Hkv, N, D, device=DEV, generator=g).half()
    V = torch.randn(B * Hkv, N, D, device=DEV, generator=g).half()
    o = run_sk(q, K, V, S, W)
    ref_full = torch.empty(B * Hq, D, device=DEV)
    for r0 in range(0, B * Hkv, 8):  # 8 KV rows (32 heads) at a time
        Kf = K[r0:r0 + 8].float().repeat_interleave(G, 0)
        Vf = V[r0:r0 + 8].float().repeat_interleave(G, 0)
        ref_full[r0 * G:(r0 + 8) * G] = ref_fp32(q[r0 * G:(r0 + 8) * G], Kf, Vf)
    kv_rows = sample_rows(B * Hkv, seed=7)
    heads = [r * G + j for r in kv_rows for j in range(G)]
    ref_rows = oracle.gqa_attention(q[heads].cpu().numpy().reshape(1, -1, D),
                                    K[kv_rows].cpu().numpy()[None], V[kv_rows].cpu().numpy()[None])[0]
    check(o, ref_full, ref_rows, heads)


@pytest.mark.parametrize("fmt,D", [("fp16", 64), ("fp16", 128), ("int8", 128), ("int8", 64), ("int4", 128), ("int4", 64)])
@pytest.mark.parametrize("per_cu", [1.5, 3.0])
def test_mha_rows_between_one_and_four_per_cu(fmt, D, per_cu):
    """Unsplit calls with more rows than CUs but fewer than four per CU: rows under
    256 bytes run 4-wave workgroups there, 256-byte rows 8-wave ones (the
    single-block entry points' wave-count rule); both against the references."""
    B = int(per_cu * fq.cu_count())
    N, W = 1024, 8
    g = torch.Generator(device=DEV).manual_seed(B + D)
    q = torch.randn(B, D, device=DEV, generator=g).half()
    rows = sample_rows(B, seed=B + D)
    if fmt == "fp16":
        K = torch.randn(B, N, D, device=DEV, generator=g).half()
        V = torch.randn(B, N, D, device=DEV, generator=g).half()
        out = fq.decode_attn_fp16_mw(q, K, V, W)
        ref_full = ref_fp32(q, K.float(), V.float())
        Kr, Vr = K[rows].float().cpu().numpy(), V[rows].float().cpu().numpy()
    else:
        quantize = fq.quantize_int8_per_token if fmt == "int8" else fq.quantize_int4_per_token
        Kq, Ks = quantize(torch.randn(B, N, D, device=DEV, generator=g))
        Vq, Vs = quantize(torch.randn(B, N, D, device=DEV, generator=g))
        if fmt == "int8":
            out = fq.decode_attn_int8_mw(q, Kq, Vq, Ks, Vs, W)
            deq, deq_gpu = oracle.dequant_int8, (lambda x, s: x.float() * s.float()[..., None])
        else:
            from fqkv_decode import quant
            out = fq.decode_attn_int4(q, Kq, Vq, Ks, Vs, W)
            deq, deq_gpu = oracle.dequant_int4, quant.dequant_int4
        ref_full = ref_fp32(q, deq_gpu(Kq, Ks), deq_gpu(Vq, Vs))
        Kr = deq(Kq[rows].cpu().numpy(), Ks[rows].cpu().numpy())
        Vr = deq(Vq[rows].cpu().numpy(), Vs[rows].cpu().numpy())
    assert out.shape == (B, D) and out.dtype == torch.float16
    check(out, ref_full, oracle.attention(q[rows].cpu().numpy(), Kr, Vr), rows)
