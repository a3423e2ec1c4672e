"""Benchmark of the GQA split-K fp16 decode path on one MI355X.

Workload (the headline metric's configuration): ``gqa_sk_fast`` with 32 query
heads / 8 KV heads, N = 16384 cached tokens, head_dim 128, batch 1, fp16
q/K/V drawn N(0,1), fp32 split scratch preallocated. One step = one call of
the entry point on the next of ``--kv-sets``
distinct KV caches, so successive steps stream >= 512 MiB of distinct KV and
the 256 MB Infinity Cache cannot serve them. A call is one kernel launch:
the partial kernel with the split merge fused in. Inputs are resident in HBM
before timing starts.

Reported: ``value`` = algorithmic bytes per call / time per call in GB/s
(bytes = 4*Hkv*N*D (K+V fp16) + 4*Hq*D (q in, o out), i.e. 67,125,248),
whole-call loop timing like the reference's flashinfer_looptimed.py:34-44.
``roofline`` covers the dominant kernel. By default a call is ONE kernel
(partial kernel with the split merge fused in), so its average duration is
the loop time per call, taken with HIP events on the stream the kernel runs
on (PyTorch's current stream). With --merge two-kernel the partial kernel is
timed per launch with HIP events recorded just around it. ``cpu_baseline``
times the reference's CPU path (repeat_interleave + scaled_dot_product_attention
on CPU tensors, every host thread) on a bounded sample of the same workload.
Further keys carry the reference's other benchmark shapes: MHA fp16 / int8 /
int4 at B=2048, N=4096, D=128; split-K at B=8, N=32768; the launch floor; the
reference's primary split-K table (D in {64, 128} x N in {512 .. 32768}, each
point swept over S/W/CW under the correctness gate); the reference's other
benchmark rows at D=128 (MHA B=32 N=512; fp16 / int8 / int4 MHA at B=8 and 256; GQA at
N=512, D=64 against repeat_kv + MHA; int8 / int4 split-K at the headline
shape); and the reference's D=64 tables with its A100 numbers alongside.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--S S --W W --CW CW]
       python bench.py --sweep      (tuning table on stderr, then the JSON line)
       python bench.py --suite FILE (secondary configurations as JSON lines in
                                     FILE and a table on stderr, then the JSON line)
       python bench.py --timeline [--n-tokens N --S S]
                                    (where a call's time goes: host issue, loop and
                                     graph-replay cost per call, and the kernel's
                                     per-stage clock stamps; one JSON line)
"""

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_PARENT = os.path.join(ROOT, "fused-quantized-kv-decode-attention_amd")
sys.path.insert(0, PKG_PARENT)

HQ, HKV, N, D = 32, 8, 16384, 128
PEAK_HBM_GBS = 8000.0
REF_A100_GBS = 519.0  # reference, D=128 N=16384 (benchmarks/flashinfer_looptimed.json:138-149)
METRIC = "achieved HBM GB/s + us/call, GQA split-K fp16 decode, 32q/8kv heads, N=16K, D=128"


def alg_bytes(hq=HQ, hkv=HKV, n=None, d=D):
    n = N if n is None else n
    return 4 * hkv * n * d + 4 * hq * d


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class HipEvents:
    """hipEvent_t handles from the HIP runtime PyTorch already loaded."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so.7")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self, n):
        out = []
        for _ in range(n):
            h = ctypes.c_void_p()
            rc = self.lib.hipEventCreate(ctypes.byref(h))
            if rc != 0:
                raise RuntimeError("hipEventCreate failed: %d" % rc)
            out.append(h.value)
        return out

    def elapsed_ms(self, a, b):
        t = ctypes.c_float()
        rc = self.lib.hipEventElapsedTime(ctypes.byref(t), a, b)
        if rc != 0:
            raise RuntimeError("hipEventElapsedTime failed: %d" % rc)
        return t.value

    def destroy(self, evs):
        for e in evs:
            self.lib.hipEventDestroy(e)


def default_splits(cus):
    # one 8-wave workgroup per CU across the 8 KV heads
    return max(1, cus // HKV)


def make_sets(torch, nsets, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(HQ, D, device="cuda", generator=g).half()
    Ks, Vs = [], []
    for _ in range(nsets):
        Ks.append(torch.randn(HKV, N, D, device="cuda", generator=g).half())
        Vs.append(torch.randn(HKV, N, D, device="cuda", generator=g).half())
    return q, Ks, Vs


def gate(torch, fq, q, K, V, S, W, CW):
    """Correctness gate before timing: fp32 torch reference on the GPU, max-abs <= 2e-3."""
    mp = torch.empty(HQ, S, device="cuda")
    lp = torch.empty(HQ, S, device="cuda")
    op = torch.empty(HQ, S, D, device="cuda")
    o = torch.empty(HQ, D, device="cuda", dtype=torch.float16)
    fq.gqa_sk_fast(q, K, V, mp, lp, op, o, S, W, CW)
    G = HQ // HKV
    Kf = K.float().repeat_interleave(G, 0)
    Vf = V.float().repeat_interleave(G, 0)
    s = torch.bmm(Kf, q.float().unsqueeze(2)).squeeze(2) / math.sqrt(D)
    ref = torch.bmm(torch.softmax(s, dim=1).unsqueeze(1), Vf).squeeze(1)
    return float((o.float() - ref).abs().max())


# Warm-up calls queued after the synchronisation that precedes a timed region: the GPU is running
# real calls when the start event is queued, so the timed calls follow back to back instead of
# starting on an idle GPU behind the host's launch latency of the first one (about 10 us through
# Python, half a microsecond per call when only 20 calls are timed). They lie outside the region.
LEAD_CALLS = 4

# A loop timed within ~0.25 s of allocating fresh device memory (multi-GB inputs through PyTorch's
# caching allocator) reads 3-5 % slow on MI355X, and a plain 1 GiB streaming read does too; 0.25 s
# later the same loop on the same buffers is back to its steady rate (int4 MHA B 2048, N 4096,
# D 128: 176 -> 169 us; headline 14.5 -> 13.9 us after a 4 GB allocation). So every timed row
# lets SETTLE_S pass between allocating its inputs and its warm-up calls. The headline waits idle
# (its warm-up is the --warmup count alone); the other rows, whose warm-up is this file's choice,
# spend the time launching the streaming-read probe over a 32 MiB buffer (128 workgroups, a grid
# the stream ceiling does not use, so kernel traces tell the two apart), since after an idle wait
# the clocks are down and a host-bound loop of small calls (GQA B 1, N 512) reads up to 45 % slow.
SETTLE_S = 0.4
_SETTLE_BUF = []


def settle(torch, fq=None):
    torch.cuda.synchronize()
    if fq is None:
        time.sleep(SETTLE_S)
        return
    if not _SETTLE_BUF:
        _SETTLE_BUF.append(torch.ones(32 << 20, dtype=torch.uint8, device="cuda"))
    t_end = time.perf_counter() + SETTLE_S
    while time.perf_counter() < t_end:
        for _ in range(100):
            fq._ext._probe_stream_read(_SETTLE_BUF[0], 128)
        torch.cuda.synchronize()


def time_calls(torch, fq, q, Ks, Vs, S, W, CW, steps, warmup):
    mp = torch.empty(HQ, S, device="cuda")
    lp = torch.empty(HQ, S, device="cuda")
    op = torch.empty(HQ, S, D, device="cuda")
    o = torch.empty(HQ, D, device="cuda", dtype=torch.float16)
    n = len(Ks)
    for i in range(warmup):
        fq.gqa_sk_fast(q, Ks[i % n], Vs[i % n], mp, lp, op, o, S, W, CW)
    torch.cuda.synchronize()
    for i in range(LEAD_CALLS):
        fq.gqa_sk_fast(q, Ks[i % n], Vs[i % n], mp, lp, op, o, S, W, CW)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(steps):
        fq.gqa_sk_fast(q, Ks[i % n], Vs[i % n], mp, lp, op, o, S, W, CW)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps  # ms per call


def time_partial(torch, fq, q, Ks, Vs, S, W, CW, steps, ev):
    """Average duration of the partial kernel: events recorded just before and after
    each partial launch on the stream it runs on (PyTorch's current stream)."""
    mp = torch.empty(HQ, S, device="cuda")
    lp = torch.empty(HQ, S, device="cuda")
    op = torch.empty(HQ, S, D, device="cuda")
    o = torch.empty(HQ, D, device="cuda", dtype=torch.float16)
    n = len(Ks)
    evs = ev.create(2 * steps)
    for i in range(min(steps, 50)):
        fq.gqa_sk_fast(q, Ks[i % n], Vs[i % n], mp, lp, op, o, S, W, CW)
    torch.cuda.synchronize()
    for i in range(steps):
        fq._ext._gqa_sk_fast_timed(q, Ks[i % n], Vs[i % n], mp, lp, op, o, S, W, CW, evs[2 * i], evs[2 * i + 1])
    torch.cuda.synchronize()
    durs = [ev.elapsed_ms(evs[2 * i], evs[2 * i + 1]) for i in range(steps)]
    ev.destroy(evs)
    durs.sort()
    return sum(durs) / len(durs), durs[len(durs) // 2]


def read_traffic():
    """HBM bytes per partial launch from the committed rocprofv3 PMC summary, if present."""
    path = os.path.join(ROOT, "profiles", "decode_partial_gqa_n16k_d128_pmc.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return float(line.split(":", 1)[1].strip())
            except ValueError:
                return None
    return None


def cpu_baseline(budget_s=12.0):
    """The reference's CPU path on the metric workload, on the host's cores.

    What the reference's tests evaluate as the expected result of a GQA
    split-K call (tests/test_kernels.py:68-69): the KV heads repeated to the
    query heads with repeat_interleave, then F.scaled_dot_product_attention,
    here on CPU tensors in the tensors' own dtype (fp16 q, K, V drawn from a
    seeded CPU generator). torch uses every host thread; 5 warm-up calls, then
    calls until at least 20 and about budget_s seconds, timed one by one with
    time.perf_counter; the median is reported. The float64 oracle checks the
    result once (max-abs 2e-3): it is the checker, not the thing timed."""
    import numpy as np
    import torch
    import torch.nn.functional as F

    sys.path.insert(0, ROOT)
    import oracle

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    G = HQ // HKV
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, HQ, 1, D, generator=g).half()
    K = torch.randn(1, HKV, N, D, generator=g).half()
    V = torch.randn(1, HKV, N, D, generator=g).half()

    def call():
        return F.scaled_dot_product_attention(q, K.repeat_interleave(G, 1), V.repeat_interleave(G, 1))

    out = call()
    ref = oracle.gqa_attention(q.numpy()[:, :, 0], K.numpy(), V.numpy())
    err = float(np.abs(out[:, :, 0].float().numpy().astype(np.float64) - ref).max())
    for _ in range(4):
        call()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 20 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        call()
        times.append(time.perf_counter() - t0)
        if len(times) >= 2000:
            break
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": round(alg_bytes() / med / 1e9, 3),
        "unit": "GB/s",
        "us_per_call": round(med * 1e6, 1),
        "cores": cores,
        "threads": torch.get_num_threads(),
        "kind": "port",
        "max_abs_err_vs_oracle": err,
        "sample": "median of %d whole calls (after 5 warm-ups) of the workload (32q/8kv heads, N=16384, D=128, fp16): "
                  "repeat_interleave + F.scaled_dot_product_attention on CPU tensors (tests/test_kernels.py:68-69), "
                  "%d torch threads, %.1f s" % (len(times), torch.get_num_threads(), sum(times)),
    }


def stream_ceiling(torch, fq, steps, warmup, nsets=10):
    """The headline's streaming ceiling: loop time of a kernel that only reads
    the bytes one call streams (K + V, 64 MiB), cycling nsets distinct
    buffers like the headline (fqkv_probe_stream_read: one contiguous span
    per workgroup, 16-byte streaming loads, best of 256, 512 and 1024
    workgroups of 256 threads)."""
    nb = 4 * HKV * N * D
    bufs = [torch.full((nb,), 1, dtype=torch.uint8, device="cuda") for _ in range(nsets)]
    settle(torch, fq)
    best = None
    for blocks in (256, 512, 1024):
        ms = _loop_ms(torch, lambda i: fq._ext._probe_stream_read(bufs[i], blocks), nsets, steps, warmup)
        if best is None or ms < best[0]:
            best = (ms, blocks)
    ms, blocks = best
    del bufs
    torch.cuda.empty_cache()
    return {"us_per_call": round(ms * 1e3, 3), "GBps": round(nb / ms / 1e6, 1),
            "frac_of_peak": round(nb / ms / 1e6 / PEAK_HBM_GBS, 4), "bytes_per_call": nb, "blocks": blocks,
            "kernel": "stream_read_kernel (read-only, 16-byte streaming loads)"}


def _frac(nbytes, ms):
    return round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4)


def secondary_results(torch, fq, steps=400, warmup=50):
    """The reference's other benchmark shapes, in the driver's line.

    * mha_b2048_n4096_d128: fp16 / int8 / int4 MHA at batch*heads 2048,
      N 4096, D 128 (the precision benchmark, benchmarks/standalone_quant.json
      at D 64 in the reference), W 8; one input set per format (4.3 / 2.2 /
      1.1 GB, each beyond the 256 MB Infinity Cache);
    * splitk_b8_n32768_d128: gqa_sk_fast at batch 8 (q [256, 128],
      K, V [64, 32768, 128], 1.07 GB of KV), best of S in {4, 8, 16} x W in {4, 8};
    * launch_floor_us: gqa_sk_fast on N = 1, D = 64, S = 1, W 2, CW 4 in a loop
      (flashinfer_looptimed.py:47-56's estimate of the per-call floor).
    Loop-timed like the headline; each row gated against fp32 PyTorch on the
    GPU (max-abs <= 2e-3 on 64 sampled rows or heads) before timing."""
    res = {}
    B, Nm, Dm, W = 2048, 4096, 128, 8
    g = torch.Generator(device="cuda").manual_seed(21)
    q = torch.randn(B, Dm, device="cuda", generator=g).half()
    rows = torch.arange(0, B, B // 64, device="cuda")
    mha = {}
    for fmt in ("fp16", "int8", "int4"):
        Kx = torch.randn(B, Nm, Dm, device="cuda", generator=g)
        Vx = torch.randn(B, Nm, Dm, device="cuda", generator=g)
        if fmt == "fp16":
            K, V = Kx.half(), Vx.half()
            del Kx, Vx
            fn = lambda: fq.decode_attn_fp16_mw(q, K, V, W)
            Kf, Vf = K[rows].float(), V[rows].float()
            nbytes = B * (4 * Nm * Dm + 4 * Dm)
        else:
            quantize = fq.quantize_int8_per_token if fmt == "int8" else fq.quantize_int4_per_token
            (K, Ks), (V, Vs) = quantize(Kx), quantize(Vx)
            del Kx, Vx
            if fmt == "int8":
                fn = lambda: fq.decode_attn_int8_mw(q, K, V, Ks, Vs, W)
                Kf, Vf = K[rows].float() * Ks[rows].float()[..., None], V[rows].float() * Vs[rows].float()[..., None]
                nbytes = B * (2 * Nm * Dm + 4 * Nm + 4 * Dm)
            else:
                from fqkv_decode import quant
                fn = lambda: fq.decode_attn_int4(q, K, V, Ks, Vs, W)
                Kf, Vf = quant.dequant_int4(K[rows], Ks[rows]), quant.dequant_int4(V[rows], Vs[rows])
                nbytes = B * (Nm * Dm + 4 * Nm + 4 * Dm)
        err = float((fn()[rows].float() - _ref_mha(torch, q[rows], Kf, Vf)).abs().max())
        if err > 2e-3:
            raise RuntimeError("secondary gate failed: MHA %s B=2048 max-abs %.3e" % (fmt, err))
        settle(torch, fq)
        ms = _loop_ms(torch, lambda i: fn(), 1, steps, warmup)
        mha[fmt] = {"us_per_call": round(ms * 1e3, 2), "GBps": round(nbytes / ms / 1e6, 1), "frac": _frac(nbytes, ms),
                    "alg_bytes": nbytes, "gate_max_abs_err": err}
        log("mha %s B=2048 N=4096 D=128: %8.2f us  %7.1f GB/s  err %.2e" % (fmt, ms * 1e3, nbytes / ms / 1e6, err))
        del K, V, Kf, Vf
        torch.cuda.empty_cache()
    mha["int8_speedup_vs_fp16"] = round(mha["fp16"]["us_per_call"] / mha["int8"]["us_per_call"], 3)
    mha["int4_speedup_vs_fp16"] = round(mha["fp16"]["us_per_call"] / mha["int4"]["us_per_call"], 3)
    res["mha_b2048_n4096_d128"] = mha

    Bs, Hq, Hkv, Ns, Ds = 8, HQ, HKV, 32768, 128
    G = Hq // Hkv
    g = torch.Generator(device="cuda").manual_seed(22)
    qs = torch.randn(Bs * Hq, Ds, device="cuda", generator=g).half()
    Ksk = torch.randn(Bs * Hkv, Ns, Ds, device="cuda", generator=g).half()
    Vsk = torch.randn(Bs * Hkv, Ns, Ds, device="cuda", generator=g).half()
    kv_rows = list(range(0, Bs * Hkv, Bs * Hkv // 16))
    heads = torch.tensor([r * G + j for r in kv_rows for j in range(G)], device="cuda")
    ref = _ref_mha(torch, qs[heads], Ksk[kv_rows].float().repeat_interleave(G, 0),
                   Vsk[kv_rows].float().repeat_interleave(G, 0))
    nbytes = Bs * (4 * Hkv * Ns * Ds + 4 * Hq * Ds)
    settle(torch, fq)
    best = None
    for S in (4, 8, 16):
        for Wk in (4, 8):
            mp = torch.empty(Bs * Hq, S, device="cuda")
            lp = torch.empty(Bs * Hq, S, device="cuda")
            op = torch.empty(Bs * Hq, S, Ds, device="cuda")
            o = torch.empty(Bs * Hq, Ds, device="cuda", dtype=torch.float16)
            fn = lambda i: fq.gqa_sk_fast(qs, Ksk, Vsk, mp, lp, op, o, S, Wk, 8)
            fn(0)
            err = float((o[heads].float() - ref).abs().max())
            if err > 2e-3:
                raise RuntimeError("secondary gate failed: split-K B=8 S%d W%d max-abs %.3e" % (S, Wk, err))
            ms = _loop_ms(torch, fn, 1, steps, warmup)
            if best is None or ms < best[0]:
                best = (ms, S, Wk, err)
    ms, S, Wk, err = best
    res["splitk_b8_n32768_d128"] = {"us_per_call": round(ms * 1e3, 2), "GBps": round(nbytes / ms / 1e6, 1),
                                    "frac": _frac(nbytes, ms), "alg_bytes": nbytes, "S": S, "W": Wk, "CW": 8,
                                    "gate_max_abs_err": err}
    log("split-K B=8 N=32768 D=128 S%d W%d: %8.2f us  %7.1f GB/s  err %.2e" % (S, Wk, ms * 1e3, nbytes / ms / 1e6, err))
    del Ksk, Vsk
    torch.cuda.empty_cache()

    q1 = torch.randn(HQ, 64, device="cuda").half()
    K1 = torch.randn(HKV, 1, 64, device="cuda").half()
    V1 = torch.randn(HKV, 1, 64, device="cuda").half()
    mp1 = torch.empty(HQ, 1, device="cuda")
    lp1 = torch.empty(HQ, 1, device="cuda")
    op1 = torch.empty(HQ, 1, 64, device="cuda")
    o1 = torch.empty(HQ, 64, device="cuda", dtype=torch.float16)
    ms = _loop_ms(torch, lambda i: fq.gqa_sk_fast(q1, K1, V1, mp1, lp1, op1, o1, 1, 2, 4), 1, 2000, 200)
    res["launch_floor_us"] = round(ms * 1e3, 3)
    log("launch floor (gqa_sk_fast N=1 D=64 S=1): %.3f us per call" % (ms * 1e3))
    return res


# ---------------------------------------------------------------------------
# Secondary configurations (the reference's other benchmarks, on MI355X).
# Each is loop-timed like the headline: warm-up, then `steps` calls between
# HIP events on the current stream, cycling through enough distinct input sets
# that >= 1 GiB of KV streams per cycle (the 256 MB Infinity Cache cannot hold
# it). Algorithmic bytes count compact K/V, scales, q and o only.

def _nsets(bytes_per_set, cap=64):
    return max(1, min(cap, -(-(1 << 30) // bytes_per_set)))


def _loop_ms(torch, fn, nsets, steps, warmup):
    for i in range(warmup):
        fn(i % nsets)
    torch.cuda.synchronize()
    for i in range(LEAD_CALLS):
        fn(i % nsets)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(steps):
        fn(i % nsets)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def _row(name, cfg, ms, nbytes, err=None, **extra):
    r = {"bench": name, "config": cfg, "us_per_call": round(ms * 1e3, 3),
         "alg_bytes": nbytes, "GBps": round(nbytes / ms / 1e6, 1),
         "frac_of_8TBps": round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4)}
    if err is not None:
        r["max_abs_err_vs_fp32"] = err
    r.update(extra)
    return r


def _ref_mha(torch, q, Kf, Vf):
    """fp32 softmax(q K^T / sqrt(D)) V on the GPU, q [B, D], K/V [B, N, D] fp32."""
    D = q.shape[-1]
    s = torch.bmm(Kf, q.float().unsqueeze(2)).squeeze(2) / math.sqrt(D)
    return torch.bmm(torch.softmax(s, dim=1).unsqueeze(1), Vf).squeeze(1)


# The reference's A100 results at its own precision shape (D 64, N 4096, W 8): fp16 / int8 / int4
# ms per call (benchmarks/standalone_quant.json:6-34; per-call events, synchronised).
REF_QUANT_D64_MS = {8: (0.2263, 0.2478, 0.2662), 256: (0.4792, 0.4864, 0.4915), 2048: (2.0951, 1.6814, 1.5585)}


def suite_mha_quant(torch, fq, steps, warmup, rows, shapes=None, formats=("fp16", "int8", "int4", "fp8")):
    """fp16 / int8 / int4 MHA decode at B in {8, 256, 2048}, N=4096, W=8, at D=128 and at the
    reference's own D=64 (its A100 numbers alongside); fp8 (no counterpart in the reference)
    through decode_attn_gqa_fp8 with one query head per KV head; shapes: (D, B) pairs to run
    instead."""
    from fqkv_decode import quant
    N, W = 4096, 8
    if shapes is None:
        shapes = [(128, b) for b in (8, 256, 2048)] + [(64, b) for b in (8, 256, 2048)]
    for Dm, B in shapes:
        g = torch.Generator(device="cuda").manual_seed(1)
        q = torch.randn(B, Dm, device="cuda", generator=g).half()
        per = {"fp16": 2 * B * N * Dm * 2, "int8": 2 * B * N * Dm + 4 * B * N, "int4": B * N * Dm + 4 * B * N,
               "fp8": 2 * B * N * Dm + 4 * B * N}
        for fmt in formats:
            ns = _nsets(per[fmt])
            sets = []
            err = None
            for k in range(ns):
                Kx = torch.randn(B, N, Dm, device="cuda", generator=g)
                Vx = torch.randn(B, N, Dm, device="cuda", generator=g)
                if fmt == "fp16":
                    Kh, Vh = Kx.half(), Vx.half()
                    sets.append((Kh, Vh))
                    if k == 0:
                        Kf, Vf = Kh.float(), Vh.float()
                elif fmt == "int8":
                    Kq, Ks = quant.quant_int8_per_token(Kx)
                    Vq, Vs = quant.quant_int8_per_token(Vx)
                    sets.append((Kq, Vq, Ks, Vs))
                    if k == 0:
                        Kf, Vf = quant.dequant_int8(Kq, Ks), quant.dequant_int8(Vq, Vs)
                elif fmt == "int4":
                    Kq, Ks = quant.quant_int4_per_token(Kx)
                    Vq, Vs = quant.quant_int4_per_token(Vx)
                    sets.append((Kq, Vq, Ks, Vs))
                    if k == 0:
                        Kf, Vf = quant.dequant_int4(Kq, Ks), quant.dequant_int4(Vq, Vs)
                else:
                    (Kq, Ks), (Vq, Vs) = fq.quantize_fp8_per_token(Kx), fq.quantize_fp8_per_token(Vx)
                    sets.append((Kq.view(B, 1, N, Dm), Vq.view(B, 1, N, Dm), Ks.view(B, 1, N), Vs.view(B, 1, N)))
                    if k == 0:
                        Kf, Vf = quant.dequant_fp8(Kq, Ks), quant.dequant_fp8(Vq, Vs)
                del Kx, Vx
            if fmt == "fp16":
                fn = lambda i: fq.decode_attn_fp16_mw(q, sets[i][0], sets[i][1], W)
                nbytes = B * (4 * N * Dm + 4 * Dm)
            elif fmt == "int8":
                fn = lambda i: fq.decode_attn_int8_mw(q, sets[i][0], sets[i][1], sets[i][2], sets[i][3], W)
                nbytes = B * (2 * N * Dm + 4 * N + 4 * Dm)
            elif fmt == "int4":
                fn = lambda i: fq.decode_attn_int4(q, sets[i][0], sets[i][1], sets[i][2], sets[i][3], W)
                nbytes = B * (N * Dm + 4 * N + 4 * Dm)
            else:
                q1 = q.view(B, 1, Dm)
                fn = lambda i: fq.decode_attn_gqa_fp8(q1, sets[i][0], sets[i][1], sets[i][2], sets[i][3], W).view(B, Dm)
                nbytes = B * (2 * N * Dm + 4 * N + 4 * Dm)
            o = fn(0)
            ref = _ref_mha(torch, q, Kf, Vf)
            err = float((o.float() - ref).abs().max())
            del Kf, Vf, ref
            settle(torch, fq)
            ms = _loop_ms(torch, fn, ns, steps, warmup)
            extra = {}
            if Dm == 64 and fmt != "fp8":
                extra = {"ref_a100_us": REF_QUANT_D64_MS[B][("fp16", "int8", "int4").index(fmt)] * 1e3}
            rows.append(_row("mha_" + fmt, {"B": B, "N": N, "D": Dm, "W": W, "sets": ns}, ms, nbytes, err, **extra))
            log("%-10s B=%-5d N=%d D=%d  %9.2f us  %7.1f GB/s  err %.2e" % (fmt, B, N, Dm, ms * 1e3, nbytes / ms / 1e6, err))
            del sets
            torch.cuda.empty_cache()


# The reference's A100 results at its own GQA shape (Hq 32, Hkv 8, D 64, N 4096, W 8):
# GQA-aware ms and repeat_kv + MHA ms per batch (benchmarks/gqa_aware.json:2-24).
REF_GQA_N4096_MS = {1: (0.2417, 0.5898), 4: (0.4588, 0.8735), 16: (0.4506, 1.6148)}


def suite_gqa(torch, fq, steps, warmup, rows, shapes=None):
    """decode_attn_gqa vs repeat_kv + MHA kernel: Hq=32, Hkv=8, D=64, B in {1,4,16}, at N=512
    and at the reference's own N=4096 (its A100 numbers alongside); shapes: (N, B) pairs to run
    instead."""
    Hq, Hkv, Dg, W = 32, 8, 64, 8
    G = Hq // Hkv
    if shapes is None:
        shapes = [(512, b) for b in (1, 4, 16)] + [(4096, b) for b in (1, 4, 16)]
    for N, B in shapes:
        g = torch.Generator(device="cuda").manual_seed(2)
        per = 2 * B * Hkv * N * Dg * 2
        ns = _nsets(per)
        q = torch.randn(B, Hq, Dg, device="cuda", generator=g).half()
        sets = [(torch.randn(B, Hkv, N, Dg, device="cuda", generator=g).half(),
                 torch.randn(B, Hkv, N, Dg, device="cuda", generator=g).half()) for _ in range(ns)]
        K0, V0 = sets[0]
        Kf = K0.float().repeat_interleave(G, 1).reshape(B * Hq, N, Dg)
        Vf = V0.float().repeat_interleave(G, 1).reshape(B * Hq, N, Dg)
        ref = _ref_mha(torch, q.reshape(B * Hq, Dg), Kf, Vf)
        o = fq.decode_attn_gqa(q, K0, V0, W)
        err = float((o.reshape(B * Hq, Dg).float() - ref).abs().max())
        nbytes = B * (4 * Hkv * N * Dg + 4 * Hq * Dg)
        settle(torch, fq)
        ms = _loop_ms(torch, lambda i: fq.decode_attn_gqa(q, sets[i][0], sets[i][1], W), ns, steps, warmup)
        qf = q.reshape(B * Hq, Dg)

        def expand(i):
            Ke = sets[i][0].repeat_interleave(G, 1).reshape(B * Hq, N, Dg)
            Ve = sets[i][1].repeat_interleave(G, 1).reshape(B * Hq, N, Dg)
            return fq.decode_attn_fp16_mw(qf, Ke, Ve, W)

        ms_x = _loop_ms(torch, expand, ns, steps, warmup)
        extra = {}
        if N == 4096:
            extra = {"ref_a100_gqa_us": REF_GQA_N4096_MS[B][0] * 1e3, "ref_a100_expand_us": REF_GQA_N4096_MS[B][1] * 1e3}
        rows.append(_row("gqa", {"B": B, "Hq": Hq, "Hkv": Hkv, "N": N, "D": Dg, "W": W, "sets": ns}, ms, nbytes, err,
                         expand_mha_us=round(ms_x * 1e3, 3), speedup_vs_expand=round(ms_x / ms, 3), **extra))
        log("gqa       B=%-3d N=%d D=%d  %8.2f us (repeat_kv + MHA %8.2f us, %.2fx)  err %.2e"
            % (B, N, Dg, ms * 1e3, ms_x * 1e3, ms_x / ms, err))
        del sets, Kf, Vf


def suite_splitk(torch, fq, steps, warmup, rows):
    """gqa_sk_fast over N in {512 .. 32K}, D in {64, 128}, best of an S/W sweep; plus B=8, N=32K, D=128."""
    Hq, Hkv = 32, 8
    G = Hq // Hkv
    cases = [(1, N, Dd) for Dd in (64, 128) for N in (512, 1024, 2048, 4096, 8192, 16384, 32768)]
    cases.append((8, 32768, 128))
    for B, N, Dd in cases:
        g = torch.Generator(device="cuda").manual_seed(3)
        per = 2 * B * Hkv * N * Dd * 2
        ns = _nsets(per)
        q = torch.randn(B * Hq, Dd, device="cuda", generator=g).half()
        sets = [(torch.randn(B * Hkv, N, Dd, device="cuda", generator=g).half(),
                 torch.randn(B * Hkv, N, Dd, device="cuda", generator=g).half()) for _ in range(ns)]
        K0, V0 = sets[0]
        ref = _ref_mha(torch, q, K0.float().repeat_interleave(G, 0), V0.float().repeat_interleave(G, 0))
        nbytes = B * (4 * Hkv * N * Dd + 4 * Hq * Dd)
        settle(torch, fq)
        best = None
        for S in (1, 2, 4, 8, 16, 32, 64, 128):
            if S > max(1, N // 16):
                continue
            for W in (4, 8):
                mp = torch.empty(B * Hq, S, device="cuda")
                lp = torch.empty(B * Hq, S, device="cuda")
                op = torch.empty(B * Hq, S, Dd, device="cuda")
                o = torch.empty(B * Hq, Dd, device="cuda", dtype=torch.float16)
                fn = lambda i: fq.gqa_sk_fast(q, sets[i][0], sets[i][1], mp, lp, op, o, S, W, 8)
                fn(0)
                err = float((o.float() - ref).abs().max())
                if err > 2e-3:
                    log("split-K B=%d N=%d D=%d S%d W%d failed the gate: %.2e" % (B, N, Dd, S, W, err))
                    continue
                ms = _loop_ms(torch, fn, ns, max(50, steps // 4), max(10, warmup // 4))
                if best is None or ms < best[0]:
                    best = (ms, S, W, err)
        ms, S, W, err = best
        # re-time the winner with the full step count
        mp = torch.empty(B * Hq, S, device="cuda")
        lp = torch.empty(B * Hq, S, device="cuda")
        op = torch.empty(B * Hq, S, Dd, device="cuda")
        o = torch.empty(B * Hq, Dd, device="cuda", dtype=torch.float16)
        ms = _loop_ms(torch, lambda i: fq.gqa_sk_fast(q, sets[i][0], sets[i][1], mp, lp, op, o, S, W, 8), ns, steps, warmup)
        rows.append(_row("gqa_sk_fast", {"B": B, "Hq": Hq, "Hkv": Hkv, "N": N, "D": Dd, "S": S, "W": W, "CW": 8,
                                         "sets": ns}, ms, nbytes, err))
        log("split-K   B=%d N=%-6d D=%-3d S%-3d W%d  %8.2f us  %7.1f GB/s  err %.2e" % (B, N, Dd, S, W, ms * 1e3, nbytes / ms / 1e6, err))
        del sets, ref


def suite_mha_small(torch, fq, steps, warmup, rows):
    """fp16 MHA, 32 heads, N=512, D=128 (the reference's CPU-runnable case)."""
    B, N, Dm, W = 32, 512, 128, 8
    g = torch.Generator(device="cuda").manual_seed(4)
    ns = _nsets(2 * B * N * Dm * 2)
    q = torch.randn(B, Dm, device="cuda", generator=g).half()
    sets = [(torch.randn(B, N, Dm, device="cuda", generator=g).half(),
             torch.randn(B, N, Dm, device="cuda", generator=g).half()) for _ in range(ns)]
    o = fq.decode_attn_fp16_mw(q, sets[0][0], sets[0][1], W)
    err = float((o.float() - _ref_mha(torch, q, sets[0][0].float(), sets[0][1].float())).abs().max())
    nbytes = B * (4 * N * Dm + 4 * Dm)
    settle(torch, fq)
    ms = _loop_ms(torch, lambda i: fq.decode_attn_fp16_mw(q, sets[i][0], sets[i][1], W), ns, steps, warmup)
    rows.append(_row("mha_fp16", {"B": B, "N": N, "D": Dm, "W": W, "sets": ns}, ms, nbytes, err))
    log("mha_fp16  B=%d N=%d D=%d  %8.2f us  %7.1f GB/s  err %.2e" % (B, N, Dm, ms * 1e3, nbytes / ms / 1e6, err))


def suite_splitk_quant(torch, fq, steps, warmup, rows, cases=((1, 16384), (8, 32768)), formats=("int8", "int4", "fp8")):
    """gqa_sk_fast_int8 / _int4 (Hq 32, Hkv 8, D 128) at N 16384 (batch 1) and B 8, N 32768:
    long-context decode over a quantized cache, best of a small S/W sweep; cases: (B, N) pairs,
    formats: a subset of int8, int4, fp8."""
    Hq, Hkv, Dd = 32, 8, 128
    G = Hq // Hkv
    for B, N in cases:
        for fmt in formats:
            g = torch.Generator(device="cuda").manual_seed(5)
            quantize = {"int8": fq.quantize_int8_per_token, "int4": fq.quantize_int4_per_token,
                        "fp8": fq.quantize_fp8_per_token}[fmt]
            per = (B * Hkv * N * Dd if fmt == "int4" else 2 * B * Hkv * N * Dd) + 4 * B * Hkv * N
            ns = _nsets(per)
            q = torch.randn(B * Hq, Dd, device="cuda", generator=g).half()
            sets = []
            for _ in range(ns):
                Kq, Ks = quantize(torch.randn(B * Hkv, N, Dd, device="cuda", generator=g))
                Vq, Vs = quantize(torch.randn(B * Hkv, N, Dd, device="cuda", generator=g))
                sets.append((Kq, Vq, Ks, Vs))
            Kq, Vq, Ks, Vs = sets[0]
            from fqkv_decode import quant
            deq = {"int8": quant.dequant_int8, "int4": quant.dequant_int4, "fp8": quant.dequant_fp8}[fmt]
            Kf, Vf = deq(Kq, Ks), deq(Vq, Vs)
            ref = _ref_mha(torch, q, Kf.repeat_interleave(G, 0), Vf.repeat_interleave(G, 0))
            del Kf, Vf
            f = {"int8": fq.gqa_sk_fast_int8, "int4": fq.gqa_sk_fast_int4, "fp8": fq.gqa_sk_fast_fp8}[fmt]
            nbytes = B * ((Hkv * N * Dd if fmt == "int4" else 2 * Hkv * N * Dd) + 4 * Hkv * N + 4 * Hq * Dd)
            settle(torch, fq)
            best = None
            for S in ((16, 32, 64) if B == 1 else (4, 8, 16)):
                for W in (4, 8):
                    mp = torch.empty(B * Hq, S, device="cuda")
                    lp = torch.empty(B * Hq, S, device="cuda")
                    op = torch.empty(B * Hq, S, Dd, device="cuda")
                    o = torch.empty(B * Hq, Dd, device="cuda", dtype=torch.float16)
                    fn = lambda i: f(q, sets[i][0], sets[i][1], sets[i][2], sets[i][3], mp, lp, op, o, S, W, 8)
                    fn(0)
                    err = float((o.float() - ref).abs().max())
                    if err > 2e-3:
                        log("split-K %s B=%d N=%d S%d W%d failed the gate: %.2e" % (fmt, B, N, S, W, err))
                        continue
                    ms = _loop_ms(torch, fn, ns, max(50, steps // 4), max(10, warmup // 4))
                    if best is None or ms < best[0]:
                        best = (ms, S, W, err)
            ms, S, W, err = best
            rows.append(_row("gqa_sk_fast_" + fmt, {"B": B, "Hq": Hq, "Hkv": Hkv, "N": N, "D": Dd, "S": S, "W": W,
                                                    "CW": 8, "sets": ns}, ms, nbytes, err))
            log("split-K %s B=%d N=%-6d S%-3d W%d  %8.2f us  %7.1f GB/s  err %.2e" % (fmt, B, N, S, W, ms * 1e3,
                                                                                 nbytes / ms / 1e6, err))
            del sets, ref
            torch.cuda.empty_cache()


def suite_paged(torch, fq, steps, warmup, rows):
    """decode_attn_gqa_paged (Hq 32, Hkv 8, D 128, B 8, N 32768) over NHD pages of 16 / 64 / 256
    tokens and head-major (HND) pages of 64 tokens at shuffled page ids, fp16 / bf16 / int8 / int4,
    next to the contiguous decode_attn_gqa[_int8|_int4] (bf16: decode_attn_gqa_strided) over the
    same tokens: what the page indirection costs at a 1 GB cache."""
    B, Hq, Hkv, N, Dd, W = 8, 32, 8, 32768, 128, 8
    G = Hq // Hkv
    g = torch.Generator(device="cuda").manual_seed(11)
    q = torch.randn(B, Hq, Dd, device="cuda", generator=g).half()
    sl = torch.full((B,), N, dtype=torch.int32, device="cuda")
    nsteps, nwarm = max(50, steps // 4), max(10, warmup // 4)
    for fmt in ("fp16", "bf16", "int8", "int4"):
        Xk = torch.randn(B * Hkv, N, Dd, device="cuda", generator=g)
        Xv = torch.randn(B * Hkv, N, Dd, device="cuda", generator=g)
        if fmt in ("fp16", "bf16"):
            dt = torch.float16 if fmt == "fp16" else torch.bfloat16
            K, V, Ks, Vs = Xk.to(dt), Xv.to(dt), None, None
            Kf, Vf = K[:Hkv].float(), V[:Hkv].float()
            entry = fq.decode_attn_gqa if fmt == "fp16" else fq.decode_attn_gqa_strided
            contiguous = lambda: entry(q, K.view(B, Hkv, N, Dd), V.view(B, Hkv, N, Dd), W)
            kvb = 4 * Hkv * N * Dd
        else:
            quantize = fq.quantize_int8_per_token if fmt == "int8" else fq.quantize_int4_per_token
            (K, Ks), (V, Vs) = quantize(Xk), quantize(Xv)
            if fmt == "int8":
                Kf, Vf = K[:Hkv].float() * Ks[:Hkv].float()[..., None], V[:Hkv].float() * Vs[:Hkv].float()[..., None]
            else:
                from fqkv_decode import quant
                Kf, Vf = quant.dequant_int4(K[:Hkv], Ks[:Hkv]), quant.dequant_int4(V[:Hkv], Vs[:Hkv])
            f = fq.decode_attn_gqa_int8 if fmt == "int8" else fq.decode_attn_gqa_int4
            rb = K.shape[-1]
            contiguous = lambda: f(q, K.view(B, Hkv, N, rb), V.view(B, Hkv, N, rb), Ks.view(B, Hkv, N),
                                   Vs.view(B, Hkv, N), W)
            kvb = 2 * Hkv * N * rb + 4 * Hkv * N
        del Xk, Xv
        # sequence 0 against float32 attention over its (dequantized) cache
        ref0 = _ref_mha(torch, q[0], Kf.repeat_interleave(G, 0), Vf.repeat_interleave(G, 0))
        del Kf, Vf
        nbytes = B * (kvb + 4 * Hq * Dd)
        o = contiguous()
        err = float((o[0].float() - ref0).abs().max())
        settle(torch, fq)
        ms = _loop_ms(torch, lambda i: contiguous(), 1, nsteps, nwarm)
        cfg = {"B": B, "Hq": Hq, "Hkv": Hkv, "N": N, "D": Dd, "W": W, "fmt": fmt}
        rows.append(_row("gqa_contiguous_" + fmt, cfg, ms, nbytes, err))
        log("paged suite: contiguous %s        %8.2f us  %7.1f GB/s  err %.2e" % (fmt, ms * 1e3, nbytes / ms / 1e6, err))
        # the same tokens token-major without pages (FlashInfer's NHD, [B, N, Hkv, ...])
        tm = lambda X: X.view(B, Hkv, N, *X.shape[2:]).transpose(1, 2).contiguous()
        Kt, Vt = tm(K), tm(V)
        Kst, Vst = (tm(Ks), tm(Vs)) if Ks is not None else (None, None)
        fn = lambda i: fq.decode_attn_gqa_nhd(q, Kt, Vt, W, Kst, Vst)
        on = fn(0)
        nerr = float((on[0].float() - ref0).abs().max())
        same = bool(torch.equal(on, o))
        settle(torch, fq)
        ms = _loop_ms(torch, fn, 1, nsteps, nwarm)
        rows.append(_row("gqa_nhd_" + fmt, cfg, ms, nbytes, nerr, equal_to_contiguous=same))
        log("paged suite: token-major %s       %8.2f us  %7.1f GB/s  err %.2e  equal to contiguous: %s"
            % (fmt, ms * 1e3, nbytes / ms / 1e6, nerr, same))
        del Kt, Vt, Kst, Vst
        for page, hnd in ((16, False), (64, False), (256, False), (64, True)):
            npb = N // page
            P = B * npb
            perm = torch.randperm(P, device="cuda", generator=g)
            table = perm.view(B, npb).to(torch.int32)

            def pages(X):  # [B*Hkv, N, ...] -> [P, page, Hkv, ...] at page ids perm
                tail = X.shape[2:]
                if hnd:  # head-major pages [P, Hkv, page, ...], handed over as the NHD view
                    Y = X.view(B, Hkv, npb, page, *tail).movedim(1, 2).reshape(P, Hkv, page, *tail)
                    out = torch.empty_like(Y)
                    out[perm] = Y
                    return out.transpose(1, 2)
                Y = X.view(B, Hkv, npb, page, *tail).movedim(1, 3).reshape(P, page, Hkv, *tail)
                out = torch.empty_like(Y)
                out[perm] = Y
                return out

            Kp, Vp = pages(K), pages(V)
            Ksp, Vsp = (pages(Ks), pages(Vs)) if Ks is not None else (None, None)
            fn = lambda i: fq.decode_attn_gqa_paged(q, Kp, Vp, table, sl, N, W, Ksp, Vsp)
            op = fn(0)
            perr = float((op[0].float() - ref0).abs().max())
            same = bool(torch.equal(op, o))
            pb = nbytes + B * npb * 4
            settle(torch, fq)
            ms = _loop_ms(torch, fn, 1, nsteps, nwarm)
            lay = "HND" if hnd else "NHD"
            rows.append(_row("gqa_paged_" + fmt, dict(cfg, page=page, pages=lay), ms, pb, perr,
                             equal_to_contiguous=same))
            log("paged suite: page %-4d %s %s   %8.2f us  %7.1f GB/s  err %.2e  equal to contiguous: %s"
                % (page, lay, fmt, ms * 1e3, pb / ms / 1e6, perr, same))
            del Kp, Vp, Ksp, Vsp
        del K, V, Ks, Vs
        torch.cuda.empty_cache()


def suite_quant(torch, fq, steps, warmup, rows):
    """quantize_int8_per_token / quantize_int4_per_token on [64, 32768, 128] rows (a B 8, Hkv 8,
    N 32768 cache side) from fp16 and fp32 inputs; bytes gated equal to the PyTorch expressions
    of fqkv_decode.quant on the same GPU tensor."""
    from fqkv_decode import quant
    rows_, N_, Dd = 64, 32768, 128
    g = torch.Generator(device="cuda").manual_seed(13)
    X32 = torch.randn(rows_, N_, Dd, device="cuda", generator=g)
    for src in ("fp16", "fp32"):
        X = X32.half() if src == "fp16" else X32
        for fmt in ("int8", "int4"):
            f = fq.quantize_int8_per_token if fmt == "int8" else fq.quantize_int4_per_token
            ref = quant.quant_int8_per_token if fmt == "int8" else quant.quant_int4_per_token
            q, s = f(X)
            rq, rs = ref(X[:4])
            same = bool(torch.equal(q[:4], rq) and torch.equal(s[:4], rs))
            if not same:
                log("quantizer %s from %s: bytes differ from the PyTorch expressions" % (fmt, src))
                continue
            elems = rows_ * N_ * Dd
            nbytes = elems * X.element_size() + (elems if fmt == "int8" else elems // 2) + 2 * rows_ * N_
            settle(torch, fq)
            ms = _loop_ms(torch, lambda i: f(X), 1, max(50, steps // 4), max(10, warmup // 4))
            rows.append(_row("quantize_" + fmt, {"rows": rows_ * N_, "D": Dd, "src": src}, ms, nbytes,
                             equal_to_torch_expressions=same))
            log("quantizer %s from %s: %8.2f us  %7.1f GB/s" % (fmt, src, ms * 1e3, nbytes / ms / 1e6))
        del X
    del X32
    # the paged writer at a serving shape: a 16384-token batch of new fp16 K and V rows (Hkv 8,
    # D 128) into shuffled head-major pages of 16 tokens (4096 pages), every slot written once;
    # bytes: the fp16 rows read, the codes and scales written, the slot ids read
    T, H, P, page = 16384, 8, 4096, 16
    Kn = torch.randn(T, H, Dd, device="cuda", generator=g).half()
    Vn = torch.randn(T, H, Dd, device="cuda", generator=g).half()
    slots = torch.randperm(P * page, device="cuda", generator=g)[:T].to(torch.int32)
    for fmt in ("int8", "int4"):
        width, qdt = (Dd, torch.int8) if fmt == "int8" else (Dd // 2, torch.uint8)
        Kp = torch.zeros(P, H, page, width, dtype=qdt, device="cuda").permute(0, 2, 1, 3)
        Vp = torch.zeros(P, H, page, width, dtype=qdt, device="cuda").permute(0, 2, 1, 3)
        Ks = torch.zeros(P, H, page, dtype=torch.float16, device="cuda").permute(0, 2, 1)
        Vs = torch.zeros(P, H, page, dtype=torch.float16, device="cuda").permute(0, 2, 1)
        fq.quantize_kv_to_pages_(Kn, Vn, slots, Kp, Vp, Ks, Vs)
        f = fq.quantize_int8_per_token if fmt == "int8" else fq.quantize_int4_per_token
        q, s = f(Kn)
        pg, off = (slots // page).long(), (slots % page).long()
        same = bool(torch.equal(Kp[pg, off], q) and torch.equal(Ks[pg, off], s))
        if not same:
            log("paged quantizer %s: bytes differ from quantize_%s_per_token" % (fmt, fmt))
            continue
        nbytes = 2 * (T * H * Dd * 2 + T * H * (width + 2)) + 4 * T
        ms = _loop_ms(torch, lambda i: fq.quantize_kv_to_pages_(Kn, Vn, slots, Kp, Vp, Ks, Vs), 1,
                      max(50, steps // 4), max(10, warmup // 4))
        rows.append(_row("quantize_kv_to_pages_" + fmt, {"tokens": T, "Hkv": H, "D": Dd, "page": page, "pages": P,
                                                        "layout": "HND", "src": "fp16"}, ms, nbytes,
                         equal_to_quantizer=same))
        log("paged quantizer %s (K+V, %d tokens): %8.2f us  %7.1f GB/s" % (fmt, T, ms * 1e3, nbytes / ms / 1e6))
        del Kp, Vp, Ks, Vs
    torch.cuda.empty_cache()


def suite_llama(torch, fq, rows, full=True):
    """End-to-end decode on a random-init Llama-3.2-1B-shaped model (16 layers, 32/8 heads,
    head_dim 64, hidden 2048, fp16) through transformers, SDPA vs the kernel hook
    (the reference's nb:1037-1123 measurements: generate tok/s at prompt 512 + 128 new
    tokens, and the median single decode step at a fixed cache length)."""
    import time

    import transformers
    from fqkv_decode import hf_llama

    name = hf_llama.register()
    cfg = transformers.LlamaConfig(vocab_size=128256, hidden_size=2048, intermediate_size=8192,
                                   num_hidden_layers=16, num_attention_heads=32, num_key_value_heads=8,
                                   head_dim=64, max_position_embeddings=8192, attn_implementation="sdpa")
    torch.manual_seed(0)
    with torch.device("cuda"):
        model = transformers.LlamaForCausalLM(cfg).half().eval()

    def set_impl(impl):
        model.config._attn_implementation = impl
        for layer in model.model.layers:
            layer.self_attn.config._attn_implementation = impl

    def cache(kv_format):
        return None if kv_format is None else hf_llama.QuantizedKVCache(cfg, kv_format)

    def tok_per_s(impl, prompt_len=512, gen=128, reps=3, kv_format=None):
        set_impl(impl)
        ids = torch.randint(0, cfg.vocab_size, (1, prompt_len), device="cuda")
        best = 1e9
        with torch.no_grad():
            model.generate(ids, max_new_tokens=8, min_new_tokens=8, do_sample=False, past_key_values=cache(kv_format))
            torch.cuda.synchronize()
            for _ in range(reps):
                t0 = time.perf_counter()
                model.generate(ids, max_new_tokens=gen, min_new_tokens=gen, do_sample=False,
                               past_key_values=cache(kv_format))
                torch.cuda.synchronize()
                best = min(best, time.perf_counter() - t0)
        return gen / best

    def decode_ms(impl, ctx, reps=100, kv_format=None):
        set_impl(impl)
        with torch.no_grad():
            ids = torch.randint(0, cfg.vocab_size, (1, ctx), device="cuda")
            out = model(ids, use_cache=True, past_key_values=cache(kv_format))
            past = out.past_key_values
            step = torch.randint(0, cfg.vocab_size, (1, 1), device="cuda")
            ts = []
            for i in range(reps + 10):
                past.crop(ctx)
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                model(step, past_key_values=past, use_cache=True)
                b.record()
                torch.cuda.synchronize()
                if i >= 10:
                    ts.append(a.elapsed_time(b))
        ts.sort()
        return ts[len(ts) // 2]

    def graphed_s(impl, prompt_len, gen, reps=3, kv_format=None):
        """Best wall time of hf_llama.generate_graphed (prefill, capture and every replay)."""
        set_impl(impl)
        ids = torch.randint(0, cfg.vocab_size, (1, prompt_len), device="cuda")
        hf_llama.generate_graphed(model, ids, 8, kv_format=kv_format)
        torch.cuda.synchronize()
        best = 1e9
        for _ in range(reps):
            t0 = time.perf_counter()
            hf_llama.generate_graphed(model, ids, gen, kv_format=kv_format)
            torch.cuda.synchronize()
            best = min(best, time.perf_counter() - t0)
        return best

    def interleaved(runs, reps=3):
        """Best time of each zero-argument run over reps rounds that take every run in turn: the
        host-bound eager loop drifts by several per cent over a minute, which measuring one
        configuration after the other would book as a difference between them."""
        best = {k: 1e9 for k in runs}
        for _ in range(reps):
            for k, fn in runs.items():
                best[k] = min(best[k], fn())
        return best

    r = {"bench": "llama_decode", "config": {"model": "random-init LlamaConfig 16L 2048h 32q/8kv hd64 fp16",
                                             "prompt": 512, "new_tokens": 128}}
    # generate tok/s, SDPA vs the kernel hook, and graph-replayed over a static cache
    # (hf_llama.generate_graphed) with the attention on the paged kernel or on transformers' SDPA
    # with its mask; each figure the best of three rounds that alternate the four
    best = interleaved({"sdpa_tok_s": lambda: 128 / tok_per_s("sdpa", reps=1),
                        "kernel_tok_s": lambda: 128 / tok_per_s(name, reps=1),
                        "sdpa_graphed_tok_s": lambda: graphed_s("sdpa", 512, 128, reps=1),
                        "kernel_graphed_tok_s": lambda: graphed_s(name, 512, 128, reps=1)})
    for k in ("sdpa_tok_s", "kernel_tok_s", "kernel_graphed_tok_s", "sdpa_graphed_tok_s"):
        r[k] = round(128 / best[k], 2)
    if not full:  # generate tok/s only (the reference's end_to_end.json)
        rows.append(r)
        set_impl("sdpa")
        del model
        torch.cuda.empty_cache()
        return
    for ctx in (512, 2048, 8192):
        r["decode_ms_sdpa_ctx%d" % ctx] = round(decode_ms("sdpa", ctx), 4)
        r["decode_ms_kernel_ctx%d" % ctx] = round(decode_ms(name, ctx), 4)
    # one replayed decode step: the time of 128 more generated tokens over 128 (capacity 1024 at
    # prompt 512, 16384 at prompt 8192, where the kernel splits over the whole capacity)
    for ctx in (512, 8192):
        for impl, key in ((name, "kernel"), ("sdpa", "sdpa")):
            r["graphed_step_ms_%s_ctx%d" % (key, ctx)] = round(
                (graphed_s(impl, ctx, 256) - graphed_s(impl, ctx, 128)) / 128 * 1e3, 4)
    # the same hook over an int8 / int4 / fp8 KV cache (hf_llama.QuantizedKVCache); KV bytes read
    # per decode step at 8192 cached tokens: 16 layers x 2 x 8 heads x 8192 x (128, 64 + 2, 32 + 2) B
    for fmt in ("int8", "int4", "fp8"):
        r["kernel_%s_tok_s" % fmt] = round(tok_per_s(name, kv_format=fmt), 2)
        r["decode_ms_kernel_%s_ctx8192" % fmt] = round(decode_ms(name, 8192, kv_format=fmt), 4)
        # graph-replayed over a static quantized cache (device-position append + paged kernel)
        r["kernel_graphed_%s_tok_s" % fmt] = round(128 / graphed_s(name, 512, 128, kv_format=fmt), 2)
        r["graphed_step_ms_kernel_%s_ctx8192" % fmt] = round(
            (graphed_s(name, 8192, 256, kv_format=fmt) - graphed_s(name, 8192, 128, kv_format=fmt)) / 128 * 1e3, 4)
    r["kv_mb_per_step_ctx8192"] = {f: round(16 * 2 * 8 * 8192 * b / 1e6, 1)
                                   for f, b in (("fp16", 128), ("int8", 66), ("int4", 34), ("fp8", 66))}
    rows.append(r)
    log("llama     generate tok/s: sdpa %.2f, kernel %.2f; decode step ms (sdpa/kernel) ctx512 %.3f/%.3f "
        "ctx2048 %.3f/%.3f ctx8192 %.3f/%.3f" % (r["sdpa_tok_s"], r["kernel_tok_s"], r["decode_ms_sdpa_ctx512"],
                                                 r["decode_ms_kernel_ctx512"], r["decode_ms_sdpa_ctx2048"],
                                                 r["decode_ms_kernel_ctx2048"], r["decode_ms_sdpa_ctx8192"],
                                                 r["decode_ms_kernel_ctx8192"]))
    log("llama     graphed static cache: generate tok/s sdpa %.2f, kernel %.2f; replayed step ms (sdpa/kernel) "
        "ctx512 %.3f/%.3f ctx8192 %.3f/%.3f" % (r["sdpa_graphed_tok_s"], r["kernel_graphed_tok_s"],
                                                r["graphed_step_ms_sdpa_ctx512"], r["graphed_step_ms_kernel_ctx512"],
                                                r["graphed_step_ms_sdpa_ctx8192"],
                                                r["graphed_step_ms_kernel_ctx8192"]))
    for fmt in ("int8", "int4", "fp8"):
        log("llama     %s KV cache: generate tok/s %.2f; decode step ms ctx8192 %.3f; graphed tok/s %.2f, "
            "replayed step ms ctx8192 %.3f" % (fmt, r["kernel_%s_tok_s" % fmt], r["decode_ms_kernel_%s_ctx8192" % fmt],
                                                r["kernel_graphed_%s_tok_s" % fmt],
                                                r["graphed_step_ms_kernel_%s_ctx8192" % fmt]))
    set_impl("sdpa")
    del model
    torch.cuda.empty_cache()


SUITES = ("mha_small", "mha_quant", "gqa", "splitk", "splitk_quant", "paged", "quant", "llama")


# The reference's end-to-end result (benchmarks/end_to_end.json): Llama-3.2-1B, prompt 512,
# 128 new tokens, SDPA vs its kernel hook, on its A100.
REF_E2E_TOK_S = (51.887, 54.680)


# The reference's primary table on its A100 (benchmarks/flashinfer_looptimed.json:6-149): gqa_sk_fast
# at Hq 32 / Hkv 8, batch 1, loop-timed µs per call and the best S/W/CW of its sweep, per (D, N).
REF_SPLITK_A100 = {
    (64, 512): (10.48, "S16W8C4"), (64, 1024): (12.57, "S16W8C4"), (64, 2048): (16.93, "S16W8C4"),
    (64, 4096): (25.05, "S32W8C8"), (64, 8192): (39.23, "S32W8C8"), (64, 16384): (94.30, "S128W8C8"),
    (128, 512): (11.86, "S16W8C4"), (128, 1024): (14.71, "S16W8C4"), (128, 2048): (20.11, "S16W8C4"),
    (128, 4096): (30.63, "S16W8C4"), (128, 8192): (74.25, "S64W8C8"), (128, 16384): (129.34, "S128W8C8"),
}
MERGE_NAMES = {0: "none (one split)", 1: "two-kernel", 2: "fused, device scope", 3: "fused, one XCD's L2"}


# ---------------------------------------------------------------------------
# Where a call's time goes (--timeline): the decode kernel's own clock stamps
# beside the host's issue cost and the GPU's back-to-back cost per call.

# stage index of the stamps -> what has happened when a wave writes it
TIMELINE_STAGES = (
    (0, "wave started"),
    (1, "every K/V load of the first pass issued"),
    (3, "last pass's P.V products issued"),
    (4, "wave totals written to LDS"),
    (5, "wave-merge barrier passed"),
    (6, "output or partials issued"),
    (7, "arrival known"),
    (8, "merge: maximum over the splits known"),
    (9, "merge done"),
    (10, "wave ended"),
)
TL_BLOCKS, TL_WAVES, TL_SLOTS = 4096, 8, 16  # g_timeline's shape in the stamped build


def _stage_stats(x):
    x = sorted(x)
    n = len(x)
    return {"n": n, "min": round(x[0], 2), "p10": round(x[n // 10], 2), "median": round(x[n // 2], 2),
            "p90": round(x[n * 9 // 10], 2), "max": round(x[-1], 2)}


def timeline_stamps(torch, q, Ks, Vs, S, W, CW, calls=30, reps=3):
    """Stage stamps of the last of `calls` back-to-back gqa_sk_fast calls, from
    libfqkv_decode_timeline.so (the same kernels built with -DFQKV_TIMELINE:
    lane 0 of every wave reads the 100 MHz real-time counter at each stage).
    Times are microseconds from the earliest wave start of that call; the
    median over `reps` repetitions of each statistic is reported."""
    import numpy as np
    from fqkv_decode._paths import PKG_DIR, TIMELINE_LIB_NAME

    path = os.path.join(PKG_DIR, TIMELINE_LIB_NAME)
    if not os.path.exists(path):
        raise SystemExit("%s is missing: build first (python -c 'import __graft_entry__ as g; g.build()')" % path)
    lib = ctypes.CDLL(path)
    call = lib.fqkv_gqa_sk_fast
    call.restype = ctypes.c_int
    call.argtypes = [ctypes.c_void_p] * 7 + [ctypes.c_int64] * 7 + [ctypes.c_void_p]
    read = lib.fqkv_timeline_read
    read.restype = ctypes.c_int
    read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    hq, n_tok, d = q.shape[0], Ks[0].shape[1], q.shape[1]
    hkv = Ks[0].shape[0]
    mp = torch.empty(hq, S, device="cuda")
    lp = torch.empty(hq, S, device="cuda")
    op = torch.empty(hq, S, d, device="cuda")
    o = torch.empty(hq, d, device="cuda", dtype=torch.float16)
    stream = torch.cuda.current_stream().cuda_stream
    buf = np.zeros((TL_BLOCKS, TL_WAVES, TL_SLOTS), dtype=np.uint64)
    per_rep = []
    for rep in range(reps):
        torch.cuda.synchronize()
        if read(None, ctypes.c_size_t(-1).value) != 0:
            raise RuntimeError("fqkv_timeline_read (clear) failed")
        for i in range(calls):
            j = (rep * calls + i) % len(Ks)
            rc = call(q.data_ptr(), Ks[j].data_ptr(), Vs[j].data_ptr(), mp.data_ptr(), lp.data_ptr(),
                      op.data_ptr(), o.data_ptr(), hq, hkv, n_tok, d, S, W, CW, stream)
            if rc != 0:
                raise RuntimeError("timeline build: fqkv_gqa_sk_fast returned %d" % rc)
        torch.cuda.synchronize()
        if read(buf.ctypes.data, buf.nbytes) != 0:
            raise RuntimeError("fqkv_timeline_read failed")
        start = buf[:, :, 0]
        t0 = start[start > 0].min()
        # stamps older than the last call's first wave were left by earlier calls
        # (a workgroup that merged then but not in the last call)
        stages = {}
        for idx, name in TIMELINE_STAGES:
            v = buf[:, :, idx]
            v = v[v >= t0]
            if v.size:
                stages[idx] = _stage_stats(((v - t0).astype(np.float64) / 100.0).tolist())
        merged = np.nonzero((buf[:, :, 9] >= t0).any(axis=1))[0]
        end = buf[:, :, 10]
        span = float((end[end >= t0].max() - t0) / 100.0)
        per_rep.append((stages, span, len(merged), int((start > 0).any(axis=1).sum())))
    out = {"calls": calls, "reps": reps, "workgroups": per_rep[0][3], "merging_workgroups": per_rep[0][2]}
    out["span_us"] = round(sorted(r[1] for r in per_rep)[reps // 2], 2)
    stages = {}
    for idx, name in TIMELINE_STAGES:
        rows = [r[0][idx] for r in per_rep if idx in r[0]]
        if not rows:
            continue
        st = {k: (sorted(r[k] for r in rows)[len(rows) // 2]) for k in rows[0]}
        st["stage"] = idx
        stages[name] = st
    out["stages_us"] = stages
    return out


def launch_costs(torch, fq, q, Ks, Vs, S, W, CW, steps=2000, warmup=200, graph_calls=100, replays=20):
    """Per-call cost of the same gqa_sk_fast call three ways:
    * loop_us: the bench's Python loop between HIP events (the headline method);
    * host_issue_us: host wall time to issue one call of that loop (nothing
      waits for the GPU inside it), i.e. the rate at which the host can feed
      the GPU through the PyTorch binding;
    * graph_us: `graph_calls` calls captured in one HIP graph and replayed
      `replays` times between events, so no host work sits between launches:
      the GPU's own back-to-back cost per call (dispatch + kernel)."""
    hq, d = q.shape
    mp = torch.empty(hq, S, device="cuda")
    lp = torch.empty(hq, S, device="cuda")
    op = torch.empty(hq, S, d, device="cuda")
    o = torch.empty(hq, d, device="cuda", dtype=torch.float16)
    n = len(Ks)
    fn = lambda i: fq.gqa_sk_fast(q, Ks[i % n], Vs[i % n], mp, lp, op, o, S, W, CW)
    loop_ms = _loop_ms(torch, fn, n, steps, warmup)
    torch.cuda.synchronize()
    t = time.perf_counter()
    for i in range(steps):
        fn(i)
    issue_s = time.perf_counter() - t
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(3):
            fn(i)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(graph_calls):
            fn(i)
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    graph_ms = a.elapsed_time(b) / (replays * graph_calls)
    del graph
    fq._ext._release_capture_slots()
    return {"loop_us": round(loop_ms * 1e3, 3), "host_issue_us": round(issue_s / steps * 1e6, 3),
            "graph_us": round(graph_ms * 1e3, 3), "graph_calls": graph_calls, "replays": replays}


def timeline_report(torch, fq, q, Ks, Vs, S, W, CW):
    res = {"launch_costs": launch_costs(torch, fq, q, Ks, Vs, S, W, CW),
           "timeline": timeline_stamps(torch, q, Ks, Vs, S, W, CW)}
    lc, tl = res["launch_costs"], res["timeline"]
    log("per call: Python loop %.3f us, host issue %.3f us, graph replay %.3f us; in-kernel span %.2f us "
        "(%d workgroups, %d merging)" % (lc["loop_us"], lc["host_issue_us"], lc["graph_us"], tl["span_us"],
                                         tl["workgroups"], tl["merging_workgroups"]))
    for name, st in tl["stages_us"].items():
        log("  stage %2d %-42s n %5d  min %6.2f  p10 %6.2f  median %6.2f  p90 %6.2f  max %6.2f"
            % (st["stage"], name, st["n"], st["min"], st["p10"], st["median"], st["p90"], st["max"]))
    return res


def splitk_primary_table(torch, fq, sweep_steps=200, sweep_warmup=20, steps=2000, warmup=200):
    """The reference's primary benchmark at its own shapes, plus N = 32768 (flashinfer_looptimed.py:59-95):
    gqa_sk_fast, Hq 32 / Hkv 8, batch 1, D in {64, 128}, N in {512 .. 32768}. Every S in
    {8, 16, 32, 64, 128} (S <= N / 16), W in {4, 8} and CW in {4, 8} that passes the correctness gate
    (max-abs <= 2e-3 against fp32 PyTorch on the GPU; the reference gates at 2e-2) is loop-timed over
    `sweep_steps` calls; the fastest is timed again over `steps` calls after `warmup`, as the reference
    does (2000 after 200). Each point cycles through >= 512 MiB of distinct KV sets (at most 512), so
    the Infinity Cache cannot serve a call from the previous one. CW sizes the combine kernel of the
    two-kernel merge; the default fused merge launches none, so CW does not change those calls."""
    G = HQ // HKV
    table = {}
    for Dd in (64, 128):
        for Nn in (512, 1024, 2048, 4096, 8192, 16384, 32768):
            per = 4 * HKV * Nn * Dd
            ns = max(1, min(512, -(-(512 << 20) // per)))
            g = torch.Generator(device="cuda").manual_seed(7)
            q = torch.randn(HQ, Dd, device="cuda", generator=g).half()
            sets = [(torch.randn(HKV, Nn, Dd, device="cuda", generator=g).half(),
                     torch.randn(HKV, Nn, Dd, device="cuda", generator=g).half()) for _ in range(ns)]
            ref = _ref_mha(torch, q, sets[0][0].float().repeat_interleave(G, 0),
                           sets[0][1].float().repeat_interleave(G, 0))
            nbytes = alg_bytes(n=Nn, d=Dd)
            settle(torch, fq)
            best = None
            for S in (8, 16, 32, 64, 128):
                if S > Nn // 16:
                    continue
                mp = torch.empty(HQ, S, device="cuda")
                lp = torch.empty(HQ, S, device="cuda")
                op = torch.empty(HQ, S, Dd, device="cuda")
                o = torch.empty(HQ, Dd, device="cuda", dtype=torch.float16)
                for Wk in (4, 8):
                    for CW in (4, 8):
                        fn = lambda i: fq.gqa_sk_fast(q, sets[i][0], sets[i][1], mp, lp, op, o, S, Wk, CW)
                        fn(0)
                        proto = fq._ext._last_merge_protocol()
                        err = float((o.float() - ref).abs().max())
                        if err > 2e-3:
                            log("split-K D=%d N=%d S%d W%d CW%d failed the gate: %.2e" % (Dd, Nn, S, Wk, CW, err))
                            continue
                        ms = _loop_ms(torch, fn, ns, sweep_steps, sweep_warmup)
                        if best is None or ms < best[0]:
                            best = (ms, S, Wk, CW, err, proto, (mp, lp, op, o))
            _, S, Wk, CW, err, proto, (mp, lp, op, o) = best
            ms = _loop_ms(torch, lambda i: fq.gqa_sk_fast(q, sets[i][0], sets[i][1], mp, lp, op, o, S, Wk, CW),
                          ns, steps, warmup)
            row = {"us_per_call": round(ms * 1e3, 3), "GBps": round(nbytes / ms / 1e6, 1), "frac": _frac(nbytes, ms),
                   "alg_bytes": nbytes, "kv_GBps": round(2 * Nn * HKV * Dd * 2 / ms / 1e6, 1),
                   "best": "S%dW%dC%d" % (S, Wk, CW), "merge": MERGE_NAMES[proto], "kv_sets": ns,
                   "kv_bytes_cycled": ns * per, "gate_max_abs_err": err}
            if (Dd, Nn) in REF_SPLITK_A100:
                ref_us, ref_cfg = REF_SPLITK_A100[(Dd, Nn)]
                row.update({"ref_a100_us": ref_us, "ref_a100_best": ref_cfg, "speedup_vs_ref_a100": round(ref_us / (ms * 1e3), 2)})
            table["D%d_N%d" % (Dd, Nn)] = row
            log("primary table D=%-3d N=%-6d %s  %8.2f us  %7.1f GB/s (%.1f %% of 8 TB/s)  err %.2e"
                % (Dd, Nn, row["best"], ms * 1e3, nbytes / ms / 1e6, 100 * row["frac"], err))
            del sets, ref
            torch.cuda.empty_cache()
    return table


def baseline_rows(torch, fq):
    """The reference's other benchmark rows at D = 128, beside the headline, the B = 2048 MHA rows
    and the primary table:
    * mha_fp16_b32_n512_d128: fp16 MHA, 32 heads, N 512, D 128 (the reference's CPU-runnable case);
    * mha_n4096_d128: fp16 / int8 / int4 MHA at B 8 and 256, N 4096, D 128 (B 2048 is
      mha_b2048_n4096_d128);
    * gqa_n512_d64: decode_attn_gqa vs repeat_kv + the MHA kernel at Hq 32 / Hkv 8, N 512, D 64,
      B in {1, 4, 16};
    * splitk_quant_n16384_d128: gqa_sk_fast_int8 / _int4 at the headline shape (Hq 32 / Hkv 8,
      N 16384, D 128, batch 1), best of S in {16, 32, 64} x W in {4, 8}.
    Loop-timed (400 calls after 40 warm-ups) over >= 1 GiB of distinct inputs per cycle, each row
    gated against fp32 PyTorch on the GPU (max-abs <= 2e-3)."""
    out = {}
    rows = []
    suite_mha_small(torch, fq, 400, 40, rows)
    r = rows[0]
    out["mha_fp16_b32_n512_d128"] = {"us_per_call": r["us_per_call"], "GBps": r["GBps"], "frac": r["frac_of_8TBps"],
                                     "alg_bytes": r["alg_bytes"], "gate_max_abs_err": r["max_abs_err_vs_fp32"]}
    rows = []
    suite_mha_quant(torch, fq, 400, 40, rows, shapes=[(128, 8), (128, 256)], formats=("fp16", "int8", "int4"))
    mq = {}
    for r in rows:
        fmt, B = r["bench"].split("_")[1], r["config"]["B"]
        mq.setdefault("B%d" % B, {})[fmt] = {"us_per_call": r["us_per_call"], "GBps": r["GBps"],
                                             "frac": r["frac_of_8TBps"], "alg_bytes": r["alg_bytes"],
                                             "gate_max_abs_err": r["max_abs_err_vs_fp32"]}
    out["mha_n4096_d128"] = mq
    rows = []
    suite_gqa(torch, fq, 400, 40, rows, shapes=[(512, b) for b in (1, 4, 16)])
    out["gqa_n512_d64"] = {"B%d" % r["config"]["B"]: {"gqa_us": r["us_per_call"], "GBps": r["GBps"],
                                                      "frac": r["frac_of_8TBps"],
                                                      "repeat_kv_mha_us": r["expand_mha_us"],
                                                      "speedup_vs_repeat_kv": r["speedup_vs_expand"],
                                                      "gate_max_abs_err": r["max_abs_err_vs_fp32"]} for r in rows}
    rows = []
    suite_splitk_quant(torch, fq, 400, 40, rows, cases=((1, 16384),), formats=("int8", "int4"))
    out["splitk_quant_n16384_d128"] = {r["bench"].rsplit("_", 1)[1]: {
        "us_per_call": r["us_per_call"], "GBps": r["GBps"], "frac": r["frac_of_8TBps"], "alg_bytes": r["alg_bytes"],
        "S": r["config"]["S"], "W": r["config"]["W"], "gate_max_abs_err": r["max_abs_err_vs_fp32"]} for r in rows}
    for name, r in out.items():
        for v in ([r] if "gate_max_abs_err" in r else r.values()):
            for x in ([v] if "gate_max_abs_err" in v else v.values()):
                if x["gate_max_abs_err"] > 2e-3:
                    raise RuntimeError("baseline-row gate failed: %s max-abs %.3e" % (name, x["gate_max_abs_err"]))
    return out


def reference_tables(torch, fq):
    """The reference's other published tables at their own shapes, for the default line:
    * standalone_quant_d64 (benchmarks/standalone_quant.json): fp16 / int8 / int4 MHA at
      B in {8, 256, 2048}, N 4096, D 64, W 8, with the int8 / int4 speed-ups over fp16;
    * gqa_aware_n4096_d64 (benchmarks/gqa_aware.json): decode_attn_gqa vs repeat_kv + the
      MHA kernel at Hq 32 / Hkv 8, N 4096, D 64, B in {1, 4, 16};
    * end_to_end_llama (benchmarks/end_to_end.json): generate tok/s at prompt 512 + 128 new
      tokens on a random-init Llama-3.2-1B-shaped model, SDPA vs the kernel hook (best of 3),
      and the same with every decode step replayed from a HIP graph over a static cache.
    Each row is gated against fp32 PyTorch on the GPU (max-abs <= 2e-3), loop-timed like the
    suite (400 calls after 40 warm-ups); the reference's A100 numbers ride along."""
    rows = []
    suite_mha_quant(torch, fq, 400, 40, rows, shapes=[(64, b) for b in (8, 256, 2048)],
                    formats=("fp16", "int8", "int4"))
    sq = {}
    for r in rows:
        fmt, B = r["bench"].split("_")[1], r["config"]["B"]
        if r["max_abs_err_vs_fp32"] > 2e-3:
            raise RuntimeError("reference-table gate failed: %s B=%d max-abs %.3e" % (fmt, B, r["max_abs_err_vs_fp32"]))
        e = sq.setdefault("B%d" % B, {"gate_max_abs_err": 0.0, "ref_a100_us": {}})
        e[fmt + "_us"] = r["us_per_call"]
        e[fmt + "_frac"] = r["frac_of_8TBps"]
        e["ref_a100_us"][fmt] = round(r["ref_a100_us"], 2)
        e["gate_max_abs_err"] = max(e["gate_max_abs_err"], r["max_abs_err_vs_fp32"])
    for e in sq.values():
        e["int8_speedup_vs_fp16"] = round(e["fp16_us"] / e["int8_us"], 3)
        e["int4_speedup_vs_fp16"] = round(e["fp16_us"] / e["int4_us"], 3)
    rows = []
    suite_gqa(torch, fq, 400, 40, rows, shapes=[(4096, b) for b in (1, 4, 16)])
    ga = {}
    for r in rows:
        if r["max_abs_err_vs_fp32"] > 2e-3:
            raise RuntimeError("reference-table gate failed: gqa B=%d" % r["config"]["B"])
        ga["B%d" % r["config"]["B"]] = {
            "gqa_us": r["us_per_call"], "repeat_kv_mha_us": r["expand_mha_us"], "speedup": r["speedup_vs_expand"],
            "ref_a100_gqa_us": round(r["ref_a100_gqa_us"], 1), "ref_a100_repeat_kv_us": round(r["ref_a100_expand_us"], 1),
            "gate_max_abs_err": r["max_abs_err_vs_fp32"]}
    out = {"standalone_quant_d64": sq, "gqa_aware_n4096_d64": ga}
    rows = []
    try:
        suite_llama(torch, fq, rows, full=False)
        r = rows[0]
        out["end_to_end_llama"] = {"sdpa_tok_s": r["sdpa_tok_s"], "kernel_tok_s": r["kernel_tok_s"],
                                   "speedup": round(r["kernel_tok_s"] / r["sdpa_tok_s"], 3),
                                   "sdpa_graphed_tok_s": r["sdpa_graphed_tok_s"],
                                   "kernel_graphed_tok_s": r["kernel_graphed_tok_s"],
                                   "model": r["config"]["model"], "prompt": 512, "new_tokens": 128,
                                   "ref_a100_tok_s": {"sdpa": REF_E2E_TOK_S[0], "kernel": REF_E2E_TOK_S[1]}}
    except ImportError as e:  # transformers absent: the row is skipped, not faked
        out["end_to_end_llama"] = {"skipped": str(e)}
    return out


def run_suite(torch, fq, path, steps=400, warmup=40, only=SUITES):
    rows = []
    if "mha_small" in only:
        suite_mha_small(torch, fq, steps, warmup, rows)
    if "mha_quant" in only:
        suite_mha_quant(torch, fq, steps, warmup, rows)
    if "gqa" in only:
        suite_gqa(torch, fq, steps, warmup, rows)
    if "splitk" in only:
        suite_splitk(torch, fq, steps, warmup, rows)
    if "splitk_quant" in only:
        suite_splitk_quant(torch, fq, steps, warmup, rows)
    if "paged" in only:
        suite_paged(torch, fq, steps, warmup, rows)
    if "quant" in only:
        suite_quant(torch, fq, steps, warmup, rows)
    if "llama" in only:
        suite_llama(torch, fq, rows)
    with open(path, "w") as f:
        for r in rows:
            f.write(json.dumps(r) + "\n")
    log("suite: %d rows -> %s" % (len(rows), path))


def main():
    global N
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--S", type=int, default=0, help="splits (0 = from the CU count)")
    ap.add_argument("--W", type=int, default=8)
    ap.add_argument("--CW", type=int, default=8)
    ap.add_argument("--kv-sets", type=int, default=10, help="distinct 64 MiB KV caches cycled through")
    ap.add_argument("--n-tokens", type=int, default=16384,
                    help="cached tokens of the timed workload (default 16384, the metric's; other values for A/B runs)")
    ap.add_argument("--sweep", action="store_true", help="tune S/W/CW first (table on stderr)")
    ap.add_argument("--merge", choices=("fused", "two-kernel"), default="fused",
                    help="split merge inside the partial kernel (default) or a separate combine kernel")
    ap.add_argument("--pv", choices=("mfma", "valu"), default="mfma",
                    help="P.V on the matrix cores (default) or, for A/B runs, on the vector ALUs "
                         "(fp16, D 128, 1 or 4 heads per work item)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the secondary keys (MHA B=2048, split-K B=8 N=32K, launch floor, primary "
                         "split-K table, the other D=128 rows, the reference's D=64 tables)")
    ap.add_argument("--suite", metavar="FILE", default="",
                    help="also measure the secondary configurations, JSON lines into FILE")
    ap.add_argument("--suite-only", metavar="NAMES", default=",".join(SUITES),
                    help="comma-separated subset of the suite: " + ", ".join(SUITES))
    ap.add_argument("--timeline", action="store_true",
                    help="instead of the benchmark line: per-call host issue / Python loop / graph replay cost and "
                         "the decode kernel's per-stage clock stamps (libfqkv_decode_timeline.so) for the workload")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="first run a plain device copy of this many MiB (counter calibration under rocprofv3 --pmc)")
    args = ap.parse_args()
    only = tuple(x for x in args.suite_only.split(",") if x)
    unknown = [x for x in only if x not in SUITES]
    if unknown:
        print("unknown suite name(s): %s (choose from %s)" % (", ".join(unknown), ", ".join(SUITES)), file=sys.stderr)
        sys.exit(2)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the decode path shards by KV head with no communication); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    N = args.n_tokens
    import torch
    import fqkv_decode as fq

    cus = fq.cu_count()
    fq._ext._set_two_kernel_merge(1 if args.merge == "two-kernel" else 0)
    fq._ext._set_pv_valu(args.pv == "valu")
    if args.calib_copy_mib:
        n = args.calib_copy_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("calibration copy: 3 x %d MiB device-to-device" % args.calib_copy_mib)
        del src, dst
    q, Ks, Vs = make_sets(torch, args.kv_sets)
    S, W, CW = (args.S or default_splits(cus)), args.W, args.CW

    if args.sweep:
        best = None
        for s in (16, 32, 64, 128, 256):
            for w in (2, 4, 8):
                for cw in (4, 8):
                    err = gate(torch, fq, q, Ks[0], Vs[0], s, w, cw)
                    if err > 2e-3:
                        log("S%d W%d CW%d FAILED gate: %.3e" % (s, w, cw, err))
                        continue
                    ms = time_calls(torch, fq, q, Ks, Vs, s, w, cw, 500, 50)
                    log("S%-4d W%d CW%d  %8.2f us  %7.1f GB/s" % (s, w, cw, ms * 1e3, alg_bytes() / ms / 1e6))
                    if best is None or ms < best[0]:
                        best = (ms, s, w, cw)
        _, S, W, CW = best
        log("best: S%d W%d CW%d" % (S, W, CW))

    err = gate(torch, fq, q, Ks[0], Vs[0], S, W, CW)
    if err > 2e-3:
        log("correctness gate failed: max-abs %.3e > 2e-3" % err)
        sys.exit(1)
    merge_protocol = fq._ext._last_merge_protocol()
    if args.timeline:
        res = timeline_report(torch, fq, q, Ks, Vs, S, W, CW)
        res["config"] = {"workload": "gqa_sk_fast fp16 decode, Hq=32, Hkv=8, N=%d, D=128, batch 1" % N,
                         "S": S, "W": W, "CW": CW, "merge": MERGE_NAMES[merge_protocol], "kv_sets": args.kv_sets,
                         "gate_max_abs_err": err}
        print(json.dumps(res), flush=True)
        return

    settle(torch)
    ms = time_calls(torch, fq, q, Ks, Vs, S, W, CW, args.steps, args.warmup)
    ms_long = time_calls(torch, fq, q, Ks, Vs, S, W, CW, 2000, 200) if args.steps < 2000 else ms
    ev = HipEvents()
    p_avg_ms, p_med_ms = time_partial(torch, fq, q, Ks, Vs, S, W, CW, min(args.steps, 1000), ev)
    value = alg_bytes() / ms / 1e6  # GB/s
    if args.merge == "fused":
        # one kernel per call: its average duration is the loop time per call
        k_ms, method = ms, ("HIP events around the timed loop of %d calls, one kernel per call; %d more warm-up "
                            "calls queued after the synchronisation, ahead of the start event" % (args.steps, LEAD_CALLS))
    else:
        k_ms, method = p_avg_ms, "HIP events recorded just before and after each partial launch"
    achieved = alg_bytes() / k_ms / 1e6
    # the committed counter summary covers the default workload only
    traffic = read_traffic() if N == 16384 and args.merge == "fused" else None
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "us_per_call": round(ms * 1e3, 3),
        "us_per_call_2000_calls": round(ms_long * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / REF_A100_GBS, 3) if N == 16384 else None,
        "baseline_note": "reference A100 result for this metric: 519 GB/s, 129.34 us/call "
                         "(benchmarks/flashinfer_looptimed.json:138-149)",
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": "gqa_sk_fast fp16 decode, Hq=32, Hkv=8, N=%d, D=128, batch 1" % N,
            "S": S, "W": W, "CW": CW, "merge": MERGE_NAMES[merge_protocol], "pv": args.pv,
            "xcd_period": fq._ext._xcd_period(torch.cuda.current_device()),
            "kv_sets": args.kv_sets,
            "kv_bytes_cycled": args.kv_sets * 4 * HKV * N * D,
            "alg_bytes_per_call": alg_bytes(),
            "cu_count": cus,
            "gate_max_abs_err": err,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_partial_kernel<fp16, D=128, HG=4>"
                      + (" (split merge fused in)" if args.merge == "fused" else ""),
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_source": ("profiles/decode_partial_gqa_n16k_d128_pmc.md (rocprofv3 --pmc FETCH_SIZE + "
                               "WRITE_SIZE of this kernel, committed; not measured in this run)") if traffic else None,
            "avg_us": round(k_ms * 1e3, 3),
            "method": method,
            "per_launch_event_avg_us": round(p_avg_ms * 1e3, 3),
            "per_launch_event_median_us": round(p_med_ms * 1e3, 3),
            "alg_bytes_per_launch": alg_bytes(),
        },
    }
    del Ks, Vs
    torch.cuda.empty_cache()
    ceil = stream_ceiling(torch, fq, args.steps, args.warmup)
    ceil["headline_frac_of_ceiling"] = round(ceil["us_per_call"] / (ms * 1e3), 4)
    line["stream_ceiling"] = ceil
    line["roofline"]["frac_of_stream_ceiling"] = ceil["headline_frac_of_ceiling"]
    log("stream ceiling (64 MiB read, %d workgroups): %.3f us  %.1f GB/s; headline at %.1f %% of it"
        % (ceil["blocks"], ceil["us_per_call"], ceil["GBps"], 100 * ceil["headline_frac_of_ceiling"]))
    if not args.no_secondary:
        line.update(secondary_results(torch, fq))
        line["splitk_primary_table"] = splitk_primary_table(torch, fq)
        line["baseline_d128_rows"] = baseline_rows(torch, fq)
        line["reference_tables"] = reference_tables(torch, fq)
    if args.suite:
        run_suite(torch, fq, args.suite, only=only)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
