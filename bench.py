"""Benchmark of the GQA split-K fp16 decode path on one MI355X.

Workload (the headline metric's configuration): ``gqa_sk_fast`` with 32 query
heads / 8 KV heads, N = 16384 cached tokens, head_dim 128, batch 1, fp16
q/K/V drawn N(0,1), fp32 split scratch preallocated. One step = one call of
the entry point (partial kernel + combine kernel) on the next of ``--kv-sets``
distinct KV caches, so successive steps stream >= 512 MiB of distinct KV and
the 256 MB Infinity Cache cannot serve them. Inputs are resident in HBM
before timing starts.

Reported: ``value`` = algorithmic bytes per call / time per call in GB/s
(bytes = 4*Hkv*N*D (K+V fp16) + 4*Hq*D (q in, o out), i.e. 67,125,248),
whole-call loop timing like the reference's flashinfer_looptimed.py:34-44.
``roofline`` covers the dominant (partial) kernel, timed per launch with HIP
events recorded around it on its own stream. ``cpu_baseline`` times the
numpy oracle on the host for a bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--S S --W W --CW CW]
       python bench.py --sweep      (tuning table on stderr, then the JSON line)
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


def alg_bytes(hq=HQ, hkv=HKV, n=N, d=D):
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


def time_calls(torch, fq, q, Ks, Vs, S, W, CW, steps, warmup):
    mp = torch.empty(HQ, S, device="cuda")
    lp = torch.empty(HQ, S, device="cuda")
    op = torch.empty(HQ, S, D, device="cuda")
    o = torch.empty(HQ, D, device="cuda", dtype=torch.float16)
    n = len(Ks)
    for i in range(warmup):
        fq.gqa_sk_fast(q, Ks[i % n], Vs[i % n], mp, lp, op, o, S, W, CW)
    torch.cuda.synchronize()
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
    path = os.path.join(ROOT, "profiles", "gqa_sk_partial_n16k_d128_pmc.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return float(line.split(":", 1)[1].strip())
            except ValueError:
                return None
    return None


def cpu_baseline(budget_s=15.0):
    """The numpy oracle on the host, on whole calls of the metric workload until ~budget_s."""
    import numpy as np
    import torch

    sys.path.insert(0, ROOT)
    import oracle

    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, HQ, D, generator=g).half().numpy()
    K = torch.randn(1, HKV, N, D, generator=g).half().numpy()
    V = torch.randn(1, HKV, N, D, generator=g).half().numpy()
    oracle.gqa_attention(q, K[:, :, :64], V[:, :, :64])  # warm-up
    t0 = time.perf_counter()
    calls = 0
    while True:
        oracle.gqa_attention(q, K, V)
        calls += 1
        el = time.perf_counter() - t0
        if el >= budget_s or calls >= 50:
            break
    per_call = el / calls
    return {
        "value": round(alg_bytes() / per_call / 1e9, 4),
        "unit": "GB/s",
        "us_per_call": round(per_call * 1e6, 1),
        "cores": 1,
        "kind": "port",
        "sample": "%d whole calls of the workload (32q/8kv heads, N=16384, D=128) through "
                  "oracle.gqa_attention (numpy float64, single-threaded einsum), %.1f s" % (calls, el),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--S", type=int, default=0, help="splits (0 = from the CU count)")
    ap.add_argument("--W", type=int, default=8)
    ap.add_argument("--CW", type=int, default=8)
    ap.add_argument("--kv-sets", type=int, default=10, help="distinct 64 MiB KV caches cycled through")
    ap.add_argument("--sweep", action="store_true", help="tune S/W/CW first (table on stderr)")
    ap.add_argument("--merge", choices=("fused", "two-kernel"), default="fused",
                    help="split merge inside the partial kernel (default) or a separate combine kernel")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="first run a plain device copy of this many MiB (counter calibration under rocprofv3 --pmc)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the decode path shards by KV head with no communication); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import fqkv_decode as fq

    cus = fq.cu_count()
    fq._ext._set_two_kernel_merge(1 if args.merge == "two-kernel" else 0)
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

    ms = time_calls(torch, fq, q, Ks, Vs, S, W, CW, args.steps, args.warmup)
    ev = HipEvents()
    p_avg_ms, p_med_ms = time_partial(torch, fq, q, Ks, Vs, S, W, CW, min(args.steps, 1000), ev)
    value = alg_bytes() / ms / 1e6  # GB/s
    achieved = alg_bytes() / p_avg_ms / 1e6
    traffic = read_traffic()
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "us_per_call": round(ms * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / REF_A100_GBS, 3),
        "baseline_note": "reference A100 result for this metric: 519 GB/s, 129.34 us/call "
                         "(benchmarks/flashinfer_looptimed.json:138-149)",
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": "gqa_sk_fast fp16 decode, Hq=32, Hkv=8, N=16384, D=128, batch 1",
            "S": S, "W": W, "CW": CW, "merge": args.merge,
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
            "avg_us": round(p_avg_ms * 1e3, 3),
            "median_us": round(p_med_ms * 1e3, 3),
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
