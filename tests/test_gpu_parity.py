"""GPU parity of the five entry points against the CPU oracle (needs an MI355X).

Bar: max |kernel - oracle| <= TOL = 2e-3 where the oracle is
softmax(q K^T / sqrt(D)) V evaluated in float64 on the same inputs (for
int8 / int4 on the exactly dequantised values); dequantised values
themselves are bit-exact. Inputs come from a CPU torch.Generator seeded
with 0 (fp32 draws, then fp16 or quantized), copied to the GPU.

Shapes: the reference's own test cases (tests/test_kernels.py:18,26,41,59),
the notebook's int4 gate (nb:457-472) generalised to D=128, the committed
golden fixtures, and edge cases (N = 1, 3, 100; S > N; every W / CW).
"""

import os
import sys

import numpy as np
import pytest
import torch

import oracle
import fqkv_decode as fq
from fqkv_decode import quant

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 2e-3  # max-abs vs the float64 oracle
DEV = "cuda"


def draw(g, *shape):
    return torch.randn(*shape, generator=g, dtype=torch.float32)


def gpu(x):
    return torch.as_tensor(x).to(DEV)


def maxerr(out, ref):
    return float(np.abs(out.float().cpu().numpy().astype(np.float64) - ref).max())


# ------------------------------------------------------------------ fp16 ----

@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("B,N,W", [(1, 1024, 8), (8, 2048, 4), (256, 4096, 8), (32, 512, 2), (3, 1, 4), (5, 3, 8), (2, 100, 2)])
def test_fp16_mha(B, N, W, D):
    g = torch.Generator().manual_seed(0)
    q, K, V = draw(g, B, D).half(), draw(g, B, N, D).half(), draw(g, B, N, D).half()
    out = fq.decode_attn_fp16_mw(gpu(q), gpu(K), gpu(V), W)
    assert out.shape == (B, D) and out.dtype == torch.float16
    assert maxerr(out, oracle.attention(q.numpy(), K.numpy(), V.numpy())) <= TOL


def test_fp16_mha_long_sequence_uses_splits(merge_mode):
    B, N, D = 2, 16384, 128
    assert fq.choose_splits(B, 1, N, D, 0, 8) > 1
    g = torch.Generator().manual_seed(0)
    q, K, V = draw(g, B, D).half(), draw(g, B, N, D).half(), draw(g, B, N, D).half()
    out = fq.decode_attn_fp16_mw(gpu(q), gpu(K), gpu(V), 8)
    assert maxerr(out, oracle.attention(q.numpy(), K.numpy(), V.numpy())) <= TOL


# ------------------------------------------------------------------ int8 ----

@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("B,N,W", [(1, 1024, 8), (8, 2048, 4), (8, 4096, 8), (4, 3, 2), (2, 1, 8)])
def test_int8(B, N, W, D):
    g = torch.Generator().manual_seed(0)
    q = draw(g, B, D).half()
    Kq, Ks = quant.quant_int8_per_token(draw(g, B, N, D))
    Vq, Vs = quant.quant_int8_per_token(draw(g, B, N, D))
    out = fq.decode_attn_int8_mw(gpu(q), gpu(Kq), gpu(Vq), gpu(Ks), gpu(Vs), W)
    ref = oracle.attention(q.numpy(), oracle.dequant_int8(Kq.numpy(), Ks.numpy()),
                           oracle.dequant_int8(Vq.numpy(), Vs.numpy()))
    assert maxerr(out, ref) <= TOL


def test_int8_full_byte_range():
    """Every int8 byte, -128 included (the quantizer never emits it, the kernel must decode it)."""
    B, N, D = 2, 512, 128
    g = torch.Generator().manual_seed(3)
    q = draw(g, B, D).half()
    Kq = torch.randint(-128, 128, (B, N, D), generator=g, dtype=torch.int8)
    Vq = torch.randint(-128, 128, (B, N, D), generator=g, dtype=torch.int8)
    Ks = (torch.rand(B, N, generator=g) * 0.03 + 1e-3).half()
    Vs = (torch.rand(B, N, generator=g) * 0.03 + 1e-3).half()
    out = fq.decode_attn_int8_mw(gpu(q), gpu(Kq), gpu(Vq), gpu(Ks), gpu(Vs), 4)
    ref = oracle.attention(q.numpy(), oracle.dequant_int8(Kq.numpy(), Ks.numpy()),
                           oracle.dequant_int8(Vq.numpy(), Vs.numpy()))
    assert maxerr(out, ref) <= TOL


# ------------------------------------------------------------------ int4 ----

@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("W", [2, 4, 8])
@pytest.mark.parametrize("B,N", [(1, 1024), (8, 2048), (256, 4096), (4, 3)])
def test_int4_notebook_gate(B, N, W, D):
    g = torch.Generator().manual_seed(0)
    q = draw(g, B, D).half()
    Kp, Ks = quant.quant_int4_per_token(draw(g, B, N, D))
    Vp, Vs = quant.quant_int4_per_token(draw(g, B, N, D))
    out = fq.decode_attn_int4(gpu(q), gpu(Kp), gpu(Vp), gpu(Ks), gpu(Vs), W)
    assert out.shape == (B, D)
    ref = oracle.attention(q.numpy(), oracle.dequant_int4(Kp.numpy(), Ks.numpy()),
                           oracle.dequant_int4(Vp.numpy(), Vs.numpy()))
    assert maxerr(out, ref) <= TOL


@pytest.mark.parametrize("fmt", ["fp16", "int8", "int4"])
@pytest.mark.parametrize("D", [64, 128])
def test_mha_large_grid_four_wave_workgroups(fmt, D):
    """Over 4 workgroups per CU the entry points run 4-wave workgroups whatever W
    asks; the result must not change: oracle parity, and W = 8 equals W = 4 bit for
    bit (same workgroup shape)."""
    B, N = 1200, 40
    g = torch.Generator().manual_seed(9)
    q = draw(g, B, D).half()
    Kx, Vx = draw(g, B, N, D), draw(g, B, N, D)
    if fmt == "fp16":
        K, V = Kx.half(), Vx.half()
        run = lambda W: fq.decode_attn_fp16_mw(gpu(q), gpu(K), gpu(V), W)
        Kf, Vf = K.float().numpy(), V.float().numpy()
    elif fmt == "int8":
        K, Ks = quant.quant_int8_per_token(Kx)
        V, Vs = quant.quant_int8_per_token(Vx)
        run = lambda W: fq.decode_attn_int8_mw(gpu(q), gpu(K), gpu(V), gpu(Ks), gpu(Vs), W)
        Kf, Vf = oracle.dequant_int8(K.numpy(), Ks.numpy()), oracle.dequant_int8(V.numpy(), Vs.numpy())
    else:
        K, Ks = quant.quant_int4_per_token(Kx)
        V, Vs = quant.quant_int4_per_token(Vx)
        run = lambda W: fq.decode_attn_int4(gpu(q), gpu(K), gpu(V), gpu(Ks), gpu(Vs), W)
        Kf, Vf = oracle.dequant_int4(K.numpy(), Ks.numpy()), oracle.dequant_int4(V.numpy(), Vs.numpy())
    out8, out4 = run(8), run(4)
    assert maxerr(out8, oracle.attention(q.numpy(), Kf, Vf)) <= TOL
    if B >= 4 * torch.cuda.get_device_properties(0).multi_processor_count:
        assert torch.equal(out8, out4)


def test_int4_all_bytes():
    B, N, D = 3, 777, 128
    g = torch.Generator().manual_seed(4)
    q = draw(g, B, D).half()
    Kp = torch.randint(0, 256, (B, N, D // 2), generator=g, dtype=torch.uint8)
    Vp = torch.randint(0, 256, (B, N, D // 2), generator=g, dtype=torch.uint8)
    Ks = (torch.rand(B, N, generator=g) * 0.5 + 0.01).half()
    Vs = (torch.rand(B, N, generator=g) * 0.5 + 0.01).half()
    out = fq.decode_attn_int4(gpu(q), gpu(Kp), gpu(Vp), gpu(Ks), gpu(Vs), 8)
    ref = oracle.attention(q.numpy(), oracle.dequant_int4(Kp.numpy(), Ks.numpy()),
                           oracle.dequant_int4(Vp.numpy(), Vs.numpy()))
    assert maxerr(out, ref) <= TOL


# ------------------------------------------------------- dequant (exact) ----

@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("path", [0, 1])
def test_dequant_bit_exact(bits, D, path):
    g = torch.Generator().manual_seed(5)
    T = 4096
    if bits == 8:
        Kq = torch.randint(-128, 128, (T, D), generator=g, dtype=torch.int8)
        Kq[:256, 0] = torch.arange(-128, 128, dtype=torch.int16).to(torch.int8)
        want = oracle.dequant_int8
    else:
        Kq = torch.randint(0, 256, (T, D // 2), generator=g, dtype=torch.uint8)
        Kq[:256, 0] = torch.arange(256, dtype=torch.int16).to(torch.uint8)
        want = oracle.dequant_int4
    Ks = (torch.rand(T, generator=g) * 4 + 1e-4).half()
    Ks[:8] = torch.tensor([1.0, 65504.0, 6.1e-5, 5.96e-8, 0.0, -0.0, 0.3333, 2.0 ** -14]).half()
    got = fq._ext._dequant_kv(gpu(Kq), gpu(Ks), path).cpu().numpy()
    exp = want(Kq.numpy(), Ks.numpy())
    np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))


# ------------------------------------------------------------------- GQA ----

@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("B,N,W", [(1, 1024, 8), (16, 4096, 8), (1, 512, 4), (4, 512, 2), (16, 512, 8), (2, 3, 4)])
def test_gqa(B, N, W, D):
    Hq, Hkv = 32, 8
    g = torch.Generator().manual_seed(0)
    q, K, V = draw(g, B, Hq, D).half(), draw(g, B, Hkv, N, D).half(), draw(g, B, Hkv, N, D).half()
    out = fq.decode_attn_gqa(gpu(q), gpu(K), gpu(V), W)
    assert out.shape == (B, Hq, D)
    assert maxerr(out, oracle.gqa_attention(q.numpy(), K.numpy(), V.numpy())) <= TOL


@pytest.mark.parametrize("Hq,Hkv", [(32, 32), (32, 16), (24, 8), (40, 5), (64, 4), (7, 1)])
def test_gqa_group_sizes(Hq, Hkv):
    B, N, D = 2, 300, 128
    g = torch.Generator().manual_seed(6)
    q, K, V = draw(g, B, Hq, D).half(), draw(g, B, Hkv, N, D).half(), draw(g, B, Hkv, N, D).half()
    out = fq.decode_attn_gqa(gpu(q), gpu(K), gpu(V), 4)
    assert maxerr(out, oracle.gqa_attention(q.numpy(), K.numpy(), V.numpy())) <= TOL


def test_gqa_equals_repeat_kv_plus_mha():
    B, Hq, Hkv, N, D = 4, 32, 8, 512, 64
    g = torch.Generator().manual_seed(7)
    q, K, V = draw(g, B, Hq, D).half(), draw(g, B, Hkv, N, D).half(), draw(g, B, Hkv, N, D).half()
    a = fq.decode_attn_gqa(gpu(q), gpu(K), gpu(V), 8).float()
    Ke = gpu(K).repeat_interleave(Hq // Hkv, 1).reshape(B * Hq, N, D).contiguous()
    Ve = gpu(V).repeat_interleave(Hq // Hkv, 1).reshape(B * Hq, N, D).contiguous()
    b = fq.decode_attn_fp16_mw(gpu(q).reshape(B * Hq, D), Ke, Ve, 8).float().reshape(B, Hq, D)
    assert float((a - b).abs().max()) <= TOL


# --------------------------------------------------------------- split-K ----

def run_sk(q, K, V, S, W, CW):
    Hq, D = q.shape
    mp = torch.full((Hq, S), float("nan"), device=DEV)
    lp = torch.full((Hq, S), float("nan"), device=DEV)
    op = torch.full((Hq, S, D), float("nan"), device=DEV)
    o = torch.empty(Hq, D, dtype=torch.float16, device=DEV)
    assert fq.gqa_sk_fast(gpu(q), gpu(K), gpu(V), mp, lp, op, o, S, W, CW) is None
    return o, mp, lp, op


@pytest.mark.parametrize("N,D,S,W,CW", [(1024, 64, 8, 8, 4), (4096, 128, 16, 8, 4), (16384, 64, 64, 8, 8),
                                        (3, 128, 8, 4, 4), (1, 64, 4, 2, 4), (100, 64, 7, 4, 4),
                                        (16384, 128, 128, 8, 8), (512, 128, 16, 2, 8), (32768, 128, 64, 4, 4)])
def test_gqa_sk_fast_reference_cases(N, D, S, W, CW, merge_mode):
    Hq, Hkv = 32, 8
    g = torch.Generator().manual_seed(0)
    q, K, V = draw(g, Hq, D).half(), draw(g, Hkv, N, D).half(), draw(g, Hkv, N, D).half()
    o, mp, lp, op = run_sk(q, K, V, S, W, CW)
    ref = oracle.gqa_attention(q.numpy()[None], K.numpy()[None], V.numpy()[None])[0]
    assert maxerr(o, ref) <= TOL


@pytest.mark.parametrize("N,S", [(100, 7), (3, 8), (1000, 16), (1, 1)])
def test_gqa_sk_fast_scratch_layout(N, S, merge_mode):
    """m_part / l_part / o_part hold the reference's per-split (m, l, acc), empty splits (-inf, 0, 0)."""
    Hq, Hkv, D = 8, 2, 128
    g = torch.Generator().manual_seed(8)
    q, K, V = draw(g, Hq, D).half(), draw(g, Hkv, N, D).half(), draw(g, Hkv, N, D).half()
    o, mp, lp, op = run_sk(q, K, V, S, 4, 4)
    m, l, acc = oracle.split_partials(q.numpy(), K.numpy(), V.numpy(), S)
    mp, lp, op = mp.cpu().numpy(), lp.cpu().numpy(), op.cpu().numpy()
    assert np.array_equal(np.isneginf(mp), np.isneginf(m))
    fin = np.isfinite(m)
    np.testing.assert_allclose(mp[fin], m[fin], rtol=0, atol=1e-4)
    np.testing.assert_allclose(lp, l, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(op, acc, rtol=1e-4, atol=2e-4)
    assert maxerr(o, oracle.combine_partials(m, l, acc)) <= TOL


def test_gqa_sk_fast_knob_invariance(merge_mode):
    Hq, Hkv, N, D = 32, 8, 5000, 128
    g = torch.Generator().manual_seed(9)
    q, K, V = draw(g, Hq, D).half(), draw(g, Hkv, N, D).half(), draw(g, Hkv, N, D).half()
    ref = oracle.gqa_attention(q.numpy()[None], K.numpy()[None], V.numpy()[None])[0]
    for S in (1, 5, 16, 64, 300):
        for W in (2, 4, 8):
            for CW in (4, 8):
                assert maxerr(run_sk(q, K, V, S, W, CW)[0], ref) <= TOL, (S, W, CW)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("S,W", [(100, 8), (256, 8), (700, 8), (257, 2)])
def test_gqa_sk_fast_one_head_per_kv_row(D, S, W, merge_mode):
    """Hq = Hkv with many splits: the merge cuts each head's splits into slices
    on several waves (and S > 256 takes the extra m blocks)."""
    Hq, Hkv, N = 2, 2, 6000
    g = torch.Generator().manual_seed(14)
    q, K, V = draw(g, Hq, D).half(), draw(g, Hkv, N, D).half(), draw(g, Hkv, N, D).half()
    ref = oracle.gqa_attention(q.numpy()[None], K.numpy()[None], V.numpy()[None])[0]
    o, mp, lp, op = run_sk(q, K, V, S, W, 8)
    assert maxerr(o, ref) <= TOL
    m, l, acc = oracle.split_partials(q.numpy(), K.numpy(), V.numpy(), S)
    assert maxerr(o, oracle.combine_partials(m, l, acc)) <= TOL


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("S,W", [(31, 8), (32, 8), (33, 8), (32, 4)])
def test_gqa_sk_fast_merge_chunk_boundary(D, S, W, merge_mode):
    """The split merge takes a one-chunk path up to 32 splits when every
    (head, 64-dim block) has a wave of its own (S 31, 32 at W 8) and the
    general path past it (S 33) or with fewer waves than blocks (D 128, W 4):
    all agree with the oracle and with the merge of the oracle's partials."""
    Hq, Hkv, N = 32, 8, 3000
    g = torch.Generator().manual_seed(16)
    q, K, V = draw(g, Hq, D).half(), draw(g, Hkv, N, D).half(), draw(g, Hkv, N, D).half()
    o, mp, lp, op = run_sk(q, K, V, S, W, 8)
    ref = oracle.gqa_attention(q.numpy()[None], K.numpy()[None], V.numpy()[None])[0]
    assert maxerr(o, ref) <= TOL
    m, l, acc = oracle.split_partials(q.numpy(), K.numpy(), V.numpy(), S)
    assert maxerr(o, oracle.combine_partials(m, l, acc)) <= TOL


def test_gqa_sk_fast_batch_folds_into_heads(merge_mode):
    """Batch B as q [B*Hq, D], K [B*Hkv, N, D]: head b*Hq+j reads KV row b*Hkv + j/G."""
    B, Hq, Hkv, N, D = 3, 32, 8, 2048, 128
    g = torch.Generator().manual_seed(10)
    q, K, V = draw(g, B, Hq, D).half(), draw(g, B, Hkv, N, D).half(), draw(g, B, Hkv, N, D).half()
    o, *_ = run_sk(q.reshape(B * Hq, D), K.reshape(B * Hkv, N, D), V.reshape(B * Hkv, N, D), 32, 8, 8)
    ref = oracle.gqa_attention(q.numpy(), K.numpy(), V.numpy()).reshape(B * Hq, D)
    assert maxerr(o, ref) <= TOL
    o2 = fq.decode_attn_gqa(gpu(q), gpu(K), gpu(V), 8).reshape(B * Hq, D)
    assert float((o.float() - o2.float()).abs().max()) <= TOL


def test_split_merge_more_groups_than_counters():
    """More (KV row, head group) pairs than one counter slot holds (16384):
    the call falls back to the partial + combine launch pair, same result."""
    Hq = Hkv = 16400
    N, D, S = 20, 64, 3
    g = torch.Generator().manual_seed(15)
    q, K, V = draw(g, Hq, D).half(), draw(g, Hkv, N, D).half(), draw(g, Hkv, N, D).half()
    o, mp, lp, op = run_sk(q, K, V, S, 2, 4)
    ref = oracle.gqa_attention(q.numpy()[None], K.numpy()[None], V.numpy()[None])[0]
    assert maxerr(o, ref) <= TOL


def test_split_merge_many_calls_in_a_row():
    """More consecutive split calls than arrival-counter slots, with changing
    shapes: every result stays correct (counters are reset by each merge)."""
    g = torch.Generator().manual_seed(12)
    cases = []
    for i, (Hq, Hkv, N, S) in enumerate([(32, 8, 1000, 16), (8, 2, 100, 7), (64, 8, 3000, 33), (4, 1, 50, 50)] * 6):
        q, K, V = draw(g, Hq, 128).half(), draw(g, Hkv, N, 128).half(), draw(g, Hkv, N, 128).half()
        ref = oracle.gqa_attention(q.numpy()[None], K.numpy()[None], V.numpy()[None])[0]
        cases.append((run_sk(q, K, V, S, 4, 8)[0], ref))
    torch.cuda.synchronize()
    for o, ref in cases:
        assert maxerr(o, ref) <= TOL


# --------------------------------------------------------- golden files ----

def _fixture(name):
    return np.load(make_golden.path_of(name), allow_pickle=False)


@pytest.mark.parametrize("name", sorted(make_golden.CASES))
def test_golden_fixture(name):
    f = _fixture(name)
    if name.startswith("mha_f16"):
        out = fq.decode_attn_fp16_mw(gpu(f["q"]), gpu(f["K"]), gpu(f["V"]), 4)
    elif name.startswith("int8"):
        out = fq.decode_attn_int8_mw(gpu(f["q"]), gpu(f["K"]), gpu(f["V"]), gpu(f["Ks"]), gpu(f["Vs"]), 8)
        got = fq._ext._dequant_kv(gpu(f["K"]), gpu(f["Ks"]), 0).cpu().numpy()
        np.testing.assert_array_equal(got, f["Kd"])
    elif name.startswith("int4"):
        out = fq.decode_attn_int4(gpu(f["q"]), gpu(f["K"]), gpu(f["V"]), gpu(f["Ks"]), gpu(f["Vs"]), 2)
        for path in (0, 1):
            got = fq._ext._dequant_kv(gpu(f["V"]), gpu(f["Vs"]), path).cpu().numpy()
            np.testing.assert_array_equal(got, f["Vd"])
    elif name.startswith("gqa"):
        out = fq.decode_attn_gqa(gpu(f["q"]), gpu(f["K"]), gpu(f["V"]), 8)
    else:
        S = int(f["S"])
        out, mp, lp, op = run_sk(torch.from_numpy(f["q"]), torch.from_numpy(f["K"]), torch.from_numpy(f["V"]), S, 2, 8)
        np.testing.assert_array_equal(np.isneginf(mp.cpu().numpy()), np.isneginf(f["m"]))
        np.testing.assert_allclose(lp.cpu().numpy(), f["l"], rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(op.cpu().numpy(), f["acc"], rtol=1e-4, atol=2e-4)
    assert maxerr(out, f["o"].astype(np.float64)) <= TOL


# ------------------------------------------------------------ semantics ----

def test_runs_on_current_stream_and_in_graphs():
    Hq, Hkv, N, D, S = 32, 8, 4096, 128, 32
    g = torch.Generator().manual_seed(11)
    q, K, V = gpu(draw(g, Hq, D).half()), gpu(draw(g, Hkv, N, D).half()), gpu(draw(g, Hkv, N, D).half())
    mp = torch.empty(Hq, S, device=DEV)
    lp = torch.empty(Hq, S, device=DEV)
    op = torch.empty(Hq, S, D, device=DEV)
    o = torch.empty(Hq, D, dtype=torch.float16, device=DEV)
    fq.gqa_sk_fast(q, K, V, mp, lp, op, o, S, 8, 8)
    eager = o.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        o.zero_()
        fq.gqa_sk_fast(q, K, V, mp, lp, op, o, S, 8, 8)
    torch.cuda.current_stream().wait_stream(side)
    assert torch.equal(o, eager)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fq.gqa_sk_fast(q, K, V, mp, lp, op, o, S, 8, 8)
    for _ in range(3):
        o.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, eager)


def test_split_calls_on_concurrent_streams():
    """Split calls in flight on four streams at once (each call takes its own
    arrival-counter slot): every output equals the same call run alone."""
    Hq, Hkv, N, D, S = 32, 8, 3000, 128, 24
    g = torch.Generator().manual_seed(16)
    calls = []
    for i in range(8):
        q, K, V = gpu(draw(g, Hq, D).half()), gpu(draw(g, Hkv, N, D).half()), gpu(draw(g, Hkv, N, D).half())
        scratch = (torch.empty(Hq, S, device=DEV), torch.empty(Hq, S, device=DEV), torch.empty(Hq, S, D, device=DEV))
        o = torch.empty(Hq, D, dtype=torch.float16, device=DEV)
        calls.append((q, K, V, scratch, o))
    alone = []
    for q, K, V, (mp, lp, op), o in calls:
        fq.gqa_sk_fast(q, K, V, mp, lp, op, o, S, 8, 8)
        alone.append(o.clone())
        o.zero_()
    streams = [torch.cuda.Stream() for _ in range(4)]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    for i, (q, K, V, (mp, lp, op), o) in enumerate(calls):
        with torch.cuda.stream(streams[i % 4]):
            fq.gqa_sk_fast(q, K, V, mp, lp, op, o, S, 8, 8)
    for st in streams:
        torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    for (_, _, _, _, o), ref in zip(calls, alone):
        assert torch.equal(o, ref)


def test_binding_error_messages():
    q = torch.zeros(2, 64, dtype=torch.float16, device=DEV)
    K = torch.zeros(2, 16, 64, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError, match="^fp16"):
        fq.decode_attn_fp16_mw(q.float(), K, K, 8)
    with pytest.raises(RuntimeError, match="^contig"):
        fq.decode_attn_fp16_mw(q, K.transpose(1, 2), K.transpose(1, 2), 8)
    with pytest.raises(RuntimeError, match="^W"):
        fq.decode_attn_fp16_mw(q, K, K, 16)
    with pytest.raises(RuntimeError, match="^D"):
        fq.decode_attn_fp16_mw(q[:, :32].contiguous(), K[..., :32].contiguous(), K[..., :32].contiguous(), 8)
    s = torch.ones(2, 16, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError, match="^int8"):
        fq.decode_attn_int8_mw(q, K, K, s, s, 8)
    with pytest.raises(RuntimeError, match="^packed uint8"):
        fq.decode_attn_int4(q, K.to(torch.int8), K.to(torch.int8), s, s, 8)
    mp = torch.zeros(2, 4, device=DEV)
    op = torch.zeros(2, 4, 64, device=DEV)
    with pytest.raises(RuntimeError, match="^CW"):
        fq.gqa_sk_fast(q, K, K, mp, mp, op, q.clone(), 4, 8, 2)
    with pytest.raises(RuntimeError, match="^partial"):
        fq.gqa_sk_fast(q, K, K, mp, mp, op[:, :2].contiguous(), q.clone(), 4, 8, 4)
    with pytest.raises(RuntimeError, match="^combine"):
        fq.gqa_sk_fast(q, K, K, mp, mp, op, q[:1].clone(), 4, 8, 4)
