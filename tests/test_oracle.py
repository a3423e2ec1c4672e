"""Pins for the CPU oracle (runs without a GPU).

Each oracle function is checked against something independent of its own
formula, chosen so that a plausible mistake (a dropped scale, a transposed
operand, a wrong GQA head map, an off-by-one split bound, a swapped nibble,
a round-half-up instead of half-even) fails at least one test:

* the reference notebook's recorded CPU-RNG output (nb:283, cell 5:
  "int4 dequant vs original: rel 7.1036e-02", "pack/unpack exact: True");
* closed forms (N = 1, q = 0, a dominant key, per-split sums);
* PyTorch library routines (scaled_dot_product_attention; fp16 / fp32
  tensor arithmetic for the quantizer rounding);
* brute-force pure-Python loops on tiny inputs;
* hand-built known-answer bytes and values.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle


def _rng(seed=0):
    return np.random.default_rng(seed)


# ----------------------------------------------------------------- scale ----

def test_softmax_scale_is_fp32_rsqrt():
    assert oracle.softmax_scale(64) == 0.125
    s128 = oracle.softmax_scale(128)
    assert s128 == float(np.float32(1) / np.sqrt(np.float32(128)))
    assert abs(s128 - 1 / math.sqrt(128)) < 1e-8


# ------------------------------------------------------------- attention ----

@pytest.mark.parametrize("R,N,D", [(3, 17, 64), (2, 300, 128), (1, 1, 64)])
def test_attention_matches_torch_sdpa(R, N, D):
    g = torch.Generator().manual_seed(1)
    q = torch.randn(R, D, generator=g, dtype=torch.float64)
    K = torch.randn(R, N, D, generator=g, dtype=torch.float64)
    V = torch.randn(R, N, D, generator=g, dtype=torch.float64)
    ref = F.scaled_dot_product_attention(q.view(R, 1, 1, D), K.view(R, 1, N, D), V.view(R, 1, N, D),
                                         scale=oracle.softmax_scale(D)).view(R, D).numpy()
    got = oracle.attention(q.numpy(), K.numpy(), V.numpy())
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-12)


def test_attention_default_scale_is_inverse_sqrt_d():
    # torch SDPA's own default scale is 1/sqrt(D): a dropped or squared scale fails here
    g = torch.Generator().manual_seed(2)
    q = torch.randn(2, 128, generator=g, dtype=torch.float64) * 3
    K = torch.randn(2, 40, 128, generator=g, dtype=torch.float64)
    V = torch.randn(2, 40, 128, generator=g, dtype=torch.float64)
    ref = F.scaled_dot_product_attention(q.view(2, 1, 1, 128), K.view(2, 1, 40, 128),
                                         V.view(2, 1, 40, 128)).view(2, 128).numpy()
    np.testing.assert_allclose(oracle.attention(q.numpy(), K.numpy(), V.numpy()), ref, atol=1e-7)


def test_attention_single_token_returns_v0():
    r = _rng(3)
    q = r.standard_normal((4, 64))
    K = r.standard_normal((4, 1, 64))
    V = r.standard_normal((4, 1, 64))
    np.testing.assert_array_equal(oracle.attention(q, K, V), V[:, 0])


def test_attention_zero_query_averages_values():
    r = _rng(4)
    K = r.standard_normal((2, 9, 64))
    V = r.standard_normal((2, 9, 64))
    got = oracle.attention(np.zeros((2, 64)), K, V)
    np.testing.assert_allclose(got, V.mean(axis=1), atol=1e-14)


def test_attention_dominant_key_selects_its_value():
    r = _rng(5)
    K = r.standard_normal((1, 12, 64)) * 0.01
    q = np.zeros((1, 64))
    q[0, 7] = 1.0
    K[0, 5, 7] = 400.0  # score 400/8 = 50 above the rest
    V = r.standard_normal((1, 12, 64))
    got = oracle.attention(q, K, V)
    np.testing.assert_allclose(got[0], V[0, 5], atol=1e-15 + 1e-20)


def test_attention_brute_force_loops():
    r = _rng(6)
    R, N, D = 2, 5, 4
    q, K, V = r.standard_normal((R, D)), r.standard_normal((R, N, D)), r.standard_normal((R, N, D))
    scale = 1 / math.sqrt(D)
    want = np.zeros((R, D))
    for i in range(R):
        scores = [sum(q[i, d] * K[i, n, d] for d in range(D)) * scale for n in range(N)]
        mx = max(scores)
        e = [math.exp(s - mx) for s in scores]
        for d in range(D):
            want[i, d] = sum(e[n] * V[i, n, d] for n in range(N)) / sum(e)
    np.testing.assert_allclose(oracle.attention(q, K, V, scale=scale), want, atol=1e-14)


def test_attention_is_token_permutation_invariant():
    r = _rng(7)
    q, K, V = r.standard_normal((2, 64)), r.standard_normal((2, 33, 64)), r.standard_normal((2, 33, 64))
    perm = r.permutation(33)
    np.testing.assert_allclose(oracle.attention(q, K, V), oracle.attention(q, K[:, perm], V[:, perm]), atol=1e-14)


def test_attention_rejects_empty_sequence():
    with pytest.raises(ValueError):
        oracle.attention(np.zeros((1, 64)), np.zeros((1, 0, 64)), np.zeros((1, 0, 64)))


# ------------------------------------------------------------------- GQA ----

def test_gqa_head_map_is_h_div_g():
    # every KV head holds a distinct constant value vector, so the output names the KV head read
    B, Hq, Hkv, N, D = 2, 12, 3, 4, 64
    G = Hq // Hkv
    q = _rng(8).standard_normal((B, Hq, D))
    K = _rng(9).standard_normal((B, Hkv, N, D))
    V = np.zeros((B, Hkv, N, D))
    for b in range(B):
        for k in range(Hkv):
            V[b, k] = 10 * b + k
    o = oracle.gqa_attention(q, K, V)
    for b in range(B):
        for h in range(Hq):
            np.testing.assert_allclose(o[b, h], 10 * b + h // G, atol=1e-12)


def test_gqa_matches_torch_sdpa_with_repeat_interleave():
    g = torch.Generator().manual_seed(10)
    B, Hq, Hkv, N, D = 2, 8, 2, 21, 64
    q = torch.randn(B, Hq, D, generator=g, dtype=torch.float64)
    K = torch.randn(B, Hkv, N, D, generator=g, dtype=torch.float64)
    V = torch.randn(B, Hkv, N, D, generator=g, dtype=torch.float64)
    ref = F.scaled_dot_product_attention(q.view(B, Hq, 1, D), K.repeat_interleave(Hq // Hkv, 1),
                                         V.repeat_interleave(Hq // Hkv, 1)).view(B, Hq, D).numpy()
    np.testing.assert_allclose(oracle.gqa_attention(q.numpy(), K.numpy(), V.numpy()), ref, atol=1e-12)


# --------------------------------------------------------------- split-K ----

def test_split_bounds_follow_ceil_chunks():
    assert oracle.split_bounds(100, 7) == [(0, 15), (15, 30), (30, 45), (45, 60), (60, 75), (75, 90), (90, 100)]
    assert oracle.split_bounds(3, 8) == [(0, 1), (1, 2), (2, 3)] + [(s, s) for s in range(3, 8)]
    assert oracle.split_bounds(1, 4) == [(0, 1), (1, 1), (2, 2), (3, 3)]
    # chunk = ceil(10/4) = 3 -> the last split is short
    assert oracle.split_bounds(10, 4) == [(0, 3), (3, 6), (6, 9), (9, 10)]


@pytest.mark.parametrize("N,S", [(100, 7), (3, 8), (1, 4), (64, 64), (1024, 8)])
def test_split_partials_combine_to_attention(N, S):
    r = _rng(11)
    Hq, Hkv, D = 8, 2, 64
    q, K, V = r.standard_normal((Hq, D)), r.standard_normal((Hkv, N, D)), r.standard_normal((Hkv, N, D))
    m, l, acc = oracle.split_partials(q, K, V, S)
    o = oracle.combine_partials(m, l, acc)
    want = oracle.gqa_attention(q[None], K[None], V[None])[0]
    np.testing.assert_allclose(o, want, atol=1e-12)


def test_split_partials_closed_form_brute_force():
    r = _rng(12)
    Hq, Hkv, N, D, S = 4, 2, 7, 4, 3
    q, K, V = r.standard_normal((Hq, D)), r.standard_normal((Hkv, N, D)), r.standard_normal((Hkv, N, D))
    sc = 0.5
    m, l, acc = oracle.split_partials(q, K, V, S, scale=sc)
    chunk = math.ceil(N / S)
    for h in range(Hq):
        kv = h // (Hq // Hkv)
        for s in range(S):
            toks = list(range(s * chunk, min(s * chunk + chunk, N)))
            x = [sum(q[h, d] * K[kv, t, d] for d in range(D)) * sc for t in toks]
            mx = max(x)
            assert m[h, s] == pytest.approx(mx, abs=1e-12)
            assert l[h, s] == pytest.approx(sum(math.exp(v - mx) for v in x), abs=1e-12)
            for d in range(D):
                want = sum(math.exp(x[i] - mx) * V[kv, t, d] for i, t in enumerate(toks))
                assert acc[h, s, d] == pytest.approx(want, abs=1e-12)


def test_empty_splits_store_neutral_partials():
    r = _rng(13)
    m, l, acc = oracle.split_partials(r.standard_normal((4, 64)), r.standard_normal((1, 3, 64)),
                                      r.standard_normal((1, 3, 64)), 8)
    assert np.all(np.isneginf(m[:, 3:]))
    assert np.all(l[:, 3:] == 0) and np.all(acc[:, 3:] == 0)
    assert np.all(np.isfinite(m[:, :3]))


def test_combine_is_invariant_to_split_order_and_shift():
    r = _rng(14)
    m = r.standard_normal((3, 5))
    l = r.random((3, 5)) + 0.5
    acc = r.standard_normal((3, 5, 64))
    o = oracle.combine_partials(m, l, acc)
    perm = r.permutation(5)
    np.testing.assert_allclose(oracle.combine_partials(m[:, perm], l[:, perm], acc[:, perm]), o, atol=1e-14)
    # (m, l, acc) and (m + c, l e^-c, acc e^-c) describe the same partial
    c = 3.0
    np.testing.assert_allclose(oracle.combine_partials(m + c, l * math.exp(-c), acc * math.exp(-c)), o, atol=1e-12)


# ------------------------------------------------------------ quantizers ----

def _torch_quant(X, qmax):
    """The reference quantizer expression as PyTorch evaluates it on the reference's CUDA
    tensors (tests/test_kernels.py:27-33): ``a / qmax`` (tensor by Python scalar) is a
    multiplication by fp32(1/qmax) there, ``X / s`` a true division. Evaluated here by
    PyTorch on CPU tensors with the multiplication written out."""
    a = X.abs().amax(-1, keepdim=True)
    s = (a * (1.0 / float(qmax))).clamp(min=1e-8)
    return torch.clamp(torch.round(X / s), -qmax, qmax).to(torch.int8), s.squeeze(-1).half()


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("qmax", [127, 7])
def test_quantizer_rounding_matches_torch_arithmetic(dtype, qmax):
    g = torch.Generator().manual_seed(15)
    X = torch.randn(4, 257, 64, generator=g, dtype=torch.float32).to(dtype)
    X[0, 0] = 0.5 * (torch.arange(64, dtype=torch.float32) - 32).to(dtype)  # ties at +-k.5 after scaling
    tq, ts = _torch_quant(X, qmax)
    oq, os_ = oracle.quant._per_token(X.numpy(), qmax)
    np.testing.assert_array_equal(oq, tq.numpy())
    np.testing.assert_array_equal(os_.view(np.uint16), ts.numpy().view(np.uint16))


def test_int8_known_answers():
    X = np.array([[[127.0, -63.5, 0.5, 1.5, -2.5, 0.0, -127.0, 64.49]]], dtype=np.float32)
    q, s = oracle.quant_int8_per_token(X)
    assert s.dtype == np.float16 and s[0, 0] == np.float16(1.0)
    # round half to even: -63.5 -> -64, 0.5 -> 0, 1.5 -> 2, -2.5 -> -2
    np.testing.assert_array_equal(q[0, 0], [127, -64, 0, 2, -2, 0, -127, 64])


def test_int8_invariants():
    X = _rng(16).standard_normal((8, 100, 128)).astype(np.float32) * 3
    q, s = oracle.quant_int8_per_token(X)
    assert q.dtype == np.int8 and np.abs(q.astype(int)).max() <= 127
    s32 = np.maximum(np.abs(X).max(-1, keepdims=True) / np.float32(127), np.float32(1e-8))
    assert np.all(np.abs(X - q * s32) <= s32 / 2 * (1 + 1e-6))
    assert np.all(np.abs(q).max(-1) == 127)  # the max element always maps to +-127


def test_int4_notebook_golden_value():
    """nb:283 (cell 5, CPU RNG): seed 0, X = randn(2,1024,64) fp16 ->
    'pack/unpack exact: True' and 'int4 dequant vs original: rel 7.1036e-02'."""
    torch.manual_seed(0)
    X = torch.randn(2, 1024, 64, dtype=torch.float16).numpy()
    P, s = oracle.quant_int4_per_token(X)
    deq = oracle.dequant_int4(P, s)
    rel = np.abs(deq - X.astype(np.float32)).max() / np.abs(X.astype(np.float32)).max()
    assert f"{rel:.4e}" == "7.1036e-02"
    q, _ = oracle.quant._per_token(X, 7)
    np.testing.assert_array_equal(oracle.unpack_int4(P), q)  # pack/unpack exact


def test_int4_edge_bytes_known_answers():
    P = np.array([[0x80, 0x7F, 0x88, 0x08, 0xF7, 0x00, 0xFF]], dtype=np.uint8)
    want = [0, -8, -1, 7, -8, -8, -8, 0, 7, -1, 0, 0, -1, -1]
    np.testing.assert_array_equal(oracle.unpack_int4(P)[0], want)
    np.testing.assert_array_equal(oracle.pack_int4(np.array([want], dtype=np.int8)), P)


def test_int4_pack_roundtrip_all_bytes():
    P = np.arange(256, dtype=np.uint8).reshape(1, 256)
    np.testing.assert_array_equal(oracle.pack_int4(oracle.unpack_int4(P)), P)
    vals = np.array([[v for v in range(-8, 8) for _ in range(2)]], dtype=np.int8)
    np.testing.assert_array_equal(oracle.unpack_int4(oracle.pack_int4(vals)), vals)


def test_int4_quantizer_never_emits_minus_eight_and_low_nibble_is_even_element():
    X = np.zeros((1, 1, 4), dtype=np.float32)
    X[0, 0] = [7.0, -3.0, 1.0, -7.0]
    P, s = oracle.quant_int4_per_token(X)
    assert s[0, 0] == np.float16(1.0)
    # byte 0 = (7 & 0xF) | ((-3 & 0xF) << 4) = 0xD7; byte 1 = 1 | (0x9 << 4) = 0x91
    np.testing.assert_array_equal(P[0, 0], [0xD7, 0x91])
    Y = _rng(17).standard_normal((16, 256, 128)).astype(np.float32)
    assert oracle.unpack_int4(oracle.quant_int4_per_token(Y)[0]).min() >= -7


@pytest.mark.parametrize("bits", [8, 4])
def test_dequant_is_exact_fp32_product(bits):
    X = _rng(18).standard_normal((4, 50, 128)).astype(np.float32)
    if bits == 8:
        q, s = oracle.quant_int8_per_token(X)
        vals = q.astype(np.float64)
        deq = oracle.dequant_int8(q, s)
    else:
        P, s = oracle.quant_int4_per_token(X)
        vals = oracle.unpack_int4(P).astype(np.float64)
        deq = oracle.dequant_int4(P, s)
    exact = vals * s.astype(np.float64)[..., None]
    assert deq.dtype == np.float32
    np.testing.assert_array_equal(deq.astype(np.float64), exact)  # no rounding happened


def test_round_fp16_is_nearest_even():
    x = np.array([1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 65519.0, -0.0])
    np.testing.assert_array_equal(oracle.round_fp16(x).astype(np.float64), [1.0, 1.0 + 2 * 2.0 ** -10, 65504.0, -0.0])


# ------------------------------------------------------------------ fp8 ----
# The fp8 e4m3 KV format has no counterpart in the reference; the oracle states
# its definition, pinned here against torch's float8_e4m3fn conversions (a
# library routine), a brute-force grid and known answers.

def test_e4m3_decode_matches_torch_for_every_code():
    import torch

    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = oracle.e4m3_decode(codes)
    assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.isnan(got).sum() == 2  # 0x7F, 0xFF
    np.testing.assert_array_equal(got[~np.isnan(got)], ref[~np.isnan(ref)])
    assert got[0x7E] == 448.0 and got[0x08] == 2.0 ** -6 and got[0x01] == 2.0 ** -9 and got[0xB8] == -1.0


def test_e4m3_encode_is_round_to_nearest_even():
    """Against torch on every representable value, every midpoint between neighbours (ties: to
    the even code), the floats next to each midpoint, subnormals and random values; and against
    a brute-force nearest search on a grid."""
    import torch

    vals = np.unique(oracle.e4m3_decode(np.arange(256, dtype=np.uint8)))
    vals = vals[~np.isnan(vals)]
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32)
    x = np.concatenate([vals, mids, np.nextafter(mids, np.float32(-1000)), np.nextafter(mids, np.float32(1000)),
                        (_rng(30).standard_normal(100000) * 60).astype(np.float32),
                        np.float32([2.0 ** -10, 3 * 2.0 ** -11, 1e-30, -1e-30])])
    x = x[np.abs(x) <= 448]
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(oracle.e4m3_encode(x), ref)
    # brute force: the nearest representable value, ties to the even mantissa
    grid = np.linspace(-448, 448, 20001).astype(np.float32)
    finite = np.arange(256, dtype=np.uint8)[~np.isnan(oracle.e4m3_decode(np.arange(256, dtype=np.uint8)))]
    fv = oracle.e4m3_decode(finite).astype(np.float64)
    for xv in grid[::37]:
        d = np.abs(fv - float(xv))
        best = finite[d == d.min()]
        code = oracle.e4m3_encode(np.float32([xv]))[0]
        assert code in best and (len(best) == 1 or (code & 1) == 0 or oracle.e4m3_decode(np.uint8([code]))[0] == 0)


def test_fp8_quantizer_known_answers_and_invariants():
    X = np.zeros((3, 8), np.float32)
    X[0, :4] = [448.0, -224.0, 1.0, 0.0]   # s = 448 * fp32(1/448), codes near the values
    X[1, :] = 0.0                           # all zero: s = 1e-8, codes 0
    X[2, :3] = [1e-3, -2e-3, -0.0]
    q, s = oracle.quant_fp8_per_token(X)
    assert s.dtype == np.float16 and q.dtype == np.uint8
    s32 = np.float32(448.0) * (np.float32(1.0) / np.float32(448.0))
    assert s[0] == np.float16(s32)
    np.testing.assert_array_equal(oracle.e4m3_decode(q[0, :4]), np.float32([448.0, -224.0, 1.0, 0.0]))
    assert not q[1].any() and s[1] == np.float16(1e-8)
    assert q[2, 2] == 0  # -0 is stored as +0
    # every code decodes within half a step of x / s; the row maximum maps to +-448
    Y = _rng(31).standard_normal((50, 128)).astype(np.float32) * 7
    q, s = oracle.quant_fp8_per_token(Y)
    s32 = np.maximum(np.abs(Y).max(-1) * (np.float32(1.0) / np.float32(448.0)), np.float32(1e-8))
    r = Y / s32[:, None]
    v = oracle.e4m3_decode(q)
    assert np.all(np.abs(v - r) <= np.abs(r) * 2.0 ** -4 + 2.0 ** -10)
    assert np.all(np.abs(v).max(-1) == 448.0)


def test_fp8_quantizer_matches_the_pytorch_restatement():
    """fqkv_decode.quant.quant_fp8_per_token (torch tensor ops, float8_e4m3fn conversion) gives the
    oracle's bytes for fp32, fp16 and bf16 rows."""
    import torch
    from fqkv_decode import quant

    g = torch.Generator().manual_seed(32)
    for dt in (torch.float32, torch.float16, torch.bfloat16):
        X = (torch.randn(16, 33, 128, generator=g) * 3).to(dt)
        X[0, 0] = 0
        X[0, 1, :5] = -0.0
        q, s = quant.quant_fp8_per_token(X)
        oq, os_ = oracle.quant_fp8_per_token(X.float().numpy())
        np.testing.assert_array_equal(q.view(torch.uint8).numpy(), oq)
        np.testing.assert_array_equal(s.numpy(), os_)
        np.testing.assert_array_equal(quant.dequant_fp8(q, s).numpy(), oracle.dequant_fp8(oq, os_))
