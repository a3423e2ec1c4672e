"""numpy restatement of the reference's decode-attention math (test oracle only).

All functions take numpy arrays of any float dtype (fp16 inputs are widened
exactly) and compute in float64, which is strictly more accurate than the
fp32 softmax(qK^T/sqrt(D))V the tolerance is stated against.
"""

import numpy as np


def softmax_scale(D):
    """The reference's score scale, ``1.0f/sqrtf((float)D)`` evaluated in fp32.

    decode_attn_fp16_mw.cu:55, decode_attn_gqa.cu:60 (via ``scale``),
    decode_attn_gqa_sk_fast.cu:98 (``1.0f/sqrtf((float)D)``),
    decode_attn_int4.cu:51 (``1.0f/sqrtf(64.0f)``).
    """
    return float(np.float32(1.0) / np.sqrt(np.float32(D)))


def round_fp16(x):
    """Round to fp16 with round-to-nearest-even (``__float2half``,
    decode_attn_fp16_mw.cu:47), going through fp32 as the kernels do."""
    return np.asarray(x, dtype=np.float64).astype(np.float32).astype(np.float16)


def attention(q, K, V, scale=None):
    """Single-query attention per row: o[r] = softmax(q[r] . K[r]^T * scale) V[r].

    q: [R, D], K, V: [R, N, D] -> float64 [R, D].
    Follows decode_attn_fp16_mw.cu:19-31 (score = dot * scale, online softmax
    over all N tokens) whose fixed point is the plain softmax; N must be >= 1
    (the reference divides by l, decode_attn_fp16_mw.cu:47).
    """
    q = np.asarray(q, dtype=np.float64)
    K = np.asarray(K, dtype=np.float64)
    V = np.asarray(V, dtype=np.float64)
    R, N, D = K.shape
    if N < 1:
        raise ValueError("N must be >= 1")
    assert q.shape == (R, D) and V.shape == (R, N, D)
    if scale is None:
        scale = softmax_scale(D)
    s = np.einsum("rnd,rd->rn", K, q) * scale
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    return np.einsum("rn,rnd->rd", p, V) / p.sum(axis=1, keepdims=True)


def gqa_attention(q, K, V, scale=None):
    """GQA decode: q [B, Hq, D], K, V [B, Hkv, N, D] -> [B, Hq, D] float64.

    Query head h reads KV head h // G with G = Hq // Hkv
    (decode_attn_gqa.cu:13 ``kvh=h/G``), i.e. ``repeat_interleave(G, dim=1)``
    as the reference test builds its oracle (tests/test_kernels.py:49-50).
    """
    q = np.asarray(q)
    K = np.asarray(K)
    V = np.asarray(V)
    B, Hq, D = q.shape
    Hkv, N = K.shape[1], K.shape[2]
    assert Hq % Hkv == 0
    G = Hq // Hkv
    Ke = np.repeat(K, G, axis=1).reshape(B * Hq, N, D)
    Ve = np.repeat(V, G, axis=1).reshape(B * Hq, N, D)
    return attention(q.reshape(B * Hq, D), Ke, Ve, scale).reshape(B, Hq, D)


def split_bounds(N, S):
    """Token range of each split: chunk = ceil(N/S), [s*chunk, min(s*chunk+chunk, N)).

    decode_attn_gqa_sk_fast.cu:13. Splits past the end are empty.
    """
    chunk = (N + S - 1) // S
    out = []
    for s in range(S):
        lo = s * chunk
        hi = min(lo + chunk, N)
        out.append((lo, max(lo, hi)))
    return out


def split_partials(q, K, V, S, scale=None):
    """Split-K partials in the reference scratch layout.

    q: [Hq, D], K, V: [Hkv, N, D]. Returns float64 (m [Hq, S], l [Hq, S],
    acc [Hq, S, D]) where, over split s's tokens t with scores
    x_t = (q . K_t) * scale: m = max x_t, l = sum exp(x_t - m),
    acc = sum exp(x_t - m) V_t (unnormalised). An empty split stores
    m = -inf, l = 0, acc = 0 (decode_attn_gqa_sk_fast.cu:39-52 with the
    guards at :45-46). Query head h reads KV head h // G (:11).
    """
    q = np.asarray(q, dtype=np.float64)
    K = np.asarray(K, dtype=np.float64)
    V = np.asarray(V, dtype=np.float64)
    Hq, D = q.shape
    Hkv, N, _ = K.shape
    G = Hq // Hkv
    if scale is None:
        scale = softmax_scale(D)
    m = np.full((Hq, S), -np.inf)
    l = np.zeros((Hq, S))
    acc = np.zeros((Hq, S, D))
    for h in range(Hq):
        kv = h // G
        x = K[kv] @ q[h] * scale
        for s, (lo, hi) in enumerate(split_bounds(N, S)):
            if hi <= lo:
                continue
            xs = x[lo:hi]
            ms = xs.max()
            p = np.exp(xs - ms)
            m[h, s] = ms
            l[h, s] = p.sum()
            acc[h, s] = p @ V[kv, lo:hi]
    return m, l, acc


def combine_partials(m, l, acc):
    """Merge split partials: o = sum_s e^(m_s-M) acc_s / sum_s e^(m_s-M) l_s.

    decode_attn_gqa_sk_fast.cu:66-72 and :85-92; a split whose m is -inf
    contributes weight 0. m, l: [H, S], acc: [H, S, D] -> float64 [H, D].
    """
    m = np.asarray(m, dtype=np.float64)
    l = np.asarray(l, dtype=np.float64)
    acc = np.asarray(acc, dtype=np.float64)
    M = m.max(axis=1, keepdims=True)
    w = np.where(np.isneginf(m), 0.0, np.exp(m - np.where(np.isneginf(M), 0.0, M)))
    L = (w * l).sum(axis=1)
    O = np.einsum("hs,hsd->hd", w, acc)
    return O / L[:, None]
