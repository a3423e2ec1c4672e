"""numpy restatement of the reference's per-token KV quantizers (test oracle only).

The reference quantizes with PyTorch tensor expressions whose rounding depends
on the input dtype: on an fp16 tensor every elementwise op is evaluated in fp32
and rounded back to fp16; on an fp32 tensor the ops are plain fp32. The
restatement follows the same dtype rule, so it reproduces the reference's
bytes for both the reference tests' fp16 draws and fp32 draws.

The reference runs its quantizers on CUDA tensors (tests/test_kernels.py:27-33,
``dev="cuda"``). There PyTorch evaluates ``a / 127.0`` -- a tensor divided by
a Python scalar -- as ``a * fp32(1/127)`` (its CUDA true-division kernel
multiplies by the reciprocal of a CPU scalar), while ``X / s`` -- tensor by
tensor -- is a true division. The restatement follows that arithmetic, which
also makes it device-independent: ``a * (1/qmax)`` rounds the same on CPU.
"""

import numpy as np


def _recip(qmax):
    """fp32(1/qmax): the multiplier PyTorch uses for ``tensor / qmax``."""
    return np.float32(1.0) / np.float32(qmax)


def _per_token(X, qmax):
    """Shared body of the int8 and int4 quantizers.

    a = max|x| over the last axis; s = max(a * fp32(1/qmax), 1e-8); q = round(x/s)
    (round-half-even, ``torch.round``) clamped to [-qmax, qmax]; the stored
    scale is ``s.half()``. tests/test_kernels.py:32-34 (qmax=127),
    nb:292-295 (qmax=7).

    Rows whose fp16 scale underflows to 0 (only possible for fp16 inputs with
    max|x| < ~4e-6) make the reference divide by zero; here x = 0 maps to 0
    and any other x to +-qmax, which is what the reference's clamp yields for
    +-inf.
    """
    X = np.asarray(X)
    if X.dtype == np.float16:
        a = np.abs(X).max(axis=-1, keepdims=True)
        s = (a.astype(np.float32) * _recip(qmax)).astype(np.float16)
        s = np.maximum(s.astype(np.float32), np.float32(1e-8)).astype(np.float16)
        s32 = s.astype(np.float32)
        with np.errstate(divide="ignore", invalid="ignore"):
            quot = (X.astype(np.float32) / s32).astype(np.float16).astype(np.float32)
        quot = np.where(s32 == 0, np.where(X == 0, 0.0, np.sign(X.astype(np.float32)) * qmax), quot)
        scale16 = s
    elif X.dtype == np.float32:
        a = np.abs(X).max(axis=-1, keepdims=True)
        s = np.maximum(a * _recip(qmax), np.float32(1e-8)).astype(np.float32)
        quot = (X / s).astype(np.float32)
        scale16 = s.astype(np.float16)
    else:
        raise TypeError("quantizer input must be float16 or float32, got %s" % X.dtype)
    q = np.clip(np.rint(quot), -qmax, qmax).astype(np.int8)
    return q, scale16[..., 0]


def quant_int8_per_token(X):
    """Per-token symmetric int8: returns (int8 [..., D], fp16 scales [...]).

    tests/test_kernels.py:32-34, nb:236-238.
    """
    return _per_token(X, 127)


def pack_int4(q):
    """Pack int4 values two per byte, low nibble first along D.

    byte t = (q[2t] & 0xF) | ((q[2t+1] & 0xF) << 4)  (nb:296-298).
    q: int8 [..., D] with values in [-8, 7] -> uint8 [..., D/2].
    """
    q = np.asarray(q).astype(np.int16)
    if q.shape[-1] % 2:
        raise ValueError("D must be even")
    if q.min(initial=0) < -8 or q.max(initial=0) > 7:
        raise ValueError("int4 values must lie in [-8, 7]")
    lo = q[..., 0::2] & 0xF
    hi = q[..., 1::2] & 0xF
    return (lo | (hi << 4)).astype(np.uint8)


def unpack_int4(P):
    """Inverse of ``pack_int4``: uint8 [..., H] -> int8 [..., 2H].

    Nibble n decodes as n - 16 when n >= 8 (decode_attn_int4.cu:22,30,
    nb:303-305), so 0x8 -> -8 is decodable although the quantizer never
    emits it.
    """
    b = np.asarray(P).astype(np.int16)
    lo = b & 0xF
    hi = (b >> 4) & 0xF
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    out = np.empty(b.shape[:-1] + (2 * b.shape[-1],), dtype=np.int8)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out


def quant_int4_per_token(X):
    """Per-token symmetric int4, packed: returns (uint8 [..., D/2], fp16 scales).

    nb:292-299 (scale max|x|/7, values clamped to [-7, 7], low nibble first).
    With s = max|x|/7 no value rounds past 7, so the [-8, 7] clamp of the
    int4 config gives the same bytes.
    """
    q, s = _per_token(X, 7)
    return pack_int4(q), s


def dequant_int8(Kq, Ks):
    """float(q) * float(scale) in fp32 (decode_attn_int8_mw.cu:24,31).

    The product of an int8 (<= 8 significant bits) and an fp16 scale
    (11 bits) is exact in fp32, so this value is unique.
    """
    return np.asarray(Kq).astype(np.float32) * np.asarray(Ks).astype(np.float32)[..., None]


def dequant_int4(P, Ks):
    """Unpack (low nibble first) then float(q) * float(scale) in fp32.

    decode_attn_int4.cu:21-23,29-31; nb:301-307.
    """
    return unpack_int4(P).astype(np.float32) * np.asarray(Ks).astype(np.float32)[..., None]


# ------------------------------------------------------------------ fp8 ----
# OCP fp8 e4m3 ("E4M3FN"): 1 sign bit, 4 exponent bits (bias 7), 3 mantissa
# bits, no infinities; S.1111.111 is NaN; the largest finite value is 448, the
# smallest normal 2^-6, the subnormal step 2^-9. The fp8 KV format has no
# counterpart in the reference: it is this library's own, defined here as the
# fp32 expressions below (the same shape as the int8 quantizer, with the
# round-to-nearest-even of e4m3 in place of round-to-integer).

FP8_MAX = 448.0


def e4m3_encode(x):
    """float32 values with |x| <= 448 -> e4m3 codes (uint8), round to nearest even."""
    x = np.asarray(x, dtype=np.float32)
    sign = np.signbit(x).astype(np.uint16) << 7
    a = np.abs(x).astype(np.float64)
    _, e = np.frexp(a)
    e = np.maximum(e - 1, -6)                 # binade of a (subnormals share 2^-6)
    step = np.ldexp(1.0, e - 3)               # 3 mantissa bits
    q = np.rint(a / step) * step              # exact in float64; may carry to 2^(e+1)
    _, e2 = np.frexp(q)
    e2 = e2 - 1
    normal = q >= 2.0 ** -6
    exp_field = np.where(normal, e2 + 7, 0).astype(np.uint16)
    mant = np.where(normal, np.rint((q / np.ldexp(1.0, e2) - 1.0) * 8.0), np.rint(q / 2.0 ** -9)).astype(np.uint16)
    return (sign | (exp_field << 3) | mant).astype(np.uint8)


def e4m3_decode(codes):
    """e4m3 codes (uint8) -> float32 values (NaN for S.1111.111)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int32)
    e = (c >> 3) & 0xF
    m = c & 0x7
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.ldexp(1.0, e - 7))
    val = np.where((c & 0x80) != 0, -mag, mag)
    return np.where((c & 0x7F) == 0x7F, np.nan, val).astype(np.float32)


def quant_fp8_per_token(X):
    """Per-token fp8 e4m3: returns (uint8 codes [..., D], fp16 scales [...]).

    In fp32 on the widened input (fp16 and bf16 widen exactly): a = max|x|,
    s = max(a * fp32(1/448), 1e-8), code = e4m3(clamp(x / s, -448, 448)) with
    a true fp32 division (an exact zero as +0); the stored scale is fp16(s).
    """
    X32 = np.asarray(X).astype(np.float32)
    a = np.abs(X32).max(axis=-1, keepdims=True)
    s = np.maximum(a * _recip(FP8_MAX), np.float32(1e-8)).astype(np.float32)
    q = np.clip(X32 / s, np.float32(-FP8_MAX), np.float32(FP8_MAX))
    q = np.where(q == 0, np.float32(0.0), q)  # an exact zero (x = -0 too) is stored as +0
    return e4m3_encode(q), s[..., 0].astype(np.float16)


def dequant_fp8(codes, Ks):
    """e4m3 value of each code times float(scale), in fp32 (exact: 4 x 11 significant bits)."""
    return e4m3_decode(codes) * np.asarray(Ks).astype(np.float32)[..., None]
