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
