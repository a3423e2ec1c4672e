"""Per-token KV quantizers: the on-memory formats the int8 / int4 kernels read.

PyTorch tensor code, as in the reference, so the bytes match the reference's
on any device for fp16 and fp32 inputs alike:

* int8: tests/test_kernels.py:32-34 (nb:236-238) -- scale = max|x|/127
  (evaluated, as PyTorch does on the reference's CUDA tensors, as
  max|x| * fp32(1/127)) clamped to >= 1e-8, values round(x/scale) clamped to
  [-127, 127], scales stored as fp16 [.., N].
* int4: nb:292-299 -- scale = max|x|/7, values clamped to [-7, 7], packed two
  per byte with the low nibble holding the even element.
* dequantisation: nb:301-307 and decode_attn_int8_mw.cu:24,31 --
  (float)q * (float)scale, exact in fp32.
"""

import torch


def _scales(X, qmax):
    # The reference writes a / qmax on CUDA tensors, which PyTorch evaluates
    # as a * fp32(1/qmax); writing the multiplication makes CPU tensors round
    # the same way, so the bytes do not depend on the device.
    a = X.abs().amax(-1, keepdim=True)
    s = (a * (1.0 / float(qmax))).clamp(min=1e-8)
    return s


def quant_int8_per_token(X):
    """X [..., N, D] (fp16 or fp32) -> (int8 [..., N, D], fp16 scales [..., N])."""
    s = _scales(X, 127)
    q = torch.clamp(torch.round(X / s), -127, 127).to(torch.int8).contiguous()
    return q, s.squeeze(-1).half().contiguous()


def pack_int4(q):
    """int8 values in [-8, 7], [..., D] -> uint8 [..., D/2], low nibble = even element."""
    q = q.view(*q.shape[:-1], q.shape[-1] // 2, 2)
    lo = q[..., 0] & 0xF
    hi = q[..., 1] & 0xF
    return (lo | (hi << 4)).to(torch.uint8).contiguous()


def unpack_int4(packed):
    """uint8 [..., H] -> int8 [..., 2H]; nibble n >= 8 decodes as n - 16."""
    b = packed.to(torch.int16)
    lo = b & 0xF
    hi = (b >> 4) & 0xF
    lo = torch.where(lo >= 8, lo - 16, lo)
    hi = torch.where(hi >= 8, hi - 16, hi)
    return torch.stack([lo, hi], dim=-1).reshape(*packed.shape[:-1], 2 * packed.shape[-1]).to(torch.int8)


def quant_int4_per_token(X):
    """X [..., N, D] -> (packed uint8 [..., N, D/2], fp16 scales [..., N])."""
    s = _scales(X, 7)
    q = torch.clamp(torch.round(X / s), -7, 7).to(torch.int8)
    return pack_int4(q), s.squeeze(-1).half().contiguous()


def dequant_int8(q, s):
    """(float)q * (float)scale -> fp32 [..., N, D]."""
    return q.float() * s.float()[..., None]


def dequant_int4(packed, s):
    """Unpack (low nibble first), then (float)q * (float)scale -> fp32 [..., N, D]."""
    return unpack_int4(packed).float() * s.float()[..., None]


def quant_fp8_per_token(X):
    """X [..., N, D] (fp16, bf16 or fp32) -> (float8_e4m3fn [..., N, D], fp16 scales [..., N]).

    The fp8 KV format (no counterpart in the reference): in fp32 on the widened
    input, s = max(max|x| * fp32(1/448), 1e-8) and code = e4m3(clamp(x / s, +-448))
    rounded to nearest even, an exact zero stored as +0; the scale is stored as fp16(s).
    """
    X32 = X.float()
    a = X32.abs().amax(-1, keepdim=True)
    s = (a * _recip32(448.0)).clamp(min=1e-8)
    q = (X32 / s).clamp(-448.0, 448.0)
    q = torch.where(q == 0, torch.zeros_like(q), q)
    return q.to(torch.float8_e4m3fn).contiguous(), s.squeeze(-1).half().contiguous()


def _recip32(x):
    """fp32(1/x) as a 0-dim fp32 tensor (the multiplier the kernels use)."""
    return torch.tensor(1.0, dtype=torch.float32) / torch.tensor(x, dtype=torch.float32)


def dequant_fp8(q, s):
    """float(code) * float(scale) -> fp32 [..., N, D]."""
    return q.float() * s.float()[..., None]
