"""transformers integration: single-token decode attention on the gfx950 kernels.

The reference plugs its GQA kernel into Hugging Face Llama through an
attention function registered in transformers' ``AttentionInterface``
(nb:1037-1064): query length 1 (decode) goes to ``decode_attn_gqa``, anything
else (prefill) to transformers' SDPA implementation. :func:`register` does the
same for this library and also registers the SDPA mask builder under the same
name, so that transformers hands the function no mask when none is needed.

Decode calls take the kernel path when the kernel computes exactly what SDPA
would: query length 1, no attention mask (no padding), no dropout, no
sliding window or soft-capping, head_dim 64 or 128, Hq a multiple of Hkv and
the softmax scale 1/sqrt(head_dim). Anything else falls back to SDPA. As in
the reference, non-fp16 tensors are converted to fp16 for the kernel and the
output is cast back to the query's dtype.

Usage::

    from fqkv_decode import hf_llama
    name = hf_llama.register()                 # "fqkv_decode"
    model.set_attn_implementation(name)        # or model.config._attn_implementation = name
"""

import math

import torch

DEFAULT_NAME = "fqkv_decode"
_W = 8  # waves per workgroup for the decode kernel


def _sdpa(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    from transformers.integrations.sdpa_attention import sdpa_attention_forward

    return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout, scaling=scaling,
                                  **kwargs)


def kernel_applies(query, key, attention_mask, scaling, dropout, **kwargs):
    """True when the decode kernel computes exactly what SDPA would for this call."""
    if query.dim() != 4 or key.dim() != 4 or query.shape[2] != 1:
        return False
    if attention_mask is not None or dropout:
        return False
    if kwargs.get("sliding_window") is not None or kwargs.get("softcap") is not None:
        return False
    B, Hq, _, D = query.shape
    Hkv = key.shape[1]
    if D not in (64, 128) or Hkv < 1 or Hq % Hkv or key.shape[0] != B or key.shape[2] < 1:
        return False
    if scaling is not None and abs(scaling * math.sqrt(D) - 1.0) > 1e-6:
        return False
    return query.is_cuda


def attention_forward(module, query, key, value, attention_mask=None, scaling=None, dropout=0.0, **kwargs):
    """transformers attention function: query [B, Hq, q, D], key/value [B, Hkv, kv, D] -> ([B, q, Hq, D], None)."""
    if getattr(module, "training", False) or not kernel_applies(query, key, attention_mask, scaling, dropout,
                                                               **kwargs):
        return _sdpa(module, query, key, value, attention_mask, scaling=scaling, dropout=dropout, **kwargs)
    from . import decode_attn_gqa

    q = query[:, :, 0, :].to(torch.float16).contiguous()  # [B, Hq, D]
    K = key.to(torch.float16).contiguous()                 # [B, Hkv, N, D]
    V = value.to(torch.float16).contiguous()
    out = decode_attn_gqa(q, K, V, _W)                     # [B, Hq, D]
    return out.unsqueeze(1).to(query.dtype), None          # [B, 1, Hq, D]


def register(name=DEFAULT_NAME):
    """Register the attention function (and the SDPA mask builder) under ``name``; returns ``name``."""
    from transformers import AttentionInterface, AttentionMaskInterface
    from transformers.masking_utils import sdpa_mask

    AttentionInterface.register(name, attention_forward)
    AttentionMaskInterface.register(name, sdpa_mask)
    return name
