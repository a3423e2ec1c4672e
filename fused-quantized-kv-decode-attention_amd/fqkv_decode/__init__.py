"""MI355X (gfx950) fused single-query decode attention.

Drop-in for the reference's five PyTorch-extension entry points
(emirabayer/Fused-Quantized-KV-Decode-Attention, kernels/*.cu):

    decode_attn_fp16_mw(q[B,D], K[B,N,D], V, W) -> o[B,D]             (decode_attn_fp16_mw.cu:50)
    decode_attn_int8_mw(q, K int8, V int8, Ks[B,N], Vs, W) -> o[B,D]  (decode_attn_int8_mw.cu:52)
    decode_attn_int4(q, K uint8 [B,N,D/2], V, Ks, Vs, W) -> o[B,D]    (decode_attn_int4.cu:47)
    decode_attn_gqa(q[B,Hq,D], K[B,Hkv,N,D], V, W) -> o[B,Hq,D]       (decode_attn_gqa.cu:56)
    gqa_sk_fast(q[Hq,D], K[Hkv,N,D], V, m_part, l_part, o_part, o, S, W, CW) -> None
                                                                      (decode_attn_gqa_sk_fast.cu:95)

Beyond the reference (same conventions, no counterpart there):

    decode_attn_gqa_int8 / decode_attn_gqa_int4(q[B,Hq,D], K[B,Hkv,N,D or D/2], V,
        Ks[B,Hkv,N], Vs, W) -> o[B,Hq,D]           GQA head mapping over an int8 / int4 cache
    gqa_sk_fast_int8 / gqa_sk_fast_int4(q[Hq,D], K[Hkv,N,D or D/2], V, Ks[Hkv,N], Vs,
        m_part, l_part, o_part, o, S, W, CW)        split-K over an int8 / int4 cache
    quantize_int8_per_token / quantize_int4_per_token(X[..., D]) -> (bytes, fp16 scales)
                                                    the KV quantizers as GPU kernels
    decode_attn_gqa_fp8 / gqa_sk_fast_fp8 / quantize_fp8_per_token
                                                    the same over OCP fp8 e4m3 codes
                                                    (float8_e4m3fn) with fp16 per-token scales
    gqa_sk_fast_bf16(q, K[Hkv,N,D] bf16, V, m_part, l_part, o_part, o, S, W, CW)
                                                    split-K over a bf16 cache (the layout entry
                                                    points below take bf16 K and V as well)
    quantize_kv_append_(K_new[B,H,n,D], V_new, K_cache[B,H,cap,D or D/2], V_cache,
        Ks_cache[B,H,cap], Vs_cache, pos) -> None  the quantizers in append form for a live
                                                    cache: one launch, in place at pos
    quantize_kv_append_at_(K_new, V_new, K_cache, V_cache, Ks_cache, Vs_cache, pos[B] int32)
                                                    the same with each sequence's position read
                                                    on the device (graph-capturable)
    quantize_kv_to_pages_(K_new[T,Hkv,D], V_new, slot_mapping[T] int32, K_pages[P,page,Hkv,·],
        V_pages, Ks_pages[P,page,Hkv], Vs_pages) -> None
                                                    the quantizers writing into paged int8 / int4
                                                    caches at slot = page * page_size + offset
    decode_attn_gqa_nhd(q[B,Hq,D], K[B,N,Hkv,D], V, W, Ks=None, Vs=None) -> o[B,Hq,D]
                                                    token-major (FlashInfer NHD) KV layout
    decode_attn_gqa_strided(q[B,Hq,D], K[B,Hkv,N,D] view, V, W, Ks=None, Vs=None) -> o[B,Hq,D]
                                                    any strided KV view with contiguous rows
                                                    (e.g. the filled part of a preallocated cache)
    decode_attn_gqa_paged(q, K_pages[P,page,Hkv,D], V_pages, page_table[B,max_pages], seq_lens[B],
        max_seq_len, W, Ks_pages=None, Vs_pages=None) -> o[B,Hq,D]      paged KV cache

Callers of the reference build each kernel with
``torch.utils.cpp_extension.load(name=..., sources=["kernels/<file>.cu"], ...)``
and call ``m.<function>(...)``; :func:`load` returns the module that serves
all five, so ``m = load(name="t_fp16", sources=[...])`` keeps working.

The functions run hand-written HIP kernels from ``libfqkv_decode.so``; there
is no CPU or PyTorch fallback: using any entry point raises ImportError if
the native libraries are not built (``python -m fqkv_decode._build``).
"""

import importlib.util
import os

import torch  # noqa: F401  (binds the HIP runtime PyTorch ships before ours loads)

from ._paths import EXT_NAME, LIB_NAME, PKG_DIR, ext_filename

__all__ = [
    "decode_attn_fp16_mw",
    "decode_attn_int8_mw",
    "decode_attn_int4",
    "decode_attn_gqa",
    "gqa_sk_fast",
    "decode_attn_gqa_int8",
    "decode_attn_gqa_int4",
    "gqa_sk_fast_int8",
    "gqa_sk_fast_int4",
    "quantize_int8_per_token",
    "quantize_int4_per_token",
    "decode_attn_gqa_fp8",
    "gqa_sk_fast_bf16",
    "gqa_sk_fast_fp8",
    "quantize_fp8_per_token",
    "quantize_kv_append_",
    "quantize_kv_append_at_",
    "quantize_kv_to_pages_",
    "decode_attn_gqa_nhd",
    "decode_attn_gqa_strided",
    "decode_attn_gqa_paged",
    "load",
    "lib_path",
    "ext_path",
]

_ENTRY_POINTS = ("decode_attn_fp16_mw", "decode_attn_int8_mw", "decode_attn_int4", "decode_attn_gqa",
                 "gqa_sk_fast", "decode_attn_gqa_int8", "decode_attn_gqa_int4", "gqa_sk_fast_int8",
                 "gqa_sk_fast_int4", "quantize_int8_per_token", "quantize_int4_per_token", "decode_attn_gqa_fp8",
                 "gqa_sk_fast_fp8", "quantize_fp8_per_token", "gqa_sk_fast_bf16", "quantize_kv_append_",
                 "quantize_kv_append_at_", "quantize_kv_to_pages_", "decode_attn_gqa_nhd", "decode_attn_gqa_strided", "decode_attn_gqa_paged")
_EXT = None


def lib_path():
    """Path of the C-ABI library libfqkv_decode.so."""
    return os.path.join(PKG_DIR, LIB_NAME)


def ext_path():
    """Path of the PyTorch binding extension module."""
    return os.path.join(PKG_DIR, ext_filename())


def _load_ext():
    """Import the PyTorch binding (once); ImportError if the native libraries are not built."""
    global _EXT
    if _EXT is not None:
        return _EXT
    path = ext_path()
    if not os.path.exists(path) or not os.path.exists(lib_path()):
        raise ImportError(
            "fqkv_decode: native libraries not built (%s); run `python -m fqkv_decode._build` "
            "from %s" % (path, os.path.dirname(PKG_DIR)))
    spec = importlib.util.spec_from_file_location("fqkv_decode." + EXT_NAME, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    _EXT = mod
    return mod


def __getattr__(name):
    # The entry points resolve to the native module on first use, so the
    # package (and its build step) imports before the libraries exist.
    if name in _ENTRY_POINTS:
        return getattr(_load_ext(), name)
    if name == "_ext":
        return _load_ext()
    raise AttributeError("module 'fqkv_decode' has no attribute %r" % name)


def load(name=None, sources=None, extra_cuda_cflags=None, verbose=False, **kwargs):
    """Stand-in for ``torch.utils.cpp_extension.load`` as the reference's callers use it.

    The reference JIT-compiles one ``.cu`` per entry point
    (tests/test_kernels.py:8-11,55; flashinfer_looptimed.py:30-31). Here the
    kernels are prebuilt, so every call returns the one extension module,
    which exposes all five entry points; the arguments are accepted and
    ignored.
    """
    return _load_ext()


def choose_splits(rows, G, N, D, kv_format, W):
    """Split count the single-block entry points use (1 = none) on the current device.

    ``kv_format`` is 0 (fp16), 1 (int8) or 2 (int4).
    """
    return _load_ext()._choose_splits(rows, G, N, D, kv_format, W)


def cu_count():
    """Compute units of the current HIP device."""
    return _load_ext()._cu_count()
