"""The drop-in boundary without a GPU: the C-ABI library loads, exports every
symbol include/fqkv_decode.h declares, and rejects bad arguments before any
HIP call; the PyTorch binding exposes the reference's five names and refuses
CPU tensors with the reference's "cuda" error."""

import ctypes
import os
import re

import pytest
import torch

import fqkv_decode

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fqkv_decode.h")

I64 = ctypes.c_int64
VP = ctypes.c_void_p


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fqkv_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    L = ctypes.CDLL(fqkv_decode.lib_path())
    L.fqkv_last_error.restype = ctypes.c_char_p
    L.fqkv_version.restype = ctypes.c_char_p
    return L


def test_header_declares_the_five_entry_points():
    syms = declared_symbols()
    for name in ("fqkv_decode_attn_fp16_mw", "fqkv_decode_attn_int8_mw", "fqkv_decode_attn_int4",
                 "fqkv_decode_attn_gqa", "fqkv_gqa_sk_fast"):
        assert name in syms


def test_library_exports_every_declared_symbol(lib):
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_library_has_no_torch_dependency():
    import subprocess

    out = subprocess.run(["readelf", "-d", fqkv_decode.lib_path()], capture_output=True, text=True).stdout
    needed = re.findall(r"NEEDED.*\[(.*)\]", out)
    assert not any("torch" in n or "c10" in n for n in needed), needed
    assert any(n.startswith("libamdhip64") for n in needed)


def test_version(lib):
    assert b"gfx950" in lib.fqkv_version()


def test_merge_diagnostics_before_any_call(lib):
    """No split call has run in this process: no protocol, no fallback, no
    XCD period; a device index out of range reads as unusable."""
    lib.fqkv_merge_fallback_count.restype = ctypes.c_int64
    assert lib.fqkv_last_merge_protocol() == 0
    assert lib.fqkv_merge_fallback_count() == 0
    assert lib.fqkv_xcd_period(0) == 0
    assert lib.fqkv_xcd_period(-1) == -1 and lib.fqkv_xcd_period(64) == -1


def _err(lib):
    return lib.fqkv_last_error().decode()


@pytest.mark.parametrize("B,N,D,W,key", [
    (1, 16, 96, 8, "D:"), (1, 16, 64, 3, "W:"), (1, 0, 64, 8, "N:"), (0, 16, 64, 8, "B:"),
])
def test_capi_fp16_rejects_bad_shapes(lib, B, N, D, W, key):
    f = lib.fqkv_decode_attn_fp16_mw
    f.argtypes = [VP, VP, VP, VP, I64, I64, I64, I64, VP, ctypes.c_size_t, VP]
    rc = f(16, 16, 16, 16, B, N, D, W, None, 0, None)
    assert rc == 1 and _err(lib).startswith(key), _err(lib)


def test_capi_rejects_null_and_misaligned_pointers(lib):
    f = lib.fqkv_decode_attn_fp16_mw
    f.argtypes = [VP, VP, VP, VP, I64, I64, I64, I64, VP, ctypes.c_size_t, VP]
    assert f(None, 16, 16, 16, 1, 16, 64, 8, None, 0, None) == 1 and "null" in _err(lib)
    assert f(16, 24, 16, 16, 1, 16, 64, 8, None, 0, None) == 1 and "aligned" in _err(lib)


def test_capi_sk_fast_rejects_bad_knobs(lib):
    f = lib.fqkv_gqa_sk_fast
    f.argtypes = [VP, VP, VP, VP, VP, VP, VP, I64, I64, I64, I64, I64, I64, I64, VP]
    args = [16] * 7
    assert f(*args, 32, 8, 1024, 128, 16, 8, 5, None) == 1 and _err(lib).startswith("CW:")
    assert f(*args, 32, 8, 1024, 128, 0, 8, 4, None) == 1 and _err(lib).startswith("S:")
    assert f(*args, 30, 8, 1024, 128, 16, 8, 4, None) == 1 and _err(lib).startswith("heads:")
    assert f(*args, 32, 8, 1024, 128, 16, 6, 4, None) == 1 and _err(lib).startswith("W:")
    assert f(*args, 32, 8, 1024, 100, 16, 8, 4, None) == 1 and _err(lib).startswith("D:")


def test_capi_quant_and_gqa_reject_bad_args(lib):
    f8 = lib.fqkv_decode_attn_int8_mw
    f8.argtypes = [VP, VP, VP, VP, VP, VP, I64, I64, I64, I64, VP, ctypes.c_size_t, VP]
    assert f8(16, 16, 16, None, 16, 16, 2, 64, 128, 8, None, 0, None) == 1 and "null" in _err(lib)
    f4 = lib.fqkv_decode_attn_int4
    f4.argtypes = f8.argtypes
    assert f4(16, 16, 16, 16, 16, 16, 2, 64, 32, 8, None, 0, None) == 1 and _err(lib).startswith("D:")
    fg = lib.fqkv_decode_attn_gqa
    fg.argtypes = [VP, VP, VP, VP, I64, I64, I64, I64, I64, I64, VP, ctypes.c_size_t, VP]
    assert fg(16, 16, 16, 16, 1, 32, 6, 64, 64, 8, None, 0, None) == 1 and _err(lib).startswith("heads:")
    fd = lib.fqkv_dequant_kv
    fd.argtypes = [VP, VP, VP, I64, I64, ctypes.c_int, ctypes.c_int, VP]
    assert fd(16, 16, 16, 4, 128, 0, 0, None) == 1 and "kv_format" in _err(lib)


def test_binding_exposes_reference_names():
    m = fqkv_decode.load(name="t_fp16", sources=["kernels/decode_attn_fp16_mw.cu"], extra_cuda_cflags=["-O3"])
    for name in ("decode_attn_fp16_mw", "decode_attn_int8_mw", "decode_attn_int4", "decode_attn_gqa", "gqa_sk_fast"):
        assert callable(getattr(m, name))
        assert getattr(fqkv_decode, name) is getattr(m, name)


def test_binding_rejects_cpu_tensors():
    q = torch.zeros(1, 64, dtype=torch.float16)
    K = torch.zeros(1, 8, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="^cuda"):
        fqkv_decode.decode_attn_fp16_mw(q, K, K, 8)
    with pytest.raises(RuntimeError, match="^cuda"):
        fqkv_decode.decode_attn_gqa(q.view(1, 1, 64), K.view(1, 1, 8, 64), K.view(1, 1, 8, 64), 8)
    Kq = torch.zeros(1, 8, 64, dtype=torch.int8)
    s = torch.zeros(1, 8, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="^cuda"):
        fqkv_decode.decode_attn_int8_mw(q, Kq, Kq, s, s, 8)
    with pytest.raises(RuntimeError, match="^cuda"):
        fqkv_decode.decode_attn_int4(q, Kq.view(torch.uint8)[..., :32].contiguous(), Kq.view(torch.uint8)[..., :32].contiguous(), s, s, 8)
    mp = torch.zeros(1, 4)
    with pytest.raises(RuntimeError, match="^cuda"):
        fqkv_decode.gqa_sk_fast(q, K, K, mp, mp, torch.zeros(1, 4, 64), q.clone(), 4, 8, 4)


def test_capi_quantizer_rejects_bad_args(lib):
    f = lib.fqkv_quantize_kv
    f.argtypes = [VP, ctypes.c_int, VP, VP, I64, I64, ctypes.c_int, VP]
    assert f(16, 0, 16, 16, 4, 128, 0, None) == 1 and "kv_format" in _err(lib)
    assert f(16, 3, 16, 16, 4, 128, 1, None) == 1 and "x_dtype" in _err(lib)  # 2 is bf16
    assert f(16, 1, 16, 16, 4, 96, 1, None) == 1 and _err(lib).startswith("D:")
    assert f(16, 1, 16, 16, 0, 128, 1, None) == 1 and _err(lib).startswith("tokens")
    assert f(None, 1, 16, 16, 4, 128, 1, None) == 1 and "null" in _err(lib)
    assert f(24, 1, 16, 16, 4, 128, 1, None) == 1 and "aligned" in _err(lib)
    assert f(16, 1, 20, 16, 4, 128, 1, None) == 1 and "aligned" in _err(lib)


def test_capi_quantize_append_rejects_bad_args(lib):
    f = lib.fqkv_quantize_kv_append
    f.argtypes = [VP, VP, ctypes.c_int] + [VP] * 4 + [I64] * 5 + [ctypes.c_int, VP]
    ok = [16, 16, 1, 16, 16, 16, 16]
    assert f(*ok, 8, 2, 100, 99, 128, 1, None) == 1 and _err(lib).startswith("pos:")
    assert f(*ok, 8, 1, 100, -1, 128, 1, None) == 1 and _err(lib).startswith("pos:")
    assert f(*ok, 8, 0, 100, 0, 128, 1, None) == 1 and "n_new" in _err(lib)
    assert f(*ok, 8, 1, 100, 0, 128, 0, None) == 1 and "kv_format" in _err(lib)
    assert f(*ok, 8, 1, 100, 0, 96, 1, None) == 1 and _err(lib).startswith("D:")
    assert f(16, None, 1, 16, 16, 16, 16, 8, 1, 100, 0, 128, 1, None) == 1 and "null" in _err(lib)
    assert f(16, 16, 1, 20, 16, 16, 16, 8, 1, 100, 0, 128, 1, None) == 1 and "aligned" in _err(lib)


def test_capi_quantize_paged_rejects_bad_args(lib):
    """The paged quantizer: slots are read on the GPU (out-of-range ones are skipped there); the
    host checks format, sizes, the page size, stride and pointer alignment."""
    f = lib.fqkv_quantize_kv_paged
    f.argtypes = [VP, VP, ctypes.c_int, VP, I64, I64, I64] + [VP] * 4 + [I64] * 8 + [ctypes.c_int, VP]
    x = [16, 16, 1, 16]               # K_new, V_new, x_dtype fp32, slot_mapping
    pages = [16, 16, 16, 16]          # K, V, Ks, Vs pages
    st = [4096, 256, 128, 32, 2, 1]   # page / token / head strides (bytes), scale strides (elements)
    assert f(*x, 0, 2, 128, *pages, 8, 16, *st, 1, None) == 0   # zero tokens: nothing to do
    assert f(*x, 10, 2, 128, *pages, 8, 12, *st, 1, None) == 1 and _err(lib).startswith("page:")
    assert f(*x, 10, 2, 128, *pages, 0, 16, *st, 1, None) == 1 and _err(lib).startswith("page:")
    assert f(*x, 10, 0, 128, *pages, 8, 16, *st, 1, None) == 1 and _err(lib).startswith("shape:")
    assert f(*x, -1, 2, 128, *pages, 8, 16, *st, 1, None) == 1 and _err(lib).startswith("shape:")
    assert f(*x, 10, 2, 128, *pages, 8, 16, 4096, 252, 128, 32, 2, 1, 1, None) == 1 and _err(lib).startswith("stride:")
    assert f(*x, 10, 2, 128, *pages, 8, 16, 4096, 256, 128, -32, 2, 1, 1, None) == 1 and _err(lib).startswith("stride:")
    assert f(*x, 10, 2, 96, *pages, 8, 16, *st, 1, None) == 1 and _err(lib).startswith("D:")
    assert f(*x, 10, 2, 128, *pages, 8, 16, *st, 0, None) == 1 and "kv_format" in _err(lib)
    assert f(16, 16, 1, None, 10, 2, 128, *pages, 8, 16, *st, 1, None) == 1 and "null" in _err(lib)
    assert f(16, 16, 1, 18, 10, 2, 128, *pages, 8, 16, *st, 1, None) == 1 and "slot_mapping" in _err(lib)
    assert f(*x, 10, 2, 128, 20, 16, 16, 16, 8, 16, *st, 1, None) == 1 and "pages must be" in _err(lib)


def test_capi_quantize_append_at_rejects_bad_args(lib):
    """The device-position append: positions are read on the GPU, so the host checks the rest
    (n_new fits the capacity, rows_per_pos divides rows, pointers and their alignment)."""
    f = lib.fqkv_quantize_kv_append_at
    f.argtypes = [VP, VP, ctypes.c_int] + [VP] * 4 + [I64] * 3 + [VP, I64, I64, ctypes.c_int, VP]
    ok = [16, 16, 1, 16, 16, 16, 16]
    assert f(*ok, 8, 101, 100, 16, 4, 128, 1, None) == 1 and _err(lib).startswith("pos:")
    assert f(*ok, 8, 1, 100, 16, 3, 128, 1, None) == 1 and "rows_per_pos" in _err(lib)
    assert f(*ok, 8, 1, 100, 16, 0, 128, 1, None) == 1 and "rows_per_pos" in _err(lib)
    assert f(*ok, 8, 1, 100, None, 4, 128, 1, None) == 1 and "null" in _err(lib)
    assert f(*ok, 8, 1, 100, 18, 4, 128, 1, None) == 1 and "aligned" in _err(lib)
    assert f(*ok, 8, 0, 100, 16, 4, 128, 1, None) == 1 and "n_new" in _err(lib)
    assert f(*ok, 8, 1, 100, 16, 4, 128, 0, None) == 1 and "kv_format" in _err(lib)
    assert f(*ok, 8, 1, 100, 16, 4, 96, 2, None) == 1 and _err(lib).startswith("D:")
    assert f(16, 16, 3, 16, 16, 16, 16, 8, 1, 100, 16, 4, 128, 1, None) == 1 and "x_dtype" in _err(lib)


def test_capi_quantized_gqa_and_split_reject_bad_args(lib):
    fg = lib.fqkv_decode_attn_gqa_quant
    fg.argtypes = [VP] * 6 + [I64] * 5 + [ctypes.c_int, I64, VP, ctypes.c_size_t, VP]
    assert fg(16, 16, 16, 16, 16, 16, 1, 32, 8, 64, 128, 0, 8, None, 0, None) == 1 and "kv_format" in _err(lib)
    assert fg(16, 16, 16, 16, 16, 16, 1, 30, 8, 64, 128, 1, 8, None, 0, None) == 1 and _err(lib).startswith("heads:")
    assert fg(16, 16, 16, None, 16, 16, 1, 32, 8, 64, 128, 2, 8, None, 0, None) == 1 and "null" in _err(lib)
    fs = lib.fqkv_gqa_sk_fast_quant
    fs.argtypes = [VP] * 9 + [I64] * 4 + [ctypes.c_int, I64, I64, I64, VP]
    assert fs(*[16] * 9, 32, 8, 64, 128, 1, 16, 8, 3, None) == 1 and _err(lib).startswith("CW:")
    assert fs(*[16] * 9, 32, 8, 64, 128, 0, 16, 8, 4, None) == 1 and "kv_format" in _err(lib)
    # fp8 (kv_format 4) is accepted, so the next check speaks; 5 is unknown
    assert fs(*[16] * 9, 32, 8, 64, 128, 4, 0, 8, 4, None) == 1 and _err(lib).startswith("S:")
    assert fs(*[16] * 9, 32, 8, 64, 128, 5, 16, 8, 4, None) == 1 and "kv_format" in _err(lib)
    assert fs(*[16] * 9, 32, 8, 64, 128, 2, 0, 8, 4, None) == 1 and _err(lib).startswith("S:")


def test_binding_exposes_quantized_and_quantizer_entry_points():
    for name in ("decode_attn_gqa_int8", "decode_attn_gqa_int4", "gqa_sk_fast_int8", "gqa_sk_fast_int4",
                 "quantize_int8_per_token", "quantize_int4_per_token", "decode_attn_gqa_nhd",
                 "decode_attn_gqa_strided", "decode_attn_gqa_paged", "decode_attn_gqa_fp8", "gqa_sk_fast_fp8",
                 "quantize_fp8_per_token", "quantize_kv_append_", "quantize_kv_append_at_", "quantize_kv_to_pages_"):
        assert callable(getattr(fqkv_decode, name))
    with pytest.raises(RuntimeError, match="^cuda"):
        fqkv_decode.quantize_int8_per_token(torch.zeros(4, 128))
    K = torch.zeros(1, 2, 40, 64, dtype=torch.float16)[:, :, :30]
    with pytest.raises(RuntimeError, match="^cuda"):
        fqkv_decode.decode_attn_gqa_strided(torch.zeros(1, 4, 64, dtype=torch.float16), K, K, 8)
    Kb = torch.zeros(1, 2, 30, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="^cuda"):
        fqkv_decode.decode_attn_gqa_strided(torch.zeros(1, 4, 64, dtype=torch.float16), Kb, Kb, 8)


def test_capi_layout_entry_points_reject_bad_args(lib):
    fs = lib.fqkv_decode_attn_gqa_strided
    fs.argtypes = [VP] * 6 + [I64] * 5 + [ctypes.c_int] + [I64] * 7 + [VP, ctypes.c_size_t, VP]
    # token stride below the row size
    assert fs(*[16] * 6, 1, 32, 8, 64, 128, 0, 65536, 256, 128, 0, 0, 1, 8, None, 0, None) == 1
    assert _err(lib).startswith("strides:")
    # strides not multiples of 16
    assert fs(*[16] * 6, 1, 32, 8, 64, 128, 0, 65536, 264, 2048, 0, 0, 1, 8, None, 0, None) == 1
    assert _err(lib).startswith("strides:")
    fp = lib.fqkv_decode_attn_gqa_paged
    fp.argtypes = [VP] * 8 + [I64] * 8 + [ctypes.c_int] + [I64] * 7 + [VP, ctypes.c_size_t, VP]
    ok = [16] * 8
    assert fp(*ok, 1, 32, 8, 10, 4, 24, 64, 128, 0, 4096, 256, 2048, 0, 0, 1, 8, None, 0, None) == 1
    assert _err(lib).startswith("page_size:")
    assert fp(*ok[:5], None, 16, 16, 1, 32, 8, 10, 4, 16, 64, 128, 0, 4096, 256, 2048, 0, 0, 1, 8, None, 0, None) == 1
    assert "null page table" in _err(lib)
    assert fp(*ok, 1, 32, 8, 0, 4, 16, 64, 128, 0, 4096, 256, 2048, 0, 0, 1, 8, None, 0, None) == 1
    assert _err(lib).startswith("pages:")
    # bf16 (kv_format 3) is a layout format: accepted, so the next check speaks (token stride < 256 B)
    assert fs(*[16] * 6, 1, 32, 8, 64, 128, 3, 65536, 256, 128, 0, 0, 1, 8, None, 0, None) == 1
    assert _err(lib).startswith("strides:") and "256" in _err(lib)
    assert fs(*[16] * 6, 1, 32, 8, 64, 128, 5, 65536, 256, 256, 0, 0, 1, 8, None, 0, None) == 1
    assert "kv_format" in _err(lib)


def test_capi_probes_reject_bad_args(lib):
    fr = lib.fqkv_probe_buffer_range
    fr.argtypes = [VP, ctypes.c_size_t, ctypes.c_int, VP, VP]
    assert fr(4096, 256, 256, 4096, None) == 1  # no room past records
    assert _err(lib).startswith("bytes:")
    assert fr(4096, 4096, 100, 4096, None) == 1
    assert _err(lib).startswith("records:")
    assert fr(None, 4096, 256, 4096, None) == 1
    fs = lib.fqkv_probe_stream_read
    fs.argtypes = [VP, ctypes.c_size_t, VP, ctypes.c_int, VP]
    assert fs(4096, 100, None, 256, None) == 1
    assert _err(lib).startswith("bytes:")
    assert fs(4096, 4096, None, 0, None) == 1
    assert _err(lib).startswith("blocks:")


def test_capi_noalloc_rejects_before_any_hip_call(lib):
    f = lib.fqkv_gqa_sk_fast_noalloc
    f.argtypes = [VP] * 4 + [I64] * 7 + [VP]
    p = 4096  # aligned, never dereferenced: every check below fails before a HIP call
    assert f(p, p, p, p, 1 << 30, 8, 1024, 128, 4, 8, 8, None) == 1
    assert _err(lib).startswith("heads:")
    assert f(p, p, p, p, 256, 8, 1024, 128, 64, 8, 8, None) == 1  # 8.4 MB of partials > 8 MiB
    assert _err(lib).startswith("S:")
    assert f(p, p, p, p, 32, 8, 1024, 128, 0, 8, 8, None) == 1
    assert _err(lib).startswith("S:")
    assert f(p, p, p, p, 30, 8, 1024, 128, 4, 8, 8, None) == 1
    assert _err(lib).startswith("heads:")


def test_capi_rejects_rows_past_the_32_bit_span(lib):
    """Byte offsets inside a KV row are 32-bit, and a pass addresses tiles up to 8 x 128 + 16
    tokens past the end of the row: the row plus that margin must fit in 4 GiB. One token
    more than the longest accepted row (2^32 / row bytes - 1040 tokens) is rejected before
    any HIP call."""
    fs = lib.fqkv_gqa_sk_fast
    fs.argtypes = [VP] * 7 + [I64] * 7 + [VP]
    assert fs(*[16] * 7, 4, 1, (1 << 24) - 1039, 128, 16, 8, 8, None) == 1  # fp16 rows of 256 B
    assert _err(lib).startswith("N:") and "4 GiB" in _err(lib), _err(lib)
    f4 = lib.fqkv_decode_attn_int4
    f4.argtypes = [VP, VP, VP, VP, VP, VP, I64, I64, I64, I64, VP, ctypes.c_size_t, VP]
    assert f4(*[16] * 6, 1, (1 << 26) - 1039, 128, 8, None, 0, None) == 1  # int4 rows of 64 B
    assert _err(lib).startswith("N:") and "4 GiB" in _err(lib), _err(lib)
    f8 = lib.fqkv_decode_attn_int8_mw
    f8.argtypes = f4.argtypes
    assert f8(*[16] * 6, 1, (1 << 25) - 1039, 128, 8, None, 0, None) == 1  # int8 rows of 128 B
    assert _err(lib).startswith("N:") and "4 GiB" in _err(lib), _err(lib)
    fst = lib.fqkv_decode_attn_gqa_strided
    fst.argtypes = [VP] * 6 + [I64] * 5 + [ctypes.c_int] + [I64] * 7 + [VP, ctypes.c_size_t, VP]
    # token-major fp16, Hkv 8 x 256-byte rows: a 2 KiB token stride
    assert fst(16, 16, 16, None, None, 16, 1, 32, 8, (1 << 21) - 1039, 128, 0, 8 << 21, 256, 2048,
               0, 0, 1, 8, None, 0, None) == 1
    assert _err(lib).startswith("N:") and "4 GiB" in _err(lib), _err(lib)
