"""GPU parity through the C ABI itself (ctypes on libfqkv_decode.so, no PyTorch
binding in between): every entry point of include/fqkv_decode.h, on device
buffers from PyTorch, against the float64 oracle at max-abs 2e-3; the
workspace contract of the single-block calls (enough, too small, none) and
the dequant helper bit-exact against the oracle's dequantisation."""

import ctypes

import numpy as np
import pytest
import torch

import oracle
import fqkv_decode
from fqkv_decode import quant

pytestmark = pytest.mark.gpu

TOL = 2e-3
I64 = ctypes.c_int64
VP = ctypes.c_void_p
SZ = ctypes.c_size_t
KV_F16, KV_I8, KV_I4 = 0, 1, 2


@pytest.fixture(scope="module")
def lib():
    L = ctypes.CDLL(fqkv_decode.lib_path())
    L.fqkv_last_error.restype = ctypes.c_char_p
    L.fqkv_workspace_bytes.restype = SZ
    L.fqkv_workspace_bytes.argtypes = [I64, I64, I64, I64, ctypes.c_int, I64]
    L.fqkv_decode_attn_fp16_mw.argtypes = [VP] * 4 + [I64] * 4 + [VP, SZ, VP]
    L.fqkv_decode_attn_int8_mw.argtypes = [VP] * 6 + [I64] * 4 + [VP, SZ, VP]
    L.fqkv_decode_attn_int4.argtypes = [VP] * 6 + [I64] * 4 + [VP, SZ, VP]
    L.fqkv_decode_attn_gqa.argtypes = [VP] * 4 + [I64] * 6 + [VP, SZ, VP]
    L.fqkv_gqa_sk_fast.argtypes = [VP] * 7 + [I64] * 7 + [VP]
    L.fqkv_dequant_kv.argtypes = [VP, VP, VP, I64, I64, ctypes.c_int, ctypes.c_int, VP]
    L.fqkv_quantize_kv.argtypes = [VP, ctypes.c_int, VP, VP, I64, I64, ctypes.c_int, VP]
    L.fqkv_decode_attn_gqa_quant.argtypes = [VP] * 6 + [I64] * 5 + [ctypes.c_int, I64, VP, SZ, VP]
    L.fqkv_gqa_sk_fast_quant.argtypes = [VP] * 9 + [I64] * 4 + [ctypes.c_int, I64, I64, I64, VP]
    return L


def stream():
    return torch.cuda.current_stream().cuda_stream


def check(lib, rc):
    assert rc == 0, lib.fqkv_last_error().decode()


def draw(g, *shape):
    return torch.randn(*shape, generator=g, dtype=torch.float32)


def maxerr(out, ref):
    return float(np.abs(out.float().cpu().numpy().astype(np.float64) - ref).max())


def workspace(lib, rows, G, N, D, fmt, W):
    n = lib.fqkv_workspace_bytes(rows, G, N, D, fmt, W)
    return torch.empty(max(n, 16), dtype=torch.uint8, device="cuda"), n


@pytest.mark.parametrize("B,N,D,W", [(1, 4096, 128, 8), (4, 100, 64, 4), (64, 512, 128, 2)])
def test_cabi_fp16_mha(lib, B, N, D, W):
    g = torch.Generator().manual_seed(20)
    q, K, V = draw(g, B, D).half(), draw(g, B, N, D).half(), draw(g, B, N, D).half()
    ref = oracle.attention(q.numpy(), K.numpy(), V.numpy())
    qd, Kd, Vd = q.cuda(), K.cuda(), V.cuda()
    ws, n = workspace(lib, B, 1, N, D, KV_F16, W)
    for wptr, wbytes in ((ws.data_ptr(), n), (ws.data_ptr(), n // 3), (None, 0)):
        o = torch.empty(B, D, dtype=torch.float16, device="cuda")
        check(lib, lib.fqkv_decode_attn_fp16_mw(qd.data_ptr(), Kd.data_ptr(), Vd.data_ptr(), o.data_ptr(),
                                                B, N, D, W, wptr, wbytes, stream()))
        torch.cuda.synchronize()
        assert maxerr(o, ref) <= TOL, (wbytes, maxerr(o, ref))


@pytest.mark.parametrize("fmt", ["int8", "int4"])
@pytest.mark.parametrize("B,N,D", [(2, 4096, 128), (16, 300, 64)])
def test_cabi_quantized_mha(lib, fmt, B, N, D):
    g = torch.Generator().manual_seed(21)
    q = draw(g, B, D).half()
    Kx, Vx = draw(g, B, N, D), draw(g, B, N, D)
    if fmt == "int8":
        Kq, Ks = quant.quant_int8_per_token(Kx)
        Vq, Vs = quant.quant_int8_per_token(Vx)
        Kf, Vf = quant.dequant_int8(Kq, Ks), quant.dequant_int8(Vq, Vs)
        f, kind = lib.fqkv_decode_attn_int8_mw, KV_I8
    else:
        Kq, Ks = quant.quant_int4_per_token(Kx)
        Vq, Vs = quant.quant_int4_per_token(Vx)
        Kf, Vf = quant.dequant_int4(Kq, Ks), quant.dequant_int4(Vq, Vs)
        f, kind = lib.fqkv_decode_attn_int4, KV_I4
    ref = oracle.attention(q.numpy(), Kf.numpy(), Vf.numpy())
    d = [t.cuda() for t in (q, Kq, Vq, Ks, Vs)]
    ws, n = workspace(lib, B, 1, N, D, kind, 8)
    o = torch.empty(B, D, dtype=torch.float16, device="cuda")
    check(lib, f(*[t.data_ptr() for t in d], o.data_ptr(), B, N, D, 8, ws.data_ptr(), n, stream()))
    torch.cuda.synchronize()
    assert maxerr(o, ref) <= TOL


@pytest.mark.parametrize("B,Hq,Hkv,N,D", [(1, 32, 8, 512, 64), (3, 16, 16, 1000, 128), (2, 24, 2, 77, 128)])
def test_cabi_gqa(lib, B, Hq, Hkv, N, D):
    g = torch.Generator().manual_seed(22)
    q, K, V = draw(g, B, Hq, D).half(), draw(g, B, Hkv, N, D).half(), draw(g, B, Hkv, N, D).half()
    ref = oracle.gqa_attention(q.numpy(), K.numpy(), V.numpy())
    qd, Kd, Vd = q.cuda(), K.cuda(), V.cuda()
    ws, n = workspace(lib, B * Hkv, Hq // Hkv, N, D, KV_F16, 4)
    o = torch.empty(B, Hq, D, dtype=torch.float16, device="cuda")
    check(lib, lib.fqkv_decode_attn_gqa(qd.data_ptr(), Kd.data_ptr(), Vd.data_ptr(), o.data_ptr(),
                                        B, Hq, Hkv, N, D, 4, ws.data_ptr(), n, stream()))
    torch.cuda.synchronize()
    assert maxerr(o, ref) <= TOL


@pytest.mark.parametrize("Hq,Hkv,N,D,S", [(32, 8, 16384, 128, 32), (8, 2, 100, 64, 7), (4, 4, 3, 128, 8)])
def test_cabi_gqa_sk_fast(lib, Hq, Hkv, N, D, S):
    g = torch.Generator().manual_seed(23)
    q, K, V = draw(g, Hq, D).half(), draw(g, Hkv, N, D).half(), draw(g, Hkv, N, D).half()
    ref = oracle.gqa_attention(q.numpy()[None], K.numpy()[None], V.numpy()[None])[0]
    m, l, acc = oracle.split_partials(q.numpy(), K.numpy(), V.numpy(), S)
    qd, Kd, Vd = q.cuda(), K.cuda(), V.cuda()
    mp = torch.empty(Hq, S, device="cuda")
    lp = torch.empty(Hq, S, device="cuda")
    op = torch.empty(Hq, S, D, device="cuda")
    o = torch.empty(Hq, D, dtype=torch.float16, device="cuda")
    check(lib, lib.fqkv_gqa_sk_fast(qd.data_ptr(), Kd.data_ptr(), Vd.data_ptr(), mp.data_ptr(), lp.data_ptr(),
                                    op.data_ptr(), o.data_ptr(), Hq, Hkv, N, D, S, 8, 8, stream()))
    torch.cuda.synchronize()
    assert maxerr(o, ref) <= TOL
    assert np.array_equal(np.isneginf(mp.cpu().numpy()), np.isneginf(m))
    np.testing.assert_allclose(lp.cpu().numpy(), l, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(op.cpu().numpy(), acc, rtol=1e-4, atol=2e-4)


@pytest.mark.parametrize("fmt", [KV_I8, KV_I4])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("path", [0, 1])
def test_cabi_dequant_bit_exact(lib, fmt, D, path):
    g = torch.Generator().manual_seed(24)
    T = 257
    X = draw(g, T, D)
    if fmt == KV_I8:
        Kq, Ks = quant.quant_int8_per_token(X)
        ref = oracle.dequant_int8(Kq.numpy(), Ks.numpy())
    else:
        Kq, Ks = quant.quant_int4_per_token(X)
        ref = oracle.dequant_int4(Kq.numpy(), Ks.numpy())
    out = torch.empty(T, D, device="cuda")
    Kd, Sd = Kq.cuda(), Ks.cuda()
    check(lib, lib.fqkv_dequant_kv(Kd.data_ptr(), Sd.data_ptr(), out.data_ptr(), T, D, fmt, path, stream()))
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), ref.astype(np.float32))


@pytest.mark.parametrize("fmt", [KV_I8, KV_I4])
@pytest.mark.parametrize("src", [0, 1])
def test_cabi_quantizer_bit_exact(lib, fmt, src):
    g = torch.Generator().manual_seed(25)
    T, D = 999, 128
    X = draw(g, T, D).to(torch.float16 if src == 0 else torch.float32)
    Xd = X.cuda()
    Q = torch.empty(T, D if fmt == KV_I8 else D // 2, dtype=torch.int8 if fmt == KV_I8 else torch.uint8,
                    device="cuda")
    S = torch.empty(T, dtype=torch.float16, device="cuda")
    check(lib, lib.fqkv_quantize_kv(Xd.data_ptr(), src, Q.data_ptr(), S.data_ptr(), T, D, fmt, stream()))
    torch.cuda.synchronize()
    oq, os_ = (oracle.quant_int8_per_token if fmt == KV_I8 else oracle.quant_int4_per_token)(X.numpy())
    assert np.array_equal(Q.cpu().numpy(), oq)
    assert np.array_equal(S.cpu().numpy().view(np.uint16), os_.view(np.uint16))


@pytest.mark.parametrize("fmt", [KV_I8, KV_I4])
def test_cabi_quantized_gqa_and_split(lib, fmt):
    g = torch.Generator().manual_seed(26)
    B, Hq, Hkv, N, D, S = 1, 32, 8, 3000, 128, 16
    q = draw(g, B, Hq, D).half()
    Kx, Vx = draw(g, B, Hkv, N, D), draw(g, B, Hkv, N, D)
    if fmt == KV_I8:
        (Kq, Ks), (Vq, Vs) = quant.quant_int8_per_token(Kx), quant.quant_int8_per_token(Vx)
        Kf, Vf = quant.dequant_int8(Kq, Ks), quant.dequant_int8(Vq, Vs)
    else:
        (Kq, Ks), (Vq, Vs) = quant.quant_int4_per_token(Kx), quant.quant_int4_per_token(Vx)
        Kf, Vf = quant.dequant_int4(Kq, Ks), quant.dequant_int4(Vq, Vs)
    ref = oracle.gqa_attention(q.numpy(), Kf.numpy(), Vf.numpy())
    d = [t.cuda() for t in (q, Kq, Vq, Ks, Vs)]
    ws, n = workspace(lib, B * Hkv, Hq // Hkv, N, D, fmt, 8)
    o = torch.empty(B, Hq, D, dtype=torch.float16, device="cuda")
    check(lib, lib.fqkv_decode_attn_gqa_quant(*[t.data_ptr() for t in d], o.data_ptr(), B, Hq, Hkv, N, D, fmt, 8,
                                              ws.data_ptr(), n, stream()))
    mp = torch.empty(Hq, S, device="cuda")
    lp = torch.empty(Hq, S, device="cuda")
    op = torch.empty(Hq, S, D, device="cuda")
    o2 = torch.empty(Hq, D, dtype=torch.float16, device="cuda")
    check(lib, lib.fqkv_gqa_sk_fast_quant(*[t.data_ptr() for t in d], mp.data_ptr(), lp.data_ptr(), op.data_ptr(),
                                          o2.data_ptr(), Hq, Hkv, N, D, fmt, S, 8, 8, stream()))
    torch.cuda.synchronize()
    assert maxerr(o, ref) <= TOL
    assert maxerr(o2, ref[0]) <= TOL


def test_plain_c_caller(tmp_path):
    """tests/c_abi_caller.c, a C program with no Python or PyTorch, built with gcc against
    include/fqkv_decode.h and libfqkv_decode.so, runs fqkv_gqa_sk_fast and
    fqkv_decode_attn_gqa on its own device buffers and checks them against a host reference."""
    import os
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not found")
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    pkg = os.path.dirname(fqkv_decode.lib_path())
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    exe = str(tmp_path / "c_abi_caller")
    build = subprocess.run([gcc, "-O2", "-std=c11", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(root, "include"),
                            "-I", os.path.join(rocm, "include"), os.path.join(here, "c_abi_caller.c"), "-o", exe,
                            "-L", pkg, "-lfqkv_decode", "-L", os.path.join(rocm, "lib"), "-lamdhip64",
                            "-Wl,-rpath," + pkg + ":" + os.path.join(rocm, "lib"), "-lm"],
                           capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    run = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.strip().splitlines()[-1].startswith("OK"), run.stdout
