"""fqkv_gqa_sk_fast_noalloc, the split-K entry point that allocates nothing
(its partials live in the library's static device scratch), through the C
ABI: two calls in a row, the second smaller, each equal bit for bit to
fqkv_gqa_sk_fast on the same inputs with caller-owned scratch, in both merge
modes; S beyond the scratch is rejected with a clear error before any HIP
call."""

import ctypes

import pytest
import torch

import fqkv_decode as fq

pytestmark = pytest.mark.gpu

I64 = ctypes.c_int64
VP = ctypes.c_void_p


@pytest.fixture(scope="module")
def lib():
    L = ctypes.CDLL(fq.lib_path())
    L.fqkv_last_error.restype = ctypes.c_char_p
    L.fqkv_gqa_sk_fast.argtypes = [VP] * 7 + [I64] * 7 + [VP]
    L.fqkv_gqa_sk_fast_noalloc.argtypes = [VP] * 4 + [I64] * 7 + [VP]
    L.fqkv_set_two_kernel_merge.argtypes = [ctypes.c_int]
    return L


def stream():
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("two_kernel", [0, 1])
def test_noalloc_equals_sk_fast_two_calls(lib, two_kernel):
    lib.fqkv_set_two_kernel_merge(two_kernel)
    try:
        g = torch.Generator().manual_seed(70)
        for Hq, Hkv, N, D, S, W, CW in ((32, 8, 16384, 128, 32, 8, 8), (8, 2, 1000, 64, 7, 4, 4)):
            q = torch.randn(Hq, D, generator=g).half().cuda()
            K = torch.randn(Hkv, N, D, generator=g).half().cuda()
            V = torch.randn(Hkv, N, D, generator=g).half().cuda()
            mp = torch.empty(Hq, S, device="cuda")
            lp = torch.empty(Hq, S, device="cuda")
            op = torch.empty(Hq, S, D, device="cuda")
            ref = torch.empty(Hq, D, dtype=torch.float16, device="cuda")
            rc = lib.fqkv_gqa_sk_fast(q.data_ptr(), K.data_ptr(), V.data_ptr(), mp.data_ptr(), lp.data_ptr(),
                                      op.data_ptr(), ref.data_ptr(), Hq, Hkv, N, D, S, W, CW, stream())
            assert rc == 0, lib.fqkv_last_error().decode()
            o = torch.full((Hq, D), float("nan"), dtype=torch.float16, device="cuda")
            rc = lib.fqkv_gqa_sk_fast_noalloc(q.data_ptr(), K.data_ptr(), V.data_ptr(), o.data_ptr(), Hq, Hkv, N, D,
                                              S, W, CW, stream())
            assert rc == 0, lib.fqkv_last_error().decode()
            torch.cuda.synchronize()
            assert torch.equal(o, ref), (Hq, N, D, S)
    finally:
        lib.fqkv_set_two_kernel_merge(0)


def test_noalloc_rejects_splits_beyond_the_scratch(lib):
    Hq, Hkv, N, D = 256, 64, 64, 128
    q = torch.zeros(Hq, D, dtype=torch.float16, device="cuda")
    K = torch.zeros(Hkv, N, D, dtype=torch.float16, device="cuda")
    o = torch.zeros(Hq, D, dtype=torch.float16, device="cuda")
    # 256 heads x 64 splits x 130 floats = 8.5 MB > 8 MiB
    rc = lib.fqkv_gqa_sk_fast_noalloc(q.data_ptr(), K.data_ptr(), K.data_ptr(), o.data_ptr(), Hq, Hkv, N, D, 64, 8, 8,
                                      stream())
    assert rc == 1
    assert lib.fqkv_last_error().decode().startswith("S:")
    # 63 splits fit (8.39e6 bytes)
    rc = lib.fqkv_gqa_sk_fast_noalloc(q.data_ptr(), K.data_ptr(), K.data_ptr(), o.data_ptr(), Hq, Hkv, N, D, 63, 8, 8,
                                      stream())
    assert rc == 0, lib.fqkv_last_error().decode()
    torch.cuda.synchronize()
