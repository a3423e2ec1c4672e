"""The package's PyTorch quantizers (the KV format producers) against the oracle, bit for bit."""

import numpy as np
import pytest
import torch

import oracle
from fqkv_decode import quant


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_int8_quantizer_bytes(dtype):
    g = torch.Generator().manual_seed(0)
    X = torch.randn(3, 200, 128, generator=g).to(dtype)
    q, s = quant.quant_int8_per_token(X)
    oq, os_ = oracle.quant_int8_per_token(X.numpy())
    assert q.dtype == torch.int8 and s.dtype == torch.float16 and s.shape == (3, 200)
    np.testing.assert_array_equal(q.numpy(), oq)
    np.testing.assert_array_equal(s.numpy().view(np.uint16), os_.view(np.uint16))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
def test_int4_quantizer_bytes(dtype, D):
    g = torch.Generator().manual_seed(1)
    X = torch.randn(2, 300, D, generator=g).to(dtype)
    P, s = quant.quant_int4_per_token(X)
    oP, os_ = oracle.quant_int4_per_token(X.numpy())
    assert P.dtype == torch.uint8 and P.shape == (2, 300, D // 2)
    np.testing.assert_array_equal(P.numpy(), oP)
    np.testing.assert_array_equal(s.numpy().view(np.uint16), os_.view(np.uint16))


def test_dequant_matches_oracle_exactly():
    g = torch.Generator().manual_seed(2)
    X = torch.randn(2, 64, 128, generator=g)
    q8, s8 = quant.quant_int8_per_token(X)
    np.testing.assert_array_equal(quant.dequant_int8(q8, s8).numpy(), oracle.dequant_int8(q8.numpy(), s8.numpy()))
    P, s4 = quant.quant_int4_per_token(X)
    np.testing.assert_array_equal(quant.dequant_int4(P, s4).numpy(), oracle.dequant_int4(P.numpy(), s4.numpy()))


def test_unpack_edge_bytes():
    P = torch.tensor([[0x80, 0x7F, 0x88, 0x08, 0xF7]], dtype=torch.uint8)
    np.testing.assert_array_equal(quant.unpack_int4(P).numpy(), oracle.unpack_int4(P.numpy()))
    np.testing.assert_array_equal(quant.pack_int4(quant.unpack_int4(P)).numpy(), P.numpy())
