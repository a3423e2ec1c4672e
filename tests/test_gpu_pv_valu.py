"""The P.V-on-vector-ALU variant (fqkv_set_pv_valu) against the float64 oracle
(needs an MI355X). It exists to time the matrix-core P.V product against a
vector-ALU one in the same kernel, so it has to compute the same attention:
GQA split-K at 32 query / 8 KV heads (4 heads per work item, the headline's
kernel) and fp16 MHA (1 head per work item), both merge modes, D = 128,
with one pass per wave and with many (where the running maximum moves and
the accumulators are rescaled)."""

import numpy as np
import pytest
import torch

import oracle
import fqkv_decode as fq

pytestmark = pytest.mark.gpu

TOL = 2e-3
DEV = "cuda"


@pytest.fixture
def pv_valu():
    fq._ext._set_pv_valu(True)
    yield
    fq._ext._set_pv_valu(False)


@pytest.mark.parametrize("N,S,W", [(16384, 32, 8), (16384, 2, 8), (4096, 1, 4), (1000, 7, 4), (37, 1, 2)])
def test_pv_valu_gqa_split_k(pv_valu, N, S, W, merge_mode):
    Hq, Hkv, D = 32, 8, 128
    g = torch.Generator().manual_seed(N + S)
    q = torch.randn(Hq, D, generator=g).half()
    K = torch.randn(Hkv, N, D, generator=g).half()
    V = torch.randn(Hkv, N, D, generator=g).half()
    ref = oracle.gqa_attention(q.numpy()[None], K.numpy()[None], V.numpy()[None])[0]
    mp = torch.empty(Hq, S, device=DEV)
    lp = torch.empty(Hq, S, device=DEV)
    op = torch.empty(Hq, S, D, device=DEV)
    o = torch.empty(Hq, D, dtype=torch.float16, device=DEV)
    fq.gqa_sk_fast(q.to(DEV), K.to(DEV), V.to(DEV), mp, lp, op, o, S, W, 8)
    err = float(np.abs(o.float().cpu().numpy().astype(np.float64) - ref).max())
    assert err <= TOL, err


@pytest.mark.parametrize("B,N", [(8, 4096), (256, 512), (256, 4096), (3, 100)])
def test_pv_valu_fp16_mha(pv_valu, B, N):
    D = 128
    g = torch.Generator().manual_seed(B * N)
    q = torch.randn(B, D, generator=g).half()
    K = torch.randn(B, N, D, generator=g).half()
    V = torch.randn(B, N, D, generator=g).half()
    ref = oracle.attention(q.numpy(), K.numpy(), V.numpy())
    o = fq.decode_attn_fp16_mw(q.to(DEV), K.to(DEV), V.to(DEV), 8)
    err = float(np.abs(o.float().cpu().numpy().astype(np.float64) - ref).max())
    assert err <= TOL, err
