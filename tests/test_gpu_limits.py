"""The longest KV rows the entry points accept (needs an MI355X).

Byte offsets inside one KV row (one KV head of one sequence) are 32-bit, and a
pass addresses tiles up to 8 x 128 + 16 tokens past the end of the row, so a row
holds up to 2^32 / row bytes - 1040 tokens: fp16 at D 128 2^24 - 1040, int4 at
D 128 2^26 - 1040. At those lengths the kernels must still read the far end of the
row: needle keys in the last tokens (and at the start and in the middle) carry
most of each head's softmax mass, so the output depends on reads at offsets
just under 4 GiB. The reference is float32 products per chunk of 2^20 tokens
and a float64 online softmax across chunks, on the GPU; max-abs 2e-3. The
argument checks that reject longer rows are CPU tests (test_boundary.py).
"""

import pytest
import torch

import fqkv_decode as fq
from fqkv_decode import quant

pytestmark = pytest.mark.gpu

TOL = 2e-3
DEV = "cuda"
CHUNK = 1 << 20


def chunked_reference(q, rowK, rowV, N, D):
    """softmax(q K^T / sqrt(D)) V for q [H, D] over tokens [0, N) of one KV row, where rowK(a, b) /
    rowV(a, b) return float32 [b - a, D] on the GPU: float64 online softmax across chunks."""
    qf = q.float()
    scale = 1.0 / (D ** 0.5)
    m = torch.full((q.shape[0], 1), -float("inf"), dtype=torch.float64, device=DEV)
    l = torch.zeros_like(m)
    acc = torch.zeros(q.shape[0], D, dtype=torch.float64, device=DEV)
    for a in range(0, N, CHUNK):
        b = min(N, a + CHUNK)
        s = torch.mm(qf, rowK(a, b).t().contiguous()).double() * scale  # [H, n]
        mn = torch.maximum(m, s.max(dim=1, keepdim=True).values)
        w = torch.exp(s - mn)
        c = torch.exp(m - mn)
        l = l * c + w.sum(dim=1, keepdim=True)
        acc = acc * c + torch.mm(w.float(), rowV(a, b)).double()
        m = mn
    return (acc / l).float()


def needles(N):
    return [N - 1, N - 2, N - 17, N - 1000, N // 2, 0]


def test_fp16_split_k_at_the_longest_row():
    """gqa_sk_fast, Hq 4 / Hkv 1, D 128, N = 2^24 - 1040 (4 GiB - 260 KiB per K and V row), S 64."""
    N, D, Hq, S = (1 << 24) - 1040, 128, 4, 64
    g = torch.Generator(device=DEV).manual_seed(70)
    q = torch.randn(Hq, D, device=DEV, generator=g).half()
    K = torch.empty(1, N, D, dtype=torch.float16, device=DEV).normal_(generator=g)
    V = torch.empty(1, N, D, dtype=torch.float16, device=DEV).normal_(generator=g)
    # needle j: head j % Hq scores ~22 there (q_h scaled to a dot of 22 sqrt(D)); its V is a ramp
    for j, t in enumerate(needles(N)):
        h = j % Hq
        qh = q[h].float()
        K[0, t] = (qh * (22.0 * D ** 0.5 / float(qh.dot(qh)))).half()
        V[0, t] = torch.linspace(-1.0, 1.0, D, device=DEV).half() * (1 + j) / 3
    mp = torch.empty(Hq, S, device=DEV)
    lp = torch.empty(Hq, S, device=DEV)
    op = torch.empty(Hq, S, D, device=DEV)
    o = torch.empty(Hq, D, dtype=torch.float16, device=DEV)
    fq.gqa_sk_fast(q, K, V, mp, lp, op, o, S, 8, 8)
    ref = chunked_reference(q, lambda a, b: K[0, a:b].float(), lambda a, b: V[0, a:b].float(), N, D)
    assert float((o.float() - ref).abs().max()) <= TOL
    del K, V
    torch.cuda.empty_cache()


def test_int4_mha_at_the_longest_row():
    """decode_attn_int4, B 1, D 128, N = 2^26 - 1040 (4 GiB - 65 KiB of packed K and of V): the
    int4 loads take their tile offsets in the SGPR offset, up to just under 4 GiB."""
    N, D = (1 << 26) - 1040, 128
    g = torch.Generator(device=DEV).manual_seed(71)
    q = torch.randn(1, D, device=DEV, generator=g).half()
    Kp = torch.randint(0, 256, (1, N, D // 2), dtype=torch.uint8, device=DEV, generator=g)
    Vp = torch.randint(0, 256, (1, N, D // 2), dtype=torch.uint8, device=DEV, generator=g)
    Ks = (torch.rand(1, N, device=DEV, generator=g) * 0.01 + 0.01).half()
    Vs = (torch.rand(1, N, device=DEV, generator=g) * 0.01 + 0.01).half()
    # needle keys: nibbles 7 sign(q), scaled for a score of ~20; needle values: nibble ramps
    qs = torch.where(q[0] >= 0, 7, -7).to(torch.int32)
    lo_hi = lambda v: ((v[0::2] & 0xF) | ((v[1::2] & 0xF) << 4)).to(torch.uint8)
    score_unit = float((q[0].float() * qs.float()).sum()) / D ** 0.5
    ramp = (torch.arange(D, device=DEV) % 15 - 7).to(torch.int32)
    for j, t in enumerate(needles(N)):
        Kp[0, t] = lo_hi(qs)
        Ks[0, t] = 20.0 / score_unit
        Vp[0, t] = lo_hi(ramp if j % 2 == 0 else -ramp)
        Vs[0, t] = 0.1 * (1 + j)
    out = fq.decode_attn_int4(q, Kp, Vp, Ks, Vs, 8)
    ref = chunked_reference(q, lambda a, b: quant.dequant_int4(Kp[0, a:b], Ks[0, a:b]).float(),
                            lambda a, b: quant.dequant_int4(Vp[0, a:b], Vs[0, a:b]).float(), N, D)
    assert float((out.float() - ref).abs().max()) <= TOL
    del Kp, Vp, Ks, Vs
    torch.cuda.empty_cache()
