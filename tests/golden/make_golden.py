"""Generate the committed golden fixtures for the decode-attention path.

Inputs are drawn from a CPU ``torch.Generator`` seeded with 0 (N(0,1), fp32,
then fp16 or quantized), so the same bits arise on any machine; expected
outputs come from the numpy oracle in ``oracle/`` (float64), which
``tests/test_oracle.py`` pins against the reference's recorded outputs,
closed forms and library routines. The int4 fixtures also embed hand-built
bytes 0x80, 0x7F, 0x88, 0x08, 0xF7 (nibble edge cases, including -8).

Usage (from the repository root): ``python tests/golden/make_golden.py``.
``tests/test_golden.py`` re-runs this generation in memory and compares it to
the committed files, so a drifting oracle fails loudly.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import oracle  # noqa: E402

EDGE_BYTES = np.array([0x80, 0x7F, 0x88, 0x08, 0xF7], dtype=np.uint8)


def randn(gen, *shape):
    return torch.randn(*shape, generator=gen, dtype=torch.float32).numpy()


def case_mha_f16(gen, B, N, D):
    q = randn(gen, B, D).astype(np.float16)
    K = randn(gen, B, N, D).astype(np.float16)
    V = randn(gen, B, N, D).astype(np.float16)
    o = oracle.attention(q, K, V)
    return dict(q=q, K=K, V=V, o=o.astype(np.float32))


def case_quant(gen, B, N, D, bits):
    q = randn(gen, B, D).astype(np.float16)
    Kf = randn(gen, B, N, D)
    Vf = randn(gen, B, N, D)
    if bits == 8:
        Kq, Ks = oracle.quant_int8_per_token(Kf)
        Vq, Vs = oracle.quant_int8_per_token(Vf)
        Kd, Vd = oracle.dequant_int8(Kq, Ks), oracle.dequant_int8(Vq, Vs)
    else:
        Kq, Ks = oracle.quant_int4_per_token(Kf)
        Vq, Vs = oracle.quant_int4_per_token(Vf)
        # plant the nibble edge bytes in token 0 of every row (K) and token 1 (V)
        Kq[:, 0, : len(EDGE_BYTES)] = EDGE_BYTES
        Vq[:, min(1, N - 1), : len(EDGE_BYTES)] = EDGE_BYTES
        Kd, Vd = oracle.dequant_int4(Kq, Ks), oracle.dequant_int4(Vq, Vs)
    o = oracle.attention(q, Kd, Vd)
    return dict(q=q, K=Kq, V=Vq, Ks=Ks, Vs=Vs, Kd=Kd, Vd=Vd, o=o.astype(np.float32))


def case_gqa(gen, B, Hq, Hkv, N, D):
    q = randn(gen, B, Hq, D).astype(np.float16)
    K = randn(gen, B, Hkv, N, D).astype(np.float16)
    V = randn(gen, B, Hkv, N, D).astype(np.float16)
    o = oracle.gqa_attention(q, K, V)
    return dict(q=q, K=K, V=V, o=o.astype(np.float32))


def case_splitk(gen, Hq, Hkv, N, D, S):
    q = randn(gen, Hq, D).astype(np.float16)
    K = randn(gen, Hkv, N, D).astype(np.float16)
    V = randn(gen, Hkv, N, D).astype(np.float16)
    m, l, acc = oracle.split_partials(q, K, V, S)
    o = oracle.combine_partials(m, l, acc)
    return dict(q=q, K=K, V=V, S=np.int64(S), m=m.astype(np.float32), l=l.astype(np.float32),
                acc=acc.astype(np.float32), o=o.astype(np.float32))


CASES = {
    "mha_f16_b3_n100_d64": lambda g: case_mha_f16(g, 3, 100, 64),
    "mha_f16_b2_n37_d128": lambda g: case_mha_f16(g, 2, 37, 128),
    "mha_f16_b4_n1_d128": lambda g: case_mha_f16(g, 4, 1, 128),
    "int8_b2_n64_d128": lambda g: case_quant(g, 2, 64, 128, 8),
    "int8_b3_n3_d64": lambda g: case_quant(g, 3, 3, 64, 8),
    "int4_b2_n64_d128": lambda g: case_quant(g, 2, 64, 128, 4),
    "int4_b4_n3_d64": lambda g: case_quant(g, 4, 3, 64, 4),
    "gqa_b2_hq8_hkv2_n50_d64": lambda g: case_gqa(g, 2, 8, 2, 50, 64),
    "gqa_b1_hq6_hkv2_n33_d128": lambda g: case_gqa(g, 1, 6, 2, 33, 128),
    "splitk_hq8_hkv2_n100_d128_s7": lambda g: case_splitk(g, 8, 2, 100, 128, 7),
    "splitk_hq8_hkv2_n3_d128_s8": lambda g: case_splitk(g, 8, 2, 3, 128, 8),
    "splitk_hq4_hkv1_n1_d64_s4": lambda g: case_splitk(g, 4, 1, 1, 64, 4),
}


def generate(name):
    gen = torch.Generator().manual_seed(0)
    return CASES[name](gen)


def path_of(name):
    return os.path.join(HERE, name + ".npz")


def main():
    for name in CASES:
        arrays = generate(name)
        np.savez_compressed(path_of(name), **arrays)
        print("wrote", path_of(name), os.path.getsize(path_of(name)), "bytes")


if __name__ == "__main__":
    main()
