"""CPU oracle for the fused single-query decode-attention path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker (the CPU baseline times the reference's own PyTorch expression and
checks its result here). The product (the HIP library and its
PyTorch binding) never imports, links or calls anything here, and has no CPU
fallback: it fails loudly when its HIP extension is missing.

The oracle restates, in numpy, what the reference computes:

* ``attention``        -- decode_attn_fp16_mw.cu:19-47, decode_attn_gqa.cu:13-55
                          (softmax(q K^T * D^-1/2) V per head, fp32 scale)
* ``split_partials``   -- decode_attn_gqa_sk_fast.cu:11-14,45-52 (per-split m, l, acc)
* ``combine_partials`` -- decode_attn_gqa_sk_fast.cu:66-72,85-92 (log-sum-exp merge)
* ``quant_int8_per_token`` -- tests/test_kernels.py:32-34 and nb:236-238
* ``quant_int4_per_token`` / ``dequant_int4`` -- nb:292-307
* ``dequant_int8``     -- decode_attn_int8_mw.cu:22-31 (float(q) * float(scale))
* ``quant_fp8_per_token`` / ``dequant_fp8`` / ``e4m3_*`` -- no counterpart in the
  reference: this library's fp8 e4m3 KV format, stated here as its definition

Every function is pinned in ``tests/test_oracle.py`` by a check that a
plausible mistake would fail: the reference notebook's recorded CPU-RNG int4
figure (nb:283, rel 7.1036e-02), hand-built known-answer bytes, closed forms
(N=1, q=0, a dominant key), the PyTorch library routines
(``scaled_dot_product_attention``, half/float tensor arithmetic and the float8_e4m3fn
conversions), and
brute-force loops on tiny inputs. No function here is "parity unpinned".
"""

from .attention import (  # noqa: F401
    softmax_scale,
    attention,
    gqa_attention,
    split_bounds,
    split_partials,
    combine_partials,
    round_fp16,
)
from .quant import (  # noqa: F401
    quant_int8_per_token,
    quant_int4_per_token,
    dequant_int8,
    dequant_int4,
    pack_int4,
    unpack_int4,
    e4m3_encode,
    e4m3_decode,
    quant_fp8_per_token,
    dequant_fp8,
)
