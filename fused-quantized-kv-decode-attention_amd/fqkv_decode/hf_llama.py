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
the reference, the query goes to the kernel in fp16 and the output is cast
back to the query's dtype; a bf16 model's KV cache is read in bf16 as it is
(``decode_attn_gqa_strided``), other dtypes are converted to fp16.

Usage::

    from fqkv_decode import hf_llama
    name = hf_llama.register()                 # "fqkv_decode"
    model.set_attn_implementation(name)        # or model.config._attn_implementation = name

Quantized KV cache (no counterpart in the reference, whose hook keeps an fp16
cache): :class:`QuantizedKVCache` stores every layer's keys and values in the
int8, int4 or fp8 per-token format of ``fqkv_decode.quant``, quantizing new tokens
with the GPU quantizer kernels, and the registered attention function runs
decode steps on it with ``decode_attn_gqa_strided`` (the filled part of the
preallocated cache is a strided view, read in place)::

    cache = hf_llama.QuantizedKVCache(model.config, kv_format="int8")
    model.generate(ids, past_key_values=cache, ...)

The prompt's own prefill attends to its exact keys and values; a later call
with more than one query token attends to the dequantized cache through SDPA.

Graph-captured decoding (no counterpart in the reference, whose decode loop
pays the host's launch cost for every kernel of every step):
:func:`StaticKVCache` keeps each layer's keys and values in preallocated
buffers with the sequence lengths on the device, and the registered
attention function runs its decode steps on ``decode_attn_gqa_paged`` (each
sequence's buffer is one page), so no host value changes from one decode
step to the next and :func:`generate_graphed` captures one whole step of the
model in a HIP graph and replays it per token::

    tokens = hf_llama.generate_graphed(model, ids, max_new_tokens=128)

With ``kv_format="int8"``, ``"int4"`` or ``"fp8"`` (on both) the static cache stores that
per-token format; each step quantizes its new token into place with
``quantize_kv_append_at_``, which reads the position from the device, so the
quantized cache is graph-replayed too.
"""

import math

import torch

DEFAULT_NAME = "fqkv_decode"
_W = 8  # waves per workgroup for the decode kernel
_KV_FORMATS = ("int8", "int4", "fp8")


def _code_storage(kv_format, D):
    """(row width, dtype) of a quantized cache's code rows."""
    return {"int8": (D, torch.int8), "int4": (D // 2, torch.uint8), "fp8": (D, torch.float8_e4m3fn)}[kv_format]


def _dequant(codes, scales):
    from . import quant

    if codes.dtype == torch.int8:
        return quant.dequant_int8(codes, scales)
    if codes.dtype == torch.float8_e4m3fn:
        return quant.dequant_fp8(codes, scales)
    return quant.dequant_int4(codes, scales)


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
    if getattr(key, "fqkv_seq_lens", None) is not None:
        return _static_attention(module, query, key, value, attention_mask, scaling, dropout, **kwargs)
    if getattr(key, "fqkv_scales", None) is not None:
        return _quantized_attention(module, query, key, value, attention_mask, scaling, dropout, **kwargs)
    if getattr(module, "training", False) or not kernel_applies(query, key, attention_mask, scaling, dropout,
                                                               **kwargs):
        return _sdpa(module, query, key, value, attention_mask, scaling=scaling, dropout=dropout, **kwargs)
    from . import decode_attn_gqa, decode_attn_gqa_strided

    q = query[:, :, 0, :].to(torch.float16).contiguous()  # [B, Hq, D]
    if key.dtype == torch.bfloat16 and key.stride(-1) == 1 and value.stride() == key.stride():
        # a bf16 model's cache is read as it is (no per-step conversion of the whole cache)
        out = decode_attn_gqa_strided(q, key, value, _W)
    else:
        K = key.to(torch.float16).contiguous()             # [B, Hkv, N, D]
        V = value.to(torch.float16).contiguous()
        out = decode_attn_gqa(q, K, V, _W)                 # [B, Hq, D]
    return out.unsqueeze(1).to(query.dtype), None          # [B, 1, Hq, D]


def _static_attention(module, query, key, value, attention_mask, scaling, dropout, **kwargs):
    """Attention over a StaticKVCache layer's whole buffers [B, Hkv, capacity, D] (fp16, or int8 /
    packed int4 carrying their fp16 scales [B, Hkv, capacity]): a decode step runs the paged kernel
    over the first seq_lens[b] tokens of sequence b's buffer (one page of ``capacity`` tokens; the
    lengths are read on the device); anything else goes to SDPA with transformers' mask (over the
    dequantized cache for int8 / int4 / fp8)."""
    B, Hq, qlen, D = query.shape
    ks, vs = getattr(key, "fqkv_scales", None), getattr(value, "fqkv_scales", None)
    # a caller's padding mask (folded into transformers' mask by the builder register() installs)
    # may hide positions below the length: that step goes to SDPA with the mask
    ok = (qlen == 1 and not dropout and not getattr(module, "training", False) and query.is_cuda
          and not getattr(attention_mask, "fqkv_padding", False)
          and (key.dtype in (torch.float16, torch.bfloat16) or ks is not None) and D in (64, 128)
          and Hq % key.shape[1] == 0
          and kwargs.get("sliding_window") is None and kwargs.get("softcap") is None
          and (scaling is None or abs(scaling * math.sqrt(D) - 1.0) <= 1e-6))
    if not ok:
        if ks is not None:
            key, value = _dequant(key, ks).to(query.dtype), _dequant(value, vs).to(query.dtype)
        return _sdpa(module, query, key, value, attention_mask, scaling=scaling, dropout=dropout, **kwargs)
    from . import decode_attn_gqa_paged

    q = query[:, :, 0, :].to(torch.float16).contiguous()
    pages = lambda t: None if t is None else t.permute(0, 2, 1)  # [B, Hkv, cap] -> [B, cap, Hkv]
    out = decode_attn_gqa_paged(q, key.permute(0, 2, 1, 3), value.permute(0, 2, 1, 3), key.fqkv_page_table,
                                key.fqkv_seq_lens, key.shape[2], _W, pages(ks), pages(vs))
    return out.unsqueeze(1).to(query.dtype), None


def _quantized_attention(module, query, key, value, attention_mask, scaling, dropout, **kwargs):
    """Attention over a QuantizedKVCache view: key/value are int8, packed uint8 (int4) or
    float8_e4m3fn [B, Hkv, kv, D or D/2] views carrying their fp16 scales [B, Hkv, kv] as
    ``fqkv_scales``."""
    ks, vs = key.fqkv_scales, value.fqkv_scales
    if not getattr(module, "training", False) and kernel_applies(query, key, attention_mask, scaling, dropout,
                                                                 **kwargs):
        from . import decode_attn_gqa_strided

        q = query[:, :, 0, :].to(torch.float16).contiguous()
        out = decode_attn_gqa_strided(q, key, value, _W, ks, vs)
        return out.unsqueeze(1).to(query.dtype), None
    K = _dequant(key, ks).to(query.dtype)
    V = _dequant(value, vs).to(query.dtype)
    return _sdpa(module, query, K, V, attention_mask, scaling=scaling, dropout=dropout, **kwargs)


def _tag(view, scales):
    view.fqkv_scales = scales
    return view


def _make_layer_class():
    # built on first use, so importing this module does not import transformers
    from transformers.cache_utils import DynamicLayer

    class QuantizedKVLayer(DynamicLayer):
        """One decoder layer's KV cache in the kernels' int8 / int4 / fp8 per-token format.

        Storage is preallocated [B, Hkv, capacity, D] int8 (or [.., D/2] packed
        uint8 for int4) plus [B, Hkv, capacity] fp16 scales, grown in blocks of
        ``block`` tokens; new tokens are quantized on the GPU straight into
        their slots (``quantize_kv_append_``, bytes identical to
        ``fqkv_decode.quant``). ``keys`` / ``values`` are views of the filled
        part. ``update`` returns the exact new states for a first (prefill)
        call and the quantized views, tagged with their scales, afterwards.
        """

        def __init__(self, kv_format="int8", block=256):
            super().__init__()
            if kv_format not in _KV_FORMATS:
                raise ValueError("kv_format must be 'int8', 'int4' or 'fp8', got %r" % (kv_format,))
            self.kv_format = kv_format
            self.block = block
            self.length = 0
            self._k = self._v = self._ks = self._vs = None

        def lazy_initialization(self, key_states, value_states):
            self.dtype, self.device = key_states.dtype, key_states.device
            self.is_initialized = True

        def _reserve(self, B, H, D, need):
            cap = 0 if self._k is None else self._k.shape[2]
            if need <= cap:
                return
            cap = -(-max(need, 2 * cap) // self.block) * self.block
            width, dt = _code_storage(self.kv_format, D)
            k = torch.empty(B, H, cap, width, dtype=dt, device=self.device)
            v = torch.empty_like(k)
            ks = torch.empty(B, H, cap, dtype=torch.float16, device=self.device)
            vs = torch.empty_like(ks)
            if self.length:
                n = self.length
                k[:, :, :n] = self._k[:, :, :n]
                v[:, :, :n] = self._v[:, :, :n]
                ks[:, :, :n] = self._ks[:, :, :n]
                vs[:, :, :n] = self._vs[:, :, :n]
            self._k, self._v, self._ks, self._vs = k, v, ks, vs

        def _views(self):
            n = self.length
            self.keys, self.values = self._k[:, :, :n], self._v[:, :, :n]
            return (_tag(self._k[:, :, :n], self._ks[:, :, :n]), _tag(self._v[:, :, :n], self._vs[:, :, :n]))

        def update(self, key_states, value_states, *args, **kwargs):
            from . import quantize_kv_append_

            if not self.is_initialized:
                self.lazy_initialization(key_states, value_states)
            B, H, n, D = key_states.shape
            first = self.length == 0
            self._reserve(B, H, D, self.length + n)
            src = (lambda t: t) if key_states.dtype in (torch.float16, torch.float32, torch.bfloat16) else (
                lambda t: t.float())
            # one launch quantizes the new K and V tokens into their cache slots
            quantize_kv_append_(src(key_states).contiguous(), src(value_states).contiguous(), self._k, self._v,
                                self._ks, self._vs, self.length)
            self.length += n
            views = self._views()
            return (key_states, value_states) if first else views

        def get_seq_length(self):
            return self.length

        def get_max_length(self):
            return -1

        def crop(self, tokens_to_remove):
            if tokens_to_remove > 0:  # legacy form: the length to keep
                n = min(tokens_to_remove, self.length)
            else:
                n = self.length + tokens_to_remove
            self.length = max(0, n)
            if self._k is not None:
                self._views()

        def batch_repeat_interleave(self, repeats):
            if self._k is not None:
                self._k, self._v, self._ks, self._vs = (t.repeat_interleave(repeats, dim=0)
                                                        for t in (self._k, self._v, self._ks, self._vs))
                self._views()

        def batch_select_indices(self, indices):
            if self._k is not None:
                self._k, self._v, self._ks, self._vs = (t[indices].contiguous()
                                                        for t in (self._k, self._v, self._ks, self._vs))
                self._views()

        def reset(self):
            self.length = 0
            if self._k is not None:
                self._views()

        def offload(self):
            raise NotImplementedError("QuantizedKVLayer does not support offloading")

        def prefetch(self):
            raise NotImplementedError("QuantizedKVLayer does not support offloading")

    return QuantizedKVLayer


_LAYER_CLASS = None


def QuantizedKVLayer(kv_format="int8", block=256):
    """A transformers cache layer holding int8 / int4 / fp8 KV (class built on first use)."""
    global _LAYER_CLASS
    if _LAYER_CLASS is None:
        _LAYER_CLASS = _make_layer_class()
    return _LAYER_CLASS(kv_format, block)


def QuantizedKVCache(config, kv_format="int8", block=256):
    """A transformers ``Cache`` whose every layer is a :func:`QuantizedKVLayer`; pass it to
    ``generate(past_key_values=...)`` or a forward call with the attention implementation
    :func:`register` installed."""
    from transformers.cache_utils import Cache

    text = config.get_text_config(decoder=True) if hasattr(config, "get_text_config") else config
    return Cache(layers=[QuantizedKVLayer(kv_format, block) for _ in range(text.num_hidden_layers)])


def _make_static_layer_class():
    from transformers.cache_utils import StaticLayer

    class DeviceLengthStaticLayer(StaticLayer):
        """transformers' StaticLayer (keys and values preallocated as [B, Hkv, capacity, D], new
        tokens written in place at a position kept on the device) that also keeps each sequence's
        length as a device int32 tensor. The key and value buffers it returns carry the lengths
        and a one-page-per-sequence page table, which the registered attention function hands
        to the paged decode kernel: nothing in a decode step reads a length on the host."""

        def __init__(self, max_cache_len):
            if max_cache_len < 16 or max_cache_len > (1 << 20) or max_cache_len & (max_cache_len - 1):
                raise ValueError("max_cache_len must be a power of two in [16, 2^20] (one kernel page per "
                                 "sequence), got %r" % (max_cache_len,))
            super().__init__(max_cache_len=max_cache_len)
            self.seq_lens = self.page_table = None
            self.tokens = 0  # tokens stored, counted on the host (graph replays do not come through here)

        def _count(self, n):
            # checked before anything is written: the kernels would clamp the lengths, so a cache that
            # overflowed would attend to its first max_cache_len tokens without a word
            if self.tokens + n > self.max_cache_len:
                raise ValueError("StaticKVCache: %d cached + %d new tokens exceed max_cache_len %d"
                                 % (self.tokens, n, self.max_cache_len))
            self.tokens += n

        def lazy_initialization(self, key_states, value_states):
            super().lazy_initialization(key_states, value_states)
            B = self.batch_size
            self.seq_lens = torch.zeros(B, dtype=torch.int32, device=self.device)
            self.page_table = torch.arange(B, dtype=torch.int32, device=self.device).view(B, 1)
            for t in (self.keys, self.values):
                t.fqkv_seq_lens = self.seq_lens
                t.fqkv_page_table = self.page_table

        def update(self, key_states, value_states, *args, **kwargs):
            self._count(key_states.shape[-2])
            keys, values = super().update(key_states, value_states, *args, **kwargs)
            self.seq_lens.add_(key_states.shape[-2])
            return keys, values

        def reset(self):
            super().reset()
            self.tokens = 0
            if self.is_initialized:
                self.cumulative_length.zero_()
                self.seq_lens.zero_()

        def _state(self):
            return (self.keys, self.values, self.seq_lens)

        def reorder_cache(self, beam_idx):
            # in place, so the buffers keep their tags and the addresses a captured graph holds
            if self.is_initialized:
                idx = beam_idx.to(self.device)
                for t in self._state():
                    t.copy_(t.index_select(0, idx))

        def offload(self):
            raise NotImplementedError("StaticKVCache layers stay on their GPU (the lengths live there)")

        def prefetch(self):
            raise NotImplementedError("StaticKVCache layers stay on their GPU (the lengths live there)")

    class DeviceLengthQuantizedLayer(DeviceLengthStaticLayer):
        """The same with int8 (or packed int4) keys and values and fp16 per-token scales, new tokens
        quantized into place at the position held on the device (``quantize_kv_append_at_``, bytes
        equal to ``fqkv_decode.quant``'s quantizers). The first call (the prompt) attends to its exact
        states, with a mask of their length; later calls get the quantized buffers, tagged with
        their scales."""

        def __init__(self, max_cache_len, kv_format):
            if kv_format not in _KV_FORMATS:
                raise ValueError("kv_format must be 'int8', 'int4' or 'fp8', got %r" % (kv_format,))
            super().__init__(max_cache_len)
            self.kv_format = kv_format
            self.prefilled = False

        def lazy_initialization(self, key_states, value_states):
            self.dtype, self.device = key_states.dtype, key_states.device
            self.batch_size, self.num_heads = key_states.shape[:2]
            B, H, D = self.batch_size, self.num_heads, key_states.shape[-1]
            self.k_head_dim = self.v_head_dim = D
            width, dt = _code_storage(self.kv_format, D)
            cap = self.max_cache_len
            self.keys = torch.zeros(B, H, cap, width, dtype=dt, device=self.device)
            self.values = torch.zeros_like(self.keys)
            self.key_scales = torch.zeros(B, H, cap, dtype=torch.float16, device=self.device)
            self.value_scales = torch.zeros_like(self.key_scales)
            self.cumulative_length = self.cumulative_length.to(self.device)
            self.seq_lens = torch.zeros(B, dtype=torch.int32, device=self.device)
            self.page_table = torch.arange(B, dtype=torch.int32, device=self.device).view(B, 1)
            for t, sc in ((self.keys, self.key_scales), (self.values, self.value_scales)):
                t.fqkv_seq_lens = self.seq_lens
                t.fqkv_page_table = self.page_table
                t.fqkv_scales = sc
            self.is_initialized = True

        def update(self, key_states, value_states, *args, **kwargs):
            from . import quantize_kv_append_at_

            n = key_states.shape[-2]
            self._count(n)
            if not self.is_initialized:
                self.lazy_initialization(key_states, value_states)
            kn, vn = key_states, value_states
            if kn.dtype not in (torch.float16, torch.float32, torch.bfloat16):
                kn, vn = kn.float(), vn.float()
            # one launch quantizes the new K and V tokens into their slots, at seq_lens on the device
            quantize_kv_append_at_(kn.contiguous(), vn.contiguous(), self.keys, self.values, self.key_scales,
                                   self.value_scales, self.seq_lens)
            self.seq_lens.add_(n)
            self.cumulative_length.add_(n)
            if not self.prefilled:
                self.prefilled = True
                return key_states, value_states
            return self.keys, self.values

        def get_mask_sizes(self, query_length):
            return (self.max_cache_len, 0) if self.prefilled else (query_length, 0)

        def _state(self):
            return (self.keys, self.values, self.key_scales, self.value_scales, self.seq_lens)

        def reset(self):
            super().reset()
            self.prefilled = False
            if self.is_initialized:
                self.key_scales.zero_()
                self.value_scales.zero_()

    return DeviceLengthStaticLayer, DeviceLengthQuantizedLayer


_STATIC_LAYER_CLASSES = None


def StaticKVCache(config, max_cache_len, kv_format=None):
    """A transformers ``Cache`` of preallocated KV buffers (the model's fp16 or bf16) with the sequence lengths on the
    device, for decode steps captured in a HIP graph (:func:`generate_graphed`). ``max_cache_len``
    (a power of two in [16, 2^20]) bounds prompt plus generated tokens. Decode steps on the kernel
    attend to the first ``length`` positions of each buffer and read no attention mask, so a call
    that passes a padding mask runs its decode steps on SDPA instead (still correct, not
    graph-replayed by :func:`generate_graphed`, which passes none). ``kv_format`` "int8", "int4" or "fp8"
    stores the cache in that per-token format, quantized on the GPU as tokens arrive (the prompt
    attends to its exact states, later calls to the quantized cache)."""
    from transformers.cache_utils import Cache

    global _STATIC_LAYER_CLASSES
    if _STATIC_LAYER_CLASSES is None:
        _STATIC_LAYER_CLASSES = _make_static_layer_class()
    fp16_layer, quant_layer = _STATIC_LAYER_CLASSES
    text = config.get_text_config(decoder=True) if hasattr(config, "get_text_config") else config
    if kv_format is None:
        return Cache(layers=[fp16_layer(max_cache_len) for _ in range(text.num_hidden_layers)])
    return Cache(layers=[quant_layer(max_cache_len, kv_format) for _ in range(text.num_hidden_layers)])


def generate_graphed(model, input_ids, max_new_tokens, max_cache_len=None, use_graph=True, kv_format=None):
    """Greedy decoding with every decode step replayed from one captured HIP graph.

    The prompt runs eagerly into a :func:`StaticKVCache` (capacity ``max_cache_len``, by default the
    next power of two, at least 16, above prompt + new tokens); the first decode step runs eagerly
    too (it initialises what the step uses lazily), the second is captured, and every later token
    is one replay: the graph embeds the token, runs the model on the cache (the attention through
    the paged kernel when the model's attention implementation is this module's), and writes its
    argmax back as the next step's input. The prompt rows are taken as unpadded (no attention mask
    is passed).
    ``use_graph=False`` runs the same steps eagerly; ``kv_format`` "int8" / "int4" / "fp8" keeps the cache in
    that format (:func:`StaticKVCache`). Returns the new tokens, [B, max_new_tokens]."""
    B, L = input_ids.shape
    if max_new_tokens < 1:
        raise ValueError("max_new_tokens must be >= 1")
    cap = max_cache_len or max(16, 1 << (L + max_new_tokens - 1).bit_length())
    if L + max_new_tokens > cap:
        raise ValueError("prompt + new tokens (%d) exceed max_cache_len (%d)" % (L + max_new_tokens, cap))
    dev = input_ids.device
    cache = StaticKVCache(model.config, cap, kv_format)
    out = torch.empty(B, max_new_tokens, dtype=torch.long, device=dev)
    with torch.no_grad():
        logits = model(input_ids, past_key_values=cache, use_cache=True).logits
        ids = logits[:, -1:].argmax(-1)
        out[:, :1] = ids
        pos = torch.full((B, 1), L, dtype=torch.long, device=dev)

        def step():
            lg = model(ids, past_key_values=cache, position_ids=pos, use_cache=True).logits
            ids.copy_(lg[:, -1:].argmax(-1))
            pos.add_(1)

        if max_new_tokens > 1:
            step()
            out[:, 1:2] = ids
        if max_new_tokens > 2 and not use_graph:
            for i in range(2, max_new_tokens):
                step()
                out[:, i:i + 1] = ids
        elif max_new_tokens > 2:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                step()
            for i in range(2, max_new_tokens):
                graph.replay()
                out[:, i:i + 1] = ids
    return out


def _sdpa_mask(*args, **kwargs):
    """transformers' SDPA mask builder; a mask that folds in a caller's 2-D padding mask is tagged
    ``fqkv_padding`` so the static-cache decode path, which reads no mask, leaves it to SDPA."""
    from transformers.masking_utils import sdpa_mask

    mask = sdpa_mask(*args, **kwargs)
    if mask is not None and kwargs.get("attention_mask") is not None:
        mask.fqkv_padding = True
    return mask


def register(name=DEFAULT_NAME):
    """Register the attention function (and the SDPA mask builder) under ``name``; returns ``name``."""
    from transformers import AttentionInterface, AttentionMaskInterface

    AttentionInterface.register(name, attention_forward)
    AttentionMaskInterface.register(name, _sdpa_mask)
    return name
