"""The transformers integration (fqkv_decode.hf_llama), the reference's HF hook
(nb:1037-1064) on a random-init Llama (no checkpoint download):

* CPU: registration, the kernel/SDPA routing rule, and a whole generate() on
  CPU tensors, which must route every call to SDPA and match it exactly;
* GPU: decode steps through the kernel against SDPA (logits within fp16
  noise) and greedy generation token-for-token equal to SDPA's (a divergence
  is accepted only where SDPA's own top-2 logit margin is below 1e-2, i.e. at
  a numerical tie), at short and long context (the latter takes the
  kernel's internal sequence split);
* GPU, int8 / int4 KV cache (hf_llama.QuantizedKVCache): stored bytes equal
  the quantizer's, attention over the cache view equals float32 attention
  over the dequantized cache, decode logits equal SDPA over the same
  dequantized cache, and generate() runs every decode step on the kernel."""

import math

import pytest
import torch

transformers = pytest.importorskip("transformers")

from fqkv_decode import hf_llama  # noqa: E402


def tiny_llama(layers=4, hidden=512, heads=8, kv_heads=2, head_dim=64, vocab=1000, init=0.2, dtype=torch.float32,
               device="cpu", intermediate=None):
    cfg = transformers.LlamaConfig(vocab_size=vocab, hidden_size=hidden, intermediate_size=intermediate or 2 * hidden,
                                   num_hidden_layers=layers, num_attention_heads=heads,
                                   num_key_value_heads=kv_heads, head_dim=head_dim,
                                   max_position_embeddings=8192, initializer_range=init,
                                   attn_implementation="sdpa")
    torch.manual_seed(0)
    with torch.device(device):
        model = transformers.LlamaForCausalLM(cfg)
    return model.to(dtype).eval()


def _quantizers():
    from fqkv_decode import quant

    return {"int8": quant.quant_int8_per_token, "int4": quant.quant_int4_per_token, "fp8": quant.quant_fp8_per_token}


class _Lazy(dict):
    def __missing__(self, k):
        self.update(_quantizers())
        return self[k]


QUANTIZERS = _Lazy()  # kv_format -> fqkv_decode.quant's quantizer


def bits(t):
    """The bytes of a code tensor (float8 tensors compare through uint8)."""
    return t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t


def set_impl(model, name):
    model.config._attn_implementation = name
    for layer in model.model.layers:
        layer.self_attn.config._attn_implementation = name


def test_routing_rule():
    q = torch.zeros(2, 8, 1, 64)
    k = torch.zeros(2, 2, 10, 64)
    ok = dict(attention_mask=None, scaling=1 / math.sqrt(64), dropout=0.0)
    assert not hf_llama.kernel_applies(q, k, **ok)  # CPU tensors never take the kernel
    if torch.cuda.is_available():
        assert hf_llama.kernel_applies(q.cuda(), k.cuda(), **ok)
    assert not hf_llama.kernel_applies(torch.zeros(2, 8, 3, 64), k, **ok)          # prefill
    assert not hf_llama.kernel_applies(q, k, torch.zeros(2, 1, 1, 10), 0.125, 0.0)  # mask
    assert not hf_llama.kernel_applies(q, k, None, 0.2, 0.0)                        # other scale
    assert not hf_llama.kernel_applies(torch.zeros(2, 6, 1, 64), torch.zeros(2, 4, 10, 64), **ok)
    assert not hf_llama.kernel_applies(torch.zeros(2, 8, 1, 80), torch.zeros(2, 2, 10, 80), None, None, 0.0)
    assert not hf_llama.kernel_applies(q, k, **ok, sliding_window=4)


def test_register_and_cpu_generation_falls_back_to_sdpa():
    name = hf_llama.register()
    assert name in transformers.AttentionInterface._global_mapping
    model = tiny_llama(layers=2, hidden=256, heads=4, kv_heads=2)
    ids = torch.randint(0, 1000, (1, 12), generator=torch.Generator().manual_seed(1))
    set_impl(model, "sdpa")
    with torch.no_grad():
        base = model.generate(ids, max_new_tokens=8, do_sample=False)
    set_impl(model, name)
    with torch.no_grad():
        ours = model.generate(ids, max_new_tokens=8, do_sample=False)
    assert torch.equal(base, ours)


def greedy(model, ids, steps, cache=None):
    """Greedy decode by hand (on ``cache`` if given); returns tokens and each step's top-2 logit margin."""
    toks, margins = [], []
    with torch.no_grad():
        out = model(ids, past_key_values=cache, use_cache=True)
        past = out.past_key_values
        logits = out.logits[:, -1].float()
        for _ in range(steps):
            top = logits.topk(2, dim=-1)
            margins.append(float((top.values[0, 0] - top.values[0, 1])))
            nxt = top.indices[:, :1]
            toks.append(int(nxt[0, 0]))
            out = model(nxt, past_key_values=past, use_cache=True)
            past = out.past_key_values
            logits = out.logits[:, -1].float()
    return toks, margins


# Llama-3.2-1B's attention geometry (nb:966): 16 layers, 32 query / 8 KV
# heads of 64, hidden 2048, MLP 8192, vocabulary 128256; random init at the
# LlamaConfig default scale (no checkpoint is fetched). "small" is a 4-layer
# model with 8 / 2 heads for a quick second geometry.
GEOMETRIES = {
    "llama32_1b": dict(layers=16, hidden=2048, heads=32, kv_heads=8, head_dim=64, vocab=128256, init=0.02,
                       intermediate=8192),
    "small": dict(),
}


@pytest.mark.gpu
@pytest.mark.parametrize("geometry", sorted(GEOMETRIES))
@pytest.mark.parametrize("ctx", [37, 3000])
def test_gpu_decode_matches_sdpa(ctx, geometry):
    name = hf_llama.register()
    model = tiny_llama(dtype=torch.float16, device="cuda", **GEOMETRIES[geometry])
    vocab = model.config.vocab_size
    ids = torch.randint(0, vocab, (1, ctx), generator=torch.Generator().manual_seed(2)).cuda()
    set_impl(model, "sdpa")
    base, margins = greedy(model, ids, 24)
    set_impl(model, name)
    ours, _ = greedy(model, ids, 24)
    for i, (a, b) in enumerate(zip(base, ours)):
        if a != b:
            assert margins[i] < 1e-2, ("divergence at step %d without a tie" % i, margins[i])
            break
    # one decode step's logits on the same cache, both ways
    with torch.no_grad():
        set_impl(model, "sdpa")
        out = model(ids, use_cache=True)
        past = out.past_key_values
        nxt = out.logits[:, -1:].argmax(-1)
        import copy
        past2 = copy.deepcopy(past)
        ref = model(nxt, past_key_values=past, use_cache=True).logits.float()
        set_impl(model, name)
        got = model(nxt, past_key_values=past2, use_cache=True).logits.float()
    assert float((got - ref).abs().max()) <= 2e-2 * max(1.0, float(ref.abs().max()) / 10)


@pytest.mark.gpu
def test_gpu_decode_path_really_runs_the_kernel(monkeypatch):
    """The decode call goes through fqkv_decode.decode_attn_gqa (not SDPA)."""
    name = hf_llama.register()
    model = tiny_llama(layers=2, dtype=torch.float16, device="cuda")
    calls = {"n": 0}
    import fqkv_decode

    real = fqkv_decode.decode_attn_gqa

    def counting(*a, **k):
        calls["n"] += 1
        return real(*a, **k)

    monkeypatch.setattr(fqkv_decode, "decode_attn_gqa", counting, raising=False)
    set_impl(model, name)
    ids = torch.randint(0, 1000, (1, 9), generator=torch.Generator().manual_seed(3)).cuda()
    with torch.no_grad():
        model.generate(ids, max_new_tokens=3, do_sample=False)
    assert calls["n"] == 2 * 2  # 2 layers x 2 decode steps (the first token comes from prefill)


# ------------------------------------------------------------ quantized KV cache ----

def _prefill(model, ids, cache):
    with torch.no_grad():
        out = model(ids, past_key_values=cache, use_cache=True)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["int8", "int4", "fp8"])
def test_gpu_quantized_cache_stores_the_quantizer_bytes(fmt):
    """After a prefill, every layer holds exactly fqkv_decode.quant's bytes and scales of the
    prompt's keys and values (the prefill itself attends to the exact states)."""
    from fqkv_decode import quant

    name = hf_llama.register()
    model = tiny_llama(layers=2, dtype=torch.float16, device="cuda")
    set_impl(model, name)
    ids = torch.randint(0, 1000, (2, 300), generator=torch.Generator().manual_seed(4)).cuda()
    dyn = transformers.DynamicCache(config=model.config)
    ref_logits = _prefill(model, ids, dyn).logits
    qc = hf_llama.QuantizedKVCache(model.config, fmt)
    logits = _prefill(model, ids, qc).logits
    assert torch.equal(logits, ref_logits)
    assert qc.get_seq_length() == 300
    qfn = QUANTIZERS[fmt]
    for lq, ld in zip(qc.layers, dyn.layers):
        for got, gs, x in ((lq._k, lq._ks, ld.keys), (lq._v, lq._vs, ld.values)):
            want, ws = qfn(x)
            assert torch.equal(bits(got[:, :, :300]), bits(want))
            assert torch.equal(gs[:, :, :300], ws)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["int8", "int4", "fp8"])
def test_gpu_quantized_cache_decode_step(fmt, monkeypatch):
    """A decode step on the quantized cache. Attention level: the kernel on the strided
    cache view equals float32 attention over the dequantized cache (max-abs 2e-3 relative
    to the output scale). Model level: the logits equal those of SDPA over the same
    dequantized cache to 2 % of the logit scale (SDPA sees fp16-rounded K/V), and, for
    int8, stay within 15 % of the logit scale of an fp16 cache (quantization error)."""
    import copy

    from fqkv_decode import quant

    name = hf_llama.register()
    model = tiny_llama(dtype=torch.float16, device="cuda")
    set_impl(model, name)
    ids = torch.randint(0, 1000, (1, 1500), generator=torch.Generator().manual_seed(5)).cuda()
    qc = hf_llama.QuantizedKVCache(model.config, fmt)
    out = _prefill(model, ids, qc)
    nxt = out.logits[:, -1:].argmax(-1)
    qc2 = copy.deepcopy(qc)
    with torch.no_grad():
        got = model(nxt, past_key_values=qc, use_cache=True).logits.float()
        monkeypatch.setattr(hf_llama, "kernel_applies", lambda *a, **k: False)
        sdpa_deq = model(nxt, past_key_values=qc2, use_cache=True).logits.float()
        monkeypatch.undo()
        dyn = transformers.DynamicCache(config=model.config)
        _prefill(model, ids, dyn)
        fp16 = model(nxt, past_key_values=dyn, use_cache=True).logits.float()
    assert qc.get_seq_length() == 1501
    top = float(fp16.abs().max())
    assert float((got - sdpa_deq).abs().max()) <= 0.02 * top
    if fmt == "int8":
        assert float((got - fp16).abs().max()) <= 0.15 * top

    # attention level, layer 0, a fresh query
    k, v = qc.layers[0]._views()
    q = torch.randn(1, 8, 1, 64, device="cuda", generator=torch.Generator(device="cuda").manual_seed(0)).half()
    o, _ = hf_llama.attention_forward(model.model.layers[0].self_attn, q, k, v, None, scaling=1 / 8)
    deq = hf_llama._dequant
    Kf = deq(k, k.fqkv_scales).float().repeat_interleave(4, 1)
    Vf = deq(v, v.fqkv_scales).float().repeat_interleave(4, 1)
    ref = torch.softmax(q.float() @ Kf.transpose(-1, -2) / 8, -1) @ Vf
    err = float((o.float().transpose(1, 2) - ref).abs().max())
    assert err <= 2e-3 * max(1.0, float(ref.abs().max())), (err, float(ref.abs().max()))


@pytest.mark.gpu
def test_gpu_generate_with_quantized_cache_runs_the_kernel(monkeypatch):
    name = hf_llama.register()
    model = tiny_llama(layers=2, dtype=torch.float16, device="cuda")
    set_impl(model, name)
    import fqkv_decode

    calls = {"n": 0}
    real = fqkv_decode.decode_attn_gqa_strided

    def counting(*a, **k):
        calls["n"] += 1
        return real(*a, **k)

    monkeypatch.setattr(fqkv_decode, "decode_attn_gqa_strided", counting, raising=False)
    ids = torch.randint(0, 1000, (1, 20), generator=torch.Generator().manual_seed(6)).cuda()
    with torch.no_grad():
        out = model.generate(ids, max_new_tokens=300, do_sample=False,
                             past_key_values=hf_llama.QuantizedKVCache(model.config, "int8", block=64))
    assert out.shape == (1, 320)
    assert calls["n"] == 2 * 299  # every decode step of both layers (the capacity grows past 256 on the way)


def test_static_cache_rejects_a_capacity_the_kernel_cannot_page():
    cfg = transformers.LlamaConfig(vocab_size=100, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=32)
    for bad in (0, 8, 100, 3 << 10, 1 << 21):
        with pytest.raises(ValueError, match="power of two"):
            hf_llama.StaticKVCache(cfg, bad)
    assert len(hf_llama.StaticKVCache(cfg, 64).layers) == 2
    with pytest.raises(ValueError, match="kv_format"):
        hf_llama.StaticKVCache(cfg, 64, "fp4")
    assert len(hf_llama.StaticKVCache(cfg, 64, "int4").layers) == 2


def test_static_cache_cpu_decode_matches_dynamic_cache():
    """On CPU every call goes to SDPA; the static cache (lengths on the device, positions passed
    in) must reproduce generate()'s greedy tokens over the dynamic cache."""
    model = tiny_llama(layers=2, hidden=256, heads=4, kv_heads=2)
    ids = torch.randint(0, 1000, (2, 12), generator=torch.Generator().manual_seed(3))
    set_impl(model, hf_llama.register())
    with torch.no_grad():
        base = model.generate(ids, max_new_tokens=6, do_sample=False)[:, 12:]
        cache = hf_llama.StaticKVCache(model.config, 32)
        tok = model(ids, past_key_values=cache, use_cache=True).logits[:, -1:].argmax(-1)
        toks, pos = [tok], torch.full((2, 1), 12, dtype=torch.long)
        for _ in range(5):
            tok = model(tok, past_key_values=cache, position_ids=pos, use_cache=True).logits[:, -1:].argmax(-1)
            toks.append(tok)
            pos += 1
    assert torch.equal(base, torch.cat(toks, 1))
    assert cache.layers[0].seq_lens.tolist() == [17, 17]


def test_static_cache_refuses_to_overflow():
    """More tokens than max_cache_len raise before anything is written (the kernels would clamp
    the lengths and attend to the first max_cache_len tokens), for the fp16 and the int8 layer."""
    model = tiny_llama(layers=2, hidden=256, heads=4, kv_heads=2)
    set_impl(model, hf_llama.register())
    cache = hf_llama.StaticKVCache(model.config, 16)
    ids = torch.randint(0, 1000, (1, 14), generator=torch.Generator().manual_seed(12))
    with torch.no_grad():
        model(ids, past_key_values=cache, use_cache=True)
        model(ids[:, :2], past_key_values=cache, position_ids=torch.tensor([[14, 15]]), use_cache=True)
        with pytest.raises(ValueError, match="exceed max_cache_len 16"):
            model(ids[:, :1], past_key_values=cache, position_ids=torch.tensor([[16]]), use_cache=True)
    assert cache.layers[0].seq_lens.tolist() == [16]
    cache.reset()
    assert cache.layers[0].tokens == 0 and cache.layers[0].seq_lens.tolist() == [0]
    layer = hf_llama.StaticKVCache(model.config, 16, "int8").layers[0]
    with pytest.raises(ValueError, match="exceed max_cache_len"):
        layer.update(torch.zeros(1, 2, 17, 64), torch.zeros(1, 2, 17, 64))
    assert not layer.is_initialized


def test_static_cache_reorders_in_place():
    """reorder_cache (beam search) on the static cache permutes the buffers and lengths in place,
    so they keep the tags the attention function reads and the addresses a graph captured."""
    model = tiny_llama(layers=2, hidden=256, heads=4, kv_heads=2)
    set_impl(model, hf_llama.register())
    ids = torch.randint(0, 1000, (3, 10), generator=torch.Generator().manual_seed(9))
    cache = hf_llama.StaticKVCache(model.config, 16)
    with torch.no_grad():
        model(ids, past_key_values=cache, use_cache=True)
    layer = cache.layers[0]
    layer.seq_lens.copy_(torch.tensor([10, 9, 8], dtype=torch.int32))
    keys, ptr, before = layer.keys, layer.keys.data_ptr(), layer.keys.clone()
    cache.reorder_cache(torch.tensor([2, 2, 0]))
    assert layer.keys is keys and layer.keys.data_ptr() == ptr and keys.fqkv_seq_lens is layer.seq_lens
    assert torch.equal(layer.keys, before[[2, 2, 0]])
    assert layer.seq_lens.tolist() == [8, 8, 10]
    with pytest.raises(NotImplementedError):
        layer.offload()


@pytest.mark.gpu
@pytest.mark.parametrize("geometry", sorted(GEOMETRIES))
def test_gpu_graphed_generation(geometry, monkeypatch):
    """generate_graphed: every decode step after the second is a replay of one captured HIP graph
    whose attention is the paged kernel reading the lengths on the device. The replayed tokens
    equal the same steps run eagerly, bit for bit, and SDPA's greedy tokens (a divergence only at
    an SDPA tie); the captured step called the paged kernel in every layer."""
    name = hf_llama.register()
    model = tiny_llama(dtype=torch.float16, device="cuda", **GEOMETRIES[geometry])
    ids = torch.randint(0, model.config.vocab_size, (1, 45), generator=torch.Generator().manual_seed(4)).cuda()
    set_impl(model, "sdpa")
    base, margins = greedy(model, ids, 40)
    set_impl(model, name)
    import fqkv_decode
    calls = {"n": 0}
    real = fqkv_decode.decode_attn_gqa_paged

    def counted(*a, **k):
        calls["n"] += 1
        return real(*a, **k)

    monkeypatch.setattr(fqkv_decode, "decode_attn_gqa_paged", counted)
    eager = hf_llama.generate_graphed(model, ids, 40, use_graph=False)
    n_eager = calls["n"]
    graphed = hf_llama.generate_graphed(model, ids, 40)
    layers = model.config.num_hidden_layers
    assert n_eager == 39 * layers          # every decode step, every layer
    assert calls["n"] - n_eager == 2 * layers  # the eager first step and the captured one
    assert torch.equal(graphed, eager)
    ours = graphed[0].tolist()
    for i, (a, b) in enumerate(zip(base, ours)):
        if a != b:
            assert margins[i] < 1e-2, ("divergence at step %d without a tie" % i, margins[i])
            break


@pytest.mark.gpu
def test_gpu_static_cache_with_a_padding_mask_goes_to_sdpa(monkeypatch):
    """A left-padded batch over the static cache: the decode step's mask folds in the padding,
    so the registered function hands the step to SDPA with that mask instead of the kernel, which
    reads no mask (the paged kernel is not called); its logits equal SDPA's over the same cache."""
    name = hf_llama.register()
    import fqkv_decode
    calls = {"n": 0}
    real = fqkv_decode.decode_attn_gqa_paged

    def counted(*a, **k):
        calls["n"] += 1
        return real(*a, **k)

    monkeypatch.setattr(fqkv_decode, "decode_attn_gqa_paged", counted)
    model = tiny_llama(layers=2, dtype=torch.float16, device="cuda")
    ids = torch.randint(0, 1000, (2, 20), generator=torch.Generator().manual_seed(5)).cuda()
    mask = torch.ones(2, 20, dtype=torch.long, device="cuda")
    mask[1, :7] = 0  # row 1 left-padded by 7 tokens
    step = torch.randint(0, 1000, (2, 1), generator=torch.Generator().manual_seed(6)).cuda()
    step_mask = torch.cat([mask, torch.ones(2, 1, dtype=torch.long, device="cuda")], 1)
    pos = mask.sum(1, keepdim=True)  # the new token's position in each row
    prefill_pos = (mask.cumsum(1) - 1).clamp(min=0)
    outs = {}
    for impl in ("sdpa", name):
        set_impl(model, impl)
        cache = hf_llama.StaticKVCache(model.config, 32)
        with torch.no_grad():
            model(ids, attention_mask=mask, position_ids=prefill_pos, past_key_values=cache, use_cache=True)
            outs[impl] = model(step, attention_mask=step_mask, position_ids=pos, past_key_values=cache,
                               use_cache=True).logits.float()
    assert calls["n"] == 0
    assert float((outs[name] - outs["sdpa"]).abs().max()) <= 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["int8", "int4", "fp8"])
def test_gpu_static_quantized_cache_prefill_and_decode(fmt):
    """StaticKVCache(kv_format=int8 / int4): the prompt attends to its exact states (logits equal
    the dynamic fp16 cache's), the buffers hold fqkv_decode.quant's bytes and scales of the
    prompt's keys and values at positions [0, L) and zeros after, and a decode step on the paged
    kernel equals float32 attention over the dequantized first L + 1 tokens (max-abs 2e-3 relative
    to the output scale). Eight decode steps fed the same tokens give the dynamic quantized
    cache's logits to 3 % of the logit scale (the two read the same bytes up to the last-bit
    differences of two kernels, which can move a later layer's new token across a rounding
    boundary of the quantizer)."""
    from fqkv_decode import quant

    name = hf_llama.register()
    model = tiny_llama(layers=2, dtype=torch.float16, device="cuda")
    set_impl(model, name)
    L = 300
    ids = torch.randint(0, 1000, (2, L), generator=torch.Generator().manual_seed(7)).cuda()
    dyn = transformers.DynamicCache(config=model.config)
    ref_logits = _prefill(model, ids, dyn).logits
    sc = hf_llama.StaticKVCache(model.config, 512, fmt)
    assert torch.equal(_prefill(model, ids, sc).logits, ref_logits)
    qfn = QUANTIZERS[fmt]
    for ls, ld in zip(sc.layers, dyn.layers):
        assert ls.seq_lens.tolist() == [L, L]
        for got, gs, x in ((ls.keys, ls.key_scales, ld.keys), (ls.values, ls.value_scales, ld.values)):
            want, ws = qfn(x)
            assert torch.equal(bits(got[:, :, :L]), bits(want)) and torch.equal(gs[:, :, :L], ws)
            assert not bits(got[:, :, L:]).any() and not gs[:, :, L:].any()

    nxt = ref_logits[:, -1:].argmax(-1)
    qc = hf_llama.QuantizedKVCache(model.config, fmt)
    _prefill(model, ids, qc)
    pos = torch.full((2, 1), L, dtype=torch.long, device="cuda")
    diffs = []
    with torch.no_grad():
        for _ in range(8):
            got = model(nxt, past_key_values=sc, position_ids=pos, use_cache=True).logits.float()
            want = model(nxt, past_key_values=qc, use_cache=True).logits.float()
            diffs.append(float((got - want).abs().max()) / float(want.abs().max()))
            nxt = want[:, -1:].argmax(-1)
            pos += 1
    assert max(diffs) <= 0.03, diffs
    for _ in range(7):  # undo the last seven steps: the attention check below reads L + 1 tokens
        for ls in sc.layers:
            ls.seq_lens.sub_(1)

    layer = sc.layers[0]
    q = torch.randn(2, 8, 1, 64, device="cuda", generator=torch.Generator(device="cuda").manual_seed(1)).half()
    o, _ = hf_llama.attention_forward(model.model.layers[0].self_attn, q, layer.keys, layer.values, None,
                                      scaling=1 / 8)
    deq = hf_llama._dequant
    n = L + 1
    Kf = deq(layer.keys[:, :, :n], layer.key_scales[:, :, :n]).float().repeat_interleave(4, 1)
    Vf = deq(layer.values[:, :, :n], layer.value_scales[:, :, :n]).float().repeat_interleave(4, 1)
    ref = torch.softmax(q.float() @ Kf.transpose(-1, -2).contiguous() / 8, -1) @ Vf
    err = float((o.float().transpose(1, 2) - ref).abs().max())
    assert err <= 2e-3 * max(1.0, float(ref.abs().max())), (err, float(ref.abs().max()))


@pytest.mark.gpu
def test_gpu_static_quantized_cache_reorders_scales_and_lengths():
    """Beam-search reordering of an int4 static cache moves the scales and lengths with the bytes:
    after reorder_cache([1, 1]) a decode step of the same token gives both rows the logits row 1
    gets without the reorder, bit for bit."""
    name = hf_llama.register()
    model = tiny_llama(layers=2, dtype=torch.float16, device="cuda")
    set_impl(model, name)
    ids = torch.randint(0, 1000, (2, 40), generator=torch.Generator().manual_seed(10)).cuda()
    tok = torch.randint(0, 1000, (2, 1), generator=torch.Generator().manual_seed(11)).cuda()
    pos = torch.full((2, 1), 40, dtype=torch.long, device="cuda")
    out = []
    for reorder in (False, True):
        cache = hf_llama.StaticKVCache(model.config, 64, "int4")
        with torch.no_grad():
            model(ids, past_key_values=cache, use_cache=True)
            if reorder:
                cache.reorder_cache(torch.tensor([1, 1]))
            out.append(model(tok[[1, 1]] if reorder else tok, past_key_values=cache, position_ids=pos,
                             use_cache=True).logits)
    assert torch.equal(out[1][0], out[0][1]) and torch.equal(out[1][1], out[0][1])


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["int8", "int4", "fp8"])
def test_gpu_graphed_generation_quantized(fmt, monkeypatch):
    """generate_graphed over an int8 / int4 / fp8 static cache: each token is appended by the
    device-position quantizer and attended by the paged kernel with scale pages, in the captured
    step too. Replayed tokens equal the eager steps bit for bit, and the greedy tokens over the
    dynamic quantized cache (int8: a divergence only where that run's top-2 margin is below 2e-2;
    int4 and fp8 are held to the measured account of their divergences in
    test_gpu_quantized_greedy_paths_part_through_rounding_flips below)."""
    name = hf_llama.register()
    model = tiny_llama(dtype=torch.float16, device="cuda")
    set_impl(model, name)
    ids = torch.randint(0, 1000, (1, 45), generator=torch.Generator().manual_seed(8)).cuda()
    if fmt == "int8":
        base, margins = greedy(model, ids, 40, hf_llama.QuantizedKVCache(model.config, fmt))
    import fqkv_decode
    calls = {"n": 0}
    real = fqkv_decode.decode_attn_gqa_paged

    def counted(*a, **k):
        assert a[7] is not None and a[8] is not None  # the scale pages
        calls["n"] += 1
        return real(*a, **k)

    monkeypatch.setattr(fqkv_decode, "decode_attn_gqa_paged", counted)
    eager = hf_llama.generate_graphed(model, ids, 40, use_graph=False, kv_format=fmt)
    n_eager = calls["n"]
    graphed = hf_llama.generate_graphed(model, ids, 40, kv_format=fmt)
    layers = model.config.num_hidden_layers
    assert n_eager == 39 * layers
    assert calls["n"] - n_eager == 2 * layers
    assert torch.equal(graphed, eager)
    if fmt != "int8":
        return
    for i, (a, b) in enumerate(zip(base, graphed[0].tolist())):
        if a != b:
            assert margins[i] < 2e-2, ("divergence at step %d without a tie" % i, margins[i])
            break


def _signed_codes(t, fmt):
    """Codes as signed integers one quantizer step apart: int8 as is, int4 unpacked, fp8 e4m3 as
    sign and magnitude of its bit pattern (adjacent values differ by one)."""
    from fqkv_decode import quant

    if fmt == "int4":
        return quant.unpack_int4(t).to(torch.int16)
    if fmt == "fp8":
        b = t.view(torch.uint8).to(torch.int16)
        return torch.where(b >= 128, -(b & 127), b)
    return t.to(torch.int16)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["int8", "int4", "fp8"])
def test_gpu_quantized_greedy_paths_part_through_rounding_flips(fmt):
    """Why the greedy tokens over the dynamic and the static quantized cache may part (int4 at
    step 23 of this prompt), measured by feeding the graphed path's 40 tokens to both caches:
    (1) after the prompt both hold the same codes and scales, and the two kernels that read them
    (strided for the dynamic cache, paged for the static one; different passes and split
    choices) agree to their error bound but not bit for bit (over 20 random queries at least one
    output element differs); (2) after the first decode step layer 0's new codes are still equal
    (its inputs are the token's embedding) and every code that differs in a later layer is one
    quantizer step from the other cache's, its scale equal or one fp16 ulp away: a last-bit
    difference of the kernels moved a value across a rounding boundary; (3) the free-running
    paths part exactly one token after the first step at which, fed the same tokens, the two
    caches' logits rank a different token first (and never if no step does)."""
    import fqkv_decode

    name = hf_llama.register()
    model = tiny_llama(dtype=torch.float16, device="cuda")
    set_impl(model, name)
    ids = torch.randint(0, 1000, (1, 45), generator=torch.Generator().manual_seed(8)).cuda()
    L, steps = ids.shape[1], 40
    graphed = hf_llama.generate_graphed(model, ids, steps, kv_format=fmt)[0].tolist()
    dynamic, _ = greedy(model, ids, steps, hf_llama.QuantizedKVCache(model.config, fmt))
    parted = next((i for i, (a, b) in enumerate(zip(dynamic, graphed)) if a != b), None)

    qc = hf_llama.QuantizedKVCache(model.config, fmt)
    sc = hf_llama.StaticKVCache(model.config, 128, fmt)
    with torch.no_grad():
        la = model(ids, past_key_values=qc, use_cache=True).logits[:, -1].float()
        lb = model(ids, past_key_values=sc, use_cache=True).logits[:, -1].float()
    assert torch.equal(la, lb)
    for lq, ls in zip(qc.layers, sc.layers):
        assert torch.equal(bits(lq._k[:, :, :L]), bits(ls.keys[:, :, :L]))
        assert torch.equal(bits(lq._v[:, :, :L]), bits(ls.values[:, :, :L]))
        assert torch.equal(lq._ks[:, :, :L], ls.key_scales[:, :, :L])
        assert torch.equal(lq._vs[:, :, :L], ls.value_scales[:, :, :L])

    # (1) the two kernels over layer 0's identical cache
    lq, ls = qc.layers[0], sc.layers[0]
    kq, vq = lq._views()
    pages = lambda t: t.permute(0, 2, 1)
    g = torch.Generator(device="cuda").manual_seed(3)
    differing, worst, scale = 0, 0.0, 0.0
    for _ in range(20):
        q = torch.randn(1, 8, 64, device="cuda", generator=g).half()
        a = fqkv_decode.decode_attn_gqa_strided(q, kq, vq, 8, kq.fqkv_scales, vq.fqkv_scales)
        b = fqkv_decode.decode_attn_gqa_paged(q, ls.keys.permute(0, 2, 1, 3), ls.values.permute(0, 2, 1, 3),
                                              ls.page_table, ls.seq_lens, ls.keys.shape[2], 8,
                                              pages(ls.key_scales), pages(ls.value_scales))
        d = (a.float() - b.float()).abs()
        differing += int((d > 0).sum())
        worst = max(worst, float(d.max()))
        scale = max(scale, float(a.float().abs().max()))
    assert differing > 0 and worst <= 4e-3 * max(1.0, scale), (differing, worst, scale)

    # (2) and (3): the graphed path's tokens fed to both caches
    first_rank = None
    with torch.no_grad():
        for t in range(steps):
            tok = torch.tensor([[graphed[t]]], device="cuda")
            la = model(tok, past_key_values=qc, use_cache=True).logits[:, -1].float()
            lb = model(tok, past_key_values=sc, position_ids=torch.tensor([[L + t]], device="cuda"),
                       use_cache=True).logits[:, -1].float()
            if first_rank is None and int(la.argmax()) != int(lb.argmax()):
                first_rank = t
            if t == 0:
                for i, (lq, ls) in enumerate(zip(qc.layers, sc.layers)):
                    for cq, cs, sq, ss in ((lq._k, ls.keys, lq._ks, ls.key_scales),
                                           (lq._v, ls.values, lq._vs, ls.value_scales)):
                        x = _signed_codes(cq[:, :, L:L + 1], fmt)
                        y = _signed_codes(cs[:, :, L:L + 1], fmt)
                        su = (sq[:, :, L:L + 1].view(torch.int16).int() - ss[:, :, L:L + 1].view(torch.int16).int()).abs()
                        if i == 0:
                            assert torch.equal(x, y) and int(su.max()) == 0
                        else:
                            assert int((x - y).abs().max()) <= 1 and int(su.max()) <= 1
    if parted is None:
        assert first_rank is None or first_rank == steps - 1
    else:
        assert first_rank == parted - 1, (first_rank, parted)


@pytest.mark.gpu
def test_gpu_bf16_model_decodes_on_the_kernel(monkeypatch):
    """A bf16 model: decode steps read the bf16 cache in place (decode_attn_gqa_strided, no
    conversion of the cache). Attention level: the hook's output on layer 0's bf16 cache equals
    float32 attention over it (max-abs 4e-3 relative to the output scale: the kernel's 2e-3 plus
    the bf16 rounding of the result, 2^-9 relative). Model level: the step's logits match SDPA's to 5 % of the logit
    scale (bf16 SDPA rounds its softmax weights to bf16; the kernel keeps them to 2^-16). Over a
    static cache the graph-replayed tokens equal the eager steps bit for bit, with the paged kernel
    in every layer."""
    import fqkv_decode

    name = hf_llama.register()
    model = tiny_llama(layers=2, dtype=torch.bfloat16, device="cuda")
    ids = torch.randint(0, 1000, (2, 300), generator=torch.Generator().manual_seed(13)).cuda()
    calls = {"strided": 0, "paged": 0}
    real_s, real_p = fqkv_decode.decode_attn_gqa_strided, fqkv_decode.decode_attn_gqa_paged

    def strided(*a, **k):
        assert a[1].dtype == torch.bfloat16
        calls["strided"] += 1
        return real_s(*a, **k)

    def paged(*a, **k):
        assert a[1].dtype == torch.bfloat16
        calls["paged"] += 1
        return real_p(*a, **k)

    monkeypatch.setattr(fqkv_decode, "decode_attn_gqa_strided", strided)
    monkeypatch.setattr(fqkv_decode, "decode_attn_gqa_paged", paged)
    logits = {}
    for impl in ("sdpa", name):
        set_impl(model, impl)
        with torch.no_grad():
            out = model(ids, use_cache=True)
            nxt = out.logits[:, -1:].argmax(-1)
            logits[impl] = model(nxt, past_key_values=out.past_key_values, use_cache=True).logits.float()
    assert calls["strided"] == 2
    top = float(logits["sdpa"].abs().max())
    assert float((logits[name] - logits["sdpa"]).abs().max()) <= 0.05 * top

    k, v = out.past_key_values.layers[0].keys, out.past_key_values.layers[0].values  # [2, 2, 301, 64] bf16
    q = torch.randn(2, 8, 1, 64, device="cuda", generator=torch.Generator(device="cuda").manual_seed(2)).bfloat16()
    o, _ = hf_llama.attention_forward(model.model.layers[0].self_attn, q, k, v, None, scaling=1 / 8)
    Kf, Vf = k.float().repeat_interleave(4, 1), v.float().repeat_interleave(4, 1)
    ref = torch.softmax(q.float() @ Kf.transpose(-1, -2).contiguous() / 8, -1) @ Vf
    assert o.dtype == torch.bfloat16
    # bound: the bf16 rounding of the output (2^-9 relative) plus the kernel's own 2e-3
    assert float((o.float().transpose(1, 2) - ref).abs().max()) <= 4e-3 * max(1.0, float(ref.abs().max()))
    eager = hf_llama.generate_graphed(model, ids[:1, :45], 20, use_graph=False)
    n = calls["paged"]
    graphed = hf_llama.generate_graphed(model, ids[:1, :45], 20)
    assert n == 19 * 2 and calls["paged"] - n == 2 * 2
    assert torch.equal(graphed, eager)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_gpu_bf16_model_quantized_cache(fmt):
    """A bf16 model over an int8 / fp8 cache: the layers hand their bf16 keys and values to the
    quantizer as they are (no conversion pass), which quantizes them as their fp32 values, so the
    cache holds fqkv_decode.quant's bytes of x.float(); a decode step then runs on the kernel."""
    name = hf_llama.register()
    model = tiny_llama(layers=2, dtype=torch.bfloat16, device="cuda")
    set_impl(model, name)
    ids = torch.randint(0, 1000, (2, 100), generator=torch.Generator().manual_seed(14)).cuda()
    dyn = transformers.DynamicCache(config=model.config)
    _prefill(model, ids, dyn)
    qc = hf_llama.QuantizedKVCache(model.config, fmt)
    _prefill(model, ids, qc)
    for lq, ld in zip(qc.layers, dyn.layers):
        for got, gs, x in ((lq._k, lq._ks, ld.keys), (lq._v, lq._vs, ld.values)):
            want, ws = QUANTIZERS[fmt](x.float())
            assert torch.equal(bits(got[:, :, :100]), bits(want)) and torch.equal(gs[:, :, :100], ws)
    with torch.no_grad():
        out = model(ids[:, :1], past_key_values=qc, use_cache=True).logits
    assert out.dtype == torch.bfloat16 and torch.isfinite(out.float()).all()
