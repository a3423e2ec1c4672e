"""The transformers integration (fqkv_decode.hf_llama), the reference's HF hook
(nb:1037-1064) on a random-init Llama (no checkpoint download):

* CPU: registration, the kernel/SDPA routing rule, and a whole generate() on
  CPU tensors, which must route every call to SDPA and match it exactly;
* GPU: decode steps through the kernel against SDPA (logits within fp16
  noise) and greedy generation token-for-token equal to SDPA's (a divergence
  is accepted only where SDPA's own top-2 logit margin is below 1e-2, i.e. at
  a numerical tie), at short and long context (the latter takes the
  kernel's internal sequence split)."""

import math

import pytest
import torch

transformers = pytest.importorskip("transformers")

from fqkv_decode import hf_llama  # noqa: E402


def tiny_llama(layers=4, hidden=512, heads=8, kv_heads=2, head_dim=64, vocab=1000, init=0.2, dtype=torch.float32,
               device="cpu"):
    cfg = transformers.LlamaConfig(vocab_size=vocab, hidden_size=hidden, intermediate_size=2 * hidden,
                                   num_hidden_layers=layers, num_attention_heads=heads,
                                   num_key_value_heads=kv_heads, head_dim=head_dim,
                                   max_position_embeddings=8192, initializer_range=init,
                                   attn_implementation="sdpa")
    torch.manual_seed(0)
    with torch.device(device):
        model = transformers.LlamaForCausalLM(cfg)
    return model.to(dtype).eval()


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


def greedy(model, ids, steps):
    """Greedy decode by hand; returns tokens and each step's top-2 logit margin."""
    toks, margins = [], []
    with torch.no_grad():
        out = model(ids, use_cache=True)
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


@pytest.mark.gpu
@pytest.mark.parametrize("ctx", [37, 3000])
def test_gpu_decode_matches_sdpa(ctx):
    name = hf_llama.register()
    model = tiny_llama(dtype=torch.float16, device="cuda")
    ids = torch.randint(0, 1000, (1, ctx), generator=torch.Generator().manual_seed(2)).cuda()
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
