"""transformers integration (fftsparse_amd.hf): registration, the prefill /
decode split of the reference's patched forward (eval/LongBench/pred.py:216-250),
and a small Llama prefill end to end on the GPU."""
from __future__ import annotations

import pytest
import torch

transformers = pytest.importorskip("transformers")
from transformers import LlamaConfig, LlamaForCausalLM  # noqa: E402
from transformers.integrations.sdpa_attention import sdpa_attention_forward  # noqa: E402

import fftsparse_amd.hf as fh  # noqa: E402
from fftsparse_amd import myattn_prefill  # noqa: E402


def _tiny(layers=2, heads=4, kv=2, hidden=512, vocab=1000):
    cfg = LlamaConfig(hidden_size=hidden, intermediate_size=2 * hidden, num_hidden_layers=layers,
                      num_attention_heads=heads, num_key_value_heads=kv, head_dim=128, vocab_size=vocab,
                      max_position_embeddings=8192)
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg)


def test_register_sets_implementation_and_settings():
    m = _tiny()
    fh.patch_model(m, corr_threshold=0.95)
    assert m.config._attn_implementation == fh.NAME
    assert m.model.layers[1].self_attn.config._attn_implementation == fh.NAME
    assert fh._state["kwargs"]["corr_threshold"] == 0.95
    assert fh._state["kwargs"]["sink_ratio"] == fh.PRODUCTION_KWARGS["sink_ratio"]
    fh.register()                                   # back to the production settings
    assert fh._state["kwargs"] == fh.PRODUCTION_KWARGS


def test_decode_step_takes_sdpa():
    """L_q != L_k (a decoding step against the cache) keeps the model's dense attention."""
    m = _tiny()
    mod = m.model.layers[0].self_attn
    g = torch.Generator().manual_seed(1)
    q = torch.randn(1, 4, 1, 128, generator=g)
    k = torch.randn(1, 2, 77, 128, generator=g)
    v = torch.randn(1, 2, 77, 128, generator=g)
    o, w = fh.fftsparse_attention(mod, q, k, v, None, scaling=128 ** -0.5)
    r, _ = sdpa_attention_forward(mod, q, k, v, None, scaling=128 ** -0.5)
    assert w is None and o.shape == (1, 1, 4, 128)
    assert torch.equal(o, r)


def test_prefill_on_cpu_raises_like_the_reference():
    m = _tiny()
    fh.patch_model(m)
    with pytest.raises(AssertionError):
        m(torch.randint(0, 1000, (1, 64)))


def test_fused_forward_on_cpu_keeps_reference_errors():
    """The fused forward falls back to the model's RoPE and the registered
    attention off the GPU, which raises like the reference (my_attn_v7.py:502);
    patch_model without fused_rope restores the class forward."""
    m = _tiny()
    fh.patch_model(m, fused_rope=True)
    assert "forward" in vars(m.model.layers[0].self_attn)
    with pytest.raises(AssertionError):
        m(torch.randint(0, 1000, (1, 64)))
    fh.patch_model(m)
    assert "forward" not in vars(m.model.layers[0].self_attn)


def test_fused_forward_follows_another_implementation():
    """With the model switched to another attention implementation, the
    patched forward is the model's own: identical logits on the CPU."""
    m = _tiny().eval()
    ids = torch.randint(0, 1000, (1, 64), generator=torch.Generator().manual_seed(5))
    m.set_attn_implementation("sdpa")
    with torch.no_grad():
        ref = m(input_ids=ids).logits
    fh.patch_model(m, fused_rope=True)
    m.set_attn_implementation("sdpa")
    with torch.no_grad():
        out = m(input_ids=ids).logits
    fh.patch_model(m)
    assert torch.equal(out, ref)


@pytest.mark.gpu
def test_prefill_rejects_batches_and_masks():
    dev = torch.device("cuda:0")
    mod = _tiny().model.layers[0].self_attn
    q = torch.zeros(2, 4, 2048, 128, device=dev, dtype=torch.bfloat16)
    k = torch.zeros(2, 2, 2048, 128, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="batch 1"):
        fh.fftsparse_attention(mod, q, k, k, None)
    mask = torch.zeros(1, 1, 2048, 2048, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="causal only"):
        fh.fftsparse_attention(mod, q[:1], k[:1], k[:1], mask)


@pytest.mark.gpu
def test_prefill_equals_myattn_prefill():
    """The registered prefill is myattn_prefill's path: identical output."""
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(2)
    L = 4096
    q = torch.randn(1, 8, L, 128, generator=g).to(dev, torch.bfloat16)
    k = torch.randn(1, 2, L, 128, generator=g).to(dev, torch.bfloat16)
    v = torch.randn(1, 2, L, 128, generator=g).to(dev, torch.bfloat16)
    print(f"[case] hf prefill L={L} 8/2 heads", flush=True)
    fh.register()
    mod = _tiny(heads=8, kv=2, hidden=1024).model.layers[0].self_attn
    o, _ = fh.fftsparse_attention(mod, q, k, v, None, scaling=128 ** -0.5)
    kw = {k_: v_ for k_, v_ in fh.PRODUCTION_KWARGS.items()}
    ref = myattn_prefill(q, k, v, 0, **kw)
    assert o.shape == (1, L, 8, 128)
    assert torch.equal(o.reshape(1, L, -1), ref)


@pytest.mark.gpu
def test_small_llama_prefill_runs():
    """A 2-layer Llama prefill of 4096 tokens with the registered attention:
    every layer takes the sparse path, the logits are finite, and a decoding
    step after it (dense, against the cache) runs."""
    dev = torch.device("cuda:0")
    m = _tiny(heads=8, kv=2, hidden=1024).to(dev, torch.bfloat16).eval()
    fh.patch_model(m)
    ids = torch.randint(0, 1000, (1, 4096), generator=torch.Generator().manual_seed(3)).to(dev)
    print("[case] hf small llama prefill 4096", flush=True)
    fh.record_prefill_events(True)
    with torch.no_grad():
        out = m(input_ids=ids, use_cache=True)
        nxt = m(input_ids=ids[:, -1:], past_key_values=out.past_key_values, use_cache=True)
    torch.cuda.synchronize()
    ev = fh.prefill_events()
    fh.record_prefill_events(False)
    assert [e.layer_idx for e in ev] == [0, 1]       # one prefill call per layer, none for the decode step
    assert all(0.0 < e.density() <= 1.0 and e.ms() > 0.0 for e in ev)
    assert torch.isfinite(out.logits.float()).all()
    assert torch.isfinite(nxt.logits.float()).all()


@pytest.mark.gpu
def test_fused_rope_forward_equals_unfused():
    """patch_model(fused_rope=True): the prefill (RoPE and block pooling in one
    pass) gives the logits of the registered attention on the model's own RoPE
    bit for bit, fills the cache with the same rotated keys, and a decoding
    step after it matches too; patching back restores the class forward."""
    dev = torch.device("cuda:0")
    m = _tiny(heads=8, kv=2, hidden=1024).to(dev, torch.bfloat16).eval()
    ids = torch.randint(0, 1000, (1, 4096), generator=torch.Generator().manual_seed(4)).to(dev)
    print("[case] hf fused rope prefill 4096", flush=True)
    outs = []
    for fused in (False, True):
        fh.patch_model(m, fused_rope=fused)
        assert ("forward" in vars(m.model.layers[0].self_attn)) == fused
        with torch.no_grad():
            out = m(input_ids=ids, use_cache=True)
            nxt = m(input_ids=ids[:, -1:], past_key_values=out.past_key_values, use_cache=True)
        outs.append((out, nxt))
    torch.cuda.synchronize()
    (a, an), (b, bn) = outs
    assert torch.equal(a.logits, b.logits)
    assert torch.equal(an.logits, bn.logits)
    for la, lb in zip(a.past_key_values.layers, b.past_key_values.layers):
        assert torch.equal(la.keys, lb.keys) and torch.equal(la.values, lb.values)
    fh.patch_model(m)
    assert "forward" not in vars(m.model.layers[0].self_attn)
