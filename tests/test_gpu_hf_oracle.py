"""The transformers integration (fftsparse_amd.hf) checked against the oracle
on the inputs transformers itself hands over: the post-RoPE query as the
projection's strided [1, Hq, L, D] view of [1, L, Hq, D] storage and the K/V
states with their native KV-head count, as LlamaAttention.forward passes them
to the registered attention (the reference's patched forward calls
myattn_prefill on the same RoPE'd states: eval/LongBench/pred.py:177-250).

For each captured call: the block lists against oracle/v7.select_mask (exact
or excused >= 99.9%), and the registered output against fp32 attention
(oracle/v7.block_sparse_attention) on sampled query blocks of every head.
The fused-RoPE forward is checked from the pre-RoPE states: transformers'
apply_rotary_pos_emb gives the reference rotation, the oracle the rest.
The last test takes one layer of BASELINE config 4's 32-layer model at 131072
tokens."""
from __future__ import annotations

import pytest
import torch

transformers = pytest.importorskip("transformers")
from transformers import AttentionInterface, LlamaConfig, LlamaForCausalLM  # noqa: E402
from transformers.models.llama.modeling_llama import apply_rotary_pos_emb  # noqa: E402

import fftsparse_amd.hf as fh  # noqa: E402
from fftsparse_amd import select_blocks  # noqa: E402
from oracle import v7  # noqa: E402
from tests.helpers import MATCH_MIN, block_match  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
PROD = dict(fh.PRODUCTION_KWARGS)


class _Stop(Exception):
    """Ends a forward pass once the layer under test has been captured."""


def _tiny(L, seed=0, head_dim=128):
    cfg = LlamaConfig(hidden_size=8 * head_dim, intermediate_size=2048, num_hidden_layers=2, num_attention_heads=8,
                      num_key_value_heads=2, head_dim=head_dim, vocab_size=1000,
                      max_position_embeddings=max(L, 8192))
    torch.manual_seed(seed)
    return LlamaForCausalLM(cfg).to(DEV, torch.bfloat16).eval()


def _capture_registered(target_layer, stop=False):
    """Re-registers the attention under fh.NAME with a wrapper that records the
    target layer's q/k/v (as passed in) and output."""
    got = {}

    def wrapper(module, query, key, value, attention_mask, **kw):
        out, w = fh.fftsparse_attention(module, query, key, value, attention_mask, **kw)
        if module.layer_idx == target_layer:
            got.update(q=query.detach(), k=key.detach(), v=value.detach(), out=out.detach(),
                       scaling=kw.get("scaling"))
            if stop:
                raise _Stop()
        return out, w

    AttentionInterface.register(fh.NAME, wrapper)
    return got


def _check_against_oracle(q, k, v, out, label, qblocks=None):
    """q [1,Hq,L,D] (any strides), k/v [1,Hk,L,D] on the GPU, out [1,L,Hq,D]."""
    L, Hq, D = q.shape[2], q.shape[1], q.shape[3]
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    ref = v7.select_mask(qc, kc, **PROD)
    sel = select_blocks(q, k, **PROD)
    got = sel.dense_mask().cpu()
    frac, exact, unexc = block_match(got, ref.mask, ref.excusable)
    N = ref.params.N
    print(f"  {label}: selection match={frac:.6f} exact={exact:.6f} unexcused={unexc}", flush=True)
    assert frac >= MATCH_MIN
    qblocks = qblocks or sorted({0, 1, N // 2, N - 2, N - 1})
    rows = torch.cat([torch.arange(i * 128, min(L, (i + 1) * 128)) for i in qblocks])
    o = out[0].float().cpu()[rows]
    masks = [("its own lists", got)] + ([("the oracle mask", ref.mask)] if exact == 1.0 else [])
    for name, m in masks:
        want = v7.block_sparse_attention(qc, kc, vc, m, 128, qblocks=qblocks)[rows]
        err = (o - want).abs()
        print(f"  {label}: attention under {name}: max_abs={err.max().item():.3e} "
              f"mean_abs={err.mean().item():.3e}", flush=True)
        assert err.max().item() <= 2e-2
        assert err.mean().item() <= 1e-3


@pytest.mark.parametrize("head_dim", [128, 64])
def test_registered_prefill_matches_oracle(head_dim):
    """A 2-layer Llama prefill of 4096 tokens (8 query / 2 KV heads, head dim
    128 or 64): the registered attention of each layer against the oracle."""
    print(f"[case] hf registered prefill vs oracle L=4096 head_dim={head_dim}", flush=True)
    m = _tiny(4096, head_dim=head_dim)
    fh.patch_model(m)
    ids = torch.randint(0, 1000, (1, 4096), generator=torch.Generator().manual_seed(7)).to(DEV)
    try:
        for layer in (0, 1):
            got = _capture_registered(layer)
            with torch.no_grad():
                m(input_ids=ids, use_cache=False)
            q, k, v = got["q"], got["k"], got["v"]
            # the layout transformers passes: the projection's [1, L, H, D] storage seen as [1, H, L, D]
            assert q.stride(1) == head_dim and q.stride(2) == 8 * head_dim and k.shape[1] == 2
            assert got["scaling"] == head_dim ** -0.5
            _check_against_oracle(q, k, v, got["out"], f"layer {layer}")
    finally:
        fh.register()


@pytest.mark.parametrize("head_dim", [128, 64])
def test_fused_rope_prefill_matches_oracle(monkeypatch, head_dim):
    """patch_model(fused_rope=True): the pre-RoPE states go through rope_pool;
    the reference rotation is transformers' apply_rotary_pos_emb of the same
    states, and the layer output is checked against the oracle on it."""
    print(f"[case] hf fused-rope prefill vs oracle L=4096 head_dim={head_dim}", flush=True)
    m = _tiny(4096, seed=1, head_dim=head_dim)
    fh.patch_model(m, fused_rope=True)
    ids = torch.randint(0, 1000, (1, 4096), generator=torch.Generator().manual_seed(8)).to(DEV)
    seen = {}
    rope_pool, v7_prefill = fh.rope_pool, fh.v7_prefill

    def cap_rope(q, k, cos, sin, **kw):
        if "pre" not in seen:
            seen["pre"] = (q.detach().clone(), k.detach().clone(), cos.detach().clone(), sin.detach().clone())
        return rope_pool(q, k, cos, sin, **kw)

    def cap_v7(q, k, v, **kw):
        r = v7_prefill(q, k, v, **kw)
        if "post" not in seen:
            seen["post"] = (q.detach(), k.detach(), v.detach(), r[0].detach())
        return r

    monkeypatch.setattr(fh, "rope_pool", cap_rope)
    monkeypatch.setattr(fh, "v7_prefill", cap_v7)
    try:
        with torch.no_grad():
            m(input_ids=ids, use_cache=False)
    finally:
        fh.patch_model(m)
        fh.register()
    q_pre, k_pre, cos, sin = seen["pre"]
    q_rot, k_rot, v, out = seen["post"]
    ref_q, ref_k = apply_rotary_pos_emb(q_pre, k_pre, cos, sin)
    assert torch.equal(q_rot, ref_q) and torch.equal(k_rot, ref_k)
    _check_against_oracle(ref_q, ref_k, v, out, "layer 0, fused RoPE")


def test_c4_layer_matches_oracle():
    """the 32-layer random-init Llama-3.1-8B-shaped model
    prefilling 131072 random tokens with the FFTSparse prefill registered;
    layer 15's post-RoPE Q and K/V as the model hands them over, its output,
    against the oracle (the forward stops after that layer)."""
    from fftsparse_amd.synth import c4_model_config
    L, layer = 131072, 15
    print(f"[case] c4 layer {layer} vs oracle L={L}", flush=True)
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with DEV:
            model = LlamaForCausalLM(c4_model_config())
    finally:
        torch.set_default_dtype(prev)
    model.eval()
    fh.patch_model(model)
    ids = torch.randint(0, model.config.vocab_size, (1, L), generator=torch.Generator().manual_seed(0)).to(DEV)
    got = _capture_registered(layer, stop=True)
    try:
        with torch.no_grad():
            model(input_ids=ids, use_cache=False, logits_to_keep=1)
    except _Stop:
        pass
    finally:
        fh.register()
    q, k, v, out = got["q"].clone(), got["k"].clone(), got["v"].clone(), got["out"].clone()
    del model, got
    torch.cuda.empty_cache()
    assert q.shape == (1, 32, L, 128) and k.shape == (1, 8, L, 128) and q.stride(2) == 32 * 128
    N = L // 128
    _check_against_oracle(q, k, v, out, f"c4 layer {layer}", qblocks=[0, 1, 300, N // 2, N - 2, N - 1])
