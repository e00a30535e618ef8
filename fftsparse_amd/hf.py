"""Hugging Face transformers integration of the FFTSparse prefill.

The reference patches ``LlamaAttention.forward`` for its evaluations
(eval/LongBench/pred.py:160-250, installed at :655-661): the prefill (key
length equal to query length) calls ``myattn_prefill`` on the RoPE'd,
``repeat_kv``-expanded states, and every other call (decoding against the KV
cache) keeps the model's dense attention.  transformers 5.x routes each
attention call through a registry (``AttentionInterface``;
models/llama/modeling_llama.py ``LlamaAttention.forward`` calls the registered
function with q [B, Hq, L_q, D], k/v [B, Hkv, L_k, D], the mask, ``scaling``
and ``dropout`` and expects ``([B, L_q, Hq, D], None)``), so the same split is
one registered function::

    import fftsparse_amd.hf as fh
    fh.register()                                   # name "fftsparse", production settings
    model = AutoModelForCausalLM.from_pretrained(path, attn_implementation="fftsparse")
    # or, on a model already loaded:
    fh.patch_model(model)

K/V arrive with their native KV-head count; the kernels read them as they
are, so the reference's ``repeat_kv`` copies are not made.

``patch_model(model, fused_rope=True)`` also replaces the forward of each
Llama-family attention module, as the reference does (pred.py:160-250): a
fresh batch-1 prefill applies the rotary embedding and forms the block means
of the rotated Q/K in one pass (``rope_pool``), so the selection does not
re-read Q and K; every other call runs the model's own RoPE and the
registered attention.
"""
from __future__ import annotations

import types
from typing import NamedTuple

import torch

from .attn import _MIN_BLOCKS, rope_pool, v7_prefill

NAME = "fftsparse"

# The selection settings of the reference's efficiency runs
# (eval/efficiency/1_run_eval_multilayer.sh:46-62,72) with threshold 0.9.
PRODUCTION_KWARGS = dict(block_size=128, sink_ratio=0.01, recent_ratio=0.0, local_span_ratio=0.02,
                         corr_threshold=0.9, column_topk_ratio=0.2, qk_topk_ratio=0.3, stripe_threshold=0.3,
                         diag_sample_ratio=0.15, min_diag_samples=5, max_diag_samples=64)

_state = {"kwargs": dict(PRODUCTION_KWARGS), "events": None, "name": NAME}


def fftsparse_attention(module, query, key, value, attention_mask, dropout=0.0, scaling=None, **kwargs):
    """The registered attention function.

    Prefill (L_q == L_k): v7 block selection and block-sparse attention on the
    GPU kernels (``myattn_prefill``'s path, with the model's ``scaling``).
    Any other call (a decoding step against the cache): the model's SDPA
    attention, as in the reference, which patches only the prefill."""
    if query.shape[2] != key.shape[2]:
        from transformers.integrations.sdpa_attention import sdpa_attention_forward
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout, scaling=scaling,
                                      **kwargs)
    assert query.is_cuda, "input tensors must be on the GPU"          # my_attn_v7.py:502
    if query.shape[0] != 1:
        raise ValueError("the FFTSparse prefill takes batch 1 (my_attn_v7.py:521)")
    if attention_mask is not None:
        raise ValueError("the FFTSparse prefill is causal only: padding or custom masks are not supported")
    if dropout:
        raise ValueError("the FFTSparse prefill has no dropout")
    kw = _state["kwargs"]
    if _state["events"] is None:
        return v7_prefill(query, key, value, softmax_scale=scaling, **kw), None   # [1, L, Hq, D]
    e0 = _event()
    out, sel = v7_prefill(query, key, value, softmax_scale=scaling, return_selection=True, **kw)
    _record(module, e0, sel, query.shape[1], query.shape[2])
    return out, None


def _event():
    e = torch.cuda.Event(enable_timing=True)
    e.record()
    return e


def _record(module, e0, sel, Hq, L):
    """Closes a prefill event: its time, and the selected tiles (a device
    scalar, read after the run) over the causal tiles."""
    e1 = _event()
    nnz = sel.blk_cnt.sum() if sel is not None else None
    nq = -(-L // _state["kwargs"].get("block_size", 128))
    _state["events"].append(PrefillEvent(getattr(module, "layer_idx", None), e0, e1, nnz, Hq * nq * (nq + 1) // 2))


# attention classes whose forward is q/k/v projections, RoPE, cache update,
# attention, o_proj (models/llama/modeling_llama.py LlamaAttention.forward)
_FUSABLE = ("LlamaAttention", "MistralAttention", "Qwen2Attention")


def fused_attention_forward(self, hidden_states, position_embeddings=None, attention_mask=None,
                            past_key_values=None, **kwargs):
    """LlamaAttention.forward with the FFTSparse prefill (the reference's
    patched forward, eval/LongBench/pred.py:160-250).  A fresh batch-1 causal
    prefill of at least 10 blocks runs ``rope_pool`` (the rotary embedding of
    pred.py:195 and the selection's block pooling in one pass), stores the
    rotated K and V in the cache, and runs the v7 selection on those block
    means and the block-sparse attention.  Any other call (decode, a chunk
    after cached tokens, masks, training) applies the model's RoPE and the
    registered attention, exactly as the unpatched forward does."""
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    bsz, q_len = hidden_states.shape[:2]
    shape = (bsz, q_len, -1, self.head_dim)
    q = self.q_proj(hidden_states).view(shape).transpose(1, 2)
    k = self.k_proj(hidden_states).view(shape).transpose(1, 2)
    v = self.v_proj(hidden_states).view(shape).transpose(1, 2)
    cos, sin = position_embeddings
    kw = _state["kwargs"]
    bs = kw.get("block_size", 128)
    fresh = past_key_values is None or past_key_values.get_seq_length(self.layer_idx) == 0
    ours = self.config._attn_implementation == _state["name"]
    if (ours and q.is_cuda and bsz == 1 and attention_mask is None and fresh and not self.training
            and q_len >= bs * _MIN_BLOCKS and q.dtype in (torch.bfloat16, torch.float16)):
        e0 = _event() if _state["events"] is not None else None
        q, k, q_b, k_b = rope_pool(q, k, cos, sin, block_size=bs)
        if past_key_values is not None:
            # transformers 5.x's LlamaAttention.forward passes no cache kwargs either
            k, v = past_key_values.update(k, v, self.layer_idx)
        if k.shape[2] == q_len:
            out, sel = v7_prefill(q, k, v, softmax_scale=self.scaling, return_selection=True, pooled=(q_b, k_b),
                                  **kw)
            if e0 is not None:
                _record(self, e0, sel, q.shape[1], q_len)
        else:
            # a cache that hands back more keys than this prefill wrote (a
            # preallocated static cache): the registered attention's path for
            # L_q != L_k, as the unpatched forward would take
            out, _ = fftsparse_attention(self, q, k, v, attention_mask, dropout=0.0, scaling=self.scaling, **kwargs)
    else:
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        if past_key_values is not None:
            k, v = past_key_values.update(k, v, self.layer_idx)
        if ours:
            out, _ = fftsparse_attention(self, q, k, v, attention_mask, dropout=0.0, scaling=self.scaling, **kwargs)
        else:
            from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
            from transformers.models.llama.modeling_llama import eager_attention_forward
            fn = ALL_ATTENTION_FUNCTIONS.get_interface(self.config._attn_implementation, eager_attention_forward)
            out, _ = fn(self, q, k, v, attention_mask, dropout=0.0 if not self.training else self.attention_dropout,
                        scaling=self.scaling, **kwargs)
    out = out.reshape(bsz, q_len, -1).contiguous()
    return self.o_proj(out), None


def register(name: str = NAME, **overrides) -> str:
    """Registers the attention function (and SDPA's mask builder, which
    leaves a plain causal prefill unmasked) under ``name``.  ``overrides``
    replace entries of ``PRODUCTION_KWARGS`` (any ``select_blocks`` keyword,
    plus ``block_size``).  Returns the name to pass as ``attn_implementation``."""
    from transformers import AttentionInterface
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, AttentionMaskInterface

    _state["kwargs"] = {**PRODUCTION_KWARGS, **overrides}
    _state["name"] = name
    AttentionInterface.register(name, fftsparse_attention)
    AttentionMaskInterface.register(name, ALL_MASK_ATTENTION_FUNCTIONS["sdpa"])
    return name


def patch_model(model, name: str = NAME, fused_rope: bool = False, **overrides):
    """Switches a loaded model to the FFTSparse prefill (the counterpart of the
    reference's forward replacement, pred.py:655-661) and returns it.  With
    ``fused_rope`` the Llama-family attention modules also take
    ``fused_attention_forward``; without it any such replacement is undone."""
    register(name, **overrides)
    model.set_attn_implementation(name)
    for m in model.modules():
        if type(m).__name__ not in _FUSABLE:
            continue
        if fused_rope:
            m.forward = types.MethodType(fused_attention_forward, m)
        elif "forward" in vars(m):
            del m.forward                           # back to the class's forward
    return model


class PrefillEvent(NamedTuple):
    layer_idx: int | None
    start: torch.cuda.Event
    end: torch.cuda.Event
    selected_tiles: torch.Tensor | None      # device scalar; None on the dense short-sequence path
    causal_tiles: int

    def ms(self) -> float:
        return self.start.elapsed_time(self.end)

    def density(self) -> float:
        return float(self.selected_tiles) / self.causal_tiles if self.selected_tiles is not None else 1.0


def record_prefill_events(enabled: bool = True):
    """Starts (or stops) recording every prefill call: a CUDA event pair around
    it and its selected tile count; ``prefill_events()`` returns them."""
    _state["events"] = [] if enabled else None


def prefill_events() -> list[PrefillEvent]:
    return list(_state["events"] or [])
