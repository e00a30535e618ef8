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
"""
from __future__ import annotations

from typing import NamedTuple

import torch

from .attn import v7_prefill

NAME = "fftsparse"

# The selection settings of the reference's efficiency runs
# (eval/efficiency/1_run_eval_multilayer.sh:46-62,72) with threshold 0.9.
PRODUCTION_KWARGS = dict(block_size=128, sink_ratio=0.01, recent_ratio=0.0, local_span_ratio=0.02,
                         corr_threshold=0.9, column_topk_ratio=0.2, qk_topk_ratio=0.3, stripe_threshold=0.3,
                         diag_sample_ratio=0.15, min_diag_samples=5, max_diag_samples=64)

_state = {"kwargs": dict(PRODUCTION_KWARGS), "events": None}


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
    ev = _state["events"]
    if ev is None:
        return v7_prefill(query, key, value, softmax_scale=scaling, **kw), None   # [1, L, Hq, D]
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    out, sel = v7_prefill(query, key, value, softmax_scale=scaling, return_selection=True, **kw)
    e1.record()
    # selected tiles (a device scalar, read after the run) over the causal tiles
    nnz = sel.blk_cnt.sum() if sel is not None else None
    nq = -(-query.shape[2] // kw.get("block_size", 128))
    ev.append(PrefillEvent(getattr(module, "layer_idx", None), e0, e1, nnz, query.shape[1] * nq * (nq + 1) // 2))
    return out, None


def register(name: str = NAME, **overrides) -> str:
    """Registers the attention function (and SDPA's mask builder, which
    leaves a plain causal prefill unmasked) under ``name``.  ``overrides``
    replace entries of ``PRODUCTION_KWARGS`` (any ``select_blocks`` keyword,
    plus ``block_size``).  Returns the name to pass as ``attn_implementation``."""
    from transformers import AttentionInterface
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, AttentionMaskInterface

    _state["kwargs"] = {**PRODUCTION_KWARGS, **overrides}
    AttentionInterface.register(name, fftsparse_attention)
    AttentionMaskInterface.register(name, ALL_MASK_ATTENTION_FUNCTIONS["sdpa"])
    return name


def patch_model(model, name: str = NAME, **overrides):
    """Switches a loaded model to the FFTSparse prefill (the counterpart of the
    reference's forward replacement, pred.py:655-661) and returns it."""
    register(name, **overrides)
    model.set_attn_implementation(name)
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
