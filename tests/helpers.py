"""Shared test utilities: production kwargs, parity bookkeeping."""
from __future__ import annotations

import torch

# eval/efficiency/1_run_eval_multilayer.sh:46-62,72 with T = 0.9
PROD = dict(block_size=128, sink_ratio=0.01, recent_ratio=0.0, local_span_ratio=0.02,
            corr_threshold=0.9, column_topk_ratio=0.2, qk_topk_ratio=0.3, stripe_threshold=0.3,
            diag_sample_ratio=0.15, min_diag_samples=5, max_diag_samples=64)

BAND = 1e-3           # relative band around a selection threshold
MATCH_MIN = 0.999     # exact + excused decisions / all causal decisions


def block_match(gpu_mask: torch.Tensor, ref_mask: torch.Tensor, excusable: torch.Tensor, causal=True):
    """Returns (fraction exact-or-excused, fraction exact, #unexcused) over the
    causal (h, i, j) decisions."""
    g = gpu_mask.cpu()
    r = ref_mask.cpu()
    e = excusable.cpu()
    H, N, Nk = r.shape
    dom = torch.ones(N, Nk, dtype=torch.bool)
    if causal:
        dom = torch.arange(N)[:, None] >= torch.arange(Nk)[None, :]
    dom = dom.unsqueeze(0).expand(H, N, Nk)
    total = int(dom.sum())
    diff = (g != r) & dom
    exact = total - int(diff.sum())
    unexc = int((diff & ~e).sum())
    return (total - unexc) / total, exact / total, unexc


def lists_from_mask(mask: torch.Tensor, device):
    """Dense [H,N,Nk] bool mask -> (blk_cnt int32 [H,N], blk_idx uint16 [H,N,Nk])."""
    H, N, Nk = mask.shape
    cnt = mask.sum(-1).to(torch.int32)
    order = torch.argsort((~mask).to(torch.int8), dim=-1, stable=True)
    idx = order.to(torch.int16).view(torch.uint16).contiguous()
    return cnt.to(device), idx.to(device)


def rope_tables(L, D, theta, dtype):
    """cos / sin [L, D] of the model's rotary embedding (transformers'
    LlamaRotaryEmbedding at positions 0 .. L-1), on the CPU."""
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding
    cfg = LlamaConfig(hidden_size=4 * D, num_attention_heads=4, num_key_value_heads=2, head_dim=D,
                      rope_theta=theta, max_position_embeddings=max(L, 2048))
    x = torch.zeros(1, dtype=dtype)
    cos, sin = LlamaRotaryEmbedding(cfg)(x, torch.arange(L)[None])
    return cos[0], sin[0]
