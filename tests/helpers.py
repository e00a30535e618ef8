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


def mask_bits(mask: torch.Tensor, device):
    """Dense [H,N,Nk] bool mask -> (blk_cnt int32 [H,N], blk_bits int64 [H,N,ceil(Nk/64)]) on device."""
    from fftsparse_amd.attn import bits_from_mask
    cnt, bits = bits_from_mask(mask)
    return cnt.to(device), bits.to(device)


def check_mask_rows(mask: torch.Tensor, rows):
    """Rows i of a [H, N, Nk] bool block mask are causal (no block past i) and
    hold block 0 and the diagonal block i."""
    for i in rows:
        r = mask[:, i]
        assert not r[:, i + 1:].any(), f"row {i}: blocks past the diagonal"
        assert r[:, 0].all() and r[:, i].all(), f"row {i}: sink or diagonal block missing"


def check_mask_words(blk_bits: torch.Tensor, blk_cnt: torch.Tensor, nk: int):
    """Every row of a block mask (words [H, N, W], on any device): its count
    is its popcount, it is causal, and it holds block 0 and the diagonal block.
    One head at a time ([N, Nk] bools)."""
    from fftsparse_amd.attn import mask_from_bits
    H, N, _ = blk_bits.shape
    pos = torch.arange(N, device=blk_bits.device)
    above = torch.arange(nk, device=blk_bits.device)[None, :] > pos[:, None]
    for h in range(H):
        m = mask_from_bits(blk_bits[h:h + 1], nk)[0]
        assert torch.equal(m.sum(-1, dtype=torch.int32), blk_cnt[h]), f"head {h}: counts"
        assert not bool((m & above).any()), f"head {h}: blocks past the diagonal"
        assert bool(m[:, 0].all()) and bool(m[pos, pos.clamp(max=nk - 1)].all()), f"head {h}: sink / diagonal"
        del m


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
