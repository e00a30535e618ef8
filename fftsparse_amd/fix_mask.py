"""Fixed-mask block-sparse prefill (the fix_mask_attn role).

Mirrors ``attn_src/fix_mask_attn/my_attn.py:82-246``: the block mask is the
deterministic sink | recent | local-window pattern (my_attn.py:39-79, with no
causal AND -- the causal kernel never visits blocks above the diagonal) and is
handed to the same block-sparse attention kernel as the v7 path.
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import SelectArgs
from .attn import BlockSelection, _check_layout, block_sparse_attention, mask_words
from .params import PrefillParams


def fixed_block_mask(L_q: int, L_k: int, H: int, device, *, block_size=128, sink_ratio=0.1,
                     recent_ratio=0.1, local_span_ratio=0.1) -> BlockSelection:
    """The block mask of create_deterministic_block_mask (my_attn.py:39-79)
    with the parameters derived at my_attn.py:133-144."""
    N = (L_q + block_size - 1) // block_size
    Nk = (L_k + block_size - 1) // block_size
    keep_sink = max(1, int(Nk * sink_ratio))
    keep_recent = max(1, int(Nk * recent_ratio))
    lw = max(2, int(Nk * local_span_ratio)) // 2
    p = PrefillParams(L_q, L_k, block_size, N, Nk, keep_sink, keep_recent, lw,
                      corr_enabled=False, remote_start=lw + 1)
    sel = BlockSelection(params=p,
                         blk_cnt=torch.empty(H, N, dtype=torch.int32, device=device),
                         blk_bits=torch.empty(H, N, mask_words(Nk), dtype=torch.int64, device=device))
    _lib.call("fs_select", SelectArgs(dtype=0, Hq=H, Hk=1, N=N, Nk=Nk, D=0, mask_causal=0,
                                      keep_sink=keep_sink, keep_recent=keep_recent, local_window=lw,
                                      remote_start=lw + 1, dyn_mode=0, col_mode=0,
                                      blk_cnt=sel.blk_cnt.data_ptr(), blk_bits=sel.blk_bits.data_ptr()),
              sel.blk_cnt.device)
    return sel


def myattn_prefill(
        query_states,
        key_states,
        value_states,
        layer_idx,
        block_size=128,
        is_causal=True,
        is_visual=True,
        sink_ratio=0.1,
        recent_ratio=0.1,
        local_span_ratio=0.1,
):
    """my_attn.py:82-246: [1,H,L_q,D] inputs -> [1, L_q, H*D].  ``is_visual``
    (mask plotting) is accepted and ignored."""
    assert query_states.is_cuda, "input tensors must be on the GPU"   # my_attn.py:99
    q = _check_layout(query_states)
    H, L_q, D = q.shape[1], q.shape[2], q.shape[3]
    L_k = key_states.shape[2]
    sel = fixed_block_mask(L_q, L_k, H, q.device, block_size=block_size, sink_ratio=sink_ratio,
                            recent_ratio=recent_ratio, local_span_ratio=local_span_ratio)
    o = block_sparse_attention(q, key_states, value_states, sel.blk_cnt, sel.blk_bits,
                               block_size=block_size, is_causal=is_causal)
    return o.reshape(1, L_q, H * D)
