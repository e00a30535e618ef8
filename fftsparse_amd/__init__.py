"""fftsparse_amd -- MI355X-native FFTSparse prefill (FFT-guided block selection
+ block-sparse causal GQA attention) on hand-written gfx950 HIP kernels.

Public API (drop-in for attn_src/fft_attn/my_attn_v7.py and
attn_src/fix_mask_attn/my_attn.py):

    myattn_prefill(q, k, v, layer_idx, ...)        v7 selection + sparse attention
    fix_mask.myattn_prefill(q, k, v, layer_idx, ...) fixed sink/recent/local mask
    select_blocks(q, k, ...)                        stage 1 only (the block mask)
    block_sparse_attention(q, k, v, cnt, bits, ...) stage 2 only (or block_mask=: base_blockmask)
    rope_pool(q, k, cos, sin, ...)                  the rotary embedding before the call, fused
                                                    with the block pooling (select_blocks(pooled=...))

The reference's comparison selectors on the same attention kernel:

    xattn.Xattention_prefill(q, k, v, ...)          attn_src/xattn/src/Xattention.py
    flex.Flexprefill_prefill(q, k, v, ...)          attn_src/Flexprefill.py
"""
from .attn import (AttentionCall, BlockSelection, block_sparse_attention, myattn_prefill, rope_pool,  # noqa: F401
                   select_blocks)
from . import fix_mask, flex, xattn  # noqa: F401

__all__ = ["myattn_prefill", "select_blocks", "block_sparse_attention", "rope_pool", "AttentionCall",
           "BlockSelection", "fix_mask", "flex", "xattn"]
