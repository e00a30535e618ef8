"""FlexPrefill's block selection on the gfx950 kernels, attending through the
same block-sparse kernel as the FFT selector.

Mirrors attn_src/Flexprefill.py: ``get_active_blocks`` (:946-1061) and
``Flexprefill_prefill`` (:1063-1098).  One C call (fs_flex) forms the
last-block attention profile, the budgets, the JS-divergence test, the
vertical / slash choice and the sparse heads' block cover, and emits per-row
block masks.  Inputs use the reference's layout, [B, L, H, D].
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import FlexArgs
from .attn import block_sparse_attention, mask_from_bits, mask_words


@dataclass
class FlexSelection:
    """Device-resident result of the FlexPrefill selection."""
    blk_cnt: torch.Tensor       # int32 [Hq, N]
    blk_bits: torch.Tensor      # int64 [Hq, N, ceil(N/64)]: the block mask (bit j % 64 of word j / 64)
    head_info: torch.Tensor     # int32 [Hq, 4]: vertical budget, slash budget, sparse head, 0
    js: torch.Tensor            # float32 [Hq]
    vertical: torch.Tensor      # float32 [Hq, L]: mean last-block attention per key
    slash: torch.Tensor         # float32 [Hq, L]: per diagonal ending at each key, / bs
    block_size: int

    def dense_mask(self) -> torch.Tensor:
        """[Hq, N, N] bool block mask."""
        return mask_from_bits(self.blk_bits, self.blk_cnt.shape[1])

    def nnz(self) -> int:
        return int(self.blk_cnt.sum().item())


def budgets(L: int, block_size: int, min_budget=None, max_budget=None):
    """Flexprefill.py:1080-1096 and :958: token budgets to blocks, the maximum
    clamped to the block count."""
    nb = -(-L // block_size)
    mn = 1 if min_budget is None else min_budget
    mx = 2147483647 if max_budget is None else max_budget
    return math.ceil(mn / block_size), min(math.ceil(mx / block_size), nb)


def flex_select(q: torch.Tensor, k: torch.Tensor, *, gamma: float = 0.9, tau: float = 0.0, min_budget=None,
                max_budget=None, gqa_interleave: bool = False, block_size: int = 32) -> FlexSelection:
    """get_active_blocks (Flexprefill.py:946-1061) as a block mask.  q [1, L, Hq, D],
    k [1, L, Hk, D] on the GPU (bf16/f16, D = 128), the reference's layout."""
    assert q.shape[1] == k.shape[1]                                   # Flexprefill.py:1077
    B, L, Hq, D = q.shape
    Hk = k.shape[2]
    assert D in {16, 32, 64, 128}                                     # :1078
    assert block_size in {16, 32, 64, 128}                            # :1079
    if B != 1:
        raise ValueError("the FlexPrefill selector takes batch 1")
    if Hq % Hk:
        raise ValueError(f"query heads {Hq} must be a multiple of key heads {Hk}")
    if q.dtype != k.dtype or q.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"unsupported dtypes {q.dtype}, {k.dtype} (bf16/f16)")
    if k.shape[0] != B or k.shape[3] != D:
        raise ValueError(f"query {tuple(q.shape)} and key {tuple(k.shape)} shapes do not match")
    dev = _lib.same_device(q, k)
    qv = q.transpose(1, 2)                                            # [1, Hq, L, D] views
    kv = k.transpose(1, 2)
    if qv.stride(3) != 1 or qv.stride(2) % 8 or qv.stride(1) % 8 or qv.data_ptr() % 16:
        qv = qv.contiguous()
    if kv.stride(3) != 1 or kv.stride(2) % 8 or kv.stride(1) % 8 or kv.data_ptr() % 16:
        kv = kv.contiguous()
    nb = -(-L // block_size)
    mnb, mxb = budgets(L, block_size, min_budget, max_budget)
    sel = FlexSelection(blk_cnt=torch.empty(Hq, nb, dtype=torch.int32, device=dev),
                        blk_bits=torch.empty(Hq, nb, mask_words(nb), dtype=torch.int64, device=dev),
                        head_info=torch.empty(Hq, 4, dtype=torch.int32, device=dev),
                        js=torch.empty(Hq, dtype=torch.float32, device=dev),
                        vertical=torch.empty(Hq, L, dtype=torch.float32, device=dev),
                        slash=torch.empty(Hq, L, dtype=torch.float32, device=dev),
                        block_size=block_size)
    lib = _lib.load()
    work = torch.empty(max(1, lib.fs_flex_work_bytes(Hq, Hk, L, block_size, float(tau))), dtype=torch.uint8, device=dev)
    _lib.call("fs_flex", FlexArgs(
        q=qv.data_ptr(), q_sh=qv.stride(1), q_sl=qv.stride(2), k=kv.data_ptr(), k_sh=kv.stride(1),
        k_sl=kv.stride(2), dtype=_lib.FS_DTYPE[q.dtype], Hq=Hq, Hk=Hk, L=L, D=D, bs=block_size,
        gamma=float(gamma), tau=float(tau), min_blocks=mnb, max_blocks=mxb, gqa_interleave=int(bool(gqa_interleave)),
        blk_cnt=sel.blk_cnt.data_ptr(), blk_bits=sel.blk_bits.data_ptr(), head_info=sel.head_info.data_ptr(),
        head_js=sel.js.data_ptr(), vertical=sel.vertical.data_ptr(), slash=sel.slash.data_ptr(),
        work=work.data_ptr()), dev)
    sel._keep = (qv, kv, work)
    return sel


def Flexprefill_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gamma: float = 0.9, tau: float = 0,
                        min_budget: int = None, max_budget: int = None, gqa_interleave: bool = False,
                        softmax_scale=None, block_size: int = 32):
    """Flexprefill.py:1063-1098: q/k/v [B, L, H, D] -> [B, L, H, D].  Sequences
    of at most max(2 bs, ceil(min_budget / bs) bs) tokens take dense causal
    attention (:1084-1085), the others the FlexPrefill selection and the
    block-sparse attention, at 16-, 32-, 64- or 128-token blocks (at most 8192
    blocks: 131072 tokens at 16, 262144 at 32).  With ``gqa_interleave``
    query head h reads KV head h % Hk in the selection and the sparse attention
    (the dense branch keeps flash_attn_func's grouped heads, as the reference)."""
    assert q.is_cuda, "input tensors must be on the GPU"
    B, L, H, D = q.shape
    assert q.shape[1] == k.shape[1]
    assert D in {16, 32, 64, 128}
    assert block_size in {16, 32, 64, 128}
    mn = 1 if min_budget is None else min_budget
    qv, kv, vv = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    if L <= max(2 * block_size, math.ceil(mn / block_size) * block_size):
        return block_sparse_attention(qv, kv, vv, block_size=128, is_causal=True, softmax_scale=softmax_scale)
    sel = flex_select(q, k, gamma=gamma, tau=tau, min_budget=min_budget, max_budget=max_budget,
                      gqa_interleave=gqa_interleave, block_size=block_size)
    return block_sparse_attention(qv, kv, vv, sel.blk_cnt, sel.blk_bits, block_size=block_size, is_causal=True,
                                  softmax_scale=softmax_scale, gqa_interleave=gqa_interleave)


def density(sel: FlexSelection) -> float:
    H, N = sel.blk_cnt.shape
    return sel.nnz() / (H * N * (N + 1) / 2)


__all__ = ["FlexSelection", "flex_select", "Flexprefill_prefill", "budgets", "density"]
