"""XAttention's block selection on the gfx950 kernels, attending through the
same block-sparse kernel as the FFT selector.

Mirrors attn_src/xattn/src/Xattention.py: ``xattn_estimate`` (:14-303) and
``Xattention_prefill`` (:306-406).  Its callers use the Triton path
(use_triton=True: "inverse" reshaping, kdb 1): reshaped antidiagonal scores, an
exp2-domain softmax per reshaped row (causal, or over the whole chunk-padded
sequence), block sums, and find_blocks_chunked's cumulative-mass choice per
block row (attn_src/xattn/src/utils.py:44-200).  use_triton=False selects the
reference's torch path (Xattention.py:72-135, 170-258): the "inverse" (with
kdb), "slash", "random", "double" and "triple" reshapings, its dtype
roundings, and softmax=False.  One C call (fs_xattn) runs all of it and emits
the block mask fs_bsattn reads.

K/V may carry Hq heads (the reference asserts that: its callers pass
repeat_kv'd K/V) or Hkv heads with Hq % Hkv == 0 (native GQA, read as they are).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import XattnArgs
from .attn import _check_layout, block_sparse_attention, mask_from_bits, mask_words


@dataclass
class XSelection:
    """Device-resident result of the XAttention selection."""
    blk_cnt: torch.Tensor       # int32 [Hq, N]
    blk_bits: torch.Tensor      # int64 [Hq, N, ceil(N/64)]: the block mask (bit j % 64 of word j / 64)
    sums: torch.Tensor          # float32 [Hq, N, N]: block sums (values of the input dtype), causal part
    stride: int
    block_size: int

    def dense_mask(self) -> torch.Tensor:
        """[Hq, N, N] bool block mask."""
        return mask_from_bits(self.blk_bits, self.blk_cnt.shape[1])

    def nnz(self) -> int:
        return int(self.blk_cnt.sum().item())


_thr_cache: dict = {}


def _thresholds(threshold, H: int, device) -> torch.Tensor:
    """Per-head float64 thresholds as find_blocks_chunked forms them
    (utils.py:90-105): a tensor (or sequence) is cast to float64 (a sequence
    becomes a float32 tensor first, as torch.tensor makes it) and truncated or
    padded with its last value to H heads; a number applies to every head."""
    if isinstance(threshold, (int, float)):
        t = torch.full((H,), float(threshold), dtype=torch.float64)
    else:
        t = torch.as_tensor(threshold)
        if not t.is_floating_point():
            t = t.float()
        t = t.detach().to("cpu", torch.float64).flatten()
        if t.numel() == 0:
            raise ValueError("empty threshold")
        t = t[:H] if t.numel() >= H else torch.cat([t, t[-1:].expand(H - t.numel())])
    # device copies are cached: a fresh host-to-device copy would wait for the stream
    key = (tuple(t.tolist()), str(device))
    d = _thr_cache.get(key)
    if d is None:
        d = t.to(device)
        _thr_cache[key] = d
    return d


_MODES = {"inverse": 0, "": 0, "slash": 1, "random": 2, "double": 3, "triple": 4}


def default_chunk_size(k_len: int) -> int:
    """Xattention_prefill's chunk size when none is given (Xattention.py:326-335):
    the next power of two of k_len, clamped to [2048, 2^28 / that power]."""
    p = 1 << (k_len - 1).bit_length()
    return int(max(min(max(2048, p), 128 * 1024 * 2048 // p), 2048))


def xattn_select(query_states: torch.Tensor, key_states: torch.Tensor, *, stride: int = 8, threshold=0.9,
                 norm: float = 1.0, block_size: int = 128, keep_sink: bool = False, keep_recent: bool = False,
                 causal: bool = True, use_triton: bool = True, select_mode: str = "inverse", kdb: int = 1,
                 softmax: bool = True, chunk_size: int | None = None, perm=None,
                 max_workspace_bytes: int = 16 << 30) -> XSelection:
    """The block selection of xattn_estimate (Xattention.py:14-303) as block
    lists.  q [1,Hq,L,D], k [1,Hq or Hkv,L,D] on the GPU (bf16/f16, D = 128).
    ``chunk_size`` (tokens; default Xattention_prefill's) sets the zero padding
    the non-causal softmax and the torch path's masks see.  ``perm``: the
    "random" reshaping's permutation; by default torch.randperm(stride), drawn
    where the reference draws it.  On the Triton path select_mode and softmax
    are not used, as in the reference.  The stored scores (about (L/S)^2
    bytes per head) are formed for as many heads at a time as fit
    ``max_workspace_bytes`` (one head at least); the result does not depend
    on the grouping."""
    q = _check_layout(query_states)
    k = _check_layout(key_states)
    assert q.shape[0] == 1 and k.shape[0] == 1, "batch size 1 only"          # Xattention.py:361
    assert block_size == 128, "block_size must be 128"                          # Xattention.py:360
    Hq, L, D = q.shape[1], q.shape[2], q.shape[3]
    Hk = k.shape[1]
    if k.shape[2] != L or k.shape[3] != D or Hq % Hk:
        raise ValueError(f"query {tuple(q.shape)} and key {tuple(k.shape)} shapes do not match")
    if q.dtype != k.dtype or q.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"unsupported dtypes {q.dtype}, {k.dtype} (bf16/f16)")
    if use_triton and kdb != 1:
        raise ValueError("use_triton and kdb cannot be used together")           # Xattention.py:144
    mode = 0
    pm = list(range(16))
    if not use_triton:
        if select_mode not in _MODES:
            raise ValueError(f"unknown select_mode {select_mode!r}")
        mode = _MODES[select_mode]
        if mode == 2:
            pv = torch.randperm(stride) if perm is None else torch.as_tensor(perm)   # Xattention.py:76
            pm[:stride] = [int(x) for x in pv.tolist()]
    chunk = default_chunk_size(L) if chunk_size is None else int(chunk_size)
    N = -(-L // block_size)
    dev = _lib.same_device(q, k)
    thr = _thresholds(threshold, Hq, dev)
    sel = XSelection(blk_cnt=torch.empty(Hq, N, dtype=torch.int32, device=dev),
                     blk_bits=torch.empty(Hq, N, mask_words(N), dtype=torch.int64, device=dev),
                     sums=torch.zeros(Hq, N, N, dtype=torch.float32, device=dev),
                     stride=stride, block_size=block_size)
    args = XattnArgs(
        q=q.data_ptr(), q_sh=q.stride(1), q_sl=q.stride(2), k=k.data_ptr(), k_sh=k.stride(1), k_sl=k.stride(2),
        dtype=_lib.FS_DTYPE[q.dtype], Hq=Hq, Hk=Hk, L=L, D=D, stride=stride, bs=block_size, norm=float(norm),
        threshold=thr.data_ptr(), keep_sink=int(bool(keep_sink)), sums=sel.sums.data_ptr(),
        blk_cnt=sel.blk_cnt.data_ptr(), blk_bits=sel.blk_bits.data_ptr(),
        non_causal=int(not causal), torch_path=int(not use_triton), select_mode=mode, kdb=int(kdb),
        no_softmax=int(not use_triton and not softmax), chunk=chunk, keep_recent=int(bool(keep_recent)))
    args.perm[:] = pm
    lib = _lib.load()
    hg = Hq
    while hg > 1:
        args.head_group = hg
        if lib.fs_xattn_work_bytes(ctypes.byref(args)) <= max_workspace_bytes:
            break
        hg -= 1
    groups = -(-Hq // hg)
    args.head_group = -(-Hq // groups)            # the same heads per group, as few groups as fit
    work = torch.empty(max(1, lib.fs_xattn_work_bytes(ctypes.byref(args))), dtype=torch.uint8, device=dev)
    args.work = work.data_ptr()
    _lib.call("fs_xattn", args, dev)
    sel._keep = (thr, work)                          # alive until the stream has used them
    return sel


def xattn_estimate(query_states, key_states, block_size, stride, norm=1, softmax=True, threshold=0.9,
                   chunk_size=16384, select_mode="inverse", use_triton=True, causal=True, kdb: int = 1,
                   keep_sink=False, keep_recent=False):
    """Xattention.py:14-303 on the GPU kernels: returns (attn_sums, simple_masks),
    [1, H, N, N] in the input dtype and bool, N = ceil(L / block_size) (the
    reference pads both to whole chunks; its Xattention_prefill keeps this
    N x N corner).  Causal sums are zero above the diagonal."""
    sel = xattn_select(query_states, key_states, stride=stride, threshold=threshold, norm=norm,
                       block_size=block_size, keep_sink=keep_sink, keep_recent=keep_recent, causal=causal,
                       use_triton=use_triton, select_mode=select_mode, kdb=kdb, softmax=softmax,
                       chunk_size=chunk_size)
    return sel.sums.to(query_states.dtype)[None], sel.dense_mask()[None]


def Xattention_prefill(query_states: torch.Tensor, key_states: torch.Tensor, value_states: torch.Tensor, stride,
                       norm=1, threshold=0.8, block_size=128, use_triton=True, causal=True, kdb=1,
                       chunk_size=None, keep_sink=False, keep_recent=False):
    """Xattention.py:306-406: the XAttention selection ("inverse" reshaping),
    then block-sparse attention over the chosen blocks (causal or not).
    q [1,H,L,D], k/v [1,H or Hkv,L,D] -> [1, H, L, D] (a view of [1, L, H, D]
    storage, as the reference returns)."""
    assert query_states.is_cuda, "input tensors must be on the GPU"
    sel = xattn_select(query_states, key_states, stride=stride, threshold=threshold, norm=norm,
                       block_size=block_size, keep_sink=keep_sink, keep_recent=keep_recent, causal=causal,
                       use_triton=use_triton, kdb=kdb, chunk_size=chunk_size)
    out = block_sparse_attention(query_states, key_states, value_states, sel.blk_cnt, sel.blk_bits,
                                 block_size=block_size, is_causal=causal)
    return out.transpose(1, 2)


def density(sel: XSelection) -> float:
    """Selected tiles over the causal tiles (row 0's keep_sink blocks above the
    diagonal are not computed and not counted)."""
    H, N = sel.blk_cnt.shape
    return min(1.0, sel.nnz() / (H * N * (N + 1) / 2))


__all__ = ["XSelection", "xattn_select", "xattn_estimate", "Xattention_prefill", "default_chunk_size", "density"]
