"""Drop-in ``myattn_prefill`` (FFTSparse v7 API) on hand-written gfx950 kernels.

Mirrors ``attn_src/fft_attn/my_attn_v7.py:454-792``: same signature, defaults,
return shape ([bsz, L_q, H*D] in the input dtype) and error types.  The
computation runs as a fixed sequence of stream-ordered kernel launches with no
host synchronisation:

    fs_pool    Q/K block means                       (:553-555)
    fs_corr    FFT lag correlation + lag threshold   (:567-576)
    fs_stats   diagonal statistics, column scores,
               last-row scores and their top-n       (:558-560, :581-596, :623-635)
    fs_select  stripe/diffuse decision, qk top-k,
               mask composition -> block mask, one bit per block (:600-641)
    fs_bsattn  block-sparse causal GQA attention     (:775-786)

K/V may carry Hq heads (the reference's repeat_kv'd layout) or Hkv heads with
Hq % Hkv == 0 (native GQA, no repetition needed).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import AttnArgs, CorrArgs, PoolArgs, RopePoolArgs, ScoresArgs, SelectArgs, StatsArgs, ptr
from .params import PrefillParams, derive, f32

_MIN_BLOCKS = 10          # my_attn_v7.py:509


def mask_words(nk: int) -> int:
    """64-bit words per row of a block mask over ``nk`` key blocks."""
    return (nk + 63) // 64


def bits_from_mask(mask: torch.Tensor):
    """Block mask bool [H, N, Nk] (or the reference's base_blockmask [1, H, N, Nk])
    -> (blk_cnt int32 [H, N], blk_bits int64 [H, N, ceil(Nk/64)]): bit b of word w
    of a row is key block 64 w + b."""
    if mask.dim() == 4:
        if mask.shape[0] != 1:
            raise ValueError("a 4-d block mask must have batch size 1")
        mask = mask[0]
    if mask.dim() != 3 or mask.dtype != torch.bool:
        raise ValueError(f"block mask must be a bool [H, N, Nk] tensor, got {mask.dtype} {tuple(mask.shape)}")
    H, N, Nk = mask.shape
    W = mask_words(Nk)
    m = torch.zeros(H, N, W * 64, dtype=torch.int64, device=mask.device)
    m[:, :, :Nk] = mask.to(torch.int64)
    m = m.view(H, N, W, 2, 32)
    sh = torch.arange(32, device=mask.device, dtype=torch.int64)
    half = (m << sh).sum(-1)                              # [H, N, W, 2], each < 2^32
    bits = half[..., 0] | (half[..., 1] << 32)
    return mask.sum(-1, dtype=torch.int32).contiguous(), bits.contiguous()


def mask_from_bits(blk_bits: torch.Tensor, nk: int) -> torch.Tensor:
    """[H, N, W] block mask words -> bool [H, N, nk]."""
    H, N, W = blk_bits.shape
    sh = torch.arange(64, device=blk_bits.device, dtype=torch.int64)
    m = ((blk_bits.to(torch.int64)[..., None] >> sh) & 1).bool().view(H, N, W * 64)
    return m[:, :, :nk]


@dataclass
class BlockSelection:
    """Device-resident result of the mask selection stage."""
    params: PrefillParams
    blk_cnt: torch.Tensor            # int32 [Hq, N], selected blocks per row
    blk_bits: torch.Tensor           # int64 [Hq, N, ceil(Nk/64)], the block mask (bit j % 64 of word j / 64)
    q_b: torch.Tensor | None = None  # [Hq, N, D]
    k_b: torch.Tensor | None = None  # [Hk, N, D]
    corr: torch.Tensor | None = None
    corr_sum: torch.Tensor | None = None
    keep_tau: torch.Tensor | None = None
    diag_var: torch.Tensor | None = None
    col_mean: torch.Tensor | None = None
    col_sel: torch.Tensor | None = None
    last_scores: torch.Tensor | None = None
    last_sel: torch.Tensor | None = None
    mean_var: torch.Tensor | None = None
    is_stripe: torch.Tensor | None = None

    def dense_mask(self) -> torch.Tensor:
        """[Hq, N, Nk] bool block mask."""
        return mask_from_bits(self.blk_bits, self.params.Nk)

    def nnz(self) -> int:
        return int(self.blk_cnt.sum().item())


# largest block count of the selection kernels: 8192 on the 16-bit path (block
# scores on MFMA; a diffuse head's 4-row score panel in LDS), 4096 on the fp32
# path (LDS FFT length 8192)
MAX_SELECT_BLOCKS = 8192
MAX_FFT_BLOCKS = 4096

_tau_cache: dict = {}


def _sample_taus_device(taus, device):
    key = (tuple(taus), str(device))
    t = _tau_cache.get(key)
    if t is None:
        t = torch.tensor(list(taus) or [0], dtype=torch.int32).to(device)
        _tau_cache[key] = t
    return t


def _check_layout(x: torch.Tensor) -> torch.Tensor:
    if x.dim() != 4:
        raise ValueError(f"expected a [B, H, L, D] tensor, got shape {tuple(x.shape)}")
    if x.stride(3) != 1 or x.stride(2) % 8 or x.stride(1) % 8 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    return x


def select_blocks(query_states: torch.Tensor, key_states: torch.Tensor, *, block_size=128,
                  sink_ratio=0.1, recent_ratio=0.1, local_span_ratio=0.1,
                  enable_correlation_mask=True, correlation_selection_mode="threshold",
                  correlation_topk_ratio=0.2, corr_threshold=0.1,
                  enable_column_mask=True, column_topk_ratio=0.1,
                  column_start_exclude_ratio=0.1, column_end_exclude_ratio=0.2,
                  enable_last_block_mask=True, diag_sample_ratio=0.15, min_diag_samples=5,
                  max_diag_samples=64, stripe_threshold=0.3, qk_topk_ratio=0.2,
                  keep_intermediates=False, pipeline_groups=None, pooled=None) -> BlockSelection:
    """Stage 1 of my_attn_v7.myattn_prefill (:533-641): the block mask of every
    (query head, query block).  q [1,Hq,L,D], k [1,Hk,L,D].  ``pooled``: the
    block means (q_b [Hq,N,D], k_b [Hk,N,D]) already formed by ``rope_pool``,
    which then replace the pooling pass."""
    q = _check_layout(query_states)
    k = _check_layout(key_states)
    if q.shape[0] != 1 or k.shape[0] != 1:
        raise ValueError("myattn_prefill supports batch size 1 (my_attn_v7.py:521)")
    Hq, L_q, D = q.shape[1], q.shape[2], q.shape[3]
    Hk, L_k = k.shape[1], k.shape[2]
    if Hq % Hk:
        raise ValueError(f"query heads {Hq} must be a multiple of key heads {Hk}")
    if k.shape[3] != D:
        raise ValueError(f"query head_dim {D} and key head_dim {k.shape[3]} differ")
    dev = _lib.same_device(q, k, *(pooled or ()))
    if L_q != L_k:
        raise ValueError(f"prefill expects L_q == L_k, got {L_q} and {L_k}")
    if q.dtype != k.dtype or q.dtype not in _lib.FS_DTYPE:
        raise TypeError(f"unsupported dtypes {q.dtype}, {k.dtype}")
    if correlation_selection_mode not in ("threshold", "topk"):
        raise ValueError(f"Unknown selection_mode: {correlation_selection_mode}")
    p = derive(L_q, L_k, block_size, sink_ratio, recent_ratio, local_span_ratio,
               enable_correlation_mask, correlation_topk_ratio, enable_column_mask,
               column_topk_ratio, column_start_exclude_ratio, column_end_exclude_ratio,
               enable_last_block_mask, diag_sample_ratio, min_diag_samples, max_diag_samples)
    if p.N > MAX_SELECT_BLOCKS:
        raise RuntimeError(f"{p.N} query blocks (L={L_q}, block_size={block_size}) exceed the selection "
                           f"kernels' maximum of {MAX_SELECT_BLOCKS}")
    if p.corr_enabled and p.remote_start >= p.N:
        # my_attn_v7.py:190-191 returns a single tensor there and the six-way
        # unpacking at :568 raises.
        raise ValueError("not enough values to unpack (expected 6, got 1)")
    dt = _lib.FS_DTYPE[q.dtype]
    N, Nk = p.N, p.Nk
    G = Hq // Hk
    need_pool = enable_last_block_mask or p.corr_enabled or p.col_enabled   # :553
    n_cols = p.n_cols if p.col_enabled else 0
    last_k = p.last_k if enable_last_block_mask else 0
    n_samples = 0 if (not p.corr_enabled or p.stripe_all_diffuse) else len(p.sample_taus)
    # 16-bit inputs: correlation and statistics in one call from MFMA block-score tiles
    use_scores = (q.dtype in (torch.bfloat16, torch.float16) and D % 16 == 0 and D <= 128
                  and (p.corr_enabled or n_cols or last_k))
    if not use_scores and (p.corr_enabled or n_cols or last_k) and N > MAX_FFT_BLOCKS:
        raise RuntimeError(f"{N} query blocks exceed the fp32 / D > 128 selection path's maximum of "
                           f"{MAX_FFT_BLOCKS} (the 16-bit path with D <= 128 takes up to {MAX_SELECT_BLOCKS})")
    thr = f32(corr_threshold)
    corr_mode = 1 if correlation_selection_mode == "topk" else 0
    corr_q = f32(1.0 - correlation_topk_ratio)                  # torch.quantile's q in fp32 (:200-201)
    # Optional pipeline over groups of KV heads (each with its query heads):
    # pooling of group g+1 (HBM bound) runs on the caller's stream while the
    # latency-bound statistics and block-list kernels of group g run on a side
    # stream.  Heads are independent, so the result does not depend on the
    # grouping.  One group is the default: at config 2 the cross-stream waits
    # cost more than the overlap saves (0.30 ms with 1 group, 0.41 ms with 4).
    ngroups = max(1, min(pipeline_groups or 1, Hk)) if need_pool else 1
    bounds = [Hk * g // ngroups for g in range(ngroups + 1)]
    lib = _lib.load()

    def pool(g):
        k0, k1 = bounds[g], bounds[g + 1]
        h0, h1 = k0 * G, k1 * G
        qg, kg = q[:, h0:h1], k[:, k0:k1]
        _lib.call("fs_pool", PoolArgs(q=qg.data_ptr(), q_sh=q.stride(1), q_sl=q.stride(2),
                                      k=kg.data_ptr(), k_sh=k.stride(1), k_sl=k.stride(2),
                                      dtype=dt, Hq=h1 - h0, Hk=k1 - k0, L=L_q, D=D, bs=block_size,
                                      q_b=sel.q_b[h0:h1].data_ptr(), k_b=sel.k_b[k0:k1].data_ptr()), dev)

    sel = BlockSelection(params=p, blk_cnt=None, blk_bits=None)
    if pooled is not None:
        q_b, k_b = pooled
        if (tuple(q_b.shape) != (Hq, N, D) or tuple(k_b.shape) != (Hk, N, D) or q_b.dtype != q.dtype
                or k_b.dtype != q.dtype or not q_b.is_contiguous() or not k_b.is_contiguous()):
            raise ValueError(f"pooled block means must be contiguous [{Hq},{N},{D}] and [{Hk},{N},{D}] in {q.dtype}")
        sel.q_b, sel.k_b = q_b, k_b
    elif need_pool:
        sel.q_b = torch.empty(Hq, N, D, dtype=q.dtype, device=dev)
        sel.k_b = torch.empty(Hk, N, D, dtype=q.dtype, device=dev)
        # The first group's pooling (the longest kernel of the stage) goes out
        # before the remaining buffers are allocated: a call on an idle GPU
        # then waits only for this much host work.
        pool(0)
    sel.blk_cnt = torch.empty(Hq, N, dtype=torch.int32, device=dev)
    sel.blk_bits = torch.empty(Hq, N, mask_words(Nk), dtype=torch.int64, device=dev)
    if p.corr_enabled:
        sel.corr = torch.empty(Hq, N, dtype=torch.float32, device=dev)
        sel.corr_sum = torch.empty(Hq, N, dtype=torch.float32, device=dev)
        sel.keep_tau = torch.empty(Hq, N, dtype=torch.uint8, device=dev)
        sel.mean_var = torch.empty(Hq, dtype=torch.float32, device=dev)
        sel.is_stripe = torch.empty(Hq, dtype=torch.uint8, device=dev)
    if n_samples or n_cols or last_k:
        _stat_buffers(sel, Hq, N, n_samples, n_cols, last_k, dev)
    taus = _sample_taus_device(p.sample_taus, dev)
    dyn_mode = 1 if p.corr_enabled else 0
    col_mode = (1 if n_cols else 0) if p.corr_enabled else (2 if n_cols else 0)

    works = []
    for g in range(ngroups):
        hq = (bounds[g + 1] - bounds[g]) * G
        if use_scores:
            nbytes = lib.fs_scores_work_bytes(hq, N, n_samples)
        elif p.corr_enabled:
            nbytes = lib.fs_corr_work_bytes(hq, N, D)
        else:
            nbytes = 0
        works.append(torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev))
    main = torch.cuda.current_stream(dev)
    side = _side_stream(dev) if ngroups > 1 else main
    if side is not main:
        side.wait_stream(main)                    # buffers above are allocated before the side work
    sl = lambda t, a0, a1: None if t is None else t[a0:a1]   # noqa: E731
    for g in range(ngroups):
        k0, k1 = bounds[g], bounds[g + 1]
        h0, h1 = k0 * G, k1 * G
        hq, hk = h1 - h0, k1 - k0
        if need_pool and pooled is None and g > 0:
            pool(g)
        if side is not main:
            ev = torch.cuda.Event()
            ev.record(main)
            side.wait_event(ev)
        with torch.cuda.stream(side):
            q_b, k_b = sl(sel.q_b, h0, h1), sl(sel.k_b, k0, k1)
            if use_scores:
                _lib.call("fs_scores", ScoresArgs(
                    q_b=ptr(q_b), k_b=ptr(k_b), dtype=dt, Hq=hq, Hk=hk, N=N, D=D,
                    local_window=p.local_window, keep_sink=p.keep_sink, remote_start=p.remote_start,
                    corr_threshold=thr, corr_mode=corr_mode, corr_quantile=corr_q,
                    corr=ptr(sl(sel.corr, h0, h1)), corr_sum=ptr(sl(sel.corr_sum, h0, h1)),
                    keep_tau=ptr(sl(sel.keep_tau, h0, h1)), sample_taus=taus.data_ptr(), n_samples=n_samples,
                    col_start=p.col_start, col_end=p.col_end, n_cols=n_cols, last_k=last_k,
                    diag_var=ptr(sl(sel.diag_var, h0, h1)), col_mean=ptr(sl(sel.col_mean, h0, h1)),
                    col_sel=ptr(sl(sel.col_sel, h0, h1)), last_scores=ptr(sl(sel.last_scores, h0, h1)),
                    last_sel=ptr(sl(sel.last_sel, h0, h1)), work=works[g].data_ptr()), dev)
            else:
                if p.corr_enabled:
                    _lib.call("fs_corr", CorrArgs(
                        q_b=ptr(q_b), k_b=ptr(k_b), dtype=dt, Hq=hq, Hk=hk, N=N, D=D,
                        local_window=p.local_window, keep_sink=p.keep_sink, remote_start=p.remote_start,
                        corr_threshold=thr, corr_mode=corr_mode, corr_quantile=corr_q,
                        work=works[g].data_ptr(), corr=ptr(sl(sel.corr, h0, h1)),
                        corr_sum=ptr(sl(sel.corr_sum, h0, h1)), keep_tau=ptr(sl(sel.keep_tau, h0, h1))), dev)
                if n_samples or n_cols or last_k:
                    _lib.call("fs_stats", StatsArgs(
                        q_b=ptr(q_b), k_b=ptr(k_b), dtype=dt, Hq=hq, Hk=hk, N=N, D=D,
                        sample_taus=taus.data_ptr(), n_samples=n_samples,
                        col_start=p.col_start, col_end=p.col_end, n_cols=n_cols, last_k=last_k,
                        diag_var=ptr(sl(sel.diag_var, h0, h1)), col_mean=ptr(sl(sel.col_mean, h0, h1)),
                        col_sel=ptr(sl(sel.col_sel, h0, h1)), last_scores=ptr(sl(sel.last_scores, h0, h1)),
                        last_sel=ptr(sl(sel.last_sel, h0, h1))), dev)
            _lib.call("fs_select", SelectArgs(
                q_b=ptr(q_b), k_b=ptr(k_b), dtype=dt, Hq=hq, Hk=hk, N=N, Nk=Nk, D=D, mask_causal=1,
                keep_sink=p.keep_sink, keep_recent=p.keep_recent, local_window=p.local_window,
                remote_start=p.remote_start, dyn_mode=dyn_mode, stripe_all_diffuse=int(p.stripe_all_diffuse),
                diag_var=ptr(sl(sel.diag_var, h0, h1)), n_samples=n_samples,
                stripe_threshold=f32(stripe_threshold), keep_tau=ptr(sl(sel.keep_tau, h0, h1)),
                qk_topk_ratio=f32(qk_topk_ratio), col_mode=col_mode, col_sel=ptr(sl(sel.col_sel, h0, h1)),
                last_sel=ptr(sl(sel.last_sel, h0, h1)), mean_var=ptr(sl(sel.mean_var, h0, h1)),
                is_stripe=ptr(sl(sel.is_stripe, h0, h1)), blk_cnt=sel.blk_cnt[h0:h1].data_ptr(),
                blk_bits=sel.blk_bits[h0:h1].data_ptr()), dev)
    if side is not main:
        main.wait_stream(side)                    # every output is ready on the caller's stream
    if not keep_intermediates:
        sel.q_b = sel.k_b = None
    return sel


def rope_pool(query_states: torch.Tensor, key_states: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, *,
              block_size=128):
    """The attention forward's rotary embedding (eval/LongBench/pred.py:195:
    transformers' apply_rotary_pos_emb) fused with the block pooling of the
    rotated states (my_attn_v7.py:105-114) in one pass over Q and K.

    q [1,Hq,L,D], k [1,Hk,L,D] before RoPE (strided views, e.g. the
    projections' ``view().transpose(1, 2)``); cos / sin [L,D] or [1,L,D], the
    model's position embeddings.  Returns (q_rot, k_rot, q_b, k_b): the rotated
    states as [1,H,L,D] views of [1,L,H,D] storage, bit-identical to
    apply_rotary_pos_emb, and their block means [H,N,D], bit-identical to the
    pooling pass of ``select_blocks`` on q_rot / k_rot."""
    q = _check_layout(query_states)
    k = _check_layout(key_states)
    if q.shape[0] != 1 or k.shape[0] != 1:
        raise ValueError("rope_pool takes batch size 1 (my_attn_v7.py:521)")
    Hq, L, D = q.shape[1], q.shape[2], q.shape[3]
    Hk = k.shape[1]
    if k.shape[2] != L or k.shape[3] != D or Hq % Hk:
        raise ValueError(f"query {tuple(q.shape)} and key {tuple(k.shape)} shapes do not match")
    if q.dtype != k.dtype or q.dtype not in _lib.FS_DTYPE:
        raise TypeError(f"unsupported dtypes {q.dtype}, {k.dtype}")
    cs = []
    for t in (cos, sin):
        t = t[0] if t.dim() == 3 else t
        if t.shape != (L, D) or t.dtype != q.dtype:
            raise ValueError(f"cos/sin must be [{L},{D}] (or [1,{L},{D}]) in {q.dtype}, got {tuple(t.shape)} {t.dtype}")
        if t.stride(1) != 1 or t.stride(0) % 8 or t.data_ptr() % 16:
            t = t.contiguous()
        cs.append(t)
    if cs[0].stride(0) != cs[1].stride(0):
        cs = [t.contiguous() for t in cs]
    N = (L + block_size - 1) // block_size
    dev = _lib.same_device(q, k, *cs)
    q_rot = torch.empty(1, L, Hq, D, dtype=q.dtype, device=dev).transpose(1, 2)
    k_rot = torch.empty(1, L, Hk, D, dtype=q.dtype, device=dev).transpose(1, 2)
    q_b = torch.empty(Hq, N, D, dtype=q.dtype, device=dev)
    k_b = torch.empty(Hk, N, D, dtype=q.dtype, device=dev)
    _lib.call("fs_rope_pool", RopePoolArgs(
        q=q.data_ptr(), q_sh=q.stride(1), q_sl=q.stride(2), k=k.data_ptr(), k_sh=k.stride(1), k_sl=k.stride(2),
        cos=cs[0].data_ptr(), sin=cs[1].data_ptr(), cs_sl=cs[0].stride(0),
        q_out=q_rot.data_ptr(), qo_sh=q_rot.stride(1), qo_sl=q_rot.stride(2),
        k_out=k_rot.data_ptr(), ko_sh=k_rot.stride(1), ko_sl=k_rot.stride(2),
        dtype=_lib.FS_DTYPE[q.dtype], Hq=Hq, Hk=Hk, L=L, D=D, bs=block_size, q_b=q_b.data_ptr(), k_b=k_b.data_ptr()),
        dev)
    return q_rot, k_rot, q_b, k_b


_side = {}


def _side_stream(dev):
    """One default-priority side stream per device for the selection pipeline."""
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    st = _side.get(key)
    if st is None:
        st = torch.cuda.Stream(device=dev)
        _side[key] = st
    return st


def _stat_buffers(sel, Hq, N, n_samples, n_cols, last_k, dev):
    u8 = torch.uint8
    sel.diag_var = torch.empty(Hq, max(1, n_samples), dtype=torch.float32, device=dev)
    sel.col_mean = torch.empty(Hq, N, dtype=torch.float32, device=dev) if n_cols else None
    sel.col_sel = torch.empty(Hq, N, dtype=u8, device=dev) if n_cols else None
    sel.last_scores = torch.empty(Hq, N, dtype=torch.float32, device=dev) if last_k else None
    sel.last_sel = torch.empty(Hq, N, dtype=u8, device=dev) if last_k else None


class AttentionCall:
    """One prepared stage-2 call: argument struct, workspace and output.

    ``prepare()`` stages V^T in the workspace (fs_bsattn_prepare), ``run()``
    orders the work items and runs the attention kernel (fs_bsattn_run), and
    ``__call__`` does both in one C call (fs_bsattn).  Every launch goes on
    torch's current stream."""

    def __init__(self, query_states, key_states, value_states, blk_cnt=None, blk_bits=None, *,
                 block_size=128, is_causal=True, softmax_scale=None, out=None, gqa_interleave=False):
        q = _check_layout(query_states)
        k = _check_layout(key_states)
        v = _check_layout(value_states)
        B, Hq, Lq, D = q.shape
        Hk, Lk = k.shape[1], k.shape[2]
        if v.shape[1] != Hk or v.shape[2] != Lk or k.shape[0] != B or v.shape[0] != B:
            raise ValueError("key/value shapes do not match")
        if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
            # flash-attention kernels accept fp16/bf16 only, as does the reference's
            # block_sparse_attn_func.
            raise RuntimeError("FlashAttention only supports fp16 and bf16 data type")
        if (blk_cnt is None) != (blk_bits is None):
            raise ValueError("blk_cnt and blk_bits go together")
        if blk_cnt is not None:
            Nq, Nk = -(-Lq // block_size), -(-Lk // block_size)
            if blk_cnt.dtype != torch.int32 or tuple(blk_cnt.shape) != (Hq, Nq) or not blk_cnt.is_contiguous():
                raise ValueError(f"blk_cnt must be a contiguous int32 [{Hq}, {Nq}] tensor, got "
                                 f"{blk_cnt.dtype} {tuple(blk_cnt.shape)}")
            W = mask_words(Nk)
            if blk_bits.dtype != torch.int64 or tuple(blk_bits.shape) != (Hq, Nq, W) or not blk_bits.is_contiguous():
                raise ValueError(f"blk_bits must be a contiguous int64 [{Hq}, {Nq}, {W}] tensor, got "
                                 f"{blk_bits.dtype} {tuple(blk_bits.shape)}")
        if k.shape[3] != D or v.shape[3] != D:
            raise ValueError(f"query, key and value head_dim differ: {D}, {k.shape[3]}, {v.shape[3]}")
        if out is not None and (tuple(out.shape) != (B, Lq, Hq, D) or out.dtype != q.dtype):
            raise ValueError(f"out must be a [{B}, {Lq}, {Hq}, {D}] {q.dtype} tensor, got {out.dtype} "
                             f"{tuple(out.shape)}")
        self.device = _lib.same_device(q, k, v, blk_cnt, blk_bits, out)
        if out is None:
            out = torch.empty(B, Lq, Hq, D, dtype=q.dtype, device=q.device)
        scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
        args = AttnArgs(
            q=q.data_ptr(), q_sb=q.stride(0), q_sh=q.stride(1), q_sl=q.stride(2),
            k=k.data_ptr(), k_sb=k.stride(0), k_sh=k.stride(1), k_sl=k.stride(2),
            v=v.data_ptr(), v_sb=v.stride(0), v_sh=v.stride(1), v_sl=v.stride(2),
            out=out.data_ptr(), o_sb=out.stride(0), o_sh=out.stride(2), o_sl=out.stride(1),
            dtype=_lib.FS_DTYPE[q.dtype], B=B, Hq=Hq, Hk=Hk, Lq=Lq, Lk=Lk, D=D, bs=block_size,
            is_causal=int(bool(is_causal)), softmax_scale=scale, gqa_interleave=int(bool(gqa_interleave)),
            blk_cnt=ptr(blk_cnt), blk_bits=ptr(blk_bits))
        self.work = torch.empty(_lib.load().fs_bsattn_work_bytes(ctypes.byref(args)), dtype=torch.uint8,
                                device=q.device)
        args.work = self.work.data_ptr()
        self.args = args
        self.out = out
        self._keep = (q, k, v, blk_cnt, blk_bits)     # the pointers in args stay valid

    def prepare(self) -> None:
        _lib.call("fs_bsattn_prepare", self.args, self.device)

    def run(self) -> torch.Tensor:
        _lib.call("fs_bsattn_run", self.args, self.device)
        return self.out

    def __call__(self) -> torch.Tensor:
        _lib.call("fs_bsattn", self.args, self.device)
        return self.out


def block_sparse_attention(query_states, key_states, value_states, blk_cnt=None, blk_bits=None, *,
                           block_mask=None, block_size=128, is_causal=True, softmax_scale=None, out=None,
                           gqa_interleave=False) -> torch.Tensor:
    """Block-sparse (or, with no block mask, dense causal) attention.

    q [B,Hq,Lq,D], k/v [B,Hk,Lk,D] -> out [B, Lq, Hq, D] in the input dtype.
    The mask is either (blk_cnt, blk_bits), as the selectors return it, or
    ``block_mask``: a bool [Hq, Nq, Nk] or [1, Hq, Nq, Nk] tensor, the
    reference's base_blockmask (my_attn_v7.py:780).
    Query head h reads KV head h // (Hq / Hk), or h % Hk with ``gqa_interleave``."""
    if block_mask is not None:
        if blk_cnt is not None or blk_bits is not None:
            raise ValueError("give either block_mask or (blk_cnt, blk_bits)")
        blk_cnt, blk_bits = bits_from_mask(block_mask)
    return AttentionCall(query_states, key_states, value_states, blk_cnt, blk_bits, block_size=block_size,
                         is_causal=is_causal, softmax_scale=softmax_scale, out=out,
                         gqa_interleave=gqa_interleave)()


def myattn_prefill(
        query_states,
        key_states,
        value_states,
        layer_idx,
        block_size=128,
        is_causal=True,
        is_visual=False,
        sink_ratio=0.1,
        recent_ratio=0.1,
        local_span_ratio=0.1,
        enable_correlation_mask=True,
        correlation_selection_mode: str = "threshold",
        correlation_topk_ratio: float = 0.2,
        corr_threshold: float = 0.1,
        collect_corr_stats: bool = False,
        enable_column_mask: bool = True,
        column_topk_ratio: float = 0.1,
        column_start_exclude_ratio: float = 0.1,
        column_end_exclude_ratio: float = 0.2,
        enable_last_block_mask=True,
        last_block_threshold=0.01,
        diag_sample_ratio: float = 0.15,
        min_diag_samples: int = 5,
        max_diag_samples: int = 64,
        stripe_threshold: float = 0.3,
        qk_topk_ratio: float = 0.2,
        attention_vis_heads=[0],
        attention_vis_dir=None,
):
    """Block-sparse prefill attention, my_attn_v7.py:454-792.

    query_states [bsz,H,L_q,D], key/value_states [bsz,H or Hkv,L_k,D] on the
    GPU -> [bsz, L_q, H*D].  ``last_block_threshold`` is accepted and unused,
    as in the reference; ``is_visual`` / ``collect_corr_stats`` (plotting and
    statistics collection) are accepted and ignored."""
    assert query_states.is_cuda, "input tensors must be on the GPU"   # :502
    bsz = query_states.shape[0]
    L_q = query_states.shape[2]
    H = query_states.shape[1]
    o = v7_prefill(query_states, key_states, value_states, block_size=block_size, is_causal=is_causal,
                   sink_ratio=sink_ratio, recent_ratio=recent_ratio, local_span_ratio=local_span_ratio,
                   enable_correlation_mask=enable_correlation_mask,
                   correlation_selection_mode=correlation_selection_mode,
                   correlation_topk_ratio=correlation_topk_ratio, corr_threshold=corr_threshold,
                   enable_column_mask=enable_column_mask, column_topk_ratio=column_topk_ratio,
                   column_start_exclude_ratio=column_start_exclude_ratio,
                   column_end_exclude_ratio=column_end_exclude_ratio,
                   enable_last_block_mask=enable_last_block_mask,
                   diag_sample_ratio=diag_sample_ratio, min_diag_samples=min_diag_samples,
                   max_diag_samples=max_diag_samples, stripe_threshold=stripe_threshold,
                   qk_topk_ratio=qk_topk_ratio)
    return o.reshape(bsz, L_q, H * query_states.shape[3])


def v7_prefill(query_states, key_states, value_states, *, block_size=128, is_causal=True, softmax_scale=None,
               return_selection=False, **select_kw):
    """The body of myattn_prefill (my_attn_v7.py:502-786) with the result left as [bsz, L_q, H, D]
    and an optional softmax scale (default 1/sqrt(D), the reference's): dense causal attention
    below 10 key blocks (:509-519), else v7 selection and block-sparse attention.  ``select_kw``
    are select_blocks' keyword arguments.  With ``return_selection`` the result is (output,
    BlockSelection or None for the dense path)."""
    assert query_states.is_cuda, "input tensors must be on the GPU"   # :502
    L_k = key_states.shape[2]
    if L_k < block_size * _MIN_BLOCKS:                                 # :509-519
        out = block_sparse_attention(query_states, key_states, value_states,
                                     block_size=block_size if block_size in (64, 128) else 128,
                                     is_causal=True, softmax_scale=softmax_scale)
        return (out, None) if return_selection else out
    if query_states.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError("FlashAttention only supports fp16 and bf16 data type")
    sel = select_blocks(query_states, key_states, block_size=block_size, **select_kw)
    out = block_sparse_attention(query_states, key_states, value_states, sel.blk_cnt, sel.blk_bits,
                                 block_size=block_size, is_causal=is_causal, softmax_scale=softmax_scale)
    return (out, sel) if return_selection else out
