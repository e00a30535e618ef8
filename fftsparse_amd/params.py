"""Host-side derivation of the integer parameters of one prefill call.

Everything here is computed with Python int/float semantics exactly as the
reference does before it launches any device work
(attn_src/fft_attn/my_attn_v7.py:533-540, 563, 579-585, 316-332, 422-432,
626-634), so that the kernels receive the same integers.
"""
from __future__ import annotations

from dataclasses import dataclass, field, replace

import numpy as np
import torch


def f32(x: float) -> float:
    """Python float rounded to fp32 (torch compares an fp32 tensor with a
    Python scalar after casting the scalar to fp32)."""
    return float(np.float32(x))


@dataclass
class PrefillParams:
    L_q: int
    L_k: int
    bs: int
    N: int                      # query blocks
    Nk: int                     # key blocks
    keep_sink: int
    keep_recent: int
    local_window: int
    corr_enabled: bool          # stripe/diffuse branch runs (my_attn_v7.py:567)
    remote_start: int           # max(lw, keep_recent - 1) + 1 (:579-580)
    sample_taus: list = field(default_factory=list)
    stripe_all_diffuse: bool = False
    col_enabled: bool = False   # :623 without the num_stripe > 0 test
    col_start: int = 0
    col_end: int = 0
    n_cols: int = 0
    last_k: int = 0


_derived: dict = {}


def derive(L_q: int, L_k: int, block_size: int = 128, sink_ratio: float = 0.1,
           recent_ratio: float = 0.1, local_span_ratio: float = 0.1,
           enable_correlation_mask: bool = True, correlation_topk_ratio: float = 0.2,
           enable_column_mask: bool = True, column_topk_ratio: float = 0.1,
           column_start_exclude_ratio: float = 0.1, column_end_exclude_ratio: float = 0.2,
           enable_last_block_mask: bool = True, diag_sample_ratio: float = 0.15,
           min_diag_samples: int = 5, max_diag_samples: int = 64) -> PrefillParams:
    """The parameters of one call.  Memoised on the arguments (a prefill
    repeats the same shapes layer after layer, and the sample positions take a
    torch.linspace); each call returns its own copy."""
    key = (L_q, L_k, block_size, sink_ratio, recent_ratio, local_span_ratio, enable_correlation_mask,
           correlation_topk_ratio, enable_column_mask, column_topk_ratio, column_start_exclude_ratio,
           column_end_exclude_ratio, enable_last_block_mask, diag_sample_ratio, min_diag_samples,
           max_diag_samples)
    p = _derived.get(key)
    if p is None:
        if len(_derived) >= 256:
            _derived.clear()
        p = _derived[key] = _derive(*key)
    return replace(p, sample_taus=list(p.sample_taus))


def _derive(L_q, L_k, block_size, sink_ratio, recent_ratio, local_span_ratio, enable_correlation_mask,
            correlation_topk_ratio, enable_column_mask, column_topk_ratio, column_start_exclude_ratio,
            column_end_exclude_ratio, enable_last_block_mask, diag_sample_ratio, min_diag_samples,
            max_diag_samples) -> PrefillParams:
    bs = block_size
    N = (L_q + bs - 1) // bs
    Nk = (L_k + bs - 1) // bs
    keep_sink = max(1, int(Nk * sink_ratio))
    keep_recent = max(1, int(Nk * recent_ratio))
    lw = max(2, int(Nk * local_span_ratio)) // 2
    corr_top_k = max(1, int(N * correlation_topk_ratio))
    p = PrefillParams(L_q, L_k, bs, N, Nk, keep_sink, keep_recent, lw,
                      corr_enabled=bool(enable_correlation_mask and N > corr_top_k),
                      remote_start=max(lw, keep_recent - 1) + 1)
    if p.corr_enabled:
        rs = p.remote_start
        n_remote = max(1, (N + rs) // 2 - rs + 1)
        n_samp = max(min_diag_samples, min(int(n_remote * diag_sample_ratio), max_diag_samples))
        if rs >= N - 1:
            p.stripe_all_diffuse = True
        else:
            n_av = max(1, (N + rs) // 2 - rs + 1)
            actual = min(n_samp, n_av)
            if actual <= 1:
                p.sample_taus = [rs]
            else:
                # same float32 linspace + truncation as the reference (my_attn_v7.py:331)
                p.sample_taus = (torch.linspace(0, n_av - 1, actual).long() + rs).tolist()
    p.col_enabled = bool(enable_column_mask and N > 1)
    if p.col_enabled:
        ratio = column_topk_ratio * min(1.0, (128.0 / N) ** 0.5)
        cs = max(1, int(N * column_start_exclude_ratio))
        ce = N - max(1, int(N * column_end_exclude_ratio))
        p.col_start, p.col_end = cs, ce
        if ce > cs:
            nvalid = ce - cs
            p.n_cols = min(max(1, int(nvalid * ratio)), nvalid)
    p.last_k = min(128, N) if enable_last_block_mask else 0
    return p
