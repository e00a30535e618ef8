"""CPU restatement of the FFTSparse v7 prefill path -- TEST INFRASTRUCTURE ONLY.

This module is the checker for the HIP product path.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only to compute expected results or to time the reference algorithm on
the host.  The product package (``fftsparse_amd``) never imports it.

Every function restates one function (or one block of orchestration) of the
reference ``attn_src/fft_attn/my_attn_v7.py`` with the same tensor semantics,
in torch on the CPU.  Where the reference runs a CUDA op whose arithmetic is
fixed by its source (torch's division of an fp32 tensor by a host scalar is a
multiplication by the fp32 reciprocal; comparisons against a Python float are
done in fp32), the CUDA form is restated.  Where the reference's result depends
on an unspecified accumulation order (cuBLAS, cuFFT, torch's tree reductions),
this module accumulates in float64 and rounds once, so it sits within one
rounding of any order.

Parity pins (what checks each function against something other than itself):
  rotary_embedding         -- transformers' apply_rotary_pos_emb (the function the
                              reference's patched forward calls) on CPU tensors,
                              bit for bit; cos = 1 / sin = 0 and cos = 0 / sin = 1
                              closed forms
  block_mean_pool          -- brute force over tokens; closed form on constant blocks
  fft_lag_correlation      -- brute-force diagonal sums of Q_b K_b^T (O(N^2 D));
                              post-processing checked on hand-built inputs
  correlation_keep         -- closed form (threshold of max-normalised values)
  correlation_keep_topk    -- hand-computed linear-interpolation quantiles and
                              numpy.quantile (the "topk" selection mode)
  block_scores             -- numpy float64 GEMM
  stripe_variance          -- numpy unbiased variance on torch.diagonal slices;
                              constant / linear diagonals (closed forms)
  qk_topk_rows             -- sort-based brute force per row
  column_scores/_select    -- brute-force suffix sums; sort-based top-n
  last_row_topk            -- sort-based brute force
  select_mask              -- invariants (causal, diagonal kept, sink columns,
                              monotone in corr_threshold, full diagonals per lag)
  block_sparse_attention   -- torch scaled_dot_product_attention (fp32) with
                              the token-expanded boolean mask
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

F32 = np.float32


def _f32(x: float) -> float:
    """Round a Python float to the nearest fp32 value (torch casts a Python
    scalar to the tensor's fp32 dtype before comparing / multiplying)."""
    return float(np.float32(x))


# ---------------------------------------------------------------------------
# Parameter derivation: my_attn_v7.py:533-540 (block counts, prior),
# :563 (correlation gate), :579-585 (remote start, diagonal samples),
# :316-332 (sampled lags), :626-634 + :422-432 (column range / count).
# ---------------------------------------------------------------------------
@dataclass
class V7Params:
    L_q: int
    L_k: int
    bs: int
    N: int                  # q_block_num (== k_block_num for prefill)
    Nk: int
    keep_sink: int
    keep_recent: int
    local_window: int
    corr_enabled: bool      # the corr/stripe branch (:567) runs
    exclude_tau_fft: int    # batch_fft_cross_correlation exclude (= lw + 1), :138
    sink_tau_start: int     # N - keep_sink - 5 (may be negative), :139
    remote_start: int       # max(lw, keep_recent - 1) + 1, :183-184 / :579-580
    sample_taus: list = field(default_factory=list)
    stripe_all_diffuse: bool = False   # remote_start >= N - 1 path, :316-319
    col_enabled: bool = False          # :623 minus the num_stripe>0 test
    col_start: int = 0
    col_end: int = 0
    n_cols: int = 0
    last_k: int = 0


def derive_params(L_q, L_k, block_size=128, sink_ratio=0.1, recent_ratio=0.1,
                  local_span_ratio=0.1, enable_correlation_mask=True,
                  correlation_topk_ratio=0.2, enable_column_mask=True,
                  column_topk_ratio=0.1, column_start_exclude_ratio=0.1,
                  column_end_exclude_ratio=0.2, enable_last_block_mask=True,
                  diag_sample_ratio=0.15, min_diag_samples=5,
                  max_diag_samples=64) -> V7Params:
    bs = block_size
    q_block_num = (L_q + bs - 1) // bs                       # :533
    k_block_num = (L_k + bs - 1) // bs                       # :534
    keep_sink = max(1, int(k_block_num * sink_ratio))        # :537
    keep_recent = max(1, int(k_block_num * recent_ratio))    # :538
    local_span = max(2, int(k_block_num * local_span_ratio))  # :539
    lw = local_span // 2                                     # :540
    correlation_top_k = max(1, int(q_block_num * correlation_topk_ratio))  # :563
    corr_enabled = bool(enable_correlation_mask and q_block_num > correlation_top_k)
    N = q_block_num
    p = V7Params(L_q=L_q, L_k=L_k, bs=bs, N=N, Nk=k_block_num,
                 keep_sink=keep_sink, keep_recent=keep_recent, local_window=lw,
                 corr_enabled=corr_enabled, exclude_tau_fft=lw + 1,
                 sink_tau_start=N - keep_sink - 5,
                 remote_start=max(lw, keep_recent - 1) + 1)
    if corr_enabled:
        rs = p.remote_start
        num_remote_diags = max(1, (q_block_num + rs) // 2 - rs + 1)          # :583
        nds = int(num_remote_diags * diag_sample_ratio)                      # :584
        nds = max(min_diag_samples, min(nds, max_diag_samples))              # :585
        if rs >= N - 1:                                                      # :316
            p.stripe_all_diffuse = True
        else:
            max_tau = (N + rs) // 2                                          # :322
            num_available = max(1, max_tau - rs + 1)                         # :325
            actual = min(nds, num_available)                                 # :326
            if actual <= 1:                                                  # :328
                p.sample_taus = [rs]
            else:
                idx = torch.linspace(0, num_available - 1, actual).long()    # :331
                p.sample_taus = (idx + rs).tolist()                          # :332
    p.col_enabled = bool(enable_column_mask and q_block_num > 1)             # :623
    if p.col_enabled:
        col_ratio_scale = min(1.0, (128.0 / N) ** 0.5)                       # :626
        ratio = column_topk_ratio * col_ratio_scale                          # :627
        cs = max(1, int(q_block_num * column_start_exclude_ratio))           # :633
        ce_off = max(1, int(q_block_num * column_end_exclude_ratio))         # :634
        ce = N - ce_off                                                      # :423
        p.col_start, p.col_end = cs, ce
        if ce > cs:                                                          # :425
            nvalid = ce - cs
            tk = max(1, int(nvalid * ratio))                                 # :431
            p.n_cols = min(tk, nvalid)                                       # :432
    p.last_k = min(128, N) if enable_last_block_mask else 0                  # :66
    return p


# ---------------------------------------------------------------------------
# Stage functions
# ---------------------------------------------------------------------------
def to_lhd(x: torch.Tensor) -> torch.Tensor:
    """[1,H,L,D] -> [L,H,D] (my_attn_v7.py:528-530)."""
    return x.squeeze(0).transpose(0, 1)


def rotary_embedding(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """The RoPE step before the path: eval/LongBench/pred.py:195 applies
    transformers' apply_rotary_pos_emb (models/llama/modeling_llama.py
    rotate_half / apply_rotary_pos_emb) to q and k:
        out = x * cos + rotate_half(x) * sin,  rotate_half(x) = cat(-x[..., D/2:], x[..., :D/2]).
    Each elementwise op runs in x's dtype, i.e. is formed in fp32 and rounded
    once to the dtype (fp32 inputs: plain fp32 ops, no fused multiply-add).
    x [..., L, D]; cos / sin [L, D] in x's dtype -> x's shape and dtype."""
    D = x.shape[-1]
    xf, c, s = x.float(), cos.float(), sin.float()
    rot = torch.cat([-xf[..., D // 2:], xf[..., :D // 2]], dim=-1)
    a = (xf * c).to(x.dtype).float()
    b = (rot * s).to(x.dtype).float()
    return (a + b).to(x.dtype)


def block_mean_pool(x: torch.Tensor, bs: int) -> torch.Tensor:
    """my_attn_v7.py:105-114.  x [L,H,D] -> [N,H,D] in x's dtype.

    Zero-pad to N*bs tokens, mean over each block of bs tokens (the divisor is
    bs even for a partial last block).  The block sum is accumulated in
    float64, scaled by 1/bs, rounded to fp32 and then to the input dtype (the
    reference reduces in fp32 and casts the fp32 mean to the input dtype)."""
    L, H, D = x.shape
    N = (L + bs - 1) // bs
    xd = x.double()
    pad = N * bs - L
    if pad:
        xd = torch.cat([xd, xd.new_zeros(pad, H, D)], 0)
    s = xd.view(N, bs, H, D).sum(1)
    m = (s * (1.0 / bs)).float()
    return m.to(x.dtype)


def fft_lag_correlation(Q_b: torch.Tensor, K_b: torch.Tensor, local_window: int,
                        keep_sink: int):
    """my_attn_v7.py:117-157 (batch_fft_cross_correlation), float32 FFT on CPU.

    Returns (corr_causal [H,N], corr_causal_sum [H,N])."""
    N, H, D = Q_b.shape
    Q_t = Q_b.permute(1, 2, 0).contiguous().float()               # :122
    K_t = K_b.permute(1, 2, 0).contiguous().float()               # :123
    n = 2 * N                                                     # :125
    Qf = torch.fft.rfft(Q_t, n=n, dim=-1)                         # :126
    Kf = torch.fft.rfft(K_t, n=n, dim=-1)                         # :127
    corr_sum = torch.fft.irfft(Qf * torch.conj(Kf), n=n, dim=-1).sum(dim=1)[:, :N]  # :129-132
    return postprocess_corr(corr_sum, local_window, keep_sink), corr_sum


def postprocess_corr(corr_sum: torch.Tensor, local_window: int, keep_sink: int) -> torch.Tensor:
    """my_attn_v7.py:134-155 on a raw lag-sum [H,N] (fp32)."""
    H, N = corr_sum.shape
    tau = torch.arange(N).float()                                 # :134
    num_pairs = (N - tau).clamp(min=1)                            # :135
    corr = corr_sum / num_pairs.unsqueeze(0)                      # :136
    ex = local_window + 1                                         # :138
    st = N - keep_sink - 5                                        # :139
    corr[:, :ex] = 0                                              # :140
    corr[:, st:] = 0                                              # :141
    if ex < st:                                                   # :144
        valid = corr[:, ex:st]
        corr[:, ex:st] = valid - valid.min(dim=-1, keepdim=True).values   # :146-147
        vt = tau[ex:st]                                           # :151
        vnp = (N - vt).clamp(min=1)                               # :152
        pw = torch.log10(vnp) / torch.log10(vnp.max()).clamp(min=1e-6)    # :153
        corr[:, ex:st] = corr[:, ex:st] * pw.unsqueeze(0)         # :154
    return corr


def correlation_keep(corr: torch.Tensor, remote_start: int, corr_threshold: float):
    """my_attn_v7.py:190-208 (threshold mode).  Returns (keep [H,N] over lags
    tau, normalised value [H,N]); entries tau < remote_start are False / nan."""
    H, N = corr.shape
    keep = torch.zeros(H, N, dtype=torch.bool)
    norm = torch.full((H, N), float("nan"))
    if remote_start >= N:
        return keep, norm
    cr = corr[:, remote_start:]                                   # :193
    cmax = cr.max(dim=-1, keepdim=True).values.clamp(min=1e-6)    # :206
    nv = cr / cmax                                                # :207
    keep[:, remote_start:] = nv >= _f32(corr_threshold)           # :208
    norm[:, remote_start:] = nv
    return keep, norm


def correlation_keep_topk(corr: torch.Tensor, remote_start: int, topk_ratio: float):
    """my_attn_v7.py:196-203 ("topk" selection mode): keep lags whose value is
    >= the (1 - topk_ratio) quantile (linear interpolation) of the remote lags."""
    H, N = corr.shape
    keep = torch.zeros(H, N, dtype=torch.bool)
    if remote_start >= N:
        return keep, None
    cr = corr[:, remote_start:]
    q = torch.quantile(cr.float(), 1.0 - topk_ratio, dim=-1, keepdim=True)
    keep[:, remote_start:] = cr >= q
    return keep, q.squeeze(-1)


def block_scores(Q_b: torch.Tensor, K_b: torch.Tensor) -> torch.Tensor:
    """my_attn_v7.py:234-249.  fp32 Q_b K_b^T / sqrt(D), [H,N,N].

    The dot products are accumulated in float64 and rounded to fp32; the
    scale is applied as a multiplication by the fp32 reciprocal of
    float(D ** 0.5), which is how torch divides a CUDA fp32 tensor by a
    host scalar."""
    N, H, D = Q_b.shape
    q = Q_b.permute(1, 0, 2).double()
    k = K_b.permute(1, 0, 2).double()
    raw = torch.bmm(q, k.transpose(1, 2)).float()
    inv = np.float32(1.0) / np.float32(D ** 0.5)
    return raw * float(inv)


def stripe_variance(scores: torch.Tensor, remote_start: int, sample_taus, stripe_threshold: float,
                    all_diffuse: bool):
    """my_attn_v7.py:301-363.  Returns (mean_var [H] fp32, is_stripe [H])."""
    H, N, _ = scores.shape
    if all_diffuse:                                               # :316-319
        return torch.full((H,), float("inf")), torch.zeros(H, dtype=torch.bool)
    vals = []
    for tau in sample_taus:                                       # :342
        dv = torch.diagonal(scores, offset=-tau, dim1=1, dim2=2)[:, :-1].double()  # :343-345
        diff = dv[:, 1:] - dv[:, :-1]                             # :346
        var = diff.var(dim=-1)                                    # :347 (unbiased)
        dm = dv.abs().mean(dim=-1).float()
        dm = torch.where(dm < 1e-6, torch.full_like(dm, 1e-6), dm)  # clamp(min=1e-6), nan kept
        vals.append(var.float() / dm)                             # :349
    mean_var = torch.stack(vals, -1).double().mean(-1).float()    # :359-360
    is_stripe = mean_var <= _f32(stripe_threshold)                # :363
    return mean_var, is_stripe


def qk_k_per_row(N: int, qk_topk_ratio: float) -> torch.Tensor:
    """my_attn_v7.py:271-272: trunc(fp32(i+1) * fp32(ratio)), clamped >= 1."""
    vis = torch.arange(1, N + 1).float()
    return (vis * _f32(qk_topk_ratio)).long().clamp(min=1)


def qk_topk_rows(scores: torch.Tensor, qk_topk_ratio: float):
    """my_attn_v7.py:256-294.  Row i keeps its top-k_i causal scores.

    Returns (mask [H,N,N], kth value per row [H,N]).  Among equal scores the
    lower column index is taken first (the reference's torch.topk leaves the
    order of ties unspecified)."""
    H, N, _ = scores.shape
    kpr = qk_k_per_row(N, qk_topk_ratio)
    mask = torch.zeros(H, N, N, dtype=torch.bool)
    kth = torch.empty(H, N)
    for i in range(N):
        k = int(kpr[i])
        row = scores[:, i, : i + 1]
        # stable descending sort: ties keep ascending column order
        order = torch.sort(row, dim=-1, descending=True, stable=True).indices[:, :k]
        mask[torch.arange(H)[:, None], i, order] = True
        kth[:, i] = torch.gather(row, 1, order[:, -1:]).squeeze(1)
    return mask, kth


def column_scores(Q_b: torch.Tensor, K_b: torch.Tensor) -> torch.Tensor:
    """my_attn_v7.py:401-420.  col_mean [H,N] fp32.

    partial[j] = sum_{i=j}^{N-2} Q_b[i] via total-minus-prefix as in the
    reference (fp32 cumsum, sequential on the CPU), partial[N-1] = 0; then
    (partial . K_b[j]) * fp32(1/sqrt(D)) / max(1, N-j-1)."""
    N, H, D = Q_b.shape
    Q_t = Q_b.permute(1, 0, 2).contiguous().float()
    K_t = K_b.permute(1, 0, 2).contiguous().float()
    Qc = Q_t.cumsum(dim=1)                                        # :407
    total = Qc[:, -2, :] if N >= 2 else torch.zeros(H, D)         # :408
    prev = torch.cat([torch.zeros(H, 1, D), Qc[:, :-1, :]], 1)    # :410-412
    partial = total.unsqueeze(1) - prev                           # :413
    partial[:, -1, :] = 0                                         # :414
    dot = (partial.double() * K_t.double()).sum(-1).float()       # :416
    inv = np.float32(1.0) / np.float32(D ** 0.5)
    dot = dot * float(inv)
    cnt = (N - torch.arange(N).float() - 1).clamp(min=1)          # :418-419
    return dot / cnt.unsqueeze(0)                                 # :420


def topk_desc_stable(vals: torch.Tensor, k: int):
    """Top-k indices per row of a [H,M] tensor, descending, ties -> lower index."""
    order = torch.sort(vals, dim=-1, descending=True, stable=True).indices[:, :k]
    kth = torch.gather(vals, 1, order[:, -1:]).squeeze(1)
    return order, kth


def column_select(col_mean: torch.Tensor, p: V7Params):
    """my_attn_v7.py:422-438.  Returns (selected [H,N] bool, n_cols-th value [H])."""
    H, N = col_mean.shape
    sel = torch.zeros(H, N, dtype=torch.bool)
    if p.n_cols <= 0:
        return sel, torch.full((H,), float("nan"))
    cm = col_mean[:, p.col_start:p.col_end]
    order, kth = topk_desc_stable(cm, p.n_cols)
    sel.scatter_(1, order + p.col_start, True)
    return sel, kth


def last_row_scores(Q_b: torch.Tensor, K_b: torch.Tensor) -> torch.Tensor:
    """my_attn_v7.py:61-64.  einsum('hd,nhd->hn') in the input dtype:
    fp32 accumulation (float64 here), result rounded to the input dtype."""
    s = torch.einsum("hd,nhd->hn", Q_b[-1].double(), K_b.double()).float()
    return s.to(Q_b.dtype)


def last_row_topk(Q_b: torch.Tensor, K_b: torch.Tensor, k: int):
    """my_attn_v7.py:54-72.  Returns (selected [H,N], scores [H,N] fp32, kth [H])."""
    s = last_row_scores(Q_b, K_b).float()
    H, N = s.shape
    order, kth = topk_desc_stable(s, k)
    sel = torch.zeros(H, N, dtype=torch.bool)
    sel.scatter_(1, order, True)
    return sel, s, kth


def prior_mask(N: int, Nk: int, keep_sink: int, keep_recent: int, lw: int) -> torch.Tensor:
    """my_attn_v7.py:74-98 for one head: [N,Nk] bool."""
    iq = torch.arange(N)[:, None]
    ik = torch.arange(Nk)[None, :]
    causal = iq >= ik
    m = (ik < keep_sink) | (ik >= Nk - keep_recent)
    if lw > 0:
        m = m | ((iq - ik).abs() <= lw)
    return m & causal


def causal_mask(N: int, Nk: int) -> torch.Tensor:
    """[N,Nk] bool, i >= j (my_attn_v7.py:86, :216, :265, :442)."""
    return torch.arange(N)[:, None] >= torch.arange(Nk)[None, :]


def lag_expand(keep: torch.Tensor, N: int, remote_start: int, keep_sink: int) -> torch.Tensor:
    """my_attn_v7.py:212-225: mask[h,i,j] = keep[h, i-j] for i-j >= rs, j >= keep_sink."""
    iq = torch.arange(N)[:, None]
    ik = torch.arange(N)[None, :]
    tau = iq - ik
    valid = (tau >= remote_start) & (ik >= keep_sink)
    m = keep[:, tau.clamp(0, N - 1)]
    return m & valid.unsqueeze(0)


# ---------------------------------------------------------------------------
# Whole selection (my_attn_v7.py:533-641) with per-block excuse flags.
# ---------------------------------------------------------------------------
@dataclass
class SelectionResult:
    params: V7Params
    Q_b: torch.Tensor
    K_b: torch.Tensor
    mask: torch.Tensor                 # [H,N,N] bool
    excusable: torch.Tensor            # [H,N,N] bool: decided within the band
    corr: torch.Tensor | None = None   # [H,N] post-processed lag correlation
    corr_sum: torch.Tensor | None = None
    corr_norm: torch.Tensor | None = None
    keep_tau: torch.Tensor | None = None
    mean_var: torch.Tensor | None = None
    is_stripe: torch.Tensor | None = None
    col_mean: torch.Tensor | None = None
    col_sel: torch.Tensor | None = None
    last_scores: torch.Tensor | None = None
    last_sel: torch.Tensor | None = None


def _near(x: torch.Tensor, thr: torch.Tensor, rel: float) -> torch.Tensor:
    return (x - thr).abs() <= rel * thr.abs()


def select_mask(q: torch.Tensor, k: torch.Tensor, layer_idx: int = 0, *, block_size=128,
                sink_ratio=0.1, recent_ratio=0.1, local_span_ratio=0.1,
                enable_correlation_mask=True, correlation_selection_mode="threshold",
                correlation_topk_ratio=0.2, corr_threshold=0.1,
                enable_column_mask=True, column_topk_ratio=0.1,
                column_start_exclude_ratio=0.1, column_end_exclude_ratio=0.2,
                enable_last_block_mask=True, diag_sample_ratio=0.15, min_diag_samples=5,
                max_diag_samples=64, stripe_threshold=0.3, qk_topk_ratio=0.2,
                band=1e-3, **_ignored) -> SelectionResult:
    """Block mask of my_attn_v7.myattn_prefill (:533-641) for q [1,Hq,L,D],
    k [1,Hk,L,D] (Hk divides Hq; K heads are repeated as repeat_kv does)."""
    Hq = q.shape[1]
    Hk = k.shape[1]
    g = Hq // Hk
    L_q, L_k = q.shape[2], k.shape[2]
    p = derive_params(L_q, L_k, block_size, sink_ratio, recent_ratio, local_span_ratio,
                      enable_correlation_mask, correlation_topk_ratio, enable_column_mask,
                      column_topk_ratio, column_start_exclude_ratio, column_end_exclude_ratio,
                      enable_last_block_mask, diag_sample_ratio, min_diag_samples,
                      max_diag_samples)
    N = p.N
    H = Hq
    Q_b = block_mean_pool(to_lhd(q), block_size)                              # :554
    K_b = block_mean_pool(to_lhd(k), block_size)                              # :555
    if g > 1:
        K_b = K_b.repeat_interleave(g, dim=1)                                 # repeat_kv
    prior = prior_mask(N, p.Nk, p.keep_sink, p.keep_recent, p.local_window)   # :542-550
    final = prior.unsqueeze(0).expand(H, N, p.Nk).clone()
    exc = torch.zeros(H, N, p.Nk, dtype=torch.bool)
    res = SelectionResult(params=p, Q_b=Q_b, K_b=K_b, mask=final, excusable=exc)

    if enable_last_block_mask:                                                 # :558-560
        sel, sc, kth = last_row_topk(Q_b, K_b, p.last_k)
        final[:, -1, :] |= sel
        exc[:, -1, :] |= _near(sc, kth.unsqueeze(1), band)
        res.last_scores, res.last_sel = sc, sel

    is_stripe = None
    if p.corr_enabled:                                                        # :567
        if p.remote_start >= N:
            # :190-191 returns one tensor; the six-way unpacking at :568 fails.
            raise ValueError("not enough values to unpack (expected 6, got 1)")
        corr, corr_sum = fft_lag_correlation(Q_b, K_b, p.local_window, p.keep_sink)
        if correlation_selection_mode == "threshold":
            keep, norm = correlation_keep(corr, p.remote_start, corr_threshold)
            near_tau = _near(norm, torch.full_like(norm, _f32(corr_threshold)), band)
            near_tau = near_tau & ~torch.isnan(norm)
        elif correlation_selection_mode == "topk":
            keep, qv = correlation_keep_topk(corr, p.remote_start, correlation_topk_ratio)
            norm = None
            near_tau = _near(corr, qv.unsqueeze(1), band)
            near_tau[:, :p.remote_start] = False
        else:
            raise ValueError(f"Unknown selection_mode: {correlation_selection_mode}")
        corr_mask = lag_expand(keep, N, p.remote_start, p.keep_sink)          # :212-225
        corr_exc = lag_expand(near_tau, N, p.remote_start, p.keep_sink)
        scores = block_scores(Q_b, K_b)                                       # :581
        mean_var, is_stripe = stripe_variance(scores, p.remote_start, p.sample_taus,
                                              stripe_threshold, p.stripe_all_diffuse)
        head_near = _near(mean_var, torch.full_like(mean_var, _f32(stripe_threshold)), band)
        res.corr, res.corr_sum, res.corr_norm, res.keep_tau = corr, corr_sum, norm, keep
        res.mean_var, res.is_stripe = mean_var, is_stripe
        if bool((~is_stripe).any()):                                          # :600
            qk_mask, kth = qk_topk_rows(scores, qk_topk_ratio)
            qk_exc = _near(scores, kth.unsqueeze(-1), band) & causal_mask(N, N).unsqueeze(0)
        else:
            qk_mask = torch.zeros(H, N, N, dtype=torch.bool)
            qk_exc = torch.zeros(H, N, N, dtype=torch.bool)
        st = is_stripe.view(H, 1, 1)
        final |= torch.where(st, corr_mask, qk_mask)                          # :606-612
        exc |= torch.where(st, corr_exc, qk_exc)
        # a head whose stripe decision sits in the band may flip as a whole
        exc |= head_near.view(H, 1, 1) & causal_mask(N, N).unsqueeze(0)

    if p.col_enabled and (is_stripe is None or bool(is_stripe.any())):        # :623
        col_mean = column_scores(Q_b, K_b)
        col_sel, kth = column_select(col_mean, p)
        causal = causal_mask(N, N)                                    # :440-445
        cm = col_sel.unsqueeze(1) & causal.unsqueeze(0)
        ce = torch.zeros(H, N, dtype=torch.bool)
        if p.n_cols > 0:
            ce[:, p.col_start:p.col_end] = _near(col_mean[:, p.col_start:p.col_end],
                                                 kth.unsqueeze(1), band)
        cex = ce.unsqueeze(1) & causal.unsqueeze(0)
        if is_stripe is not None:                                             # :636-639
            cm = cm & is_stripe.view(H, 1, 1)
            cex = cex & is_stripe.view(H, 1, 1)
        final |= cm                                                           # :641
        exc |= cex
        res.col_mean, res.col_sel = col_mean, col_sel
    return res


def fixed_mask(N: int, Nk: int, H: int, keep_sink: int, keep_recent: int, lw: int) -> torch.Tensor:
    """attn_src/fix_mask_attn/my_attn.py:39-79: sink | recent | local, with no
    causal AND (the kernel's is_causal drops the blocks above the diagonal)."""
    ik = torch.arange(Nk)
    m = ((ik < keep_sink) | (ik >= Nk - keep_recent))[None, :].expand(N, Nk)
    if lw > 0:
        iq = torch.arange(N)[:, None]
        m = m | ((iq - ik[None, :]).abs() <= lw)
    return m.unsqueeze(0).expand(H, N, Nk).clone()


# ---------------------------------------------------------------------------
# Stage 2: block-sparse attention (the block_sparse_attn_func role,
# my_attn_v7.py:775-786) and the dense fallback (:509-519).
# ---------------------------------------------------------------------------
def block_sparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: torch.Tensor,
                           bs: int, is_causal: bool = True, heads=None, qblocks=None) -> torch.Tensor:
    """fp32 attention of q [1,Hq,L,D] over k/v [1,Hk,L,D] where query token t
    sees key s iff block (t//bs, s//bs) is set in mask[h] (and s <= t when
    causal).  Returns [L,Hq,D] fp32 (rows of heads/qblocks not requested are 0).

    The block loop visits only the selected key blocks of each query block."""
    Hq, L, D = q.shape[1], q.shape[2], q.shape[3]
    Hk = k.shape[1]
    g = Hq // Hk
    N = (L + bs - 1) // bs
    scale = 1.0 / math.sqrt(D)
    out = torch.zeros(L, Hq, D)
    heads = range(Hq) if heads is None else heads
    qblocks = range(N) if qblocks is None else qblocks
    for h in heads:
        qh = q[0, h].float()
        kh = k[0, h // g].float()
        vh = v[0, h // g].float()
        for i in qblocks:
            t0, t1 = i * bs, min(L, (i + 1) * bs)
            cols = torch.nonzero(mask[h, i]).flatten().tolist()
            if not cols:
                continue
            kidx = torch.cat([torch.arange(j * bs, min(L, (j + 1) * bs)) for j in cols])
            s = (qh[t0:t1] @ kh[kidx].T) * scale
            if is_causal:
                s = s.masked_fill(kidx[None, :] > torch.arange(t0, t1)[:, None], float("-inf"))
            pr = torch.softmax(s, dim=-1)
            pr = torch.nan_to_num(pr, nan=0.0)
            out[t0:t1, h] = pr @ vh[kidx]
    return out


def dense_causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Dense causal fp32 attention (flash_attn_func(causal=True) role,
    my_attn_v7.py:509-519), bottom-right aligned when L_q < L_k.
    q [B,Hq,Lq,D], k/v [B,Hk,Lk,D] -> [B,Lq,Hq,D]."""
    B, Hq, Lq, D = q.shape
    Hk, Lk = k.shape[1], k.shape[2]
    g = Hq // Hk
    kk = k.float().repeat_interleave(g, 1)
    vv = v.float().repeat_interleave(g, 1)
    s = q.float() @ kk.transpose(-1, -2) / math.sqrt(D)
    off = Lk - Lq
    bad = torch.arange(Lk)[None, :] > (torch.arange(Lq)[:, None] + off)
    s = s.masked_fill(bad, float("-inf"))
    o = torch.softmax(s, -1) @ vv
    return o.transpose(1, 2)
