"""CPU restatement of FlexPrefill's block selection -- TEST INFRASTRUCTURE ONLY.

The checker for fftsparse_amd's FlexPrefill selector (fs_flex).  Only ``tests/``
and ``bench.py``'s ``cpu_baseline`` leg may import it; the product package
never does.

Restates attn_src/Flexprefill.py:946-1061 (get_active_blocks) with its helpers
(:873-883 score_cover_topk / score_cover_idx, :886-893 sum_all_diagonal_matrix,
:859-870 torch_bhn_sumpool, :656-782 the average pooling of K, :896-920
transform_veritcal_slash_idx, :939-943 square_root_js_divergence) and the
budget arithmetic of Flexprefill_prefill (:1063-1098), in torch on the CPU:

  last-block scores  qk = (q[-bs:] / sqrt(D)) k^T in the input dtype (the
                     bf16 products accumulated here in float64, rounded once),
                     causal inside the last block, softmax in fp32;
  vertical           mean of qk over the bs rows;  slash: sums of qk along the
                     diagonals ending at each column of the last row, / bs;
  budgets            cover(x) = (number of sorted-descending prefix sums <= gamma) + 1,
                     // 128 + 1, clamped to [min_budget, max_budget] blocks;
  pooled             block sums of vertical / slash; the mean of last_q against
                     the block means of K, softmax; square-root JS divergence to
                     the pooled vertical decides the "sparse" heads (js < tau),
                     which take min_budget blocks each and, in addition, the
                     cover of gamma * N of the block-level attention of the
                     pooled Q against the pooled K (all N x N causal blocks);
  block set          the top pooled vertical columns (column 0 forced) in every
                     row at or after them, the top pooled slash offsets (offset
                     0 forced) as block diagonals, and the sparse heads' cover.

Reductions whose order the reference leaves to CUDA (the bf16 matmul, torch's
sums and cumsums) run here in torch's CPU order; torch.topk / torch.sort's
order among equal values is unspecified, and ties are broken here by the lower
index.

Parity pins (tests/test_oracle_flex.py): the last-block probabilities element
by element in Python floats; diagonal sums and pooling by brute force; the
cover count against a direct greedy count; the top-k with ties against
Python's sort; the sparse heads' block cover against a greedy walk over
sorted entries in float64; the vertical / slash block sets against a direct
construction; JS divergence against scipy.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch


def round_to(x: torch.Tensor, dtype) -> torch.Tensor:
    return x.to(dtype)


def last_block_probs(q: torch.Tensor, k: torch.Tensor, bs: int, gqa_interleave: bool = False):
    """Flexprefill.py:958-984: last_q = q[-bs:] / sqrt(D) (in the input dtype),
    qk = last_q k^T per head (input dtype), the last bs columns causal, softmax
    in fp32.  q [1, L, H, D], k [1, L, Hk, D] -> (p [H, bs, L] fp32, last_q [bs, H, D])."""
    _, L, H, D = q.shape
    Hk = k.shape[2]
    G = H // Hk
    last_q = q[0, -bs:] / math.sqrt(D)
    p = torch.empty(H, bs, L, dtype=torch.float32)
    tri = torch.arange(bs)[:, None] >= torch.arange(bs)[None, :]
    for h in range(H):
        kv = (h % Hk) if gqa_interleave else (h // G)
        s = (last_q[:, h].double() @ k[0, :, kv].double().T).to(q.dtype).float()
        s[:, L - bs:] = s[:, L - bs:].masked_fill(~tri, float("-inf"))
        p[h] = torch.softmax(s, dim=-1)
    return p, last_q


def diagonal_sums(p: torch.Tensor) -> torch.Tensor:
    """Flexprefill.py:886-893 (sum_all_diagonal_matrix): out[x] = sum_i p[i][x + i - (n-1)],
    zero where the column is negative.  p [H, n, m] -> [H, m]."""
    H, n, m = p.shape
    out = torch.zeros(H, m, dtype=p.dtype)
    for i in range(n):
        off = i - (n - 1)                          # column = x + off
        lo = max(0, -off)
        out[:, lo:] += p[:, i, lo + off:m + off]
    return out


def sumpool(x: torch.Tensor, bs: int) -> torch.Tensor:
    """Flexprefill.py:859-870: zero-pad the last dimension to whole blocks, sum each block."""
    H, m = x.shape
    nb = -(-m // bs)
    xp = torch.zeros(H, nb * bs, dtype=x.dtype)
    xp[:, :m] = x
    return xp.view(H, nb, bs).sum(-1)


def cover_count(x: torch.Tensor, gamma: float) -> torch.Tensor:
    """Flexprefill.py:873-876 (score_cover_topk): (number of prefix sums of
    the descending sort that are <= gamma) + 1.  x [H, m] -> int64 [H]."""
    c = torch.cumsum(torch.sort(x, dim=-1, descending=True).values, dim=-1)
    return (c <= gamma).sum(-1) + 1


def mean_pool_k(k: torch.Tensor, bs: int) -> torch.Tensor:
    """Flexprefill.py:656-782 (triton_bnhd_pool, "avg"): the mean over each
    block's real rows (float64 here), in the input dtype.  k [1, L, Hk, D] -> [nb, Hk, D]."""
    _, L, Hk, D = k.shape
    nb = -(-L // bs)
    kd = torch.zeros(nb * bs, Hk, D, dtype=torch.float64)
    kd[:L] = k[0].double()
    cnt = torch.tensor([min(bs, L - j * bs) for j in range(nb)], dtype=torch.float64)
    return (kd.view(nb, bs, Hk, D).sum(1) / cnt[:, None, None]).to(k.dtype)


def js_divergence(p: torch.Tensor, q: torch.Tensor) -> torch.Tensor:
    """Flexprefill.py:939-943 (a zero in p or q gives nan, as there)."""
    m = (p + q) / 2
    return torch.sqrt(0.5 * (p * torch.log(p / m)).sum(-1) + 0.5 * (q * torch.log(q / m)).sum(-1))


def topk_lower_first(x: torch.Tensor, K: int) -> torch.Tensor:
    """Indices of the K largest values of each row, ties by the lower index."""
    H, m = x.shape
    out = torch.empty(H, K, dtype=torch.int64)
    for h in range(H):
        order = sorted(range(m), key=lambda j: (-float(x[h, j]), j))
        out[h] = torch.tensor(order[:K])
    return out


@dataclass
class FlexSelection:
    mask: torch.Tensor          # [H, nb, nb] bool
    num_vertical: torch.Tensor  # [H] blocks
    num_slash: torch.Tensor     # [H]
    js: torch.Tensor            # [H]
    sparse: torch.Tensor        # [H] bool
    vertical: torch.Tensor      # [H, nb] pooled (column 0 set to inf)
    slash: torch.Tensor         # [H, nb] pooled (offset 0 set to inf)
    v_budget_margin: torch.Tensor  # [H] distance of gamma to the nearest prefix sum that changes the vertical budget
    s_budget_margin: torch.Tensor  # [H] (slash)
    cover_attn: torch.Tensor    # [H, nb, nb] sparse heads: the block-level attention the cover is taken over (nan otherwise)
    cover_boundary: torch.Tensor  # [H] sparse heads: the smallest kept value of the cover (nan otherwise)
    vertical_t: torch.Tensor    # [H, L] per-token vertical profile
    slash_t: torch.Tensor       # [H, L] per-token slash profile


def budgets(L: int, bs: int, min_budget=None, max_budget=None):
    """Flexprefill.py:1080-1096: token budgets to block budgets, max clamped to
    the block count (get_active_blocks :958)."""
    nb = -(-L // bs)
    mn = 1 if min_budget is None else min_budget
    mx = 2147483647 if max_budget is None else max_budget
    return math.ceil(mn / bs), min(math.ceil(mx / bs), nb)


def active_blocks(q: torch.Tensor, k: torch.Tensor, bs: int, gamma: float, tau: float = 0.0,
                  min_budget=None, max_budget=None, gqa_interleave: bool = False,
                  profiles=None) -> FlexSelection:
    """Flexprefill.py:946-1061 (get_active_blocks).  q [1, L, H, D], k [1, L, Hk, D].
    ``profiles`` = (vertical_t, slash_t) [H, L] replaces the per-token profiles
    computed from the last block (to apply the rest of the rule to another
    implementation's profiles)."""
    _, L, H, D = q.shape
    Hk = k.shape[2]
    G = H // Hk
    nb = -(-L // bs)
    mnb, mxb = budgets(L, bs, min_budget, max_budget)
    p, last_q = last_block_probs(q, k, bs, gqa_interleave)
    if profiles is None:
        slash_t = diagonal_sums(p) / bs
        vertical_t = p.mean(-2)
    else:
        vertical_t, slash_t = (x.float().cpu() for x in profiles)
    nv = cover_count(vertical_t, gamma) // 128 + 1
    ns = cover_count(slash_t, gamma) // 128 + 1
    v_margin = _budget_margin(vertical_t, gamma)
    s_margin = _budget_margin(slash_t, gamma)
    nv = nv.clamp(min=mnb, max=mxb)
    ns = ns.clamp(min=mnb, max=mxb)
    vertical = sumpool(vertical_t, bs)
    slash = sumpool(slash_t, bs)
    avg_k = mean_pool_k(k, bs)                                   # [nb, Hk, D]
    kv_of = [(h % Hk) if gqa_interleave else (h // G) for h in range(H)]
    lq_mean = last_q.mean(0)                                      # [H, D], input dtype
    avg_qk = torch.stack([(lq_mean[h].double() @ avg_k[:, kv_of[h]].double().T).to(q.dtype).float()
                          for h in range(H)])
    avg_qk = torch.softmax(avg_qk, dim=-1)
    js = js_divergence(avg_qk, vertical)
    sparse = js < tau
    nv[sparse] = mnb
    ns[sparse] = mnb
    vertical[:, :1] = math.inf
    slash[:, -1:] = math.inf
    Ks = min(int(ns.max()), nb)
    Kv = min(int(nv.max()), nb)
    s_idx = (nb - 1) - topk_lower_first(slash, Ks)
    v_idx = topk_lower_first(vertical, Kv)
    mask = torch.zeros(H, nb, nb, dtype=torch.bool)
    rows = torch.arange(nb)
    for h in range(H):
        for p_ in range(Kv):
            v = int(v_idx[h, p_]) if p_ < nv[h] else 0
            mask[h, v:, v] = True                                # rows r >= v
        for p_ in range(Ks):
            s = int(s_idx[h, p_]) if p_ < ns[h] else 0
            r = rows[:nb - s]
            mask[h, r + s, r] = True                             # block (r + s, r)
    cover_attn = torch.full((H, nb, nb), math.nan)
    cover_boundary = torch.full((H,), math.nan)
    for h in torch.nonzero(sparse).flatten().tolist():
        cov, cover_attn[h], cover_boundary[h] = _sparse_cover(q, avg_k[:, kv_of[h]], h, bs, gamma)
        mask[h] |= cov
    mask[:, 0, 0] = True
    return FlexSelection(mask=mask, num_vertical=nv, num_slash=ns, js=js, sparse=sparse,
                         vertical=vertical, slash=slash, v_budget_margin=v_margin, s_budget_margin=s_margin,
                         cover_attn=cover_attn, cover_boundary=cover_boundary, vertical_t=vertical_t,
                         slash_t=slash_t)


def _budget_margin(x: torch.Tensor, gamma: float) -> torch.Tensor:
    """How far gamma lies from changing the block budget n // 128 + 1 of the
    cover count n = #(prefix sums <= gamma) + 1: the distance to the prefix sum
    that would raise n to the next multiple of 128, and to the one that would
    drop it below the current multiple (float64)."""
    c = torch.cumsum(torch.sort(x, dim=-1, descending=True).values, dim=-1).double()
    H, m = c.shape
    n = (c <= gamma).sum(-1) + 1
    out = torch.full((H,), math.inf, dtype=torch.float64)
    for h in range(H):
        up = 128 * (int(n[h]) // 128 + 1) - 2          # index whose prefix sum must be <= gamma to reach it
        down = 128 * (int(n[h]) // 128) - 2            # index whose prefix sum must be > gamma to drop
        if up < m:
            out[h] = min(out[h], float(c[h, up]) - gamma)
        if 0 <= down < m:
            out[h] = min(out[h], gamma - float(c[h, down]))
    return out


def _sparse_cover(q: torch.Tensor, avg_k_h: torch.Tensor, h: int, bs: int, gamma: float) -> torch.Tensor:
    """Flexprefill.py:1038-1060 for one "sparse" head: block means of q (zero
    padded, the last block's mean rescaled to its real rows), the block-level
    causal attention softmax(avg_q / sqrt(D) avg_k^T), flattened, and the
    score_cover_idx (:879-883) of gamma * N: every entry whose descending prefix
    sum is <= gamma * N, plus entry 0.  Returns ([nb, nb] bool, the attention
    [nb, nb], the smallest value kept by the prefix-sum rule)."""
    _, L, H, D = q.shape
    nb = -(-L // bs)
    pad = nb * bs - L
    qd = torch.zeros(nb * bs, D, dtype=torch.float64)
    qd[:L] = q[0, :, h].double()
    avg_q = qd.view(nb, bs, D).mean(1).to(q.dtype)
    if pad:
        last = (avg_q[-1] * bs).to(q.dtype)
        avg_q[-1] = last / (bs - pad)
    s = ((avg_q / math.sqrt(D)).double() @ avg_k_h.double().T).to(q.dtype).float()
    s = s.masked_fill(~torch.tril(torch.ones(nb, nb, dtype=torch.bool)), float("-inf"))
    a = torch.softmax(s, dim=-1).view(-1)
    vals, idx = torch.sort(a, descending=True, stable=True)
    c = torch.cumsum(vals, 0)
    keep = idx[c <= gamma * nb]
    out = torch.zeros(nb * nb, dtype=torch.bool)
    out[keep] = True
    out[0] = True
    n = int((c <= gamma * nb).sum())
    boundary = float(vals[n - 1]) if n > 0 else float(vals[0])
    return out.view(nb, nb), a.view(nb, nb), boundary


def flex_mask(q, k, *, block_size, gamma, tau=0.0, min_budget=None, max_budget=None, gqa_interleave=False):
    """The block mask Flexprefill_prefill (:1063-1098) attends with, [H, nb, nb] bool."""
    return active_blocks(q, k, block_size, gamma, tau, min_budget, max_budget, gqa_interleave)
