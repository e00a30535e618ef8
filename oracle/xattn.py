"""CPU restatement of XAttention's block selection -- TEST INFRASTRUCTURE ONLY.

The checker for fftsparse_amd's XAttention selector (fs_xattn).  Only
``tests/`` and ``bench.py``'s ``cpu_baseline`` leg may import it; the product
package never does.

Restates, in torch on the CPU:
  attn_src/xattn/src/Xattention.py:14-303 (xattn_estimate, the Triton path the
  reference's callers use: use_triton=True, select_mode "inverse", kdb 1, causal)
  with its kernels attn_src/xattn/src/kernels.py:195-234
  (flat_group_gemm_fuse_reshape: antidiagonal sums, result in the input dtype)
  and :5-97 (softmax_fuse_block_sum_kernel_causal: exp2-domain softmax over the
  causal reshaped keys, block sums in the input dtype), and
  attn_src/xattn/src/utils.py:44-200 (find_blocks_chunked, causal prefill branch:
  the first and the diagonal block forced, the rest added in decreasing order
  while the mass before them is below threshold x row total, in float64), and
  Xattention.py:278-301 (causal tril, keep_sink, keep_recent).

Accumulation orders the reference leaves to Triton (the GEMM's and the block
sums' fp32 reductions) are done here in float64 and rounded once; torch.sort's
order among equal values is unspecified, and ties are broken here by the lower
block index.

Parity pins (tests/test_oracle_xattn.py):
  reshaped_scores   -- brute force over token pairs (antidiagonal sums of q k^T)
  block_sums        -- softmax rows sum to one; brute-force block sums
  select_blocks     -- hand-built rows with closed-form selections; the sorted
                       cumulative rule checked against a direct greedy loop
"""
from __future__ import annotations

import math

import torch

LOG2E = 1.4426950408889634


def padded_len(L: int, block_size: int) -> int:
    """Token length after padding to whole blocks.  The reference pads to whole
    chunks (Xattention.py:36-40); the padding rows are zero and excluded, and the
    padding keys lie beyond every real row's causal limit, so any padding to a
    multiple of the block size gives the same result for the real blocks."""
    return -(-L // block_size) * block_size


def reshaped_scores(q: torch.Tensor, k: torch.Tensor, stride: int, block_size: int = 128) -> torch.Tensor:
    """kernels.py:195-234 (flat_group_gemm_fuse_reshape, "inverse" mode):
    A[h, r, n] = sum_{j<S} q[h, r S + S-1-j] . k[h, n S + j], accumulated in
    float64 here, rounded to the input dtype (the kernel stores its fp32
    accumulator in the output's dtype).  q [1,H,L,D], k [1,H or Hkv,L,D];
    returns [H, Lr, Lr] float32 (values of the input dtype), Lr = padded L / S."""
    _, H, L, D = q.shape
    g = H // k.shape[1]
    Lp = padded_len(L, block_size)
    S = stride
    Lr = Lp // S
    qp = torch.zeros(H, Lp, D, dtype=torch.float64)
    kp = torch.zeros(k.shape[1], Lp, D, dtype=torch.float64)
    qp[:, :L] = q[0].double()
    kp[:, :L] = k[0].double()
    # Q'[r] = (q[rS+S-1], ..., q[rS]) and K'[n] = (k[nS], ..., k[nS+S-1]) as S*D rows
    qr = qp.view(H, Lr, S, D).flip(2).reshape(H, Lr, S * D)
    kr = kp.view(-1, Lr, S * D).repeat_interleave(g, 0)
    A = qr @ kr.transpose(1, 2)
    return A.float().to(q.dtype).float()


def block_sums(A: torch.Tensor, L: int, stride: int, block_size: int = 128, norm: float = 1.0,
               head_dim: int = 128) -> torch.Tensor:
    """kernels.py:5-97 (softmax_fuse_block_sum_kernel_causal) over the whole
    sequence: x = A * log2(e) / sqrt(D) / S / norm; for reshaped row r the keys
    n <= r; p = exp2(x - max) / sum exp2(x - max) (rows at or past the real
    length ceil(L/S) are zero); block sums over (block/S) x (block/S) squares,
    rounded to the input dtype -- here from float64.  A [H, Lr, Lr] -> [H, Nb, Nb]."""
    H, Lr, _ = A.shape
    S = stride
    rbs = block_size // S
    real = -(-L // S)
    scale = LOG2E / math.sqrt(head_dim) / S / norm
    x = A.double() * scale
    causal = torch.arange(Lr)[None, :] <= torch.arange(Lr)[:, None]
    x = x.masked_fill(~causal, float("-inf"))
    m = x.max(-1, keepdim=True).values
    e = torch.exp2(x - m)
    p = e / e.sum(-1, keepdim=True)
    p[:, real:] = 0
    Nb = Lr // rbs
    s = p.view(H, Nb, rbs, Nb, rbs).sum((2, 4))
    return s


def round_to(x: torch.Tensor, dtype) -> torch.Tensor:
    return x.float().to(dtype).float()


def select_rows(sums: torch.Tensor, threshold):
    """utils.py:44-200 (find_blocks_chunked, causal prefill) on the block sums
    [H, Nb, Nb] (values of the input dtype), for every block row I:
      forced   F = {0, I};  others sorted by value, decreasing (ties: lower index first);
      required = (sum over the row) * threshold   (float64; threshold per head);
      the j-th other is selected iff  sum(F) + (sum of the j larger others) < required.
    Returns (mask [H, Nb, Nb] bool, crossing [H, Nb, Nb] float64): crossing holds,
    for every other block, (mass before it + sum(F)) / required - 1 (its margin to
    the selection threshold; 0 for forced blocks)."""
    H, Nb, _ = sums.shape
    thr = _head_thresholds(threshold, H)
    v = sums.double()
    mask = torch.zeros(H, Nb, Nb, dtype=torch.bool)
    margin = torch.zeros(H, Nb, Nb, dtype=torch.float64)
    for h in range(H):
        for i in range(Nb):
            row = v[h, i]
            total = float(row.sum())
            req = total * thr[h]
            forced = {0, i}
            fs = sum(float(row[j]) for j in forced)
            others = [j for j in range(Nb) if j not in forced]
            others.sort(key=lambda j: (-float(row[j]), j))
            before = fs
            for j in forced:
                mask[h, i, j] = True
            for j in others:
                margin[h, i, j] = (before / req - 1.0) if req > 0 else math.inf
                if before < req:
                    mask[h, i, j] = True
                before += float(row[j])
    return mask, margin


def _head_thresholds(threshold, H):
    """Per-head thresholds as the reference forms them (utils.py:90-105): a
    tensor is cast to float64 and truncated, or padded with its last value, to H
    heads; a Python float applies to every head."""
    if isinstance(threshold, (int, float)):
        return [float(threshold)] * H
    t = torch.as_tensor(threshold).double().flatten()
    if t.numel() >= H:
        t = t[:H]
    else:
        t = torch.cat([t, t[-1:].expand(H - t.numel())])
    return t.tolist()


def xattn_mask(q: torch.Tensor, k: torch.Tensor, *, stride: int, threshold, block_size: int = 128,
               norm: float = 1.0, keep_sink: bool = False, keep_recent: bool = False):
    """xattn_estimate (Xattention.py:14-303) + the slice of Xattention_prefill
    (:389): returns (mask [H, N, N] bool, sums [H, Nb, Nb] in the input dtype as
    float32, margin [H, Nb, Nb]), N = ceil(L / block_size)."""
    L, D = q.shape[2], q.shape[3]
    A = reshaped_scores(q, k, stride, block_size)
    sums = round_to(block_sums(A, L, stride, block_size, norm, D), q.dtype)
    mask, margin = select_rows(sums, threshold)
    Nb = sums.shape[1]
    mask &= torch.tril(torch.ones(Nb, Nb, dtype=torch.bool))
    if keep_sink:
        mask[:, 0, :] = True
    if keep_recent:
        mask |= torch.eye(Nb, dtype=torch.bool)
    N = -(-L // block_size)
    return mask[:, :N, :N], sums, margin
