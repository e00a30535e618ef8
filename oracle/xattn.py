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

The other paths of xattn_estimate, restated in ``estimate``:
  - causal=False on the Triton path: the softmax over every key of the
    chunk-padded sequence (Xattention.py:36-55: Q and K zero-padded to whole
    chunks; kernels.py:98-156 normalises over all of them), and
    find_blocks_chunked's non-causal branch (utils.py:163-188: no forced
    blocks, every block sorted, and block 0 always marked because unselected
    positions scatter to index 0);
  - use_triton=False (Xattention.py:72-135, 170-258): the reshapings
    "inverse" (with kdb), "slash", "random", "double", "triple"; scores from a
    matmul in the input dtype, divided by sqrt(D), S and norm in that dtype; the
    causal mask (the kdb-subsampled rows take mask rows kdb-1, 2kdb-1, ...; the
    padding-column marks are overwritten by each chunk's own square);
    softmax in float32 (or exp when softmax=False) rounded to the input dtype;
    padded query rows zeroed; block sums as two sums in the input dtype (over a
    block's keys, then its rows).

Accumulation orders the reference leaves to Triton (the GEMM's and the block
sums' fp32 reductions) are done here in float64 and rounded once; torch.sort's
order among equal values is unspecified, and ties are broken here by the lower
block index.

Parity pins (tests/test_oracle_xattn.py):
  reshaped_scores   -- brute force over token pairs (antidiagonal sums of q k^T)
  block_sums        -- softmax rows sum to one; brute-force block sums
  select_blocks     -- hand-built rows with closed-form selections; the sorted
                       cumulative rule checked against a direct greedy loop
  general_scores    -- every reshaping against sums of the token score matrix
                       over the permutation's entries (double / triple: the
                       neighbouring-key sums); kdb rows equal every kdb-th row
  estimate          -- the Triton causal path equals xattn_mask; probabilities
                       of every real row sum to one over the chunk-padded keys
                       (non-causal) or its visible keys; softmax=False gives
                       exp of the scaled scores; the non-causal selection on
                       closed-form rows, block 0 kept; default_chunk_size's
                       closed forms
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


# ---- the other paths of xattn_estimate ---------------------------------------

def default_chunk_size(k_len: int) -> int:
    """Xattention_prefill's chunk_size when none is given (Xattention.py:326-335):
    the next power of two of k_len, clamped to [2048, 2^28 / that power]."""
    p = 1 << (k_len - 1).bit_length()
    return int(max(min(max(2048, p), 128 * 1024 * 2048 // p), 2048))


def query_order(select_mode: str, stride: int, perm=None):
    """The token offset within a stride group that query chunk i takes
    (Xattention.py:74-135): "inverse" / "" and "double" / "triple" reverse the
    group (S-1-i), "slash" keeps it (i), "random" takes perm[i]."""
    if select_mode in ("inverse", "", "double", "triple"):
        return [stride - 1 - i for i in range(stride)]
    if select_mode == "slash":
        return list(range(stride))
    if select_mode == "random":
        return [int(x) for x in perm]
    raise ValueError(f"unknown select_mode {select_mode!r}")


def reshaped_keys(k: torch.Tensor, Lp: int, stride: int, select_mode: str) -> torch.Tensor:
    """K' [Hk, Lp/S, S, D] (values of k's dtype, as float64): chunk j of
    reshaped key n is k[nS + j] (zero past L); "double" adds chunk j + 1 (mod S),
    "triple" then adds the doubled chunk j - 1 (mod S), each sum rounded to the
    dtype as the reference's tensor additions are (Xattention.py:103-135)."""
    _, Hk, L, D = k.shape
    kp = torch.zeros(Hk, Lp, D, dtype=torch.float64)
    kp[:, :L] = k[0].double()
    R = kp.view(Hk, Lp // stride, stride, D)
    if select_mode in ("double", "triple"):
        R = round_to(R + R.roll(-1, dims=2), k.dtype).double()
        if select_mode == "triple":
            R = round_to(R + R.roll(1, dims=2), k.dtype).double()
    return R


def general_scores(q: torch.Tensor, k: torch.Tensor, *, stride: int, Lp: int, select_mode: str = "inverse",
                   kdb: int = 1, perm=None) -> torch.Tensor:
    """Reshaped scores A [H, Lp/(S kdb), Lp/S] rounded to the input dtype (as
    float32).  Query row m takes the tokens m*QS + order[i], QS = S*kdb for
    "inverse" (its reshaping strides by S*kdb) and S for the other modes (which
    ignore kdb when reshaping; the kdb-th rows are then sliced by position,
    Xattention.py:172-178); key n the chunks of reshaped_keys."""
    _, H, L, D = q.shape
    S = stride
    g = H // k.shape[1]
    order = query_order(select_mode, S, perm)
    QS = S * kdb if select_mode in ("inverse", "") else S
    nq = Lp // (S * kdb)
    qp = torch.zeros(H, Lp + QS, D, dtype=torch.float64)
    qp[:, :L] = q[0].double()
    Qr = torch.stack([qp[:, torch.arange(nq) * QS + o] for o in order], dim=2)   # [H, nq, S, D]
    Kr = reshaped_keys(k, Lp, S, select_mode).repeat_interleave(g, 0)             # [H, Lp/S, S, D]
    A = torch.einsum("hmsd,hnsd->hmn", Qr, Kr)
    return round_to(A, q.dtype)


def _visible(nq: int, nk: int, *, causal: bool, kdb: int, own_chunk: int = 0) -> torch.Tensor:
    """[nq, nk] keys a query row may attend: causal row m sees keys
    n <= m*kdb + kdb - 1 (the mask row the kdb-th slice takes); own_chunk > 0:
    only keys from the start of the row's chunk of own_chunk reshaped rows on
    (see torch_sums)."""
    if not causal:
        return torch.ones(nq, nk, dtype=torch.bool)
    m = torch.arange(nq)[:, None]
    n = torch.arange(nk)[None, :]
    vis = n <= m * kdb + kdb - 1
    if own_chunk:
        vis &= n >= (m * kdb // own_chunk) * own_chunk
    return vis


def triton_sums(A: torch.Tensor, L: int, *, stride: int, bs: int, norm: float, head_dim: int,
                causal: bool) -> torch.Tensor:
    """kernels.py:5-156 on A [H, Lr, Lk]: x = A log2(e) / sqrt(D) / S / norm,
    per row the exp2-domain softmax over the keys it sees (causal: n <= r;
    non-causal: every key of the padded sequence), rows at or past ceil(L/S)
    zero, summed over (bs/S) x (bs/S) squares in float64, rounded to the
    input dtype by the caller."""
    H, Lr, Lk = A.shape
    rbs = bs // stride
    real = -(-L // stride)
    x = A.double() * (LOG2E / math.sqrt(head_dim) / stride / norm)
    vis = _visible(Lr, Lk, causal=causal, kdb=1)
    x = x.masked_fill(~vis, float("-inf"))
    e = torch.exp2(x - x.max(-1, keepdim=True).values)
    p = e / e.sum(-1, keepdim=True)
    p[:, real:] = 0
    return p.view(H, Lr // rbs, rbs, Lk // rbs, rbs).sum((2, 4))


def torch_zero_rows(L: int, Lp: int, *, stride: int, chunk_size: int, kdb: int) -> int:
    """Query rows (of the Lp/(S kdb) the torch path keeps) zeroed at the end:
    the last q_reshaped_num_to_pad // kdb (Xattention.py:248-249); when that is
    0 but some reshaped rows are padding, the slice [-0:] zeroes the whole last
    chunk (chunk_size / (S kdb) rows)."""
    pad_r = (Lp - L) // stride
    z = pad_r // kdb
    if z == 0 and pad_r != 0:
        z = chunk_size // stride // kdb
    return z


def torch_sums(A: torch.Tensor, L: int, Lp: int, *, stride: int, bs: int, norm: float, head_dim: int,
               causal: bool, kdb: int, softmax: bool, dtype, chunk_size: int) -> torch.Tensor:
    """Xattention.py:180-258 on A [H, nq, Lk] (the matmul's output in dtype):
    the divisions by sqrt(D), S and norm each rounded to dtype (a division by a
    Python number runs as a multiplication by its float32 reciprocal on the
    GPU), the causal mask, softmax in float32 -- here float64 -- or exp,
    rounded to dtype, the padded query rows zeroed (torch_zero_rows); then a
    sum over each block's keys and one over its rows, each rounded to dtype.
    The causal mask first marks the last k_num_to_pad // S key columns (:205),
    then writes each query chunk's own square upper-triangular (:206-217) over
    them: the padding columns lie in the last chunk, so a row of that chunk sees
    a padding key at or before its mask row (with kdb > 1 some kept rows do).
    When the padding count is 0 the slice [-0:] marks every column and only the
    own square is cleared again, so each row then sees the keys of its own
    chunk only.  Returns [H, Lp/bs, Lk*S/bs] block sums (float32)."""
    H, nq, Lk = A.shape
    S = stride
    rbs = bs // S

    def div(x, v):
        inv = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(v, dtype=torch.float32)
        return round_to(x.float() * inv, dtype)
    x = div(div(div(A, math.sqrt(head_dim)), S), norm).double()
    k_pad_r = (Lp - L) // S                        # k_num_to_pad // stride
    vis = _visible(nq, Lk, causal=causal, kdb=kdb, own_chunk=chunk_size // S if k_pad_r == 0 else 0)
    x = x.masked_fill(~vis, float("-inf"))
    if softmax:
        mx = x.max(-1, keepdim=True).values
        e = torch.exp(x - mx)
        p = e / e.sum(-1, keepdim=True)
    else:
        p = torch.exp(x)
    zero_rows = torch_zero_rows(L, Lp, stride=S, chunk_size=chunk_size, kdb=kdb)
    if zero_rows:
        p[:, nq - zero_rows:] = 0
    p = torch.nan_to_num(round_to(p, dtype).double(), nan=0.0)
    s1 = round_to(p.view(H, nq, Lk // rbs, rbs).sum(-1), dtype).double()          # over the block's keys
    s = s1.view(H, nq // (rbs // kdb), rbs // kdb, Lk // rbs).sum(2)                # over its rows
    return round_to(s, dtype)


def select_rows_noncausal(sums: torch.Tensor, threshold):
    """find_blocks_chunked's non-causal prefill branch (utils.py:163-188) on
    [H, Nq, Nk] sums: every block in decreasing order (ties: lower index
    first) is selected while the mass before it is below total * threshold
    (float64); block 0 is always marked (the unselected positions scatter to
    index 0).  Returns (mask, margin) as select_rows."""
    H, Nq, Nk = sums.shape
    thr = _head_thresholds(threshold, H)
    v = sums.double()
    mask = torch.zeros(H, Nq, Nk, dtype=torch.bool)
    margin = torch.zeros(H, Nq, Nk, dtype=torch.float64)
    for h in range(H):
        for i in range(Nq):
            row = v[h, i]
            req = float(row.sum()) * thr[h]
            order = sorted(range(Nk), key=lambda j: (-float(row[j]), j))
            before = 0.0
            for j in order:
                margin[h, i, j] = (before / req - 1.0) if req > 0 else math.inf
                if before < req:
                    mask[h, i, j] = True
                before += float(row[j])
            mask[h, i, 0] = True
            margin[h, i, 0] = -math.inf                # kept whatever the masses
    return mask, margin


def estimate(q: torch.Tensor, k: torch.Tensor, *, stride: int, threshold, block_size: int = 128,
             norm: float = 1.0, softmax: bool = True, chunk_size: int = 16384, select_mode: str = "inverse",
             use_triton: bool = True, causal: bool = True, kdb: int = 1, keep_sink: bool = False,
             keep_recent: bool = False, perm=None):
    """xattn_estimate (Xattention.py:14-303) with every path, for L_q == L_k:
    returns (mask [H, N, N] bool, sums [H, N, N] float32 values of the input
    dtype, margin [H, N, N], sums_padded [H, Nqp, Nkp]) with N = ceil(L / bs)
    (the corner Xattention_prefill keeps) and the chunk-padded sums behind the
    selection.  ``perm``: the random mode's permutation (torch.randperm(stride)
    in the reference)."""
    _, H, L, D = q.shape
    if use_triton:
        if kdb != 1:
            raise ValueError("use_triton and kdb cannot be used together")
        select_mode = "inverse"
    Lp = -(-L // chunk_size) * chunk_size
    A = general_scores(q, k, stride=stride, Lp=Lp, select_mode=select_mode, kdb=kdb, perm=perm)
    if use_triton:
        sums = round_to(triton_sums(A, L, stride=stride, bs=block_size, norm=norm, head_dim=D, causal=causal),
                        q.dtype)
    else:
        sums = torch_sums(A, L, Lp, stride=stride, bs=block_size, norm=norm, head_dim=D, causal=causal,
                          kdb=kdb, softmax=softmax, dtype=q.dtype, chunk_size=chunk_size)
    Nb = sums.shape[1]
    if causal:
        mask, margin = select_rows(sums, threshold)
        mask &= torch.tril(torch.ones(Nb, Nb, dtype=torch.bool))
    else:
        mask, margin = select_rows_noncausal(sums, threshold)
    if keep_sink:
        mask[:, 0, :] = True
    if keep_recent:
        mask[:, :, :Nb] |= torch.eye(Nb, dtype=torch.bool)
    N = -(-L // block_size)
    return mask[:, :N, :N], sums[:, :N, :N], margin[:, :N, :N], sums
