"""CPU pins of the XAttention oracle (oracle/xattn.py): brute force, closed
forms, and the reference's sort / cumsum formulation of the row selection
written out as tensor operations (a second reading of utils.py:106-160)."""
from __future__ import annotations

import math

import pytest
import torch

from oracle import xattn as xo

G = torch.Generator().manual_seed(4321)


def _rand(*shape, dtype=torch.float32):
    return torch.randn(*shape, generator=G).to(dtype)


@pytest.mark.parametrize("S,L", [(4, 128), (8, 200), (16, 256)])
def test_reshaped_scores_are_antidiagonal_sums(S, L):
    """A[r][n] = sum_j q[rS+S-1-j] . k[nS+j], brute force over token pairs,
    with the zero padding past L (GQA: key head h // 2)."""
    D = 16
    q = _rand(1, 2, L, D, dtype=torch.bfloat16)
    k = _rand(1, 1, L, D, dtype=torch.bfloat16)
    A = xo.reshaped_scores(q, k, S, block_size=64)
    Lr = xo.padded_len(L, 64) // S
    assert A.shape == (2, Lr, Lr)
    qd, kd = q[0].double(), k[0].double()
    for h in range(2):
        for r in (0, 1, Lr // 2, Lr - 1):
            for n in (0, r // 3, r):
                s = 0.0
                for j in range(S):
                    t1, t2 = r * S + S - 1 - j, n * S + j
                    if t1 < L and t2 < L:
                        s += float(qd[h, t1] @ kd[0, t2])
                assert A[h, r, n].item() == float(torch.tensor(s).float().to(torch.bfloat16).float())


def test_block_sums_are_row_softmax_masses():
    """Every real reshaped row's probabilities sum to one over its causal keys,
    so a block row's sums add to its number of real rows; padding rows add
    nothing; blocks above the diagonal are zero; one block equals the sum of
    its rows' direct softmax masses."""
    S, bs, L, D = 4, 32, 100, 16
    q = _rand(1, 1, L, D)
    k = _rand(1, 1, L, D)
    A = xo.reshaped_scores(q, k, S, bs)
    s = xo.block_sums(A, L, S, bs, head_dim=D)
    rbs = bs // S
    real = math.ceil(L / S)
    Nb = s.shape[1]
    for I in range(Nb):
        rows_real = max(0, min(real, (I + 1) * rbs) - I * rbs)
        assert abs(s[0, I].sum().item() - rows_real) < 1e-9
        if I + 1 < Nb:
            assert s[0, I, I + 1:].abs().max().item() == 0
    I, J = 2, 1
    direct = sum(_row_block(A, r, S, D, J, rbs) for r in range(I * rbs, (I + 1) * rbs))
    assert abs(s[0, I, J].item() - direct) < 1e-12


def _row_block(A, r, S, D, J, rbs):
    """Mass of reshaped row r in key block J, from a direct (natural-base) softmax."""
    x = A[0, r, :r + 1].double() / math.sqrt(D) / S
    p = torch.softmax(x, 0)
    return p[J * rbs:(J + 1) * rbs].sum().item()


def test_select_rows_closed_form():
    """Row 4 of five blocks, threshold 0.9: forced blocks 0 and 4 carry 0.55;
    block 2 (0.3) is taken at 0.55 < 0.9, block 1 (0.1) at 0.85 < 0.9, block 3
    is not (0.95)."""
    sums = torch.zeros(1, 5, 5)
    sums[0, 4] = torch.tensor([0.5, 0.1, 0.3, 0.05, 0.05])
    for i in range(4):
        sums[0, i, :i + 1] = 1.0 / (i + 1)
    mask, margin = xo.select_rows(sums, 0.9)
    assert mask[0, 4].tolist() == [True, True, True, False, True]
    assert abs(margin[0, 4, 3] - (0.95 / 0.9 - 1)) < 1e-12
    # threshold 0.5: the forced mass already covers it
    mask, _ = xo.select_rows(sums, 0.5)
    assert mask[0, 4].tolist() == [True, False, False, False, True]


def _reference_form(row: torch.Tensor, i: int, thr: float) -> torch.Tensor:
    """The causal branch of utils.py:106-160 for one row, as tensor ops: forced
    mask, others zeroed and sorted, the [0, forced mass, sorted[:-2]] list, its
    exclusive cumsum against threshold x total, and the selected positions of
    the (forced-first) index order scattered back (ties: lower index first)."""
    nb = row.numel()
    v = row.double()
    forced = torch.zeros(nb, dtype=torch.bool)
    forced[0] = True
    forced[i] = True
    other = v.masked_fill(forced, 0)
    order_vals = torch.where(forced, 100000 * (1 + v), v)
    # descending by value, ascending index among equal values
    idx = sorted(range(nb), key=lambda j: (-float(order_vals[j]), j))
    sorted_other = torch.tensor(sorted(other.tolist(), reverse=True), dtype=torch.float64)
    s = torch.cat([torch.zeros(1, dtype=torch.float64), torch.where(forced, v, 0).sum().view(1), sorted_other[:-2]])
    cws = torch.cat([torch.zeros(1, dtype=torch.float64), s[:-1]]).cumsum(0)
    req = v.sum() * thr
    sel = torch.zeros(nb, dtype=torch.bool)
    sel |= forced
    for p in range(nb):
        if cws[p] < req:
            sel[idx[p]] = True
    return sel


@pytest.mark.parametrize("seed", range(6))
def test_select_rows_matches_reference_form(seed):
    """The greedy reading of the oracle equals the reference's sort / cumsum /
    scatter formulation on random causal rows (distinct values), rows >= 1."""
    g = torch.Generator().manual_seed(seed)
    nb = 24
    sums = torch.zeros(1, nb, nb)
    for i in range(nb):
        sums[0, i, :i + 1] = torch.rand(i + 1, generator=g) ** 3
    thr = [0.5, 0.8, 0.9, 0.95, 0.99, 1.0][seed]
    mask, _ = xo.select_rows(sums, thr)
    for i in range(1, nb):
        ref = _reference_form(sums[0, i], i, thr)
        assert torch.equal(mask[0, i] & (torch.arange(nb) <= i), ref & (torch.arange(nb) <= i)), (i, thr)


def test_head_thresholds_truncate_and_pad():
    assert xo._head_thresholds(0.9, 3) == [0.9] * 3
    t = xo._head_thresholds(torch.tensor([0.5, 0.6, 0.7, 0.8]), 2)
    assert t == [float(torch.tensor(0.5)), float(torch.tensor(0.6))]
    t = xo._head_thresholds([0.5, 0.75], 4)
    assert t == [0.5, 0.75, 0.75, 0.75]


def test_xattn_mask_invariants():
    """Causal; the first and the diagonal block of every row kept; monotone in
    the threshold; keep_sink fills row 0, keep_recent the diagonal."""
    L = 1024
    q = _rand(1, 2, L, 32, dtype=torch.bfloat16)
    k = _rand(1, 2, L, 32, dtype=torch.bfloat16)
    m9, sums, _ = xo.xattn_mask(q, k, stride=8, threshold=0.9, block_size=128)
    m5, _, _ = xo.xattn_mask(q, k, stride=8, threshold=0.5, block_size=128)
    N = m9.shape[1]
    assert not (m9 & ~torch.tril(torch.ones(N, N, dtype=torch.bool))).any()
    assert m9[:, :, 0].all() and m9[:, torch.arange(N), torch.arange(N)].all()
    assert not (m5 & ~m9).any()
    ms, _, _ = xo.xattn_mask(q, k, stride=8, threshold=0.9, block_size=128, keep_sink=True, keep_recent=True)
    assert ms[:, 0].all()
    assert torch.equal(ms[:, 1:], m9[:, 1:])
