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


# ---- the other paths of xattn_estimate (oracle/xattn.py ``estimate``) -------

def _int_qk(L, H, Hk, D=16, seed=0):
    """Small-integer q, k (exact in bf16; their sums and products exact in float64)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-3, 4, (1, H, L, D), generator=g).to(torch.bfloat16)
    k = torch.randint(-3, 4, (1, Hk, L, D), generator=g).to(torch.bfloat16)
    return q, k


@pytest.mark.parametrize("mode", ["inverse", "slash", "random", "double", "triple"])
def test_general_scores_are_token_score_sums(mode):
    """Every reshaping against the token score matrix T = q k^T: A[m][n] =
    sum_i T[m S + o_i][n S + i] (o_i = S-1-i, i, perm[i]); double adds
    T[.][n S + (i+1) % S]; triple adds the (i-1) and (i+1) neighbours and twice
    the key itself -- with integer inputs every sum is exact."""
    S, L, D = 8, 200, 16
    q, k = _int_qk(L, 2, 1, D)
    perm = [3, 0, 7, 1, 6, 2, 5, 4]
    Lp = 256
    A = xo.general_scores(q, k, stride=S, Lp=Lp, select_mode=mode, perm=perm)
    T = torch.zeros(2, Lp + S, Lp + S, dtype=torch.float64)
    T[:, :L, :L] = q[0].double() @ k[0, 0].double().T
    o = {"inverse": [S - 1 - i for i in range(S)], "slash": list(range(S)), "random": perm,
         "double": [S - 1 - i for i in range(S)], "triple": [S - 1 - i for i in range(S)]}[mode]
    w = {"double": {0: 1, 1: 1}, "triple": {-1: 1, 0: 2, 1: 1}}.get(mode, {0: 1})
    for h in range(2):
        for m in (0, 3, 11, Lp // S - 1):
            for n in (0, 5, m):
                s = sum(c * T[h, m * S + o[i], n * S + (i + d) % S] for i in range(S) for d, c in w.items())
                want = float(torch.tensor(float(s)).to(torch.bfloat16).float())
                assert A[h, m, n].item() == want, (mode, h, m, n)


def test_general_scores_kdb_rows():
    """kdb: "inverse" takes every kdb-th reshaped row (its query stride is S kdb);
    the other reshapings keep rows 0, 1, ... (they ignore kdb when reshaping)."""
    q, k = _int_qk(512, 1, 1)
    full = xo.general_scores(q, k, stride=4, Lp=512, select_mode="inverse")
    sub = xo.general_scores(q, k, stride=4, Lp=512, select_mode="inverse", kdb=2)
    assert torch.equal(sub, full[:, ::2])
    full_s = xo.general_scores(q, k, stride=4, Lp=512, select_mode="slash")
    sub_s = xo.general_scores(q, k, stride=4, Lp=512, select_mode="slash", kdb=2)
    assert torch.equal(sub_s, full_s[:, :sub_s.shape[1]])


def test_estimate_triton_causal_equals_xattn_mask():
    q, k, = _rand(1, 2, 700, 32, dtype=torch.bfloat16), _rand(1, 1, 700, 32, dtype=torch.bfloat16)
    m1, s1, g1 = xo.xattn_mask(q, k, stride=8, threshold=0.9)
    m2, s2, g2, _ = xo.estimate(q, k, stride=8, threshold=0.9, chunk_size=2048)
    assert torch.equal(m1, m2) and torch.equal(s1[:, :6, :6], s2) and torch.equal(g1[:, :6, :6], g2)


def test_triton_noncausal_rows_sum_to_one_over_padded_keys():
    """Non-causal: every real reshaped row's probabilities sum to one over all
    keys of the chunk-padded sequence (the padding keys score 0 and take mass),
    so a block row's sums add to its count of real rows; padding rows add none."""
    S, bs, L, D, Lp = 4, 32, 100, 16, 256
    q, k = _rand(1, 1, L, D), _rand(1, 1, L, D)
    A = xo.general_scores(q, k, stride=S, Lp=Lp)
    s = xo.triton_sums(A, L, stride=S, bs=bs, norm=1.0, head_dim=D, causal=False)
    rbs, real = bs // S, math.ceil(L / S)
    for I in range(s.shape[1]):
        rows_real = max(0, min(real, (I + 1) * rbs) - I * rbs)
        assert abs(s[0, I].sum().item() - rows_real) < 1e-9
    # a padding key's probability: exp2(-max) / sum, the same for every padding key of a row
    x = A[0, 0].double() * (xo.LOG2E / math.sqrt(D) / S)
    p = torch.exp2(x - x.max()) / torch.exp2(x - x.max()).sum()
    assert abs(p[-1].item() - p[-2].item()) == 0 and p[-1].item() > 0


def _visible_counts(nq, nk, rbs, kdb, vis):
    """Block sums when every visible probability is 1: the count of visible
    (row, key) pairs per block, rows grouped rbs // kdb at a time."""
    c = vis.double().view(nq, nk // rbs, rbs).sum(-1)
    return c.view(nq // (rbs // kdb), rbs // kdb, nk // rbs).sum(1)


@pytest.mark.parametrize("L,chunk,kdb,causal", [
    (200, 256, 1, True),      # padded: the padding key columns masked, rows past ceil(L/S) zeroed
    (200, 256, 2, True),      # kdb 2: row m sees keys <= 2m + 1
    (256, 128, 1, True),      # no padding: each row sees its own chunk only
    (256, 128, 2, True),
    (200, 256, 1, False),     # non-causal: every key, the padding ones included
    (248, 256, 2, True),      # one padded reshaped row, kdb 2: the [-0:] slice zeroes the last chunk
])
def test_torch_path_visibility_by_counts(L, chunk, kdb, causal):
    """Zero queries and softmax=False: every score is 0 and every visible
    probability exp(0) = 1, so each block sum counts the visible (row, key)
    pairs -- a closed form of the torch path's mask: causal row m sees keys
    n <= m kdb + kdb - 1 below the real keys, or, with no key padding, those of
    its own chunk only; the last q_pad // kdb rows (or, when that is 0, the
    whole last chunk) are zero."""
    S, bs, D = 8, 32, 16
    q = torch.zeros(1, 1, L, D, dtype=torch.bfloat16)
    k = _rand(1, 1, L, D, dtype=torch.bfloat16)
    Lp = -(-L // chunk) * chunk
    A = xo.general_scores(q, k, stride=S, Lp=Lp, kdb=kdb)
    s = xo.torch_sums(A, L, Lp, stride=S, bs=bs, norm=1.0, head_dim=D, causal=causal, kdb=kdb, softmax=False,
                      dtype=torch.bfloat16, chunk_size=chunk)
    nq, nk, rbs = Lp // (S * kdb), Lp // S, bs // S
    vis = _reference_style_visibility(L, Lp, S, chunk, kdb, causal)
    want = _visible_counts(nq, nk, rbs, kdb, vis)
    assert torch.equal(s[0].double(), want)


def _reference_style_visibility(L, Lp, S, chunk, kdb, causal):
    """The torch path's mask built chunk by chunk as Xattention.py:196-249 reads,
    with Python's slice semantics (a slice [-0:] covers everything): per query
    chunk a [rows, keys] mask, the last k_pad // S key columns marked, the
    chunk's own square upper-triangular (above the diagonal), the keys after it
    marked, in the last chunk the last q_pad // kdb rows marked; the kdb-1,
    2kdb-1, ... rows kept; after the softmax the last q_pad // kdb rows of the
    last chunk zeroed.  Returns [rows, keys] bool: visible and not zeroed."""
    rc, nk = chunk // S, Lp // S
    pad = (Lp - L) // S
    n_chunks = Lp // chunk
    out = []
    for c in range(n_chunks):
        m = torch.zeros(rc, nk, dtype=torch.bool)                  # True = masked
        if causal:
            m[:, -pad:] = True
            cs, ce = c * rc, c * rc + rc
            m[:, cs:ce] = torch.triu(torch.ones(rc, rc, dtype=torch.bool), diagonal=1)
            m[:, ce:] = True
            if c == n_chunks - 1 and pad != 0:
                m[-(pad // kdb):, :] = True
            m = m[kdb - 1::kdb]
        else:
            m = m[:rc // kdb]
        vis = ~m
        if c == n_chunks - 1 and pad != 0:
            vis[-(pad // kdb):, :] = False
        out.append(vis)
    return torch.cat(out)


def test_torch_path_uniform_softmax():
    """Zero queries with softmax: each row's probabilities are 1 / (its visible
    key count), rounded to bf16, summed per block in bf16."""
    S, bs, D, L = 4, 32, 16, 128
    q = torch.zeros(1, 1, L, D, dtype=torch.bfloat16)
    k = _rand(1, 1, L, D, dtype=torch.bfloat16)
    A = xo.general_scores(q, k, stride=S, Lp=L)
    s = xo.torch_sums(A, L, L, stride=S, bs=bs, norm=1.0, head_dim=D, causal=False, kdb=1, softmax=True,
                      dtype=torch.bfloat16, chunk_size=L)
    p = float(torch.tensor(1.0 / (L // S)).to(torch.bfloat16))       # one row's probability of a key
    row_block = float(torch.tensor(p * (bs // S)).to(torch.bfloat16))
    want = float(torch.tensor(row_block * (bs // S)).to(torch.bfloat16))
    assert (s[0] == want).all()


def test_select_rows_noncausal_closed_form():
    """Non-causal: blocks in decreasing order while the mass before them is
    below total x threshold; block 0 is marked whatever its mass (unselected
    positions scatter to index 0); ties go to the lower index."""
    sums = torch.tensor([[[0.1, 0.5, 0.3, 0.1], [0.25, 0.25, 0.25, 0.25], [0.0, 0.0, 0.9, 0.1]]])
    mask, margin = xo.select_rows_noncausal(sums, 0.7)
    assert mask[0, 0].tolist() == [True, True, True, False]     # 1 (before 0), 2 (0.5), not 0 by mass (0.8)
    assert mask[0, 1].tolist() == [True, True, True, False]     # 0, 1, 2 (before 0.5 < 0.7), not 3 (0.75)
    assert mask[0, 2].tolist() == [True, False, True, False]    # 2 only by mass, 0 always
    assert margin[0, 0, 3].item() == pytest.approx(0.9 / 0.7 - 1)


def test_default_chunk_size_closed_forms():
    assert [xo.default_chunk_size(n) for n in (100, 4096, 6000, 16384, 131072, 1 << 20)] == \
        [2048, 4096, 8192, 16384, 2048, 2048]
    assert xo.torch_zero_rows(8190, 8192, stride=8, chunk_size=8192, kdb=2) == 0
    assert xo.torch_zero_rows(8184, 8192, stride=8, chunk_size=8192, kdb=2) == 512     # [-0:] quirk
    assert xo.torch_zero_rows(6000, 8192, stride=8, chunk_size=8192, kdb=2) == 137
