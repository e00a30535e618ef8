"""CPU pins of the FlexPrefill oracle (oracle/flex.py): brute force, closed
forms and scipy, each computed a different way from the oracle itself."""
from __future__ import annotations

import math

import pytest
import torch

from oracle import flex as fo

G = torch.Generator().manual_seed(777)


def _rand(*shape, dtype=torch.float32):
    return torch.randn(*shape, generator=G).to(dtype)


def test_diagonal_sums_brute_force():
    """out[x] = sum_i p[i][x + i - (n-1)], by the strided view's definition
    (Flexprefill.py:886-893), checked element by element."""
    p = torch.rand(2, 5, 13, generator=G)
    out = fo.diagonal_sums(p)
    n, m = 5, 13
    for h in range(2):
        for x in range(m):
            s = sum(float(p[h, i, x + i - (n - 1)]) for i in range(n) if x + i - (n - 1) >= 0)
            assert abs(out[h, x].item() - s) < 1e-6
    # the last row's own column lies on every diagonal: a one-hot last row moves to out[x]
    q = torch.zeros(1, 4, 9)
    q[0, 3, 6] = 1.0
    assert fo.diagonal_sums(q)[0].tolist() == [0.0] * 6 + [1.0, 0.0, 0.0]


def test_sumpool_and_cover_count():
    x = torch.tensor([[0.5, 0.1, 0.3, 0.05, 0.05]])
    assert fo.sumpool(x, 2).tolist() == [[pytest.approx(0.6), pytest.approx(0.35), pytest.approx(0.05)]]
    # sorted 0.5 0.3 0.1 0.05 0.05 -> prefix sums 0.5 0.8 0.9 0.95 1.0
    assert fo.cover_count(x, 0.85).item() == 2 + 1
    assert fo.cover_count(x, 0.4).item() == 0 + 1
    y = torch.rand(3, 200, generator=G)
    y /= y.sum(-1, keepdim=True)
    for g in (0.5, 0.9, 0.95):
        c = fo.cover_count(y, g)
        for h in range(3):
            s, n = 0.0, 0
            for v in sorted(y[h].tolist(), reverse=True):
                s += v
                if s <= g:
                    n += 1
            assert c[h].item() in (n + 1, n, n + 2)        # fp32 cumsum vs Python float64
            assert abs(c[h].item() - (n + 1)) <= 1


def test_mean_pool_k_partial_last_block():
    """The last block's mean is over its real rows (triton_bnhd_pool divides by
    cur_block_size_n), not over the block size."""
    k = torch.zeros(1, 10, 1, 2)
    k[0, :, 0, 0] = torch.arange(10, dtype=torch.float32)
    m = fo.mean_pool_k(k, 4)
    assert m[:, 0, 0].tolist() == [1.5, 5.5, 8.5]


def test_js_divergence_matches_scipy():
    scipy = pytest.importorskip("scipy.spatial.distance")
    p = torch.rand(4, 30, generator=G, dtype=torch.float64) + 0.01
    q = torch.rand(4, 30, generator=G, dtype=torch.float64) + 0.01
    p /= p.sum(-1, keepdim=True)
    q /= q.sum(-1, keepdim=True)
    got = fo.js_divergence(p, q)
    for h in range(4):
        assert abs(got[h].item() - scipy.jensenshannon(p[h].numpy(), q[h].numpy())) < 1e-12
    z = p.clone()
    z[0, 3] = 0.0
    assert math.isnan(fo.js_divergence(z, q)[0].item())       # a zero probability gives nan, as in the reference


def test_active_blocks_structure():
    """Causal; block (0,0), column 0 in every row and the diagonal always
    present; every row holds exactly the chosen vertical columns at or before
    it and the chosen slash offsets that fit, for the non-sparse heads; sparse
    heads hold at least that."""
    L, H, Hk, D, bs = 1024, 4, 2, 32, 64
    q = _rand(1, L, H, D, dtype=torch.bfloat16)
    k = _rand(1, L, Hk, D, dtype=torch.bfloat16)
    sel = fo.active_blocks(q, k, bs, gamma=0.9, tau=0.1)
    nb = L // bs
    m = sel.mask
    assert not (m & ~torch.tril(torch.ones(nb, nb, dtype=torch.bool))).any()
    assert m[:, :, 0].all() and m[:, torch.arange(nb), torch.arange(nb)].all()
    for h in range(H):
        Kv = int(sel.num_vertical[h])
        Ks = int(sel.num_slash[h])
        vset = set(fo.topk_lower_first(sel.vertical[h:h + 1], min(Kv, nb))[0].tolist())
        sset = set((nb - 1 - fo.topk_lower_first(sel.slash[h:h + 1], min(Ks, nb))[0]).tolist())
        direct = torch.zeros(nb, nb, dtype=torch.bool)
        for r in range(nb):
            for v in vset:
                if v <= r:
                    direct[r, v] = True
            for s in sset:
                if r - s >= 0:
                    direct[r, r - s] = True
        direct[0, 0] = True
        if bool(sel.sparse[h]):
            assert not (direct & ~m[h]).any()
        else:
            assert torch.equal(direct, m[h]), h


def test_budgets_follow_the_reference_arithmetic():
    assert fo.budgets(4096, 128) == (1, 32)
    assert fo.budgets(4096, 32, min_budget=1024, max_budget=2048) == (32, 64)
    assert fo.budgets(100, 32, max_budget=10 ** 9) == (1, 4)


def test_last_block_probs_brute_force():
    """Flexprefill.py:958-984 element by element in Python floats: scores of the
    scaled last queries (rounded to bf16 at each step the reference rounds),
    the last bs columns causal, softmax per row."""
    L, H, Hk, D, bs = 10, 2, 1, 8, 4
    q = _rand(1, L, H, D, dtype=torch.bfloat16)
    k = _rand(1, L, Hk, D, dtype=torch.bfloat16)
    p, _ = fo.last_block_probs(q, k, bs)
    for h in range(H):
        for i in range(bs):
            t = L - bs + i
            lq = [float(torch.tensor(float(q[0, t, h, d]) / math.sqrt(D)).to(torch.bfloat16)) for d in range(D)]
            s = []
            for c in range(L):
                if c > t:
                    s.append(-math.inf)
                    continue
                dot = sum(lq[d] * float(k[0, c, 0, d]) for d in range(D))
                s.append(float(torch.tensor(dot, dtype=torch.float64).to(torch.bfloat16)))
            m = max(s)
            e = [math.exp(x - m) for x in s]
            z = sum(e)
            for c in range(L):
                assert abs(p[h, i, c].item() - e[c] / z) < 1e-6, (h, i, c)


def test_topk_lower_first_brute_force():
    """The K largest by value, equal values by the lower index: against
    Python's sort of (-value, index) on rows full of ties."""
    x = torch.tensor([[3.0, 1.0, 3.0, 2.0, 3.0, 1.0], [0.5, 0.5, 0.5, 0.5, 0.1, 0.9]])
    assert fo.topk_lower_first(x, 3).tolist() == [[0, 2, 4], [5, 0, 1]]
    y = torch.randint(0, 4, (3, 40), generator=G).float()
    for K in (1, 7, 40):
        got = fo.topk_lower_first(y, K)
        for h in range(3):
            want = sorted(range(40), key=lambda j: (-float(y[h, j]), j))[:K]
            assert got[h].tolist() == want


def test_sparse_cover_rule_brute_force():
    """Flexprefill.py:1038-1060 / score_cover_idx (:879-883): the kept entries
    of the N x N block attention are those whose descending prefix sum (ties by
    the lower flat index) stays <= gamma * N, plus entry 0 -- checked by a
    direct greedy walk over Python-sorted entries in float64."""
    L, H, D, bs, gamma = 96, 1, 16, 16, 0.7
    q = _rand(1, L, H, D, dtype=torch.bfloat16)
    k = _rand(1, L, H, D, dtype=torch.bfloat16)
    avg_k = fo.mean_pool_k(k, bs)
    cov, attn, boundary = fo._sparse_cover(q, avg_k[:, 0], 0, bs, gamma)
    nb = L // bs
    flat = attn.reshape(-1).tolist()
    order = sorted(range(nb * nb), key=lambda j: (-flat[j], j))
    want = set([0])
    run = 0.0
    for j in order:
        run += flat[j]
        if run <= gamma * nb + 1e-6:
            want.add(j)
    got = set(torch.nonzero(cov.reshape(-1)).flatten().tolist())
    assert got == want
    # rows of the block attention are causal softmaxes
    assert torch.allclose(attn.sum(-1), torch.ones(nb), atol=1e-6)
    assert not (attn.triu(1) != 0).any()
