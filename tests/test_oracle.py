"""CPU pins of the oracle (oracle/v7.py) against closed forms, brute force and
invariants -- each check is computed a different way from the oracle itself."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from fftsparse_amd.synth import make_qkv
from oracle import v7
from tests.helpers import PROD, rope_tables

G = torch.Generator().manual_seed(1234)


def _rand(*shape, dtype=torch.float32):
    return torch.randn(*shape, generator=G).to(dtype)


# --------------------------------------------------------------------------- parameters
# Derived integers for the five benchmark shapes (production kwargs of
# eval/efficiency/1_run_eval_multilayer.sh:46-62), worked out by hand from the
# reference formulas (my_attn_v7.py:533-585) independently of oracle/v7.py.
CONFIG_TABLE = [
    # L, bs, N, keep_sink, lw, rs, n_samples, first tau, last tau, cs, ce, n_cols, k_max, last_k
    (8192, 128, 64, 1, 1, 2, 5, 2, 33, 6, 52, 9, 19, 64),
    (32768, 128, 256, 2, 2, 3, 19, 3, 129, 25, 205, 25, 76, 128),
    (131072, 128, 1024, 10, 10, 11, 64, 11, 517, 102, 820, 50, 307, 128),
    (65536, 64, 1024, 10, 10, 11, 64, 11, 517, 102, 820, 50, 307, 128),
    (65536, 128, 512, 5, 5, 6, 38, 6, 259, 51, 410, 35, 153, 128),
]


@pytest.mark.parametrize("row", CONFIG_TABLE)
def test_derived_params_match_config_table(row):
    L, bs, N, ks, lw, rs, ns, t0, t1, cs, ce, nc, kmax, lk = row
    p = v7.derive_params(L, L, bs, sink_ratio=0.01, recent_ratio=0.0, local_span_ratio=0.02,
                         column_topk_ratio=0.2)
    assert (p.N, p.keep_sink, p.local_window, p.remote_start) == (N, ks, lw, rs)
    assert len(p.sample_taus) == ns and p.sample_taus[0] == t0 and p.sample_taus[-1] == t1
    assert (p.col_start, p.col_end, p.n_cols, p.last_k) == (cs, ce, nc, lk)
    assert int(v7.qk_k_per_row(N, 0.3).max()) == kmax
    # linspace(...).long() == floor(i (n-1) / (k-1)) for these shapes
    n_av = (N + rs) // 2 - rs + 1
    assert p.sample_taus == [rs + (i * (n_av - 1)) // (ns - 1) for i in range(ns)]


def test_k_per_row_is_fp32_product_truncated():
    N = 5000
    k = v7.qk_k_per_row(N, 0.3)
    ref = np.maximum(1, np.trunc(np.arange(1, N + 1, dtype=np.float32) * np.float32(0.3))).astype(np.int64)
    assert np.array_equal(k.numpy(), ref)


# --------------------------------------------------------------------------- pooling
# --------------------------------------------------------------------------- rotary embedding
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_rotary_embedding_matches_transformers(dtype):
    """The restatement equals the library function the reference's forward
    calls (transformers apply_rotary_pos_emb), bit for bit, on the projections'
    strided [1, H, L, D] views."""
    pytest.importorskip("transformers")
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    L, D = 1500, 128
    cos, sin = rope_tables(L, D, 500000.0, dtype)
    q = (_rand(1, L, 4, D) * 3).to(dtype).transpose(1, 2)
    k = (_rand(1, L, 2, D) * 3).to(dtype).transpose(1, 2)
    qr, kr = apply_rotary_pos_emb(q, k, cos[None], sin[None])
    assert torch.equal(v7.rotary_embedding(q, cos, sin), qr)
    assert torch.equal(v7.rotary_embedding(k, cos, sin), kr)


def test_rotary_embedding_closed_forms():
    """cos = 1, sin = 0 is the identity; cos = 0, sin = 1 is rotate_half exactly;
    a half-turn (cos = -1) negates."""
    x = _rand(2, 10, 16).to(torch.bfloat16)
    one, zero = torch.ones(10, 16, dtype=torch.bfloat16), torch.zeros(10, 16, dtype=torch.bfloat16)
    assert torch.equal(v7.rotary_embedding(x, one, zero), x)
    assert torch.equal(v7.rotary_embedding(x, zero, one), torch.cat([-x[..., 8:], x[..., :8]], -1))
    assert torch.equal(v7.rotary_embedding(x, -one, zero), -x)


@pytest.mark.parametrize("L,bs", [(1000, 128), (1024, 128), (700, 64)])
def test_block_mean_pool_brute_force(L, bs):
    x = _rand(L, 3, 16)
    out = v7.block_mean_pool(x, bs)
    N = (L + bs - 1) // bs
    for n in range(N):
        s = x[n * bs: min(L, (n + 1) * bs)].double().sum(0)
        torch.testing.assert_close(out[n], (s / bs).float(), rtol=1e-6, atol=1e-7)


def test_block_mean_pool_constant_blocks_exact_bf16():
    x = torch.zeros(300, 2, 8, dtype=torch.bfloat16)
    x[:128] = 1.5
    x[128:256] = -0.25
    x[256:] = 2.0                                   # partial block: 44 tokens, divisor 128
    out = v7.block_mean_pool(x, 128).float()
    assert torch.all(out[0] == 1.5) and torch.all(out[1] == -0.25)
    assert torch.allclose(out[2], torch.full_like(out[2], 2.0 * 44 / 128), rtol=4e-3)


# --------------------------------------------------------------------------- FFT correlation
@pytest.mark.parametrize("N,H,D", [(20, 2, 8), (64, 3, 16), (37, 1, 4)])
def test_fft_lag_sum_equals_diagonal_sums(N, H, D):
    Qb, Kb = _rand(N, H, D), _rand(N, H, D)
    _, corr_sum = v7.fft_lag_correlation(Qb, Kb, 1, 1)
    for h in range(H):
        for t in range(N):
            ref = sum(float(Qb[i, h].double() @ Kb[i - t, h].double()) for i in range(t, N))
            assert abs(float(corr_sum[h, t]) - ref) <= 1e-4 * (1 + abs(ref))


def test_postprocess_closed_forms():
    N, lw, ks = 40, 2, 3
    ex, st = lw + 1, N - ks - 5
    # constant per-pair correlation -> flat band -> zero after the min shift
    c = 0.7
    corr_sum = torch.tensor([[c * (N - t) for t in range(N)]], dtype=torch.float32)
    out = v7.postprocess_corr(corr_sum.clone(), lw, ks)
    assert out.abs().max() < 1e-6
    # a single spike: value (spike / (N - t0) - base) * log10(N - t0) / log10(N - ex)
    base = 0.1
    cs = torch.tensor([[base * (N - t) for t in range(N)]], dtype=torch.float32)
    t0 = 17
    cs[0, t0] += 5.0
    out = v7.postprocess_corr(cs.clone(), lw, ks)
    expect = (5.0 / (N - t0)) * math.log10(N - t0) / math.log10(N - ex)
    assert abs(float(out[0, t0]) - expect) < 1e-5
    assert torch.all(out[0, :ex] == 0) and torch.all(out[0, st:] == 0)
    others = torch.cat([out[0, ex:t0], out[0, t0 + 1:st]])
    assert others.abs().max() < 1e-5


def test_correlation_keep_threshold_semantics():
    corr = torch.tensor([[0.0, 9.0, 1.0, 0.5, 0.9, 0.89, 0.0]])
    keep, norm = v7.correlation_keep(corr, 2, 0.9)
    # max over tau >= 2 is 1.0, so 0.9 and 1.0 pass; tau < 2 never kept
    assert keep[0].tolist() == [False, False, True, False, True, False, False]
    keep_all, _ = v7.correlation_keep(corr, 7, 0.9)
    assert not keep_all.any()


# --------------------------------------------------------------------------- scores / stripes
def test_block_scores_vs_numpy():
    Qb, Kb = _rand(30, 2, 16), _rand(30, 2, 16)
    S = v7.block_scores(Qb, Kb)
    ref = np.einsum("ihd,jhd->hij", Qb.double().numpy(), Kb.double().numpy()) / np.sqrt(16)
    np.testing.assert_allclose(S.numpy(), ref, rtol=1e-6, atol=1e-6)


def test_stripe_variance_closed_forms():
    N, H = 30, 3
    S = torch.zeros(H, N, N)
    i = torch.arange(N)
    # head 0: constant diagonals -> zero variance; head 1: linear along the
    # diagonal -> constant differences -> zero variance; head 2: alternating
    for h in range(H):
        for r in range(N):
            for c in range(r + 1):
                S[h, r, c] = [2.0, 0.5 * c + 1.0, (1.0 if c % 2 else -1.0)][h]
    mv, st = v7.stripe_variance(S, 2, [2, 5, 9], 0.3, False)
    assert float(mv[0]) == 0.0 and float(mv[1]) < 1e-6
    # alternating +-1: n = N-t-2 diffs of +-2 starting at +2, mean m = 2/n for odd n else 0,
    # unbiased var = (4n - n m^2) / (n - 1), mean |x| = 1
    def alt_var(n):
        m = 2.0 / n if n % 2 else 0.0
        return (4 * n - n * m * m) / (n - 1)
    exp = np.mean([alt_var(N - t - 2) for t in (2, 5, 9)])
    assert abs(float(mv[2]) - exp) < 1e-5
    assert st.tolist() == [True, True, False]
    mv2, st2 = v7.stripe_variance(S, 2, [2], 0.3, True)
    assert torch.isinf(mv2).all() and not st2.any()


def test_stripe_variance_matches_numpy_on_random_scores():
    S = _rand(2, 50, 50)
    taus = [3, 10, 20]
    mv, _ = v7.stripe_variance(S, 3, taus, 0.3, False)
    for h in range(2):
        vals = []
        for t in taus:
            d = np.array([float(S[h, j + t, j]) for j in range(50 - t)])[:-1]
            vals.append(np.var(np.diff(d), ddof=1) / max(np.mean(np.abs(d)), 1e-6))
        assert abs(float(mv[h]) - np.mean(vals)) < 1e-5 * (1 + abs(np.mean(vals)))


# --------------------------------------------------------------------------- top-k selections
def test_correlation_keep_topk_closed_forms():
    """my_attn_v7.py:196-203: keep lags >= torch.quantile(corr[rs:], 1 - ratio),
    linear interpolation.  Pinned by hand-computed quantiles and by numpy."""
    corr = torch.tensor([[9.0, 9.0, 0.0, 1.0, 2.0, 3.0, 4.0]])      # remote lags 0..4 (rs = 2)
    keep, q = v7.correlation_keep_topk(corr, 2, 0.2)                   # rank 0.8 * 4 = 3.2 -> 3.2
    assert abs(float(q) - 3.2) < 1e-6
    assert keep.tolist() == [[False, False, False, False, False, False, True]]
    keep, q = v7.correlation_keep_topk(corr, 2, 0.5)                   # rank 2 -> the median, 2
    assert float(q) == 2.0 and keep.tolist() == [[False, False, False, False, True, True, True]]
    keep, q = v7.correlation_keep_topk(corr, 2, 1.0)                   # q = 0: the minimum, all kept
    assert float(q) == 0.0 and keep[0, 2:].all() and not keep[0, :2].any()
    keep, q = v7.correlation_keep_topk(torch.full((1, 6), 5.0), 1, 0.3)  # all equal: all kept
    assert float(q) == 5.0 and keep[0, 1:].all()
    g = torch.Generator().manual_seed(0)
    c = torch.randn(4, 300, generator=g)
    for ratio in (0.2, 0.05, 0.37):
        keep, q = v7.correlation_keep_topk(c, 11, ratio)
        ref = np.quantile(c[:, 11:].double().numpy(), 1 - ratio, axis=-1)
        assert np.allclose(q.double().numpy(), ref, rtol=1e-6, atol=1e-6)
        for h in range(4):
            assert keep[h].sum() == int((c[h, 11:] >= q[h]).sum())


def test_qk_topk_rows_brute_force():
    S = _rand(2, 40, 40)
    mask, kth = v7.qk_topk_rows(S, 0.3)
    kpr = v7.qk_k_per_row(40, 0.3)
    for h in range(2):
        for i in range(40):
            row = S[h, i, : i + 1].numpy()
            k = int(kpr[i])
            order = sorted(range(i + 1), key=lambda j: (-row[j], j))[:k]
            assert set(torch.nonzero(mask[h, i]).flatten().tolist()) == set(order)
            assert float(kth[h, i]) == row[order[-1]]
            assert not mask[h, i, i + 1:].any()


def test_qk_topk_ties_take_lower_index():
    S = torch.zeros(1, 12, 12)                      # all equal
    mask, _ = v7.qk_topk_rows(S, 0.3)
    kpr = v7.qk_k_per_row(12, 0.3)
    for i in range(12):
        assert torch.nonzero(mask[0, i]).flatten().tolist() == list(range(int(kpr[i])))


def test_column_scores_brute_force_suffix_sums():
    N, H, D = 25, 2, 8
    Qb, Kb = _rand(N, H, D), _rand(N, H, D)
    cm = v7.column_scores(Qb, Kb)
    for h in range(H):
        for j in range(N):
            suf = Qb[j: N - 1, h].double().sum(0) if j < N - 1 else torch.zeros(D, dtype=torch.float64)
            ref = float(suf @ Kb[j, h].double()) / math.sqrt(D) / max(1, N - j - 1)
            assert abs(float(cm[h, j]) - ref) <= 1e-5 * (1 + abs(ref))


def test_column_and_last_row_select_brute_force():
    p = v7.derive_params(64 * 128, 64 * 128, 128, sink_ratio=0.01, recent_ratio=0.0,
                         local_span_ratio=0.02, column_topk_ratio=0.2)
    cm = _rand(3, 64)
    sel, kth = v7.column_select(cm, p)
    for h in range(3):
        vals = cm[h, p.col_start:p.col_end].numpy()
        top = sorted(range(len(vals)), key=lambda j: (-vals[j], j))[: p.n_cols]
        assert set(torch.nonzero(sel[h]).flatten().tolist()) == {p.col_start + j for j in top}
    Qb, Kb = _rand(64, 2, 16, dtype=torch.bfloat16), _rand(64, 2, 16, dtype=torch.bfloat16)
    lsel, sc, kth = v7.last_row_topk(Qb, Kb, 10)
    for h in range(2):
        s = [float((Qb[-1, h].double() @ Kb[j, h].double())) for j in range(64)]
        s = [float(torch.tensor(x).to(torch.bfloat16).float()) for x in s]
        top = sorted(range(64), key=lambda j: (-s[j], j))[:10]
        assert set(torch.nonzero(lsel[h]).flatten().tolist()) == set(top)


# --------------------------------------------------------------------------- composed mask
@pytest.fixture(scope="module")
def sel_small():
    q, k, _ = make_qkv(8192, 4, 2, dtype=torch.bfloat16, seed=3)
    return q, k, v7.select_mask(q, k, **PROD)


def test_mask_invariants(sel_small):
    _, _, r = sel_small
    p = r.params
    N = p.N
    causal = torch.arange(N)[:, None] >= torch.arange(N)[None, :]
    assert not (r.mask & ~causal).any()
    assert r.mask[:, torch.arange(N), torch.arange(N)].all()              # diagonal (local window)
    assert r.mask[:, :, : p.keep_sink][:, causal[:, : p.keep_sink]].all()  # sink columns
    # every kept lag of a stripe head yields its full diagonal for j >= keep_sink
    for h in range(r.mask.shape[0]):
        if not r.is_stripe[h]:
            continue
        for t in torch.nonzero(r.keep_tau[h]).flatten().tolist():
            js = torch.arange(p.keep_sink, N - t)
            assert r.mask[h, js + t, js].all()
        for j in torch.nonzero(r.col_sel[h]).flatten().tolist():
            assert r.mask[h, j:, j].all()                                # whole column from the diagonal
        assert r.mask[h, -1][r.last_sel[h]].all()


def test_mask_monotone_in_threshold(sel_small):
    q, k, r = sel_small
    lo = v7.select_mask(q, k, **{**PROD, "corr_threshold": 0.5}).mask
    hi = v7.select_mask(q, k, **{**PROD, "corr_threshold": 0.99}).mask
    assert not (r.mask & ~lo).any() and not (hi & ~r.mask).any()


def test_diffuse_rows_hold_k_i_qk_blocks(sel_small):
    q, k, _ = sel_small
    r = v7.select_mask(q, k, **{**PROD, "stripe_threshold": -1.0})   # every head diffuse
    p = r.params
    kpr = v7.qk_k_per_row(p.N, PROD["qk_topk_ratio"])
    prior = v7.prior_mask(p.N, p.N, p.keep_sink, p.keep_recent, p.local_window)
    S = v7.block_scores(r.Q_b, r.K_b)
    for h in range(r.mask.shape[0]):
        for i in range(p.N - 1):
            dyn = r.mask[h, i] & ~prior[i]
            # blocks outside the prior all come from the row's top-k_i scores
            if dyn.any():
                assert float(S[h, i][dyn].min()) >= float(torch.topk(S[h, i, : i + 1], int(kpr[i])).values[-1])
            assert int(r.mask[h, i].sum()) <= int(prior[i].sum()) + int(kpr[i])


def test_disabled_corr_puts_columns_on_every_head(sel_small):
    q, k, _ = sel_small
    r = v7.select_mask(q, k, **{**PROD, "enable_correlation_mask": False})
    assert r.is_stripe is None and r.col_sel is not None
    for h in range(r.mask.shape[0]):
        for j in torch.nonzero(r.col_sel[h]).flatten().tolist():
            assert r.mask[h, j:, j].all()


# --------------------------------------------------------------------------- attention oracle
def test_block_sparse_attention_matches_sdpa_with_token_mask():
    q, k, v = make_qkv(640, 4, 2, dtype=torch.float32, seed=5)
    N, bs = 5, 128
    mask = torch.rand(4, N, N, generator=G) < 0.5
    mask |= torch.eye(N, dtype=torch.bool)
    out = v7.block_sparse_attention(q, k, v, mask, bs)
    tok = mask.repeat_interleave(bs, 1).repeat_interleave(bs, 2)[:, :640, :640]
    tok &= torch.ones(640, 640, dtype=torch.bool).tril()
    ref = torch.nn.functional.scaled_dot_product_attention(
        q, k.repeat_interleave(2, 1), v.repeat_interleave(2, 1), attn_mask=tok.unsqueeze(0))
    torch.testing.assert_close(out, ref[0].transpose(0, 1), rtol=1e-5, atol=1e-5)


def test_dense_causal_attention_matches_sdpa():
    q, k, v = make_qkv(300, 4, 1, dtype=torch.float32, seed=6)
    out = v7.dense_causal_attention(q, k, v)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k.expand(1, 4, 300, 128),
                                                           v.expand(1, 4, 300, 128), is_causal=True)
    torch.testing.assert_close(out, ref.transpose(1, 2), rtol=1e-5, atol=1e-5)


# --------------------------------------------------------------------------- committed fixtures
def test_c0_selection_matches_committed_fixture():
    """Regression pin: the oracle's config-0 selection (tests/golden/c0_select.npz)."""
    from pathlib import Path
    from fftsparse_amd.synth import make_config, sha256_of
    g = np.load(Path(__file__).resolve().parent / "golden" / "c0_select.npz")
    q, k, v = make_config("c0")
    want = dict(l.split() for l in (Path(__file__).resolve().parent / "golden" / "synth_sha256.txt")
                .read_text().splitlines() if l.strip())
    assert sha256_of(q, k, v) == want["c0_seed0"]
    r = v7.select_mask(q, k, **PROD)
    mask = np.unpackbits(g["mask"], axis=-1)[..., : int(g["shape"][-1])].astype(bool)
    assert np.array_equal(mask, r.mask.numpy())
    assert np.array_equal(g["keep_tau"], r.keep_tau.numpy())
    assert np.array_equal(g["col_sel"], r.col_sel.numpy())
    assert np.array_equal(g["last_sel"], r.last_sel.numpy())
    np.testing.assert_allclose(g["mean_var"], r.mean_var.numpy(), rtol=1e-6)
