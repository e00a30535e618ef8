"""Threshold sweep / target-sparsity calibration (fftsparse_amd.sweep), the
counterpart of eval/efficiency/benchmark_attention_multilayer.py:179-395."""
from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

import fftsparse_amd.sweep as sw
from oracle import v7


@pytest.mark.parametrize("N,rs,sink", [(64, 2, 1), (40, 5, 3), (16, 15, 0)])
def test_corr_retention_equals_the_lag_expanded_mask(N, rs, sink):
    """The closed-form pair count per kept lag equals the oracle's lag
    expansion (my_attn_v7.py:212-225) summed over the mask."""
    g = torch.Generator().manual_seed(N + rs)
    H = 3
    keep = torch.rand(H, N, generator=g) < 0.4
    keep[:, :rs] = False
    sel = SimpleNamespace(params=SimpleNamespace(Nk=N, keep_sink=sink, remote_start=rs),
                          blk_cnt=torch.randint(0, N, (H, N), generator=g, dtype=torch.int32),
                          keep_tau=keep.to(torch.uint8))
    c, f = sw.retention(sel)
    ref = v7.lag_expand(keep, N, rs, sink)
    assert c == pytest.approx(float(ref.sum()) / (H * N * N), abs=1e-12)
    assert f == pytest.approx(float(sel.blk_cnt.sum()) / (H * N * N), abs=1e-12)


@pytest.mark.parametrize("mode,target", [("threshold", 0.3), ("threshold", 0.05), ("topk", 0.12)])
def test_calibrate_bisection_direction_and_stop(monkeypatch, mode, target):
    """Threshold mode: a higher value keeps less; topk mode: more.  The
    search stops within 0.01 of the target (benchmark_attention_multilayer.py:233-253)."""
    calls = []

    def fake(layers, m, val, **kw):
        calls.append(val)
        r = (1.0 - val) ** 2 if m == "threshold" else 0.5 * val
        return r, r / 2

    monkeypatch.setattr(sw, "measure_retention", fake)
    best, c, f = sw.calibrate([None], target, mode)
    assert abs(c - target) < 0.01
    assert len(calls) <= 21


@pytest.mark.gpu
def test_calibrate_reaches_target_on_a_layer():
    dev = torch.device("cuda:0")
    from fftsparse_amd.synth import make_qkv
    q, k, v = make_qkv(16384, 8, 2, seed=9)
    layers = [(q.to(dev), k.to(dev), v.to(dev))]
    kw = {kk: vv for kk, vv in sw.PRODUCTION_KWARGS.items() if kk != "corr_threshold"}
    print("[case] calibrate 16K target 0.05", flush=True)
    best, c, f = sw.calibrate(layers, 0.05, "threshold", **kw)
    assert 0.0 < best < 1.0
    assert abs(c - 0.05) < 0.01
    assert c <= f                     # the final mask contains the stripe heads' lag diagonals and more


@pytest.mark.gpu
def test_sweep_layout_and_monotone_retention():
    dev = torch.device("cuda:0")
    from fftsparse_amd.synth import make_qkv
    q, k, v = make_qkv(16384, 8, 2, seed=10)
    layers = [(q.to(dev), k.to(dev), v.to(dev))]
    kw = {kk: vv for kk, vv in sw.PRODUCTION_KWARGS.items() if kk != "corr_threshold"}
    print("[case] sweep 16K", flush=True)
    res = sw.sweep(layers, [0.5, 0.9, 0.99], "threshold", warmup=1, iters=2, **kw)
    assert res["full"]["time_ms"] > 0
    rows = [res[f"myattn_thres{t}"] for t in (0.5, 0.9, 0.99)]
    for r in rows:
        assert r["selection_mode"] == "threshold" and r["time_ms"] > 0 and 0 < r["density"] <= 1
    assert rows[0]["corr_retention"] >= rows[1]["corr_retention"] >= rows[2]["corr_retention"]
    assert rows[0]["final_retention"] >= rows[2]["final_retention"]
