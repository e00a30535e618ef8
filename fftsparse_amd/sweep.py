"""Threshold sweep and target-sparsity calibration of the FFTSparse prefill.

Counterpart of the reference's efficiency harness
(eval/efficiency/benchmark_attention_multilayer.py): ``benchmark_multilayer``
(:280-395) times the prefill summed over a set of layers, and
``calibrate_from_qk`` (:179-262) bisects the correlation threshold (or the
"topk" ratio) until the correlation mask keeps a target fraction of the block
mask.  The reference reads that fraction from a collector that only its v4
module fills (``my_attn_v4.py:657-664``), so calibrating the v7 prefill reads
nothing; here the fractions come from the v7 selection itself:

  corr retention  = pairs (h, i, j) of the lag-expanded correlation mask
                    (my_attn_v7.py:212-225: i - j = t kept, t >= remote_start,
                    j >= keep_sink) over H * N * N;
  final retention = selected blocks over H * N * N (the reference's
                    final_mask.numel() denominator).

The results use the reference's layout: {"<L/1024>K": {"full": {"time_ms"},
"<label>": {"time_ms", "selection_mode", "corr_val", ...}}}.

    python -m fftsparse_amd.sweep --lens 32 --layers 2 --thresholds 0.9 0.95 --targets 0.05
"""
from __future__ import annotations

import argparse
import json
import sys

import torch

from .attn import block_sparse_attention, select_blocks, v7_prefill
from .hf import PRODUCTION_KWARGS


def retention(sel) -> tuple[float | None, float]:
    """(corr retention or None without a correlation mask, final retention)
    of a BlockSelection made with ``keep_intermediates=True``."""
    p = sel.params
    H, N = sel.blk_cnt.shape
    total = float(H) * N * p.Nk
    final = float(sel.blk_cnt.sum()) / total
    if sel.keep_tau is None:
        return None, final
    t = torch.arange(N, device=sel.keep_tau.device)
    per_lag = (N - t - p.keep_sink).clamp(min=0) * (t >= p.remote_start)   # pairs on diagonal t
    kept = (sel.keep_tau.to(torch.int64) * per_lag).sum()
    return float(kept) / total, final


def _select_kw(mode: str, val: float, kw: dict) -> dict:
    """Selection settings for one sweep point (benchmark_attention_multilayer.py:196-201):
    threshold mode varies corr_threshold, topk mode varies correlation_topk_ratio."""
    out = {k: v for k, v in kw.items() if k != "block_size"}
    out["correlation_selection_mode"] = mode
    if mode == "threshold":
        out["corr_threshold"] = val
    else:
        out["correlation_topk_ratio"] = val
    return out


def measure_retention(layers, mode: str, val: float, **kw) -> tuple[float, float]:
    """Mean (corr, final) retention over the layers' (q, k) at one setting."""
    bs = kw.get("block_size", 128)
    cs, fs = [], []
    for q, k, *_ in layers:
        sel = select_blocks(q, k, block_size=bs, keep_intermediates=True, **_select_kw(mode, val, kw))
        c, f = retention(sel)
        if c is not None:
            cs.append(c)
        fs.append(f)
    return (sum(cs) / len(cs) if cs else float("nan")), sum(fs) / len(fs)


def calibrate(layers, target: float, mode: str = "threshold", steps: int = 20, tol: float = 0.01, log=None,
              **kw) -> tuple[float, float, float]:
    """Bisection of benchmark_attention_multilayer.py:233-253 on [0, 1]:
    returns (value, corr retention, final retention).  A higher threshold
    keeps fewer lags, a higher topk ratio more."""
    lo, hi, best = 0.0, 1.0, 0.5
    for step in range(steps):
        mid = (lo + hi) / 2
        c, f = measure_retention(layers, mode, mid, **kw)
        if log:
            log(f"  step {step + 1}/{steps}: {mode} value {mid:.4f}: corr retention {c:.4f}, "
                f"final retention {f:.4f} (target {target})")
        best = mid
        if abs(c - target) < tol:
            break
        if (c > target) == (mode == "threshold"):
            lo = mid
        else:
            hi = mid
    c, f = measure_retention(layers, mode, best, **kw)
    return best, c, f


def _time_layers(fn, layers, warmup: int, iters: int) -> list[float]:
    """Per iteration, the sum over layers of each layer's HIP-event time
    (benchmark_attention_multilayer.py:355-391)."""
    for _ in range(warmup):
        for lay in layers:
            fn(*lay)
    torch.cuda.synchronize()
    out = []
    for _ in range(iters):
        ev = []
        for lay in layers:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn(*lay)
            e1.record()
            ev.append((e0, e1))
        torch.cuda.synchronize()
        out.append(sum(a.elapsed_time(b) for a, b in ev))
    return out


def sweep(layers, values, mode: str = "threshold", warmup: int = 1, iters: int = 3, full: bool = True,
          labels=None, **kw) -> dict:
    """One length's results: dense causal ("full", this build's kernel over
    the whole causal mask) and the FFTSparse prefill at every value."""
    bs = kw.get("block_size", 128)
    res = {}
    if full:
        t = _time_layers(lambda q, k, v: block_sparse_attention(q, k, v, block_size=bs), layers, warmup, iters)
        res["full"] = {"time_ms": round(sum(t) / len(t), 4)}
    for i, val in enumerate(values):
        label = labels[i] if labels else (f"myattn_thres{val}" if mode == "threshold" else f"myattn_topk{val}")
        skw = _select_kw(mode, val, kw)
        t = _time_layers(lambda q, k, v: v7_prefill(q, k, v, block_size=bs, **skw), layers, warmup, iters)
        c, f = measure_retention(layers, mode, val, **kw)
        nq = -(-layers[0][0].shape[2] // bs)
        entry = {"time_ms": round(sum(t) / len(t), 4), "selection_mode": mode, "corr_val": val,
                 "corr_retention": round(c, 5), "final_retention": round(f, 5),
                 "density": round(f * nq / ((nq + 1) / 2), 5)}
        if "full" in res:
            entry["speedup"] = round(res["full"]["time_ms"] / entry["time_ms"], 3)
        res[label] = entry
    return res


def _synthetic_layers(L: int, n: int, Hq: int, Hk: int, dev):
    from .synth import make_qkv
    out = []
    for s in range(n):
        q, k, v = make_qkv(L, Hq, Hk, seed=100 + s)
        out.append((q.to(dev), k.to(dev), v.to(dev)))
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--lens", type=int, nargs="+", default=[128], help="sequence lengths in K tokens")
    ap.add_argument("--layers", type=int, default=2, help="synthetic layers per length (seeds 100, 101, ...)")
    ap.add_argument("--heads", type=int, nargs=2, default=[32, 8], metavar=("HQ", "HKV"))
    ap.add_argument("--mode", choices=["threshold", "topk"], default="threshold")
    ap.add_argument("--thresholds", type=float, nargs="*", default=[0.9, 0.95],
                    help="corr_threshold values (threshold mode) or topk ratios (topk mode)")
    ap.add_argument("--targets", type=float, nargs="*", default=None,
                    help="target corr retentions to calibrate instead of the fixed values")
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--iters", type=int, default=3)
    ap.add_argument("--save", default=None)
    args = ap.parse_args(argv)
    dev = torch.device("cuda:0")
    kw = dict(PRODUCTION_KWARGS)
    kw.pop("corr_threshold")
    results = {}
    for lk in args.lens:
        layers = _synthetic_layers(lk * 1024, args.layers, args.heads[0], args.heads[1], dev)
        values, labels = list(args.thresholds), None
        if args.targets:
            values, labels = [], []
            for sp in args.targets:
                print(f"calibrating {lk}K, target {sp}", file=sys.stderr, flush=True)
                best, c, f = calibrate(layers, sp, args.mode, log=lambda m: print(m, file=sys.stderr, flush=True),
                                       **kw)
                values.append(best)
                labels.append(f"sp{sp}")
        results[f"{lk}K"] = sweep(layers, values, args.mode, args.warmup, args.iters, labels=labels, **kw)
        print(json.dumps({f"{lk}K": results[f"{lk}K"]}), flush=True)
        del layers
        torch.cuda.empty_cache()
    if args.save:
        with open(args.save, "w") as fh:
            json.dump(results, fh, indent=2)
    return results


if __name__ == "__main__":
    main()
