"""Per-layer FFTSparse prefill benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2] [--threshold 0.9]

A step is one attention layer of BASELINE config 2 (Llama-3.1-8B shape:
L=131072, 32 query / 8 KV heads, head_dim 128, bf16, block 128): FFT-guided
block selection followed by block-sparse causal GQA attention, on inputs
already resident in HBM.  Prints one JSON line (metric of BASELINE.json):
per-layer milliseconds, plus the dense-attention comparison, per-stage times,
the roofline of the dominant kernel (sparse attention, bf16 MFMA) and of the
selection stage (HBM), and the CPU baseline (the oracle's restatement of the
reference path, timed on this host on a bounded sample).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "per-layer prefill ms (mask select + sparse attn) at 128K, speedup vs dense, 1 GPU"
PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E

PROD = dict(block_size=128, sink_ratio=0.01, recent_ratio=0.0, local_span_ratio=0.02,
            column_topk_ratio=0.2, qk_topk_ratio=0.3, stripe_threshold=0.3,
            diag_sample_ratio=0.15, min_diag_samples=5, max_diag_samples=64)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c2")
    ap.add_argument("--threshold", type=float, default=0.9)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-dense", action="store_true", help="skip the dense comparators")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--select-groups", type=int, default=None,
                    help="KV-head groups of the selection pipeline (default: the library's choice)")
    ap.add_argument("--cpu-heads", type=int, default=2,
                    help="query heads (all their query blocks) timed for the CPU attention sample")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (5 times) to calibrate "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE, then exit")
    return ap.parse_args()


def _ev():
    import torch
    return torch.cuda.Event(enable_timing=True)


def cpu_baseline(q, k, v, kw, bs, nnz_total, sample_heads):
    """Oracle restatement of the reference path on this host's cores: full
    selection, and fp32 block-sparse attention over every query block of the
    first sample_heads query heads, scaled to the whole layer by the
    selected-tile count (heads are independent)."""
    import torch
    from oracle import v7
    threads = torch.get_num_threads()
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    t0 = time.perf_counter()
    ref = v7.select_mask(qc, kc, **kw)
    t_sel = time.perf_counter() - t0
    heads = list(range(min(sample_heads, q.shape[1])))
    tiles = int(ref.mask[heads].sum())
    t0 = time.perf_counter()
    v7.block_sparse_attention(qc, kc, vc, ref.mask, bs, heads=heads)
    t_att_sample = time.perf_counter() - t0
    t_att = t_att_sample * nnz_total / max(1, tiles)
    return {
        "value": round((t_sel + t_att) * 1e3, 1),
        "unit": "ms",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle/v7.py on this host ({threads} torch threads): full v7 selection ({t_sel:.1f} s) + "
                   f"fp32 block-sparse attention over all query blocks of heads {heads} ({tiles} tiles, "
                   f"{t_att_sample:.1f} s) scaled x{nnz_total / max(1, tiles):.1f} to the layer's {nnz_total} "
                   f"selected tiles"),
        "select_ms": round(t_sel * 1e3, 1),
        "attn_ms_scaled": round(t_att * 1e3, 1),
        "cpu_model": _cpu_model(),
        "os_cpu_count": os.cpu_count(),
    }


def pmc_traffic(kernel, config):
    """HBM bytes per launch of a kernel from the committed rocprofv3 --pmc
    summary (FETCH_SIZE and WRITE_SIZE, calibrated against a plain copy), or
    None when that kernel/config was not profiled."""
    path = os.path.join(ROOT, "profiles", "traffic.txt")
    try:
        for line in open(path):
            f = line.split()
            if len(f) >= 4 and not line.startswith("#") and f[0] == kernel and f[1] == config:
                return int(float(f[2]) + float(f[3]))
    except OSError:
        pass
    return None


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU sharding is a design "
                                   "note (DESIGN.md), not a code path", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    if args.copy_calib:
        n = args.copy_calib * (1 << 20)
        x = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        y = torch.empty_like(x)
        for _ in range(5):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes": n, "launches": 5}))
        return
    import fftsparse_amd  # noqa: F401
    from fftsparse_amd import AttentionCall, block_sparse_attention, select_blocks
    from fftsparse_amd.synth import CONFIGS, make_config

    cfg = CONFIGS[args.config]
    dev = torch.device("cuda:0")
    t_gen = time.perf_counter()
    q, k, v = make_config(cfg, seed=args.seed)
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    torch.cuda.synchronize()
    t_gen = time.perf_counter() - t_gen
    kw = dict(PROD, block_size=cfg.block_size, corr_threshold=args.threshold)
    bs = cfg.block_size
    Hq, L, D = q.shape[1], q.shape[2], q.shape[3]
    Hk = k.shape[1]

    # One step = selection (pool, corr, stats, select) + attention (V^T
    # pre-pass, then order + attention kernel), all on torch's current stream,
    # which is the stream the events below are recorded on.
    def step(ev=None):
        if ev:
            ev[0].record()
        sel = select_blocks(q, k, pipeline_groups=args.select_groups, **kw)
        if ev:
            ev[1].record()
        call = AttentionCall(q, k, v, sel.blk_cnt, sel.blk_idx, block_size=bs)
        call.prepare()
        if ev:
            ev[2].record()
        out = call.run()
        if ev:
            ev[3].record()
        return sel, out

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    events = [(_ev(), _ev(), _ev(), _ev()) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        sel, _ = step(events[i])
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / args.steps
    sel_ms = [e[0].elapsed_time(e[1]) for e in events]
    att_ms = [e[1].elapsed_time(e[3]) for e in events]
    run_ms = [e[2].elapsed_time(e[3]) for e in events]
    tot_ms = [e[0].elapsed_time(e[3]) for e in events]
    ms = statistics.mean(tot_ms)

    nnz = sel.nnz()
    N = sel.params.N
    density = nnz / (Hq * N * (N + 1) / 2)
    attn_flops = 4.0 * D * bs * bs * nnz
    t_att = statistics.mean(att_ms)
    t_run = statistics.mean(run_ms)
    achieved = attn_flops / (t_run * 1e-3) / 1e12
    esz = q.element_size()
    sel_bytes = L * Hq * D * esz + L * Hk * D * esz
    t_sel = statistics.mean(sel_ms)
    stripe = int(sel.is_stripe.sum().item()) if sel.is_stripe is not None else None

    dense = {}
    if not args.no_dense:
        # our kernel on the full causal block set
        e = [(_ev(), _ev()) for _ in range(3)]
        block_sparse_attention(q, k, v, block_size=bs)
        for a, b in e:
            a.record()
            block_sparse_attention(q, k, v, block_size=bs)
            b.record()
        torch.cuda.synchronize()
        dense["own_dense_ms"] = statistics.mean(a.elapsed_time(b) for a, b in e)
        # torch SDPA flash attention (ROCm), K/V expanded to the query heads
        try:
            from torch.nn.attention import SDPBackend, sdpa_kernel
            kx = k.repeat_interleave(Hq // Hk, 1)
            vx = v.repeat_interleave(Hq // Hk, 1)
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
                torch.nn.functional.scaled_dot_product_attention(q, kx, vx, is_causal=True)
                e = [(_ev(), _ev()) for _ in range(3)]
                for a, b in e:
                    a.record()
                    torch.nn.functional.scaled_dot_product_attention(q, kx, vx, is_causal=True)
                    b.record()
                torch.cuda.synchronize()
            dense["sdpa_flash_ms"] = statistics.mean(a.elapsed_time(b) for a, b in e)
            del kx, vx
        except Exception as ex:  # noqa: BLE001 -- report, do not fail the benchmark line
            dense["sdpa_flash_error"] = f"{type(ex).__name__}: {ex}"[:200]
    dense_ms = min([x for x in (dense.get("sdpa_flash_ms"), dense.get("own_dense_ms")) if x] or [float("nan")])

    cpu = None
    if not args.no_cpu:
        torch.cuda.synchronize()
        cpu = cpu_baseline(q, k, v, kw, bs, nnz, args.cpu_heads)

    line = {
        "metric": METRIC,
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if q.dtype == torch.bfloat16 else str(q.dtype).replace("torch.", ""),
        "data": f"synthetic (fftsparse_amd.synth recipe, seed {args.seed})",
        "config": {"workload": f"{cfg.name}: one layer, L={L}, Hq={Hq}, Hkv={Hk}, D={D}, block {bs}, "
                               f"corr_threshold {args.threshold}, production kwargs",
                   "seq_len": L, "global_batch": 1, "block_size": bs, "corr_threshold": args.threshold,
                   "parallelism": "none (1 GPU)"},
        "speedup_vs_dense": round(dense_ms / ms, 3) if dense_ms == dense_ms else None,
        "dense_ms": round(dense_ms, 3) if dense_ms == dense_ms else None,
        "dense": {k2: (round(v2, 3) if isinstance(v2, float) else v2) for k2, v2 in dense.items()},
        "select_ms": round(t_sel, 4),
        "attn_ms": round(t_att, 4),
        "select_ms_median": round(statistics.median(sel_ms), 4),
        "attn_ms_median": round(statistics.median(att_ms), 4),
        "attn_kernel_ms": round(t_run, 4),
        "host_wall_ms_per_step": round(wall, 4),
        "density": round(density, 5),
        "selected_tiles": nnz,
        "stripe_heads": stripe,
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": pmc_traffic("bsattn", cfg.name),
                     "kernel": f"fs::bsattn_kernel<{bs},{'bf16' if q.dtype == torch.bfloat16 else 'f16'}>",
                     "work": f"4*D*bs^2 flop per selected (query block, key block) tile x {nnz} tiles",
                     "timed": "fs_bsattn_run (order pass + attention kernel), HIP events on the launch stream"},
        "roofline_select": {"bound": "hbm", "achieved": round(sel_bytes / (t_sel * 1e-3) / 1e9, 1),
                            "peak": PEAK_HBM_GBS, "unit": "GB/s",
                            "frac": round(sel_bytes / (t_sel * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                            "traffic": pmc_traffic("select", cfg.name),
                            "work": "Q and K read once (L*(Hq+Hkv)*D*2 bytes)",
                            "timed": "select_blocks: pool, block-score tiles + statistics (2 launches), block lists (2 launches)"},
        "cpu_baseline": cpu,
        "input_gen_s": round(t_gen, 1),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
