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
    ap.add_argument("--selector", choices=("fftsparse", "xattn", "flex"), default="fftsparse",
                    help="block selection: FFTSparse v7 (default), XAttention (attn_src/xattn) or FlexPrefill "
                         "(attn_src/Flexprefill.py), the reference's comparison selectors, all attending with "
                         "the same block-sparse kernel")
    ap.add_argument("--xattn-stride", type=int, default=8, help="XAttention's antidiagonal stride")
    ap.add_argument("--flex-gamma", type=float, default=0.95,
                    help="FlexPrefill's gamma (the reference benchmark's default)")
    ap.add_argument("--flex-tau", type=float, default=0.1, help="FlexPrefill's tau (the reference benchmark's default)")
    ap.add_argument("--flex-block", type=int, default=32, choices=(32, 64, 128),
                    help="FlexPrefill's block size (the reference benchmark calls it with its default, 32)")
    ap.add_argument("--no-dense", action="store_true", help="skip the dense comparators")
    ap.add_argument("--selection-only", action="store_true",
                    help="time only the block selection (select_blocks) and print its own JSON line; with "
                         "--dtype float32 this is the fp32 path (LDS radix-FFT lag correlation, fs_corr + fs_stats)")
    ap.add_argument("--dtype", choices=("bfloat16", "float16", "float32"), default=None,
                    help="cast the config's synthetic Q/K/V to this dtype (default: the config's own)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--select-groups", type=int, default=None,
                    help="KV-head groups of the selection pipeline (default: the library's choice)")
    ap.add_argument("--tp-share", type=int, default=1, metavar="G",
                    help="run one GPU's share of G-way sharding by KV-head group: the first Hkv / G KV heads "
                         "and their query heads of the config's inputs, at the config's length")
    ap.add_argument("--cpu-heads", type=int, default=2,
                    help="query heads (all their query blocks) timed for the CPU attention sample")
    ap.add_argument("--c4-len", type=int, default=131072, help="config c4: prefill length")
    ap.add_argument("--dense-steps", type=int, default=1, help="config c4: timed SDPA forwards")
    ap.add_argument("--c4-rope", choices=("fused", "model"), default="fused",
                    help="config c4: rotary embedding fused with the block pooling (fs_rope_pool, default) "
                         "or the model's own RoPE before the registered attention")
    ap.add_argument("--c4-compare-rope", action="store_true",
                    help="config c4: also time the other --c4-rope variant (same steps)")
    ap.add_argument("--gemm-ceiling", action="store_true",
                    help="only time a bf16 8192^3 torch.matmul (hipBLASLt) 3 + 60 times, the practical MFMA ceiling "
                         "the attention kernel is compared with in the profiles, then exit")
    ap.add_argument("--power-sample", action="store_true",
                    help="only sample board power and the shader clock (amdsmi, every 50 ms) while the config's "
                         "attention runs back to back on its lists, then on the full causal set, then a bf16 "
                         "8192^3 torch.matmul and a 1 GiB device copy, about 4 s each; one JSON line, then exit")
    ap.add_argument("--traffic-rows", nargs=4, default=None,
                    metavar=("FETCH_CSV", "WRITE_CSV", "CAL_FETCH_CSV", "CAL_WRITE_CSV"),
                    help="only print the profiles/traffic.txt rows of --config from rocprofv3 --pmc FETCH_SIZE / "
                         "WRITE_SIZE collections of this bench and of --copy-calib 1024, then exit (no GPU)")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (5 times) to calibrate "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE, then exit")
    return ap.parse_args()


def _ev():
    import torch
    return torch.cuda.Event(enable_timing=True)


def _block_match(got, ref, excusable):
    """(exact-or-excused fraction, exact fraction, unexcused count) of the
    causal (head, query block, key block) decisions of two [H, N, Nk] masks."""
    import torch
    H, N, Nk = ref.shape
    dom = (torch.arange(N)[:, None] >= torch.arange(Nk)[None, :]).unsqueeze(0).expand(H, N, Nk)
    total = int(dom.sum())
    diff = (got != ref) & dom
    unexc = int((diff & ~excusable).sum())
    return (total - unexc) / total, (total - int(diff.sum())) / total, unexc


def cpu_baseline(q, k, v, kw, bs, nnz_total, sample_heads, sel=None, out=None):
    """Oracle restatement of the reference path on this host's cores: full
    selection, and fp32 block-sparse attention over every query block of the
    first sample_heads query heads, scaled to the whole layer by the
    selected-tile count (heads are independent).

    The oracle's selection also checks the timed step: the block match of the
    GPU's lists (sel) against it, and the GPU's output (out) against fp32
    attention under those lists on the first, middle and last query block of
    every head.  Returns (baseline, parity)."""
    import torch
    from oracle import v7
    threads = torch.get_num_threads()
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    t0 = time.perf_counter()
    ref = v7.select_mask(qc, kc, **kw)
    t_sel = time.perf_counter() - t0
    parity = None
    if sel is not None and out is not None:
        got = sel.dense_mask().cpu()
        frac, exact, unexc = _block_match(got, ref.mask, ref.excusable)
        N, L = ref.params.N, q.shape[2]
        qblocks = sorted({0, N // 2, N - 1})
        want = v7.block_sparse_attention(qc, kc, vc, got, bs, qblocks=qblocks)
        rows = torch.cat([torch.arange(i * bs, min(L, (i + 1) * bs)) for i in qblocks])
        err = (out[0].float().cpu()[rows] - want[rows]).abs()
        parity = {"block_match": round(frac, 6), "block_exact": round(exact, 6), "unexcused": unexc,
                  "bar": "exact or within 1e-3 of the threshold >= 0.999; attention max-abs <= 2e-2, mean-abs <= 1e-3",
                  "attn_max_abs": float(f"{err.max().item():.3e}"), "attn_mean_abs": float(f"{err.mean().item():.3e}"),
                  "attn_sample": f"query blocks {qblocks} of all {q.shape[1]} heads, fp32 oracle under the timed lists",
                  "pass": bool(frac >= 0.999 and err.max().item() <= 2e-2 and err.mean().item() <= 1e-3)}
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
    }, parity


def cpu_baseline_xattn(q, k, v, args, bs, nnz_total, sel):
    """The XAttention oracle (oracle/xattn.py) on this host's cores, on a
    bounded sample: the selection of one head over the first 16384 tokens,
    scaled by the reshaped-score count to all heads and the full length (the
    estimate is quadratic in L), and fp32 block-sparse attention over the first
    query head's selected tiles, scaled by the tile count.  The same sample
    checks the GPU's selection.  Returns (baseline, parity)."""
    import torch
    from oracle import v7, xattn as xo
    threads = torch.get_num_threads()
    Ls = min(16384, q.shape[2])
    qs, ks = q[:, :1, :Ls].cpu(), k[:, :1, :Ls].cpu()
    t0 = time.perf_counter()
    ref_mask, _, margin = xo.xattn_mask(qs, ks, stride=args.xattn_stride, threshold=args.threshold, block_size=bs)
    t_s = time.perf_counter() - t0
    # parity on the same sample: the GPU's selection of head 0 over the first Ls tokens
    from fftsparse_amd.xattn import xattn_select
    g = xattn_select(q[:, :1, :Ls], k[:, :1, :Ls], stride=args.xattn_stride, threshold=args.threshold,
                     block_size=bs).dense_mask().cpu()
    n = ref_mask.shape[1]
    tril = torch.tril(torch.ones(n, n, dtype=torch.bool))
    diff = (g != ref_mask) & tril
    unexc = int((diff & ~(margin[:, :n, :n].abs() <= 1e-3)).sum())
    total = int(tril.sum())
    parity = {"block_match": round((total - unexc) / total, 6), "block_exact": round(1 - int(diff.sum()) / total, 6),
              "unexcused": unexc, "sample": f"query head 0 over the first {Ls} tokens, oracle/xattn.py",
              "bar": "exact or within 1e-3 of the required mass >= 0.999",
              "pass": bool((total - unexc) / total >= 0.999)}
    L, Hq = q.shape[2], q.shape[1]
    t_sel = t_s * (L / Ls) ** 2 * Hq
    mask = sel.dense_mask().cpu()
    heads = [0]
    tiles = int(mask[heads].sum())
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    t0 = time.perf_counter()
    v7.block_sparse_attention(qc, kc, vc, mask, bs, heads=heads)
    t_a = time.perf_counter() - t0
    t_att = t_a * nnz_total / max(1, tiles)
    return {
        "value": round((t_sel + t_att) * 1e3, 1), "unit": "ms", "cores": threads, "kind": "port",
        "sample": (f"oracle/xattn.py on this host ({threads} torch threads): selection of head 0 over the first "
                   f"{Ls} tokens ({t_s:.1f} s) scaled x{(L / Ls) ** 2 * Hq:.0f} (quadratic in L, all heads); fp32 "
                   f"block-sparse attention over head 0 ({tiles} tiles, {t_a:.1f} s) scaled x"
                   f"{nnz_total / max(1, tiles):.1f} to {nnz_total} tiles"),
        "select_ms": round(t_sel * 1e3, 1), "attn_ms_scaled": round(t_att * 1e3, 1),
        "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count(),
    }, parity


# The sources each traffic row depends on (fftsparse_amd/csrc, plus the C-ABI header).
TRAFFIC_SOURCES = {"bsattn": ("attn.hip", "common.h"),
                   "select": ("pool.hip", "scores.hip", "select.hip", "common.h")}
# rocprofv3 kernel names summed into each row
TRAFFIC_KERNELS = {"bsattn": ("bsattn_kernel",),
                   "select": ("pool_kernel", "scores_kernel", "scores_final_kernel", "select_kernel")}


def src_hash(kernel):
    """First 16 hex digits of the sha256 of the sources a traffic row was
    measured with (TRAFFIC_SOURCES, then include/fftsparse_amd.h)."""
    import hashlib
    h = hashlib.sha256()
    paths = [os.path.join(ROOT, "fftsparse_amd", "csrc", n) for n in TRAFFIC_SOURCES[kernel]]
    for path in paths + [os.path.join(ROOT, "include", "fftsparse_amd.h")]:
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def pmc_traffic(kernel, config):
    """HBM bytes per launch of a kernel from the committed rocprofv3 --pmc
    summary profiles/traffic.txt (FETCH_SIZE and WRITE_SIZE, calibrated
    against a plain copy), or None when that kernel/config was not profiled
    or was profiled with other sources than these (the row's source hash
    differs from src_hash)."""
    path = os.path.join(ROOT, "profiles", "traffic.txt")
    try:
        cur = src_hash(kernel)
        for line in open(path):
            f = line.split()
            if len(f) >= 5 and not line.startswith("#") and f[0] == kernel and f[1] == config:
                return int(float(f[2]) + float(f[3])) if f[4] == cur else None
    except OSError:
        pass
    return None


def traffic_rows(config, fetch_csv, write_csv, cal_fetch_csv, cal_write_csv):
    """Rows of profiles/traffic.txt from four rocprofv3 --pmc counter
    collections (run_counter_collection.csv): FETCH_SIZE and WRITE_SIZE of
    `bench.py --no-cpu --no-dense --steps 1 --warmup 1` on the config, and of
    `bench.py --copy-calib 1024` (a plain 1 GiB copy, which fixes the scale of
    each counter).  Each row is the per-launch average summed over the row's
    kernels, scaled to bytes, with the source hash of the build measured."""
    import csv

    def load(path):
        acc = {}
        for row in csv.DictReader(open(path)):
            acc.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
        return acc

    def copy_kib(acc):
        vals = [v for name, vs in acc.items() if "copyBuffer" in name for v in vs]
        if not vals:
            raise SystemExit("no copy kernel in the calibration collection")
        return sum(vals) / len(vals)

    copy_kib_true = 1024 * 1024                      # 1 GiB read and written, in KiB
    f_scale = copy_kib_true / copy_kib(load(cal_fetch_csv)) * 1024
    w_scale = copy_kib_true / copy_kib(load(cal_write_csv)) * 1024
    fetch, write = load(fetch_csv), load(write_csv)
    rows = []
    for kernel, names in TRAFFIC_KERNELS.items():
        fb = wb = 0.0
        for name, vs in fetch.items():
            if any(n in name for n in names):
                fb += sum(vs) / len(vs) * f_scale
        for name, vs in write.items():
            if any(n in name for n in names):
                wb += sum(vs) / len(vs) * w_scale
        rows.append(f"{kernel} {config} {fb:.0f} {wb:.0f} {src_hash(kernel)}")
    return rows


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_flex(q, k, v, args, bs, nnz_total, sel, sample_heads=None):
    """The FlexPrefill oracle (oracle/flex.py) on this host's cores: the
    selection of the first ``sample_heads`` query heads (all by default; whole
    KV groups) over the full length, scaled by the head count (heads are
    independent), and fp32 block-sparse attention over the first query head's
    selected tiles, scaled by the tile count.  The timed lists of the sampled
    heads are checked against the oracle's.  Returns (baseline, parity)."""
    import torch
    from oracle import flex as fo, v7
    threads = torch.get_num_threads()
    Hq, Hk = q.shape[1], k.shape[1]
    g = Hq // Hk
    hs = max(g, (min(sample_heads or Hq, Hq) // g) * g)
    qs = q[:, :hs].cpu().transpose(1, 2).contiguous()
    ks = k[:, :hs // g].cpu().transpose(1, 2).contiguous()
    t0 = time.perf_counter()
    ref = fo.active_blocks(qs, ks, bs, args.flex_gamma, args.flex_tau)
    t_s = time.perf_counter() - t0
    t_sel = t_s * Hq / hs
    mask = sel.dense_mask().cpu()
    # parity of the timed lists on the sampled heads: exact block decisions (the
    # GPU tests also excuse near ties of the profiles; here the exact share)
    nb = mask.shape[1]
    tril = torch.tril(torch.ones(nb, nb, dtype=torch.bool))
    diff = (mask[:hs] != ref.mask) & tril
    total = int(tril.sum()) * hs
    exact = 1 - int(diff.sum()) / total
    parity = {"block_exact": round(exact, 6), "differing": int(diff.sum()),
              "sample": f"query heads 0..{hs - 1} at full length, oracle/flex.py",
              "bar": "exact >= 0.99 (the GPU tests: exact or a near tie >= 0.999)", "pass": bool(exact >= 0.99)}
    heads = [0]
    tiles = int(mask[heads].sum())
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    t0 = time.perf_counter()
    v7.block_sparse_attention(qc, kc, vc, mask, bs, heads=heads)
    t_a = time.perf_counter() - t0
    t_att = t_a * nnz_total / max(1, tiles)
    return {
        "value": round((t_sel + t_att) * 1e3, 1), "unit": "ms", "cores": threads, "kind": "port",
        "sample": (f"oracle/flex.py on this host ({threads} torch threads): selection of query heads 0..{hs - 1} "
                   f"({t_s:.1f} s) scaled x{Hq / hs:.0f} to all heads; fp32 block-sparse attention over head 0 "
                   f"({tiles} tiles, {t_a:.1f} s) scaled x{nnz_total / max(1, tiles):.1f} to {nnz_total} tiles"),
        "select_ms": round(t_sel * 1e3, 1), "attn_ms_scaled": round(t_att * 1e3, 1),
        "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count(),
    }, parity


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the path would shard by KV-head group "
                                   "(one KV head and its query heads per GPU, no exchange), which is not a "
                                   "code path here", "n_gpus": args.gpus}))
        sys.exit(2)
    if args.traffic_rows:
        print("\n".join(traffic_rows(args.config, *args.traffic_rows)))
        return
    import torch
    if args.gemm_ceiling:
        n = 8192
        a = torch.randn(n, n, device="cuda:0", dtype=torch.bfloat16)
        b = torch.randn(n, n, device="cuda:0", dtype=torch.bfloat16)
        for _ in range(3):
            a @ b
        torch.cuda.synchronize()
        e0, e1 = _ev(), _ev()
        e0.record()
        for _ in range(60):
            a @ b
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / 60
        print(json.dumps({"gemm_ceiling": f"bf16 {n}^3 torch.matmul", "ms": round(ms, 4),
                          "tflops": round(2 * n ** 3 / ms / 1e9, 1), "launches": 60}))
        return
    if args.copy_calib:
        n = args.copy_calib * (1 << 20)
        x = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        y = torch.empty_like(x)
        for _ in range(5):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes": n, "launches": 5}))
        return
    if args.config == "c4":
        return run_c4(args)
    import fftsparse_amd  # noqa: F401
    from fftsparse_amd import AttentionCall, block_sparse_attention, select_blocks
    from fftsparse_amd.synth import CONFIGS, make_config

    cfg = CONFIGS[args.config]
    dev = torch.device("cuda:0")
    flex = args.selector == "flex"
    t_gen = time.perf_counter()
    q, k, v = make_config(cfg, seed=args.seed)
    if args.tp_share > 1:
        G = args.tp_share
        if k.shape[1] % G:
            raise SystemExit(f"--tp-share {G} must divide the config's {k.shape[1]} KV heads")
        q, k, v = (x[:, :x.shape[1] // G].contiguous() for x in (q, k, v))
    if args.dtype:
        q, k, v = (x.to(getattr(torch, args.dtype)) for x in (q, k, v))
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    torch.cuda.synchronize()
    t_gen = time.perf_counter() - t_gen
    kw = dict(PROD, block_size=cfg.block_size, corr_threshold=args.threshold)
    bs = args.flex_block if flex else cfg.block_size
    Hq, L, D = q.shape[1], q.shape[2], q.shape[3]
    Hk = k.shape[1]

    if args.selection_only:
        return run_selection_only(args, cfg, q, k, kw)
    if args.power_sample:
        return run_power_sample(args, cfg, q, k, v, kw)

    # One step = selection (pool, corr, stats, select) + attention (V^T
    # pre-pass, then order + attention kernel), all on torch's current stream,
    # which is the stream the events below are recorded on.
    xattn = args.selector == "xattn"
    if xattn:
        from fftsparse_amd.xattn import xattn_select
    if flex:
        from fftsparse_amd.flex import flex_select
        q_blhd, k_blhd = q.transpose(1, 2), k.transpose(1, 2)      # the reference's [B, L, H, D] views

    host_sel = []

    def step(ev=None):
        if ev:
            ev[0].record()
        th = time.perf_counter()
        if xattn:
            sel = xattn_select(q, k, stride=args.xattn_stride, threshold=args.threshold, block_size=bs)
        elif flex:
            sel = flex_select(q_blhd, k_blhd, gamma=args.flex_gamma, tau=args.flex_tau, block_size=bs)
        else:
            sel = select_blocks(q, k, pipeline_groups=args.select_groups, **kw)
        if ev:
            host_sel.append((time.perf_counter() - th) * 1e3)
            ev[1].record()
        call = AttentionCall(q, k, v, sel.blk_cnt, sel.blk_bits, block_size=bs)
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
        sel, out = step(events[i])
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / args.steps
    sel_ms = [e[0].elapsed_time(e[1]) for e in events]
    att_ms = [e[1].elapsed_time(e[3]) for e in events]
    run_ms = [e[2].elapsed_time(e[3]) for e in events]
    tot_ms = [e[0].elapsed_time(e[3]) for e in events]
    ms = statistics.mean(tot_ms)

    nnz = sel.nnz()
    N = -(-L // bs)
    density = nnz / (Hq * N * (N + 1) / 2)
    attn_flops = 4.0 * D * bs * bs * nnz
    t_att = statistics.mean(att_ms)
    t_run = statistics.mean(run_ms)
    achieved = attn_flops / (t_run * 1e-3) / 1e12
    esz = q.element_size()
    sel_bytes = L * Hq * D * esz + L * Hk * D * esz
    t_sel = statistics.mean(sel_ms)
    # the traffic rows were measured on the config's default workload: threshold
    # 0.9, its own dtype, every head
    traffic_key = cfg.name if (args.threshold == 0.9 and not args.dtype and args.tp_share == 1) else None
    stripe = (int(sel.is_stripe.sum().item()) if not (xattn or flex) and sel.is_stripe is not None else None)

    dense = {}
    if not args.no_dense:
        # our kernel on the full causal block set
        e = [(_ev(), _ev()) for _ in range(3)]
        block_sparse_attention(q, k, v, block_size=cfg.block_size)
        for a, b in e:
            a.record()
            block_sparse_attention(q, k, v, block_size=cfg.block_size)
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

    cpu = parity = None
    if not args.no_cpu:
        torch.cuda.synchronize()
        if xattn:
            cpu, parity = cpu_baseline_xattn(q, k, v, args, bs, nnz, sel)
        elif flex:
            cpu, parity = cpu_baseline_flex(q, k, v, args, bs, nnz, sel)
        else:
            cpu, parity = cpu_baseline(q, k, v, kw, bs, nnz, args.cpu_heads, sel=sel, out=out)

    if xattn:
        # the two MFMA passes over the causal reshaped scores: 2 * S*D MACs per entry per pass
        S = args.xattn_stride
        Lr = N * bs // S
        est_flops = 2 * Hq * (Lr * (Lr + 1) / 2) * 2.0 * S * D
        roofline_select = {"bound": "mfma", "achieved": round(est_flops / (t_sel * 1e-3) / 1e12, 1),
                           "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                           "frac": round(est_flops / (t_sel * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4), "traffic": None,
                           "work": f"2 passes x 2*S*D flop per causal reshaped score (S={S}, {Lr} reshaped rows per head)",
                           "timed": "xattn_select: scores pass 1 (row stats), pass 2 (block sums), selection"}
    elif flex:
        # K read by the two last-block score passes and by the block means; the
        # sparse heads' Q read for their block means; the fp32 profiles written once
        n_sparse = int(sel.head_info[:, 2].sum().item())
        flex_bytes = 3 * L * Hk * D * esz + n_sparse * L * D * esz + 2 * Hq * L * 4
        roofline_select = {"bound": "hbm", "achieved": round(flex_bytes / (t_sel * 1e-3) / 1e9, 1),
                           "peak": PEAK_HBM_GBS, "unit": "GB/s",
                           "frac": round(flex_bytes / (t_sel * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "traffic": None,
                           "work": ("K read 3x (2 score passes + block means: 3*L*Hkv*D*2 bytes), the sparse heads' Q "
                                    f"({n_sparse} heads), vertical/slash profiles written (2*Hq*L*4 bytes)"),
                           "timed": "flex_select: last-block scores (2 passes), K block means, per-head budgets / "
                                    "JS test / top-k, sparse-head cover (2 launches), block mask"}
    else:
        t_sel_med = statistics.median(sel_ms)
        roofline_select = {"bound": "hbm", "achieved": round(sel_bytes / (t_sel * 1e-3) / 1e9, 1),
                           "peak": PEAK_HBM_GBS, "unit": "GB/s",
                           "frac": round(sel_bytes / (t_sel * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                           # the same on the median step (the mean includes the first timed step,
                           # which starts on an idle GPU)
                           "frac_median": round(sel_bytes / (t_sel_med * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                           "traffic": pmc_traffic("select", traffic_key),
                           "work": "Q and K read once (L*(Hq+Hkv)*D*2 bytes)",
                           "timed": "select_blocks: pool, block-score tiles + statistics (2 launches), block masks "
                                    "(1 launch)"}
    sel_desc = (f"XAttention selection (stride {args.xattn_stride}, threshold {args.threshold})" if xattn
                else f"FlexPrefill selection and attention at {bs}-token blocks (gamma {args.flex_gamma}, tau "
                     f"{args.flex_tau}; the reference benchmark's call uses the default block size, 32)" if flex
                else f"corr_threshold {args.threshold}, production kwargs")
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
        "config": {"workload": f"{cfg.name}: one layer, L={L}, Hq={Hq}, Hkv={Hk}, D={D}, block {bs}, {sel_desc}",
                   "selector": args.selector,
                   "seq_len": L, "global_batch": 1, "block_size": bs,
                   **({"flex_gamma": args.flex_gamma, "flex_tau": args.flex_tau} if flex else
                      {("xattn_threshold" if xattn else "corr_threshold"): args.threshold}),
                   "parallelism": ("none (1 GPU)" if args.tp_share == 1 else
                                   f"one GPU's share of {args.tp_share}-way sharding by KV-head group "
                                   f"(the first {Hk} KV heads and their {Hq} query heads)")},
        "speedup_vs_dense": round(dense_ms / ms, 3) if dense_ms == dense_ms else None,
        "dense_ms": round(dense_ms, 3) if dense_ms == dense_ms else None,
        "dense": {k2: (round(v2, 3) if isinstance(v2, float) else v2) for k2, v2 in dense.items()},
        "select_ms": round(t_sel, 4),
        "attn_ms": round(t_att, 4),
        "select_ms_median": round(statistics.median(sel_ms), 4),
        "select_ms_steps": [round(x, 4) for x in sel_ms],
        "select_host_enqueue_ms": round(statistics.mean(host_sel), 4),
        "attn_ms_median": round(statistics.median(att_ms), 4),
        "attn_kernel_ms": round(t_run, 4),
        "host_wall_ms_per_step": round(wall, 4),
        "density": round(density, 5),
        "selected_tiles": nnz,
        "stripe_heads": stripe,
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": None if (xattn or flex) else pmc_traffic("bsattn", traffic_key),
                     "kernel": (f"fs::bsattn_kernel<128, 64, {'bf16' if q.dtype == torch.bfloat16 else 'f16'}, {bs}>"
                                + (" (union of 128 / bs rows' lists per workgroup)" if bs < 64 else "")),
                     "work": f"4*D*bs^2 flop per selected (query block, key block) tile x {nnz} tiles",
                     "timed": "fs_bsattn_run (order pass + attention kernel), HIP events on the launch stream"},
        "roofline_select": roofline_select,
        "cpu_baseline": cpu,
        "parity": parity,
        "input_gen_s": round(t_gen, 1),
    }
    print(json.dumps(line), flush=True)


def run_power_sample(args, cfg, q, k, v, kw, secs=4.0):
    """Board power and shader clock while one kernel runs back to back: a
    thread samples amdsmi every 50 ms; the first second of each run (the
    clock's ramp) is dropped.  The attention runs on the config's own lists
    (one selection first), then on the full causal block set; the references
    are a bf16 8192^3 torch.matmul (hipBLASLt) and a 1 GiB device copy."""
    import threading
    import amdsmi
    import torch
    from fftsparse_amd import AttentionCall, select_blocks
    amdsmi.amdsmi_init()
    handle = amdsmi.amdsmi_get_processor_handles()[0]

    def sample(stop, out):
        while not stop.is_set():
            p = amdsmi.amdsmi_get_power_info(handle)
            c = amdsmi.amdsmi_get_clock_info(handle, amdsmi.AmdSmiClkType.GFX)
            out.append((time.perf_counter(), p.get("current_socket_power"), c.get("clk"), p.get("power_limit")))
            time.sleep(0.05)

    def run(fn):
        fn()
        torch.cuda.synchronize()
        out, stop = [], threading.Event()
        th = threading.Thread(target=sample, args=(stop, out))
        th.start()
        t0 = time.perf_counter()
        n = 0
        while time.perf_counter() - t0 < secs:
            for _ in range(4):
                fn()
            torch.cuda.synchronize()
            n += 4
        t1 = time.perf_counter()
        stop.set()
        th.join()
        rows = [r for r in out if r[0] - t0 > 1.0 and isinstance(r[1], (int, float)) and isinstance(r[2], (int, float))]
        return {"launches": n, "ms_per_launch": round((t1 - t0) * 1e3 / n, 4), "samples": len(rows),
                "power_w_median": statistics.median(r[1] for r in rows) if rows else None,
                "power_w_range": [min(r[1] for r in rows), max(r[1] for r in rows)] if rows else None,
                "gfx_mhz_median": statistics.median(r[2] for r in rows) if rows else None,
                "gfx_mhz_range": [min(r[2] for r in rows), max(r[2] for r in rows)] if rows else None,
                "power_limit_w": (out[0][3] / 1e6 if out and isinstance(out[0][3], (int, float)) else None)}

    sel = select_blocks(q, k, **kw)
    lists = AttentionCall(q, k, v, sel.blk_cnt, sel.blk_bits, block_size=cfg.block_size)
    lists.prepare()
    res = {"attention_lists": run(lists.run)}
    dense = AttentionCall(q, k, v, block_size=cfg.block_size)
    dense.prepare()
    res["attention_dense"] = run(dense.run)
    del dense, lists
    n = 8192
    a = torch.randn(n, n, device=q.device, dtype=torch.bfloat16)
    b = torch.randn(n, n, device=q.device, dtype=torch.bfloat16)
    res["gemm_8192"] = run(lambda: a @ b)
    del a, b
    x = torch.ones(1 << 30, dtype=torch.uint8, device=q.device)
    y = torch.empty_like(x)
    res["copy_1gib"] = run(lambda: y.copy_(x))
    print(json.dumps({"power_sample": cfg.name, "secs_each": secs, **res}), flush=True)


def run_selection_only(args, cfg, q, k, kw):
    """The v7 block selection alone (select_blocks: pool, lag correlation and
    statistics, block masks) on the config's inputs in their dtype, HIP events
    on torch's current stream; one JSON line with its time and HBM roofline."""
    import torch
    from fftsparse_amd import select_blocks
    for _ in range(args.warmup):
        select_blocks(q, k, **kw)
    torch.cuda.synchronize()
    ev = [(_ev(), _ev()) for _ in range(args.steps)]
    for a, b in ev:
        a.record()
        sel = select_blocks(q, k, **kw)
        b.record()
    torch.cuda.synchronize()
    ms = [a.elapsed_time(b) for a, b in ev]
    L, Hq, Hk, D = q.shape[2], q.shape[1], k.shape[1], q.shape[3]
    nbytes = L * (Hq + Hk) * D * q.element_size()
    t = statistics.mean(ms)
    N = -(-L // kw["block_size"])
    print(json.dumps({
        "metric": "block selection ms (select_blocks)", "value": round(t, 4), "unit": "ms",
        "higher_is_better": False, "steps": args.steps, "warmup": args.warmup,
        "dtype": str(q.dtype).replace("torch.", ""),
        "config": {"workload": f"{cfg.name} shape: L={L}, Hq={Hq}, Hkv={Hk}, D={D}, block {kw['block_size']}, "
                               f"corr_threshold {kw['corr_threshold']}, production kwargs, selection only",
                   "seq_len": L},
        "median_ms": round(statistics.median(ms), 4),
        "density": round(sel.nnz() / (Hq * N * (N + 1) / 2), 5),
        "roofline_select": {"bound": "hbm", "achieved": round(nbytes / (t * 1e-3) / 1e9, 1), "peak": PEAK_HBM_GBS,
                            "unit": "GB/s", "frac": round(nbytes / (t * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                            "work": "Q and K read once (L*(Hq+Hkv)*D*element bytes)"},
    }), flush=True)


C4_METRIC = "end-to-end prefill ms, 32-layer random-init Llama-3.1-8B at 128K, attention share, 1 GPU"


def run_c4(args):
    """Config 4: a full 32-layer Llama-3.1-8B-shaped model (random init, bf16,
    built on the GPU) prefilling 131072 random token ids, with the FFTSparse
    prefill registered as the model's attention (fftsparse_amd.hf) in every
    layer, then the same model on torch SDPA (flash) for the dense
    comparison.  A step is one forward pass without KV cache that keeps the
    last position's logits only.  The attention share is the sum of the
    per-layer prefill call times (HIP events around each registered call;
    with the fused RoPE, around the rotary embedding + pooling pass and the
    attention) over the forward time."""
    import torch
    from transformers import LlamaForCausalLM
    import fftsparse_amd.hf as fh
    from fftsparse_amd.synth import c4_model_config

    L = args.c4_len
    cfg = c4_model_config()
    dev = torch.device("cuda:0")
    t0 = time.perf_counter()
    torch.manual_seed(args.seed)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    with dev:
        model = LlamaForCausalLM(cfg)
    torch.set_default_dtype(prev)
    model.eval()
    n_params = sum(p.numel() for p in model.parameters())
    g = torch.Generator().manual_seed(args.seed)
    ids = torch.randint(0, cfg.vocab_size, (1, L), generator=g).to(dev)
    torch.cuda.synchronize()
    t_build = time.perf_counter() - t0
    print(f"[c4] model built: {n_params / 1e9:.2f} B parameters, {t_build:.1f} s", file=sys.stderr, flush=True)

    def forward():
        with torch.no_grad():
            return model(input_ids=ids, use_cache=False, logits_to_keep=1).logits

    def timed(n):
        out = []
        for _ in range(n):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            logits = forward()
            e1.record()
            torch.cuda.synchronize()
            out.append(e0.elapsed_time(e1))
            print(f"[c4] forward ({model.config._attn_implementation}): {out[-1]:.1f} ms", file=sys.stderr, flush=True)
        return out, logits

    fused = args.c4_rope == "fused"
    fh.patch_model(model, fused_rope=fused, corr_threshold=args.threshold)
    fh.record_prefill_events(False)
    timed(args.warmup)
    fh.record_prefill_events(True)
    sparse_ms, logits = timed(args.steps)
    ev = fh.prefill_events()
    fh.record_prefill_events(False)
    other_ms = None
    if args.c4_compare_rope:
        fh.patch_model(model, fused_rope=not fused, corr_threshold=args.threshold)
        timed(1)
        o, _ = timed(args.steps)
        other_ms = sum(o) / len(o)
        fh.patch_model(model, fused_rope=fused, corr_threshold=args.threshold)
    attn_total = sum(e.ms() for e in ev) / args.steps
    per_layer = [0.0] * cfg.num_hidden_layers
    density = [0.0] * cfg.num_hidden_layers
    for e in ev:
        per_layer[e.layer_idx] += e.ms() / args.steps
        density[e.layer_idx] = e.density()
    finite = bool(torch.isfinite(logits.float()).all())
    ms = sum(sparse_ms) / len(sparse_ms)

    dense_ms = float("nan")
    if not args.no_dense:
        fh.patch_model(model, fused_rope=False)        # class forwards back
        model.set_attn_implementation("sdpa")
        d, _ = timed(1 + args.dense_steps)
        dense_ms = sum(d[1:]) / max(1, len(d) - 1) if len(d) > 1 else d[0]
    line = {
        "metric": C4_METRIC, "value": round(ms, 2), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 2), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": f"random-init weights (seed {args.seed}), random token ids",
        "config": {"workload": f"c4: 32-layer Llama-3.1-8B shape ({n_params / 1e9:.2f} B parameters), "
                               f"prefill of {L} tokens, FFTSparse prefill in every layer, "
                               f"corr_threshold {args.threshold}, production kwargs, "
                               f"RoPE {'fused with the block pooling' if fused else 'of the model'}",
                   "seq_len": L, "global_batch": 1, "parallelism": "none (1 GPU)"},
        "rope": args.c4_rope,
        "attention_ms": round(attn_total, 2), "attention_share": round(attn_total / ms, 4),
        "non_attention_ms": round(ms - attn_total, 2),
        "attention_ms_per_layer": [round(x, 3) for x in per_layer],
        "density_per_layer": [round(x, 4) for x in density],
        "dense_sdpa_ms": round(dense_ms, 2) if dense_ms == dense_ms else None,
        "speedup_vs_dense_model": round(dense_ms / ms, 3) if dense_ms == dense_ms else None,
        "logits_finite": finite, "build_s": round(t_build, 1),
        "other_rope_ms": round(other_ms, 2) if other_ms is not None else None,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
