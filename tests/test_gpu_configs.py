"""GPU parity at the BASELINE workloads themselves: configs 1, 2 (thresholds
0.9 and 0.95) and 3 (block 64 and block 128) at full length, on the seeded
synthetic inputs the benchmark times (fftsparse_amd.synth).

For each workload:
  - the full v7 selection on the GPU against the oracle's
    (oracle/v7.select_mask, my_attn_v7.py:533-641): exact or excused block
    decisions >= 99.9% of all causal decisions, stripe decisions equal
    outside the band;
  - stage 2 under the oracle's own mask (the reference's block_sparse_attn_func
    call, my_attn_v7.py:775-786): the whole layer on the GPU, then fp32
    attention on the first, a middle and the last query block of every head
    plus a fixed random sample: max-abs 2e-2, mean-abs 1e-3;
  - myattn_prefill end to end: its output against fp32 attention under the
    block lists it selected itself, on the same sampled rows.

Parameters are the reference's production settings
(eval/efficiency/1_run_eval_multilayer.sh:46-62,72).
"""
from __future__ import annotations

import functools

import pytest
import torch

from fftsparse_amd import block_sparse_attention, myattn_prefill, select_blocks
from fftsparse_amd.synth import CONFIGS, make_config
from oracle import v7
from tests.helpers import BAND, MATCH_MIN, PROD, block_match, mask_bits

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@functools.lru_cache(maxsize=1)
def _inputs(name):
    return make_config(name)


def _sample_blocks(N, n_random=5, seed=0):
    g = torch.Generator().manual_seed(seed)
    rnd = torch.randint(1, N - 1, (n_random,), generator=g).tolist()
    return sorted({0, N // 2, N - 1, *rnd})


def _attn_rows_check(out_lhd, ref_lhd, qblocks, bs, L, label):
    rows = torch.cat([torch.arange(i * bs, min(L, (i + 1) * bs)) for i in qblocks])
    o = out_lhd.float().cpu()[rows]
    r = ref_lhd[rows]
    err = (o - r).abs()
    print(f"  {label}: max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}", flush=True)
    assert err.max().item() <= 2e-2
    assert err.mean().item() <= 1e-3


@pytest.mark.parametrize("name,thr", [("c1", 0.9), ("c2", 0.9), ("c2", 0.95), ("c3a", 0.9), ("c3b", 0.9)])
def test_baseline_workload_parity(name, thr):
    cfg = CONFIGS[name]
    print(f"[case] workload={name} threshold={thr} L={cfg.L} Hq={cfg.Hq} Hkv={cfg.Hkv} bs={cfg.block_size}",
          flush=True)
    q, k, v = _inputs(name)
    kw = {**PROD, "block_size": cfg.block_size, "corr_threshold": thr}
    bs = cfg.block_size
    L, Hq, D = q.shape[2], q.shape[1], q.shape[3]
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)

    # stage 1: the whole selection against the oracle
    sel = select_blocks(qg, kg, **kw)
    got = sel.dense_mask().cpu()
    ref = v7.select_mask(q, k, **kw)
    frac, exact, unexc = block_match(got, ref.mask, ref.excusable)
    N = ref.params.N
    dens = float(ref.mask.sum()) / (Hq * N * (N + 1) / 2)
    print(f"  selection: match={frac:.6f} exact={exact:.6f} unexcused={unexc} density={dens:.4f}", flush=True)
    assert frac >= MATCH_MIN
    if ref.is_stripe is not None:
        gs = sel.is_stripe.cpu().bool()
        near = (ref.mean_var - PROD["stripe_threshold"]).abs() <= BAND * PROD["stripe_threshold"]
        assert not ((gs != ref.is_stripe) & ~near).any()

    # stage 2 under the oracle's mask
    qblocks = _sample_blocks(N)
    cnt, bits = mask_bits(ref.mask, DEV)
    out = block_sparse_attention(qg, kg, vg, cnt, bits, block_size=bs)
    torch.cuda.synchronize()
    want = v7.block_sparse_attention(q, k, v, ref.mask, bs, qblocks=qblocks)
    _attn_rows_check(out[0], want, qblocks, bs, L, "attention under the oracle mask")
    del out, cnt, bits

    # end to end: the layer's output under the lists it selected
    o = myattn_prefill(qg, kg, vg, layer_idx=0, **kw)
    torch.cuda.synchronize()
    assert o.shape == (1, L, Hq * D) and o.dtype == q.dtype
    want = v7.block_sparse_attention(q, k, v, got, bs, qblocks=qblocks)
    _attn_rows_check(o.view(L, Hq, D), want, qblocks, bs, L, "myattn_prefill under its own lists")
