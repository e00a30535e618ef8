"""The v7 selection (select_blocks through the C ABI) on seeded random
parameter sets against oracle/v7.select_mask: block sizes 32, 64 and 128,
ragged lengths up to 40000 tokens, GQA, bf16 / fp16 / fp32 (the fp32 inputs
take the FFT path), sink / recent / local-window ratios including 0, the
correlation mask on or off in threshold and topk modes, the column and
last-row masks on or off, sampled-diagonal counts, and stripe thresholds that
make every head stripe or diffuse.  Bar: exact or excused block decisions
>= 99.9% of all causal decisions."""
from __future__ import annotations

import random

import pytest
import torch

from fftsparse_amd import select_blocks
from fftsparse_amd.synth import make_qkv
from oracle import v7
from tests.helpers import MATCH_MIN, block_match

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _case(i: int):
    rng = random.Random(104729 * (i + 1))
    bs = rng.choice([32, 64, 128])
    Hk = rng.choice([1, 2])
    Hq = Hk * rng.choice([1, 2, 4])
    L = rng.randint(12 * bs, min(40000, 600 * bs))
    dtype = rng.choice([torch.bfloat16, torch.bfloat16, torch.float16, torch.float32])
    kw = dict(block_size=bs,
              sink_ratio=rng.choice([0.0, 0.01, 0.05, 0.1]),
              recent_ratio=rng.choice([0.0, 0.01, 0.1]),
              local_span_ratio=rng.choice([0.0, 0.02, 0.05, 0.1]),
              enable_correlation_mask=rng.random() < 0.85,
              correlation_selection_mode=rng.choice(["threshold", "threshold", "topk"]),
              correlation_topk_ratio=rng.choice([0.05, 0.2, 0.5]),
              corr_threshold=rng.choice([0.1, 0.5, 0.9, 0.95]),
              enable_column_mask=rng.random() < 0.8,
              column_topk_ratio=rng.choice([0.05, 0.1, 0.2]),
              column_start_exclude_ratio=rng.choice([0.0, 0.1]),
              column_end_exclude_ratio=rng.choice([0.1, 0.2]),
              enable_last_block_mask=rng.random() < 0.8,
              diag_sample_ratio=rng.choice([0.05, 0.15, 0.3]),
              min_diag_samples=rng.choice([2, 5]),
              max_diag_samples=rng.choice([16, 64]),
              stripe_threshold=rng.choice([0.0, 0.3, 1.0, 10.0]),
              qk_topk_ratio=rng.choice([0.05, 0.2, 0.3]))
    return bs, Hq, Hk, L, dtype, kw


@pytest.mark.parametrize("i", range(40))
def test_random_parameters_against_oracle(i):
    bs, Hq, Hk, L, dtype, kw = _case(i)
    print(f"[case] random-select {i}: L={L} Hq={Hq} Hk={Hk} {dtype} {kw}", flush=True)
    q, k, _ = make_qkv(L, Hq, Hk, dtype=dtype, seed=100 + i)
    try:
        ref = v7.select_mask(q, k, **kw)
    except ValueError:
        # the reference's own error (the six-way unpack when the window covers the sequence)
        with pytest.raises(ValueError):
            select_blocks(q.to(DEV), k.to(DEV), **kw)
        return
    sel = select_blocks(q.to(DEV), k.to(DEV), **kw)
    frac, exact, unexc = block_match(sel.dense_mask().cpu(), ref.mask, ref.excusable)
    print(f"  match={frac:.6f} exact={exact:.6f} unexcused={unexc}", flush=True)
    assert frac >= MATCH_MIN
