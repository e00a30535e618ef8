"""FlexPrefill and XAttention selection (fs_flex / fs_xattn through the C ABI)
on seeded random cases against oracle/flex.py and oracle/xattn.py, with the
checks of test_gpu_flex.py and test_gpu_xattn.py: ragged lengths from 1200 to
9000 tokens, GQA group sizes 1, 2 and 4, bf16 and fp16; FlexPrefill at 16-,
32-, 64- and 128-token blocks with gamma 0.9 / 0.95 / 0.99 and token budgets,
tau between the heads' divergences (0 for a single head); XAttention at
strides 4, 8 and 16 with thresholds 0.8 / 0.9 / 0.95."""
from __future__ import annotations

import random

import pytest
import torch

import tests.test_gpu_flex as F
import tests.test_gpu_xattn as X
from fftsparse_amd.synth import make_qkv

pytestmark = pytest.mark.gpu


def _shape(rng):
    L = rng.randint(1200, 9000)
    Hk = rng.choice([1, 2])
    Hq = Hk * rng.choice([1, 2, 4])
    dtype = rng.choice([torch.bfloat16, torch.bfloat16, torch.float16])
    return L, Hq, Hk, dtype


@pytest.mark.parametrize("i", range(24))
def test_flex_random_against_oracle(i):
    rng = random.Random(7777 * (i + 1))
    L, Hq, Hk, dtype = _shape(rng)
    bs = rng.choice([16, 32, 64, 128])
    gamma = rng.choice([0.9, 0.95, 0.99])
    mn = rng.choice([None, None, 256, 1024])
    mx = rng.choice([None, None, 2048, 4096])
    F._case(i=i, L=L, Hq=Hq, Hk=Hk, bs=bs, gamma=gamma, dtype=dtype, budget=(mn, mx))
    q, k, _ = make_qkv(L, Hq, Hk, dtype=dtype, seed=500 + i)
    q, k = F._blhd(q, k)
    tau = F._pick_tau(q, k, bs, gamma, min_budget=mn, max_budget=mx) if Hq > 1 else 0.0
    F._check(q, k, bs=bs, gamma=gamma, tau=tau, min_budget=mn, max_budget=mx)


@pytest.mark.parametrize("i", range(24))
def test_xattn_random_against_oracle(i):
    rng = random.Random(7777 * (i + 1) + 13)
    L, Hq, Hk, dtype = _shape(rng)
    stride = rng.choice([4, 8, 16])
    thr = rng.choice([0.8, 0.9, 0.95])
    X._case(i=i, L=L, Hq=Hq, Hk=Hk, stride=stride, threshold=thr, dtype=dtype)
    q, k, _ = make_qkv(L, Hq, Hk, dtype=dtype, seed=500 + i)
    X._check(q, k, stride, thr, dtype)
