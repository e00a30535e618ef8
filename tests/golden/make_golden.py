"""Writes the committed fixtures of this directory (run from the repo root):

    python tests/golden/make_golden.py

  synth_sha256.txt  SHA-256 of small synthetic inputs (pins the generator)
  c0_select.npz     oracle selection for BASELINE config 0 with the
                    production arguments: bit-packed [H,N,N] mask, lag keeps,
                    stripe statistics, column / last-row selections.

The reference ships no golden vectors and no captured Q/K; these fixtures are
regression pins of this repository's oracle, which is itself checked against
closed forms and brute force in tests/test_oracle.py.
"""
from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from fftsparse_amd.synth import make_config, make_qkv, sha256_of  # noqa: E402
from oracle import v7  # noqa: E402
from tests.helpers import PROD  # noqa: E402


def main():
    lines = []
    q, k, v = make_qkv(2048, 4, 1, dtype=torch.float32, seed=0)
    lines.append(f"small_f32_seed0 {sha256_of(q, k, v)}")
    q, k, v = make_qkv(2048, 4, 2, dtype=torch.bfloat16, seed=0, stripe_density=0.005, period=512)
    lines.append(f"small_bf16_seed0 {sha256_of(q, k, v)}")
    q, k, v = make_config("c0")
    lines.append(f"c0_seed0 {sha256_of(q, k, v)}")
    (HERE / "synth_sha256.txt").write_text("\n".join(lines) + "\n")

    r = v7.select_mask(q, k, **PROD)
    np.savez_compressed(
        HERE / "c0_select.npz",
        mask=np.packbits(r.mask.numpy(), axis=-1),
        shape=np.array(r.mask.shape),
        keep_tau=r.keep_tau.numpy(),
        mean_var=r.mean_var.numpy(),
        is_stripe=r.is_stripe.numpy(),
        col_sel=r.col_sel.numpy(),
        last_sel=r.last_sel.numpy(),
        corr=r.corr.numpy(),
    )
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
