"""GPU parity of the XAttention selector (fs_xattn through the C ABI) against
the CPU oracle (oracle/xattn.py), and of attention under its block lists.

Bars: block sums equal to the oracle's in the input dtype, or one unit in the
last place apart (the fp32 reductions' order differs), for >= 99% of the
causal blocks; block decisions exact, or excused where the mass before the
block is within 1e-3 relative of the row's required mass, for >= 99.9% of the
causal decisions; the selection applied by the oracle to the kernel's own block
sums reproduces the kernel's lists exactly (decisions within 1e-9 of the
threshold aside); attention under the lists within max-abs 2e-2 and mean-abs
1e-3 of fp32 attention.
"""
from __future__ import annotations

import pytest
import torch

from fftsparse_amd.synth import make_qkv
from fftsparse_amd.xattn import Xattention_prefill, density, xattn_estimate, xattn_select
from tests.helpers import check_mask_words
from oracle import v7
from oracle import xattn as xo

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
CAUSAL_BAND = 1e-3


def _case(**kw):
    print("[case] xattn " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _ulp_diff(a: torch.Tensor, b: torch.Tensor, dtype) -> torch.Tensor:
    ai = a.to(dtype).view(torch.int16).to(torch.int32)
    bi = b.to(dtype).view(torch.int16).to(torch.int32)
    return (ai - bi).abs()


def _check(q, k, stride, threshold, dtype, keep_sink=False):
    sel = xattn_select(q.to(DEV), k.to(DEV), stride=stride, threshold=threshold, keep_sink=keep_sink)
    torch.cuda.synchronize()
    mask_ref, sums_ref, margin = xo.xattn_mask(q, k, stride=stride, threshold=threshold, keep_sink=keep_sink)
    N = mask_ref.shape[1]
    tril = torch.tril(torch.ones(N, N, dtype=torch.bool))
    # block sums: equal, or one unit in the last place apart
    g_sums = sel.sums.cpu()
    ud = _ulp_diff(g_sums[:, tril], sums_ref[:, :N, :N][:, tril], dtype)
    print(f"  sums: equal {(ud == 0).float().mean().item():.5f}, max ulp {ud.max().item()}")
    assert ud.max().item() <= 1
    assert (ud == 0).float().mean().item() >= 0.99
    # decisions vs the oracle (causal part), margins within the band excused
    g_mask = sel.dense_mask().cpu()
    diff = (g_mask != mask_ref) & tril
    excused = margin[:, :N, :N].abs() <= CAUSAL_BAND
    if keep_sink:
        diff[:, 0] = False
    total = int(tril.sum()) * g_mask.shape[0]
    unexc = int((diff & ~excused).sum())
    frac = (total - unexc) / total
    print(f"  decisions: exact {1 - int(diff.sum()) / total:.6f}, exact-or-excused {frac:.6f}, unexcused {unexc}")
    assert frac >= 0.999
    # the oracle's selection rule on the kernel's own sums gives the kernel's lists
    own_mask, own_margin = xo.select_rows(g_sums, threshold)
    own_mask &= tril
    if keep_sink:
        own_mask[:, 0, :] = True
    d2 = (own_mask != g_mask) & ~(own_margin.abs() <= 1e-9)
    assert not d2.any(), torch.nonzero(d2)[:5]
    # invariants: causal (keep_sink aside), first and diagonal blocks kept
    body = g_mask.clone()
    if keep_sink:
        body[:, 0] = tril[0]
    assert not (body & ~tril).any()
    assert g_mask[:, :, 0].all() and g_mask[:, torch.arange(N), torch.arange(N)].all()
    return sel, g_mask


@pytest.mark.parametrize("L,Hq,Hk,stride,dtype", [
    (8192, 2, 1, 8, torch.bfloat16),
    (8192, 2, 2, 16, torch.bfloat16),
    (6000, 4, 2, 8, torch.bfloat16),          # ragged: L % 128 != 0
    (4100, 2, 1, 16, torch.float16),          # ragged, L % 16 != 0
    (4096, 2, 1, 4, torch.bfloat16),
])
def test_xattn_selection_parity(L, Hq, Hk, stride, dtype):
    _case(L=L, Hq=Hq, Hk=Hk, stride=stride, dtype=dtype)
    q, k, _ = make_qkv(L, Hq, Hk, dtype=dtype, seed=31)
    _check(q, k, stride, 0.9, dtype)


def test_xattn_per_head_thresholds_and_keep_sink():
    """A per-head threshold tensor padded with its last value (3 values for 4
    heads), keep_sink filling row 0."""
    _case(L=4096, thr="per-head", keep_sink=True)
    q, k, _ = make_qkv(4096, 4, 1, dtype=torch.bfloat16, seed=32)
    thr = torch.tensor([0.5, 0.8, 0.95])
    sel, mask = _check(q, k, 8, thr, torch.bfloat16, keep_sink=True)
    assert mask[:, 0].all()
    # monotone in the threshold: head 0 (0.5) keeps no more than under 0.95 everywhere
    hi = xattn_select(q.to(DEV), k.to(DEV), stride=8, threshold=0.95).dense_mask().cpu()
    assert not (mask[0, 1:] & ~hi[0, 1:]).any()


def test_xattn_native_gqa_equals_expanded_and_strided_views():
    """K with its KV heads, K repeat_kv'd to the query heads, and the
    projections' [1, L, H, D] layout viewed as [1, H, L, D] give the same lists."""
    _case(L=4096, layout="gqa/strided")
    q, k, _ = make_qkv(4096, 4, 2, dtype=torch.bfloat16, seed=33)
    a = xattn_select(q.to(DEV), k.to(DEV), stride=8, threshold=0.9)
    b = xattn_select(q.to(DEV), k.repeat_interleave(2, 1).to(DEV), stride=8, threshold=0.9)
    qs = q.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    ks = k.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    c = xattn_select(qs, ks, stride=8, threshold=0.9)
    for x in (b, c):
        assert torch.equal(a.blk_cnt, x.blk_cnt)
        assert torch.equal(a.dense_mask(), x.dense_mask())
        assert torch.equal(a.sums, x.sums)


def test_xattn_prefill_attention_parity():
    """Xattention_prefill: attention under the kernel's own lists against fp32
    attention under the same mask; xattn_estimate's outputs agree with the lists."""
    _case(L=8192, prefill=True)
    q, k, v = make_qkv(8192, 4, 1, dtype=torch.bfloat16, seed=34)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    out = Xattention_prefill(qg, kg, vg, stride=8, threshold=0.9)
    torch.cuda.synchronize()
    assert out.shape == (1, 4, 8192, 128)
    sel = xattn_select(qg, kg, stride=8, threshold=0.9)
    mask = sel.dense_mask().cpu()
    ref = v7.block_sparse_attention(q, k, v, mask, 128)            # [L, H, D]
    err = (out[0].transpose(0, 1).float().cpu() - ref).abs()
    print(f"  density {density(sel):.4f} max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}")
    assert err.max().item() <= 2e-2 and err.mean().item() <= 1e-3
    sums, masks = xattn_estimate(qg, kg, 128, 8, threshold=0.9)
    assert masks.shape == (1, 4, 64, 64) and sums.dtype == torch.bfloat16
    assert torch.equal(masks[0].cpu(), mask)


def test_xattn_full_length_properties():
    """Config-2 shape (L = 131072, 32 / 8 heads, stride 8): rows causal, first
    and diagonal blocks present, deterministic across calls, and
    every block row's sums add to its number of reshaped rows (one per
    probability row, up to the input dtype's rounding of each block)."""
    _case(L=131072, full=True)
    from fftsparse_amd.synth import make_config
    q, k, _ = make_config("c2")
    qg, kg = q.to(DEV), k.to(DEV)
    del q, k
    a = xattn_select(qg, kg, stride=8, threshold=0.9)
    b = xattn_select(qg, kg, stride=8, threshold=0.9)
    torch.cuda.synchronize()
    assert torch.equal(a.blk_cnt, b.blk_cnt) and torch.equal(a.blk_bits, b.blk_bits)
    H, N = a.blk_cnt.shape
    check_mask_words(a.blk_bits, a.blk_cnt, N)                       # causal, block 0, the diagonal
    row_mass = a.sums.sum(-1)                                        # [H, N]
    assert bool(((row_mass - 16.0).abs() <= 16.0 * 2 ** -7).all())
    print(f"  density {density(a):.4f}")


@pytest.mark.parametrize("L,Hq,Hk,stride", [
    (16, 1, 1, 8),            # shorter than one block: one partial row tile of 16 rows
    (100, 2, 1, 8),           # one block, ragged
    (129, 2, 1, 8),           # one token past a block
    (1025, 2, 2, 16),         # one token past 8 blocks
    (2049, 2, 1, 4),          # 513 reshaped rows: one row past 4 row tiles
])
def test_xattn_edge_lengths(L, Hq, Hk, stride):
    _case(L=L, Hq=Hq, Hk=Hk, stride=stride, edge=True)
    q, k, _ = make_qkv(L, Hq, Hk, dtype=torch.bfloat16, seed=32)
    _check(q, k, stride, 0.9, torch.bfloat16)
