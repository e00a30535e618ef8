"""GPU parity of XAttention's other paths (fs_xattn through the C ABI) against
the CPU oracle (oracle/xattn.py ``estimate``): causal=False on the Triton path
(softmax over the chunk-padded keys, find_blocks_chunked's non-causal branch),
and use_triton=False (Xattention.py:72-135, 170-258) with every reshaping, kdb,
softmax=False, with and without chunk padding; non-causal attention under the
lists.

Bars: block sums equal to the oracle's in the input dtype, or within two units
in the last place (the torch path rounds each probability and each row's block
sum, so one flipped rounding in a block's sum moves it by one unit), for >= 98%
of the compared blocks; block decisions exact, or excused where the mass before
the block is within 1e-3 relative of the row's required mass, for >= 99.9%;
attention within max-abs 2e-2 and mean-abs 1e-3 of fp32 attention under the
same mask.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from fftsparse_amd import _lib
from fftsparse_amd.synth import make_qkv
from fftsparse_amd.xattn import Xattention_prefill, default_chunk_size, xattn_estimate, xattn_select
from oracle import v7
from oracle import xattn as xo

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
BAND = 1e-3


def _ulp_diff(a: torch.Tensor, b: torch.Tensor, dtype) -> torch.Tensor:
    ai = a.to(dtype).view(torch.int16).to(torch.int32)
    bi = b.to(dtype).view(torch.int16).to(torch.int32)
    return (ai - bi).abs()


def _check(q, k, *, stride, threshold=0.9, causal=True, use_triton=True, select_mode="inverse", kdb=1,
           softmax=True, chunk_size=None, perm=None, keep_sink=False, keep_recent=False):
    dtype = q.dtype
    L = q.shape[2]
    chunk = default_chunk_size(L) if chunk_size is None else chunk_size
    print(f"[case] xattn-mode L={L} H={q.shape[1]}/{k.shape[1]} S={stride} causal={causal} triton={use_triton} "
          f"mode={select_mode} kdb={kdb} softmax={softmax} chunk={chunk} dtype={dtype}", flush=True)
    sel = xattn_select(q.to(DEV), k.to(DEV), stride=stride, threshold=threshold, causal=causal,
                       use_triton=use_triton, select_mode=select_mode, kdb=kdb, softmax=softmax,
                       chunk_size=chunk, perm=perm, keep_sink=keep_sink, keep_recent=keep_recent)
    torch.cuda.synchronize()
    mask_ref, sums_ref, margin, _ = xo.estimate(
        q, k, stride=stride, threshold=threshold, causal=causal, use_triton=use_triton, select_mode=select_mode,
        kdb=kdb, softmax=softmax, chunk_size=chunk, perm=perm, keep_sink=keep_sink, keep_recent=keep_recent)
    N = mask_ref.shape[1]
    region = torch.tril(torch.ones(N, N, dtype=torch.bool)) if causal else torch.ones(N, N, dtype=torch.bool)
    g_sums = sel.sums.cpu()
    ud = _ulp_diff(g_sums[:, region], sums_ref[:, region], dtype)
    eq = (ud == 0).float().mean().item()
    print(f"  sums: equal {eq:.5f}, max ulp {ud.max().item()}", flush=True)
    assert ud.max().item() <= 2
    assert eq >= 0.98
    g_mask = sel.dense_mask().cpu()
    diff = g_mask != mask_ref
    excused = margin.abs() <= BAND
    total = int(region.sum()) * g_mask.shape[0]
    unexc = int((diff & ~excused).sum())
    frac = (total - unexc) / total
    print(f"  decisions: exact {1 - int(diff.sum()) / total:.6f}, exact-or-excused {frac:.6f}, unexcused {unexc}, "
          f"density {g_mask.float().mean().item():.4f}", flush=True)
    assert frac >= 0.999
    if causal:
        body = g_mask.clone()
        if keep_sink:
            body[:, 0] = region[0]
        assert not (body & ~region).any()
        assert g_mask[:, :, 0].all() and g_mask[:, torch.arange(N), torch.arange(N)].all()
    else:
        assert g_mask[:, :, 0].all()                 # the reference always marks block 0
    if keep_sink:
        assert g_mask[:, 0].all()
    if keep_recent:
        assert g_mask[:, torch.arange(N), torch.arange(N)].all()
    return sel, g_mask


@pytest.mark.parametrize("L,Hq,Hk,stride,chunk", [
    (6000, 4, 2, 8, None),        # chunk 8192: 2192 padding keys in every row's softmax
    (4096, 2, 1, 16, 4096),       # no padding
    (4100, 2, 2, 4, 16384),       # the estimate's default chunk: 12284 padding keys
])
def test_noncausal_triton_parity(L, Hq, Hk, stride, chunk):
    q, k, _ = make_qkv(L, Hq, Hk, dtype=torch.bfloat16, seed=41)
    _check(q, k, stride=stride, causal=False, chunk_size=chunk)


def test_noncausal_keep_sink_keep_recent_fp16():
    q, k, _ = make_qkv(5000, 2, 1, dtype=torch.float16, seed=42)
    _check(q, k, stride=8, causal=False, threshold=0.6, keep_sink=True, keep_recent=True)


@pytest.mark.parametrize("L,stride,kdb,chunk", [
    (6000, 8, 1, None),           # padded: the padding key columns masked
    (6000, 8, 2, None),           # every second reshaped row, mask rows 1, 3, ...
    (4100, 4, 4, None),
    (8192, 8, 1, 4096),           # no padding: each row sees its own chunk only
    (4096, 16, 2, 2048),
])
def test_torch_path_inverse_parity(L, stride, kdb, chunk):
    q, k, _ = make_qkv(L, 4, 2, dtype=torch.bfloat16, seed=43)
    _check(q, k, stride=stride, use_triton=False, kdb=kdb, chunk_size=chunk)


@pytest.mark.parametrize("mode", ["slash", "random", "double", "triple"])
def test_torch_path_reshapings_parity(mode):
    q, k, _ = make_qkv(5000, 4, 2, dtype=torch.bfloat16, seed=44)
    perm = torch.randperm(8, generator=torch.Generator().manual_seed(5)) if mode == "random" else None
    _check(q, k, stride=8, use_triton=False, select_mode=mode, perm=perm)


@pytest.mark.parametrize("causal", [True, False])
def test_torch_path_no_softmax_parity(causal):
    q, k, _ = make_qkv(4500, 2, 1, dtype=torch.bfloat16, seed=45)
    _check(q, k, stride=8, use_triton=False, softmax=False, causal=causal)


def test_torch_path_noncausal_kdb_fp16():
    q, k, _ = make_qkv(6000, 2, 2, dtype=torch.float16, seed=46)
    _check(q, k, stride=8, use_triton=False, causal=False, kdb=2)


def test_random_mode_draws_the_reference_permutation():
    """perm=None draws torch.randperm(stride) from the global generator, as
    xattn_estimate does: the same seed gives the oracle's lists for that draw."""
    q, k, _ = make_qkv(4096, 2, 1, dtype=torch.bfloat16, seed=47)
    torch.manual_seed(123)
    a = xattn_select(q.to(DEV), k.to(DEV), stride=8, use_triton=False, select_mode="random").dense_mask().cpu()
    torch.manual_seed(123)
    perm = torch.randperm(8)
    b = xattn_select(q.to(DEV), k.to(DEV), stride=8, use_triton=False, select_mode="random",
                     perm=perm).dense_mask().cpu()
    assert torch.equal(a, b)


def test_noncausal_prefill_attention_parity():
    """Xattention_prefill(causal=False): non-causal attention under the kernel's
    own lists against fp32 attention under the same mask; xattn_estimate agrees."""
    L = 6000
    print(f"[case] xattn-mode noncausal prefill L={L}", flush=True)
    q, k, v = make_qkv(L, 4, 2, dtype=torch.bfloat16, seed=48)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    out = Xattention_prefill(qg, kg, vg, stride=8, threshold=0.9, causal=False)
    torch.cuda.synchronize()
    sel = xattn_select(qg, kg, stride=8, threshold=0.9, causal=False)
    mask = sel.dense_mask().cpu()
    ref = v7.block_sparse_attention(q, k, v, mask, 128, is_causal=False)
    err = (out[0].transpose(0, 1).float().cpu() - ref).abs()
    print(f"  density {mask.float().mean().item():.4f} max_abs={err.max().item():.3e} "
          f"mean_abs={err.mean().item():.3e}", flush=True)
    assert err.max().item() <= 2e-2 and err.mean().item() <= 1e-3
    sums, masks = xattn_estimate(qg, kg, 128, 8, threshold=0.9, causal=False, chunk_size=default_chunk_size(L))
    assert torch.equal(masks[0].cpu(), mask)


def test_torch_path_prefill_kdb_attention():
    """Xattention_prefill(use_triton=False, kdb=2): causal attention under its
    lists against fp32 attention."""
    L = 4096
    print(f"[case] xattn-mode torch-path prefill kdb=2 L={L}", flush=True)
    q, k, v = make_qkv(L, 2, 1, dtype=torch.bfloat16, seed=49)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    out = Xattention_prefill(qg, kg, vg, stride=8, threshold=0.9, use_triton=False, kdb=2)
    torch.cuda.synchronize()
    mask = xattn_select(qg, kg, stride=8, threshold=0.9, use_triton=False, kdb=2).dense_mask().cpu()
    ref = v7.block_sparse_attention(q, k, v, mask, 128)
    err = (out[0].transpose(0, 1).float().cpu() - ref).abs()
    print(f"  max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}", flush=True)
    assert err.max().item() <= 2e-2 and err.mean().item() <= 1e-3


@pytest.mark.parametrize("causal,use_triton", [(True, True), (False, True), (True, False)])
def test_head_groups_give_the_same_lists(causal, use_triton):
    """A workspace too small for every head's scores: the passes run head group
    by head group (here 1 head, and 2 when 3 of the 4 fit) and give the lists,
    sums and decisions of one pass over all heads."""
    L = 5000
    print(f"[case] xattn-mode head groups causal={causal} triton={use_triton} L={L}", flush=True)
    q, k, _ = make_qkv(L, 4, 2, dtype=torch.bfloat16, seed=50)
    qg, kg = q.to(DEV), k.to(DEV)
    kw = dict(stride=8, threshold=0.9, causal=causal, use_triton=use_triton)
    full = xattn_select(qg, kg, **kw)
    one = xattn_select(qg, kg, max_workspace_bytes=1, **kw)
    lib = _lib.load()

    def work(hg):
        a = _lib.XattnArgs(dtype=1, Hq=4, Hk=2, L=L, D=128, stride=8, bs=128, norm=1.0, non_causal=int(not causal),
                           torch_path=int(not use_triton), chunk=default_chunk_size(L), head_group=hg)
        return lib.fs_xattn_work_bytes(ctypes.byref(a))
    assert work(1) < work(3) < work(4)
    three = xattn_select(qg, kg, max_workspace_bytes=work(3), **kw)        # groups of 2 heads (3 do not divide 4)
    torch.cuda.synchronize()
    for x in (one, three):
        assert torch.equal(full.blk_cnt, x.blk_cnt)
        assert torch.equal(full.dense_mask(), x.dense_mask())
        assert torch.equal(full.sums, x.sums)
