"""Block-sparse attention (fs_bsattn through the C ABI) on seeded random
cases against fp32 attention under the same block mask: block sizes 16, 32,
64 and 128 (16 and 32 in union mode), ragged lengths, GQA group sizes 1, 2,
4 and 7, causal and not, fewer queries than keys (bottom-right aligned), bf16
and fp16, head dims 128 and 64, densities from 5% to every block, and empty
rows.  Bar: max-abs 2e-2 on six sampled query blocks of every head (rows with
no visible key: 0)."""
from __future__ import annotations

import random

import pytest
import torch

from tests.helpers import mask_bits

from fftsparse_amd import block_sparse_attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _case(i: int):
    rng = random.Random(7919 * (i + 1))
    bs = rng.choice([16, 32, 64, 128])
    Hk = rng.choice([1, 2, 4])
    g = rng.choice([1, 2, 4, 7])
    Lk = rng.randint(bs + 1, min(6000, 300 * bs))
    causal = rng.random() < 0.75
    Lq = Lk if (not causal or rng.random() < 0.7) else rng.randint(1, Lk)
    dtype = rng.choice([torch.bfloat16, torch.float16])
    dens = rng.choice([0.05, 0.3, 0.7, 1.0])
    empty_rows = rng.random() < 0.5
    return rng, bs, Hk, g, Lq, Lk, causal, dtype, dens, empty_rows


def _random_case(i: int, D: int):
    rng, bs, Hk, g, Lq, Lk, causal, dtype, dens, empty_rows = _case(i)
    Hq = Hk * g
    print(f"[case] random-attn {i}: D={D} bs={bs} Hq={Hq} Hk={Hk} Lq={Lq} Lk={Lk} causal={causal} {dtype} "
          f"density={dens} empty_rows={empty_rows}", flush=True)
    Nq, Nk = -(-Lq // bs), -(-Lk // bs)
    gen = torch.Generator().manual_seed(1000 + i)
    q = torch.randn(1, Hq, Lq, D, generator=gen).to(dtype)
    k = torch.randn(1, Hk, Lk, D, generator=gen).to(dtype)
    v = torch.randn(1, Hk, Lk, D, generator=gen).to(dtype)
    mask = torch.rand(Hq, Nq, Nk, generator=gen) < dens
    if empty_rows:
        mask[:, ::3] = False
    # the reference's base_blockmask form (bool [1, H, Nq, Nk]), packed to bits by the wrapper
    out = block_sparse_attention(q.to(DEV), k.to(DEV), v.to(DEV), block_mask=mask[None].to(DEV),
                                 block_size=bs, is_causal=causal)
    torch.cuda.synchronize()
    o = out[0].float().cpu()
    off, scale = Lk - Lq, D ** -0.5
    worst = 0.0
    for h in range(Hq):
        kh, vh = k[0, h // g].float(), v[0, h // g].float()
        for r in rng.sample(range(Nq), min(Nq, 6)):
            t0, t1 = r * bs, min(Lq, (r + 1) * bs)
            cols = torch.nonzero(mask[h, r]).flatten().tolist()
            ref = torch.zeros(t1 - t0, D)
            if cols:
                kidx = torch.cat([torch.arange(j * bs, min(Lk, (j + 1) * bs)) for j in cols])
                s = (q[0, h, t0:t1].float() @ kh[kidx].T) * scale
                if causal:
                    s = s.masked_fill(kidx[None, :] > torch.arange(t0, t1)[:, None] + off, float("-inf"))
                ref = torch.nan_to_num(torch.softmax(s, -1), nan=0.0) @ vh[kidx]
            worst = max(worst, (o[t0:t1, h] - ref).abs().max().item())
    print(f"  max_abs {worst:.3e}", flush=True)
    assert worst <= 2e-2


@pytest.mark.parametrize("i", range(100))
def test_random_lists_against_fp32(i):
    _random_case(i, 128)


@pytest.mark.parametrize("i", range(100, 132))
def test_random_lists_against_fp32_head_dim_64(i):
    """Head dim 64 (block_sparse_attn's other supported size): K tiles of
    128-byte rows, the same V^T layout."""
    _random_case(i, 64)


@pytest.mark.parametrize("bs,Lk", [(16, 131072), (32, 200000)])
def test_union_lists_beyond_4096_key_blocks(bs, Lk):
    """16- and 32-token masks over more than 4096 key blocks (8192 and 6250):
    rows of 128 64-bit words, and union lists over them.  Random masks at 3%,
    causal; sampled query blocks (both ends and around block 4096) against fp32."""
    Hk, g = 1, 2
    Hq = Hk * g
    print(f"[case] union-attn bs={bs} Lk={Lk} Hq={Hq}", flush=True)
    N = -(-Lk // bs)
    gen = torch.Generator().manual_seed(31 + bs)
    q = torch.randn(1, Hq, Lk, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(1, Hk, Lk, 128, generator=gen).to(torch.bfloat16)
    v = torch.randn(1, Hk, Lk, 128, generator=gen).to(torch.bfloat16)
    mask = torch.rand(Hq, N, N, generator=gen) < 0.03
    mask |= torch.eye(N, dtype=torch.bool)[None]
    mask &= torch.tril(torch.ones(N, N, dtype=torch.bool))[None]
    cnt, bits = mask_bits(mask, DEV)
    out = block_sparse_attention(q.to(DEV), k.to(DEV), v.to(DEV), cnt, bits, block_size=bs, is_causal=True)
    torch.cuda.synchronize()
    o = out[0].float().cpu()
    scale, worst = 128 ** -0.5, 0.0
    for h in range(Hq):
        kh, vh = k[0, h // g].float(), v[0, h // g].float()
        for r in (0, 5, 4095, 4096, 4097, N - 2, N - 1):
            t0, t1 = r * bs, min(Lk, (r + 1) * bs)
            cols = torch.nonzero(mask[h, r]).flatten().tolist()
            kidx = torch.cat([torch.arange(j * bs, min(Lk, (j + 1) * bs)) for j in cols])
            s = (q[0, h, t0:t1].float() @ kh[kidx].T) * scale
            s = s.masked_fill(kidx[None, :] > torch.arange(t0, t1)[:, None], float("-inf"))
            ref = torch.softmax(s, -1) @ vh[kidx]
            worst = max(worst, (o[t0:t1, h] - ref).abs().max().item())
    print(f"  max_abs {worst:.3e}", flush=True)
    assert worst <= 2e-2


@pytest.mark.parametrize("bs,L,Hq,Hk", [
    (128, 1024, 2, 1),        # 8 query blocks x 2 heads: 16 work units, the shared pool takes 1
    (128, 640, 1, 1),         # 5 work units: no shared pool (fewer than 10 units)
    (128, 16384, 2, 1),       # 128 query blocks: runs of 2 query blocks per work unit
    (64, 16384, 2, 2),        # block 64: 256 query blocks, runs of 4
    (32, 16384, 2, 1),        # union mode: groups of 4 rows of 32-token blocks
    (16, 16384, 2, 1),        # union mode: groups of 8 rows of 16-token blocks
])
def test_every_query_block_is_written(bs, L, Hq, Hk):
    """The work-unit tickets reach every query block: the output buffer is
    filled with NaN before the call (AttentionCall(out=...)), and every row of
    every head must come back finite and within max-abs 2e-2 / mean-abs 1e-3
    of fp32 attention under the same mask (every block row holds its
    diagonal block, so no row is empty)."""
    from fftsparse_amd import AttentionCall
    from oracle import v7
    print(f"[case] all-rows bs={bs} L={L} Hq={Hq} Hk={Hk}", flush=True)
    gen = torch.Generator().manual_seed(4242 + bs + L)
    q = torch.randn(1, Hq, L, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(1, Hk, L, 128, generator=gen).to(torch.bfloat16)
    v = torch.randn(1, Hk, L, 128, generator=gen).to(torch.bfloat16)
    N = -(-L // bs)
    mask = torch.rand(Hq, N, N, generator=gen) < (0.15 if N > 64 else 0.5)
    mask |= torch.eye(N, dtype=torch.bool)[None]
    mask &= torch.tril(torch.ones(N, N, dtype=torch.bool))[None]
    cnt, bits = mask_bits(mask, DEV)
    out = torch.full((1, L, Hq, 128), float("nan"), dtype=torch.bfloat16, device=DEV)
    AttentionCall(q.to(DEV), k.to(DEV), v.to(DEV), cnt, bits, block_size=bs, out=out)()
    torch.cuda.synchronize()
    o = out[0].float().cpu()
    assert bool(torch.isfinite(o).all()), f"{int((~torch.isfinite(o)).sum())} output values never written"
    ref = v7.block_sparse_attention(q, k, v, mask, bs)
    err = (o - ref).abs()
    print(f"  max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}", flush=True)
    assert err.max().item() <= 2e-2 and err.mean().item() <= 1e-3
