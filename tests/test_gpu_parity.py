"""GPU parity: the HIP path (through the C ABI) against the CPU oracle.

Bars: block decisions exact except those within 1e-3
relative of their selection threshold, >= 99.9% of all causal decisions;
attention under the reference mask within max-abs 2e-2 and mean-abs 1e-3 of
fp32 attention; integer outputs (block lists) bit-exact and deterministic.
"""
from __future__ import annotations

import math

import pytest
import torch

from fftsparse_amd import _lib, block_sparse_attention, fix_mask, myattn_prefill, rope_pool, select_blocks
from fftsparse_amd.synth import make_qkv, make_config
from oracle import v7
from tests.helpers import BAND, MATCH_MIN, PROD, block_match, check_mask_rows, mask_bits, rope_tables

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _gpu(*ts):
    return [t.to(DEV) for t in ts]


def _orig_layout(xb, Hq):
    """GPU pooled [H,N,D] -> oracle layout [N,Hq,D] (key heads repeated)."""
    H = xb.shape[0]
    x = xb.permute(1, 0, 2).cpu()
    return x.repeat_interleave(Hq // H, dim=1) if H != Hq else x


def _print_case(case, **kw):
    print(f"[case] {case} " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


# --------------------------------------------------------------------------- pooling
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("L,bs", [(8192, 128), (5000, 128), (4096, 64)])
def test_pool_parity(dtype, L, bs):
    _print_case("pool", dtype=dtype, L=L, bs=bs)
    q, k, _ = make_qkv(L, 4, 2, dtype=dtype, seed=1)
    sel = select_blocks(*_gpu(q, k), **{**PROD, "block_size": bs}, keep_intermediates=True)
    torch.cuda.synchronize()
    ref_q = v7.block_mean_pool(v7.to_lhd(q), bs)
    ref_k = v7.block_mean_pool(v7.to_lhd(k), bs)
    for got, ref in ((sel.q_b, ref_q), (sel.k_b, ref_k)):
        got = got.permute(1, 0, 2).cpu()
        if dtype == torch.float32:
            torch.testing.assert_close(got, ref, rtol=2e-6, atol=1e-7)
        else:
            # one rounding of an fp32 sum: at most one ulp apart, almost always equal
            gi = got.view(torch.int16).to(torch.int32)
            ri = ref.view(torch.int16).to(torch.int32)
            assert (gi - ri).abs().max().item() <= 1
            assert (gi == ri).float().mean().item() >= 0.999


# --------------------------------------------------------------------------- RoPE + pooling
def _fs_pool(q, k, bs):
    """fs_pool alone on [1,H,L,D] views -> (q_b [Hq,N,D], k_b [Hk,N,D])."""
    Hq, L, D = q.shape[1:]
    N = (L + bs - 1) // bs
    q_b = torch.empty(Hq, N, D, dtype=q.dtype, device=DEV)
    k_b = torch.empty(k.shape[1], N, D, dtype=q.dtype, device=DEV)
    _lib.call("fs_pool", _lib.PoolArgs(q=q.data_ptr(), q_sh=q.stride(1), q_sl=q.stride(2), k=k.data_ptr(),
                                       k_sh=k.stride(1), k_sl=k.stride(2), dtype=_lib.FS_DTYPE[q.dtype], Hq=Hq,
                                       Hk=k.shape[1], L=L, D=D, bs=bs, q_b=q_b.data_ptr(), k_b=k_b.data_ptr()))
    return q_b, k_b


def _proj_layout(L, H, dtype, g, scale=3.0):
    """A projection's output as the attention forward sees it: [1,H,L,D] view of [1,L,H,D] storage."""
    return (torch.randn(1, L, H, 128, generator=g) * scale).to(dtype).to(DEV).transpose(1, 2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("L,bs,Hq,Hk", [(8192, 128, 4, 1), (5000, 128, 4, 2), (4100, 64, 8, 8)])
def test_rope_pool_parity(dtype, L, bs, Hq, Hk):
    """fs_rope_pool: rotated Q/K bit-identical to transformers' apply_rotary_pos_emb
    on the GPU (the reference's RoPE step) and to the oracle; block means
    bit-identical to fs_pool on the rotated tensors."""
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    _print_case("rope_pool", dtype=dtype, L=L, bs=bs, Hq=Hq, Hk=Hk)
    g = torch.Generator().manual_seed(21)
    q, k = _proj_layout(L, Hq, dtype, g), _proj_layout(L, Hk, dtype, g)
    cos, sin = rope_tables(L, 128, 500000.0, dtype)
    cg, sg = cos.to(DEV), sin.to(DEV)
    q_rot, k_rot, q_b, k_b = rope_pool(q, k, cg, sg, block_size=bs)
    ref_q, ref_k = apply_rotary_pos_emb(q, k, cg[None], sg[None])
    assert torch.equal(q_rot, ref_q) and torch.equal(k_rot, ref_k)
    assert torch.equal(q_rot.cpu(), v7.rotary_embedding(q.cpu(), cos, sin))
    assert q_rot.stride() == ref_q.stride()
    p_q, p_k = _fs_pool(q_rot, k_rot, bs)
    assert torch.equal(q_b, p_q) and torch.equal(k_b, p_k)


def test_select_blocks_on_fused_means_equals_unfused():
    """select_blocks(pooled=rope_pool's means) gives the block lists of
    select_blocks on the rotated tensors (bf16, config-0 shape)."""
    g = torch.Generator().manual_seed(22)
    q, k = _proj_layout(8192, 4, torch.bfloat16, g, 1.0), _proj_layout(8192, 1, torch.bfloat16, g, 1.0)
    cos, sin = rope_tables(8192, 128, 500000.0, torch.bfloat16)
    q_rot, k_rot, q_b, k_b = rope_pool(q, k, cos.to(DEV), sin.to(DEV))
    a = select_blocks(q_rot, k_rot, **PROD)
    b = select_blocks(q_rot, k_rot, pooled=(q_b, k_b), **PROD)
    assert torch.equal(a.blk_cnt, b.blk_cnt)
    assert torch.equal(a.dense_mask(), b.dense_mask())
    with pytest.raises(ValueError):
        select_blocks(q_rot, k_rot, pooled=(q_b[:, :-1], k_b), **PROD)


# --------------------------------------------------------------------------- FFT correlation
@pytest.mark.parametrize("dtype,L,Hq,Hk", [(torch.float32, 8192, 4, 1), (torch.bfloat16, 32768, 8, 2),
                                         (torch.bfloat16, 20000, 4, 4)])
def test_corr_parity(dtype, L, Hq, Hk):
    _print_case("corr", dtype=dtype, L=L, Hq=Hq, Hk=Hk)
    q, k, _ = make_qkv(L, Hq, Hk, dtype=dtype, seed=2)
    sel = select_blocks(*_gpu(q, k), **PROD, keep_intermediates=True)
    torch.cuda.synchronize()
    p = sel.params
    Qb, Kb = _orig_layout(sel.q_b, Hq), _orig_layout(sel.k_b, Hq)
    corr_ref, corr_sum_ref = v7.fft_lag_correlation(Qb, Kb, p.local_window, p.keep_sink)
    # closed form: the lag sums are the diagonal sums of Q_b K_b^T
    S = torch.einsum("ihd,jhd->hij", Qb.double(), Kb.double())
    diag = torch.stack([torch.diagonal(S, offset=-t, dim1=1, dim2=2).sum(-1) for t in range(p.N)], -1)
    scale = diag.abs().max().item()
    assert (sel.corr_sum.cpu().double() - diag).abs().max().item() <= 2e-5 * scale
    assert (corr_sum_ref.double() - diag).abs().max().item() <= 2e-5 * scale
    keep_ref, norm_ref = v7.correlation_keep(corr_ref, p.remote_start, PROD["corr_threshold"])
    keep = sel.keep_tau.cpu().bool()
    diff = keep != keep_ref
    near = ((norm_ref - PROD["corr_threshold"]).abs() <= BAND * PROD["corr_threshold"])
    assert not (diff & ~near).any(), f"lag decisions differ outside the band: {torch.nonzero(diff & ~near)}"
    cmax = corr_ref[:, p.remote_start:].abs().max()
    torch.testing.assert_close(sel.corr.cpu(), corr_ref, rtol=0, atol=float(2e-4 * cmax))


# --------------------------------------------------------------------------- statistics
@pytest.mark.parametrize("dtype,L,Hq,Hk", [(torch.float32, 8192, 4, 1), (torch.bfloat16, 32768, 8, 2)])
def test_stats_parity(dtype, L, Hq, Hk):
    _print_case("stats", dtype=dtype, L=L)
    q, k, _ = make_qkv(L, Hq, Hk, dtype=dtype, seed=3)
    sel = select_blocks(*_gpu(q, k), **PROD, keep_intermediates=True)
    torch.cuda.synchronize()
    p = sel.params
    Qb, Kb = _orig_layout(sel.q_b, Hq), _orig_layout(sel.k_b, Hq)
    S = v7.block_scores(Qb, Kb)
    # per-sample normalised diagonal variance
    for si, tau in enumerate(p.sample_taus):
        dv = torch.diagonal(S, offset=-tau, dim1=1, dim2=2)[:, :-1].double()
        ref = dv.diff(dim=-1).var(dim=-1) / dv.abs().mean(-1).clamp(min=1e-6)
        torch.testing.assert_close(sel.diag_var[:, si].cpu().double(), ref, rtol=2e-4, atol=1e-9)
    mv_ref, st_ref = v7.stripe_variance(S, p.remote_start, p.sample_taus, PROD["stripe_threshold"],
                                        p.stripe_all_diffuse)
    torch.testing.assert_close(sel.mean_var.cpu(), mv_ref, rtol=2e-4, atol=1e-9)
    # column scores + top-n
    cm_ref = v7.column_scores(Qb, Kb)
    scale = cm_ref.abs().max().item()
    torch.testing.assert_close(sel.col_mean.cpu(), cm_ref, rtol=0, atol=2e-5 * scale)
    cs_ref, kth = v7.column_select(cm_ref, p)
    diff = sel.col_sel.cpu().bool() != cs_ref
    near = (cm_ref - kth[:, None]).abs() <= BAND * kth.abs()[:, None]
    assert not (diff & ~near).any()
    # last row: scores rounded to the input dtype (one rounding apart at most)
    ls_ref = v7.last_row_scores(Qb, Kb).float()
    gs = sel.last_scores.cpu()
    torch.testing.assert_close(gs, ls_ref, rtol=8e-3 if dtype != torch.float32 else 1e-5, atol=1e-6)
    sel_ref, _, kth = v7.last_row_topk(Qb, Kb, p.last_k)
    diff = sel.last_sel.cpu().bool() != sel_ref
    near = ((ls_ref - kth[:, None]).abs() <= BAND * kth.abs()[:, None]) | (gs != ls_ref)
    assert not (diff & ~near).any()


# --------------------------------------------------------------------------- full selection
SEL_CASES = [
    ("c0", dict()),
    ("c0-diffuse", dict(stripe_threshold=0.0)),
    ("c0-nocorr", dict(enable_correlation_mask=False)),
    ("c0-nocol-nolast", dict(enable_column_mask=False, enable_last_block_mask=False)),
    ("c0-defaults", "defaults"),
    ("c0-T0.95", dict(corr_threshold=0.95)),
    ("c0-topk", dict(correlation_selection_mode="topk")),
    ("c0-topk-0.05", dict(correlation_selection_mode="topk", correlation_topk_ratio=0.05)),
]


@pytest.mark.parametrize("name,over", SEL_CASES)
def test_selection_parity_c0(name, over):
    _print_case("selection", name=name)
    q, k, _ = make_config("c0")
    kw = {} if over == "defaults" else {**PROD, **over}
    sel = select_blocks(*_gpu(q, k), **kw)
    ref = v7.select_mask(q, k, **kw)
    frac, exact, unexc = block_match(sel.dense_mask(), ref.mask, ref.excusable)
    print(f"  match={frac:.6f} exact={exact:.6f} unexcused={unexc}")
    assert frac >= MATCH_MIN
    if ref.is_stripe is not None:
        gs = sel.is_stripe.cpu().bool()
        near = (ref.mean_var - PROD["stripe_threshold"]).abs() <= BAND * PROD["stripe_threshold"]
        assert not ((gs != ref.is_stripe) & ~near).any()


@pytest.mark.parametrize("L,Hq,Hk,bs,dtype,over", [
    (32768, 32, 8, 128, torch.bfloat16, {}),                     # config 1 shape
    (32768, 8, 2, 128, torch.bfloat16, dict(stripe_threshold=0.0)),
    (24000, 7, 1, 64, torch.bfloat16, {}),                       # ragged L, bs 64, GQA 7
    (16384, 4, 4, 128, torch.float16, dict(corr_threshold=0.5)),
    (32768, 8, 2, 128, torch.bfloat16, dict(correlation_selection_mode="topk")),
    (24000, 7, 1, 64, torch.bfloat16, dict(correlation_selection_mode="topk", correlation_topk_ratio=0.3)),
    (300000, 4, 1, 64, torch.bfloat16, {}),                      # N = 4688 > 4096 blocks
    (300000, 2, 1, 64, torch.bfloat16, dict(stripe_threshold=0.0)),   # diffuse heads' score panel at N = 4688
    (131072, 2, 1, 16, torch.bfloat16, {}),                      # N = 8192, the selection kernels' maximum
    (131072, 1, 1, 16, torch.bfloat16, dict(stripe_threshold=0.0)),   # a diffuse head's panel at N = 8192
])
def test_selection_parity_bf16(L, Hq, Hk, bs, dtype, over):
    _print_case("selection", L=L, Hq=Hq, Hk=Hk, bs=bs, dtype=dtype, over=over)
    q, k, _ = make_qkv(L, Hq, Hk, dtype=dtype, seed=4)
    kw = {**PROD, "block_size": bs, **over}
    sel = select_blocks(*_gpu(q, k), **kw)
    ref = v7.select_mask(q, k, **kw)
    frac, exact, unexc = block_match(sel.dense_mask(), ref.mask, ref.excusable)
    print(f"  match={frac:.6f} exact={exact:.6f} unexcused={unexc}")
    assert frac >= MATCH_MIN


@pytest.mark.parametrize("dtype,ratio", [(torch.float32, 0.2), (torch.bfloat16, 0.2), (torch.bfloat16, 0.01),
                                         (torch.bfloat16, 0.999)])
def test_topk_lag_keep_matches_quantile_of_own_corr(dtype, ratio):
    """The "topk" lag selection (my_attn_v7.py:196-203) applied by the kernel
    to its own corr values equals torch.quantile's selection on the same
    values, up to values within 1e-6 of the quantile (the lerp's rounding)."""
    _print_case("topk keep", dtype=dtype, ratio=ratio)
    q, k, _ = make_qkv(16384, 8, 2, dtype=dtype, seed=6)
    kw = {**PROD, "correlation_selection_mode": "topk", "correlation_topk_ratio": ratio}
    sel = select_blocks(*_gpu(q, k), keep_intermediates=True, **kw)
    corr = sel.corr.cpu()
    rs = sel.params.remote_start
    keep_ref, qv = v7.correlation_keep_topk(corr, rs, ratio)
    keep = sel.keep_tau.cpu().bool()
    near = (corr - qv[:, None]).abs() <= 1e-6 * qv.abs()[:, None]
    assert not ((keep != keep_ref) & ~near).any()
    assert not keep[:, :rs].any()
    assert (keep.sum(-1) >= 1).all()


def test_block_mask_is_causal_and_deterministic():
    """The block mask of two identical calls is the same word for word (every
    word written), each row's count is its popcount, and the sampled rows are
    causal with the sink block and the diagonal."""
    q, k, _ = make_qkv(32768, 8, 2, seed=5)
    qg, kg = _gpu(q, k)
    a = select_blocks(qg, kg, **PROD)
    b = select_blocks(qg, kg, **PROD)
    assert torch.equal(a.blk_cnt, b.blk_cnt)
    assert torch.equal(a.blk_bits, b.blk_bits)
    N = a.params.N
    m = a.dense_mask().cpu()
    assert torch.equal(m.sum(-1, dtype=torch.int32), a.blk_cnt.cpu())
    check_mask_rows(m, range(0, N, 17))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_pipeline_grouping_does_not_change_the_mask(dtype):
    """The head-group pipeline (pooling of one group overlapping the statistics
    of the previous one on a side stream) gives a bit-identical block mask and
    statistics for every grouping."""
    q, k, _ = make_qkv(32768, 8, 4, dtype=dtype, seed=9)
    qg, kg = _gpu(q, k)
    ref = select_blocks(qg, kg, **PROD, keep_intermediates=True, pipeline_groups=1)
    for groups in (2, 4):
        got = select_blocks(qg, kg, **PROD, keep_intermediates=True, pipeline_groups=groups)
        torch.cuda.synchronize()
        assert torch.equal(got.dense_mask(), ref.dense_mask()), groups
        for f in ("corr", "keep_tau", "diag_var", "col_mean", "last_scores", "mean_var"):
            assert torch.equal(getattr(got, f), getattr(ref, f)), (groups, f)


# --------------------------------------------------------------------------- attention
def _attn_check(out, ref, rows=None):
    o = out.float().cpu()
    if rows is not None:
        o, ref = o[rows], ref[rows]
    err = (o - ref).abs()
    print(f"  max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}")
    assert err.max().item() <= 2e-2
    assert err.mean().item() <= 1e-3


@pytest.mark.parametrize("L,Hq,Hk,bs,dtype", [
    (8192, 4, 1, 128, torch.bfloat16),
    (6000, 4, 2, 128, torch.bfloat16),
    (4096, 4, 1, 64, torch.bfloat16),
    (8192, 4, 4, 128, torch.float16),
    (4000, 4, 2, 32, torch.bfloat16),        # 32-token blocks: 125 key blocks (odd), ragged L
])
def test_attention_parity_reference_mask(L, Hq, Hk, bs, dtype):
    """Stage 2 alone, under the oracle's mask."""
    _print_case("attention", L=L, Hq=Hq, Hk=Hk, bs=bs, dtype=dtype)
    q, k, v = make_qkv(L, Hq, Hk, dtype=dtype, seed=6)
    ref_sel = v7.select_mask(q, k, **{**PROD, "block_size": bs})
    cnt, bits = mask_bits(ref_sel.mask, DEV)
    out = block_sparse_attention(*_gpu(q, k, v), cnt, bits, block_size=bs)
    torch.cuda.synchronize()
    ref = v7.block_sparse_attention(q, k, v, ref_sel.mask, bs)
    _attn_check(out[0], ref)


def test_attention_noncausal_and_dense():
    q, k, v = make_qkv(2048, 4, 2, seed=7)
    N = 16
    mask = torch.rand(4, N, N, generator=torch.Generator().manual_seed(0)) < 0.3
    mask |= torch.eye(N, dtype=torch.bool)
    cnt, bits = mask_bits(mask, DEV)
    out = block_sparse_attention(*_gpu(q, k, v), cnt, bits, block_size=128, is_causal=False)
    ref = v7.block_sparse_attention(q, k, v, mask, 128, is_causal=False)
    _attn_check(out[0], ref)
    out = block_sparse_attention(*_gpu(q, k, v), block_size=128, is_causal=True)
    ref = v7.dense_causal_attention(q, k, v)[0]
    _attn_check(out[0], ref)


@pytest.mark.parametrize("growth", [300.0, 3000.0])
def test_attention_running_max_raises(growth):
    """Scores that grow along the keys (k_t carries t/L * growth along q's
    shared direction): the running max is raised on nearly every tile, and at
    growth 3000 the exponentials taken against the stale max overflow to inf
    before the check replaces them.  Dense causal and listed (every causal
    block, ascending) paths, every block size."""
    _print_case("attention-raise", growth=growth)
    L, D = 2048, 128
    g = torch.Generator().manual_seed(11)
    u = torch.randn(D, generator=g)
    u /= u.norm()
    q = torch.randn(1, 2, L, D, generator=g) + 10.0 * u
    ramp = (torch.arange(L, dtype=torch.float32) / L * growth)[:, None]
    k = torch.randn(1, 1, L, D, generator=g) + ramp * u
    v = torch.randn(1, 1, L, D, generator=g)
    q, k, v = (x.to(torch.bfloat16) for x in (q, k, v))
    ref = v7.dense_causal_attention(q, k, v)[0]
    out = block_sparse_attention(*_gpu(q, k, v), block_size=128, is_causal=True)
    _attn_check(out[0], ref)
    for bs in (128, 64, 32, 16):
        N = L // bs
        mask = torch.tril(torch.ones(2, N, N, dtype=torch.bool))
        cnt, bits = mask_bits(mask, DEV)
        out = block_sparse_attention(*_gpu(q, k, v), cnt, bits, block_size=bs)
        _attn_check(out[0], ref)


@pytest.mark.parametrize("bs", [32, 16])
@pytest.mark.parametrize("L,Hq,Hk,dtype,density,causal", [
    (4000, 4, 2, torch.bfloat16, 0.3, True),      # 125 key blocks at 32 (250 at 16): odd union lengths
    (2048, 2, 1, torch.float16, 0.5, True),
    (1000, 2, 2, torch.bfloat16, 0.4, False),     # non-causal, ragged
    (3000, 4, 1, torch.bfloat16, 0.05, True),     # sparse rows: union entries selected by one row only
])
def test_attention_short_blocks(bs, L, Hq, Hk, dtype, density, causal):
    """16- and 32-token blocks (a workgroup of 128 queries walks the union of
    its 128 / bs rows' lists, masking per row) under random block lists of odd
    and even lengths, against fp32 attention under the same mask; and the
    dense causal path at that block size."""
    _print_case("attention-short-blocks", bs=bs, L=L, Hq=Hq, Hk=Hk, dtype=dtype, density=density, causal=causal)
    q, k, v = make_qkv(L, Hq, Hk, dtype=dtype, seed=12)
    N = (L + bs - 1) // bs
    g = torch.Generator().manual_seed(13)
    mask = torch.rand(Hq, N, N, generator=g) < density
    mask |= torch.eye(N, dtype=torch.bool)
    mask[:, :, 0] = True
    if causal:
        mask &= torch.ones(N, N, dtype=torch.bool).tril()
    mask[0, 5] = False                          # a row holding only ...
    mask[0, 5, 5] = True                        # ... its diagonal block
    mask[-1, 9] = False                         # a row with no block at all (output 0)
    cnt, bits = mask_bits(mask, DEV)
    out = block_sparse_attention(*_gpu(q, k, v), cnt, bits, block_size=bs, is_causal=causal)
    torch.cuda.synchronize()
    ref = v7.block_sparse_attention(q, k, v, mask, bs, is_causal=causal)
    _attn_check(out[0], ref)
    if causal:
        out = block_sparse_attention(*_gpu(q, k, v), block_size=bs, is_causal=True)
        _attn_check(out[0], v7.dense_causal_attention(q, k, v)[0])


def test_attention_prepare_run_equals_single_call():
    """fs_bsattn_prepare + fs_bsattn_run give fs_bsattn's output bit for bit,
    and run() may be repeated on one prepared workspace."""
    from fftsparse_amd import AttentionCall
    q, k, v = make_qkv(3000, 4, 2, dtype=torch.bfloat16, seed=8)
    N = (3000 + 127) // 128
    mask = torch.rand(4, N, N, generator=torch.Generator().manual_seed(1)) < 0.4
    mask = (mask | torch.eye(N, dtype=torch.bool)) & torch.ones(N, N, dtype=torch.bool).tril()
    cnt, bits = mask_bits(mask, DEV)
    qg, kg, vg = _gpu(q, k, v)
    whole = block_sparse_attention(qg, kg, vg, cnt, bits).clone()
    call = AttentionCall(qg, kg, vg, cnt, bits)
    call.prepare()
    first = call.run().clone()
    second = call.run()
    torch.cuda.synchronize()
    assert torch.equal(first, whole) and torch.equal(second, whole)


def test_myattn_prefill_end_to_end_c1_shape():
    """myattn_prefill on config 1's shape: output vs fp32 attention under the
    oracle mask on a sample of query blocks of every head."""
    _print_case("myattn_prefill", config="c1")
    q, k, v = make_config("c1")
    qg, kg, vg = _gpu(q, k, v)
    out = myattn_prefill(qg, kg, vg, layer_idx=0, **PROD)
    torch.cuda.synchronize()
    assert out.shape == (1, q.shape[2], q.shape[1] * q.shape[3]) and out.dtype == q.dtype
    ref_sel = v7.select_mask(q, k, **PROD)
    sel = select_blocks(qg, kg, **PROD)
    frac, exact, unexc = block_match(sel.dense_mask(), ref_sel.mask, ref_sel.excusable)
    print(f"  match={frac:.6f} exact={exact:.6f}")
    assert frac >= MATCH_MIN
    qblocks = [0, 1, 37, 128, 200, 255]
    ref = v7.block_sparse_attention(q, k, v, sel.dense_mask().cpu(), 128, qblocks=qblocks)
    rows = torch.cat([torch.arange(i * 128, (i + 1) * 128) for i in qblocks])
    _attn_check(out.view(q.shape[2], q.shape[1], q.shape[3]), ref, rows)


@pytest.mark.parametrize("bs", [128, 64])
def test_myattn_prefill_head_dim_64(bs):
    """Head dim 64: the selection against the oracle's, and myattn_prefill's
    output against fp32 attention under its own lists on sampled query blocks
    of every head."""
    _print_case("myattn_prefill", D=64, bs=bs)
    q, k, v = make_qkv(32768, 8, 2, D=64, dtype=torch.bfloat16, seed=9)
    qg, kg, vg = _gpu(q, k, v)
    kw = {**PROD, "block_size": bs}
    out = myattn_prefill(qg, kg, vg, layer_idx=0, **kw)
    sel = select_blocks(qg, kg, **kw)
    torch.cuda.synchronize()
    assert out.shape == (1, q.shape[2], q.shape[1] * 64) and out.dtype == q.dtype
    ref_sel = v7.select_mask(q, k, **kw)
    frac, exact, unexc = block_match(sel.dense_mask(), ref_sel.mask, ref_sel.excusable)
    print(f"  match={frac:.6f} exact={exact:.6f}")
    assert frac >= MATCH_MIN
    N = sel.params.N
    qblocks = [0, 1, N // 3, N // 2, N - 2, N - 1]
    ref = v7.block_sparse_attention(q, k, v, sel.dense_mask().cpu(), bs, qblocks=qblocks)
    rows = torch.cat([torch.arange(i * bs, (i + 1) * bs) for i in qblocks])
    _attn_check(out.view(q.shape[2], q.shape[1], 64), ref, rows)


def test_short_sequence_fallback_is_dense_causal():
    q, k, v = make_qkv(1000, 4, 2, seed=8)                      # L < 10 * bs
    out = myattn_prefill(*_gpu(q, k, v), layer_idx=0, **PROD)
    assert out.shape == (1, 1000, 4 * 128)
    ref = v7.dense_causal_attention(q, k, v)[0]
    _attn_check(out.view(1000, 4, 128), ref)


def test_fix_mask_role():
    q, k, v = make_qkv(8192, 4, 4, seed=9)
    out = fix_mask.myattn_prefill(*_gpu(q, k, v), layer_idx=0, sink_ratio=0.05, recent_ratio=0.05,
                                  local_span_ratio=0.1)
    N = 64
    ks, kr, lw = max(1, int(N * 0.05)), max(1, int(N * 0.05)), max(2, int(N * 0.1)) // 2
    mask = v7.fixed_mask(N, N, 4, ks, kr, lw)
    ref = v7.block_sparse_attention(q, k, v, mask, 128, is_causal=True)
    _attn_check(out.view(8192, 4, 128), ref)


def test_fp32_attention_rejected_like_flash_attn():
    q, k, v = make_config("c0", L=2048)
    with pytest.raises(RuntimeError, match="fp16 and bf16"):
        myattn_prefill(*_gpu(q, k, v), layer_idx=0, **PROD)


def test_full_length_c2_properties():
    """Config 2 length (128K) on device-generated data: pooled blocks against
    the oracle's downstream stages, plus invariants of the block lists."""
    _print_case("c2-properties")
    g = torch.Generator(device=DEV).manual_seed(11)
    L, Hq, Hk = 131072, 32, 8
    q = torch.randn(1, Hq, L, 128, device=DEV, generator=g, dtype=torch.bfloat16)
    k = torch.randn(1, Hk, L, 128, device=DEV, generator=g, dtype=torch.bfloat16)
    k[:, :, :4] *= 6
    sel = select_blocks(q, k, **PROD, keep_intermediates=True)
    torch.cuda.synchronize()
    p = sel.params
    assert p.N == 1024
    Qb, Kb = _orig_layout(sel.q_b, Hq), _orig_layout(sel.k_b, Hq)
    corr_ref, _ = v7.fft_lag_correlation(Qb, Kb, p.local_window, p.keep_sink)
    keep_ref, norm_ref = v7.correlation_keep(corr_ref, p.remote_start, PROD["corr_threshold"])
    near = (norm_ref - PROD["corr_threshold"]).abs() <= BAND * PROD["corr_threshold"]
    assert not ((sel.keep_tau.cpu().bool() != keep_ref) & ~near).any()
    cnt = sel.blk_cnt.cpu()
    assert int(cnt.min()) >= 1 and bool((cnt <= torch.arange(1, p.N + 1)[None, :]).all())
    m = sel.dense_mask().cpu()
    assert torch.equal(m.sum(-1, dtype=torch.int32), cnt)
    check_mask_rows(m[[0, 13, 31]], (0, 511, 1023))


def test_maximum_block_count_properties():
    """The largest supported selection, N = 8192 blocks (L = 1048576 at block
    128): rows causal, with the sink block and the diagonal, counts equal to
    the rows' popcounts; selection deterministic; attention output finite,
    and on sampled query blocks within the bars of fp32 attention under the
    same lists.  The mask takes N * N / 8 bytes per head (8 MiB)."""
    _print_case("max-blocks", L=8192 * 128, Hq=2, Hk=1)
    g = torch.Generator(device=DEV).manual_seed(12)
    L, Hq, Hk = 8192 * 128, 2, 1
    q = torch.randn(1, Hq, L, 128, device=DEV, generator=g, dtype=torch.bfloat16)
    k = torch.randn(1, Hk, L, 128, device=DEV, generator=g, dtype=torch.bfloat16)
    v = torch.randn(1, Hk, L, 128, device=DEV, generator=g, dtype=torch.bfloat16)
    k[:, :, :4] *= 6
    sel = select_blocks(q, k, **PROD)
    sel2 = select_blocks(q, k, **PROD)
    torch.cuda.synchronize()
    assert sel.params.N == 8192
    assert torch.equal(sel.blk_cnt, sel2.blk_cnt)
    cnt = sel.blk_cnt.cpu()
    assert bool((cnt >= 1).all()) and bool((cnt <= torch.arange(1, 8193)[None, :]).all())
    assert sel.blk_bits.numel() * 8 == Hq * 8192 * 8192 // 8
    assert torch.equal(sel.blk_bits, sel2.blk_bits)
    m = sel.dense_mask().cpu()
    assert torch.equal(m.sum(-1, dtype=torch.int32), cnt)
    rows = (0, 1, 4095, 4096, 8190, 8191)
    check_mask_rows(m, rows)
    out = block_sparse_attention(q, k, v, sel.blk_cnt, sel.blk_bits)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all())
    # sampled query blocks against fp32 attention under the same lists
    want = v7.block_sparse_attention(q.cpu(), k.cpu(), v.cpu(), m, 128, qblocks=rows)
    t = torch.cat([torch.arange(i * 128, (i + 1) * 128) for i in rows])
    err = (out[0].float().cpu()[t] - want[t]).abs()                  # [L, Hq, D] rows
    print(f"  attention max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}", flush=True)
    assert err.max().item() <= 2e-2 and err.mean().item() <= 1e-3


def test_block_count_above_the_limit_is_rejected():
    """N = 8193 blocks is past the selection kernels' limit, and N = 4097 past
    the fp32 path's (one LDS FFT of length 2N): clear errors, no launch."""
    _print_case("over-limit", L=8193 * 128)
    L = 8193 * 128
    q = torch.zeros(1, 1, L, 128, device=DEV, dtype=torch.bfloat16)
    k = torch.zeros(1, 1, L, 128, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="exceed the selection kernels' maximum of 8192"):
        select_blocks(q, k, **PROD)
        torch.cuda.synchronize()
    del q, k
    L = 4097 * 128
    q = torch.zeros(1, 1, L, 128, device=DEV, dtype=torch.float32)
    k = torch.zeros(1, 1, L, 128, device=DEV, dtype=torch.float32)
    with pytest.raises(RuntimeError, match="maximum of 4096"):
        select_blocks(q, k, **PROD)
        torch.cuda.synchronize()


@pytest.mark.parametrize("bs", [16, 32, 64, 128])
def test_dense_causal_fewer_queries_than_keys(bs):
    """Dense causal attention with L_q < L_k (bottom-right aligned, as
    flash_attn_func(causal=True) with a key prefix), every block size."""
    _print_case("attention-offset", bs=bs)
    q, _, _ = make_qkv(1000, 4, 2, seed=14)
    _, k, v = make_qkv(1500, 4, 2, seed=15)
    out = block_sparse_attention(*_gpu(q, k, v), block_size=bs, is_causal=True)
    torch.cuda.synchronize()
    ref = v7.dense_causal_attention(q, k, v)[0]
    _attn_check(out[0], ref)
