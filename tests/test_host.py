"""CPU tests of the host side: the C ABI library loads and exports what the
header declares, struct layouts agree, parameter derivation agrees with the
oracle, and the Python API raises the reference's error types."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

import fftsparse_amd
from fftsparse_amd import _lib, params
from fftsparse_amd.synth import CONFIGS, make_qkv, sha256_of
from oracle import v7

HEADER = Path(__file__).resolve().parents[1] / "include" / "fftsparse_amd.h"


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = re.findall(r"FS_API\s+[\w\s\*]+?\b(fs_\w+)\s*\(", HEADER.read_text())
    assert set(declared) == set(_lib.ENTRY_POINTS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.fs_abi_version() == _lib.ABI_VERSION


def test_struct_layouts_match_library():
    lib = _lib.load()
    for i, st in enumerate(_lib.STRUCTS):
        assert lib.fs_sizeof_args(i) == ctypes.sizeof(st), st.__name__


def test_null_args_rejected_without_gpu():
    lib = _lib.load()
    for name in ("fs_pool", "fs_rope_pool", "fs_xattn", "fs_flex", "fs_corr", "fs_stats", "fs_scores", "fs_select", "fs_bsattn", "fs_bsattn_prepare",
                 "fs_bsattn_run"):
        rc = getattr(lib, name)(None, None)
        assert rc == -1
        assert b"null args" in lib.fs_last_error()


def test_bad_shapes_rejected_without_gpu():
    lib = _lib.load()
    r = _lib.RopePoolArgs(q=16, k=16, cos=16, sin=16, q_out=16, k_out=16, q_b=16, k_b=16, dtype=1, Hq=4, Hk=1,
                          L=10, D=96, bs=128)
    assert lib.fs_rope_pool(ctypes.byref(r), None) == -2          # 12 chunks per row: not a power of two
    assert b"D=96" in lib.fs_last_error()
    r.D, r.q_sl = 128, 100                                       # 200-byte row stride
    assert lib.fs_rope_pool(ctypes.byref(r), None) == -1
    x = _lib.XattnArgs(q=16, k=16, threshold=16, sums=16, blk_cnt=16, blk_bits=16, work=16, dtype=1, Hq=4, Hk=1,
                       L=4096, D=128, stride=8, bs=64, norm=1.0)
    assert lib.fs_xattn(ctypes.byref(x), None) == -2              # the reference asserts block_size == 128
    assert b"block size" in lib.fs_last_error()
    x.bs, x.stride = 128, 32
    assert lib.fs_xattn(ctypes.byref(x), None) == -2
    x.stride, x.Hk = 8, 3
    assert lib.fs_xattn(ctypes.byref(x), None) == -1
    f = _lib.FlexArgs(q=16, k=16, blk_cnt=16, blk_bits=16, work=16, dtype=1, Hq=4, Hk=1, L=4096, D=128, bs=8,
                      gamma=0.9, tau=0.1, min_blocks=1, max_blocks=64, q_sl=128, k_sl=128, q_sh=128, k_sh=128)
    assert lib.fs_flex(ctypes.byref(f), None) == -2              # the reference asserts 16, 32, 64 or 128
    assert b"block size" in lib.fs_last_error()
    f.bs, f.L = 64, 64                                           # one block: the reference attends densely
    assert lib.fs_flex(ctypes.byref(f), None) == -1
    f.L, f.Hk = 4096, 3
    assert lib.fs_flex(ctypes.byref(f), None) == -1
    f.Hk, f.q_sl = 1, 100                                        # 200-byte row stride
    assert lib.fs_flex(ctypes.byref(f), None) == -1
    f.q_sl, f.L, f.bs = 128, 8192 * 16 + 1, 16                   # 8193 blocks
    assert lib.fs_flex(ctypes.byref(f), None) == -2
    assert lib.fs_flex_work_bytes(4, 1, 4096, 64, 0.1) > 4 * 4096 * 4 * 2
    # tau <= 0 (the reference's default) makes no head sparse: no room for the
    # block-level attention [Hq][nb][nb] fp32 and the covers
    nb = 4096 // 64
    assert lib.fs_flex_work_bytes(4, 1, 4096, 64, 0.1) - lib.fs_flex_work_bytes(4, 1, 4096, 64, 0.0) >= 4 * nb * nb * 4
    x = _lib.AttnArgs(q=16, k=16, v=16, out=16, work=16, dtype=1, B=1, Hq=4, Hk=2, Lq=1280, Lk=1280, D=128, bs=128,
                      q_sl=128, k_sl=128, v_sl=128, o_sl=512, blk_cnt=18, blk_bits=16)
    assert lib.fs_bsattn(ctypes.byref(x), None) == -1             # counts are read as 32-bit words
    assert b"4- / 8-byte aligned" in lib.fs_last_error()
    x.blk_cnt, x.blk_bits = 16, 20                                # mask words are 64-bit
    assert lib.fs_bsattn(ctypes.byref(x), None) == -1
    assert b"4- / 8-byte aligned" in lib.fs_last_error()
    x.blk_bits = 16
    x.blk_cnt, x.bs, x.Lq, x.Lk = 16, 16, 8193 * 16, 8193 * 16    # union lists of 8193 key blocks
    assert lib.fs_bsattn(ctypes.byref(x), None) == -2
    assert b"8192 key blocks" in lib.fs_last_error()
    a = _lib.AttnArgs(q=16, k=16, v=16, out=16, dtype=1, B=1, Hq=3, Hk=2, Lq=10, Lk=10, D=128, bs=128)
    assert lib.fs_bsattn(ctypes.byref(a), None) == -1
    a = _lib.AttnArgs(q=16, k=16, v=16, out=16, work=16, dtype=1, B=1, Hq=4, Hk=2, Lq=10, Lk=10, D=96, bs=128)
    assert lib.fs_bsattn(ctypes.byref(a), None) == -2
    assert b"head_dim" in lib.fs_last_error()


@pytest.mark.parametrize("L", [1280, 8192, 10000, 32768, 65536, 131072, 262144])
@pytest.mark.parametrize("bs", [64, 128])
@pytest.mark.parametrize("ratios", [(0.01, 0.0, 0.02, 0.2), (0.1, 0.1, 0.1, 0.1), (0.3, 0.05, 0.5, 0.05)])
def test_params_agree_with_oracle(L, bs, ratios):
    sink, recent, local, col = ratios
    kw = dict(sink_ratio=sink, recent_ratio=recent, local_span_ratio=local, column_topk_ratio=col)
    a = params.derive(L, L, bs, **kw)
    b = v7.derive_params(L, L, bs, **kw)
    for f in ("N", "Nk", "keep_sink", "keep_recent", "local_window", "corr_enabled", "remote_start",
              "sample_taus", "stripe_all_diffuse", "col_enabled", "col_start", "col_end", "n_cols", "last_k"):
        assert getattr(a, f) == getattr(b, f), f


def test_api_asserts_gpu_tensors_like_reference():
    q = torch.zeros(1, 4, 2048, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        fftsparse_amd.myattn_prefill(q, q, q, layer_idx=0)
    with pytest.raises(AssertionError):
        fftsparse_amd.fix_mask.myattn_prefill(q, q, q, layer_idx=0)


def test_signature_matches_reference_v7():
    import inspect
    sig = inspect.signature(fftsparse_amd.myattn_prefill)
    expected = ["query_states", "key_states", "value_states", "layer_idx", "block_size", "is_causal",
                "is_visual", "sink_ratio", "recent_ratio", "local_span_ratio", "enable_correlation_mask",
                "correlation_selection_mode", "correlation_topk_ratio", "corr_threshold",
                "collect_corr_stats", "enable_column_mask", "column_topk_ratio",
                "column_start_exclude_ratio", "column_end_exclude_ratio", "enable_last_block_mask",
                "last_block_threshold", "diag_sample_ratio", "min_diag_samples", "max_diag_samples",
                "stripe_threshold", "qk_topk_ratio", "attention_vis_heads", "attention_vis_dir"]
    assert list(sig.parameters) == expected
    d = {k: p.default for k, p in sig.parameters.items()}
    assert (d["block_size"], d["sink_ratio"], d["corr_threshold"], d["qk_topk_ratio"],
            d["stripe_threshold"], d["max_diag_samples"]) == (128, 0.1, 0.1, 0.2, 0.3, 64)


def test_synthetic_inputs_are_pinned():
    golden = Path(__file__).resolve().parent / "golden" / "synth_sha256.txt"
    want = dict(line.split() for line in golden.read_text().splitlines() if line.strip())
    q, k, v = make_qkv(2048, 4, 1, dtype=torch.float32, seed=0)
    assert sha256_of(q, k, v) == want["small_f32_seed0"]
    q, k, v = make_qkv(2048, 4, 2, dtype=torch.bfloat16, seed=0, stripe_density=0.005, period=512)
    assert sha256_of(q, k, v) == want["small_bf16_seed0"]
    assert CONFIGS["c2"].period == 512 and CONFIGS["c3a"].theta == 1000000.0


def test_block_masks_checked_before_any_launch():
    """Masks of the wrong dtype, shape or layout raise ValueError on the host."""
    q = torch.zeros(1, 4, 1280, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 1280, 128, dtype=torch.bfloat16)
    cnt = torch.ones(4, 10, dtype=torch.int32)
    bits = torch.zeros(4, 10, 1, dtype=torch.int64)
    wide = torch.zeros(4, 10, 2, dtype=torch.int64)
    bad = [(cnt.to(torch.int64), bits), (cnt[:, :9], bits), (cnt, bits[:3]), (cnt, bits.to(torch.int32)),
           (cnt, wide), (cnt, wide[:, :, ::2]), (cnt, None), (None, bits)]
    for c, b in bad:
        with pytest.raises(ValueError):
            fftsparse_amd.AttentionCall(q, k, k, c, b)
    with pytest.raises(ValueError):                               # a block mask of the wrong size
        fftsparse_amd.block_sparse_attention(q, k, k, block_mask=torch.ones(4, 10, 9, dtype=torch.bool))
    with pytest.raises(ValueError):                               # mask and words together
        fftsparse_amd.block_sparse_attention(q, k, k, cnt, bits, block_mask=torch.ones(4, 10, 10, dtype=torch.bool))


def test_mask_bits_round_trip():
    """bits_from_mask / mask_from_bits: bit b of word w is key block 64 w + b,
    counts are the rows' popcounts, for row lengths around word boundaries."""
    from fftsparse_amd.attn import bits_from_mask, mask_from_bits
    g = torch.Generator().manual_seed(3)
    for nk in (1, 63, 64, 65, 128, 130, 1000):
        m = torch.rand(3, 5, nk, generator=g) < 0.4
        m[0, 0] = True                                           # a full row: every word all ones
        cnt, bits = bits_from_mask(m)
        assert bits.shape == (3, 5, (nk + 63) // 64) and bits.dtype == torch.int64
        assert torch.equal(mask_from_bits(bits, nk), m) and torch.equal(cnt, m.sum(-1, dtype=torch.int32))
        w = int(bits[1, 2, 0]) & (2 ** 64 - 1)
        assert all(((w >> b) & 1) == int(m[1, 2, b]) for b in range(min(64, nk)))
    assert int(bits_from_mask(torch.ones(1, 1, 64, dtype=torch.bool))[1][0, 0, 0]) == -1   # all 64 bits set


def test_noalloc_scores_rejects_sizes_past_its_static_buffer_without_gpu():
    """fs_scores_noalloc checks its size against the static buffer before any
    HIP call: 32 heads at N = 4096 with 64 sampled diagonals need 56.75 MiB."""
    lib = _lib.load()
    a = _lib.ScoresArgs(q_b=16, k_b=16, dtype=1, Hq=32, Hk=8, N=4096, D=128, n_samples=64, sample_taus=16,
                        diag_var=16, n_cols=0, last_k=0)
    assert lib.fs_scores_work_bytes(32, 4096, 64) > 32 << 20
    assert lib.fs_scores_noalloc(ctypes.byref(a), None) == -2
    assert b"exceed the static buffer" in lib.fs_last_error()
    a.Hq, a.Hk = 3, 2
    assert lib.fs_scores_noalloc(ctypes.byref(a), None) == -1
    assert b"fs_scores_noalloc: Hq=3" in lib.fs_last_error()


def test_selection_block_limits_without_gpu():
    """The 16-bit selection kernels take up to 8192 blocks (a diffuse head's
    4-row score panel in LDS); the fp32 path's LDS FFT of length 2N up to 4096.
    Past those, unsupported (-2) before any HIP call."""
    lib = _lib.load()
    sc = _lib.ScoresArgs(q_b=16, k_b=16, work=16, dtype=1, Hq=1, Hk=1, N=8193, D=128, n_cols=0, last_k=0)
    assert lib.fs_scores(ctypes.byref(sc), None) == -2
    assert b"N=8193 > 8192" in lib.fs_last_error()
    se = _lib.SelectArgs(q_b=16, k_b=16, dtype=1, Hq=1, Hk=1, N=8193, Nk=8193, D=128, blk_cnt=16, blk_bits=16)
    assert lib.fs_select(ctypes.byref(se), None) == -2
    assert b"N=8193 > 8192" in lib.fs_last_error()
    co = _lib.CorrArgs(q_b=16, k_b=16, dtype=0, Hq=1, Hk=1, N=4097, D=128, work=16, corr=16, corr_sum=16,
                       keep_tau=16, corr_threshold=0.9)
    assert lib.fs_corr(ctypes.byref(co), None) == -2
    assert b"N=4097" in lib.fs_last_error()


def test_api_rejects_host_tensors_and_bad_shapes_before_any_launch():
    """Every public entry point checks devices and shapes on the host: a host
    tensor (its pointer would reach a kernel), a wrong-sized ``out`` (written
    through its strides) or a key head_dim unlike the query's raise ValueError."""
    from fftsparse_amd import AttentionCall, block_sparse_attention, select_blocks
    from fftsparse_amd.flex import flex_select
    from fftsparse_amd.xattn import xattn_select
    q = torch.zeros(1, 4, 1280, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 1280, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="on the GPU"):
        block_sparse_attention(q, k, k)
    with pytest.raises(ValueError, match="out must be"):
        AttentionCall(q, k, k, out=torch.zeros(1, 1280, 4, 64, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="head_dim"):
        AttentionCall(q, k[..., :64], k[..., :64])
    with pytest.raises(ValueError, match="on the GPU"):
        select_blocks(q, k)
    with pytest.raises(ValueError, match="head_dim"):
        select_blocks(q, k[..., :64])
    with pytest.raises(ValueError, match="do not match"):
        flex_select(q.transpose(1, 2), k[..., :64].transpose(1, 2))
    with pytest.raises(ValueError, match="on the GPU"):
        flex_select(q.transpose(1, 2), k.transpose(1, 2))
    with pytest.raises(ValueError, match="on the GPU"):
        xattn_select(q, k)
