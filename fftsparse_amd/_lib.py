"""ctypes binding of the C ABI in ``include/fftsparse_amd.h``.

The shared library is built in-tree (``python -m fftsparse_amd.build``).  torch
is imported first so that the library's HIP runtime dependency resolves to the
runtime torch already loaded: device pointers and streams are shared.
Loading fails loudly when the library is missing -- there is no fallback.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_int32, c_int64, c_size_t, c_uint8, c_uint16, c_void_p
from pathlib import Path

import torch  # noqa: F401  (must precede the library load, see module docstring)

# FFTSPARSE_AMD_LIB may name another build of the same library (e.g. one built
# with different compile-time options); by default the in-tree build is used.
LIB_PATH = Path(os.environ.get("FFTSPARSE_AMD_LIB") or Path(__file__).resolve().with_name("libfftsparse_amd.so"))

FS_DTYPE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
ABI_VERSION = 12


class PoolArgs(ctypes.Structure):
    _fields_ = [("q", c_void_p), ("q_sh", c_int64), ("q_sl", c_int64),
                ("k", c_void_p), ("k_sh", c_int64), ("k_sl", c_int64),
                ("dtype", c_int), ("Hq", c_int), ("Hk", c_int), ("L", c_int), ("D", c_int), ("bs", c_int),
                ("q_b", c_void_p), ("k_b", c_void_p)]


class RopePoolArgs(ctypes.Structure):
    _fields_ = [("q", c_void_p), ("q_sh", c_int64), ("q_sl", c_int64),
                ("k", c_void_p), ("k_sh", c_int64), ("k_sl", c_int64),
                ("cos", c_void_p), ("sin", c_void_p), ("cs_sl", c_int64),
                ("q_out", c_void_p), ("qo_sh", c_int64), ("qo_sl", c_int64),
                ("k_out", c_void_p), ("ko_sh", c_int64), ("ko_sl", c_int64),
                ("dtype", c_int), ("Hq", c_int), ("Hk", c_int), ("L", c_int), ("D", c_int), ("bs", c_int),
                ("q_b", c_void_p), ("k_b", c_void_p)]


class XattnArgs(ctypes.Structure):
    _fields_ = [("q", c_void_p), ("q_sh", c_int64), ("q_sl", c_int64),
                ("k", c_void_p), ("k_sh", c_int64), ("k_sl", c_int64),
                ("dtype", c_int), ("Hq", c_int), ("Hk", c_int), ("L", c_int), ("D", c_int), ("stride", c_int),
                ("bs", c_int), ("norm", c_float), ("threshold", c_void_p), ("keep_sink", c_int),
                ("sums", c_void_p), ("blk_cnt", c_void_p), ("blk_bits", c_void_p), ("work", c_void_p),
                ("non_causal", c_int), ("torch_path", c_int), ("select_mode", c_int), ("perm", c_int * 16),
                ("kdb", c_int), ("no_softmax", c_int), ("chunk", c_int), ("keep_recent", c_int),
                ("head_group", c_int)]


class FlexArgs(ctypes.Structure):
    _fields_ = [("q", c_void_p), ("q_sh", c_int64), ("q_sl", c_int64),
                ("k", c_void_p), ("k_sh", c_int64), ("k_sl", c_int64),
                ("dtype", c_int), ("Hq", c_int), ("Hk", c_int), ("L", c_int), ("D", c_int), ("bs", c_int),
                ("gamma", c_float), ("tau", c_float), ("min_blocks", c_int), ("max_blocks", c_int),
                ("gqa_interleave", c_int), ("blk_cnt", c_void_p), ("blk_bits", c_void_p),
                ("head_info", c_void_p), ("head_js", c_void_p), ("vertical", c_void_p), ("slash", c_void_p),
                ("work", c_void_p)]


class CorrArgs(ctypes.Structure):
    _fields_ = [("q_b", c_void_p), ("k_b", c_void_p),
                ("dtype", c_int), ("Hq", c_int), ("Hk", c_int), ("N", c_int), ("D", c_int),
                ("local_window", c_int), ("keep_sink", c_int), ("remote_start", c_int),
                ("corr_threshold", c_float), ("corr_mode", c_int), ("corr_quantile", c_float),
                ("work", c_void_p), ("corr", c_void_p), ("corr_sum", c_void_p), ("keep_tau", c_void_p)]


class StatsArgs(ctypes.Structure):
    _fields_ = [("q_b", c_void_p), ("k_b", c_void_p),
                ("dtype", c_int), ("Hq", c_int), ("Hk", c_int), ("N", c_int), ("D", c_int),
                ("sample_taus", c_void_p), ("n_samples", c_int),
                ("col_start", c_int), ("col_end", c_int), ("n_cols", c_int),
                ("last_k", c_int),
                ("diag_var", c_void_p), ("col_mean", c_void_p), ("col_sel", c_void_p),
                ("last_scores", c_void_p), ("last_sel", c_void_p)]


class ScoresArgs(ctypes.Structure):
    _fields_ = [("q_b", c_void_p), ("k_b", c_void_p),
                ("dtype", c_int), ("Hq", c_int), ("Hk", c_int), ("N", c_int), ("D", c_int),
                ("local_window", c_int), ("keep_sink", c_int), ("remote_start", c_int),
                ("corr_threshold", c_float), ("corr_mode", c_int), ("corr_quantile", c_float),
                ("corr", c_void_p), ("corr_sum", c_void_p), ("keep_tau", c_void_p),
                ("sample_taus", c_void_p), ("n_samples", c_int),
                ("col_start", c_int), ("col_end", c_int), ("n_cols", c_int),
                ("last_k", c_int),
                ("diag_var", c_void_p), ("col_mean", c_void_p), ("col_sel", c_void_p),
                ("last_scores", c_void_p), ("last_sel", c_void_p),
                ("work", c_void_p)]


class SelectArgs(ctypes.Structure):
    _fields_ = [("q_b", c_void_p), ("k_b", c_void_p),
                ("dtype", c_int), ("Hq", c_int), ("Hk", c_int), ("N", c_int), ("Nk", c_int), ("D", c_int),
                ("mask_causal", c_int),
                ("keep_sink", c_int), ("keep_recent", c_int), ("local_window", c_int), ("remote_start", c_int),
                ("dyn_mode", c_int), ("stripe_all_diffuse", c_int),
                ("diag_var", c_void_p), ("n_samples", c_int), ("stripe_threshold", c_float),
                ("keep_tau", c_void_p),
                ("qk_topk_ratio", c_float),
                ("col_mode", c_int), ("col_sel", c_void_p), ("last_sel", c_void_p),
                ("mean_var", c_void_p), ("is_stripe", c_void_p),
                ("blk_cnt", c_void_p), ("blk_bits", c_void_p)]


class AttnArgs(ctypes.Structure):
    _fields_ = [("q", c_void_p), ("q_sb", c_int64), ("q_sh", c_int64), ("q_sl", c_int64),
                ("k", c_void_p), ("k_sb", c_int64), ("k_sh", c_int64), ("k_sl", c_int64),
                ("v", c_void_p), ("v_sb", c_int64), ("v_sh", c_int64), ("v_sl", c_int64),
                ("out", c_void_p), ("o_sb", c_int64), ("o_sh", c_int64), ("o_sl", c_int64),
                ("dtype", c_int), ("B", c_int), ("Hq", c_int), ("Hk", c_int), ("Lq", c_int), ("Lk", c_int),
                ("D", c_int), ("bs", c_int),
                ("is_causal", c_int), ("softmax_scale", c_float), ("gqa_interleave", c_int),
                ("blk_cnt", c_void_p), ("blk_bits", c_void_p), ("work", c_void_p)]


STRUCTS = [PoolArgs, CorrArgs, StatsArgs, SelectArgs, AttnArgs, ScoresArgs, RopePoolArgs, XattnArgs, FlexArgs]

ENTRY_POINTS = ["fs_pool", "fs_rope_pool", "fs_corr_work_bytes", "fs_corr", "fs_stats", "fs_scores_work_bytes",
                "fs_scores", "fs_scores_noalloc", "fs_select", "fs_bsattn_work_bytes",
                "fs_bsattn", "fs_bsattn_prepare", "fs_bsattn_run", "fs_xattn_work_bytes", "fs_xattn",
                "fs_flex_work_bytes", "fs_flex",
                "fs_last_error", "fs_abi_version", "fs_sizeof_args"]

_lib = None


def load() -> ctypes.CDLL:
    """Load the in-tree library once; raise if it is missing or stale."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"fftsparse_amd native library not found at {LIB_PATH}; build it with "
            "`python -m fftsparse_amd.build` (no CPU fallback exists)")
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.fs_last_error.restype = ctypes.c_char_p
    lib.fs_abi_version.restype = c_int
    lib.fs_sizeof_args.restype = c_size_t
    lib.fs_sizeof_args.argtypes = [c_int]
    lib.fs_corr_work_bytes.restype = c_size_t
    lib.fs_corr_work_bytes.argtypes = [c_int, c_int, c_int]
    lib.fs_scores_work_bytes.restype = c_size_t
    lib.fs_scores_work_bytes.argtypes = [c_int, c_int, c_int]
    lib.fs_flex_work_bytes.restype = c_size_t
    lib.fs_flex_work_bytes.argtypes = [c_int, c_int, c_int, c_int, c_float]
    lib.fs_xattn_work_bytes.restype = c_size_t
    lib.fs_xattn_work_bytes.argtypes = [ctypes.POINTER(XattnArgs)]
    lib.fs_bsattn_work_bytes.restype = c_size_t
    lib.fs_bsattn_work_bytes.argtypes = [POINTER(AttnArgs)]
    for name, st in [("fs_pool", PoolArgs), ("fs_rope_pool", RopePoolArgs), ("fs_corr", CorrArgs),
                     ("fs_stats", StatsArgs), ("fs_scores", ScoresArgs), ("fs_scores_noalloc", ScoresArgs),
                     ("fs_select", SelectArgs), ("fs_bsattn", AttnArgs), ("fs_bsattn_prepare", AttnArgs),
                     ("fs_bsattn_run", AttnArgs), ("fs_xattn", XattnArgs),
                     ("fs_flex", FlexArgs)]:
        fn = getattr(lib, name)
        fn.restype = c_int
        fn.argtypes = [POINTER(st), c_void_p]
    if lib.fs_abi_version() != ABI_VERSION:
        raise RuntimeError("fftsparse_amd: library ABI version mismatch; rebuild it")
    for i, st in enumerate(STRUCTS):
        if lib.fs_sizeof_args(i) != ctypes.sizeof(st):
            raise RuntimeError(f"fftsparse_amd: {st.__name__} layout differs from the library; rebuild it")
    _lib = lib
    return lib


def same_device(*tensors) -> torch.device:
    """The one GPU that every given tensor (None entries skipped) lives on.
    The kernels dereference the tensors' pointers on that GPU, so a host
    tensor, or tensors on two GPUs, raise ValueError before any launch."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"tensors must be on the GPU, got one on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no tensor given")
    return dev


def call(name: str, args, device: torch.device | None = None) -> None:
    """Invoke an entry point on torch's current stream of ``device`` (default:
    the current device), with that device current; raise on a non-zero status."""
    lib = load()
    with torch.cuda.device(device if device is not None else torch.cuda.current_device()):
        stream = torch.cuda.current_stream().cuda_stream
        rc = getattr(lib, name)(ctypes.byref(args), c_void_p(stream))
    if rc != 0:
        msg = lib.fs_last_error().decode(errors="replace")
        if rc == -1:
            raise ValueError(msg)
        raise RuntimeError(msg)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
