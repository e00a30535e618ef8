"""fs_scores_noalloc (the allocation-free variant of fs_scores, partials in a
static device array) against fs_scores with a caller workspace: every output
bit for bit, on two calls in a row, the second with a smaller input, so the
second call runs over what the first left in the static array."""
from __future__ import annotations

import pytest
import torch

from fftsparse_amd import _lib, select_blocks
from fftsparse_amd.synth import make_qkv
from tests.helpers import PROD

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

FIELDS = ("corr", "corr_sum", "keep_tau", "diag_var", "col_mean", "col_sel", "last_scores", "last_sel")


def _outputs(Hq, N, n_samples):
    f32, u8 = torch.float32, torch.uint8
    return dict(corr=torch.full((Hq, N), -7.0, dtype=f32, device=DEV),
                corr_sum=torch.full((Hq, N), -7.0, dtype=f32, device=DEV),
                keep_tau=torch.full((Hq, N), 9, dtype=u8, device=DEV),
                diag_var=torch.full((Hq, max(1, n_samples)), -7.0, dtype=f32, device=DEV),
                col_mean=torch.full((Hq, N), -7.0, dtype=f32, device=DEV),
                col_sel=torch.full((Hq, N), 9, dtype=u8, device=DEV),
                last_scores=torch.full((Hq, N), -7.0, dtype=f32, device=DEV),
                last_sel=torch.full((Hq, N), 9, dtype=u8, device=DEV))


def _args(sel, Hq, Hk, D, taus, out, work):
    p = sel.params
    return _lib.ScoresArgs(
        q_b=sel.q_b.data_ptr(), k_b=sel.k_b.data_ptr(), dtype=_lib.FS_DTYPE[sel.q_b.dtype], Hq=Hq, Hk=Hk, N=p.N, D=D,
        local_window=p.local_window, keep_sink=p.keep_sink, remote_start=p.remote_start,
        corr_threshold=PROD["corr_threshold"], corr_mode=0, corr_quantile=0.8,
        corr=out["corr"].data_ptr(), corr_sum=out["corr_sum"].data_ptr(), keep_tau=out["keep_tau"].data_ptr(),
        sample_taus=taus.data_ptr(), n_samples=len(p.sample_taus), col_start=p.col_start, col_end=p.col_end,
        n_cols=p.n_cols, last_k=p.last_k, diag_var=out["diag_var"].data_ptr(), col_mean=out["col_mean"].data_ptr(),
        col_sel=out["col_sel"].data_ptr(), last_scores=out["last_scores"].data_ptr(),
        last_sel=out["last_sel"].data_ptr(), work=work)


def test_noalloc_scores_equal_workspace_scores_twice():
    lib = _lib.load()
    for L, Hq, Hk, dtype in ((32768, 32, 8, torch.bfloat16), (16384, 4, 1, torch.float16)):
        print(f"[case] fs_scores_noalloc L={L} Hq={Hq} Hk={Hk} dtype={dtype}", flush=True)
        q, k, _ = make_qkv(L, Hq, Hk, dtype=dtype, seed=31)
        sel = select_blocks(q.to(DEV), k.to(DEV), **PROD, keep_intermediates=True)
        p = sel.params
        assert p.corr_enabled and p.n_cols > 0 and p.last_k > 0 and len(p.sample_taus) > 0
        taus = torch.tensor(p.sample_taus, dtype=torch.int32, device=DEV)
        ns = len(p.sample_taus)
        work = torch.empty(lib.fs_scores_work_bytes(Hq, p.N, ns), dtype=torch.uint8, device=DEV)
        ref, got = _outputs(Hq, p.N, ns), _outputs(Hq, p.N, ns)
        _lib.call("fs_scores", _args(sel, Hq, Hk, 128, taus, ref, work.data_ptr()))
        _lib.call("fs_scores_noalloc", _args(sel, Hq, Hk, 128, taus, got, None))
        torch.cuda.synchronize()
        for f in FIELDS:
            assert torch.equal(got[f], ref[f]), f
        # and the selection's own (workspace) statistics agree with both
        assert torch.equal(got["keep_tau"], sel.keep_tau) and torch.equal(got["col_sel"], sel.col_sel)
