"""bench.py's host-side helpers (no GPU): the traffic rows it reports next to
its roofline are used only when they were measured with the sources it runs."""
from __future__ import annotations

import csv
import os

import bench


def _tree(tmp_path, monkeypatch):
    root = tmp_path / "repo"
    (root / "fftsparse_amd").mkdir(parents=True)
    (root / "profiles").mkdir()
    os.symlink(os.path.join(bench.ROOT, "fftsparse_amd", "csrc"), root / "fftsparse_amd" / "csrc")
    os.symlink(os.path.join(bench.ROOT, "include"), root / "include")
    monkeypatch.setattr(bench, "ROOT", str(root))
    return root


def test_traffic_row_needs_the_current_source_hash(tmp_path, monkeypatch):
    root = _tree(tmp_path, monkeypatch)
    cur = bench.src_hash("bsattn")
    assert len(cur) == 16 and cur != bench.src_hash("select")
    (root / "profiles" / "traffic.txt").write_text(
        "# kernel config fetch_bytes write_bytes src_hash\n"
        f"bsattn c2 1000 24 {cur}\n"
        "bsattn c1 1000 24 0123456789abcdef\n"
        "select c2 1000 24\n")
    assert bench.pmc_traffic("bsattn", "c2") == 1024
    assert bench.pmc_traffic("bsattn", "c1") is None      # measured with other sources
    assert bench.pmc_traffic("select", "c2") is None      # no source hash recorded
    assert bench.pmc_traffic("bsattn", "c3a") is None     # not profiled


def test_traffic_rows_scale_by_the_copy_calibration(tmp_path, monkeypatch):
    _tree(tmp_path, monkeypatch)

    def coll(path, rows):
        with open(path, "w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Counter_Value"])
            w.writeheader()
            for name, v in rows:
                w.writerow({"Kernel_Name": name, "Counter_Value": v})
        return str(path)

    gib_kib = 1024 * 1024
    fetch = coll(tmp_path / "f.csv", [("void fs::bsattn_kernel<128>(x)", 100.0), ("void fs::bsattn_kernel<128>(x)", 300.0),
                                      ("void fs::pool_kernel<bf16>(x)", 10.0), ("fs::scores_final_kernel(x)", 2.0)])
    write = coll(tmp_path / "w.csv", [("void fs::bsattn_kernel<128>(x)", 8.0), ("void fs::select_kernel<bf16>(x)", 4.0)])
    cal_f = coll(tmp_path / "cf.csv", [("__amd_rocclr_copyBuffer", gib_kib / 2)])   # FETCH_SIZE reads half
    cal_w = coll(tmp_path / "cw.csv", [("__amd_rocclr_copyBuffer", gib_kib)])
    rows = [r.split() for r in bench.traffic_rows("c2", fetch, write, cal_f, cal_w)]
    got = {r[0]: (int(r[2]), int(r[3]), r[4]) for r in rows}
    assert got["bsattn"] == (200 * 2 * 1024, 8 * 1024, bench.src_hash("bsattn"))
    assert got["select"] == (12 * 2 * 1024, 4 * 1024, bench.src_hash("select"))
