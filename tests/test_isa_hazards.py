"""Guard against reading an MFMA result too early on some path through the code.

Every HIP source of the library is compiled to gfx950 assembly (hipcc
--cuda-device-only -S, on the CPU).  For each MFMA the walk follows every path
up to two branches deep and counts wait states (one per instruction,
`s_nop N` as N + 1) until the first instruction that reads one of the MFMA's
destination registers.  The compiler's own wait in straight-line code before
the first read of a 32x32x16 result is 12 (`s_nop 11`).  A path that reaches
the read in fewer was found once, across a branch leaving an MFMA chain early
(the read saw the accumulator without the last MFMA's contribution), so any
such path fails here.
"""
from __future__ import annotations

import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "fftsparse_amd" / "csrc"
HIPCC = shutil.which("hipcc") or ("/opt/rocm/bin/hipcc" if Path("/opt/rocm/bin/hipcc").exists() else None)
MIN_WAIT = 12
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         f"-I{ROOT / 'include'}", f"-I{CSRC}", "--cuda-device-only", "-S"]


def _regs(spec: str) -> set:
    m = re.match(r"([va])\[(\d+):(\d+)\]", spec)
    if m:
        return {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([va])(\d+)$", spec)
    return {f"{m.group(1)}{m.group(2)}"} if m else set()


def _operands(ins: str) -> list:
    parts = ins.split(None, 1)
    return [p.strip() for p in parts[1].split(",")] if len(parts) == 2 else []


def _reads(ins: str) -> set:
    ops = _operands(ins)
    if not ops:
        return set()
    src = ops if ins.startswith(("s_", "ds_write", "global_store", "buffer_store")) else ops[1:]
    out = set()
    for o in src:
        out |= _regs(o.split()[0])
    return out


def short_paths(asm: str, limit: int = MIN_WAIT, depth: int = 2):
    """[(function, line of the MFMA, wait states)] for reads of an MFMA's
    destination closer than `limit` along some path."""
    code = []
    for line in asm.splitlines():
        t = line.split(";")[0].strip()
        if t and (not t.startswith(".") or re.match(r"^\.LBB\w+:$", t)):
            code.append(t)
    labels = {t[:-1]: i for i, t in enumerate(code) if re.match(r"^\.LBB\w+:$", t)}
    found, func = [], None
    for k, ins in enumerate(code):
        m = re.match(r"^(_Z\w+):$", ins)
        if m:
            func = m.group(1)
        if not ins.startswith("v_mfma"):
            continue
        dst = _regs(_operands(ins)[0])
        stack = [(k + 1, 0, 0)]
        while stack:
            j, ws, d = stack.pop()
            while j < len(code) and ws < limit:
                t = code[j]
                if t.endswith(":"):
                    j += 1
                    continue
                if t.startswith("v_mfma") and _regs(_operands(t)[0]) == dst:
                    break                                  # chained into the same accumulator
                if _reads(t) & dst:
                    found.append((func, k, ws))
                    break
                ws += int(t.split()[1]) + 1 if t.startswith("s_nop") else 1
                if t.startswith("s_cbranch") and d < depth and t.split()[-1] in labels:
                    stack.append((labels[t.split()[-1]] + 1, ws, d + 1))
                if t.startswith("s_branch"):
                    if t.split()[-1] in labels and d < depth:
                        j, d = labels[t.split()[-1]] + 1, d + 1
                        continue
                    break
                if t.startswith("s_endpgm"):
                    break
                j += 1
    return found


def _compile(src: Path, out: Path) -> str:
    r = subprocess.run([HIPCC, *FLAGS, str(src), "-o", str(out)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text()


@pytest.mark.skipif(HIPCC is None, reason="hipcc is not installed")
def test_no_mfma_result_read_early_on_any_path(tmp_path):
    srcs = sorted(CSRC.glob("*.hip"))
    assert srcs
    with ThreadPoolExecutor(max_workers=8) as ex:
        asms = list(ex.map(lambda s: _compile(s, tmp_path / (s.stem + ".s")), srcs))
    bad = {s.name: short_paths(a) for s, a in zip(srcs, asms)}
    bad = {k: v for k, v in bad.items() if v}
    assert not bad, bad


def test_scanner_flags_a_short_path():
    """The walk itself: an MFMA whose result is read 7 wait states later on the
    branch-taken path is flagged; the fall-through path's 12 is not."""
    asm = "\n".join([
        "_Z4testv:",
        "\tv_mfma_f32_32x32x16_bf16 a[16:31], v[2:5], v[94:97], a[16:31]",
        "\ts_cbranch_vccnz .LBB0_2",
        "\ts_nop 11",
        "\tv_accvgpr_read_b32 v1, a20",
        ".LBB0_2:",
        "\ts_nop 5",
        "\tv_accvgpr_read_b32 v65, a31",
        "\ts_endpgm",
    ])
    found = short_paths(asm)
    assert found and all(ws < MIN_WAIT for _, _, ws in found)
    assert short_paths(asm.replace("s_nop 5", "s_nop 11")) == []
