"""Build the gfx950 shared library ``fftsparse_amd/libfftsparse_amd.so`` in-tree.

    python -m fftsparse_amd.build            # compile (always recompiles)

Each ``csrc/*.hip`` file is compiled to an object by ``hipcc`` in parallel,
then linked into one shared library that exports only the C ABI declared in
``include/fftsparse_amd.h``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libfftsparse_amd.so"
ARCH = "gfx950"

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

# -packed-fp32-ops: keep hipcc from emitting packed fp32 VALU ops.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden", "-Wno-unused-result",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]


def _compile(src: Path, obj: Path) -> None:
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    noise = "is not a recognized feature for this target"
    msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if msg.strip():
        print(msg, file=sys.stderr)


def build(verbose: bool = True) -> Path:
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    objs = [objdir / (s.stem + ".o") for s in srcs]
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(lambda so: _compile(*so), zip(srcs, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} ({LIB.stat().st_size // 1024} KiB)")
    return LIB


if __name__ == "__main__":
    build()
