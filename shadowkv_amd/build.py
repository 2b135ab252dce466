"""Build recipe for libshadowkv_amd.so: hand-written HIP kernels for gfx950 behind a C ABI.

Each csrc/*.hip is compiled by hipcc into an object under _build/, in parallel, and the
objects are linked into shadowkv_amd/libshadowkv_amd.so (in-tree, next to this file).
`python -m shadowkv_amd.build` runs it from the command line.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
BUILD_DIR = PKG_DIR.parent / "_build"
LIB_NAME = "libshadowkv_amd.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming packed fp32 math (v_pk_*_f32).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build shadowkv_amd")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def scratch_kernels(remarks: str) -> list[tuple[str, int]]:
    """(kernel, bytes per lane) for every kernel whose resource-usage remark reports scratch."""
    out, name = [], None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and int(m.group(1)) and name:
            out.append((name, int(m.group(1))))
    return out


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-Rpass-analysis=kernel-resource-usage", f"-I{INCLUDE}", f"-I{CSRC}", "-c",
           str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    # No kernel may touch scratch memory: a register spill or a stack object (a device function
    # left as a call, an array indexed at run time) in a hot loop costs more than any kernel here
    # saves, and nothing else reports it.
    bad = scratch_kernels(proc.stderr)
    if bad:
        raise RuntimeError(f"{src.name}: kernels using scratch memory (bytes per lane): {bad}")
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source for gfx950 and link the shared library. Always rebuilds."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
