"""Build recipe for ``libwisp_hip.so`` (gfx950 only).

``python -m wisp_amd.build`` compiles every HIP source under ``wisp_amd/csrc``
with hipcc for ``--offload-arch=gfx950`` and links the in-tree shared library
``wisp_amd/libwisp_hip.so`` that ``wisp_amd._lib`` loads.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libwisp_hip.so"
ROOT = PKG.parent

SOURCES = [
    "pager.hip",
    "route.hip",
    "experts_gemv.hip",
    "experts_mfma.hip",
    "experts_fp8.hip",
    "pagein.hip",
    "packed.hip",
    "prefetch.hip",
    "layer.hip",
    "probes.hip",
    "noalloc.hip",
]

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # keep the compiler away from packed fp32 ALU forms
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the HIP toolchain is required to build wisp_hip")
    return exe


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *_size_flags(), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")
    # surface real warnings, drop the host pass's note about the ALU feature
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l
                    and "target-feature" not in l and l.strip())
    if err:
        print(f"[wisp build] {src.name}:\n{err}", file=sys.stderr)


def _size_flags() -> list[str]:
    """``WISP_NOALLOC_SCRATCH_MIB`` (default 64): MiB of the static device
    array of wisp_moe_experts_noalloc, which every process that loads the
    library holds on each GPU it runs on."""
    mib = os.environ.get("WISP_NOALLOC_SCRATCH_MIB")
    if mib is None:
        return []
    n = int(mib)
    if not 1 <= n <= 4096:
        raise ValueError(f"WISP_NOALLOC_SCRATCH_MIB={mib} outside 1..4096")
    return [f"-DWISP_NOALLOC_SCRATCH_BYTES=({n}ull<<20)"]


def build(verbose: bool = True) -> Path:
    OBJ.mkdir(exist_ok=True)
    objs = [OBJ / (Path(s).stem + ".o") for s in SOURCES]
    jobs = max(1, min(len(SOURCES), os.cpu_count() or 1, 8))
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_compile, CSRC / s, o) for s, o in zip(SOURCES, objs)]
        for f in futs:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[wisp build] {LIB} ({LIB.stat().st_size // 1024} KiB)")
    return LIB


if __name__ == "__main__":
    build()
