"""Compile the gfx950 HIP sources into ``edgerag_amd/libedgerag_amd.so``, in-tree.

hipcc cross-compiles for gfx950 without a GPU, so this runs anywhere the ROCm toolchain is
installed. Every call recompiles. Objects go to ``edgerag_amd/_build/`` (ignored by git); the
shared library lands next to the package so it travels with the source tree.

Flags that matter:

* ``--offload-arch=gfx950`` only: this library targets MI355X and nothing else.
* ``-mcode-object-version=5``: loadable by the ROCm 7.0 runtime that torch bundles as well as by
  ROCm 7.2.
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: keep the compiler from emitting packed
  fp32 VALU instructions (v_pk_fma_f32 and friends), which are not used in this library.
* ``-mllvm -amdgpu-kernarg-preload-count=16``: the leading kernel arguments (13-14 dwords, as
  many as the free user SGPRs hold) arrive in SGPRs at wave launch instead of through a scalar
  load from the kernel-argument buffer, a memory round trip before a kernel's first load can be
  addressed. The kernels put the arguments of their first loads first. The few-microsecond
  launches gain most (INT8 GEMV at one token, 2048 x 2048: 3.19 -> 2.85 us).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC = PACKAGE_DIR / "csrc"
BUILD_DIR = PACKAGE_DIR / "_build"
LIB_NAME = "libedgerag_amd.so"
LIB_PATH = PACKAGE_DIR / LIB_NAME
# Bench-only measurement probes (access-pattern ceilings), kept out of the product library.
PROBE_SOURCES = [CSRC / "probe" / "probe.hip", CSRC / "capi.cpp"]
PROBE_LIB_PATH = PACKAGE_DIR / "libedgerag_probe.so"

ARCH = "gfx950"
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-mcode-object-version=5",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-mllvm",
    "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
    f"-I{PACKAGE_DIR.parent / 'include'}",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build edgerag_amd")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _compile(src: Path, verbose: bool, build_dir: Path, defines: list[str]) -> Path:
    obj = build_dir / (src.parent.name + "_" + src.stem + ".o" if src.parent != CSRC
                       else src.stem + ".o")
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    cmd = [hipcc(), *COMMON_FLAGS, *[f"-D{d}" for d in defines], *lang, "-c", str(src), "-o",
           str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stdout}\n{proc.stderr}")
    if verbose and proc.stderr.strip():
        print(proc.stderr, file=sys.stderr)
    return obj


def build(
    verbose: bool = False,
    jobs: int | None = None,
    defines: list[str] | None = None,
    out: Path | None = None,
    build_dir: Path | None = None,
) -> Path:
    """Compile every HIP source and link the shared library. Returns its path.

    ``defines`` (``NAME=VALUE`` strings) override the tuning macros of the sources; ``out`` and
    ``build_dir`` redirect the library and objects (the defaults are the in-tree locations).
    """
    out = Path(out) if out is not None else LIB_PATH
    build_dir = Path(build_dir) if build_dir is not None else BUILD_DIR
    build_dir.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    with_probe = out == LIB_PATH
    extra = [PROBE_SOURCES[0]] if with_probe else []
    jobs = jobs or min(len(srcs) + len(extra), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, verbose, build_dir, defines or []),
                             srcs + extra))
    _link(objs[: len(srcs)], out, verbose)
    if with_probe:  # probe kernels + the error/version entry points, in their own library
        capi = objs[srcs.index(CSRC / "capi.cpp")]
        _link([objs[-1], capi], PROBE_LIB_PATH, verbose)
    return out


def _link(objs: list[Path], out: Path, verbose: bool) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
