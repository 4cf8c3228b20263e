"""Builds the engine's shared libraries in-tree with hipcc (gfx950 only).

Outputs (git-ignored, shipped to the GPU box with the tree):
  cellerator_amd/libcellerator_amd.so   -- HIP kernels + C-ABI (include/cellerator_amd.h)
  cellerator_amd/libcx_synth.so         -- seeded synthetic single-cell inputs on the GPU
                                           (bench/test support, include/cellerator_amd_synth.h)
  cellerator_amd/libcellerator_amd_cpmath.so
                                        -- CP-Math operation-core candidates (cpmath/), built
                                           with g++ against the Cellerator headers when they
                                           are present (CELLERATOR_INCLUDE, default
                                           /root/reference/include); links the engine library

Every HIP translation unit is compiled with packed-FP32 instruction selection disabled
(`-Xclang -target-feature -Xclang -packed-fp32-ops`); the host pass warns that it does
not know the feature, which is expected.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
ARCH = "gfx950"

ENGINE_SOURCES = [
    "cx_runtime.hip",
    "qcsr_spmm.hip",
    "qcsr_backward.hip",
    "qcsr_parts.hip",
    "sort.hip",
    "bell_spmm.hip",
    "cpbp_reduce.hip",
    "csr_spmv.hip",
    "abi.cpp",
    "cpbp_build.cpp",
    "cpbp_build_device.hip",
    "cpk1.cpp",
    "bell_plan.cpp",
    "exec_order.hip",
    "native_tile.cpp",
    "exec_csr.cpp",
    "bell_lowering.cpp",
    "spmm_request.cpp",
    "qcsr_codec.hip",
    "cpe2.cpp",
    "qcsr_hybrid.hip",
    "qcsr_stream.hip",
    "qcsr_exec.hip",
]
SYNTH_SOURCES = ["synth.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
CELLERATOR_INCLUDE = Path(os.environ.get("CELLERATOR_INCLUDE", "/root/reference/include"))
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _compile(src: Path, obj: Path) -> None:
    cmd = [HIPCC, *COMMON, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd = [HIPCC, *COMMON, "-x", "hip", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def _link(objs: list[Path], out: Path) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed for {out.name}:\n{res.stderr}")
    os.replace(tmp, out)


def build_cpmath(verbose: bool = True) -> Path | None:
    """Builds the CP-Math candidate library where the Cellerator headers are available;
    elsewhere a previously built library is left in place."""
    out = PKG / "libcellerator_amd_cpmath.so"
    header = CELLERATOR_INCLUDE / "Cellerator/compute/math/operation_core/operation_core.hh"
    if not header.exists():
        if verbose:
            print(f"Cellerator headers not found under {CELLERATOR_INCLUDE}: "
                  f"{out.name} not rebuilt", file=sys.stderr)
        return out if out.exists() else None
    tmp = out.with_suffix(".so.tmp")
    cmd = [CXX, "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra",
           f"-I{CELLERATOR_INCLUDE}", f"-I{ROOT / 'include'}",
           str(PKG / "cpmath" / "cpmath_backend.cc"), "-o", str(tmp),
           f"-L{PKG}", "-lcellerator_amd", "-Wl,-rpath,$ORIGIN"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"CP-Math backend build failed:\n{res.stderr}")
    os.replace(tmp, out)
    return out


def build(verbose: bool = True) -> dict[str, Path]:
    """Compiles every HIP/C++ source (always, also when a library exists) and links."""
    BUILD.mkdir(exist_ok=True)
    jobs = []
    for name in ENGINE_SOURCES + SYNTH_SOURCES:
        src = CSRC / name
        jobs.append((src, BUILD / (src.stem + ".o")))
    workers = min(len(jobs), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        list(ex.map(lambda j: _compile(*j), jobs))
    engine = PKG / "libcellerator_amd.so"
    synth = PKG / "libcx_synth.so"
    _link([BUILD / (Path(n).stem + ".o") for n in ENGINE_SOURCES], engine)
    _link([BUILD / (Path(n).stem + ".o") for n in SYNTH_SOURCES], synth)
    shutil.rmtree(BUILD, ignore_errors=True)
    cpmath = build_cpmath(verbose)
    if verbose:
        extra = f" and {cpmath.name}" if cpmath is not None else ""
        print(f"built {engine.name}, {synth.name} for {ARCH}{extra}")
    return {"engine": engine, "synth": synth, "cpmath": cpmath}


if __name__ == "__main__":
    build()
