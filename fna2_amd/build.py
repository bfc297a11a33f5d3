"""Build recipe for the gfx950 HIP library ``fna2_amd/libfna2_hip.so``.

Every source in ``fna2_amd/csrc`` is compiled by ``hipcc`` for gfx950 only and
linked into one shared library that exports the C ABI of ``include/fna2.h``.
Objects go to ``fna2_amd/_build`` (git-ignored); the library is written in-tree
so that it travels with the source tree.

Run as ``python -m fna2_amd.build``.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libfna2_hip.so"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# Packed FP32 (v_pk_*_f32) is switched off for all device code.
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]

SOURCES = ["fna2_capi.cpp", "fna2_sched.hip", "fna2_fwd.hip", "fna2_bwd.hip", "fna2_bwd_dkdv.hip",
           "fna2_bwd_dq.hip", "fna2_rope.hip", "fna2_decode.hip"]


def _compile(src: Path, obj: Path, verbose: bool) -> None:
    cmd = [HIPCC, *COMMON, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd[1:1] = ["-x", "hip"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature: drop that note.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False, jobs: int = 4) -> Path:
    """Compile all HIP sources for gfx950 and link ``libfna2_hip.so``."""
    BUILD.mkdir(exist_ok=True)
    srcs = [CSRC / s for s in SOURCES]
    objs = [BUILD / (s.stem + ".o") for s in srcs]
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, s, o, verbose) for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    # The library must load (an unresolved host symbol would only show at dlopen).
    chk = subprocess.run([sys.executable, "-c", f"import ctypes; ctypes.CDLL({str(tmp)!r})"],
                         capture_output=True, text=True)
    if chk.returncode != 0:
        raise RuntimeError(f"built library does not load:\n{chk.stderr.strip()}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
