"""Build libkda_bt16_hip.so in-tree with hipcc for gfx950.

Usage: ``python -m kda_bt16._build`` (with ``kda-ascendc_amd`` on sys.path),
or ``build()`` from Python.  The library lands next to this file, where
:mod:`kda_bt16._hip` loads it from.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR.parent / "csrc"
INCLUDE = PKG_DIR.parents[1] / "include"
LIB_NAME = "libkda_bt16_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
SOURCES = ["kda_capi.hip", "kda_k1.hip", "kda_k2.hip", "kda_k2w.hip", "kda_fused.hip",
           "kda_recurrent.hip", "kda_bwd.hip"]
HEADERS = ["kda_common.h", "kda_k2_shared.h", "kda_k1_chunk.h", "kda_k2w_step.h"]

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    # Keep the compiler from forming packed fp32 VALU ops.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Matrix-op accumulators in ordinary VGPRs: stage 2 scales its state
    # with VALU ops every chunk, and AGPR-resident accumulators would need a
    # copy out and back each time.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # No implicit multiply-add fusion: each product and sum rounds where the
    # source writes it (explicit fmaf() stays fused), so that variants of a
    # kernel (full-chunk or not, one sequence per work-group or several)
    # give identical bits, and the rounding follows the oracle's order.
    "-ffp-contract=off",
    # Loop heads on 64-byte boundaries: the fused kernel's timing followed
    # where its loops happened to land (B=16 T=2048 H=32: 504 against 524 us
    # for the same instructions shifted by 148 bytes, with instruction-cache
    # misses negligible either way); aligned, both layouts ran 510 us, and
    # every other kernel's time is unchanged.
    "-falign-loops=64",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (looked in $HIPCC, /opt/rocm/bin, PATH)")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    # hipcc's host pass does not know the packed-fp32 feature flag: harmless
    out = "\n".join(ln for ln in (res.stdout + res.stderr).splitlines()
                    if ln.strip() and "packed-fp32-ops' is not a recognized feature" not in ln)
    if verbose and out:
        print(out, flush=True)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source (one hipcc process per source, in parallel)
    and link ``libkda_bt16_hip.so``; return its path.  Objects go to a
    scratch folder beside the sources (``_build/``)."""
    cc = hipcc()
    objdir = PKG_DIR.parent / "_build"
    objdir.mkdir(exist_ok=True)
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    jobs = []
    for s in SOURCES:
        obj = objdir / (Path(s).stem + ".o")
        jobs.append(([cc, *compile_flags, f"-I{INCLUDE}", "-c", str(CSRC / s), "-o", str(obj)], obj))
    workers = max(1, min(len(jobs), os.cpu_count() or 1, 16))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        for f in [ex.submit(_run, cmd, verbose) for cmd, _ in jobs]:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *(str(o) for _, o in jobs), "-o", str(tmp)],
         verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
