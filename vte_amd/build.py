"""Build the gfx950 artefacts of vte_amd in-tree with hipcc.

Produces, next to this file:
  * libvte_amd.so         - kernels + the C ABI declared in include/vte_amd.h
  * vte_kernels_gfx950.hsaco - the reference-named extern "C" kernels as a
    plain code object for hipModuleLoad / hipModuleGetFunction callers
    (the reference's loading path, vte/bridge/hip_runtime.py:793-803).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
ARCH = "gfx950"
LIB = HERE / "libvte_amd.so"
HSACO = HERE / f"vte_kernels_{ARCH}.hsaco"
SOURCES = ["gemv.hip", "fused.hip", "fused_f32.hip", "gemm_mfma.hip", "fused_mm.hip", "attention.hip", "glue.hip", "decode_persistent.hip", "decode_persistent_mm.hip", "capi.hip"]
MODULE_SOURCE = "module.hip"
# Packed FP32 instructions are disabled for every HIP compile: some of their
# forms have given silently wrong results on the target machines.
COMMON = ["-O3", "-std=c++17", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
          "-packed-fp32-ops", "-Wno-unused-result"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def build(verbose: bool = False) -> None:
    cc = hipcc()
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)

    def compile_one(src):
        obj = objdir / (Path(src).stem + ".o")
        _run([cc, *COMMON, "-fPIC", "-c", str(CSRC / src), "-o", str(obj)])
        return obj

    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES) + 1)) as ex:
        futs = [ex.submit(compile_one, s) for s in SOURCES]
        hs = ex.submit(_run, [cc, *COMMON, "--genco", "-o", str(HSACO) + ".tmp",
                              str(CSRC / MODULE_SOURCE)])
        objs = [f.result() for f in futs]
        hs.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, *COMMON, "-shared", "-fPIC", "-Wl,--no-undefined", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    os.replace(str(HSACO) + ".tmp", HSACO)
    if verbose:
        print(f"built {LIB} and {HSACO}")


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
