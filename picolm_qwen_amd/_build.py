"""Builds libpqa.so (the HIP backend behind include/pqa.h) in-tree with hipcc
for gfx950."""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import tempfile

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libpqa.so")
# the same sources with -DPQA_PHASE_STAMPS: kernels also write s_memrealtime
# stamps at their phase boundaries (measurement only, bench.py --phase-stamps)
STAMPS_LIB = os.path.join(PKG, "libpqa_stamps.so")
# the stamped build with the prefill tile loop's per-step stamps as well
# (-DPQA_STEP_STAMPS; they cost time, so the per-phase stamps come from the
# build without them)
STEP_STAMPS_LIB = os.path.join(PKG, "libpqa_stepstamps.so")
SOURCES = ["pqa_api.hip", "pqa_decode.hip", "pqa_prefill.hip", "pqa_util.hip", "pqa_kvc.hip", "pqa_proj.hip", "pqa_batch.hip",
           "pqa_gemm.hip", "pqa_general.hip", "pqa_exact.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -ffp-contract=off: the K row written to the cache must round like the
# reference (no fused multiply-add in RMSNorm or RoPE); kernels that want an
# FMA call fmaf() explicitly. Packed fp32 instructions are disabled.
# -amdgpu-kernarg-preload-count: the leading scalar kernel arguments (up to
# 14 words) arrive in SGPRs at dispatch, not by a load from the argument
# segment; the code object keeps a fallback prologue that loads them.
CFLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-mllvm", "-amdgpu-kernarg-preload-count=16",
          "-I" + os.path.join(ROOT, "include"), "-I" + CSRC]


def _compile(src: str, obj: str, extra=()) -> None:
    cmd = [HIPCC, *CFLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")


def build(verbose: bool = False, stamps: bool = False, step_stamps: bool = False) -> str:
    """Compiles every csrc/*.hip source and links libpqa.so (with stamps:
    libpqa_stamps.so, the phase-stamped variant; with step_stamps as well:
    libpqa_stepstamps.so); returns its path."""
    out = (STEP_STAMPS_LIB if step_stamps else STAMPS_LIB) if stamps else LIB
    extra = (["-DPQA_PHASE_STAMPS"] + (["-DPQA_STEP_STAMPS"] if step_stamps else [])) if stamps else []
    with tempfile.TemporaryDirectory(prefix="pqa_build_") as tmp:
        objs = [os.path.join(tmp, s.replace(".hip", ".o")) for s in SOURCES]
        with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
            list(ex.map(lambda s_o: _compile(*s_o, extra), zip(SOURCES, objs)))
        tmp_lib = out + ".tmp"
        cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp_lib, *objs]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
        os.replace(tmp_lib, out)
    if verbose:
        print(f"built {out}")
    return out


ADAPTER = os.path.join(PKG, "adapter")
DEMO_LIB = os.path.join(ADAPTER, "libpqa_forward_demo.so")


def build_adapter() -> str:
    """Compiles adapter/forward_demo.cpp, the forward loops of include/pqa_forward.hpp
    behind one C entry point, with g++ against libpqa.so (warnings are errors)."""
    tmp_lib = DEMO_LIB + ".tmp"
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", "-Werror", "-pedantic", "-fPIC", "-shared",
           "-I" + os.path.join(ROOT, "include"), os.path.join(ADAPTER, "forward_demo.cpp"), "-o", tmp_lib,
           "-L" + PKG, "-lpqa", "-Wl,-rpath,$ORIGIN/.."]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"adapter build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp_lib, DEMO_LIB)
    return DEMO_LIB


def build_oracle(with_reference: bool = True) -> None:
    """Builds the CPU oracle (test infrastructure: the checker and its timing
    build) and, when the reference tree is present, the reference harness into
    oracle/_ref/."""
    odir = os.path.join(ROOT, "oracle")
    subprocess.run(["make", "-s", "-C", odir, "-B", "liboracle.so", "liboracle_bench.so"], check=True)
    if with_reference and os.path.isdir("/root/reference/cpp"):
        subprocess.run(["make", "-s", "-C", odir, "-B", "ref"], check=True)


if __name__ == "__main__":
    import sys

    if "--stamps" in sys.argv:
        build(verbose=True, stamps=True)
        build(verbose=True, stamps=True, step_stamps=True)
        sys.exit(0)
    build(verbose=True)
    build_adapter()
    build_oracle()
