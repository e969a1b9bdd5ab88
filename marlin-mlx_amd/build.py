"""Build libmq4.so (HIP, gfx950 only) in-tree.

Each csrc/*.hip file is compiled with hipcc to an object under _build/ (in
parallel) and linked into marlin-mlx_amd/libmq4.so.  Flags:
  --offload-arch=gfx950        the only target
  -fhip-fp32-correctly-rounded-divide-sqrt
                               IEEE division, needed for bit-exact quantize
  -Xclang -target-feature -Xclang -packed-fp32-ops
                               no packed FP32 (v_pk_*_f32) code generation
No fast-math flags are used anywhere.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmq4.so")
CPP_DEMO_SRC = os.path.join(ROOT, "tests", "cpp", "mq4_cpp_demo.cpp")
CPP_DEMO = os.path.join(BUILD, "mq4_cpp_demo")
CACHE_TOOL_SRC = os.path.join(ROOT, "tests", "cpp", "mq4_cache_tool.cpp")
CACHE_TOOL = os.path.join(BUILD, "mq4_cache_tool")
DEVCHECK_SRC = os.path.join(ROOT, "tests", "hip", "mq4_device_check.hip")
DEVCHECK = os.path.join(BUILD, "libmq4_devcheck.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-variable", "-Wno-unused-function",
    "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
]


# Per-source extra flags.  mq4_gemm.hip: MFMA results and accumulators in
# VGPRs (-amdgpu-mfma-vgpr-form).  Its per-group fold (acc += s * D) is VALU
# work on the MFMA results; with them in AGPRs every group moved 128 values
# between AGPRs and VGPRs (v_accvgpr_read/write), half the loop's VALU
# instructions.
# mq4_rows.hip: no wave-level atomic combining.  Its one arrival count per
# workgroup would otherwise be rewritten into a combined add whose result is
# read back at once, which stalls the issuing wave on every load issued
# before it (the count's result is only needed at the end of the kernel).
EXTRA_FLAGS = {
    "mq4_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "mq4_rows.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}

# Sources whose kernels wait for their LDS DMA with exact vmcnt counts: that
# count assumes no other vector memory traffic in the loop, and register
# spills to scratch are vector memory operations (a spilling build waits too
# little and reads stages before their DMA has landed).  The build fails if
# any kernel in them uses scratch.  (mq4_gemm16.hip waits for all of its
# DMA every group, but a spilling build would also be a slow one.)
NO_SCRATCH = {"mq4_gemm.hip", "mq4_gemm16.hip", "mq4_decode.hip"}


def _scratch_users(remarks: str) -> list[tuple[str, int]]:
    """(kernel, bytes per lane) for every function the resource-usage remarks
    report with a nonzero ScratchSize."""
    out, name = [], None
    for line in remarks.splitlines():
        if "Function Name: " in line:
            name = line.split("Function Name: ", 1)[1].split()[0]
        elif "ScratchSize [bytes/lane]: " in line and name is not None:
            n = int(line.split("ScratchSize [bytes/lane]: ", 1)[1].split()[0])
            if n > 0:
                out.append((name, n))
    return out


def _compile(src: str) -> str:
    base = os.path.basename(src)
    obj = os.path.join(BUILD, base + ".o")
    check = base in NO_SCRATCH
    cmd = [HIPCC, *CFLAGS, *EXTRA_FLAGS.get(base, []),
           *(["-Rpass-analysis=kernel-resource-usage", "-fno-caret-diagnostics"] if check else []),
           "-c", src, "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature; that notice is harmless.
    lines = [l for l in p.stderr.splitlines() if "packed-fp32-ops" not in l]
    if check:
        spills = _scratch_users("\n".join(lines))
        lines = [l for l in lines if "kernel-resource-usage" not in l]
        if spills and p.returncode == 0:
            raise RuntimeError(f"{base}: kernels use scratch memory, which breaks their exact vmcnt waits "
                               f"for LDS DMA: " + ", ".join(f"{k} ({n} B/lane)" for k, n in spills))
    err = "\n".join(lines)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(verbose: bool = True) -> str:
    """Compile every csrc/*.hip and link libmq4.so; returns the library path."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not srcs:
        raise RuntimeError("no HIP sources found")
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("link failed:\n" + p.stderr)
    os.replace(tmp, LIB)
    if os.path.exists(CPP_DEMO_SRC):
        # C++ caller of the header-only host API (tests/cpp), linked to libmq4.so
        cmd = [HIPCC, "-O2", "-std=c++17", "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
               CPP_DEMO_SRC, "-o", CPP_DEMO, "-L" + HERE, "-lmq4", "-Wl,-rpath,$ORIGIN/.."]
        p = subprocess.run(cmd, capture_output=True, text=True)
        if p.returncode != 0:
            raise RuntimeError("C++ demo build failed:\n" + p.stderr)
    if os.path.exists(CACHE_TOOL_SRC):
        # host-only C++ check of the safetensors Q4 cache header (tests/cpp)
        cmd = [HIPCC, "-O2", "-std=c++17", "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
               CACHE_TOOL_SRC, "-o", CACHE_TOOL]
        p = subprocess.run(cmd, capture_output=True, text=True)
        if p.returncode != 0:
            raise RuntimeError("C++ cache tool build failed:\n" + p.stderr)
    if os.path.exists(DEVCHECK_SRC):
        # device-helper checks for the tests (tests/hip), with the library's flags
        cmd = [HIPCC, *CFLAGS, "-shared", DEVCHECK_SRC, "-o", DEVCHECK]
        p = subprocess.run(cmd, capture_output=True, text=True)
        if p.returncode != 0:
            raise RuntimeError("device check build failed:\n" + p.stderr)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)
    if os.path.exists(LIB):
        os.remove(LIB)


if __name__ == "__main__":
    if "--clean" in sys.argv:
        clean()
    build()
