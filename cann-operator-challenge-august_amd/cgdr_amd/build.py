"""Build the in-tree HIP library ``lib/libcgdr_fwd_h.so`` for gfx950 and the golden-case
runner ``lib/cgdr_golden_runner`` (host C++ linked against the library and the HIP runtime).

``python -m cgdr_amd.build`` (with ``cann-operator-challenge-august_amd`` on sys.path), or
``build_library()`` from Python.  hipcc cross-compiles without a GPU.
"""

from __future__ import annotations

import os
import subprocess
import sys

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REPO_ROOT = os.path.dirname(_PKG_ROOT)
CSRC = os.path.join(_PKG_ROOT, "csrc")
LIB_DIR = os.path.join(_PKG_ROOT, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libcgdr_fwd_h.so")
RUNNER_PATH = os.path.join(LIB_DIR, "cgdr_golden_runner")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in device code.
# -amdgpu-mfma-vgpr-form: MFMA accumulators in VGPRs, so the state is not shuttled between
# AGPRs and VGPRs around every chunk's VALU work.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-function",
    # The direct-to-LDS DMA asm clobbers M0; no other code in these kernels uses M0
    # (checked on the generated assembly), so the reserved-register warning is noise.
    "-Wno-inline-asm",
]

SOURCES = [os.path.join(CSRC, n) for n in ("cgdr_fwd_h_k128.hip", "cgdr_fwd_h_k64.hip", "cgdr_fwd_h_k256.hip",
                                           "cgdr_fwd_h_k32.hip", "cgdr_fwd_h.hip", "cgdr_chunk_o.hip", "cgdr_wy.hip")]
RUNNER_SOURCE = os.path.join(CSRC, "cgdr_golden_runner.cpp")
HEADERS = [os.path.join(CSRC, n) for n in ("cgdr_kernels.h", "cgdr_fwd_h_dispatch.h", "cgdr_schedule.h", "cgdr_host.h",
                                          "cgdr_chunk_common.h", "cgdr_chunk_o_kernel.h", "cgdr_wy_kernel.h")] + \
    [os.path.join(REPO_ROOT, "include", n) for n in ("cgdr_fwd_h.h", "cgdr_chunk_o.h", "cgdr_wy.h")]


def build_library(verbose: bool = False) -> str:
    """Compile the library (always, even if a built copy exists) and return its path.

    Each translation unit is compiled in its own hipcc process (in parallel), then linked."""
    os.makedirs(LIB_DIR, exist_ok=True)
    objs = [os.path.join(LIB_DIR, os.path.basename(src) + ".o") for src in SOURCES]
    noise = "is not a recognized feature for this target"
    cflags = [f for f in HIP_FLAGS if f != "-shared"]
    procs = []
    for src, obj in zip(SOURCES, objs):
        cmd = [HIPCC, *cflags, "-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append(subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True))
    errors = []
    for pr in procs:
        _, err = pr.communicate()
        err = "\n".join(l for l in (err or "").splitlines() if noise not in l)
        if pr.returncode != 0:
            errors.append(err)
        elif verbose and err.strip():
            print(err, file=sys.stderr)
    if errors:
        raise RuntimeError("hipcc failed:\n" + "\n".join(errors))
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed ({res.returncode}):\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    for obj in objs:
        os.remove(obj)
    return LIB_PATH


def build_runner(verbose: bool = False) -> str:
    """Compile the golden-case runner (host code only) against the built library."""
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} missing: build_library() first")
    tmp = RUNNER_PATH + ".tmp"
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
           "-I", os.path.join(REPO_ROOT, "include"), "-I", os.path.join(ROCM, "include"),
           RUNNER_SOURCE, "-o", tmp, "-L", LIB_DIR, "-lcgdr_fwd_h",
           "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
           "-Wl,-rpath,$ORIGIN", "-Wl,-rpath," + os.path.join(ROCM, "lib")]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed ({res.returncode}):\n{res.stderr}")
    if verbose and res.stderr.strip():
        print(res.stderr, file=sys.stderr)
    os.replace(tmp, RUNNER_PATH)
    return RUNNER_PATH


def build_all(verbose: bool = False) -> list[str]:
    return [build_library(verbose), build_runner(verbose)]


if __name__ == "__main__":
    print("\n".join(build_all(verbose=True)))
