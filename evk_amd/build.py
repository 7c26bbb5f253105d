"""Build script for the gfx950 kernel library and its C++ API layer.

    python -m evk_amd.build            # builds evk_amd/libevkhip.so and evk_amd/libevk.so

libevkhip.so  - the C ABI of include/evkhip.h (hipcc, --offload-arch=gfx950)
libevk.so     - the evk / evk::ai C++ API of include/evk.h, include/evk_ai.h,
                implemented over libevkhip.so
Both are written in-tree so they travel with the repository snapshot.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("EVK_OFFLOAD_ARCH", "gfx950")

KERNEL_SOURCES = ["capi.hip", "gemm.hip", "flash.hip", "flash_wide.hip", "decode_ops.hip", "model.hip", "decode_persist.hip",
                  "kv_step.hip", "train_ops.hip"]
API_SOURCES = ["evk_runtime.cpp", "evk_ai.cpp"]

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # packed fp32 instructions are kept out of the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-Wno-unused-result",
]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("build failed:\n" + " ".join(cmd) + "\n" + r.stdout + r.stderr)
    return r


# Files whose MFMA accumulators fit in the architectural VGPRs: keep them there
# (no AGPR<->VGPR copies around the softmax / epilogue arithmetic).
VGPR_MFMA = {"flash.hip", "flash_wide.hip"}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    extra = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"] if src in VGPR_MFMA else []
    cmd = [HIPCC] + HIP_FLAGS + extra + ["-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd = [HIPCC, "-x", "hip"] + HIP_FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj]
    _run(cmd)
    return obj


def build(verbose: bool = False) -> None:
    os.makedirs(BUILD, exist_ok=True)
    srcs = KERNEL_SOURCES + [s for s in API_SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = dict(zip(srcs, ex.map(_compile, srcs)))
    kern = os.path.join(HERE, "libevkhip.so")
    tmp = kern + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + [objs[s] for s in KERNEL_SOURCES])
    os.replace(tmp, kern)
    api = [objs[s] for s in API_SOURCES if s in objs]
    if api:
        lib = os.path.join(HERE, "libevk.so")
        tmp = lib + ".tmp"
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + api +
             ["-L", HERE, "-levkhip", "-Wl,-rpath,$ORIGIN"])
        os.replace(tmp, lib)
    if api:
        # programs over the evk / evk::ai API (tests/cpp), linked against
        # libevk.so: the API tests and the main_llm decode tool
        os.makedirs(os.path.join(HERE, "bin"), exist_ok=True)

        def program(name):
            exe = os.path.join(HERE, "bin", name)
            _run([HIPCC, "-x", "hip", "--offload-arch=" + ARCH] + HIP_FLAGS[1:] +
                 [os.path.join(ROOT, "tests", "cpp", name + ".cpp"), "-o", exe + ".tmp",
                  "-L", HERE, "-levk", "-levkhip", "-Wl,-rpath,$ORIGIN/.."])
            os.replace(exe + ".tmp", exe)

        with cf.ThreadPoolExecutor(max_workers=2) as ex:
            list(ex.map(program, ["api_tests", "kv_decoder_tool"]))
    if verbose:
        print("built", kern)


def build_decode_trace(verbose: bool = False) -> str:
    """evk_amd/_trace/libevkhip.so: the library with the persistent decode's
    stage timestamps compiled in (EVKHIP_DECODE_TRACE); evk_amd/decode_trace.py
    loads it.  The other objects come from the last build()."""
    out_dir = os.path.join(HERE, "_trace")
    os.makedirs(out_dir, exist_ok=True)
    obj = os.path.join(out_dir, "decode_persist.hip.o")
    _run([HIPCC] + HIP_FLAGS + ["-DEVKHIP_DECODE_TRACE", "-c", os.path.join(CSRC, "decode_persist.hip"), "-o", obj])
    objs = [obj if s == "decode_persist.hip" else os.path.join(BUILD, s + ".o") for s in KERNEL_SOURCES]
    lib = os.path.join(out_dir, "libevkhip.so")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", lib + ".tmp"] + objs)
    os.replace(lib + ".tmp", lib)
    if verbose:
        print("built", lib)
    return lib


if __name__ == "__main__":
    build(verbose=True)
    if "--decode-trace" in sys.argv:
        build_decode_trace(verbose=True)
    sys.exit(0)
