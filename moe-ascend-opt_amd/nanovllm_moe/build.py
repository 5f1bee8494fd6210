"""Build recipes for the native parts of the package (run on the CPU host).

* ``libmimoe.so`` -- the HIP kernels + C ABI (include/mi_moe.h), built with
  hipcc for gfx950 only.  No torch dependency.
* ``libnanovllm_shim.so`` -- the TorchBind / dispatcher registration
  (``torch.classes.nanovllm.MoEInfer``, ``torch.ops.nanovllm.moe_forward``),
  linked against libmimoe.so.

Both land next to this file so they travel with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)                    # moe-ascend-opt_amd/
CSRC = os.path.join(ROOT, "csrc")
INCLUDE = os.path.join(os.path.dirname(ROOT), "include")
LIB = os.path.join(PKG_DIR, "libmimoe.so")
SHIM = os.path.join(PKG_DIR, "libnanovllm_shim.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_SOURCES = ["capi.hip", "common_kernels.hip", "w4a16.hip", "w4a16_fused.hip", "qint.hip", "hybrid.hip"]
# Host-only C++ (no HIP): the host executor of the hybrid offload path and the
# CPU engine of the Q8_0 / Q4_0 layer (its C ABI too).  Inner loops are
# compiled per instruction set (target attributes) and picked at run time;
# -ffp-contract=off keeps the stated fp32 order.
CXX = os.environ.get("CXX", "g++")
CPP_SOURCES = ["host_experts.cpp", "cpu_moe.cpp", "capi_cpu.cpp"]
CPP_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-pthread", "-ffp-contract=off", "-fvisibility=hidden"]
# Packed-FP32 instructions are disabled for all device code (only scalar /
# float2 source is written; the compiler must not form v_pk_* fp32 ops).
NO_PK_FP32 = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# Per-file device flags.  The grouped GEMMs read every MFMA result with VALU
# ops (the per-block fp32 scaling, the W4A16 zero/scale fold); the VGPR form
# of the MFMA saves a v_accvgpr_read per result register.  The W4A16 decode
# kernels compile to the same code either way.  Kernel-argument preloading
# (gfx950: the first 14 dwords of a kernel's scalar arguments arrive in SGPRs
# at wave launch) takes the argument fetch off the decode kernels' chain of
# dependent loads; the kernels pass their first-needed fields as leading
# scalar arguments (a by-value struct is not preloaded).
FILE_FLAGS = {"qint.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-amdgpu-kernarg-preload-count=16"],
              "w4a16.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-amdgpu-kernarg-preload-count=16"],
              "w4a16_fused.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-amdgpu-kernarg-preload-count=16"],
              "common_kernels.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"]}


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        sys.stderr.write(out + "\n")
        raise RuntimeError("build step failed: " + " ".join(cmd[:3]) + " ...")
    return out


def build_lib(verbose: bool = False) -> str:
    from concurrent.futures import ThreadPoolExecutor
    srcs = [s for s in HIP_SOURCES if os.path.exists(os.path.join(CSRC, s))]
    objdir = os.path.join(PKG_DIR, "_obj")
    os.makedirs(objdir, exist_ok=True)

    def compile_one(src):
        obj = os.path.join(objdir, src.replace(".hip", ".o"))
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-c",
               "-fvisibility=hidden", f"-I{INCLUDE}", f"-I{CSRC}", *NO_PK_FP32,
               *FILE_FLAGS.get(src, []), os.path.join(CSRC, src), "-o", obj]
        return obj, _run(cmd)

    def compile_cpp(src):
        obj = os.path.join(objdir, src.replace(".cpp", ".o"))
        cmd = [CXX, *CPP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", os.path.join(CSRC, src), "-o", obj]
        return obj, _run(cmd)

    cpp = [s for s in CPP_SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        jobs = [ex.submit(compile_one, s) for s in srcs] + [ex.submit(compile_cpp, s) for s in cpp]
        results = [j.result() for j in jobs]
    tmp = LIB + ".tmp"
    out = _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *[o for o, _ in results], "-o", tmp,
                "-pthread"])
    text = "\n".join(t for _, t in results if t.strip()) + out
    if verbose and text.strip():
        print(text)
    os.replace(tmp, LIB)
    return LIB


def _torch_paths():
    import torch
    tdir = os.path.dirname(torch.__file__)
    inc = [os.path.join(tdir, "include"), os.path.join(tdir, "include", "torch", "csrc", "api", "include")]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return inc, os.path.join(tdir, "lib"), abi


def build_shim(verbose: bool = False) -> str:
    inc, libdir, abi = _torch_paths()
    tmp = SHIM + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-DTORCH_EXTENSION_NAME=nanovllm_shim",
           *[f"-I{p}" for p in inc], "-I/opt/rocm/include", f"-I{INCLUDE}",
           os.path.join(CSRC, "nanovllm_shim.cpp"), "-o", tmp,
           f"-L{libdir}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
           f"-L{PKG_DIR}", "-lmimoe",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}", "-Wl,--no-as-needed"]
    out = _run(cmd)
    if verbose and out.strip():
        print(out)
    os.replace(tmp, SHIM)
    return SHIM


FLOOR = os.path.join(PKG_DIR, "mimoe_read_floor")


def build_read_floor(verbose: bool = False) -> str:
    """The read-only floor probe (csrc/read_floor.hip): a standalone HIP program
    that `bench.py --read-floor` runs."""
    tmp = FLOOR + ".tmp"
    out = _run([HIPCC, f"--offload-arch={ARCH}", "-O3", "-std=c++17", *NO_PK_FP32,
                os.path.join(CSRC, "read_floor.hip"), "-o", tmp])
    if verbose and out.strip():
        print(out)
    os.replace(tmp, FLOOR)
    return FLOOR


def build_all(verbose: bool = False):
    build_lib(verbose)
    build_shim(verbose)
    build_read_floor(verbose)
    return LIB, SHIM


if __name__ == "__main__":
    build_all(verbose=True)
    print("built", LIB, SHIM)
