"""Build the gfx950 library and the hipkittens-compatible Python modules in-tree.

    python amd-kernels_amd/build.py            # libhkq.so + pybind modules
    python amd-kernels_amd/build.py --isa      # also dump device ISA + resource usage

Outputs (git-ignored, but shipped with the tree):
    amd-kernels_amd/lib/libhkq.so                       C ABI (include/hkq.h)
    amd-kernels_amd/hipkittens/kernels/<name>_tk<EXT>   pybind11 modules
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import re
import shutil
import subprocess
import sys
import sysconfig

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB_DIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIB_DIR, "libhkq.so")
MOD_DIR = os.path.join(PKG, "hipkittens", "kernels")
INCLUDE = os.path.join(ROOT, "include")
EXT_SUFFIX = sysconfig.get_config_var("EXT_SUFFIX")
PY_INCLUDE = sysconfig.get_paths()["include"]

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
ARCH = "gfx950"
# Packed-FP32 VALU forms are disabled for all device code (some of their forms
# have produced wrong results on this pool's MI355X boxes).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE, "-I", CSRC,
    "-Wno-unused-command-line-argument",
]

HIP_SOURCES = ["quant.hip", "gemm.hip", "gemm_blockscale.hip", "moe.hip", "moe_blockscale.hip", "routing.hip",
               "norm_quant.hip"]
CPP_SOURCES = ["hkq_error.cpp"]
# Per-source code generation options. The block-scale GEMM promotes every
# K group on the VALU (acc += P * scale): its MFMAs must write the partial P
# to arch VGPRs, which the compiler's default register-class choice does not
# do (it writes AGPRs and then copies every element out).
SRC_FLAGS = {"gemm_blockscale.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}

# pybind11 module name -> binding source (module names are the reference's)
MODULES = {
    "quant_tk": "bind_quant.cpp",
    "quant_moe_tk": "bind_quant_moe.cpp",
    "gemm_a8w8_tk": "bind_gemm_a8w8.cpp",
    "gemm_a8w8_per_token_scale_tk": "bind_gemm_a8w8_per_token_scale.cpp",
    "gemm_afp4wfp4_tk": "bind_gemm_afp4wfp4.cpp",
    "gemm_a8w8_blockscale_tk": "bind_gemm_a8w8_blockscale.cpp",
    "gemm_a16w16_tk": "bind_gemm_a16w16.cpp",
    "batched_gemm_a8w8_tk": "bind_batched_gemm_a8w8.cpp",
    "batched_gemm_bf16_tk": "bind_batched_gemm_bf16.cpp",
    "fused_gemm_a8w8_blockscale_mul_add_tk": "bind_fused_gemm_a8w8_blockscale_mul_add.cpp",
    "fused_gemm_a8w8_blockscale_a16w16_tk": "bind_fused_gemm_a8w8_blockscale_a16w16.cpp",
    "moe_op_gemm_a8w8_tk": "bind_moe_op_gemm_a8w8.cpp",
    "moe_op_gemm_a8w8_blockscale_tk": "bind_moe_op_gemm_a8w8_blockscale.cpp",
    "moe_op_mxfp4_tk": "bind_moe_op_mxfp4.cpp",
    "fused_fp8_quant_tk": "bind_fused_fp8_quant.cpp",
    "fused_mxfp4_quant_tk": "bind_fused_mxfp4_quant.cpp",
    "moe_topk_tk": "bind_moe_topk.cpp",
    "moe_bitmatrix_tk": "bind_moe_bitmatrix.cpp",
    "moe_expt_data_tk": "bind_moe_expt_data.cpp",
    "moe_align_block_size_tk": "bind_moe_align_block_size.cpp",
    "moe_routing_tk": "bind_moe_routing.cpp",
}


def _run(cmd, log=None):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {os.path.basename(cmd[-1])}")
    if log is not None:
        with open(log, "w") as f:
            f.write(r.stdout + r.stderr)
    return r


def _obj(src):
    return os.path.join(BUILD, os.path.basename(src) + ".o")


def compile_hip(src, isa=False):
    path = os.path.join(CSRC, src)
    out = _obj(src)
    flags = [*HIP_FLAGS, *SRC_FLAGS.get(src, [])]
    cmd = [HIPCC, *flags, "-Rpass-analysis=kernel-resource-usage", "-c", path, "-o", out]
    _run(cmd, log=os.path.join(BUILD, src + ".resource.txt"))
    if isa:
        s = os.path.join(BUILD, src + ".s")
        _run([HIPCC, *flags, "--cuda-device-only", "-S", path, "-o", s])
    return out


def compile_cpp(src):
    out = _obj(src)
    inc = ["-I", INCLUDE, "-I", CSRC, "-I", "/opt/rocm/include"]
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-D__HIP_PLATFORM_AMD__", *inc, "-c", os.path.join(CSRC, src), "-o", out])
    return out


def link_lib(objs):
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    # A kernel template whose host-side instantiation failed leaves its launch
    # stub undefined without any compiler diagnostic: refuse such a library.
    und = subprocess.run(["nm", "-C", "--undefined-only", tmp], capture_output=True, text=True).stdout
    missing = [l.strip() for l in und.splitlines() if "hkq::" in l]
    if missing:
        os.remove(tmp)
        raise RuntimeError("libhkq.so has undefined library symbols:\n  " + "\n  ".join(missing))
    os.replace(tmp, LIB)


def build_module(name, src):
    import pybind11

    os.makedirs(MOD_DIR, exist_ok=True)
    out = os.path.join(MOD_DIR, name + EXT_SUFFIX)
    tmp = out + ".tmp"
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
        f"-DHKQ_MODULE_NAME={name}",
        "-I", pybind11.get_include(), "-I", PY_INCLUDE, "-I", INCLUDE, "-I", CSRC,
        os.path.join(CSRC, "bind", src), "-o", tmp,
        "-L", LIB_DIR, "-lhkq", "-Wl,-rpath,$ORIGIN/../../lib",
    ]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build(isa: bool = False, jobs: int | None = None) -> None:
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(compile_hip, s, isa) for s in HIP_SOURCES]
        futs += [ex.submit(compile_cpp, s) for s in CPP_SOURCES]
        objs = [f.result() for f in futs]
    link_lib(objs)
    with cf.ThreadPoolExecutor(jobs) as ex:
        for f in [ex.submit(build_module, n, s) for n, s in MODULES.items()]:
            f.result()
    if isa:
        check_isa()


_MFMA = re.compile(r"v_mfma\S*\s+v\[(\d+):(\d+)\],\s*v\[(\d+):(\d+)\],\s*v\[(\d+):(\d+)\]")


def check_isa():
    """Report spills and per-kernel register usage from the resource remarks."""
    for src in HIP_SOURCES:
        txt = open(os.path.join(BUILD, src + ".resource.txt")).read()
        for m in re.finditer(r"Function Name: (\S+)[\s\S]*?VGPRs: (\d+)[\s\S]*?AGPRs: (\d+)[\s\S]*?ScratchSize \[bytes/lane\]: (\d+)[\s\S]*?LDS Size \[bytes/block\]: (\d+)", txt):
            name, v, a, scratch, lds = m.groups()
            flag = "  <-- SPILLS" if int(scratch) else ""
            print(f"{src}: {name[:90]} VGPR={v} AGPR={a} scratch={scratch} LDS={lds}{flag}")


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--isa", action="store_true")
    ap.add_argument("-j", type=int, default=None)
    a = ap.parse_args()
    build(isa=a.isa, jobs=a.j)
    print("built", LIB)
