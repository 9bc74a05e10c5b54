"""Builds the gfx950 DSA indexer in-tree.

  hcu_ops/libdsa_indexer.so   HIP kernels + the C ABI of include/dsa_indexer.h (hipcc, gfx950)
  hcu_ops/_C.<abi>.so         thin PyTorch-ROCm bind over that ABI (g++, links the library above)

Usage: python build.py [--jobs N] [--no-bind]
"""
import argparse
import json
import os
import re
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
PKG = os.path.join(HERE, "hcu_ops")
OBJ = os.path.join(HERE, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

HIP_SOURCES = ["status.cpp", "dequant.hip", "quant.hip", "mqa_logits_decode.hip", "topk.hip", "prefill_indexer.cpp",
               "mfma_probe.hip"]
# Packed fp32 VALU ops (v_pk_fma_f32 and friends) are switched off for every HIP source.  MFMA
# results are written to VGPRs directly (the epilogues read them with VALU ops; the AGPR form
# would add one v_accvgpr_read per result element).
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form=1", "-Wall", "-Wno-unused-command-line-argument"]


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"build step failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    return out


def kernel_resources(remarks):
    """{kernel: {field: value}} from hipcc's -Rpass-analysis=kernel-resource-usage remarks (VGPRs,
    AGPRs, scratch bytes per lane, LDS bytes per block, occupancy in waves per SIMD)."""
    fields = {"VGPRs": "vgpr", "AGPRs": "agpr", "ScratchSize [bytes/lane]": "scratch",
              "LDS Size [bytes/block]": "lds", "Occupancy [waves/SIMD]": "occupancy"}
    res, cur = {}, None
    for line in remarks.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            cur = res.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+(.+?): (\d+)\s*\[", line)
        if cur is not None and m and m.group(1) in fields:
            cur[fields[m.group(1)]] = int(m.group(2))
    return res


def build_library(jobs):
    os.makedirs(OBJ, exist_ok=True)
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    objs = []

    def compile_one(src):
        obj = os.path.join(OBJ, src.rsplit(".", 1)[0] + ".o")
        out = _run([hipcc, *HIP_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-x", "hip", "-c",
                    os.path.join(CSRC, src), "-o", obj])
        return obj, kernel_resources(out)

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        built = list(ex.map(compile_one, HIP_SOURCES))
    objs = [o for o, _ in built]
    usage = {}
    for _, r in built:
        usage.update(r)
    # per-kernel register / scratch / LDS use of this build (tests/test_build_resources.py reads it)
    with open(os.path.join(OBJ, "kernel_resources.json"), "w") as f:
        json.dump(usage, f, indent=1, sort_keys=True)
    lib = os.path.join(PKG, "libdsa_indexer.so")
    tmp = lib + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp, "-Wl,-soname,libdsa_indexer.so"])
    os.replace(tmp, lib)
    return lib


def build_bind():
    import torch  # noqa: F401
    import torch.utils.cpp_extension as ce
    import pybind11

    torch_lib = os.path.join(os.path.dirname(ce.__file__), "..", "lib")
    torch_lib = os.path.abspath(torch_lib)
    inc = ce.include_paths() + [pybind11.get_include(), sysconfig.get_paths()["include"],
                                os.path.join(ROCM, "include"), os.path.join(ROOT, "include")]
    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(PKG, "_C" + suffix)
    tmp = out + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi_flag()}",
           *[f"-I{p}" for p in inc], os.path.join(CSRC, "bind.cpp"), "-o", tmp,
           f"-L{PKG}", "-ldsa_indexer", f"-L{torch_lib}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
           "-lc10_hip", "-ltorch_hip", f"-L{os.path.join(ROCM, 'lib')}", "-lamdhip64",
           "-Wl,-rpath,$ORIGIN"]
    _run(cmd)
    os.replace(tmp, out)
    return out


def abi_flag():
    import torch
    return "1" if torch._C._GLIBCXX_USE_CXX11_ABI else "0"


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--no-bind", action="store_true")
    args = ap.parse_args(argv)
    lib = build_library(args.jobs)
    print("built", os.path.relpath(lib, ROOT), flush=True)
    if not args.no_bind:
        b = build_bind()
        print("built", os.path.relpath(b, ROOT), flush=True)


if __name__ == "__main__":
    sys.exit(main())
