"""Build the MI355X extension in-tree.

  libtpo_hip.so  -- HIP kernels + C ABI (include/tpo.h), hipcc for gfx950
  _C.so          -- torch operator registrations (csrc/torch_ops.cpp), g++

Both land in torch_point_ops/ so the package finds them next to itself
(_C.so carries an $ORIGIN rpath to libtpo_hip.so).

    python torch-point-ops_amd/build.py [--jobs N] [--verbose]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
PKG = os.path.join(HERE, "torch_point_ops")
BUILD = os.path.join(HERE, "_build")
INCLUDE = os.path.join(REPO, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

HIP_SOURCES = ["capi.hip", "chamfer.hip", "chamfer_grid.hip", "knn.hip", "knn_hd.hip", "knn_bwd.hip", "knn_grid.hip", "knn_bf16.hip", "fps.hip", "gather.hip", "emd.hip"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # distance sums are contracted only where the source says __builtin_fma
    "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero",
    # no packed-FP32 VALU forms (v_pk_{add,mul,fma}_f32) anywhere
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    "-Wall",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
]

# fps.hip: its one-lane LDS atomic needs no wave-level pre-reduction.
# knn_bf16.hip: MFMA results in VGPRs, read by the VALU without AGPR copies.
HIPCC_FILE_FLAGS: dict = {"fps.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
                          "knn_bf16.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops" not in l and "not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def build_hip_lib(jobs: int = 8, verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, *HIPCC_FILE_FLAGS.get(src, []), "-c",
                     os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    out = os.path.join(PKG, "libtpo_hip.so")
    tmp = out + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
          "-Wl,-soname,libtpo_hip.so"], verbose)
    os.replace(tmp, out)
    return out


SHIM_SOURCES = ["torch_ops.cpp", "cpu_ops.cpp"]


def build_torch_shim(jobs: int = 8, verbose: bool = False) -> str:
    import torch
    from torch.utils import cpp_extension as ce

    inc = ce.include_paths("cuda") + [INCLUDE, sysconfig.get_paths()["include"]]
    libdirs = ce.library_paths("cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    os.makedirs(BUILD, exist_ok=True)
    cflags = [
        "g++", "-O3", "-std=c++17", "-fPIC",
        # the CPU kernels round after every + and *, as the reference's
        # plain x86-64 build does; at::parallel_for needs OpenMP
        "-ffp-contract=off", "-fopenmp",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-DTORCH_EXTENSION_NAME=_C", "-Wno-deprecated-declarations",
        *[f"-I{p}" for p in inc],
    ]
    objs, cmds = [], []
    for src in SHIM_SOURCES:
        obj = os.path.join(BUILD, src.replace(".cpp", ".o"))
        objs.append(obj)
        cmds.append([*cflags, "-c", os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(cmds)))) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    out = os.path.join(PKG, "_C.so")
    tmp = out + ".tmp"
    cmd = [
        "g++", "-shared", "-fopenmp", *objs, "-o", tmp,
        *[f"-L{p}" for p in libdirs],
        f"-L{PKG}", "-ltpo_hip",
        "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch",
        "-Wl,-rpath,$ORIGIN",
    ]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(jobs: int = 8, verbose: bool = False) -> None:
    build_hip_lib(jobs, verbose)
    build_torch_shim(jobs, verbose)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--verbose", action="store_true")
    a = ap.parse_args()
    build(a.jobs, a.verbose)
    print("built", os.path.join(PKG, "libtpo_hip.so"), os.path.join(PKG, "_C.so"))
    sys.exit(0)
