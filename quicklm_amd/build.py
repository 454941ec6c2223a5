"""Build the native libraries in-tree.

  quicklm_amd/libqlm_hip.so     gfx950 HIP kernels + runtime plumbing (C ABI,
                                include/qlm_hip.h), compiled with hipcc.
  quicklm_amd/libqlm_engine.so  C++17 host engine (safetensors loader, model
                                assembly, graph-captured decode loop; C ABI in
                                include/qlm_engine.h), compiled with g++; it
                                reaches the GPU only through libqlm_hip.so.

Run as `python -m quicklm_amd.build`. Object files go to quicklm_amd/_build/.
"""

from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, "include")
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=fast-honor-pragmas",
    # Packed-fp32 VALU forms are disabled for every device compile.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument", "-I", INCLUDE,
]
# Per-file additions. gemm.hip: MFMA results in ordinary VGPRs; with the
# default accumulator-register form the group-32 prefill matmul copied every
# product back (two v_accvgpr_read per MFMA before its scale FMA), at the same
# register total.
# deltanet.hip: the column-split mixer's one ticket atomic (a single lane)
# is issued as it is; the atomic optimizer would turn it into a wave
# aggregation that waits for the returned value at once, in the middle of
# the mixer's chain, where the value is needed only at the kernel's end.
FILE_FLAGS = {"gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
              "deltanet.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"]}
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function", "-pthread",
             "-I", INCLUDE, "-I", os.path.join(CSRC, "host")]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops" not in l and "not a recognized feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")


def build_hip(jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "kernels", "*.hip")))
    objs = []
    cmds = []
    for s in srcs:
        o = os.path.join(BUILD, os.path.basename(s) + ".o")
        objs.append(o)
        extra = FILE_FLAGS.get(os.path.basename(s), [])
        cmds.append([HIPCC, *HIP_FLAGS, *extra, "-c", s, "-o", o])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    lib = os.path.join(PKG, "libqlm_hip.so")
    _run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", lib, *objs])
    return lib


def build_engine(jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "host", "*.cpp")))
    objs = []
    cmds = []
    for s in srcs:
        o = os.path.join(BUILD, os.path.basename(s) + ".o")
        objs.append(o)
        cmds.append(["g++", *CXX_FLAGS, "-c", s, "-o", o])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    lib = os.path.join(PKG, "libqlm_engine.so")
    _run(["g++", "-shared", "-o", lib, *objs, "-L", PKG, "-lqlm_hip",
          "-Wl,-rpath,$ORIGIN", "-pthread"])
    return lib


def build_all() -> None:
    build_hip()
    if glob.glob(os.path.join(CSRC, "host", "*.cpp")):
        build_engine()


if __name__ == "__main__":
    build_all()
    print("built:", ", ".join(sorted(glob.glob(os.path.join(PKG, "*.so")))))
    sys.exit(0)
