"""Builds libprism_amd.so (the gfx950 HIP kernels and their C ABI) in-tree with hipcc.

    python startlux-prism_amd/build.py [-j N]

Each csrc/*.hip compiles to an object under csrc/_build/, then one shared library links next to the Python package
(startlux-prism_amd/prism_amd/libprism_amd.so), which prism_amd._lib loads.  Flags:
  --offload-arch=gfx950                        MI355X / MI350X only; no other targets, no host fallback
  -fhip-fp32-correctly-rounded-divide-sqrt     '/' on fp32 is the IEEE division the quantizers are specified with
  -ffp-contract=off                            no implicit a*b+c contraction: roundings are the ones written
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed-fp32 VALU instructions in the generated code
"""
import argparse
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(CSRC, "_build")
LIB = os.path.join(HERE, "prism_amd", "libprism_amd.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
         "-fhip-fp32-correctly-rounded-divide-sqrt", "-fvisibility=hidden",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-function", "-Wno-unused-variable"]


# per-file additions: the packed Q8_0 kernels fold MFMA results with VALU ops, which the VGPR form of the MFMA saves
# a copy per value
FILE_FLAGS = {"w8a8_packed.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src):
    obj = os.path.join(OBJ, os.path.basename(src).replace(".hip", ".o"))
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in (r.stderr or "").splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    return obj, err


def build(jobs=8, verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max(1, jobs)) as ex:
        res = list(ex.map(_compile, srcs))
    for _, err in res:
        if err.strip() and verbose:
            print(err, file=sys.stderr)
    objs = [o for o, _ in res]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=8)
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    print(build(a.j, a.v))
