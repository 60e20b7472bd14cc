"""Build libmiq.so (HIP kernels + C ABI) for gfx950 with hipcc, in-tree.

    python -m webpytorch_amd.build        # compiles every source, links webpytorch_amd/libmiq.so

Each `csrc/*.hip` file is compiled to an object in `csrc/_build/` in parallel, then linked
into one shared library next to this file. The library links only the HIP runtime.
"""
import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(CSRC, "_build")
LIB = os.path.join(HERE, "libmiq.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
ARCH = "gfx950"


def hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (ROCm is required to build libmiq)")


FLAGS = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=" + ARCH, "-munsafe-fp-atomics",
         # packed fp32 VALU ops are kept out of the generated code on this target
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wno-unused-result", "-I" + INCLUDE, "-I" + CSRC]


# per-source flags: the matrix-core kernels keep their MFMA accumulators in ordinary VGPRs, so
# the per-group scale fold reads them without a copy out of the accumulation registers
FILE_FLAGS = {"gptq_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src):
    obj = os.path.join(OBJ, os.path.basename(src).replace(".hip", ".o"))
    cmd = [hipcc()] + FLAGS + FILE_FLAGS.get(os.path.basename(src), []) + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed for %s:\n%s" % (src, r.stderr[-4000:]))
    return obj


def build(jobs=None, verbose=True):
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    jobs = jobs or min(8, len(srcs))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", "--offload-arch=" + ARCH, "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr[-4000:])
    os.replace(tmp, LIB)
    if verbose:
        print("built %s from %d sources" % (LIB, len(srcs)))
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
