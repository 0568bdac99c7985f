"""Build recipe for libkernix.so (gfx950 HIP kernels + C host runtime) and the CPU oracle used by the tests.

    python -m kernix_amd.build          # or __graft_entry__.build()

Every HIP source is compiled with hipcc for gfx950 only; host C with gcc.  Objects go to kernix_amd/_build/, the
library to kernix_amd/libkernix.so.  HIP code is compiled with -ffp-contract=off (no FMA contraction: the int8
epilogue is bit-exact against the oracle) and without packed-fp32 instruction selection.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "kernix_amd")
SRC = os.path.join(PKG, "csrc")
OUT = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libkernix.so")
INC = os.path.join(ROOT, "include")

HIP_SOURCES = ["knx_runtime", "knx_i8gemm", "knx_sgemm", "knx_conv", "knx_rows", "knx_attn", "knx_chain", "knx_rnn"]
C_SOURCES = ["knx_decode", "knx_graph", "knx_forward", "knx_capi"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-pragma-unroll-threshold=1000000",
    "-Wall", "-Wno-unused-function",
]
# KNX_TUNING=1: also build the kernel variants that only the forcing switches (KNX_I8_KERNEL, KNX_SGEMM_KERNEL) reach
if os.environ.get("KNX_TUNING", "") not in ("", "0"):
    HIP_FLAGS.append("-DKNX_TUNING")
C_FLAGS = ["-O2", "-std=c11", "-fPIC", "-fvisibility=hidden", "-D_GNU_SOURCE", "-ffp-contract=off",
           "-Wall", "-Wextra", "-Wno-unused-parameter"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    return err


def _hip(name):
    src = os.path.join(SRC, "hip", name + ".hip")
    obj = os.path.join(OUT, name + ".o")
    return _run([HIPCC, *HIP_FLAGS, "-I", INC, "-I", os.path.join(SRC, "hip"), "-c", src, "-o", obj]), obj


def _c(name):
    src = os.path.join(SRC, "host", name + ".c")
    obj = os.path.join(OUT, name + ".o")
    return _run(["gcc", *C_FLAGS, "-I", INC, "-I", os.path.join(SRC, "host"), "-c", src, "-o", obj]), obj


def build_lib(verbose=False):
    os.makedirs(OUT, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        jobs = [ex.submit(_hip, n) for n in HIP_SOURCES] + [ex.submit(_c, n) for n in C_SOURCES]
        objs = []
        for j in jobs:
            warn, obj = j.result()
            if verbose and warn.strip():
                print(warn, file=sys.stderr)
            objs.append(obj)
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs, "-Wl,--no-undefined", "-lm", "-lpthread"])
    os.replace(tmp, LIB)
    return LIB


def build_oracle():
    odir = os.path.join(ROOT, "oracle")
    make = shutil.which("make")
    if make is None:
        raise RuntimeError("make not found")
    _run([make, "-s", "-C", odir])
    return os.path.join(odir, "_build", "libknx_oracle.so")


def build_all(verbose=False):
    lib = build_lib(verbose)
    orc = build_oracle()
    return lib, orc


if __name__ == "__main__":
    print(build_all(verbose="-v" in sys.argv))
