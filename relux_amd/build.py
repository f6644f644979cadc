"""Build librelux_kv.so (HIP, gfx950) in-tree and the CPU oracle.

    python -m relux_amd.build            # library only
    python -m relux_amd.build --oracle   # library + oracle/liboracle.so

The library is compiled with hipcc for gfx950 only.  Packed-FP32 VALU
instructions are disabled (-packed-fp32-ops) for every device object.
"""
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "librelux_kv.so")
SOURCES = ["rlx_runtime.hip", "rlx_cache_kernels.hip", "rlx_gqa_decode.hip", "rlx_mla_decode.hip",
           "rlx_prefill.hip", "rlx_mla_prefill.hip", "rlx_project.hip", "rlx_sampling.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: librelux_kv needs ROCm's hipcc to build")


def build_library(verbose=False):
    """Compile every HIP source to an object, then link the shared library."""
    hipcc = _hipcc()
    objdir = os.path.join(PKG, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs = []
    procs = []
    for src in SOURCES:
        obj = os.path.join(objdir, src.replace(".hip", ".o"))
        cmd = [hipcc, *HIPCC_FLAGS, "-I", os.path.join(ROOT, "include"), "-c",
               os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        objs.append(obj)
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        text = out.decode(errors="replace")
        # hipcc's host pass does not know the device-only feature flag.
        lines = [ln for ln in text.splitlines() if "packed-fp32-ops" not in ln]
        if lines and (verbose or p.returncode):
            print("\n".join(lines), flush=True)
        if p.returncode:
            failed.append(src)
    if failed:
        raise RuntimeError("hipcc failed for: " + ", ".join(failed))
    tmp = LIB + ".tmp"
    cmd = [hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


def build_oracle(verbose=False):
    """Compile the CPU oracle (test infrastructure) with its own Makefile."""
    odir = os.path.join(ROOT, "oracle")
    subprocess.run(["make", "-s", "-B", "-C", odir], check=True,
                   stdout=None if verbose else subprocess.DEVNULL)
    return os.path.join(odir, "liboracle.so")


if __name__ == "__main__":
    v = "-v" in sys.argv
    print(build_library(verbose=v))
    if "--oracle" in sys.argv:
        print(build_oracle(verbose=v))
