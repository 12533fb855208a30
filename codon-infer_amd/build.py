"""Builds codon-infer_amd/codon_hip/libcodon_hip.so for gfx950.

Every .hip and .cpp file under csrc/ is compiled with hipcc (in parallel)
and linked into one shared library exporting the C ABI of
include/codon_hip.h.  Usage: python codon-infer_amd/build.py
"""
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "codon_hip", "libcodon_hip.so")
ARCH = os.environ.get("CIH_OFFLOAD_ARCH", "gfx950")


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src):
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [hipcc(), "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result", "-c", src, "-o", obj]
    if src.endswith(".hip"):
        # packed FP32 (v_pk_*_f32) is disabled for all device code
        cmd[1:1] = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose=True):
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs + ["-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print("built", OUT)
    build_capi(verbose)
    return OUT


CAPI_SRC = os.path.join(HERE, "capi", "pipeline.c")
CAPI_OUT = os.path.join(HERE, "capi", "pipeline")


def build_capi(verbose=True):
    """The C caller of the ABI (capi/pipeline.c), compiled as C99 against
    include/codon_hip.h with gcc and linked to the library next to it."""
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no C compiler for capi/pipeline.c")
    cmd = [cc, "-O2", "-std=c99", "-D_POSIX_C_SOURCE=200809L", "-Wall", "-Wextra", "-Werror", CAPI_SRC, "-o",
           CAPI_OUT + ".tmp", "-L" + os.path.dirname(OUT), "-lcodon_hip", "-Wl,-rpath,$ORIGIN/../codon_hip", "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(CAPI_OUT + ".tmp", CAPI_OUT)
    if verbose:
        print("built", CAPI_OUT)


if __name__ == "__main__":
    try:
        build()
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
