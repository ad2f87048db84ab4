"""Builds libsmol_attn.so (gfx950) in-tree with hipcc.

    python smol-genius_amd/build.py

Every HIP source is compiled with -Xclang -target-feature -Xclang
-packed-fp32-ops, which keeps the compiler from emitting packed fp32 VALU
instructions (the host pass warns that it does not know the feature; that is
expected).
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ROOT = os.path.dirname(HERE)
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libsmol_attn.so")
SOURCES = ["attn_prep.hip", "attn_decode.hip", "attn_fa.hip", "attn_fb.hip", "attn_win.hip", "attn_api.hip", "qkn_attn.hip", "linear.hip", "gemm.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("SMOL_ATTN_ARCH", "gfx950")

FLAGS = [
    "--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result", "-Wno-unused-value", "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
]


KERNEL_FLAGS = {}
LIBS = []


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC] + FLAGS + KERNEL_FLAGS.get(src, []) + ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed for %s:\n%s" % (src, msg))
    if msg.strip():
        print(msg)
    return obj


def build():
    os.makedirs(BUILD, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    subprocess.check_call([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp] + objs + LIBS)
    os.replace(tmp, LIB)
    print("built", LIB)
    return LIB


if __name__ == "__main__":
    try:
        build()
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
