"""Build libqwn_hip.so (gfx950) in-tree with hipcc.

The library is also written as ``qwn_cuda.so`` beside it, the file name the
qwnrun loader opens from its executable's directory
(c/qwanto_decode.c:289-301).
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
OBJDIR = os.path.join(PKG, "_build")
LIB = os.path.join(LIBDIR, "libqwn_hip.so")
LOADER_NAME = os.path.join(LIBDIR, "qwn_cuda.so")
SOURCES = ["qwn_runtime.hip", "qwn_gemv.hip", "qwn_attention.hip", "qwn_decoder.hip", "qwn_noalloc.hip",
           "qwn_head.hip"]
ARCH = os.environ.get("QWN_HIP_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-fvisibility=hidden", "-Wall", "-Wno-unused-result",
    # never emit packed fp32 arithmetic (v_pk_*_f32) on gfx950
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed for {src}")
    # the host pass does not know the gfx feature name; drop that one note
    noise = "is not a recognized feature for this target"
    for line in (res.stdout + res.stderr).splitlines():
        if line.strip() and noise not in line:
            sys.stderr.write(line + "\n")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    shutil.copyfile(LIB, LOADER_NAME + ".tmp")
    os.replace(LOADER_NAME + ".tmp", LOADER_NAME)
    build_host_decoder()
    if verbose:
        print(f"built {LIB}")
    return LIB


HOST_DECODER = os.path.join(LIBDIR, "libqwn_host_decoder.so")


SANITIZE_FLAGS = ("-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
                  "-fno-sanitize-recover=all")


def build_host_decoder(out: str = HOST_DECODER, sanitize: bool = False) -> str:
    """The host-side decoder (plain C, above the ABI): gcc, no contraction so
    its explicit fused multiply-adds are the only ones.  ``sanitize`` builds
    it with AddressSanitizer and UndefinedBehaviorSanitizer into ``out``."""
    tmp = out + ".tmp"
    cmd = [os.environ.get("CC", "gcc"), "-O2", "-std=gnu11", "-fPIC", "-shared", "-ffp-contract=off",
           "-Wall", "-Wextra", *(SANITIZE_FLAGS if sanitize else ()), "-I" + os.path.join(ROOT, "include"),
           os.path.join(PKG, "host", "qwn_host_decoder.c"), "-o", tmp, "-ldl", "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    build()
