"""Build of the gfx950 C-ABI library scope_amd/lib/libwsgpu.so.

Compiles every scope_amd/csrc/*.hip with hipcc for gfx950 only and links one
shared library that exports the entry points declared in include/wsgpu.h.
Runs on a machine without a GPU (hipcc cross-compiles).
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
OBJDIR = os.path.join(HERE, "_obj")
LIB = os.path.join(LIBDIR, "libwsgpu.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed-fp32 VALU forms are disabled for all device code; the host pass warns
# that it does not know the feature, which is harmless.
DEVICE_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def sources() -> list[str]:
    return sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip")
    )


def _compile(src: str) -> str:
    obj = os.path.join(OBJDIR, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *DEVICE_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile all HIP sources and link libwsgpu.so; returns its path."""
    os.makedirs(LIBDIR, exist_ok=True)
    os.makedirs(OBJDIR, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


# ---------------------------------------------------------------------------
# Host partial: scope_amd/lib/libwshost.so (g++, OpenMP).  The kernels file is
# built for AVX-512 BF16; the ABI file for the baseline ISA, so a CPU without
# the kernels' instructions gets WH_ENOTSUP instead of an illegal instruction.

HOST_LIB = os.path.join(LIBDIR, "libwshost.so")
CXX = os.environ.get("CXX", "g++")
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-fopenmp", "-Wall", "-Wextra", "-fno-math-errno"]
HOST_SOURCES = {
    "wh_attn.cpp": [],
    "wh_kernels.cpp": ["-mavx512f", "-mavx512bw", "-mavx512vl", "-mavx512dq", "-mavx512bf16",
                       "-mfma"],
}


def build_host(verbose: bool = False) -> str:
    """Compile the host partial and link libwshost.so; returns its path."""
    os.makedirs(LIBDIR, exist_ok=True)
    os.makedirs(OBJDIR, exist_ok=True)

    def one(item):
        name, extra = item
        obj = os.path.join(OBJDIR, name[:-4] + ".host.o")
        cmd = [CXX, *HOST_FLAGS, *extra, "-c", os.path.join(CSRC, name), "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"{CXX} failed for {name}:\n{r.stdout}\n{r.stderr}")
        return obj

    with ThreadPoolExecutor(max_workers=len(HOST_SOURCES)) as ex:
        objs = list(ex.map(one, HOST_SOURCES.items()))
    tmp = HOST_LIB + ".tmp"
    r = subprocess.run([CXX, "-shared", "-fopenmp", *objs, "-o", tmp], capture_output=True,
                       text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, HOST_LIB)
    if verbose:
        print(f"built {HOST_LIB}", file=sys.stderr)
    return HOST_LIB


# ---------------------------------------------------------------------------
# Layer driver: scope_amd/lib/libwslayer.so, host code (hipcc, no kernels) over
# the two libraries above, found next to it at run time.

LAYER_LIB = os.path.join(LIBDIR, "libwslayer.so")


def build_layer(verbose: bool = False) -> str:
    """Compile the two-sided layer driver and link libwslayer.so against
    libwsgpu.so and libwshost.so (build those first); returns its path."""
    os.makedirs(OBJDIR, exist_ok=True)
    obj = os.path.join(OBJDIR, "wl_layer.o")
    cmd = [HIPCC, "-O3", "-std=c++17", "-fPIC", "-Wall", "-c",
           os.path.join(CSRC, "wl_layer.cpp"), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for wl_layer.cpp:\n{r.stdout}\n{r.stderr}")
    tmp = LAYER_LIB + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", obj, "-L", LIBDIR, "-lwsgpu", "-lwshost",
           "-Wl,-rpath,$ORIGIN", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LAYER_LIB)
    if verbose:
        print(f"built {LAYER_LIB}", file=sys.stderr)
    return LAYER_LIB


if __name__ == "__main__":
    print(build(verbose=True))
    print(build_host(verbose=True))
    print(build_layer(verbose=True))
