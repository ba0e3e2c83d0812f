"""Build libshadowinfer_hip.so for gfx950 with hipcc.

Usage: ``python shadow-infer_amd/build.py`` (also called by
``__graft_entry__.build()``). Each ``csrc/*.hip`` file is compiled to an
object in parallel, then linked into
``shadowinfer_amd/_lib/libshadowinfer_hip.so`` next to the Python package, so
the library travels with the source tree. The small host extension
``_hostmask`` (csrc/host_masks.c) is built next to it with the system C
compiler.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "shadowinfer_amd", "_lib")
OBJ_DIR = os.path.join(HERE, "_build")
LIB_NAME = "libshadowinfer_hip.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("SI_OFFLOAD_ARCH", "gfx950")

CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    # Every expression rounds as written: no implicit multiply-add fusion, and
    # fp32 division / sqrt are correctly rounded (bit-exact quantization).
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # Packed-fp32 instructions are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mcode-object-version=5",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build_host_ext(verbose: bool = False) -> str:
    """The CPython extension ``_hostmask`` (csrc/host_masks.c): the reference's
    set / dict token-head arguments as dense masks. Plain host C, built with
    the system compiler against this interpreter's headers."""
    inc = sysconfig.get_paths()["include"]
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = os.path.join(OUT_DIR, "_hostmask" + suffix)
    tmp = out + ".tmp%d" % os.getpid()
    cmd = [os.environ.get("CC", "gcc"), "-O2", "-shared", "-fPIC", "-Wall", f"-I{inc}",
           os.path.join(CSRC, "host_masks.c"), "-o", tmp, "-lm"]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError("host extension build failed:\n" + proc.stdout)
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    lines = [ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln]
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n" + "\n".join(lines))
    if lines:
        sys.stderr.write("\n".join(lines) + "\n")
    return obj


def build(verbose: bool = False) -> str:
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), max(1, min(os.cpu_count() or 1, 8)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(_compile, srcs))
    lib = os.path.join(OUT_DIR, LIB_NAME)
    tmp = lib + ".tmp%d" % os.getpid()
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError("hipcc link failed:\n" + proc.stdout)
    os.replace(tmp, lib)
    shutil.rmtree(OBJ_DIR, ignore_errors=True)
    if verbose:
        print(f"built {lib}")
    build_host_ext(verbose)
    return lib


if __name__ == "__main__":
    build(verbose=True)
