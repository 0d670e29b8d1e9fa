"""Build the gfx950 shared library in-tree: checkers_amd/libcheckers_amd.so.

Run as `python -m checkers_amd.build` (or through __graft_entry__.build()).
hipcc cross-compiles for gfx950 without a GPU present.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libcheckers_amd.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["ckr_kernels.hip", "ckr_repair.hip", "ckr_api.cpp", "ckr_checkpoint.cpp"]

# -packed-fp32-ops: no v_pk_*_f32 generated anywhere (wrong results seen with
# some of their forms on these machines).
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


CLI = os.path.join(HERE, "ckr_prefix_mask_repair")


def build(verbose=True):
    cmd = [HIPCC] + FLAGS + ["-x", "hip"] + [os.path.join(CSRC, s) for s in SOURCES] + ["-o", LIB + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(LIB + ".tmp", LIB)
    # the prefix-mask-repair command line: host code over the C ABI
    cli = [HIPCC, "-O2", "-std=c++17", "-Wall", "-I", os.path.join(ROOT, "include"),
           os.path.join(CSRC, "ckr_repair_cli.cpp"), "-o", CLI + ".tmp",
           "-L", HERE, "-lcheckers_amd", "-Wl,-rpath,$ORIGIN"]
    if verbose:
        print(" ".join(cli), flush=True)
    subprocess.run(cli, check=True)
    os.replace(CLI + ".tmp", CLI)
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
