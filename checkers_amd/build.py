"""Build the gfx950 shared library in-tree: checkers_amd/libcheckers_amd.so.

Run as `python -m checkers_amd.build` (or through __graft_entry__.build()).
hipcc cross-compiles for gfx950 without a GPU present.  Each source is
compiled to its own object in parallel, then the objects are linked.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libcheckers_amd.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["ckr_kernels.hip", "ckr_repair.hip", "ckr_api.cpp", "ckr_checkpoint.cpp", "ckr_context.hip",
           "ckr_container.hip", "ckr_analyzer.hip"]

# -packed-fp32-ops: no v_pk_*_f32 generated anywhere (wrong results seen with
# some of their forms on these machines).
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


CLI = os.path.join(HERE, "ckr_prefix_mask_repair")

# HBM probes for bench.py's ceiling figures, a library of their own
PROBE_SRC = os.path.join(CSRC, "ckr_probe.hip")
PROBE_LIB = os.path.join(HERE, "libckr_probe.so")

# the pybind11 module `checkers_py` (the reference's module name), at the
# repository root so that `import checkers_py` finds it; host code only, not
# linked to the library or the HIP runtime (it loads checkers_amd/ at run time)
PY_SOURCES = ["checkers_api.cpp", "python_bindings.cpp"]


def py_module_path():
    import sysconfig
    return os.path.join(ROOT, "checkers_py" + sysconfig.get_config_var("EXT_SUFFIX"))


def _py_module_cmd():
    import sysconfig
    import pybind11
    return (["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-fvisibility=hidden", "-Wall",
             "-D__HIP_PLATFORM_AMD__", "-I", "/opt/rocm/include", "-I", os.path.join(ROOT, "include"),
             "-I", pybind11.get_include(), "-I", sysconfig.get_paths()["include"]]
            + [os.path.join(CSRC, s) for s in PY_SOURCES]
            + ["-o", py_module_path() + ".tmp", "-ldl"])


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature: harmless, not shown
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if out.strip():
        print(out, flush=True)
    if r.returncode:
        raise subprocess.CalledProcessError(r.returncode, cmd)


def _stale(src, obj):
    """An object older than its source or a shared header."""
    if not os.path.exists(obj):
        return True
    deps = [src, os.path.join(ROOT, "include", "checkers_amd.h"), os.path.join(CSRC, "ckr_internal.h"),
            os.path.join(CSRC, "ckr_table.h"),
            os.path.join(CSRC, "ckr_container.h")]
    return any(os.path.getmtime(d) > os.path.getmtime(obj) for d in deps)


def build(verbose=True, incremental=False):
    """Compile every source (incremental: only those whose object is stale) and link."""
    os.makedirs(OBJ, exist_ok=True)
    objs = [os.path.join(OBJ, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    cmds = [[HIPCC] + FLAGS + ["-x", "hip", "-c", os.path.join(CSRC, s), "-o", o] for s, o in zip(SOURCES, objs)
            if not incremental or _stale(os.path.join(CSRC, s), o)]
    with ThreadPoolExecutor(max(len(cmds), 1)) as ex:
        for f in [ex.submit(_run, c, verbose) for c in cmds]:
            f.result()
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC"] + objs + ["-o", LIB + ".tmp"], verbose)
    os.replace(LIB + ".tmp", LIB)
    # the prefix-mask-repair command line: host code over the C ABI
    _run([HIPCC, "-O2", "-std=c++17", "-Wall", "-I", os.path.join(ROOT, "include"),
          os.path.join(CSRC, "ckr_repair_cli.cpp"), "-o", CLI + ".tmp",
          "-L", HERE, "-lcheckers_amd", "-Wl,-rpath,$ORIGIN"], verbose)
    os.replace(CLI + ".tmp", CLI)
    if not incremental or not os.path.exists(PROBE_LIB) or os.path.getmtime(PROBE_SRC) > os.path.getmtime(PROBE_LIB):
        _run([HIPCC] + FLAGS + ["-shared", "-x", "hip", PROBE_SRC, "-o", PROBE_LIB + ".tmp"], verbose)
        os.replace(PROBE_LIB + ".tmp", PROBE_LIB)
    mod = py_module_path()
    if not incremental or any(not os.path.exists(mod) or os.path.getmtime(d) > os.path.getmtime(mod)
                              for d in [LIB, os.path.join(ROOT, "include", "checkers_api.hpp")]
                              + [os.path.join(CSRC, s) for s in PY_SOURCES]):
        _run(_py_module_cmd(), verbose)
        os.replace(mod + ".tmp", mod)
    return LIB


if __name__ == "__main__":
    build(incremental="--incremental" in sys.argv)
    sys.exit(0)
