"""In-tree build of the gfx950 library and its torch extension.

* ``lib/libpa_mi355x.so`` -- the HIP kernels plus the C ABI of
  ``include/pa_mi355x.h`` (hipcc, ``--offload-arch=gfx950``).
* ``lib/paged_attn_opt.so`` -- the thin torch extension (g++ against
  torch's headers), linked to the library above with an ``$ORIGIN`` rpath.
  The same object also initialises as ``paged_attn_naive``.
* ``lib/libpa_bench_probe.so`` -- streaming-rate probes the benchmark uses
  (``csrc/bench/``); not part of the decode path.

Object files go to ``_build/`` next to this package.  Every call rebuilds
from source; nothing is fetched.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sysconfig

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)                     # .../cuda-pa-int8_amd
REPO = os.path.dirname(ROOT)
CSRC = os.path.join(ROOT, "csrc")
INCLUDE = os.path.join(REPO, "include")
LIB_DIR = os.path.join(PKG_DIR, "lib")
OBJ_DIR = os.path.join(ROOT, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

LIB_NAME = "libpa_mi355x.so"
EXT_NAME = "paged_attn_opt.so"
PROBE_LIB_NAME = "libpa_bench_probe.so"

# head_dims of the decode kernels: pa_decode_inst.hip is compiled once per
# entry (keep in step with PA_FOR_EACH_HEAD_DIM in csrc/pa_internal.hpp).
HEAD_DIMS = tuple(range(8, 257, 8))
HIP_SOURCES = [
    "pa_quant.hip",
    "pa_cache_write.hip",
    "pa_fill.hip",
    "pa_noalloc.hip",
]
HOST_SOURCES = ["pa_capi.cpp"]
PROBE_SOURCES = ["bench/pa_probe.hip", "bench/pa_probe_decode.hip", "bench/pa_probe_write.hip"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # Keep the compiler from forming packed fp32 ops (v_pk_fma_f32 & co.).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Preload the first 14 kernel-argument dwords into SGPRs (the decode
    # kernels put what their prologue needs there); the compiler adds the
    # fallback that loads them itself under firmware that does not preload.
    "-mllvm", "-amdgpu-kernarg-preload-count=14",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def _hipcc():
    return os.path.join(ROCM, "bin", "hipcc")


def _compile_cmd(src, obj, defines=()):
    extra = ["-x", "hip"] if src.endswith(".hip") else []
    return [_hipcc(), *HIPCC_FLAGS, *defines, *extra, "-c", os.path.join(CSRC, src), "-o", obj]


def _link(objs, name, verbose, libs=()):
    out = os.path.join(LIB_DIR, name)
    tmp = out + ".tmp"
    _run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, *libs,
          f"-Wl,-rpath,{ROCM}/lib", f"-Wl,-soname,{name}"], verbose)
    os.replace(tmp, out)
    return out


def build_library(verbose=False, jobs=None):
    """Compile every HIP / host source of the library (and the probe library)
    in parallel, then link both."""
    os.makedirs(os.path.join(OBJ_DIR, "bench"), exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    jobs = jobs or max(1, min(8, int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    cmds, objs, probe_objs = [], [], []
    for d in HEAD_DIMS:
        obj = os.path.join(OBJ_DIR, f"pa_decode_d{d}.o")
        objs.append(obj)
        cmds.append(_compile_cmd("pa_decode_inst.hip", obj, [f"-DPA_HEAD_DIM={d}"]))
    for src in HIP_SOURCES + HOST_SOURCES:
        obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        cmds.append(_compile_cmd(src, obj))
    for src in PROBE_SOURCES:
        obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
        probe_objs.append(obj)
        cmds.append(_compile_cmd(src, obj))
    # the slowest units (the decode instantiations) first
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for f in [ex.submit(_run, c, verbose) for c in cmds]:
            f.result()
    out = _link(objs, LIB_NAME, verbose)
    _link(probe_objs, PROBE_LIB_NAME, verbose)
    return out


def build_extension(verbose=False):
    import torch
    from torch.utils import cpp_extension

    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    incs = cpp_extension.include_paths() + [sysconfig.get_paths()["include"], INCLUDE,
                                            os.path.join(ROCM, "include")]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cxx = shutil.which("g++") or "g++"
    out = os.path.join(LIB_DIR, EXT_NAME)
    tmp = out + ".tmp"
    cmd = [cxx, "-shared", "-fPIC", "-O2", "-std=c++17", "-w",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-DTORCH_EXTENSION_NAME=paged_attn_opt", "-DTORCH_API_INCLUDE_EXTENSION_H",
           *[f"-I{p}" for p in incs],
           os.path.join(CSRC, "paged_attn_opt.cpp"),
           f"-L{torch_lib}", f"-L{LIB_DIR}",
           "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip", "-ltorch_hip",
           "-lpa_mi355x",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}",
           "-o", tmp]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(verbose=False):
    """Compile the HIP library and the torch extension in-tree."""
    lib = build_library(verbose=verbose)
    ext = build_extension(verbose=verbose)
    return lib, ext


if __name__ == "__main__":
    for p in build(verbose=True):
        print("built", p)
