"""Loads the in-tree gfx950 library and its torch extension.

``torch`` is imported first so that its HIP runtime (``libamdhip64.so.7``,
bundled in torch/lib) is the one the library binds to: the library's
``NEEDED`` entry resolves by soname to the copy already in the process, and
one HIP runtime serves both.

There is no fallback: when the built files are missing the import fails
with an error that names the build command.
"""

from __future__ import annotations

import ctypes
import functools
import importlib.machinery
import importlib.util
import os
import sys

import torch  # noqa: F401  (must precede the library load, see above)

from . import _build

LIB_PATH = os.path.join(_build.LIB_DIR, _build.LIB_NAME)
EXT_PATH = os.path.join(_build.LIB_DIR, _build.EXT_NAME)
PROBE_LIB_PATH = os.path.join(_build.LIB_DIR, _build.PROBE_LIB_NAME)

_BUILD_HINT = ("build it with `python -c 'import __graft_entry__ as g; g.build()'` "
               "from the repository root")


def _require(path):
    if not os.path.exists(path):
        raise ImportError(f"{os.path.basename(path)} is not built ({path}); {_BUILD_HINT}")


def _load_ext(name):
    _require(LIB_PATH)
    _require(EXT_PATH)
    loader = importlib.machinery.ExtensionFileLoader(name, EXT_PATH)
    spec = importlib.util.spec_from_file_location(name, EXT_PATH, loader=loader)
    mod = importlib.util.module_from_spec(spec)
    loader.exec_module(mod)
    # importable by name afterwards, as the reference's JIT-built modules are
    sys.modules.setdefault(name, mod)
    return mod


@functools.lru_cache(maxsize=1)
def ext():
    """The ``paged_attn_opt`` torch extension module (the reference's module
    name and ops, kernels/bindings.cpp:45-58)."""
    return _load_ext("paged_attn_opt")


@functools.lru_cache(maxsize=1)
def naive_ext():
    """The ``paged_attn_naive`` module: the naive stage's op under its own
    module name (kernels/paged_attention_naive.cu:169-172), from the same
    shared object."""
    return _load_ext("paged_attn_naive")


# C-ABI prototypes of include/pa_mi355x.h used from Python (tests, bench).
_i32, _i64, _f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_float
_p, _sz = ctypes.c_void_p, ctypes.c_size_t

# decode: out, q, k, v, [k_scales, v_scales,] block_table, context_lens, scale, block_size,
# S, H, D, Hkv, NB, x, max_blocks, max_context_len, partition, counters, counter_bytes,
# workspace, workspace_bytes, stream
_DECODE_TAIL = [_f32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p, _sz, _p,
                _sz, _p]
_DECODE_F16_ARGS = [_p] * 6 + _DECODE_TAIL
_DECODE_I8_ARGS = [_p] * 8 + _DECODE_TAIL

PROTOTYPES = {
    "pa_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "pa_version": (ctypes.c_char_p, []),
    "pa_validate_decode": (ctypes.c_int, [ctypes.c_int, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                          _i32]),
    "pa_check_context_lens": (ctypes.c_int, [_p, _i32, ctypes.POINTER(_i32)]),
    "pa_decode_plan": (ctypes.c_int, [ctypes.c_int, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                      _i32, ctypes.POINTER(_i32), ctypes.POINTER(_i32)]),
    "pa_decode_workspace_bytes": (_sz, [ctypes.c_int, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                        _i32]),
    "pa_decode_counter_bytes": (_sz, [_i32, _i32, _i32]),
    "pa_decode_counters_reset": (ctypes.c_int, [_p, _sz, _p]),
    "pa_decode_set_waves_per_group": (ctypes.c_int, [_i32]),
    "pa_decode_set_schedule": (ctypes.c_int, [_i32]),
    "pa_decode_set_load_policy": (ctypes.c_int, [_i32]),
    "pa_decode_set_max_head_tile": (ctypes.c_int, [_i32]),
    "pa_decode_plan_detail": (ctypes.c_int, [ctypes.c_int, _i32, _i32, _i32, _i32, _i32, _i32,
                                             _i32, _i32, _p, _i32]),
    "pa_paged_decode_attn_warp": (ctypes.c_int, _DECODE_F16_ARGS),
    "pa_paged_decode_attn_splitk": (ctypes.c_int, _DECODE_F16_ARGS),
    "pa_paged_decode_attn_warp_int8": (ctypes.c_int, _DECODE_I8_ARGS),
    "pa_paged_decode_attn_splitk_int8": (ctypes.c_int, _DECODE_I8_ARGS),
    "pa_paged_decode_attn_noalloc": (ctypes.c_int, [ctypes.c_int] + [_p] * 8 + _DECODE_TAIL[:11]
                                     + [_p]),
    "pa_reshape_and_cache_int8": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _i64, _p, _i32, _i32,
                                                 _i32, _p, _p, _p, _p, _i32, _i32, _i32, _p]),
    "pa_reshape_and_cache_int8_static": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _i64, _p,
                                                        _i32, _i32, _i32, _p, _p, _p, _p, _p,
                                                        _p, _i32, _i32, _i32, _p]),
    "pa_reshape_and_cache_int8_bf16": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _i64, _p, _i32,
                                                      _i32, _i32, _p, _p, _p, _p, _i32, _i32, _i32,
                                                      _p]),
    "pa_reshape_and_cache_int8_static_bf16": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _i64, _p,
                                                             _i32, _i32, _i32, _p, _p, _p, _p, _p,
                                                             _p, _i32, _i32, _i32, _p]),
    "pa_reshape_and_cache_f16": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _i64, _p, _i32, _i32,
                                                _i32, _p, _p, _i32, _i32, _i32, _p]),
}

# libpa_bench_probe.so (csrc/bench/pa_probe.h): measurement probes of the benchmark.
PROBE_PROTOTYPES = {
    "pa_probe_read_contiguous": (ctypes.c_int, [_p, _sz, _p, _i32, _p]),
    "pa_probe_read_chunks": (ctypes.c_int, [_p, _sz, _p, _i32, _i32, _p, _i32, _p]),
    "pa_probe_read_write": (ctypes.c_int, [_p, _sz, _p, _i32, _p]),
    "pa_probe_decode_stream": (ctypes.c_int, [_i32, _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _i32,
                                              _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p, _p]),
    "pa_probe_quant_write": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _i64, _p, _i32, _i32, _p, _p,
                                            _p, _p, _i32, _i32, _p]),
}


def _cdll(path, prototypes):
    _require(path)
    lib = ctypes.CDLL(path)
    for name, (res, args) in prototypes.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


@functools.lru_cache(maxsize=1)
def capi():
    """ctypes handle on libpa_mi355x.so with every exported prototype set
    (include/pa_mi355x.h and the test hooks of include/pa_mi355x_tuning.h)."""
    return _cdll(LIB_PATH, PROTOTYPES)


@functools.lru_cache(maxsize=1)
def probe_capi():
    """ctypes handle on the benchmark's probe library (not the decode path)."""
    return _cdll(PROBE_LIB_PATH, PROBE_PROTOTYPES)
