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

import torch  # noqa: F401  (must precede the library load, see above)

from . import _build

LIB_PATH = os.path.join(_build.LIB_DIR, _build.LIB_NAME)
EXT_PATH = os.path.join(_build.LIB_DIR, _build.EXT_NAME)

_BUILD_HINT = ("build it with `python -c 'import __graft_entry__ as g; g.build()'` "
               "from the repository root")


def _require(path):
    if not os.path.exists(path):
        raise ImportError(f"{os.path.basename(path)} is not built ({path}); {_BUILD_HINT}")


@functools.lru_cache(maxsize=1)
def ext():
    """The ``paged_attn_opt`` torch extension module."""
    _require(LIB_PATH)
    _require(EXT_PATH)
    loader = importlib.machinery.ExtensionFileLoader("paged_attn_opt", EXT_PATH)
    spec = importlib.util.spec_from_file_location("paged_attn_opt", EXT_PATH, loader=loader)
    mod = importlib.util.module_from_spec(spec)
    loader.exec_module(mod)
    return mod


# C-ABI prototypes of include/pa_mi355x.h used from Python (tests, bench).
_i32, _i64, _f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_float
_p, _sz = ctypes.c_void_p, ctypes.c_size_t

_DECODE_F16_ARGS = [_p, _p, _p, _p, _p, _p, _f32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                    _i32, _i32, _i32, _p, _sz, _p]
_DECODE_I8_ARGS = [_p, _p, _p, _p, _p, _p, _p, _p, _f32, _i32, _i32, _i32, _i32, _i32, _i32,
                   _i32, _i32, _i32, _i32, _p, _sz, _p]

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
    "pa_decode_set_waves_per_group": (ctypes.c_int, [_i32]),
    "pa_decode_set_schedule": (ctypes.c_int, [_i32]),
    "pa_decode_set_load_policy": (ctypes.c_int, [_i32]),
    "pa_paged_decode_attn_warp": (ctypes.c_int, _DECODE_F16_ARGS),
    "pa_paged_decode_attn_splitk": (ctypes.c_int, _DECODE_F16_ARGS),
    "pa_paged_decode_attn_warp_int8": (ctypes.c_int, _DECODE_I8_ARGS),
    "pa_paged_decode_attn_splitk_int8": (ctypes.c_int, _DECODE_I8_ARGS),
    "pa_reshape_and_cache_int8": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _i64, _p, _i32, _i32,
                                                 _i32, _p, _p, _p, _p, _i32, _i32, _i32, _p]),
    "pa_reshape_and_cache_int8_static": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _i64, _p,
                                                        _i32, _i32, _i32, _p, _p, _p, _p, _p,
                                                        _p, _i32, _i32, _i32, _p]),
    "pa_reshape_and_cache_f16": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _i64, _p, _i32, _i32,
                                                _i32, _p, _p, _i32, _i32, _i32, _p]),
    "pa_probe_read_contiguous": (ctypes.c_int, [_p, _sz, _p, _i32, _p]),
    "pa_probe_read_chunks": (ctypes.c_int, [_p, _sz, _p, _i32, _i32, _p, _i32, _p]),
    "pa_probe_read_write": (ctypes.c_int, [_p, _sz, _p, _i32, _p]),
}


@functools.lru_cache(maxsize=1)
def capi():
    """ctypes handle on libpa_mi355x.so with every exported prototype set."""
    _require(LIB_PATH)
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib
