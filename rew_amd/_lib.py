"""ctypes binding of librew_mi355x.so (declared in include/rew_mi355x.h).

The library is found the way rew's resolvePluginPath finds a plugin
(src/rew/binaries/resolver.nim:22-78) and loading fails loudly when it is
missing: there is no fallback execution path.  The library is one
self-contained file (the run-time kernel compiler's headers are built in).
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_NAME = "librew_mi355x.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME  # the in-tree build


class ResolveError(RuntimeError):
    """No librew_mi355x.so where the resolution order looks."""


def resolve_plugin_path() -> Path:
    """resolvePluginPath for the mi355x target (resolver.nim:22-78):

    1. REW_PJRT_PLUGIN_PATH, a list of directories separated by ':' -- the
       first one holding librew_mi355x.so wins;
    2. REW_BUILD=1 / true -- the in-tree build, which must exist;
    3. the library next to this package (the in-tree build, or an
       installed copy).

    There is no step 4 (download and extract): the library is built from
    this repository."""
    explicit = os.environ.get("REW_PJRT_PLUGIN_PATH", "")
    for d in explicit.split(os.pathsep):
        d = d.strip()
        if d and (Path(d) / LIB_NAME).is_file():
            return Path(d) / LIB_NAME
    if os.environ.get("REW_BUILD", "") in ("1", "true"):
        if LIB_PATH.is_file():
            return LIB_PATH
        raise ResolveError(f"REW_BUILD=true but no built library at {LIB_PATH}: "
                           "build it with `python -m rew_amd.build`")
    if LIB_PATH.is_file():
        return LIB_PATH
    raise ResolveError(
        f"{LIB_NAME} not found in REW_PJRT_PLUGIN_PATH ({explicit or 'unset'}) nor at "
        f"{LIB_PATH}: build it with `python -m rew_amd.build` (there is no CPU fallback "
        "for the mi355x backend)")

# Every symbol include/rew_mi355x.h declares, with (restype, argtypes).
_c_buf = C.c_void_p
_c_ctx = C.c_void_p
SIGNATURES = {
    "rew_mi355x_abi_version": (C.c_int, []),
    "rew_mi355x_last_error": (C.c_char_p, []),
    "rew_mi355x_device_count": (C.c_int, [C.POINTER(C.c_int)]),
    "rew_mi355x_init": (C.c_int, [C.c_int, C.POINTER(_c_ctx)]),
    "rew_mi355x_shutdown": (C.c_int, [_c_ctx]),
    "rew_mi355x_from_host": (C.c_int, [_c_ctx, C.c_int, C.POINTER(C.c_int64), C.c_int,
                                       C.c_void_p, C.c_int64, C.POINTER(_c_buf)]),
    "rew_mi355x_to_host": (C.c_int, [_c_buf, C.c_void_p, C.c_int64]),
    "rew_mi355x_buf_meta": (C.c_int, [_c_buf, C.POINTER(C.c_int), C.POINTER(C.c_int),
                                      C.POINTER(C.c_int64)]),
    "rew_mi355x_alloc": (C.c_int, [_c_ctx, C.c_int, C.POINTER(C.c_int64), C.c_int,
                                   C.POINTER(_c_buf)]),
    "rew_mi355x_buf_device_ptr": (C.c_int, [_c_buf, C.POINTER(C.c_void_p)]),
    "rew_mi355x_retain": (C.c_int, [_c_buf]),
    "rew_mi355x_release": (None, [_c_buf]),
    "rew_mi355x_execute": (C.c_int, [_c_ctx, C.c_char_p, C.POINTER(_c_buf), C.c_int,
                                     C.POINTER(C.c_char_p), C.POINTER(C.c_char_p), C.c_int,
                                     C.POINTER(_c_buf), C.c_int, C.POINTER(C.c_int)]),
    "rew_mi355x_execute_ex": (C.c_int, [_c_ctx, C.c_char_p, C.POINTER(_c_buf), C.c_int,
                                        C.POINTER(C.c_char_p), C.POINTER(C.c_char_p), C.c_int,
                                        C.POINTER(_c_buf), C.c_int, C.POINTER(C.c_int),
                                        C.POINTER(C.c_int64)]),
    "rew_mi355x_execute_jit": (C.c_int, [_c_ctx, C.c_char_p, C.c_char_p, C.c_char_p, C.c_int64,
                                         C.POINTER(_c_buf), C.c_int, C.POINTER(C.c_int),
                                         C.c_int, C.POINTER(_c_buf), C.c_int,
                                         C.POINTER(C.c_int), C.POINTER(C.c_int64)]),
    "rew_mi355x_clear_jit_cache": (C.c_int, [_c_ctx]),
    "rew_mi355x_flush": (C.c_int, [_c_ctx]),
    "rew_mi355x_sync": (C.c_int, [_c_ctx]),
    "rew_mi355x_set_mode": (C.c_int, [_c_ctx, C.c_int]),
    "rew_mi355x_clear_cache": (C.c_int, [_c_ctx]),
    "rew_mi355x_get_stats": (C.c_int, [_c_ctx, C.c_void_p]),
    "rew_mi355x_reset_stats": (C.c_int, [_c_ctx]),
    "rew_mi355x_profile_begin": (C.c_int, [_c_ctx]),
    "rew_mi355x_profile_end": (C.c_int, [_c_ctx]),
    "rew_mi355x_profile_entry": (C.c_int, [_c_ctx, C.c_int, C.c_char_p, C.c_int,
                                           C.POINTER(C.c_int64), C.POINTER(C.c_double)]),
    "rew_mi355x_stream": (C.c_int, [_c_ctx, C.POINTER(C.c_void_p)]),
    "rew_mi355x_moe_routed_ffn": (C.c_int, [_c_ctx, C.c_void_p]),
    "rew_mi355x_moe_routed_ffn_noalloc": (C.c_int, [_c_ctx, C.c_void_p]),
    "rew_mi355x_rng_split": (None, [C.c_uint32, C.c_uint32, C.c_int, C.POINTER(C.c_uint32)]),
    "rew_mi355x_rng_fold_in": (None, [C.c_uint32, C.c_uint32, C.c_uint64,
                                      C.POINTER(C.c_uint32)]),
    "rew_mi355x_rng_uniform_f32": (None, [C.c_uint32, C.c_uint32, C.c_int64, C.c_float,
                                          C.c_float, C.c_void_p]),
    "rew_mi355x_rng_normal_f32": (None, [C.c_uint32, C.c_uint32, C.c_int64, C.c_float,
                                         C.c_float, C.c_void_p]),
}


class MoeArgs(C.Structure):
    """rew_mi355x_moe_args (include/rew_mi355x.h)."""
    _fields_ = [("x", C.c_void_p), ("x_row_stride", C.c_int64),
                ("start", C.c_void_p), ("start_row_stride", C.c_int64),
                ("top_ids", C.c_void_p), ("top_weights", C.c_void_p),
                ("tokens", C.c_int64), ("hidden", C.c_int64), ("ffn", C.c_int64),
                ("k", C.c_int), ("router_width", C.c_int), ("n_experts", C.c_int),
                ("expert_ids", C.c_void_p),
                ("gate_w", C.c_void_p), ("up_w", C.c_void_p), ("gate_b", C.c_void_p),
                ("up_b", C.c_void_p), ("down_w", C.c_void_p), ("down_b", C.c_void_p),
                ("out", C.c_void_p)]


class Stats(C.Structure):
    _fields_ = [(n, C.c_int64) for n in (
        "ops_recorded", "kernels_launched", "flushes", "fused_groups",
        "bytes_in_use", "bytes_cached", "plan_cache_hits", "jit_module_compiles",
        "jit_module_hits", "programs_compiled", "programs_loaded", "flush_plan_hits",
        "flush_host_ns")]


_lib = None
loaded_path: Path | None = None


def load() -> C.CDLL:
    """Returns the loaded library, raising if it has not been built."""
    global _lib, loaded_path
    if _lib is not None:
        return _lib
    path = resolve_plugin_path()
    lib = C.CDLL(str(path))
    loaded_path = path
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
