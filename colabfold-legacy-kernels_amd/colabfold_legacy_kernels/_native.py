"""ctypes binding of the C ABI declared in include/clk.h.

Loads the gfx950 library that ``library_path`` names and declares every entry point's argument
and return types. There is no fallback: if the library is missing, ``lib()`` raises
FileNotFoundError, and every op in ``colabfold_legacy_kernels.ops`` fails with it.
"""

import ctypes
import threading

from . import library_path

_lock = threading.Lock()
_lib = None

c_void_p = ctypes.c_void_p
c_i64 = ctypes.c_int64
c_f32 = ctypes.c_float
c_int = ctypes.c_int
c_size = ctypes.c_size_t

# name -> (restype, argtypes); the same order as the prototypes in include/clk.h.
PROTOTYPES = {
    "clk_last_error": (ctypes.c_char_p, []),
    "clk_version": (ctypes.c_char_p, []),
    "clk_profile_enable": (None, [c_int]),
    "clk_profile_collect": (c_int, [ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(c_f32),
                                    c_int]),
    "clk_attention_fwd": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                  c_void_p, c_void_p, c_void_p, c_i64, c_i64, c_i64, c_i64,
                                  c_i64, c_f32, c_i64, c_i64]),
    "clk_attention_fwd_nshd": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_void_p, c_void_p, c_i64, c_i64, c_i64, c_i64,
                                       c_i64, c_f32]),
    "clk_attention_fwd_gated": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p,
                                        c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                        c_void_p, c_void_p, c_void_p, c_i64, c_i64, c_i64,
                                        c_i64, c_i64, c_i64, c_f32]),
    "clk_attention_bwd_workspace_size": (c_size, [c_i64, c_i64, c_i64, c_i64, c_i64]),
    "clk_attention_bwd": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                  c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                  c_void_p, c_void_p, c_void_p, c_size, c_i64, c_i64, c_i64,
                                  c_i64, c_i64, c_f32]),
    "clk_attention_bwd_nshd": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_void_p, c_void_p, c_void_p, c_size, c_i64,
                                       c_i64, c_i64, c_i64, c_i64, c_f32]),
    "clk_attention_bwd_noalloc_limit": (c_size, []),
    "clk_attention_bwd_noalloc": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p,
                                          c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                          c_void_p, c_void_p, c_void_p, c_void_p, c_i64, c_i64,
                                          c_i64, c_i64, c_i64, c_f32]),
    "clk_stream_copy": (c_int, [c_void_p, c_void_p, c_void_p, c_size]),
    "clk_issue_calibration": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p]),
    "clk_layer_norm_fwd": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                   c_i64, c_i64, c_f32]),
    "clk_layer_norm_bwd_workspace_size": (c_size, [c_i64, c_i64]),
    "clk_layer_norm_bwd": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                   c_void_p, c_void_p, c_void_p, c_size, c_i64, c_i64, c_f32]),
    "clk_gated_dual_proj": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                    c_void_p, c_void_p, c_void_p, c_i64, c_i64, c_i64]),
    "clk_gated_dual_proj_bwd_workspace_size": (c_size, [c_i64, c_i64, c_i64]),
    "clk_gated_dual_proj_bwd": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                        c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                        c_void_p, c_void_p, c_void_p, c_void_p, c_size, c_i64,
                                        c_i64, c_i64, c_int]),
    "clk_ln_gated_dual_proj": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_i64,
                                       c_i64, c_i64, c_f32]),
    "clk_ln_pair_bias": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                 c_void_p, c_i64, c_i64, c_i64, c_f32]),
    "clk_attention_gate": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                   c_void_p, c_i64, c_i64, c_i64, c_i64, c_i64]),
    "clk_attention_gate_bwd_workspace_size": (c_size, [c_i64, c_i64, c_i64, c_i64, c_i64]),
    "clk_attention_gate_bwd": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_size, c_i64, c_i64, c_i64, c_i64, c_i64,
                                       c_int]),
    "clk_triangle_einsum": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_i64,
                                    c_i64]),
    "clk_triangle_multiply_workspace_size": (c_size, [c_i64, c_i64]),
    "clk_triangle_multiply": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_void_p, c_void_p, c_size, c_i64, c_i64, c_int,
                                      c_f32]),
}

# Status codes (clk_status) and dtype codes (clk_dtype).
OK, INVALID_ARGUMENT, UNIMPLEMENTED, INTERNAL = 0, 3, 12, 13
U8, F16, F32, BF16 = 6, 10, 11, 16


def load(path=None):
    """Load the library at ``path`` (default: the packaged gfx950 library) and declare types."""
    lib = ctypes.CDLL(path or library_path("attention", "gfx950"))
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def lib():
    """The process-wide handle of the packaged library."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                _lib = load()
    return _lib


def last_error():
    return lib().clk_last_error().decode()


class profile:
    """Context manager: record per-launch HIP event times of every kernel the library launches
    from this thread; ``records`` holds (kernel name, milliseconds) after exit."""

    def __init__(self):
        self.records = []

    def __enter__(self):
        lib().clk_profile_enable(1)
        return self

    def __exit__(self, *exc):
        lib().clk_profile_enable(0)
        self.records = collect()
        return False


def collect(max_records=65536):
    """Wait for and return the (name, ms) records taken so far on this thread, clearing them."""
    names = (ctypes.c_char_p * max_records)()
    ms = (c_f32 * max_records)()
    n = lib().clk_profile_collect(names, ms, max_records)
    return [(names[i].decode(), float(ms[i])) for i in range(min(n, max_records))]
