"""ctypes binding of the C ABI declared in ``include/deltanet_amd.h``.

The shared library ``libdeltanet_amd.so`` is built in-tree by
``deltanet_tpu_amd._build.build()`` (hipcc, gfx950).  There is no fallback:
if the library is missing, every entry point raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libdeltanet_amd.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

DN_ABI_VERSION = 2
DN_F32, DN_BF16, DN_F16, DN_I32, DN_I64 = 0, 1, 2, 3, 4

_c_i32 = ctypes.c_int32
_c_ptr = ctypes.c_void_p


class PrefillArgs(ctypes.Structure):
    """Mirror of ``dn_prefill_args``."""

    _fields_ = [
        ("abi_version", _c_i32),
        ("B", _c_i32), ("L", _c_i32), ("Hk", _c_i32), ("Hv", _c_i32), ("K", _c_i32), ("V", _c_i32),
        ("t0", _c_i32), ("nt", _c_i32),
        ("q", _c_ptr), ("k", _c_ptr), ("v", _c_ptr),
        ("qk_dtype", _c_i32), ("v_dtype", _c_i32),
        ("g", _c_ptr), ("g_dtype", _c_i32), ("g_heads", _c_i32), ("g_chans", _c_i32),
        ("b", _c_ptr), ("b_dtype", _c_i32), ("b_heads", _c_i32), ("b_chans", _c_i32),
        ("w", _c_ptr), ("w_dtype", _c_i32), ("w_heads", _c_i32), ("w_chans", _c_i32),
        ("seg", _c_ptr), ("seg_dtype", _c_i32), ("seg_batched", _c_i32),
        ("init_state", _c_ptr),
        ("init_seg", _c_ptr),
        ("out", _c_ptr),
        ("final_state", _c_ptr),
        ("scale", ctypes.c_float),
        ("qk_l2norm", _c_i32), ("fuse_prologue", _c_i32), ("stability_guard", _c_i32),
        ("precision", _c_i32), ("gates_at_hv", _c_i32), ("block_tokens", _c_i32), ("recompute_states", _c_i32),
    ]


class DecodeArgs(ctypes.Structure):
    """Mirror of ``dn_decode_args``."""

    _fields_ = [
        ("abi_version", _c_i32),
        ("B", _c_i32), ("Hk", _c_i32), ("Hv", _c_i32), ("K", _c_i32), ("V", _c_i32),
        ("q", _c_ptr), ("k", _c_ptr), ("v", _c_ptr),
        ("qk_dtype", _c_i32), ("v_dtype", _c_i32),
        ("g", _c_ptr), ("g_dtype", _c_i32), ("g_heads", _c_i32), ("g_chans", _c_i32),
        ("b", _c_ptr), ("b_dtype", _c_i32), ("b_heads", _c_i32), ("b_chans", _c_i32),
        ("w", _c_ptr), ("w_dtype", _c_i32), ("w_heads", _c_i32), ("w_chans", _c_i32),
        ("state_in", _c_ptr), ("state_in_dtype", _c_i32),
        ("state_out", _c_ptr), ("state_out_dtype", _c_i32),
        ("reset", _c_ptr),
        ("out", _c_ptr),
        ("scale", ctypes.c_float),
        ("qk_l2norm", _c_i32),
        ("stability_guard", _c_i32),
        ("stability_tau", ctypes.c_float),
    ]


class BackwardArgs(ctypes.Structure):
    """Mirror of ``dn_backward_args``."""

    _fields_ = [
        ("abi_version", _c_i32),
        ("B", _c_i32), ("L", _c_i32), ("H", _c_i32), ("K", _c_i32), ("V", _c_i32),
        ("q", _c_ptr), ("k", _c_ptr), ("v", _c_ptr), ("g", _c_ptr), ("b", _c_ptr), ("w", _c_ptr),
        ("seg", _c_ptr),
        ("init_state", _c_ptr),
        ("d_out", _c_ptr),
        ("d_final", _c_ptr),
        ("dq", _c_ptr), ("dk", _c_ptr), ("dv", _c_ptr), ("dg", _c_ptr), ("db", _c_ptr), ("dw", _c_ptr),
        ("d_init", _c_ptr),
        ("recompute_states", _c_i32),
    ]


EXPORTED_SYMBOLS = (
    "dn_prefill_workspace_size",
    "dn_prefill_fwd",
    "dn_prefill_fwd_noalloc",
    "dn_decode_step",
    "dn_decode_steps",
    "dn_prefill_bwd_workspace_size",
    "dn_prefill_bwd",
    "dn_prefill_bwd_raw_workspace_size",
    "dn_prefill_bwd_raw",
    "dn_state_frob_cap",
    "dn_last_error",
    "dn_abi_version",
    "dn_profile_begin",
    "dn_profile_end",
)
PROFILE_KINDS = ("prepass", "value", "chain", "decode", "backward")

_lock = threading.Lock()
_lib = None


def load_library(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises RuntimeError if absent."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise RuntimeError(
                f"deltanet_tpu_amd: HIP library {p} is missing; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` (hipcc, gfx950).")
        lib = ctypes.CDLL(p)
        lib.dn_prefill_workspace_size.argtypes = [ctypes.POINTER(PrefillArgs)]
        lib.dn_prefill_workspace_size.restype = ctypes.c_size_t
        lib.dn_prefill_fwd.argtypes = [ctypes.POINTER(PrefillArgs), _c_ptr, ctypes.c_size_t, _c_ptr]
        lib.dn_prefill_fwd.restype = ctypes.c_int
        lib.dn_prefill_fwd_noalloc.argtypes = [ctypes.POINTER(PrefillArgs), _c_ptr]
        lib.dn_prefill_fwd_noalloc.restype = ctypes.c_int
        lib.dn_decode_step.argtypes = [ctypes.POINTER(DecodeArgs), _c_ptr]
        lib.dn_decode_step.restype = ctypes.c_int
        lib.dn_decode_steps.argtypes = [ctypes.POINTER(DecodeArgs), _c_i32, _c_ptr]
        lib.dn_decode_steps.restype = ctypes.c_int
        lib.dn_prefill_bwd_workspace_size.argtypes = [ctypes.POINTER(BackwardArgs)]
        lib.dn_prefill_bwd_workspace_size.restype = ctypes.c_size_t
        lib.dn_prefill_bwd.argtypes = [ctypes.POINTER(BackwardArgs), _c_ptr, ctypes.c_size_t, _c_ptr]
        lib.dn_prefill_bwd.restype = ctypes.c_int
        lib.dn_prefill_bwd_raw_workspace_size.argtypes = [ctypes.POINTER(PrefillArgs)]
        lib.dn_prefill_bwd_raw_workspace_size.restype = ctypes.c_size_t
        lib.dn_prefill_bwd_raw.argtypes = [ctypes.POINTER(PrefillArgs)] + [_c_ptr] * 9 + [_c_ptr, ctypes.c_size_t, _c_ptr]
        lib.dn_prefill_bwd_raw.restype = ctypes.c_int
        lib.dn_state_frob_cap.argtypes = [_c_ptr, ctypes.c_int64, _c_i32, _c_i32, ctypes.c_float, _c_ptr]
        lib.dn_state_frob_cap.restype = ctypes.c_int
        lib.dn_last_error.argtypes = []
        lib.dn_last_error.restype = ctypes.c_char_p
        lib.dn_abi_version.argtypes = []
        lib.dn_abi_version.restype = ctypes.c_int
        lib.dn_profile_begin.argtypes = []
        lib.dn_profile_begin.restype = ctypes.c_int
        lib.dn_profile_end.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64)]
        lib.dn_profile_end.restype = ctypes.c_int
        if lib.dn_abi_version() != DN_ABI_VERSION:
            raise RuntimeError("deltanet_tpu_amd: library ABI version mismatch; rebuild it")
        if path is None:
            _lib = lib
        return lib


def profile_begin() -> None:
    check(load_library().dn_profile_begin(), "dn_profile_begin")


def profile_end() -> dict:
    """Per kernel kind: (summed milliseconds, launches) since profile_begin()."""
    n = len(PROFILE_KINDS)
    ms = (ctypes.c_double * n)()
    cnt = (ctypes.c_int64 * n)()
    check(load_library().dn_profile_end(ms, cnt), "dn_profile_end")
    return {k: (ms[i], cnt[i]) for i, k in enumerate(PROFILE_KINDS)}


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load_library().dn_last_error().decode(errors="replace")
        raise RuntimeError(f"deltanet_tpu_amd: {what} failed (code {rc}): {msg}")
