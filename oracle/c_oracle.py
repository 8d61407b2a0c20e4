"""ctypes access to the C token-serial restatement (oracle/gdn_serial.c).

TEST INFRASTRUCTURE ONLY (tests/, smoke(), bench.py's cpu_baseline leg).
Build with `make -C oracle`; the library lands in oracle/_build/.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_build", "libdn_oracle.so")
_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} missing: run `make -C oracle`")
        _lib = ctypes.CDLL(LIB)
        for name in ("dn_oracle_serial_f64", "dn_oracle_serial_f32"):
            fn = getattr(_lib, name)
            fn.restype = ctypes.c_int
    return _lib


def _gate(x, B, L, dt):
    x = np.asarray(x, dt)
    if x.ndim == 3:
        x = x[..., None]
    return np.ascontiguousarray(x), x.shape[2], x.shape[3]


def serial(qh, kh, v, g, b, w, seg, init_state=None, prev_seg=None, nthreads=None, dtype=np.float64):
    """Token-serial recurrence on prepared inputs (see gdn_oracle.token_serial).

    Gates keep their own head / channel counts (H in {1, Hk, Hv}, C in {1, K}).
    Returns (out (B,L,Hv,V), final_state (B,Hv,K,V)) in `dtype`."""
    lib = load()
    fn = lib.dn_oracle_serial_f64 if dtype == np.float64 else lib.dn_oracle_serial_f32
    B, L, Hk, K = qh.shape
    Hv, V = v.shape[2], v.shape[3]
    c = lambda a: np.ascontiguousarray(np.asarray(a, dtype))
    qh, kh, v = c(qh), c(kh), c(v)
    g, Hg, Cg = _gate(g, B, L, dtype)
    b, Hb, Cb = _gate(b, B, L, dtype)
    w, Hw, Cw = _gate(w, B, L, dtype)
    seg = np.ascontiguousarray(np.broadcast_to(np.asarray(seg, np.int64), (B, L)))
    out = np.zeros((B, L, Hv, V), dtype)
    fin = np.zeros((B, Hv, K, V), dtype)
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p) if a is not None else None
    init = c(init_state) if init_state is not None else None
    prev = np.ascontiguousarray(np.asarray(prev_seg, np.int64)) if prev_seg is not None else None
    nt = nthreads or os.cpu_count() or 1
    rc = fn(B, L, Hk, Hv, K, V, P(qh), P(kh), P(v), P(g), Hg, Cg, P(b), Hb, Cb, P(w), Hw, Cw,
            P(seg), P(init), P(prev), P(out), P(fin), nt)
    if rc != 0:
        raise RuntimeError(f"dn_oracle_serial failed: {rc}")
    return out, fin
