"""Shared input generators and error metrics for the tests."""

from __future__ import annotations

import numpy as np

from oracle import gdn_oracle as O


def sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def make_inputs(seed, B, L, Hk, Hv, K=128, V=128, g_layout="channel_hk", b_layout="channel_hk",
                w_layout="channel_hv", qscale=1.0, g_shift=-1.0, g_spread=0.39):
    """Seeded inputs following the reference tests' generator (test_parity.py:18-26):
    q,k,v ~ N(0,1)*qscale; b, w = sigmoid(0.39 N); g = -exp(0.39 N - 1).
    Layouts: "<channel|scalar|rank3>_<hk|hv|one>"."""
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s)
    q = f(B, L, Hk, K) * qscale
    k = f(B, L, Hk, K) * qscale
    v = f(B, L, Hv, V) * qscale

    def gate_shape(layout, last):
        kind, heads = layout.split("_")
        H = {"hk": Hk, "hv": Hv, "one": 1}[heads]
        if kind == "channel":
            return (B, L, H, last)
        if kind == "scalar":
            return (B, L, H, 1)
        return (B, L, H)

    g = -np.exp(g_spread * f(*gate_shape(g_layout, K)) + g_shift)
    b = sig(0.39 * f(*gate_shape(b_layout, K)))
    w = sig(0.39 * f(*gate_shape(w_layout, V)))
    return q, k, v, g, b, w


def maxabs_over_rms(out, ref):
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(out - ref).max() / (np.sqrt(np.mean(ref ** 2)) + 1e-30))


def maxabs_over_rms_bf16_out(out, ref):
    """max |out - ref| / rms(ref) after removing the unavoidable rounding of a
    bf16 output: each element may differ by half a bf16 ulp of ref."""
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    a = np.abs(ref).astype(np.float32).view(np.uint32)
    ulp = ((a & 0x7F800000).view(np.float32).astype(np.float64)) * 2.0 ** -7
    excess = np.maximum(np.abs(out - ref) - 0.5 * ulp, 0.0)
    return float(excess.max() / (np.sqrt(np.mean(ref ** 2)) + 1e-30))


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-30))


def rel_frob(a, b):
    return rel_l2(a, b)


def bf16(x):
    return O.bf16_round(x).astype(np.float64)
