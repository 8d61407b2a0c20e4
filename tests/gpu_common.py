"""Helpers for the GPU parity tests: run the HIP path and the CPU oracle on
the same seeded inputs and compare with the north_star tolerances."""

from __future__ import annotations

import numpy as np
import torch

from oracle import c_oracle as C
from oracle import gdn_oracle as O
from tests._util import bf16, maxabs_over_rms, maxabs_over_rms_bf16_out, rel_frob, rel_l2

# north_star parity bars
TOL = {
    "fp32": dict(out=1e-4, state=1e-3),
    "bf16": dict(out=2e-2, state=1e-2),
}
TDT = {"fp32": torch.float32, "bf16": torch.bfloat16}


def to_dev(x, dtype=torch.float32):
    if x is None:
        return None
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0", dtype)


def as_np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def round_in(x, dt):
    """Value the device sees for an input array stored as dtype dt."""
    return bf16(x) if dt == "bf16" else np.asarray(x, np.float64)


def check(out, ref_out, state=None, ref_state=None, precision="fp32", out_dtype="fp32", tag=""):
    tol = TOL[precision]
    o = as_np(out)
    e = maxabs_over_rms_bf16_out(o, ref_out) if out_dtype == "bf16" else maxabs_over_rms(o, ref_out)
    r = rel_l2(o, ref_out)
    msg = f"{tag} out maxabs/rms={e:.3e} relL2={r:.3e}"
    if state is not None:
        se = rel_frob(as_np(state), ref_state)
        msg += f" state relF={se:.3e}"
    print("[measured]", msg, flush=True)
    assert np.isfinite(o).all(), msg
    assert e <= tol["out"], msg
    if state is not None:
        assert se <= tol["state"], msg
    return e


def oracle_prefill(q, k, v, g, b, w, *, qk_dtype="fp32", use_c=False, **kw):
    """Oracle chunk_gdn2; q, k, v already rounded as the device sees them."""
    if not use_c:
        return O.chunk_gdn2(q, k, v, g, b, w, qk_dtype=qk_dtype, **kw)
    # C restatement for large shapes (no streaming cap support needed there)
    B, L = q.shape[:2]
    qh, kh, vv, ga, ba, wa = O.prepare_prefill(q, k, v, g, b, w, scale=kw.get("scale"),
                                               qk_l2norm=kw.get("qk_l2norm", False),
                                               fuse_prologue=kw.get("fuse_prologue", False),
                                               qk_dtype=qk_dtype, broadcast=False)
    seg = O.canonical_segments(kw.get("segment_ids"), B, L)
    return C.serial(qh, kh, vv, ga, ba, wa, seg)
