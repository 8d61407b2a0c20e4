"""GPU checks of chunk_gdn2's precision options against the float64 oracles
(forward: oracle/gdn_oracle.py, gradients: oracle/gdn_grad.py), following the
reference's tests/test_precision_flags.py:18-80.

Inputs are the reference test's: B=1, L=256, Hk=1, Hv=2, q/k/v ~ 0.1 N(0,1),
three documents (0-49, 50-199, 200-255; the first two share chunk 0) and,
for the strong case, a decay of -2000 per token in document 0 and -1e-4 after
it.  The bounds are the reference's: output and every gradient within rel L2
1e-4 of the fp32 reference with ``mask_lambda_by_doc`` in "fp32" mode, 2e-2
for each option in "bf16" mode, and ``truncate_bwd_dT_bf16`` leaves the
forward unchanged.
"""

import numpy as np
import pytest
import torch

from oracle import gdn_grad as GR
from oracle import gdn_oracle as O
from tests._util import rel_l2, sig
from tests.gpu_common import as_np, to_dev

pytestmark = pytest.mark.gpu

NAMES = ("dq", "dk", "dv", "dg", "db", "dw")


def flag_inputs(strong_first_doc):
    B, L, Hk, Hv = 1, 256, 1, 2
    rng = np.random.default_rng(3)
    f = lambda *s: rng.standard_normal(s)
    q = f(B, L, Hk, 128) * 0.1
    k = f(B, L, Hk, 128) * 0.1
    v = f(B, L, Hv, 128) * 0.1
    g = -np.exp(f(B, L, Hk, 128) * 0.39 - 1.0)
    b = sig(f(B, L, Hk, 128))
    w = sig(f(B, L, Hv, 128))
    seg = np.concatenate([np.zeros(50), np.ones(150), 2 * np.ones(56)]).astype(np.int32)[None]
    if strong_first_doc:
        g = np.where((np.arange(L) < 50)[None, :, None, None], -2000.0, -1e-4 * np.ones_like(g))
    do = f(B, L, Hv, 128)
    return (q, k, v, g, b, w), seg, do


def run(args, seg, do, **kw):
    from deltanet_tpu_amd import chunk_gdn2
    ts = [to_dev(x).requires_grad_(True) for x in args]
    out = chunk_gdn2(*ts, segment_ids=to_dev(seg, torch.int32), is_inference=False, **kw)
    (out.float() * to_dev(do)).sum().backward()
    torch.cuda.synchronize()
    return as_np(out), {n: as_np(t.grad) for n, t in zip(NAMES, ts)}


def errors(args, seg, do, **kw):
    out, grads = run(args, seg, do, **kw)
    o_ref, _ = O.chunk_gdn2(*args, segment_ids=seg)
    g_ref = GR.chunk_gdn2_vjp(*args, do, segment_ids=seg)
    assert np.isfinite(out).all() and all(np.isfinite(x).all() for x in grads.values())
    errs = {n: rel_l2(grads[n], g_ref[n]) for n in NAMES}
    e_o = rel_l2(out, o_ref)
    print("[measured]", kw, f"out={e_o:.2e}", " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    return e_o, errs


@pytest.mark.parametrize("fallback_scan", [False, True])
def test_mask_lambda_by_doc_after_strong_decay(fallback_scan):
    args, seg, do = flag_inputs(strong_first_doc=True)
    e_o, errs = errors(args, seg, do, precision="fp32", fallback_scan=fallback_scan, mask_lambda_by_doc=True)
    assert e_o < 1e-4, e_o
    assert max(errs.values()) < 1e-4, errs
    # without the mask the result is never more accurate than with it
    e_o2, errs2 = errors(args, seg, do, precision="fp32", fallback_scan=fallback_scan)
    assert e_o <= e_o2 + 1e-7
    assert max(errs.values()) <= max(errs2.values()) + 1e-7


@pytest.mark.parametrize("flag", ["state_fp32_matmul", "truncate_bwd_dT_bf16", "mask_lambda_by_doc"])
def test_precision_flags_bf16(flag):
    args, seg, do = flag_inputs(strong_first_doc=False)
    e_o, errs = errors(args, seg, do, precision="bf16", **{flag: True})
    assert e_o < 2e-2, e_o
    assert max(errs.values()) < 2e-2, errs


def test_truncate_bwd_dT_bf16_leaves_forward_unchanged():
    from deltanet_tpu_amd import chunk_gdn2
    args, seg, _ = flag_inputs(strong_first_doc=False)
    ts = [to_dev(x) for x in args]
    sg = to_dev(seg, torch.int32)
    o0 = chunk_gdn2(*ts, segment_ids=sg, precision="bf16")
    o1 = chunk_gdn2(*ts, segment_ids=sg, precision="bf16", truncate_bwd_dT_bf16=True)
    assert torch.equal(o0, o1)


def test_later_document_gradients_independent_of_earlier_decay():
    # tests/test_precision_and_doc_lambda.py:78-116: with document 0 decaying
    # by -2000 per token, the gradients of every later token equal, bit for
    # bit, those with no decay in document 0 (the two documents share a chunk)
    args, seg, do = flag_inputs(strong_first_doc=True)
    clean = list(args)
    clean[3] = np.where((np.arange(256) < 50)[None, :, None, None], 0.0, args[3])
    _, g_strong = run(args, seg, do, precision="fp32")
    _, g_clean = run(tuple(clean), seg, do, precision="fp32")
    for n in NAMES:
        a, b = g_strong[n][:, 50:], g_clean[n][:, 50:]
        assert np.array_equal(a, b), (n, float(np.abs(a - b).max()))
