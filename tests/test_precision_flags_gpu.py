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


def test_forward_paths_after_a_strongly_decayed_document():
    # the forward paths that accumulate decay over a chunk (general prepass in
    # both precisions, the scalar-gate prepass, the chunked multi-token
    # decode across a reset) on a document decaying by -2000 per token
    # followed by ones decaying by -1e-4: each within its precision's bar
    import deltanet_tpu_amd as D
    from tests._util import maxabs_over_rms
    from tests.test_decode_gpu import chain_oracle
    rng = np.random.default_rng(3)
    B, L, Hk, Hv = 1, 256, 1, 2
    _, seg, _ = flag_inputs(strong_first_doc=True)
    q, k = 0.1 * rng.standard_normal((2, B, L, Hk, 128))
    v = 0.1 * rng.standard_normal((B, L, Hv, 128))
    first = (np.arange(L) < 50)[None, :, None]
    g = np.where(first[..., None], -2000.0, -1e-4 * np.ones((B, L, Hk, 128)))
    b, w = sig(rng.standard_normal((B, L, Hk, 128))), sig(rng.standard_normal((B, L, Hv, 128)))
    ro, _ = O.chunk_gdn2(q, k, v, g, b, w, segment_ids=seg)
    for prec, tol in (("fp32", 1e-5), ("bf16", 5e-3)):
        o = D.chunk_gdn2(*(to_dev(x) for x in (q, k, v, g, b, w)), segment_ids=to_dev(seg, torch.int32),
                         precision=prec, is_inference=True)
        assert rel_l2(as_np(o), ro) < tol, prec
    gs = np.where(first, -2000.0, -1e-4 * np.ones((B, L, Hv)))
    bs = sig(rng.standard_normal((B, L, Hv)))
    qb, kb = (O.bf16_round(x).astype(np.float64) for x in (q, k))
    ro2, _ = O.chunk_gdn2(qb, kb, v, gs, bs, bs, segment_ids=seg, qk_l2norm=True, qk_dtype="bf16")
    o2 = D.chunk_gdn(to_dev(qb, torch.bfloat16), to_dev(kb, torch.bfloat16), to_dev(v, torch.bfloat16), to_dev(gs),
                     to_dev(bs), segment_ids=to_dev(seg, torch.int32), precision="bf16", is_inference=True, qk_l2norm=True)
    assert rel_l2(as_np(o2), ro2) < 1e-2
    T, Bd = 32, 2
    qd, kd = rng.standard_normal((2, Bd, T, Hk, 128))
    vd = rng.standard_normal((Bd, T, Hv, 128))
    gd = np.where((np.arange(T) % 16 < 6)[None, :, None, None], -2000.0, -1e-4 * np.ones((Bd, T, Hk, 128)))
    bd, wd = sig(rng.standard_normal((Bd, T, Hk, 128))), sig(rng.standard_normal((Bd, T, Hv, 128)))
    reset = np.zeros((Bd, T), bool)
    reset[:, 6] = reset[:, 22] = True   # inside each 16-token chunk, after the strong decay
    S0 = to_dev(0.2 * rng.standard_normal((Bd, Hv, 128, 128)))
    o, s = D.gdn2_decode_steps(*(to_dev(x) for x in (qd, kd, vd, gd, bd, wd)), S0, reset=torch.tensor(reset),
                               qk_l2norm=True)
    rod, rsd = chain_oracle(qd, kd, vd, gd, bd, wd, as_np(S0), reset, qk_l2norm=True)
    assert maxabs_over_rms(as_np(o).reshape(Bd, T * Hv, 128), rod.reshape(Bd, T * Hv, 128)) < 1e-4
    assert rel_l2(as_np(s), rsd) < 1e-5
