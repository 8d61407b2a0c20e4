"""Pins the gradient oracle (oracle/gdn_grad.py) before it is trusted as the
parity reference of the HIP backward.  The reference's gradient tests compare
its kernels with JAX autodiff of the token-serial recurrence
(tests/test_parity.py:37-68, 160-221); JAX is absent here, so the oracle is
pinned by:

* central finite differences of the float64 forward oracle, for every input
  (q, k, v, g, b, w, initial state, final-state cotangent) with document
  resets inside the sequence and at token 0;
* agreement of two independent derivations: the hand-written NumPy adjoint and
  torch.autograd through a torch restatement of the recurrence;
* the public-API wrapper derivative (fused prologue, L2-norm, scale, gate
  broadcast, GQA) against finite differences of ``gdn_oracle.chunk_gdn2``;
* the reference's gradient properties: full pass-through at g = 0
  (tests/test_strong_decay.py:91-109) and zero gradient for positive g
  without the prologue (tests/test_bwd_nonpositive.py).
"""

import numpy as np
import pytest

from oracle import gdn_grad as GR
from oracle import gdn_oracle as O
from tests._util import rel_l2, sig


def _core_inputs(seed, B=2, L=9, Hk=1, Hv=2, K=4, V=3):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s)
    qh, kh = f(B, L, Hk, K) * 0.7, f(B, L, Hk, K) * 0.7
    v = f(B, L, Hv, V)
    g = -np.exp(0.5 * f(B, L, Hv, K) - 1.0)
    b = sig(f(B, L, Hv, K))
    w = sig(f(B, L, Hv, V))
    init = f(B, Hv, K, V) * 0.3
    do = f(B, L, Hv, V)
    df = f(B, Hv, K, V)
    # batch 0: one reset mid-sequence, continues the initial state;
    # batch 1: starts a new document (initial state dropped) and resets twice
    seg = np.array([[0, 0, 0, 0, 1, 1, 1, 1, 1], [1, 1, 2, 2, 2, 3, 3, 3, 3]])[:, :L]
    return qh, kh, v, g, b, w, init, do, df, seg


def _core_loss(args, seg, do, df, prev):
    qh, kh, v, g, b, w, init = args
    out, S = O.token_serial(qh, kh, v, g, b, w, seg, init, prev_seg=prev)
    return float(np.sum(out * do) + np.sum(S * df))


def test_core_adjoint_vs_finite_differences():
    qh, kh, v, g, b, w, init, do, df, seg = _core_inputs(0)
    prev = np.zeros((2,), np.int64)
    gr = GR.token_serial_vjp(qh, kh, v, g, b, w, seg, init, prev, do, df)
    args = [qh, kh, v, g, b, w, init]
    names = ["dq", "dk", "dv", "dg", "db", "dw", "dinit"]
    eps = 1e-6
    for ai, name in enumerate(names):
        x = args[ai]
        num = np.zeros_like(x)
        it = np.nditer(x, flags=["multi_index"])
        for _ in it:
            i = it.multi_index
            xp = [a.copy() for a in args]; xm = [a.copy() for a in args]
            xp[ai][i] += eps; xm[ai][i] -= eps
            num[i] = (_core_loss(xp, seg, do, df, prev) - _core_loss(xm, seg, do, df, prev)) / (2 * eps)
        err = rel_l2(gr[name], num)
        assert err < 1e-7, f"{name}: adjoint vs finite differences rel L2 {err:.2e}"
    # batch 1 starts a new document: the initial state gets no gradient
    assert np.all(gr["dinit"][1] == 0.0) and np.abs(gr["dinit"][0]).max() > 0


def test_core_adjoint_vs_torch_autograd():
    import torch
    qh, kh, v, g, b, w, init, do, df, seg = _core_inputs(1, B=2, L=9, Hk=1, Hv=3, K=6, V=5)
    prev = np.zeros((2,), np.int64)
    gr = GR.token_serial_vjp(qh, kh, v, g, b, w, seg, init, prev, do, df)
    ts = [torch.tensor(x, requires_grad=True) for x in (qh, kh, v, g, b, w, init)]
    out, S = GR.torch_token_serial(*ts[:6], seg, ts[6], prev)
    ((out * torch.as_tensor(do)).sum() + (S * torch.as_tensor(df)).sum()).backward()
    for t, name in zip(ts, ["dq", "dk", "dv", "dg", "db", "dw", "dinit"]):
        err = rel_l2(gr[name], t.grad.numpy())
        assert err < 1e-12, f"{name}: adjoint vs autograd rel L2 {err:.2e}"


@pytest.mark.parametrize("mode", ["plain", "l2norm_gqa", "fused_guard"])
def test_public_vjp_vs_finite_differences(mode):
    rng = np.random.default_rng({"plain": 3, "l2norm_gqa": 4, "fused_guard": 5}[mode])
    f = lambda *s: rng.standard_normal(s)
    B, L, Hk, Hv, K, V = 1, 7, 1, 2, 4, 3
    q, k, v = f(B, L, Hk, K), f(B, L, Hk, K), f(B, L, Hv, V)
    kw = dict(scale=0.7)
    if mode == "plain":
        g = -np.exp(0.5 * f(B, L, Hv, K) - 1.0)     # channel gates at value heads
        b = sig(f(B, L, Hk, 1))                     # scalar b at key heads
        w = sig(f(B, L, 1, V))                      # one w for all heads
    elif mode == "l2norm_gqa":
        g = -np.exp(0.5 * f(B, L, Hk) - 1.0)        # rank-3 decay
        b = sig(f(B, L, Hk, K))
        w = sig(f(B, L, Hk, V))
        kw["qk_l2norm"] = True
    else:
        g = 0.5 * f(B, L, Hk, K) - 1.0              # raw prologue inputs
        b = f(B, L, Hk, K)
        w = f(B, L, Hv, V)
        kw.update(qk_l2norm=True, fuse_prologue=True, stability_guard=True)
    init = f(B, Hv, K, V) * 0.3
    seg = np.array([[0, 0, 0, 1, 1, 1, 1]])
    do, df = f(B, L, Hv, V), f(B, Hv, K, V)
    kw.update(segment_ids=seg, initial_state=init)
    gr = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do, df, **kw)
    args = {"dq": q, "dk": k, "dv": v, "dg": g, "db": b, "dw": w, "dinit": init}

    def loss(a):
        kk = dict(kw)
        kk["initial_state"] = a["dinit"]
        out, S = O.chunk_gdn2(a["dq"], a["dk"], a["dv"], a["dg"], a["db"], a["dw"], is_inference=False, **kk)
        return float(np.sum(out * do) + np.sum(S * df))

    for name, x in args.items():
        # the fused prologue rounds q and k to float32 first (gdn2.py:133-142):
        # a wider step keeps that rounding out of the difference quotient
        f32_in = mode == "fused_guard" and name in ("dq", "dk")
        eps, tol = (1e-3, 1e-4) if f32_in else (1e-6, 1e-6)
        num = np.zeros_like(x)
        it = np.nditer(x, flags=["multi_index"])
        for _ in it:
            i = it.multi_index
            ap = {n: a.copy() for n, a in args.items()}; am = {n: a.copy() for n, a in args.items()}
            ap[name][i] += eps; am[name][i] -= eps
            num[i] = (loss(ap) - loss(am)) / (2 * eps)
        err = rel_l2(gr[name], num)
        assert err < tol, f"{mode} {name}: vjp vs finite differences rel L2 {err:.2e}"
    ga = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do, df, core="autograd", **kw)
    for name in args:
        assert rel_l2(gr[name], ga[name]) < 1e-12, name


def test_gate_pass_through_at_zero_and_positive_cut():
    """g = 0 passes the full gradient (tests/test_strong_decay.py:91-109); g > 0
    (clamped to 0) passes none (tests/test_bwd_nonpositive.py)."""
    rng = np.random.default_rng(7)
    f = lambda *s: rng.standard_normal(s)
    B, L, H, K, V = 1, 6, 1, 4, 3
    q, k, v = f(B, L, H, K), f(B, L, H, K), f(B, L, H, V)
    b, w = sig(f(B, L, H, K)), sig(f(B, L, H, V))
    do = f(B, L, H, V)
    g0 = np.zeros((B, L, H, K))
    gp = np.full((B, L, H, K), 0.3)
    r0 = GR.chunk_gdn2_vjp(q, k, v, g0, b, w, do)
    rp = GR.chunk_gdn2_vjp(q, k, v, gp, b, w, do)
    qh = q / np.sqrt(K)
    core = GR.token_serial_vjp(qh, k, v, g0, b, w, np.zeros((B, L), np.int64), None, None, do)
    assert np.abs(r0["dg"]).max() > 0
    np.testing.assert_allclose(r0["dg"], core["dg"], rtol=1e-12, atol=1e-14)
    assert np.all(rp["dg"] == 0.0)
    # the value gradients do not depend on which side of the clamp g sits
    np.testing.assert_allclose(rp["dv"], r0["dv"], rtol=1e-12)
