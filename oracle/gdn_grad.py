"""CPU gradient oracle for the GDN-2 recurrence (the training backward).

TEST INFRASTRUCTURE ONLY.  Nothing in the product path may import this module:
only ``tests/`` use it, and only as the checker.

The reference (maelie-labs/deltanet-tpu v0.3.0, ``src/deltanet_tpu/``) trains
through a ``jax.custom_vjp`` (gdn2.py:1446-1769) whose backward kernels
(gdn2.py:243-493, 496-582, 698-769) are checked in the reference's own tests
against JAX autodiff of the token-serial recurrence (reference.py:123-161;
tests/test_parity.py:37-68, 160-221).  This module restates that checker:

* ``token_serial_vjp``   -- a hand-derived reverse-mode adjoint of the
  token-serial recurrence (float64 NumPy), reverse over tokens:
      dS += q do^T ; dq = S_t do ; dk = dS u ; du = dS^T k
      dw = du*v ; dv = du*w ; dSd = dS - beta du^T ; dbeta = -Sd du
      db = dbeta*k ; dk += dbeta*b ; dg = rowsum(dSd * Sd) ; dS = e^g dSd
  with dS cut at every document reset (reference.py:141-143).
* ``torch_token_serial`` -- the same forward written with torch float64 ops,
  differentiated by torch.autograd: a second, independent derivation.
* ``chunk_gdn2_vjp``     -- gradients of the public ``chunk_gdn2`` with respect
  to its raw inputs: the wrapper semantics of gdn2.py:1970-2125 (nonpositive
  gate with its pass-through gradient at g <= 0, gdn2.py:38-62; guard clamps;
  fused prologue; q/k L2-norm and scale; gate broadcast and GQA head repeat)
  differentiated by torch.autograd in float64, around the core adjoint above.

Pinning (tests/test_oracle_grad.py): central finite differences of the
float64 forward oracle for every input, including resets, initial state and
the fused prologue; agreement of the two independent derivations; and the
reference's own gradient properties (pass-through at g = 0,
tests/test_strong_decay.py:91-109; zero gradient for positive g without the
prologue, tests/test_bwd_nonpositive.py).
"""

from __future__ import annotations

import math

import numpy as np

from . import gdn_oracle as _o

__all__ = ["token_serial_vjp", "torch_token_serial", "chunk_gdn2_vjp", "prepare_torch"]


def token_serial_vjp(qh, kh, v, g, b, w, seg, init_state, prev_seg, dout, dfinal=None):
    """Reverse-mode adjoint of ``gdn_oracle.token_serial`` (reference.py:123-161).

    Shapes as ``token_serial``: qh, kh (B, L, Hk, K); v, w (B, L, Hv, V);
    g, b (B, L, Hv, K) (g already clamped); seg (B, L) canonical; prev_seg (B,)
    the segment id the initial state belongs to (-1 = none).
    Returns dict dq, dk (B, L, Hk, K) summed over the value heads sharing a key
    head; dv, dw (B, L, Hv, V); dg, db (B, L, Hv, K); dinit (B, Hv, K, V).
    """
    qh = np.asarray(qh, np.float64); kh = np.asarray(kh, np.float64)
    v = np.asarray(v, np.float64); g = np.asarray(g, np.float64)
    b = np.asarray(b, np.float64); w = np.asarray(w, np.float64)
    dout = np.asarray(dout, np.float64)
    B, L, Hk, K = qh.shape
    Hv, V = v.shape[2], v.shape[3]
    G = Hv // Hk
    hk_of = np.arange(Hv) // G
    prev = np.full((B,), -1, np.int64) if prev_seg is None else np.asarray(prev_seg, np.int64)
    # forward, keeping the state before each token (after its reset) and after it
    S = np.zeros((B, Hv, K, V))
    if init_state is not None:
        S[:] = np.asarray(init_state, np.float64)
    pre = np.zeros((L, B, Hv, K, V))
    resets = np.zeros((L, B), bool)
    p = prev.copy()
    for t in range(L):
        r = seg[:, t] != p
        resets[t] = r
        S[r] = 0.0
        p = seg[:, t]
        pre[t] = S
        kt = kh[:, t][:, hk_of]
        d = np.exp(g[:, t])
        Sd = S * d[..., None]
        beta = b[:, t] * kt
        u = w[:, t] * v[:, t] - np.einsum("bhk,bhkv->bhv", beta, Sd)
        S = Sd + kt[..., None] * u[:, :, None, :]
    # reverse
    dS = np.zeros((B, Hv, K, V)) if dfinal is None else np.array(dfinal, np.float64)
    dq = np.zeros((B, L, Hv, K)); dk = np.zeros((B, L, Hv, K)); dv = np.zeros((B, L, Hv, V))
    dg = np.zeros((B, L, Hv, K)); db = np.zeros((B, L, Hv, K)); dw = np.zeros((B, L, Hv, V))
    for t in range(L - 1, -1, -1):
        qt = qh[:, t][:, hk_of]; kt = kh[:, t][:, hk_of]
        d = np.exp(g[:, t])
        Sd = pre[t] * d[..., None]
        beta = b[:, t] * kt
        u = w[:, t] * v[:, t] - np.einsum("bhk,bhkv->bhv", beta, Sd)
        St = Sd + kt[..., None] * u[:, :, None, :]
        do = dout[:, t]
        dS = dS + qt[..., None] * do[:, :, None, :]
        dq[:, t] = np.einsum("bhkv,bhv->bhk", St, do)
        dkt = np.einsum("bhkv,bhv->bhk", dS, u)
        du = np.einsum("bhkv,bhk->bhv", dS, kt)
        dw[:, t] = du * v[:, t]
        dv[:, t] = du * w[:, t]
        dSd = dS - beta[..., None] * du[:, :, None, :]
        dbeta = -np.einsum("bhkv,bhv->bhk", Sd, du)
        db[:, t] = dbeta * kt
        dk[:, t] = dkt + dbeta * b[:, t]
        dg[:, t] = np.sum(dSd * Sd, axis=-1)
        dS = dSd * d[..., None]
        dS[resets[t]] = 0.0
    dqk = np.zeros((B, L, Hk, K)); dkk = np.zeros((B, L, Hk, K))
    for h in range(Hv):
        dqk[:, :, hk_of[h]] += dq[:, :, h]
        dkk[:, :, hk_of[h]] += dk[:, :, h]
    return {"dq": dqk, "dk": dkk, "dv": dv, "dg": dg, "db": db, "dw": dw, "dinit": dS}


def torch_token_serial(qh, kh, v, g, b, w, seg, init_state, prev_seg):
    """The token-serial forward (reference.py:123-161) in torch, for autograd.

    Tensors are torch tensors of one dtype and device (float64 on the CPU for
    pinning; float32 on a GPU for full-size references), qh/kh at key heads,
    gates at value heads; returns (out (B, L, Hv, V), final state (B, Hv, K, V)).
    """
    import torch
    B, L, Hk, K = qh.shape
    Hv, V = v.shape[2], v.shape[3]
    G = Hv // Hk
    dev, dt = qh.device, qh.dtype
    idx = torch.arange(Hv, device=dev) // G
    S = torch.zeros((B, Hv, K, V), dtype=dt, device=dev) if init_state is None else init_state
    prev = torch.as_tensor(np.full((B,), -1) if prev_seg is None else np.asarray(prev_seg)).long().to(dev)
    seg_t = torch.as_tensor(np.asarray(seg)).long().to(dev)
    outs = []
    for t in range(L):
        keep = (seg_t[:, t] == prev).to(dt)[:, None, None, None]
        S = S * keep
        prev = seg_t[:, t]
        qt = qh[:, t][:, idx]; kt = kh[:, t][:, idx]
        Sd = S * torch.exp(g[:, t])[..., None]
        beta = b[:, t] * kt
        u = w[:, t] * v[:, t] - torch.einsum("bhk,bhkv->bhv", beta, Sd)
        S = Sd + kt[..., None] * u[:, :, None, :]
        outs.append(torch.einsum("bhk,bhkv->bhv", qt, S))
    return torch.stack(outs, 1), S


def _gate_hv_torch(x, B, L, Hk, Hv, last):
    import torch
    if x.ndim == 3:
        x = x[..., None]
    H = x.shape[2]
    if H == Hk and Hv != Hk:
        x = torch.repeat_interleave(x, Hv // Hk, dim=2)
    elif H == 1:
        x = x.expand(B, L, Hv, x.shape[3])
    return x.expand(B, L, Hv, last)


def prepare_torch(q, k, v, g, b, w, *, scale=None, qk_l2norm=False, fuse_prologue=False,
                  stability_guard=False, qk_round=None):
    """The wrapper semantics of gdn2.py:1970-2125 as differentiable torch float64 ops.

    ``qk_round`` (a callable or None) rounds the normalised q/k like the wrapper's
    cast back to a bf16 input dtype (gdn2.py:2113-2122); its gradient is the
    identity, as for JAX's convert_element_type.
    Returns (qh, kh, v, g, b, w) with gates at (B, L, Hv, K|V).
    """
    import torch
    B, L, Hk, K = q.shape
    Hv, V = v.shape[2], v.shape[3]
    if scale is None:
        scale = 1.0 / math.sqrt(K)

    def l2(x):
        return x * torch.rsqrt(torch.sum(x * x, -1, keepdim=True) + 1e-6)

    if fuse_prologue:
        qh = l2(q) * scale
        kh = l2(k)
        ga = -torch.exp(torch.clamp(g, max=5.0))
        if stability_guard:
            ga = torch.clamp(ga, max=-1e-6)
        ba = torch.sigmoid(b)
        wa = torch.sigmoid(w)
    else:
        # gdn2.py:38-62: value where g <= 0 else 0, gradient passed where g <= 0
        ga = torch.where(g <= 0.0, g, torch.zeros_like(g))
        ba = b
        if stability_guard:
            ba = torch.clamp(ba, min=0.0)
            ga = torch.clamp(ga, max=-1e-6)
        wa = w
        if qk_l2norm:
            qh = l2(q) * scale
            kh = l2(k)
        else:
            qh = q * scale
            kh = k
        if qk_round is not None:
            qh = qh + (qk_round(qh.detach()) - qh.detach())
            kh = kh + (qk_round(kh.detach()) - kh.detach())
    return (qh, kh, v, _gate_hv_torch(ga, B, L, Hk, Hv, K), _gate_hv_torch(ba, B, L, Hk, Hv, K),
            _gate_hv_torch(wa, B, L, Hk, Hv, V))


def chunk_gdn2_vjp(q, k, v, g, b, w, dout, dfinal=None, *, segment_ids=None, cu_seqlens=None,
                   initial_state=None, initial_state_segment_id=None, scale=None, qk_l2norm=False,
                   fuse_prologue=False, stability_guard=False, qk_bf16=False, core="adjoint"):
    """Gradients of the training-mode ``chunk_gdn2`` (gdn2.py:1772-2286 with
    is_inference=False) for the loss sum(out * dout) + sum(final * dfinal).

    Inputs are NumPy arrays (any float dtype, taken as float64).  ``core`` picks
    the recurrence derivative: "adjoint" (``token_serial_vjp``) or "autograd"
    (``torch_token_serial``).  Returns a dict with dq, dk, dv, dg, db, dw in the
    raw inputs' shapes and dinit (or None).
    """
    import torch
    B, L, Hk, K = np.asarray(q).shape
    Hv = np.asarray(v).shape[2]
    T = lambda x: torch.tensor(np.asarray(x, np.float64), requires_grad=True)
    tq, tk, tv, tg, tb, tw = (T(x) for x in (q, k, v, g, b, w))
    has_init = initial_state is not None
    tinit = T(initial_state) if has_init else None
    rnd = (lambda x: torch.as_tensor(_o.bf16_round(x.numpy()), dtype=torch.float64)) if qk_bf16 else None
    qh, kh, vv, ga, ba, wa = prepare_torch(tq, tk, tv, tg, tb, tw, scale=scale, qk_l2norm=qk_l2norm,
                                           fuse_prologue=fuse_prologue, stability_guard=stability_guard,
                                           qk_round=rnd)
    seg_raw = _o.cu_seqlens_to_segments(cu_seqlens, L) if cu_seqlens is not None else segment_ids
    seg = _o.canonical_segments(seg_raw, B, L, initial_state_segment_id, has_init)
    prev0 = np.zeros((B,), np.int64) if has_init else None
    do = np.asarray(dout, np.float64)
    df = None if dfinal is None else np.asarray(dfinal, np.float64)
    if core == "autograd":
        out, fin = torch_token_serial(qh, kh, vv, ga, ba, wa, seg, tinit, prev0)
        loss = (out * torch.as_tensor(do)).sum()
        if df is not None:
            loss = loss + (fin * torch.as_tensor(df)).sum()
        loss.backward()
    else:
        gr = token_serial_vjp(qh.detach().numpy(), kh.detach().numpy(), vv.detach().numpy(),
                              ga.detach().numpy(), ba.detach().numpy(), wa.detach().numpy(),
                              seg, tinit.detach().numpy() if has_init else None, prev0, do, df)
        outs = [qh, kh, vv, ga, ba, wa]
        grads = [gr["dq"], gr["dk"], gr["dv"], gr["dg"], gr["db"], gr["dw"]]
        if has_init:
            outs.append(tinit)
            grads.append(gr["dinit"])
        torch.autograd.backward(
            [o for o in outs if o.requires_grad],
            [torch.as_tensor(x) for o, x in zip(outs, grads) if o.requires_grad])
    res = {n: t.grad.numpy() if t.grad is not None else np.zeros(t.shape)
           for n, t in zip(("dq", "dk", "dv", "dg", "db", "dw"), (tq, tk, tv, tg, tb, tw))}
    res["dinit"] = (tinit.grad.numpy() if tinit.grad is not None else np.zeros(tinit.shape)) if has_init else None
    return res
