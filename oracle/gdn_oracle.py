"""CPU oracle for the delta-rule recurrence core (GDN-2 / Gated DeltaNet forward).

TEST INFRASTRUCTURE ONLY.  Nothing in the product path may import this module:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker.  The product path
(``deltanet_tpu_amd``) runs hand-written HIP kernels and raises when they are
missing; it never falls back to this code.

Everything here is float64 NumPy restating the reference algorithm
(maelie-labs/deltanet-tpu v0.3.0, paths relative to ``src/deltanet_tpu/``):

* ``prepare_prefill``     -- the ``chunk_gdn2`` wrapper semantics
  (gdn2.py:1970-2125): nonpositive clamp of g (gdn2.py:1970-1971, 38-47),
  stability clamps (1972-1974), default scale (1978-1979), q/k L2-norm in fp32
  rounded back to the input dtype (2113-2122), gate broadcast rules
  (2009-2031), segment-id canonicalisation (2087-2094) and
  ``initial_state_segment_id`` (2081-2085), fused prologue (115-142).
* ``token_serial``        -- the token-serial recurrence of
  reference.py:123-161 (``token_serial_gdn2``), which is also the recurrence of
  ``reference_gdn`` (reference.py:253-274) once beta is both gates.
* ``chunk_gdn2`` / ``chunk_gdn`` -- the public-API oracle, including the
  streaming-prefill block loop with its between-block Frobenius cap
  (gdn2.py:2129-2196) and the final-state cap (2224-2226, 2236-2238).
* ``chunked_wy``          -- a second, independent restatement that follows
  the chunked WY algorithm of the prepass / state kernels (gdn2.py:115-240,
  585-652; chunk flags 1291-1302).  It exposes the per-chunk intermediates
  (Lambda, A, M, T, W, U, qe, ke) so tests can pin them by invariants.
* ``decode_step`` / ``gdn_decode_step`` -- gdn2.py:2289-2490 and
  variants.py:288-333.

Parity pinning (how each function is checked against something other than a
retyped formula) is listed in ``tests/test_oracle.py``.
"""

from __future__ import annotations

import math

import numpy as np

__all__ = [
    "bf16_round",
    "canonical_segments",
    "prepare_prefill",
    "token_serial",
    "chunk_gdn2",
    "chunk_gdn",
    "chunked_wy",
    "unit_lower_inverse",
    "decode_step",
    "gdn_decode_step",
    "frob_cap",
]


# ----------------------------------------------------------------------------
# helpers
# ----------------------------------------------------------------------------

def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float values to bfloat16 (round-to-nearest-even), returned as float32."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    # keep NaN as NaN
    return np.where(np.isnan(a), a, out)


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _nonpositive(x):
    # gdn2.py:38-41 -- the default guard: x <= 0 ? x : 0
    return np.where(x <= 0.0, x, 0.0)


def frob_cap(S: np.ndarray, tau: float) -> np.ndarray:
    """Frobenius cap S * min(1, tau / sqrt(||S||^2 + 1e-6)) over the last two axes
    (gdn2.py:2180-2188, 2224-2226, 2484-2487)."""
    n = np.sqrt(np.sum(S * S, axis=(-2, -1), keepdims=True) + 1e-6)
    return S * np.minimum(1.0, tau / n)


def canonical_segments(seg_ids, B: int, L: int, init_seg=None, has_init=False):
    """Canonical segment ids (B, L) int64 (gdn2.py:2033-2094).

    ``seg_ids`` may be None (one document), (L,) or (B, L).  ``init_seg`` is the
    ``initial_state_segment_id`` (int or (B,)); it only matters with an initial
    state.  Returns ids with ``seg'[t] = first_new + #changes in seg[1..t]``.
    """
    if seg_ids is None:
        s = np.zeros((B, L), dtype=np.int64)
    else:
        s = np.asarray(seg_ids).astype(np.int64)
        if s.ndim == 1:
            s = np.broadcast_to(s[None, :], (B, L))
    if has_init and init_seg is not None:
        first_new = (s[:, 0] != np.broadcast_to(np.asarray(init_seg, dtype=np.int64), (B,))).astype(np.int64)
    else:
        first_new = np.zeros((B,), dtype=np.int64)
    if L > 1:
        ch = np.concatenate([np.zeros((B, 1), np.int64), np.cumsum(s[:, 1:] != s[:, :-1], axis=1)], axis=1)
        return first_new[:, None] + ch
    return np.broadcast_to(first_new[:, None], (B, L)).copy()


def cu_seqlens_to_segments(cu_seqlens, L: int) -> np.ndarray:
    bounds = np.asarray(cu_seqlens, dtype=np.int64)
    lens = np.diff(bounds)
    return np.repeat(np.arange(len(lens), dtype=np.int64), lens)[:L]


def _gate_to_hv(x, B, L, Hk, Hv, last):
    """Broadcast a gate of shape (B,L,H) / (B,L,H,1) / (B,L,H,last) with H in
    {1, Hk, Hv} to (B, L, Hv, last) following the head-repeat rule ``hv // G``
    (reference.py:80-104; gdn2.py:1992-2031)."""
    x = np.asarray(x, dtype=np.float64)
    if x.ndim == 3:
        x = x[..., None]
    H = x.shape[2]
    if H == Hv:
        pass
    elif H == Hk:
        x = np.repeat(x, Hv // Hk, axis=2)
    elif H == 1:
        x = np.broadcast_to(x, (B, L, Hv, x.shape[3]))
    else:
        raise ValueError(f"bad gate head count {H}")
    return np.broadcast_to(x, (B, L, Hv, last))


# ----------------------------------------------------------------------------
# wrapper semantics
# ----------------------------------------------------------------------------

def prepare_prefill(q, k, v, g, b, w, *, scale=None, qk_l2norm=False, fuse_prologue=False,
                    stability_guard=False, qk_dtype="fp32", broadcast=True):
    """Apply the chunk_gdn2 prologue semantics and return float64
    (q_hat, k_hat, v, g_act, b_act, w_act), gates broadcast to value heads
    (``broadcast=False`` keeps each gate's own (B, L, H, C) layout, C = 1 for
    rank-3 gates, for the C restatement which maps heads itself).

    ``qk_dtype`` = "bf16" reproduces the wrapper storing the normalised q/k back in
    the bf16 input dtype (gdn2.py:2113-2122).
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, L, Hk, K = q.shape
    Hv, V = v.shape[2], v.shape[3]
    if scale is None:
        scale = 1.0 / math.sqrt(K)
    g = np.asarray(g, np.float64)
    b = np.asarray(b, np.float64)
    w = np.asarray(w, np.float64)
    if fuse_prologue:
        # gdn2.py:133-142 (prepass fused prologue), in fp32 arithmetic on the raw inputs
        q32 = q.astype(np.float32).astype(np.float64)
        k32 = k.astype(np.float32).astype(np.float64)
        qh = q32 / np.sqrt(np.sum(q32 * q32, -1, keepdims=True) + 1e-6) * scale
        kh = k32 / np.sqrt(np.sum(k32 * k32, -1, keepdims=True) + 1e-6)
        g_act = -np.exp(np.minimum(g, 5.0))
        if stability_guard:
            g_act = np.minimum(g_act, -1e-6)
        b_act = _sigmoid(b)
        w_act = _sigmoid(w)
    else:
        g_act = _nonpositive(g)  # gdn2.py:1970-1971
        b_act = b
        if stability_guard:  # gdn2.py:1972-1974
            b_act = np.maximum(b_act, 0.0)
            g_act = np.minimum(g_act, -1e-6)
        w_act = w
        if qk_l2norm:
            qh = q / np.sqrt(np.sum(q * q, -1, keepdims=True) + 1e-6) * scale
            kh = k / np.sqrt(np.sum(k * k, -1, keepdims=True) + 1e-6)
        else:
            qh = q * scale
            kh = k
        if qk_dtype == "bf16":
            qh = bf16_round(qh).astype(np.float64)
            kh = bf16_round(kh).astype(np.float64)
    if not broadcast:
        four = lambda x: x[..., None] if x.ndim == 3 else x
        return qh, kh, v, four(g_act), four(b_act), four(w_act)
    g_hv = _gate_to_hv(g_act, B, L, Hk, Hv, K)
    b_hv = _gate_to_hv(b_act, B, L, Hk, Hv, K)
    w_hv = _gate_to_hv(w_act, B, L, Hk, Hv, V)
    return qh, kh, v, g_hv, b_hv, w_hv


# ----------------------------------------------------------------------------
# token-serial recurrence
# ----------------------------------------------------------------------------

def token_serial(qh, kh, v, g, b, w, seg, init_state=None, prev_seg=None, heads=None):
    """Token-serial GDN-2 recurrence in float64 (reference.py:123-161).

    qh, kh: (B, L, Hk, K) prepared (normalised, scaled) queries/keys.
    v: (B, L, Hv, V); g, b: (B, L, Hv, K) activated; w: (B, L, Hv, V).
    seg: (B, L) canonical segment ids.  A reset happens at token t when
    seg[t] != prev (prev = seg[t-1], and for t = 0 ``prev_seg``: -1 without an
    initial state, seg[:,0] with one -- reference.py:151-156 -- unless the
    caller passes its own ``prev_seg``).
    heads: optional list of value heads to evaluate (others are skipped; the
    returned arrays then hold only those heads, in that order, and
    ``init_state`` must hold those heads only).
    Returns out (B, L, Hv', V) float64 and final state (B, Hv', K, V) float64.
    """
    B, L, Hk, K = qh.shape
    Hv, V = v.shape[2], v.shape[3]
    G = Hv // Hk
    hv_idx = np.arange(Hv) if heads is None else np.asarray(heads)
    hk_idx = hv_idx // G
    nh = len(hv_idx)
    S = np.zeros((B, nh, K, V), np.float64)
    if init_state is not None:
        S[:] = np.asarray(init_state, np.float64)
    if prev_seg is None:
        prev = seg[:, 0].copy() if init_state is not None else np.full((B,), -1, np.int64)
    else:
        prev = np.asarray(prev_seg, np.int64).copy()
    out = np.zeros((B, L, nh, V), np.float64)
    for t in range(L):
        st = seg[:, t]
        reset = st != prev
        if np.any(reset):
            S[reset] = 0.0
        prev = st
        qt = qh[:, t][:, hk_idx]            # (B, nh, K)
        kt = kh[:, t][:, hk_idx]
        d = np.exp(g[:, t][:, hv_idx])      # (B, nh, K)
        S *= d[..., None]
        beta = b[:, t][:, hv_idx] * kt
        e = np.einsum("bhk,bhkv->bhv", beta, S)
        vn = w[:, t][:, hv_idx] * v[:, t][:, hv_idx] - e
        S += kt[..., None] * vn[:, :, None, :]
        out[:, t] = np.einsum("bhk,bhkv->bhv", qt, S)
    return out, S


# ----------------------------------------------------------------------------
# public-API oracle
# ----------------------------------------------------------------------------

def chunk_gdn2(q, k, v, g, b, w, *, segment_ids=None, cu_seqlens=None, initial_state=None,
               initial_state_segment_id=None, output_final_state=False, chunk_size=128,
               precision="bf16", scale=None, qk_l2norm=False, fuse_prologue=False,
               streaming_prefill=False, prefill_block_size=4096, stability_guard=False,
               stability_tau=1000.0, is_inference=True, heads=None, **_unused):
    """Oracle for ``chunk_gdn2`` (gdn2.py:1772-2286) in float64.

    Returns float64 (out, final_state) always; ``heads`` restricts evaluation to
    a subset of value heads.  ``precision`` only selects whether q/k are rounded
    to bf16 after normalisation (which the wrapper does when the inputs are bf16).
    """
    q = np.asarray(q)
    B, L, Hk, K = q.shape
    Hv, V = v.shape[2], v.shape[3]
    bf16_in = (str(getattr(q, "dtype", "")) in ("bfloat16",)) or _unused.get("qk_dtype") == "bf16"
    qh, kh, vv, ga, ba, wa = prepare_prefill(
        q, k, v, g, b, w, scale=scale, qk_l2norm=qk_l2norm, fuse_prologue=fuse_prologue,
        stability_guard=stability_guard, qk_dtype="bf16" if bf16_in else "fp32")
    if cu_seqlens is not None:
        seg_raw = cu_seqlens_to_segments(cu_seqlens, L)
    else:
        seg_raw = segment_ids
    has_init = initial_state is not None
    seg = canonical_segments(seg_raw, B, L, initial_state_segment_id, has_init)
    # chunk 0 of a call with an initial state continues it unless the canonical id
    # says otherwise (gdn2.py:1291-1294: prev = 0 when has_init, else -1)
    prev0 = np.zeros((B,), np.int64) if has_init else np.full((B,), -1, np.int64)

    hv_idx = np.arange(Hv) if heads is None else np.asarray(heads)
    state = np.asarray(initial_state, np.float64)[:, hv_idx] if has_init else None
    if is_inference and streaming_prefill and L > prefill_block_size:
        # gdn2.py:2129-2196: blocks of prefill_block_size tokens, state carried,
        # block ids rebased so a block starts a new document iff seg[sb] != seg[sb-1]
        outs = []
        for sb in range(0, L, prefill_block_size):
            eb = min(sb + prefill_block_size, L)
            if sb == 0:
                p = prev0 if has_init else None
            else:
                p = seg[:, sb - 1]
            o, state = token_serial(qh[:, sb:eb], kh[:, sb:eb], vv[:, sb:eb], ga[:, sb:eb], ba[:, sb:eb],
                                    wa[:, sb:eb], seg[:, sb:eb], state, prev_seg=p, heads=heads)
            if stability_guard:
                state = frob_cap(state, stability_tau)
            outs.append(o)
        return np.concatenate(outs, axis=1), state

    out, S = token_serial(qh, kh, vv, ga, ba, wa, seg, state,
                          prev_seg=prev0 if has_init else None, heads=heads)
    if stability_guard and is_inference and output_final_state:
        S = frob_cap(S, stability_tau)
    return out, S


def chunk_gdn(q, k, v, g, beta, **kw):
    """Oracle for ``chunk_gdn`` (variants.py:17-88): GDN-2 with b = w = beta."""
    beta = np.asarray(beta)
    if beta.ndim == 4 and beta.shape[-1] > 1:
        raise ValueError("channel-wise beta is not supported")
    return chunk_gdn2(q, k, v, g, beta, beta, **kw)


# ----------------------------------------------------------------------------
# chunked WY restatement (second, independent algorithm)
# ----------------------------------------------------------------------------

def unit_lower_inverse(A: np.ndarray) -> np.ndarray:
    """T = (I + A)^-1 for strictly-lower-triangular A, by forward substitution.

    The reference computes the same matrix by block doubling + Neumann series
    (gdn2.py:67-111); the algorithm differs, the result is the same matrix."""
    C = A.shape[-1]
    T = np.zeros_like(A)
    for i in range(C):
        T[..., i, i] = 1.0
        # row i: T[i, :] = e_i - sum_{j<i} A[i, j] T[j, :]
        T[..., i, :i] -= np.einsum("...j,...jc->...c", A[..., i, :i], T[..., :i, :i])
    return T


def chunked_wy(qh, kh, v, g, b, w, seg, init_state=None, prev_seg=None, chunk_size=128):
    """Chunked WY/UT-transform forward for one batch element and one value head.

    Shapes (already prepared, one head): qh, kh, g, b (L, K); v, w (L, V);
    seg (L,) canonical.  Follows gdn2.py:115-240 (prepass) and 585-652 (state
    pass), with the per-chunk flags of gdn2.py:1291-1302; L is padded to a
    multiple of chunk_size with inert tokens (gdn2.py:2096-2111).
    Returns out (L, V), final state (K, V) and a list of per-chunk dicts.
    """
    L, K = qh.shape
    V = v.shape[1]
    C = chunk_size
    NC = (L + C - 1) // C
    Lp = NC * C
    pad = Lp - L

    def padz(x):
        return np.concatenate([x, np.zeros((pad,) + x.shape[1:])], 0) if pad else x

    qh, kh, v, g, b, w = map(padz, (qh, kh, v, g, b, w))
    seg = np.concatenate([seg, np.full((pad,), seg[-1])]) if pad else seg
    S = np.zeros((K, V)) if init_state is None else np.array(init_state, np.float64)
    if prev_seg is None:
        prev_seg = 0 if init_state is not None else -1
    out = np.zeros((Lp, V))
    inter = []
    tri = np.tril(np.ones((C, C)))
    for c in range(NC):
        sl = slice(c * C, (c + 1) * C)
        q_c, k_c, v_c, g_c, b_c, w_c, s_c = qh[sl], kh[sl], v[sl], g[sl], b[sl], w[sl], seg[sl]
        Lam = tri @ g_c                                        # inclusive cumsum (gdn2.py:150-155)
        beta = b_c * k_c
        same = s_c[:, None] == s_c[None, :]
        D = np.exp(_nonpositive(Lam[:, None, :] - Lam[None, :, :]))   # (i, j, kappa)
        A = np.einsum("ik,ijk,jk->ij", beta, D, k_c)
        M = np.einsum("ik,ijk,jk->ij", q_c, D, k_c)
        i_ = np.arange(C)
        A = np.where((i_[:, None] > i_[None, :]) & same, A, 0.0)
        M = np.where((i_[:, None] >= i_[None, :]) & same, M, 0.0)
        first = (s_c == s_c[0])[:, None]
        last = (s_c == s_c[-1])[:, None]
        eL = np.exp(_nonpositive(Lam))
        be = np.where(first, beta * eL, 0.0)
        qe = np.where(first, q_c * eL, 0.0)
        Lend = Lam[-1]
        ke = np.where(last, k_c * np.exp(_nonpositive(Lend[None, :] - Lam)), 0.0)
        T = unit_lower_inverse(A)
        W = T @ be
        U = T @ (w_c * v_c)
        # chunk flags (gdn2.py:1291-1302)
        prev = prev_seg if c == 0 else seg[c * C - 1]
        is_new = s_c[0] != prev
        all_same = s_c[0] == s_c[-1]
        if is_new:
            S = np.zeros((K, V))
        Vn = U - W @ S
        out[sl] = qe @ S + M @ Vn
        S_dec = S * np.exp(_nonpositive(Lend))[:, None] if all_same else np.zeros((K, V))
        S = S_dec + ke.T @ Vn
        inter.append(dict(Lambda=Lam, A=A, M=M, T=T, W=W, U=U, qe=qe, ke=ke, Lend=Lend))
    return out[:L], S, inter


# ----------------------------------------------------------------------------
# decode step
# ----------------------------------------------------------------------------

def decode_step(q, k, v, g, b, w, state, *, reset=None, scale=None, qk_l2norm=False,
                stability_guard=False, stability_tau=1000.0):
    """Oracle for ``gdn2_decode_step`` (gdn2.py:2289-2490), float64.

    q, k: (B, Hk, K) or (B, 1, Hk, K); v: (B, Hv, V) or (B, 1, Hv, V); gates per the
    reference's accepted shapes; state (B, Hv, K, V).  Returns (o (B, Hv, V),
    new_state (B, Hv, K, V)) in float64 (no output/state rounding).
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    g = np.asarray(g, np.float64)
    b = np.asarray(b, np.float64)
    w = np.asarray(w, np.float64)
    if q.ndim == 4:
        q, k, v = q[:, 0], k[:, 0], v[:, 0]
        if g.ndim in (3, 4) and g.shape[1] == 1:
            g = g[:, 0]
        if b.ndim in (3, 4) and b.shape[1] == 1:
            b = b[:, 0]
        if w.ndim in (3, 4) and w.shape[1] == 1:
            w = w[:, 0]
    B, Hk, K = q.shape
    Hv, V = v.shape[1], v.shape[2]
    G = Hv // Hk
    S = np.array(state, np.float64)
    g = _nonpositive(g)
    if stability_guard:
        b = np.maximum(b, 0.0)
        g = np.minimum(g, -1e-6)
    if reset is not None:
        r = np.broadcast_to(np.asarray(reset, bool).reshape(-1), (B,))
        S[r] = 0.0
    if scale is None:
        scale = 1.0 / math.sqrt(K)
    if qk_l2norm:
        q = q / np.sqrt(np.sum(q * q, -1, keepdims=True) + 1e-6) * scale
        k = k / np.sqrt(np.sum(k * k, -1, keepdims=True) + 1e-6)
    else:
        q = q * scale

    def hv(x, last):
        if x.ndim == 2:
            x = x[:, :, None]
        H = x.shape[1]
        if H == Hv:
            pass
        elif H == Hk:
            x = np.repeat(x, G, axis=1)
        elif H == 1:
            x = np.broadcast_to(x, (B, Hv, x.shape[2]))
        return np.broadcast_to(x, (B, Hv, last))

    qv = np.repeat(q, G, axis=1)
    kv = np.repeat(k, G, axis=1)
    gv, bv, wv = hv(g, K), hv(b, K), hv(w, V)
    Sd = S * np.exp(gv)[..., None]
    e = np.einsum("bhk,bhkv->bhv", bv * kv, Sd)
    vn = wv * v - e
    Sn = Sd + kv[..., None] * vn[:, :, None, :]
    o = np.einsum("bhk,bhkv->bhv", qv, Sn)
    if stability_guard:
        Sn = frob_cap(Sn, stability_tau)
    return o, Sn


def gdn_decode_step(q, k, v, g, beta, state, **kw):
    """Oracle for ``gdn_decode_step`` (variants.py:308-333): b = w = beta."""
    beta = np.asarray(beta)
    if beta.ndim == 3 and beta.shape[1] == 1:
        beta = beta[:, 0]
    elif beta.ndim == 4:
        if beta.shape[-1] > 1:
            raise ValueError("channel-wise beta is not supported")
        if beta.shape[1] == 1:
            beta = beta[:, 0]
    return decode_step(q, k, v, g, beta, beta, state, **kw)
