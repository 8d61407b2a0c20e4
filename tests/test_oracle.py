"""Pins the CPU oracle (oracle/gdn_oracle.py, oracle/gdn_serial.c) before it is
trusted as the parity reference.  The reference holds no golden vectors for
this path (its tests compute expectations live with JAX, which is absent), so
each oracle function is pinned by checks that a plausible slip (dropped term,
wrong sign or index, transposed operand) fails:

* three independent algorithms agree: NumPy token-serial (reference.py:123-161),
  NumPy chunked WY (gdn2.py:115-240, 585-652) and the C token-serial loop;
* closed forms: GLA (b = 0, w = 1) is a decayed linear-attention sum; the
  delta rule with unit keys and b = w = 1 retrieves the last written value;
  with g = 0 and b = 0 the state is the plain outer-product sum;
* T = (I + A)^-1 matches scipy's triangular solve and (I + A) T = I;
* the API-level invariants the reference tests assert: decode x N == chunked
  prefill with a reset (test_inference.py:64-110), split prefill with
  state passing == one call (test_state_passing.py), streaming == monolithic
  (test_streaming_and_stability.py:28-62), initial_state_segment_id reset ==
  zero init (test_doc_reset_and_streaming.py:9-58), reused segment ids are
  distinct documents and cu_seqlens == segment_ids
  (test_document_boundaries.py), causality (test_causality.py);
* bf16_round agrees with torch's float32 -> bfloat16 conversion.
"""

import numpy as np
import pytest
import scipy.linalg

from oracle import c_oracle as C
from oracle import gdn_oracle as O
from tests._util import make_inputs, rel_l2, sig

K_SMALL = 16


def _prep(seed, B, L, Hk, Hv, K=K_SMALL, **kw):
    q, k, v, g, b, w = make_inputs(seed, B, L, Hk, Hv, K, K, **kw)
    return q, k, v, g, b, w


@pytest.mark.parametrize("L,chunk", [(1, 8), (7, 8), (64, 16), (100, 32), (130, 64)])
@pytest.mark.parametrize("docs", [False, True])
@pytest.mark.parametrize("init", [False, True])
def test_serial_vs_chunked_wy(L, chunk, docs, init):
    B, Hk, Hv, K = 2, 1, 2, K_SMALL
    q, k, v, g, b, w = _prep(L + 3 * docs + 7 * init, B, L, Hk, Hv)
    qh, kh, vv, ga, ba, wa = O.prepare_prefill(q, k, v, g, b, w, qk_l2norm=True)
    seg_raw = None
    if docs:
        rng = np.random.default_rng(L)
        seg_raw = np.sort(rng.integers(0, 4, size=(B, L)), axis=1)
    seg = O.canonical_segments(seg_raw, B, L, has_init=init)
    s0 = 0.3 * np.random.default_rng(1).standard_normal((B, Hv, K, K)) if init else None
    out, S = O.token_serial(qh, kh, vv, ga, ba, wa, seg, s0, prev_seg=np.zeros(B, np.int64) if init else None)
    for bb in range(B):
        for hv in range(Hv):
            o2, S2, _ = O.chunked_wy(qh[bb, :, hv // 2], kh[bb, :, hv // 2], vv[bb, :, hv], ga[bb, :, hv],
                                     ba[bb, :, hv], wa[bb, :, hv], seg[bb],
                                     init_state=None if s0 is None else s0[bb, hv], chunk_size=chunk)
            assert rel_l2(o2, out[bb, :, hv]) < 1e-12
            assert rel_l2(S2, S[bb, hv]) < 1e-12


def test_c_serial_matches_numpy_serial():
    B, L, Hk, Hv, K = 2, 90, 2, 4, 32
    q, k, v, g, b, w = make_inputs(3, B, L, Hk, Hv, K, K, g_layout="scalar_hv", b_layout="rank3_hk",
                                   w_layout="channel_hk")
    qh, kh, vv, ga, ba, wa = O.prepare_prefill(q, k, v, g, b, w, qk_l2norm=True, broadcast=False)
    seg_raw = (np.arange(L) >= 40).astype(np.int64)[None].repeat(B, 0)
    seg = O.canonical_segments(seg_raw, B, L)
    s0 = 0.1 * np.random.default_rng(0).standard_normal((B, Hv, K, K))
    ref_o, ref_s = O.token_serial(*O.prepare_prefill(q, k, v, g, b, w, qk_l2norm=True), seg, s0,
                                  prev_seg=np.zeros(B, np.int64))
    o, s = C.serial(qh, kh, vv, ga, ba, wa, seg, s0, prev_seg=np.zeros(B, np.int64))
    assert rel_l2(o, ref_o) < 1e-13 and rel_l2(s, ref_s) < 1e-13
    o32, s32 = C.serial(qh, kh, vv, ga, ba, wa, seg, s0, prev_seg=np.zeros(B, np.int64), dtype=np.float32)
    assert rel_l2(o32, ref_o) < 1e-5 and rel_l2(s32, ref_s) < 1e-5


def test_gla_closed_form():
    # b = 0, w = 1: S_t = sum_{s<=t} diag(exp(Lam_t - Lam_s)) k_s v_s^T
    B, L, H, K = 1, 40, 1, 8
    rng = np.random.default_rng(5)
    q, k, v = (rng.standard_normal((B, L, H, K)) for _ in range(3))
    g = -np.exp(0.5 * rng.standard_normal((B, L, H, K)) - 1.0)
    out, S = O.chunk_gdn2(q, k, v, g, np.zeros_like(k), np.ones_like(v), scale=1.0, output_final_state=True)
    Lam = np.cumsum(g[0, :, 0], axis=0)
    exp_o = np.zeros((L, K))
    for t in range(L):
        for s in range(t + 1):
            exp_o[t] += (q[0, t, 0] * np.exp(Lam[t] - Lam[s])) @ k[0, s, 0][:, None] * v[0, s, 0]
    assert rel_l2(out[0, :, 0], exp_o) < 1e-12
    exp_S = sum(np.exp(Lam[-1] - Lam[s])[:, None] * np.outer(k[0, s, 0], v[0, s, 0]) for s in range(L))
    assert rel_l2(S[0, 0], exp_S) < 1e-12


def test_delta_rule_retrieval_property():
    # g = 0, b = w = 1, |k| = 1, q = k, scale = 1: after writing (k_t, v_t) the
    # state maps k_t to v_t exactly, so o_t = v_t.
    B, L, H, K = 1, 30, 1, 16
    rng = np.random.default_rng(9)
    k = rng.standard_normal((B, L, H, K))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, L, H, K))
    out, _ = O.chunk_gdn2(k, k, v, np.zeros((B, L, H)), np.ones((B, L, H)), np.ones((B, L, H)), scale=1.0)
    assert rel_l2(out, v) < 1e-12


def test_no_erase_no_decay_is_outer_product_sum():
    B, L, H, K = 1, 25, 1, 8
    rng = np.random.default_rng(2)
    q, k, v = (rng.standard_normal((B, L, H, K)) for _ in range(3))
    w = sig(rng.standard_normal((B, L, H, K)))
    _, S = O.chunk_gdn2(q, k, v, np.zeros((B, L, H)), np.zeros((B, L, H)), w, output_final_state=True)
    exp = sum(np.outer(k[0, t, 0], w[0, t, 0] * v[0, t, 0]) for t in range(L))
    assert rel_l2(S[0, 0], exp) < 1e-12


@pytest.mark.parametrize("C_", [16, 64, 128])
def test_unit_lower_inverse(C_):
    rng = np.random.default_rng(C_)
    A = np.tril(rng.standard_normal((C_, C_)) * 0.3, -1)
    T = O.unit_lower_inverse(A)
    ref = scipy.linalg.solve_triangular(np.eye(C_) + A, np.eye(C_), lower=True, unit_diagonal=True)
    assert np.abs(T - ref).max() < 1e-10 * max(1.0, np.abs(ref).max())
    assert np.abs((np.eye(C_) + A) @ T - np.eye(C_)).max() < 1e-10
    # all-ones strictly-lower A (test_nan_adversarial.py:102-112): I + A is the
    # prefix-sum matrix, whose inverse is the first-difference matrix I - shift
    A1 = np.tril(np.ones((C_, C_)), -1)
    T1 = O.unit_lower_inverse(A1)
    assert np.array_equal(T1, np.eye(C_) - np.eye(C_, k=-1))


def test_decode_steps_equal_prefill_with_reset():
    # test_inference.py:64-110
    B, N, Hk, Hv, K = 1, 40, 1, 2, K_SMALL
    q, k, v, g, b, w = _prep(11, B, N, Hk, Hv)
    reset_idx = N // 2
    seg = (np.arange(N) >= reset_idx).astype(np.int64)[None]
    out_c, st_c = O.chunk_gdn2(q, k, v, g, b, w, segment_ids=seg, output_final_state=True, qk_l2norm=True)
    state = np.zeros((B, Hv, K, K))
    outs = []
    for t in range(N):
        o, state = O.decode_step(q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1], g[:, t:t + 1], b[:, t:t + 1],
                                 w[:, t:t + 1], state, reset=(t == reset_idx), qk_l2norm=True)
        outs.append(o[:, None])
    assert rel_l2(np.concatenate(outs, 1), out_c) < 1e-12
    assert rel_l2(state, st_c) < 1e-12


@pytest.mark.parametrize("split", [1, 17, 33])
def test_split_prefill_equals_single(split):
    B, L, Hk, Hv, K = 1, 50, 1, 2, K_SMALL
    q, k, v, g, b, w = _prep(12, B, L, Hk, Hv)
    o, s = O.chunk_gdn2(q, k, v, g, b, w, output_final_state=True, qk_l2norm=True)
    sl1, sl2 = slice(0, split), slice(split, L)
    o1, s1 = O.chunk_gdn2(*(x[:, sl1] for x in (q, k, v, g, b, w)), output_final_state=True, qk_l2norm=True)
    o2, s2 = O.chunk_gdn2(*(x[:, sl2] for x in (q, k, v, g, b, w)), initial_state=s1, output_final_state=True,
                          qk_l2norm=True)
    assert rel_l2(np.concatenate([o1, o2], 1), o) < 1e-12 and rel_l2(s2, s) < 1e-12


def test_streaming_equals_monolithic():
    B, L, Hk, Hv, K = 1, 300, 1, 2, K_SMALL
    q, k, v, g, b, w = _prep(13, B, L, Hk, Hv)
    seg = np.repeat(np.array([0, 0, 1, 1, 1, 2]), 50)[None]
    o, s = O.chunk_gdn2(q, k, v, g, b, w, segment_ids=seg, output_final_state=True, qk_l2norm=True)
    o2, s2 = O.chunk_gdn2(q, k, v, g, b, w, segment_ids=seg, output_final_state=True, qk_l2norm=True,
                          streaming_prefill=True, prefill_block_size=128)
    assert rel_l2(o2, o) < 1e-12 and rel_l2(s2, s) < 1e-12


def test_initial_state_segment_id_reset():
    B, L, Hk, Hv, K = 1, 20, 1, 1, K_SMALL
    q, k, v, g, b, w = _prep(14, B, L, Hk, Hv)
    seg = np.full((1, L), 5)
    s0 = np.random.default_rng(0).standard_normal((B, Hv, K, K))
    o0, s_0 = O.chunk_gdn2(q, k, v, g, b, w, segment_ids=seg, output_final_state=True)
    o1, s_1 = O.chunk_gdn2(q, k, v, g, b, w, segment_ids=seg, initial_state=s0, initial_state_segment_id=4,
                           output_final_state=True)
    assert np.array_equal(o0, o1) and np.array_equal(s_0, s_1)
    o2, _ = O.chunk_gdn2(q, k, v, g, b, w, segment_ids=seg, initial_state=s0, initial_state_segment_id=5)
    assert rel_l2(o2, o0) > 1e-3


def test_reused_ids_and_cu_seqlens():
    B, L, Hk, Hv, K = 1, 30, 1, 1, K_SMALL
    q, k, v, g, b, w = _prep(15, B, L, Hk, Hv)
    seg = np.array([0] * 10 + [1] * 10 + [0] * 10)[None]
    o1, _ = O.chunk_gdn2(q, k, v, g, b, w, segment_ids=seg)
    o2, _ = O.chunk_gdn2(q, k, v, g, b, w, cu_seqlens=[0, 10, 20, 30])
    assert np.array_equal(o1, o2)
    # third document must not see the first one
    o3, _ = O.chunk_gdn2(*(x[:, 20:] for x in (q, k, v, g, b, w)))
    assert rel_l2(o1[:, 20:], o3) < 1e-13


def test_causality():
    B, L, Hk, Hv, K = 1, 40, 1, 1, K_SMALL
    q, k, v, g, b, w = _prep(16, B, L, Hk, Hv)
    o1, _ = O.chunk_gdn2(q, k, v, g, b, w)
    v2 = v.copy()
    v2[:, 25:] += 1.0
    o2, _ = O.chunk_gdn2(q, k, v2, g, b, w)
    assert np.array_equal(o1[:, :25], o2[:, :25]) and not np.allclose(o1[:, 25:], o2[:, 25:])


def test_fused_prologue_equals_activated_inputs():
    B, L, Hk, Hv, K = 1, 20, 1, 2, K_SMALL
    rng = np.random.default_rng(17)
    q, k = rng.standard_normal((2, B, L, Hk, K))
    v = rng.standard_normal((B, L, Hv, K))
    graw, braw = rng.standard_normal((2, B, L, Hk, K))
    wraw = rng.standard_normal((B, L, Hv, K))
    o1, _ = O.chunk_gdn2(q, k, v, graw, braw, wraw, fuse_prologue=True, qk_l2norm=True)
    o2, _ = O.chunk_gdn2(q, k, v, -np.exp(np.minimum(graw, 5.0)), sig(braw), sig(wraw), qk_l2norm=True)
    assert rel_l2(o1, o2) < 1e-6  # fused path normalises in fp32


def test_decode_gate_broadcast_rules():
    # scalar-per-head, Hk-headed and one-headed gates all map value head hv to hv // G
    B, Hk, Hv, K = 2, 2, 4, K_SMALL
    rng = np.random.default_rng(18)
    q, k = rng.standard_normal((2, B, Hk, K))
    v = rng.standard_normal((B, Hv, K))
    S = rng.standard_normal((B, Hv, K, K))
    g_hk = -np.exp(rng.standard_normal((B, Hk)))
    b_hk = sig(rng.standard_normal((B, Hk)))
    o1, s1 = O.decode_step(q, k, v, g_hk, b_hk, sig(np.zeros((B, 1))), S)
    o2, s2 = O.decode_step(q, k, v, np.repeat(g_hk, 2, 1)[..., None].repeat(K, -1),
                           np.repeat(b_hk, 2, 1)[..., None].repeat(K, -1), np.full((B, Hv, K), 0.5), S)
    assert rel_l2(o1, o2) < 1e-14 and rel_l2(s1, s2) < 1e-14


def test_bf16_round_matches_torch():
    torch = pytest.importorskip("torch")
    x = np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 10.0 ** np.random.default_rng(1).integers(-5, 5, 100000)
    x[:4] = [0.0, -0.0, 1.00390625, 1.01171875]  # exact ties: round to even
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(O.bf16_round(x), ref)


# ----------------------------------------------------------------------------
# frob_cap (gdn2.py:2180-2188 streaming cap, 2224-2226 final cap, 2484-2487
# decode cap): pinned by what the cap must do, not by its formula
# ----------------------------------------------------------------------------

def test_frob_cap_properties():
    rng = np.random.default_rng(30)
    tau = 7.5
    # a batch of matrices: some far above tau, some below, one exactly zero
    S = rng.standard_normal((6, 16, 24))
    S[0] *= 50.0          # ||S|| ~ 1000 >> tau
    S[1] *= 3.0           # ||S|| ~ 60 > tau
    S[2] *= 0.1           # ||S|| ~ 2 < tau
    S[3] = 0.0
    S[4] *= tau / np.linalg.norm(S[4]) * 0.999   # just below tau
    S[5] *= tau / np.linalg.norm(S[5]) * 1.001   # just above tau
    out = O.frob_cap(S, tau)
    nrm = np.linalg.norm(S.reshape(6, -1), axis=1)
    onrm = np.linalg.norm(out.reshape(6, -1), axis=1)
    for i in range(6):
        if nrm[i] > tau:
            # capped: the Frobenius norm lands on tau (the 1e-6 inside the
            # square root moves it by tau * 5e-7 / ||S||^2 at most)
            assert abs(onrm[i] - tau) <= tau * 1e-6, (i, onrm[i])
            # the direction is kept: a positive multiple of S
            c = out[i] / S[i]
            assert np.allclose(c, c.flat[0], rtol=1e-13) and c.flat[0] > 0
        else:
            # below the cap the matrix comes back bit-identical
            assert np.array_equal(out[i], S[i]), i
    # each matrix is capped on its own norm: capping one alone gives the same
    for i in range(6):
        assert np.array_equal(O.frob_cap(S[i:i + 1], tau)[0], out[i])
    # idempotent up to the 1e-6 inside the square root (a relative change of
    # 5e-7 / tau^2), and the cap of a scaled matrix does not depend on the scale
    assert np.allclose(O.frob_cap(out, tau), out, rtol=1e-8, atol=0)
    assert np.allclose(O.frob_cap(S[:2] * 10.0, tau), out[:2], rtol=1e-9)


# ----------------------------------------------------------------------------
# fused prologue (gdn2.py:133-142): pinned by inverse functions.  Raw inputs
# built as graw = log(-g), braw = logit(b), wraw = logit(w) from activated
# targets must reproduce the unfused result on the targets; graw above 5
# saturates at g = -e^5.
# ----------------------------------------------------------------------------

def test_fused_prologue_by_inverse_functions():
    B, L, Hk, Hv, K = 1, 24, 1, 2, K_SMALL
    rng = np.random.default_rng(31)
    q, k = rng.standard_normal((2, B, L, Hk, K))
    v = rng.standard_normal((B, L, Hv, K))
    g_t = -rng.uniform(0.05, 3.0, (B, L, Hk, K))          # target decay in (-e^5, 0)
    b_t = rng.uniform(0.02, 0.98, (B, L, Hk, K))
    w_t = rng.uniform(0.02, 0.98, (B, L, Hv, K))
    graw = np.log(-g_t)
    braw = np.log(b_t) - np.log1p(-b_t)
    wraw = np.log(w_t) - np.log1p(-w_t)
    o1, s1 = O.chunk_gdn2(q, k, v, graw, braw, wraw, fuse_prologue=True, qk_l2norm=True, output_final_state=True)
    o2, s2 = O.chunk_gdn2(q, k, v, g_t, b_t, w_t, qk_l2norm=True, output_final_state=True)
    # the fused path normalises q / k in fp32 (gdn2.py:133-137)
    assert rel_l2(o1, o2) < 1e-6 and rel_l2(s1, s2) < 1e-6
    # saturation: every raw decay above 5 acts as 5, i.e. g = -e^5
    g_hi = graw.copy()
    g_hi[:, ::3] = 5.0 + rng.uniform(0.0, 40.0, g_hi[:, ::3].shape)
    g_5 = graw.copy()
    g_5[:, ::3] = 5.0
    oh, _ = O.chunk_gdn2(q, k, v, g_hi, braw, wraw, fuse_prologue=True, qk_l2norm=True)
    o5, _ = O.chunk_gdn2(q, k, v, g_5, braw, wraw, fuse_prologue=True, qk_l2norm=True)
    assert np.array_equal(oh, o5)
    g_t5 = g_t.copy()
    g_t5[:, ::3] = -np.exp(5.0)
    ot, _ = O.chunk_gdn2(q, k, v, g_t5, b_t, w_t, qk_l2norm=True)
    assert rel_l2(o5, ot) < 1e-6
    # large raw gates saturate the sigmoids at 0 / 1: braw -> -inf erases
    # nothing, wraw -> +inf writes the whole value
    o_sat, _ = O.chunk_gdn2(q, k, v, graw, np.full_like(braw, -60.0), np.full_like(wraw, 60.0),
                            fuse_prologue=True, qk_l2norm=True)
    o_ref, _ = O.chunk_gdn2(q, k, v, g_t, np.zeros_like(b_t), np.ones_like(w_t), qk_l2norm=True)
    assert rel_l2(o_sat, o_ref) < 1e-6


def test_fused_prologue_decay_saturation_level():
    # The saturated decay -e^5 is observable only through a state that is read
    # after it: write k0 v0^T at token 0 (w = 1, no erase), decay with a raw
    # gate above 5 at token 1, write nothing there (v1 = 0), and read.  Then
    # o1 / o0 = e^{-e^5} (q1 . k0) / (q0 . k0) per column, in float64.
    K = K_SMALL
    rng = np.random.default_rng(32)
    q, k = rng.standard_normal((2, 1, 2, 1, K))
    v = rng.standard_normal((1, 2, 1, K))
    v[:, 1] = 0.0
    graw = np.full((1, 2, 1, K), 7.0)
    braw = np.full((1, 2, 1, K), -np.inf)
    wraw = np.full((1, 2, 1, K), np.inf)
    o, _ = O.chunk_gdn2(q, k, v, graw, braw, wraw, fuse_prologue=True, qk_l2norm=True)
    q32, k32 = q.astype(np.float32).astype(np.float64), k.astype(np.float32).astype(np.float64)
    qn = q32[0, :, 0] / np.sqrt((q32[0, :, 0] ** 2).sum(-1, keepdims=True) + 1e-6)
    kn = k32[0, :, 0] / np.sqrt((k32[0, :, 0] ** 2).sum(-1, keepdims=True) + 1e-6)
    ratio = o[0, 1, 0] / o[0, 0, 0]
    expect = np.exp(-np.exp(5.0)) * (qn[1] @ kn[0]) / (qn[0] @ kn[0])
    assert np.allclose(ratio, expect, rtol=1e-9, atol=0)
