"""GPU parity of the decode step (gdn2_decode_step and variants) against the
oracle, mirroring the reference's test_inference.py:64-185, test_matrix.py
decode cases (367-428), test_variants.py decode cases and
test_streaming_and_stability.py:65-91."""

import numpy as np
import pytest
import torch

from deltanet_tpu_amd import (chunk_gdn2, delta_rule_decode_step, gdn2_decode_step, gdn2_decode_steps,
                              gdn_decode_step, gla_decode_step, kda_decode_step)
from oracle import gdn_oracle as O
from tests._util import rel_l2, sig
from tests.gpu_common import as_np, check, to_dev

pytestmark = pytest.mark.gpu


def dec_inputs(seed, B, Hk, Hv, g_shape="hk_k", b_shape="hk_k", w_shape="hv_v", four_d=True):
    rng = np.random.default_rng(seed)
    K = 128

    def gate(spec, last):
        heads, chan = spec.split("_")
        H = {"hk": Hk, "hv": Hv, "one": 1}[heads]
        shape = (B, H) if chan == "none" else (B, H, 1 if chan == "1" else last)
        return shape

    q = rng.standard_normal((B, Hk, K))
    k = rng.standard_normal((B, Hk, K))
    v = rng.standard_normal((B, Hv, K))
    g = -np.exp(rng.standard_normal(gate(g_shape, K)) - 1.0)
    b = sig(rng.standard_normal(gate(b_shape, K)))
    w = sig(rng.standard_normal(gate(w_shape, K)))
    if four_d:
        q, k, v = q[:, None], k[:, None], v[:, None]
        if g.ndim == 3:
            g = g[:, None]
        if b.ndim == 3:
            b = b[:, None]
        if w.ndim == 3:
            w = w[:, None]
    return q, k, v, g, b, w


@pytest.mark.parametrize("layout", [("hk_k", "hk_k", "hv_v"), ("hv_none", "hv_none", "hv_none"),
                                    ("hk_1", "hk_none", "hk_v"), ("one_k", "one_1", "one_none")])
@pytest.mark.parametrize("Hk,Hv", [(2, 2), (2, 4), (1, 4)])
@pytest.mark.parametrize("four_d", [True, False])
def test_decode_matrix(layout, Hk, Hv, four_d):
    B = 3
    q, k, v, g, b, w = dec_inputs(Hk * 7 + Hv, B, Hk, Hv, *layout, four_d=four_d)
    S = 0.1 * np.random.default_rng(1).standard_normal((B, Hv, 128, 128))
    reset = np.array([False, True, False])
    T = lambda x: to_dev(x)
    o, s = gdn2_decode_step(T(q), T(k), T(v), T(g), T(b), T(w), T(S), reset=torch.tensor(reset), qk_l2norm=True)
    ro, rs = O.decode_step(q, k, v, g, b, w, S, reset=reset, qk_l2norm=True)
    assert o.shape == ((B, 1, Hv, 128) if four_d else (B, Hv, 128))
    check(o.reshape(B, Hv, 128), ro, s, rs, "fp32", "fp32", f"decode {layout} {Hk}/{Hv} 4d={four_d}")


@pytest.mark.parametrize("state_dtype", [None, "bfloat16", torch.float32, torch.bfloat16])
def test_decode_state_dtype_contract(state_dtype):
    B, Hk, Hv = 2, 2, 4
    q, k, v, g, b, w = dec_inputs(3, B, Hk, Hv)
    S = 0.1 * np.random.default_rng(2).standard_normal((B, Hv, 128, 128))
    T = lambda x: to_dev(x)
    o, s = gdn2_decode_step(T(q), T(k), T(v), T(g), T(b), T(w), T(S), state_dtype=state_dtype)
    exp = torch.bfloat16 if state_dtype in ("bfloat16", torch.bfloat16) else torch.float32
    assert s.dtype == exp and o.dtype == torch.float32
    ro, rs = O.decode_step(q, k, v, g, b, w, S)
    tol = 1e-2 if exp == torch.bfloat16 else 1e-5
    assert rel_l2(as_np(s), rs) < tol
    if state_dtype is None:
        # test_inference.py:150-154: with no state_dtype a bf16 state comes back as float32
        _, s2 = gdn2_decode_step(T(q), T(k), T(v), T(g), T(b), T(w), T(S).to(torch.bfloat16))
        assert s2.dtype == torch.float32


@pytest.mark.parametrize("guard", [False, True])
def test_decode_bf16_state_in_fp32_state_out(guard):
    # a bf16 state read and an fp32 state written: the kernel's column layout
    # follows the input format, the store widens it
    B, Hk, Hv = 3, 2, 4
    q, k, v, g, b, w = dec_inputs(8, B, Hk, Hv)
    S = 0.1 * np.random.default_rng(6).standard_normal((B, Hv, 128, 128))
    T = lambda x: to_dev(x)
    s16 = T(S).to(torch.bfloat16)
    o, s = gdn2_decode_step(T(q), T(k), T(v), T(g), T(b), T(w), s16, reset=torch.tensor([False, True, False]),
                            state_dtype=torch.float32, stability_guard=guard, stability_tau=5.0)
    assert s.dtype == torch.float32
    ro, rs = O.decode_step(q, k, v, g, b, w, as_np(s16), reset=[False, True, False],
                           stability_guard=guard, stability_tau=5.0)
    check(o.reshape(B, Hv, 128), ro, s, rs, "fp32", "fp32", f"decode bf16->fp32 guard={guard}")


def test_decode_bf16_state_tracks_fp32_over_10_steps():
    # test_inference.py:150-185
    B, Hk, Hv = 2, 2, 4
    T = lambda x: to_dev(x)
    S0 = 0.02 * np.random.default_rng(3).standard_normal((B, Hv, 128, 128))
    s32 = T(S0)
    s16 = T(S0).to(torch.bfloat16)
    for t in range(10):
        q, k, v, g, b, w = dec_inputs(100 + t, B, Hk, Hv)
        args = [T(x) for x in (q, k, v, g, b, w)]
        o32, s32 = gdn2_decode_step(*args, s32, qk_l2norm=True)
        o16, s16 = gdn2_decode_step(*args, s16, qk_l2norm=True, state_dtype="bfloat16")
    assert rel_l2(as_np(s16), as_np(s32)) < 1e-2
    assert rel_l2(as_np(o16), as_np(o32)) < 1e-2


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_decode_steps_equal_chunk_gdn2_with_reset(dtype):
    # test_inference.py:64-110
    B, N, Hk, Hv = 1, 128, 2, 4
    rng = np.random.default_rng(101)
    tdt = torch.float32 if dtype == "fp32" else torch.bfloat16
    q = to_dev(0.1 * rng.standard_normal((B, N, Hk, 128)), tdt)
    k = to_dev(0.1 * rng.standard_normal((B, N, Hk, 128)), tdt)
    v = to_dev(0.1 * rng.standard_normal((B, N, Hv, 128)), tdt)
    g = to_dev(-np.exp(rng.standard_normal((B, N, Hk, 128)) - 1.0))
    b = to_dev(sig(rng.standard_normal((B, N, Hk, 128))))
    w = to_dev(sig(rng.standard_normal((B, N, Hv, 128))))
    reset_idx = N // 2
    seg = to_dev((np.arange(N) >= reset_idx)[None], torch.int32)
    out_c, st_c = chunk_gdn2(q, k, v, g, b, w, segment_ids=seg, is_inference=True, output_final_state=True,
                             precision=dtype)
    state = torch.zeros(B, Hv, 128, 128, device="cuda:0")
    outs = []
    for t in range(N):
        ot, state = gdn2_decode_step(q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1], g[:, t:t + 1], b[:, t:t + 1],
                                     w[:, t:t + 1], state, reset=(t == reset_idx))
        outs.append(ot)
    tol = 1e-4 if dtype == "fp32" else 1e-2
    assert rel_l2(as_np(torch.cat(outs, 1)), as_np(out_c)) < tol
    assert rel_l2(as_np(state), as_np(st_c)) < tol


def test_decode_stability_guard():
    # test_streaming_and_stability.py:65-91: the returned state is capped, the
    # output of the step uses the uncapped state
    B, Hk, Hv = 2, 2, 4
    q, k, v, g, b, w = dec_inputs(5, B, Hk, Hv)
    S = 10.0 * np.random.default_rng(4).standard_normal((B, Hv, 128, 128))
    S[:, 1] *= 0.01   # value head 1 stays below the cap
    T = lambda x: to_dev(x)
    tau = 100.0
    o, s = gdn2_decode_step(T(q), T(k), T(v), T(g), T(b), T(w), T(S), stability_guard=True, stability_tau=tau)
    # independently: the guard's gate clamps by hand, no guard, then the cap
    # must put capped heads on ||S||_F = tau along the uncapped direction and
    # leave the others bit-identical (gdn2.py:2484-2487)
    o_unc, s_unc = gdn2_decode_step(T(q), T(k), T(v), T(np.minimum(g, -1e-6)), T(np.maximum(b, 0.0)), T(w), T(S))
    n_unc = torch.linalg.vector_norm(s_unc.double(), dim=(-2, -1))
    norms = torch.linalg.vector_norm(s.double(), dim=(-2, -1))
    capped = n_unc > tau
    assert bool(capped.any()) and bool((~capped).any())
    assert torch.allclose(norms[capped], torch.full_like(norms[capped], tau), rtol=1e-5, atol=0)
    scale = tau / torch.sqrt(n_unc ** 2 + 1e-6)
    assert torch.allclose(s.double()[capped], (s_unc.double() * scale[..., None, None])[capped], rtol=1e-5,
                          atol=1e-6 * tau / 128)
    assert torch.equal(s[~capped], s_unc[~capped])
    # the step's output uses the uncapped state
    assert torch.equal(o, o_unc)
    ro, rs = O.decode_step(q, k, v, g, b, w, S, stability_guard=True, stability_tau=tau)
    check(o.reshape(B, Hv, 128), ro, s, rs, "fp32", "fp32", "decode guard")


def test_decode_in_place_state():
    B, Hk, Hv = 2, 2, 4
    q, k, v, g, b, w = dec_inputs(6, B, Hk, Hv)
    S = 0.1 * np.random.default_rng(5).standard_normal((B, Hv, 128, 128))
    T = lambda x: to_dev(x)
    st = T(S)
    o1, s1 = gdn2_decode_step(T(q), T(k), T(v), T(g), T(b), T(w), st)
    o2, s2 = gdn2_decode_step(T(q), T(k), T(v), T(g), T(b), T(w), st, out_state=st)
    assert s2.data_ptr() == st.data_ptr()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)


@pytest.mark.parametrize("variant", ["gdn", "kda", "gla", "delta"])
def test_decode_variants(variant):
    B, Hk, Hv = 2, 2, 4
    rng = np.random.default_rng(7)
    q, k = rng.standard_normal((2, B, 1, Hk, 128))
    v = rng.standard_normal((B, 1, Hv, 128))
    S = 0.1 * rng.standard_normal((B, Hv, 128, 128))
    T = lambda x: to_dev(x)
    beta = sig(rng.standard_normal((B, 1, Hv)))
    if variant == "gdn":
        g = -np.exp(rng.standard_normal((B, 1, Hv)))
        o, s = gdn_decode_step(T(q), T(k), T(v), T(g), T(beta), T(S), qk_l2norm=True)
        ro, rs = O.gdn_decode_step(q, k, v, g, beta, S, qk_l2norm=True)
    elif variant == "kda":
        g = -np.exp(rng.standard_normal((B, 1, Hk, 128)))
        o, s = kda_decode_step(T(q), T(k), T(v), T(g), T(beta), T(S), qk_l2norm=True)
        ro, rs = O.gdn_decode_step(q, k, v, g, beta, S, qk_l2norm=True)
    elif variant == "gla":
        g = -np.exp(rng.standard_normal((B, 1, Hk, 128)))
        o, s = gla_decode_step(T(q), T(k), T(v), T(g), T(S), qk_l2norm=True)
        ro, rs = O.decode_step(q, k, v, g, np.zeros((B, 1)), np.ones((B, 1)), S, qk_l2norm=True)
    else:
        o, s = delta_rule_decode_step(T(q), T(k), T(v), T(beta), T(S), qk_l2norm=True)
        ro, rs = O.decode_step(q, k, v, np.zeros((B, 1)), beta[:, 0], beta[:, 0], S, qk_l2norm=True)
    check(o.reshape(B, Hv, 128), ro, s, rs, "fp32", "fp32", f"decode {variant}")


def steps_inputs(seed, B, T, Hk, Hv, gate_heads="hk"):
    rng = np.random.default_rng(seed)
    Hg = Hk if gate_heads == "hk" else Hv
    q = rng.standard_normal((B, T, Hk, 128))
    k = rng.standard_normal((B, T, Hk, 128))
    v = rng.standard_normal((B, T, Hv, 128))
    g = -np.exp(0.39 * rng.standard_normal((B, T, Hg, 128)) - 1)
    b = sig(0.39 * rng.standard_normal((B, T, Hg, 128)))
    w = sig(0.39 * rng.standard_normal((B, T, Hv, 128)))
    return q, k, v, g, b, w


def chain_oracle(q, k, v, g, b, w, S0, reset, **kw):
    """T chained oracle steps (float64, no rounding between tokens)."""
    ref_s, ro = S0, []
    for t in range(q.shape[1]):
        o1, ref_s = O.decode_step(q[:, t], k[:, t], v[:, t], g[:, t], b[:, t], w[:, t], ref_s,
                                  reset=reset[:, t], **kw)
        ro.append(o1)
    return np.stack(ro, 1), ref_s


@pytest.mark.parametrize("state_dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("guard", [False, True])
@pytest.mark.parametrize("T", [5, 20])
def test_decode_steps_equal_chained_steps(state_dtype, guard, T):
    # one launch over T tokens == T chained single steps (per-token resets,
    # stability cap after every token).  T = 5 and launches with the guard run
    # the per-token kernel; T = 20 without it runs two 16-token chunks in the
    # WY form, a reset inside each.
    B, Hk, Hv = 3, 2, 4
    q, k, v, g, b, w = steps_inputs(31, B, T, Hk, Hv)
    S0 = 0.3 * np.random.default_rng(32).standard_normal((B, Hv, 128, 128))
    reset = np.zeros((B, T), bool)
    reset[1, 0] = reset[2, 3] = True
    if T > 16:
        reset[0, 17] = True
    tb = lambda x: to_dev(x, torch.bfloat16)
    st0 = to_dev(S0)
    if state_dtype == "bfloat16":
        st0 = st0.to(torch.bfloat16)
    kw = dict(qk_l2norm=True, state_dtype=state_dtype, stability_guard=guard, stability_tau=20.0)
    o_m, s_m = gdn2_decode_steps(tb(q), tb(k), tb(v), to_dev(g), to_dev(b), to_dev(w), st0,
                                 reset=torch.tensor(reset), **kw)
    st = st0
    outs = []
    for t in range(T):
        o1, st = gdn2_decode_step(tb(q[:, t]), tb(k[:, t]), tb(v[:, t]), to_dev(g[:, t]), to_dev(b[:, t]),
                                  to_dev(w[:, t]), st, reset=torch.tensor(reset[:, t]), **kw)
        outs.append(o1)
    o_c = torch.stack(outs, 1)
    assert o_m.shape == (B, T, Hv, 128) and o_m.dtype == torch.bfloat16
    assert s_m.dtype == st.dtype
    ro, rs = rel_l2(as_np(o_m), as_np(o_c)), rel_l2(as_np(s_m), as_np(st))
    print(f"multi vs chained T={T}: out {ro:.2e} state {rs:.2e}")
    if state_dtype == "bfloat16":
        if T < 6 or guard:
            # the per-token kernel rounds the state after every token, as the
            # chained steps do: the same values up to the summation order
            assert ro < 2e-4 and rs < 2e-4
        else:
            # the chunked launch rounds the state once, the chained steps
            # after every token: they agree at the bf16 rounding level
            assert ro < 1e-2 and rs < 1e-2
        # and either stays within bf16 rounding of the unrounded recurrence
        bfr = lambda x: O.bf16_round(x).astype(np.float64)
        ref_o, ref_s = chain_oracle(bfr(q), bfr(k), bfr(v), g, b, w, as_np(st0).astype(np.float64), reset,
                                    qk_l2norm=True, stability_guard=guard, stability_tau=20.0)
        eo, es = rel_l2(as_np(o_m), ref_o), rel_l2(as_np(s_m), ref_s)
        print(f"multi vs unrounded oracle: out {eo:.2e} state {es:.2e}")
        assert eo < 4e-3 and es < 4e-3
    else:
        # the same recurrence, the sums in another order (and, for the chunked
        # form, another association): fp32 results a few roundings apart; a
        # bf16-rounded output may land one bf16 step apart
        a, c = as_np(o_m).astype(np.float64), as_np(o_c).astype(np.float64)
        assert np.all(np.abs(a - c) <= 2.0 ** -7 * np.abs(c) + 1e-6 * np.abs(c).max())
        assert rs < 1e-5


@pytest.mark.parametrize("gate_heads", ["hk", "hv"])
def test_decode_steps_vs_oracle(gate_heads):
    B, T, Hk, Hv = 2, 8, 2, 4
    q, k, v, g, b, w = steps_inputs(33, B, T, Hk, Hv, gate_heads)
    S0 = 0.1 * np.random.default_rng(34).standard_normal((B, Hv, 128, 128))
    reset = np.zeros((B, T), bool)
    reset[0, 5] = True
    o, s = gdn2_decode_steps(to_dev(q), to_dev(k), to_dev(v), to_dev(g), to_dev(b), to_dev(w), to_dev(S0),
                             reset=torch.tensor(reset), qk_l2norm=True)
    ref_s = S0
    ro = []
    for t in range(T):
        o1, ref_s = O.decode_step(q[:, t], k[:, t], v[:, t], g[:, t], b[:, t], w[:, t], ref_s,
                                  reset=reset[:, t], qk_l2norm=True)
        ro.append(o1)
    ro = np.stack(ro, 1)
    check(o.reshape(B, T * Hv, 128), ro.reshape(B, T * Hv, 128), s, ref_s, "fp32", "fp32", f"decode_steps {gate_heads}")


def test_decode_steps_in_place_and_single_token():
    B, Hk, Hv = 2, 2, 4
    q, k, v, g, b, w = steps_inputs(35, B, 1, Hk, Hv)
    S0 = 0.1 * np.random.default_rng(36).standard_normal((B, Hv, 128, 128))
    args = [to_dev(x) for x in (q, k, v, g, b, w)]
    o1, s1 = gdn2_decode_step(*[x[:, 0] for x in args], to_dev(S0), qk_l2norm=True)
    st = to_dev(S0)
    o2, s2 = gdn2_decode_steps(*args, st, qk_l2norm=True, out_state=st)
    assert s2.data_ptr() == st.data_ptr()
    assert torch.equal(o1, o2[:, 0]) and torch.equal(s1, s2)


@pytest.mark.parametrize("state_dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("B,Hk,Hv", [(3, 1, 1), (1, 1, 3), (5, 1, 3)])
def test_decode_odd_matrix_count(state_dtype, B, Hk, Hv):
    # an odd number of (batch, value head) state matrices: the last workgroup
    # of the two-matrices-per-workgroup fp32 kernel has an idle second half;
    # every matrix (the last one included) must match the oracle, and the
    # in-place call (out_state = state) must give the same bits
    q, k, v, g, b, w = dec_inputs(90 + B * Hv, B, Hk, Hv)
    S = 0.1 * np.random.default_rng(91).standard_normal((B, Hv, 128, 128))
    reset = np.zeros(B, bool)
    reset[-1] = B > 1
    T = lambda x: to_dev(x)
    sdt = torch.float32 if state_dtype == "float32" else torch.bfloat16
    S_in = to_dev(S, sdt)
    S_ref = as_np(S_in)   # the oracle starts from the stored (possibly bf16) state
    kw = dict(reset=torch.tensor(reset), qk_l2norm=True, state_dtype=state_dtype)
    o, s = gdn2_decode_step(T(q), T(k), T(v), T(g), T(b), T(w), S_in, **kw)
    ro, rs = O.decode_step(q, k, v, g, b, w, S_ref, reset=reset, qk_l2norm=True)
    if state_dtype == "float32":
        check(o.reshape(B, Hv, 128), ro, s, rs, "fp32", "fp32", f"odd decode B={B} Hv={Hv}")
    else:
        assert rel_l2(as_np(o).reshape(B, Hv, 128), ro) < 1e-2
        assert rel_l2(as_np(s), rs) < 1e-2
        # every matrix, the last one included, is written
        for i in range(B):
            assert rel_l2(as_np(s)[i], rs[i]) < 1e-2
    st = S_in.clone()
    o2, s2 = gdn2_decode_step(T(q), T(k), T(v), T(g), T(b), T(w), st, out_state=st, **kw)
    assert s2.data_ptr() == st.data_ptr()
    assert torch.equal(o, o2) and torch.equal(s, s2)


@pytest.mark.parametrize("state_dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("B,Hk,Hv", [(3, 1, 1), (1, 1, 3)])
@pytest.mark.parametrize("Tn", [4, 12])
def test_decode_steps_odd_matrix_count(state_dtype, B, Hk, Hv, Tn):
    # T tokens in one launch with an odd number of state matrices: equal to
    # T chained single steps up to the summation order (the kernels split the
    # state rows differently over lanes; Tn = 12 runs the chunked form, which
    # rounds a bf16 state once instead of after every token), and the fp32
    # run to the oracle
    q, k, v, g, b, w = steps_inputs(92 + B, B, Tn, Hk, Hv)
    S0 = 0.3 * np.random.default_rng(93).standard_normal((B, Hv, 128, 128))
    reset = np.zeros((B, Tn), bool)
    reset[-1, 2] = True
    sdt = torch.float32 if state_dtype == "float32" else torch.bfloat16
    args = [to_dev(x) for x in (q, k, v, g, b, w)]
    kw = dict(qk_l2norm=True, state_dtype=state_dtype)
    o_m, s_m = gdn2_decode_steps(*args, to_dev(S0, sdt), reset=torch.tensor(reset), **kw)
    st = to_dev(S0, sdt)
    outs = []
    for t in range(Tn):
        o1, st = gdn2_decode_step(*[x[:, t] for x in args], st, reset=torch.tensor(reset[:, t]), **kw)
        outs.append(o1)
    ro, rs = rel_l2(as_np(o_m), as_np(torch.stack(outs, 1))), rel_l2(as_np(s_m), as_np(st))
    print(f"odd multi vs chained: out {ro:.2e} state {rs:.2e}")
    bound = (2e-4 if Tn < 6 else 1e-2) if state_dtype == "bfloat16" else (1e-6 if Tn < 6 else 1e-5)
    assert ro < bound and rs < bound
    # every matrix, the last one included, carries its own state
    for i in range(B):
        assert rel_l2(as_np(s_m)[i], as_np(st)[i]) < bound
    if state_dtype == "float32":
        ref_s = S0
        for t in range(Tn):
            o1, ref_s = O.decode_step(q[:, t], k[:, t], v[:, t], g[:, t], b[:, t], w[:, t], ref_s,
                                      reset=reset[:, t], qk_l2norm=True)
        check(o_m[:, -1].reshape(B, Hv, 128), o1, s_m, ref_s, "fp32", "fp32", f"odd decode_steps B={B} Hv={Hv}")


# Launches of 8 or more tokens without the stability guard run 16-token chunks
# in the WY form: parity with the float64 token-by-token oracle across ragged
# chunk counts, resets at and inside chunk boundaries, gate layouts and dtypes,
# no L2 norm, and a decay strong enough to take the one-exponential-per-pair
# path for A and M (a chunk's decay span above 80 nats).  Seeds are fixed per
# case: without the L2 norm the state grows to ~1e8 (each token's transition
# has an eigenvalue near 1 - b |k|^2 ~ -63), and for some seeds a plain fp32
# token-by-token recurrence is itself ~2e-4 max-abs/rms from float64.
CHUNK_CASES = {
    "T6_hk": dict(seed=504, T=6, gates="hk"),
    "T8_hk": dict(seed=505, T=8, gates="hk"),
    "T16_hv_resets": dict(seed=500, T=16, gates="hv", resets=[(0, 0), (1, 7), (1, 15)]),
    "T37_scalar": dict(seed=503, T=37, gates="scalar", resets=[(0, 16), (1, 20), (1, 21)]),
    "T24_no_l2norm_f16_gates": dict(seed=502, T=24, gates="hk", l2norm=False, scale=0.2, gate_dtype="f16"),
    "T19_strong_decay": dict(seed=501, T=19, gates="hv", strong=True, resets=[(1, 9)]),
    "T12_one_head_gates": dict(seed=506, T=12, gates="one", resets=[(1, 3)]),
}


@pytest.mark.parametrize("state_dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("case", sorted(CHUNK_CASES))
def test_decode_steps_chunked_vs_oracle(case, state_dtype):
    c = CHUNK_CASES[case]
    B, Hk, Hv, T = 2, 2, 4, c["T"]
    seed = c["seed"]
    rng = np.random.default_rng(seed)
    q, k, v, g, b, w = steps_inputs(seed, B, T, Hk, Hv, "hv" if c["gates"] == "hv" else "hk")
    if c["gates"] == "one":   # one channel-wise gate head shared by every head
        g = -np.exp(0.39 * rng.standard_normal((B, T, 1, 128)) - 1)
        b = sig(0.39 * rng.standard_normal((B, T, 1, 128)))
        w = sig(0.39 * rng.standard_normal((B, T, 1, 128)))
    if c["gates"] == "scalar":
        g = -np.exp(0.39 * rng.standard_normal((B, T, Hv)) - 1)
        b = sig(0.39 * rng.standard_normal((B, T, Hv)))
        w = sig(0.39 * rng.standard_normal((B, T, Hv)))
    if c.get("strong"):
        g = -np.exp(rng.uniform(0, np.log(40.0), g.shape))   # up to 40 nats per token
    reset = np.zeros((B, T), bool)
    for bi, ti in c.get("resets", []):
        reset[bi, ti] = True
    S0 = 0.2 * rng.standard_normal((B, Hv, 128, 128))
    sdt = torch.float32 if state_dtype == "float32" else torch.bfloat16
    gdt = torch.float16 if c.get("gate_dtype") == "f16" else torch.float32
    if gdt == torch.float16:
        g, b, w = (x.astype(np.float16).astype(np.float64) for x in (g, b, w))
    kw = dict(qk_l2norm=c.get("l2norm", True))
    if "scale" in c:
        kw["scale"] = c["scale"]
    st0 = to_dev(S0, sdt)
    o, s = gdn2_decode_steps(to_dev(q), to_dev(k), to_dev(v), to_dev(g, gdt), to_dev(b, gdt), to_dev(w, gdt),
                             st0, reset=torch.tensor(reset), state_dtype=state_dtype, **kw)
    ro, rs = chain_oracle(q, k, v, g, b, w, as_np(st0).astype(np.float64), reset, **kw)
    prec = "fp32" if state_dtype == "float32" else "bf16"
    check(o.reshape(B, T * Hv, 128), ro.reshape(B, T * Hv, 128), s, rs, prec, "fp32",
          f"decode_steps chunked {case} {state_dtype}")


# 16-bit inputs: the decode kernels read a token's elements as words through
# a bounds-checked resource per row, so this covers odd element indices (the
# high half of a word), rows that start 2 bytes into a word (one-head,
# one-channel 16-bit gates at odd batch rows), bf16 / f16 q, k, v and a reset
# on an odd row, on the single-step kernel (T = 1) and the per-token kernel
# (T = 4), against the float64 oracle.
@pytest.mark.parametrize("T", [1, 4])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_decode_16bit_inputs_and_word_offsets(T, dt):
    B, Hk, Hv = 3, 2, 4
    rng = np.random.default_rng(900 + 2 * T + (dt == "f16"))
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    stored = lambda x: as_np(to_dev(x, tdt)).astype(np.float64)   # values as the device holds them
    q = stored(rng.standard_normal((B, T, Hk, 128)))
    k = stored(rng.standard_normal((B, T, Hk, 128)))
    v = stored(rng.standard_normal((B, T, Hv, 128)))
    g = stored(-np.exp(0.39 * rng.standard_normal((B, T, 1)) - 1))   # one head, one channel
    b = stored(sig(0.39 * rng.standard_normal((B, T, Hk))))          # key heads, one channel
    w = stored(sig(0.39 * rng.standard_normal((B, T, Hv, 128))))     # value heads, channel-wise
    S0 = 0.2 * rng.standard_normal((B, Hv, 128, 128))
    reset = np.zeros((B, T), bool)
    reset[1, T - 1] = True
    o, s = gdn2_decode_steps(*(to_dev(x, tdt) for x in (q, k, v, g, b, w)), to_dev(S0),
                             reset=torch.tensor(reset), qk_l2norm=True)
    assert o.dtype == tdt
    ro, rs = chain_oracle(q, k, v, g, b, w, S0, reset, qk_l2norm=True)
    check(o.reshape(B, T * Hv, 128), ro.reshape(B, T * Hv, 128), s, rs, "fp32", "bf16",
          f"decode 16-bit inputs T={T} {dt}")


# tests/test_matrix.py:367-429: every decode step x batch {1, 2} x heads
# {(2, 2), (2, 4)} x reset of the first row x decay negative / zero /
# positive (clamped), 3-D inputs, b at key heads and w at value heads with
# one channel; output and state within rel L2 1e-4 of the float64 oracle
@pytest.mark.parametrize("step_name", ["gdn2", "gdn", "kda", "gla", "delta_rule"])
@pytest.mark.parametrize("B", [1, 2])
@pytest.mark.parametrize("Hk,Hv", [(2, 2), (2, 4)])
@pytest.mark.parametrize("has_reset", [False, True])
@pytest.mark.parametrize("g_regime", ["negative", "zero", "positive"])
def test_decode_step_matrix(step_name, B, Hk, Hv, has_reset, g_regime):
    from deltanet_tpu_amd import gdn_decode_step, gla_decode_step, kda_decode_step
    rng = np.random.default_rng(77)
    q = 0.1 * rng.standard_normal((B, Hk, 128))
    k = 0.1 * rng.standard_normal((B, Hk, 128))
    v = 0.1 * rng.standard_normal((B, Hv, 128))
    S = 0.05 * rng.standard_normal((B, Hv, 128, 128))
    reset = np.array([True] + [False] * (B - 1)) if has_reset else None
    if g_regime == "negative":
        g = -rng.uniform(0.1, 2.0, (B, Hk, 128))
    elif g_regime == "zero":
        g = np.zeros((B, Hk, 128))
    else:
        g = rng.uniform(0.1, 1.0, (B, Hk, 128))
    b = sig(0.39 * rng.standard_normal((B, Hk, 1)))
    w = sig(0.39 * rng.standard_normal((B, Hv, 1)))
    T = lambda x: to_dev(x)
    kw = dict(reset=torch.tensor(reset) if reset is not None else None)
    if step_name == "gdn2":
        o, s = gdn2_decode_step(T(q), T(k), T(v), T(g), T(b), T(w), T(S), **kw)
        ro, rs = O.decode_step(q, k, v, g, b, w, S, reset=reset)
    elif step_name == "gdn":
        o, s = gdn_decode_step(T(q), T(k), T(v), T(g[:, :, :1]), T(b), T(S), **kw)
        ro, rs = O.gdn_decode_step(q, k, v, g[:, :, :1], b, S, reset=reset)
    elif step_name == "kda":
        o, s = kda_decode_step(T(q), T(k), T(v), T(g), T(b), T(S), **kw)
        ro, rs = O.decode_step(q, k, v, g, b, b, S, reset=reset)
    elif step_name == "gla":
        o, s = gla_decode_step(T(q), T(k), T(v), T(g), T(S), **kw)
        ro, rs = O.decode_step(q, k, v, g, np.zeros((B, Hk, 1)), np.ones((B, Hv, 1)), S, reset=reset)
    else:
        o, s = delta_rule_decode_step(T(q), T(k), T(v), T(b), T(S), **kw)
        ro, rs = O.decode_step(q, k, v, np.zeros((B, Hk, 128)), b, b, S, reset=reset)
    eo, es = rel_l2(as_np(o).reshape(ro.shape), ro), rel_l2(as_np(s), rs)
    assert eo < 1e-4 and es < 1e-4, (step_name, eo, es)


@pytest.mark.parametrize("Hk,Hv", [(1, 2), (1, 1)])
def test_decode_step_equals_one_token_prefill(Hk, Hv):
    # tests/test_variants.py:421-481: with one key head, every decode step
    # equals the matching one-token chunk call (decode and prefill kernels
    # agree), output and state within rel L2 1e-5
    import deltanet_tpu_amd as D
    B = 1
    rng = np.random.default_rng(980)
    q, k = rng.standard_normal((2, B, Hk, 128))
    v = rng.standard_normal((B, Hv, 128))
    g = -np.exp(rng.standard_normal((B, Hk, 128)) - 1.0)
    b = sig(0.39 * rng.standard_normal((B, Hk, 128)))
    w = sig(0.39 * rng.standard_normal((B, Hv, 128)))
    beta = sig(0.39 * rng.standard_normal((B, Hk, 1)))
    S = to_dev(0.05 * rng.standard_normal((B, Hv, 128, 128)))
    T = lambda x: to_dev(x)
    T1 = lambda x: to_dev(x[:, None])
    kw = dict(initial_state=S, output_final_state=True, precision="fp32")
    pairs = [
        (D.gdn2_decode_step(T(q), T(k), T(v), T(g), T(b), T(w), S), D.chunk_gdn2(*(T1(x) for x in (q, k, v, g, b, w)), **kw)),
        (D.gdn_decode_step(T(q), T(k), T(v), T(g[:, :, :1]), T(beta), S), D.chunk_gdn(*(T1(x) for x in (q, k, v, g[:, :, :1], beta)), **kw)),
        (D.kda_decode_step(T(q), T(k), T(v), T(g), T(beta), S), D.chunk_kda(*(T1(x) for x in (q, k, v, g, beta)), **kw)),
        (D.gla_decode_step(T(q), T(k), T(v), T(g), S), D.chunk_gla(*(T1(x) for x in (q, k, v, g)), **kw)),
        (D.delta_rule_decode_step(T(q), T(k), T(v), T(beta), S), D.chunk_delta_rule(*(T1(x) for x in (q, k, v, beta)), **kw)),
    ]
    for name, ((od, sd), (oc, sc)) in zip(("gdn2", "gdn", "kda", "gla", "delta_rule"), pairs):
        eo = rel_l2(as_np(od).reshape(B, Hv, 128), as_np(oc)[:, 0])
        es = rel_l2(as_np(sd), as_np(sc))
        assert eo < 1e-5 and es < 1e-5, (name, eo, es)


def test_decode_guard_caps_a_large_state():
    # test_streaming_and_stability.py:65-90: negative erase gate, positive
    # decay and a state of 100 everywhere; with the guard every head's
    # Frobenius norm ends at most tau, and equals the oracle's
    B, Hk, Hv = 1, 2, 2
    rng = np.random.default_rng(1234)
    q, k = rng.standard_normal((2, B, Hk, 128))
    v = rng.standard_normal((B, Hv, 128))
    b = np.full((B, Hk, 128), -0.5)
    g = np.full((B, Hk, 128), 0.5)
    w = np.ones((B, Hv, 128))
    S = np.full((B, Hv, 128, 128), 100.0)
    T = lambda x: to_dev(x)
    o, s = gdn2_decode_step(T(q), T(k), T(v), T(g), T(b), T(w), T(S), stability_guard=True, stability_tau=50.0)
    norms = np.linalg.norm(as_np(s), axis=(-2, -1))
    assert norms.max() <= 50.0 + 1e-2
    ro, rs = O.decode_step(q, k, v, g, b, w, S, stability_guard=True, stability_tau=50.0)
    assert rel_l2(as_np(s), rs) < 1e-5 and rel_l2(as_np(o).reshape(ro.shape), ro) < 1e-5
