"""GPU parity of chunk_gdn2 / chunk_gdn prefill (HIP path through the C ABI)
against the float64 oracle, mirroring the reference's tests:
test_parity.py, test_arbitrary_lengths.py, test_matrix.py (gate layouts x head
ratios x documents x initial state), test_doc_reset_and_streaming.py,
test_document_boundaries.py, test_state_passing.py, test_inference.py,
test_streaming_and_stability.py, test_causality.py, test_strong_decay.py,
test_nan_adversarial.py and test_variants.py (forward parts)."""

import numpy as np
import pytest
import torch

from deltanet_tpu_amd import chunk_delta_rule, chunk_gdn, chunk_gdn2, chunk_gla, chunk_kda
from oracle import gdn_oracle as O
from tests._util import make_inputs, rel_l2, sig
from tests.gpu_common import TDT, as_np, check, oracle_prefill, round_in, to_dev

pytestmark = pytest.mark.gpu


def run_pair(q, k, v, g, b, w, *, dt="fp32", precision="fp32", seg=None, init=None, use_c=False, **kw):
    """Run the device path and the oracle on the same inputs; return both."""
    out, st = chunk_gdn2(to_dev(q, TDT[dt]), to_dev(k, TDT[dt]), to_dev(v, TDT[dt]), to_dev(g), to_dev(b),
                         to_dev(w), segment_ids=to_dev(seg, torch.int32) if seg is not None else None,
                         initial_state=to_dev(init), output_final_state=True, is_inference=True,
                         precision=precision, **kw)
    torch.cuda.synchronize()
    ro, rs = oracle_prefill(round_in(q, dt), round_in(k, dt), round_in(v, dt), g, b, w, segment_ids=seg,
                            initial_state=init, output_final_state=True, qk_dtype=dt, use_c=use_c, **kw)
    return out, st, ro, rs


@pytest.mark.parametrize("precision,dt", [("fp32", "fp32"), ("bf16", "fp32"), ("bf16", "bf16")])
@pytest.mark.parametrize("L", [1, 127, 128, 300, 1000])
def test_parity_lengths(precision, dt, L):
    q, k, v, g, b, w = make_inputs(42 + L, 1, L, 2, 4)
    out, st, ro, rs = run_pair(q, k, v, g, b, w, dt=dt, precision=precision, qk_l2norm=True)
    check(out, ro, st, rs, precision, dt, f"L={L} {precision}/{dt}")


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_no_l2norm_with_scale(precision):
    q, k, v, g, b, w = make_inputs(5, 1, 256, 2, 4, qscale=0.1)
    out, st, ro, rs = run_pair(q, k, v, g, b, w, precision=precision, scale=0.5)
    check(out, ro, st, rs, precision, "fp32", f"scale=0.5 {precision}")


GATE_LAYOUTS = [
    ("channel_hk", "channel_hk", "channel_hv"),   # GDN-2 (value-head fusion)
    ("scalar_hk", "rank3_hk", "rank3_hv"),        # scalar gates at Hk
    ("rank3_hv", "rank3_hv", "rank3_hv"),         # Qwen3.5-4B / Qwen3-Next: gates at Hv
    ("channel_hv", "channel_hk", "channel_hk"),   # decay at Hv, erase at Hk, write at Hk
    ("channel_one", "rank3_one", "scalar_one"),   # single-head gates
]


@pytest.mark.parametrize("layout", GATE_LAYOUTS, ids=lambda x: "-".join(x))
@pytest.mark.parametrize("Hk,Hv", [(2, 2), (1, 2), (2, 6)])
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_matrix_gate_layouts(layout, Hk, Hv, precision):
    gl, bl, wl = layout
    B, L = 2, 300
    q, k, v, g, b, w = make_inputs(hash((gl, Hk, Hv)) % 1000, B, L, Hk, Hv, g_layout=gl, b_layout=bl, w_layout=wl)
    seg = np.stack([np.repeat([0, 1, 2], [100, 120, 80]), np.repeat([3, 3, 4], [50, 150, 100])])
    init = 0.05 * np.random.default_rng(0).standard_normal((B, Hv, 128, 128))
    out, st, ro, rs = run_pair(q, k, v, g, b, w, precision=precision, seg=seg, init=init, qk_l2norm=True)
    check(out, ro, st, rs, precision, "fp32", f"{layout} Hk={Hk} Hv={Hv} {precision}")


# One decay and one b per (token, head) with bf16 q / k in precision "bf16"
# takes the scalar-gate prepass (Gram products on the normalised bf16 rows,
# one exponential per token pair): its edge cases against the oracle.
SCALAR_CASES = {
    "hv_docs_init": dict(L=300, layout=("rank3_hv", "rank3_hv", "rank3_hv"), docs=True, init=True),
    "hk_gates": dict(L=384, layout=("rank3_hk", "rank3_hk", "channel_hv"), docs=True),
    "scalar4d_one": dict(L=129, layout=("scalar_hv", "scalar_one", "rank3_hv")),
    "one_token": dict(L=1, layout=("rank3_hv", "rank3_hv", "rank3_hv"), init=True),
    "no_l2norm": dict(L=256, layout=("rank3_hv", "rank3_hv", "rank3_hv"), l2norm=False, scale=0.3, qscale=0.1),
    "guard": dict(L=520, layout=("rank3_hv", "rank3_hv", "rank3_hv"), docs=True, init=True, guard=True),
    "strong_decay": dict(L=640, layout=("rank3_hv", "rank3_hv", "rank3_hv"), docs=True, strong=True),
    "weak_decay": dict(L=512, layout=("rank3_hk", "rank3_hk", "rank3_hk"), init=True, g_shift=-7.0),
}


@pytest.mark.parametrize("case", sorted(SCALAR_CASES))
def test_scalar_gate_prefill_bf16(case):
    c = SCALAR_CASES[case]
    B, Hk, Hv, L = 2, 2, 4, c["L"]
    seed = sorted(SCALAR_CASES).index(case) + 900
    q, k, v, g, b, w = make_inputs(seed, B, L, Hk, Hv, g_layout=c["layout"][0], b_layout=c["layout"][1],
                                   w_layout=c["layout"][2], qscale=c.get("qscale", 1.0),
                                   g_shift=c.get("g_shift", -1.0))
    rng = np.random.default_rng(seed)
    if c.get("strong"):
        # Qwen3-Next decay: -exp(A_log) softplus(a), A_log up to log(64)
        A_log = rng.uniform(0.0, np.log(64.0), g.shape[2])
        g = -np.exp(A_log) * np.log1p(np.exp(rng.standard_normal(g.shape[:3])))
    seg = None
    if c.get("docs"):
        cuts = np.sort(rng.choice(np.arange(1, L), size=(B, 3), replace=False), axis=1)
        seg = np.stack([np.searchsorted(cuts[i], np.arange(L), side="right") + 5 * i for i in range(B)])
    init = 0.1 * rng.standard_normal((B, Hv, 128, 128)) if c.get("init") else None
    kw = dict(qk_l2norm=c.get("l2norm", True))
    if "scale" in c:
        kw["scale"] = c["scale"]
    if c.get("guard"):
        kw["stability_guard"] = True
    out, st, ro, rs = run_pair(q, k, v, g, b, w, dt="bf16", precision="bf16", seg=seg, init=init, **kw)
    check(out, ro, st, rs, "bf16", "bf16", f"scalar gates {case}")


# With more 16-column tiles than 512 (bf16 mode), the chain runs 2 or 4 tiles
# per workgroup: (B=2 / B=4) x 32 heads x 8 tiles, short sequences, both
# prepass forms (channel gates; one decay and b per token and head).
@pytest.mark.parametrize("B", [2, 4])
@pytest.mark.parametrize("gates", ["channel_hv", "scalar"])
def test_chain_tiles_per_workgroup(B, gates):
    Hk, Hv, L = 16, 32, 300
    layout = ("channel_hv", "channel_hv", "channel_hv") if gates == "channel_hv" else ("rank3_hv", "rank3_hv", "rank3_hv")
    q, k, v, g, b, w = make_inputs(70 + B, B, L, Hk, Hv, g_layout=layout[0], b_layout=layout[1], w_layout=layout[2])
    rng = np.random.default_rng(71 + B)
    seg = np.stack([np.repeat([0, 1, 2], [100, 120, 80]) + 3 * i for i in range(B)])
    init = 0.1 * rng.standard_normal((B, Hv, 128, 128))
    out, st, ro, rs = run_pair(q, k, v, g, b, w, dt="bf16", precision="bf16", seg=seg, init=init, qk_l2norm=True)
    check(out, ro, st, rs, "bf16", "bf16", f"chain tiles B={B} {gates}")


@pytest.mark.parametrize("L", [300, 384])
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_fused_prologue_docs_init(L, precision):
    rng = np.random.default_rng(L)
    B, Hk, Hv = 1, 2, 4
    q, k = rng.standard_normal((2, B, L, Hk, 128))
    v = rng.standard_normal((B, L, Hv, 128))
    g, b = rng.standard_normal((2, B, L, Hk, 128))
    w = rng.standard_normal((B, L, Hv, 128))
    seg = np.repeat([0, 1, 2], [L // 3, L // 3, L - 2 * (L // 3)])[None]
    init = 0.05 * rng.standard_normal((B, Hv, 128, 128))
    out, st, ro, rs = run_pair(q, k, v, g, b, w, precision=precision, seg=seg, init=init, qk_l2norm=True,
                               fuse_prologue=True)
    check(out, ro, st, rs, precision, "fp32", f"fused L={L} {precision}")


def test_initial_state_segment_id_reset():
    # test_doc_reset_and_streaming.py:9-58: a different id at token 0 resets the
    # initial state exactly
    q, k, v, g, b, w = make_inputs(3, 1, 200, 2, 4)
    seg = np.full((1, 200), 7)
    init = np.random.default_rng(1).standard_normal((1, 4, 128, 128))
    kw = dict(segment_ids=to_dev(seg, torch.int32), output_final_state=True, is_inference=True, qk_l2norm=True)
    T = lambda x: to_dev(x)
    o0, s0 = chunk_gdn2(T(q), T(k), T(v), T(g), T(b), T(w), **kw)
    o1, s1 = chunk_gdn2(T(q), T(k), T(v), T(g), T(b), T(w), initial_state=T(init), initial_state_segment_id=6, **kw)
    o2, s2 = chunk_gdn2(T(q), T(k), T(v), T(g), T(b), T(w), initial_state=T(init), initial_state_segment_id=7, **kw)
    assert torch.equal(o0, o1) and torch.equal(s0, s1)
    ro, rs = O.chunk_gdn2(q, k, v, g, b, w, segment_ids=seg, initial_state=init, initial_state_segment_id=7,
                          output_final_state=True, qk_l2norm=True)
    check(o2, ro, s2, rs, "bf16", "fp32", "init_seg continue")


def test_cu_seqlens_equals_segment_ids_and_reused_ids():
    q, k, v, g, b, w = make_inputs(4, 1, 384, 1, 2)
    T = lambda x: to_dev(x)
    seg = np.array([0] * 100 + [1] * 150 + [0] * 134)[None]
    kw = dict(is_inference=True, qk_l2norm=True, precision="fp32")
    o1 = chunk_gdn2(T(q), T(k), T(v), T(g), T(b), T(w), segment_ids=to_dev(seg, torch.int64), **kw)
    o2 = chunk_gdn2(T(q), T(k), T(v), T(g), T(b), T(w), cu_seqlens=[0, 100, 250, 384], **kw)
    o3 = chunk_gdn2(T(q), T(k), T(v), T(g), T(b), T(w), segment_ids=to_dev(seg[0], torch.int32), **kw)
    assert torch.equal(o1, o2) and torch.equal(o1, o3)
    ro, _ = O.chunk_gdn2(q, k, v, g, b, w, segment_ids=seg, qk_l2norm=True)
    check(o1, ro, precision="fp32", tag="reused ids")


@pytest.mark.parametrize("split", [64, 128, 192, 300])
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_state_passing_continuity(split, precision):
    # test_state_passing.py / test_inference.py:11-61
    q, k, v, g, b, w = make_inputs(split, 1, 512, 2, 4)
    T = lambda x: to_dev(x)
    kw = dict(is_inference=True, qk_l2norm=True, output_final_state=True, precision=precision)
    o, s = chunk_gdn2(T(q), T(k), T(v), T(g), T(b), T(w), **kw)
    a, bsl = slice(0, split), slice(split, 512)
    o1, s1 = chunk_gdn2(*(T(x[:, a]) for x in (q, k, v, g, b, w)), **kw)
    o2, s2 = chunk_gdn2(*(T(x[:, bsl]) for x in (q, k, v, g, b, w)), initial_state=s1, **kw)
    tol = 1e-4 if precision == "fp32" else 1e-2
    assert rel_l2(as_np(torch.cat([o1, o2], 1)), as_np(o)) < tol
    assert rel_l2(as_np(s2), as_np(s)) < tol


@pytest.mark.parametrize("L,block", [(512, 256), (1024, 512), (300, 128)])
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_streaming_matches_monolithic(L, block, precision):
    # test_streaming_and_stability.py:28-62 and test_doc_reset_and_streaming.py:61-104
    q, k, v, g, b, w = make_inputs(L + block, 1, L, 2, 4)
    seg = np.repeat(np.arange(4), [L // 4] * 3 + [L - 3 * (L // 4)])
    seg[block: block + 1] = seg[block - 1]  # reused id across a block boundary
    T = lambda x: to_dev(x)
    kw = dict(is_inference=True, qk_l2norm=True, output_final_state=True, precision=precision,
              segment_ids=to_dev(seg, torch.int32))
    o, s = chunk_gdn2(T(q), T(k), T(v), T(g), T(b), T(w), **kw)
    o2, s2 = chunk_gdn2(T(q), T(k), T(v), T(g), T(b), T(w), streaming_prefill=True, prefill_block_size=block, **kw)
    tol = 1e-5 if precision == "fp32" else 1e-2
    assert rel_l2(as_np(o2), as_np(o)) < tol and rel_l2(as_np(s2), as_np(s)) < tol
    ro, rs = O.chunk_gdn2(q, k, v, g, b, w, segment_ids=seg, output_final_state=True, qk_l2norm=True,
                          streaming_prefill=True, prefill_block_size=block)
    check(o2, ro, s2, rs, precision, "fp32", f"streaming L={L} block={block}")


def test_stability_guard_caps_state():
    # test_streaming_and_stability.py:93-112
    q, k, v, g, b, w = make_inputs(9, 1, 512, 2, 4, qscale=10.0)
    v = v * 100.0
    v[:, :, 1] *= 1e-3   # value head 1 stays below the cap
    T = lambda x: to_dev(x)
    tau = 50.0
    o, s = chunk_gdn2(T(q), T(k), T(v), T(g), T(b), T(w), is_inference=True, output_final_state=True,
                      qk_l2norm=True, stability_guard=True, stability_tau=tau, precision="fp32")
    # The uncapped state, independently: the guard's input clamps applied by
    # hand (gdn2.py:1972-1974) and no guard.  Capped heads must land on
    # ||S||_F = tau along the uncapped direction (gdn2.py:2224-2226); heads
    # below tau must come back bit-identical.
    _, s_unc = chunk_gdn2(T(q), T(k), T(v), T(np.minimum(g, -1e-6)), T(np.maximum(b, 0.0)), T(w),
                          is_inference=True, output_final_state=True, qk_l2norm=True, precision="fp32")
    n_unc = torch.linalg.vector_norm(s_unc.double(), dim=(-2, -1))
    norms = torch.linalg.vector_norm(s.double(), dim=(-2, -1))
    capped = n_unc > tau
    assert bool(capped.any()) and bool((~capped).any())
    assert torch.allclose(norms[capped], torch.full_like(norms[capped], tau), rtol=1e-5, atol=0)
    scale = tau / torch.sqrt(n_unc ** 2 + 1e-6)
    assert torch.allclose(s.double()[capped], (s_unc.double() * scale[..., None, None])[capped], rtol=1e-5,
                          atol=1e-6 * tau / 128)
    assert torch.equal(s[~capped], s_unc[~capped])
    ro, rs = O.chunk_gdn2(q, k, v, g, b, w, output_final_state=True, qk_l2norm=True, stability_guard=True,
                          stability_tau=tau)
    check(o, ro, s, rs, "fp32", "fp32", "guard")
    o2, s2 = chunk_gdn2(T(q), T(k), T(v), T(g), T(b), T(w), is_inference=True, output_final_state=True,
                        qk_l2norm=True, stability_guard=True, stability_tau=tau, precision="fp32",
                        streaming_prefill=True, prefill_block_size=128)
    ro2, rs2 = O.chunk_gdn2(q, k, v, g, b, w, output_final_state=True, qk_l2norm=True, stability_guard=True,
                            stability_tau=tau, streaming_prefill=True, prefill_block_size=128)
    check(o2, ro2, s2, rs2, "fp32", "fp32", "guard streaming")


@pytest.mark.parametrize("t_cut", [0, 100, 255])
def test_causality_bit_exact(t_cut):
    # test_causality.py:27-74: perturbing the future leaves past outputs bit-identical
    q, k, v, g, b, w = make_inputs(t_cut, 1, 384, 2, 4)
    T = lambda x: to_dev(x, torch.bfloat16)
    o1 = chunk_gdn2(T(q), T(k), T(v), to_dev(g), to_dev(b), to_dev(w), is_inference=True, qk_l2norm=True)
    v2, k2 = v.copy(), k.copy()
    v2[:, t_cut + 1:] += 1.0
    k2[:, t_cut + 1:] *= -1.0
    o2 = chunk_gdn2(T(q), T(k2), T(v2), to_dev(g), to_dev(b), to_dev(w), is_inference=True, qk_l2norm=True)
    assert torch.equal(o1[:, :t_cut + 1], o2[:, :t_cut + 1])
    assert not torch.equal(o1[:, t_cut + 1:], o2[:, t_cut + 1:])


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_strong_decay_finite(precision):
    # test_strong_decay.py:34-70: g <= -150 stays finite and matches
    q, k, v, g, b, w = make_inputs(1, 1, 256, 2, 4)
    g = g - 150.0
    g[:, 100:140] = -0.01
    out, st, ro, rs = run_pair(q, k, v, g, b, w, precision=precision, qk_l2norm=True)
    assert torch.isfinite(out).all() and torch.isfinite(st).all()
    check(out, ro, st, rs, precision, "fp32", f"strong decay {precision}")


@pytest.mark.parametrize("decay", ["mild", "near_bound", "wide", "mixed"])
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_decay_span_paths(decay, precision):
    # Off-diagonal A / M tiles factor around the chunk's row 64 when the decay
    # on either side of it stays within 2^100 ("mild": ~2^9, "near_bound":
    # ~2^92 per side), and fall back to per-pair rescaling otherwise ("wide":
    # ~2^147 per side, each 16-token block still within bounds).  "mixed"
    # varies the span per channel across the threshold, with a reset.
    q, k, v, g, b, w = make_inputs(11, 1, 384, 2, 4)
    rng = np.random.default_rng(12)
    nat = {"mild": 0.1, "near_bound": 1.0, "wide": 1.6}
    if decay == "mixed":
        rate = np.where(np.arange(128) % 3 == 0, 1.6, np.where(np.arange(128) % 3 == 1, 0.9, 0.02))
        g = -rate * np.exp(0.05 * rng.standard_normal(g.shape))
    else:
        g = -nat[decay] * np.exp(0.05 * rng.standard_normal(g.shape))
    seg = (np.arange(384) >= 200).astype(np.int32)[None] if decay == "mixed" else None
    init = 0.1 * rng.standard_normal((1, 4, 128, 128))
    out, st, ro, rs = run_pair(q, k, v, g, b, w, precision=precision, qk_l2norm=True, seg=seg, init=init)
    assert torch.isfinite(out).all() and torch.isfinite(st).all()
    check(out, ro, st, rs, precision, "fp32", f"decay {decay} {precision}")


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_units_fill_every_cu(precision):
    # When the (batch, head, chunk) units leave no CU idle during the prepass,
    # the value kernel forms (w*v)^T itself instead of reading the fragments
    # the prepass launch's spare workgroups write.  Size B so that the units
    # cover every CU of this device.
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    L, Hk, Hv = 512, 4, 8
    B = -(-cus // (Hk * (L // 128)))
    q, k, v, g, b, w = make_inputs(21, B, L, Hk, Hv)
    out, st, ro, rs = run_pair(q, k, v, g, b, w, precision=precision, qk_l2norm=True)
    check(out, ro, st, rs, precision, "fp32", f"units fill CUs B={B} {precision}")


def test_positive_decay_clamped():
    # test_strong_decay.py:72-89: g > 0 behaves as g = 0
    q, k, v, g, b, w = make_inputs(2, 1, 200, 2, 4)
    gp = np.abs(g) * 0.5
    T = lambda x: to_dev(x)
    o1 = chunk_gdn2(T(q), T(k), T(v), T(gp), T(b), T(w), is_inference=True, qk_l2norm=True, precision="fp32")
    o2 = chunk_gdn2(T(q), T(k), T(v), T(np.zeros_like(g)), T(b), T(w), is_inference=True, qk_l2norm=True,
                    precision="fp32")
    assert torch.equal(o1, o2)


@pytest.mark.parametrize("kind", ["identical", "near", "periodic", "opposite"])
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_adversarial_keys(kind, precision):
    # test_nan_adversarial.py:116-264 (through the fused prologue)
    rng = np.random.default_rng(3)
    B, L, Hk, Hv = 1, 256, 1, 2
    base = rng.standard_normal((B, 1, Hk, 128))
    if kind == "identical":
        k = np.repeat(base, L, 1)
    elif kind == "near":
        k = np.repeat(base, L, 1) + 1e-3 * rng.standard_normal((B, L, Hk, 128))
    elif kind == "periodic":
        k = np.repeat(rng.standard_normal((B, 4, Hk, 128)), L // 4, 1)[:, np.arange(L) % 4 * (L // 4)]
    else:
        k = np.repeat(base, L, 1) * np.where(np.arange(L) % 2, 1.0, -1.0)[None, :, None, None]
    q = rng.standard_normal((B, L, Hk, 128))
    v = rng.standard_normal((B, L, Hv, 128))
    g, b = rng.standard_normal((2, B, L, Hk, 128))
    w = rng.standard_normal((B, L, Hv, 128))
    out, st, ro, rs = run_pair(q, k, v, g, b, w, precision=precision, qk_l2norm=True, fuse_prologue=True)
    assert torch.isfinite(out).all()
    check(out, ro, st, rs, precision, "fp32", f"adversarial {kind} {precision}")


def test_chunk_gdn_qwen_layout():
    # test_variants.py:73-122: Qwen3.5-4B / Qwen3-Next layout, gates at Hv
    B, L, Hk, Hv = 2, 300, 2, 4
    rng = np.random.default_rng(6)
    q, k = rng.standard_normal((2, B, L, Hk, 128))
    v = rng.standard_normal((B, L, Hv, 128))
    A_log = rng.uniform(np.log(1), np.log(16), Hv)
    a = rng.standard_normal((B, L, Hv))
    g = -np.exp(A_log) * np.log1p(np.exp(a))
    beta = sig(rng.standard_normal((B, L, Hv)))
    out, st = chunk_gdn(to_dev(q), to_dev(k), to_dev(v), to_dev(g), to_dev(beta), qk_l2norm=True,
                        output_final_state=True, is_inference=True, precision="fp32")
    ro, rs = O.chunk_gdn(q, k, v, g, beta, qk_l2norm=True, output_final_state=True)
    check(out, ro, st, rs, "fp32", "fp32", "chunk_gdn qwen")


@pytest.mark.parametrize("variant", ["kda", "gla", "delta"])
def test_other_variants(variant):
    B, L, Hk, Hv = 1, 200, 2, 4
    q, k, v, g, b, w = make_inputs(8, B, L, Hk, Hv)
    beta = sig(np.random.default_rng(1).standard_normal((B, L, Hk)))
    T = lambda x: to_dev(x)
    kw = dict(qk_l2norm=True, output_final_state=True, is_inference=True, precision="fp32")
    if variant == "kda":
        out, st = chunk_kda(T(q), T(k), T(v), T(g), T(beta), **kw)
        ro, rs = O.chunk_gdn2(q, k, v, g, beta, beta, qk_l2norm=True, output_final_state=True)
    elif variant == "gla":
        out, st = chunk_gla(T(q), T(k), T(v), T(g), **kw)
        ro, rs = O.chunk_gdn2(q, k, v, g, np.zeros((B, L, 1)), np.ones((B, L, 1)), qk_l2norm=True,
                              output_final_state=True)
    else:
        out, st = chunk_delta_rule(T(q), T(k), T(v), T(beta), **kw)
        ro, rs = O.chunk_gdn2(q, k, v, np.zeros((B, L, 1)), beta, beta, qk_l2norm=True, output_final_state=True)
    check(out, ro, st, rs, "fp32", "fp32", variant)


def test_differentiation_raises():
    q, k, v, g, b, w = make_inputs(1, 1, 128, 1, 1)
    qt = to_dev(q).requires_grad_(True)
    out = chunk_gdn2(qt, to_dev(k), to_dev(v), to_dev(g), to_dev(b), to_dev(w), is_inference=True, qk_l2norm=True)
    with pytest.raises(ValueError, match="differentiation is not supported when is_inference=True"):
        out.sum().backward()


def test_streaming_block_edge_boundaries_and_reused_id():
    # test_doc_reset_and_streaming.py:61-104: documents starting exactly at the
    # block edges 128 and 256 (id 0 reused at 256), L = 300, positive decay
    # entries (clamped), L2-norm with scale 0.25, 1-D segment ids: streaming
    # equals the single pass within 1e-5
    rng = np.random.default_rng(202)
    B, L, Hk, Hv = 1, 300, 1, 2
    q, k = rng.standard_normal((2, B, L, Hk, 128))
    v = rng.standard_normal((B, L, Hv, 128))
    g = 0.5 * rng.standard_normal((B, L, Hk, 128))
    b, w = sig(rng.standard_normal((B, L, Hk, 128))), sig(rng.standard_normal((B, L, Hv, 128)))
    seg = np.concatenate([np.zeros(128), np.ones(128), np.zeros(44)]).astype(np.int32)
    T = lambda x: to_dev(x)
    kw = dict(segment_ids=to_dev(seg, torch.int32), output_final_state=True, qk_l2norm=True, scale=0.25,
              is_inference=True, precision="fp32")
    o1, s1 = chunk_gdn2(*(T(x) for x in (q, k, v, g, b, w)), **kw)
    o2, s2 = chunk_gdn2(*(T(x) for x in (q, k, v, g, b, w)), streaming_prefill=True, prefill_block_size=128, **kw)
    assert np.allclose(as_np(o2), as_np(o1), rtol=1e-5, atol=1e-5)
    assert np.allclose(as_np(s2), as_np(s1), rtol=1e-5, atol=1e-5)
    ro, rs = O.chunk_gdn2(q, k, v, g, b, w, segment_ids=seg[None], output_final_state=True, qk_l2norm=True, scale=0.25)
    check(o2, ro, s2, rs, "fp32", "fp32", "streaming block-edge documents")
