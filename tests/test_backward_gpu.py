"""GPU parity of the training backward (``chunk_gdn2(..., is_inference=False)``
under torch.autograd, HIP kernels of ``dn_prefill_bwd``) against the gradient
oracle (oracle/gdn_grad.py, pinned in tests/test_oracle_grad.py).

Cases and tolerances follow the reference's gradient tests: rel L2 per
gradient < 1e-5 in "fp32" mode and < 1e-2 in "bf16" mode
(tests/test_parity.py:32-68), the L2-norm / scale / GQA case
(test_parity.py:71-99), the fused prologue with an unaligned length, initial
state, segment ids and a final-state cotangent (test_parity.py:160-221),
strong decay g <= -150 (tests/test_strong_decay.py:35-69, tolerance 1e-3 /
1e-2), gate layouts (tests/test_matrix.py) and chunk_gdn (variants.py:17-88).
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


def ref_inputs(seed, B, L, Hk, Hv, K=128, V=128):
    """The reference tests' generator (test_parity.py:18-26), seeded NumPy."""
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s)
    q = f(B, L, Hk, K) * 0.1
    k = f(B, L, Hk, K) * 0.1
    v = f(B, L, Hv, V) * 0.1
    b = sig(f(B, L, Hk, K) * 0.39)
    w = sig(f(B, L, Hv, V) * 0.39)
    g = -np.exp(f(B, L, Hk, K) * 0.39 - 1.0)
    return q, k, v, g, b, w


def run_dev(q, k, v, g, b, w, do, df=None, init=None, qkv_dtype=torch.float32, fn=None, **kw):
    ts = [to_dev(x, qkv_dtype if i < 3 else torch.float32).requires_grad_(True)
          for i, x in enumerate((q, k, v, g, b, w))]
    ti = to_dev(init).requires_grad_(True) if init is not None else None
    if fn is None:
        from deltanet_tpu_amd import chunk_gdn2 as fn
    res = fn(*ts, initial_state=ti, output_final_state=df is not None, is_inference=False, **kw)
    if df is not None:
        out, fin = res
        loss = (out.float() * to_dev(do)).sum() + (fin * to_dev(df)).sum()
    else:
        out = res
        loss = (out.float() * to_dev(do)).sum()
    loss.backward()
    torch.cuda.synchronize()
    grads = {n: as_np(t.grad) for n, t in zip(NAMES, ts)}
    grads["dinit"] = as_np(ti.grad) if ti is not None else None
    return as_np(out), grads


def compare(got, ref, tol, tag):
    errs = {n: rel_l2(got[n], ref[n]) for n in (*NAMES, "dinit") if ref.get(n) is not None and n in got}
    print("[measured]", tag, " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    for n, e in errs.items():
        assert np.isfinite(got[n]).all(), (tag, n, "non-finite")
        assert e < tol, f"{tag}: gradient {n} rel L2 {e:.2e} exceeds {tol:.1e}"


# bf16 mode: split-bf16 products (16 significant bits) measure ~5e-6; the bound
# leaves 10x headroom
@pytest.mark.parametrize("precision, tol", [("fp32", 1e-5), ("bf16", 5e-5)])
@pytest.mark.parametrize("L", [128, 256, 512])
def test_backward_parity(precision, tol, L):
    B, Hk, Hv = 1, 2, 4
    q, k, v, g, b, w = ref_inputs(42 + L, B, L, Hk, Hv)
    do = np.random.default_rng(100 + L).standard_normal((B, L, Hv, 128))
    out, got = run_dev(q, k, v, g, b, w, do, precision=precision)
    ref = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do)
    o_ref, _ = O.chunk_gdn2(q, k, v, g, b, w, is_inference=False)
    e_o = rel_l2(out, o_ref)
    print(f"[measured] L={L} {precision}: out rel L2 {e_o:.2e}", flush=True)
    # the forward's bf16 mode runs its plain products on bf16 MFMA: ~9e-5
    assert e_o < (tol if precision == "fp32" else 5e-4)
    compare(got, ref, tol, f"parity L={L} {precision}")


def test_backward_l2norm_scale_gqa():
    B, L, Hk, Hv = 1, 256, 2, 4
    q, k, v, g, b, w = ref_inputs(7, B, L, Hk, Hv)
    do = np.random.default_rng(8).standard_normal((B, L, Hv, 128))
    _, got = run_dev(q, k, v, g, b, w, do, precision="fp32", qk_l2norm=True, scale=0.5)
    ref = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do, qk_l2norm=True, scale=0.5)
    compare(got, ref, 1e-5, "l2norm scale=0.5 G=2")


@pytest.mark.parametrize("precision, tol", [("fp32", 1e-5), ("bf16", 5e-5)])
@pytest.mark.parametrize("L", [300, 384])
def test_backward_fuse_prologue_unaligned(L, precision, tol):
    """Initial state, final-state cotangent, three documents, unaligned L; in
    bf16 mode this drives the split-bf16 scans' state load (init / d_final)
    and store (d_init) paths."""
    B, Hk, Hv, K, V = 1, 2, 4, 128, 128
    rng = np.random.default_rng(2026 + L)
    f = lambda *s: rng.standard_normal(s)
    q, k, v = f(B, L, Hk, K) * 0.1, f(B, L, Hk, K) * 0.1, f(B, L, Hv, V) * 0.1
    g = f(B, L, Hk, K) * 0.39 - 1.0
    b = f(B, L, Hk, K) * 0.39
    w = f(B, L, Hv, V) * 0.39
    init = f(B, Hv, K, V) * 0.05
    seg = np.array([[0] * (L // 3) + [1] * (L // 3) + [2] * (L - 2 * (L // 3))], dtype=np.int32)
    do, df = f(B, L, Hv, V), f(B, Hv, K, V)
    kw = dict(qk_l2norm=True, fuse_prologue=True)
    _, got = run_dev(q, k, v, g, b, w, do, df=df, init=init, precision=precision,
                     segment_ids=torch.from_numpy(seg).cuda(), **kw)
    ref = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do, df, initial_state=init, segment_ids=seg, **kw)
    compare(got, ref, tol, f"fuse_prologue L={L} {precision}")


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_backward_strong_decay(precision):
    B, L, Hk, Hv = 1, 256, 2, 4
    q, k, v, _, b, w = ref_inputs(501, B, L, Hk, Hv)
    g = -150.0 - np.abs(np.random.default_rng(502).standard_normal((B, L, Hk, 128)) * 50.0)
    do = np.random.default_rng(503).standard_normal((B, L, Hv, 128))
    _, got = run_dev(q, k, v, g, b, w, do, precision=precision)
    ref = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do)
    # measured 2e-7 (fp32) and 4e-6 (bf16)
    compare(got, ref, 1e-5 if precision == "fp32" else 5e-5, f"strong decay {precision}")



@pytest.mark.parametrize("precision, tol", [("fp32", 1e-5), ("bf16", 5e-5)])
def test_backward_odd_heads_two_batches(precision, tol):
    """B = 2, three value heads on one key head (G = 3) and an unaligned length:
    24 chain workgroups per direction (not a multiple of 8 heads per XCD) and a
    partial last chunk in every kernel's index mapping."""
    B, L, Hk, Hv = 2, 130, 1, 3
    q, k, v, g, b, w = ref_inputs(701, B, L, Hk, Hv)
    do = np.random.default_rng(702).standard_normal((B, L, Hv, 128))
    _, got = run_dev(q, k, v, g, b, w, do, precision=precision)
    ref = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do)
    compare(got, ref, tol, f"B=2 Hk=1 Hv=3 L=130 {precision}")


def test_backward_mixed_decay_spans():
    """16-token blocks whose decay span is below 2^64 in every channel form
    their diagonal A / M tiles as factored MFMA products, the others
    element by element; here both kinds share chunks and channels (per-token
    log-decay -0.05, -2.7 -- a span of about 2^58 -- and -6 in half of the
    channels of some blocks)."""
    B, L, Hk, Hv = 1, 256, 2, 4
    q, k, v, _, b, w = ref_inputs(601, B, L, Hk, Hv)
    rng = np.random.default_rng(602)
    blk = (np.arange(L) // 16) % 4
    per_tok = np.choose(blk, [-0.05, -2.7, -0.5, -0.05])[None, :, None, None] * np.ones((B, L, Hk, 128))
    strong = (blk == 3)[None, :, None, None] & (np.arange(128) % 2 == 0)[None, None, None, :]
    g = np.where(strong, -6.0, per_tok) * (1.0 + 0.01 * np.abs(rng.standard_normal((B, L, Hk, 128))))
    do = rng.standard_normal((B, L, Hv, 128))
    _, got = run_dev(q, k, v, g, b, w, do, precision="fp32")
    ref = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do)
    compare(got, ref, 1e-5, "mixed decay spans fp32")


def test_backward_positive_decay_and_guard():
    """Positive g is clamped (zero gradient, test_strong_decay.py:72-89);
    stability_guard clamps b >= 0 and g <= -1e-6 (gdn2.py:1972-1974)."""
    B, L, Hk, Hv = 1, 192, 2, 4
    q, k, v, g, b, w = ref_inputs(9, B, L, Hk, Hv)
    rng = np.random.default_rng(10)
    g = np.where(rng.random(g.shape) < 0.3, np.abs(g) * 0.2 + 0.01, g)
    b = b - 0.3
    do = rng.standard_normal((B, L, Hv, 128))
    _, got = run_dev(q, k, v, g, b, w, do, precision="fp32", stability_guard=True)
    ref = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do, stability_guard=True)
    compare(got, ref, 1e-5, "guard + positive g")
    assert np.all(got["dg"][g > 0] == 0.0)


@pytest.mark.parametrize("layout", ["scalar_hk", "rank3_one", "gates_at_hv"])
def test_backward_gate_layouts(layout):
    B, L, Hk, Hv = 2, 200, 1, 2
    rng = np.random.default_rng(11)
    f = lambda *s: rng.standard_normal(s)
    q, k, v = f(B, L, Hk, 128) * 0.1, f(B, L, Hk, 128) * 0.1, f(B, L, Hv, 128) * 0.1
    if layout == "scalar_hk":
        g, b, w = -np.exp(f(B, L, Hk, 1) * 0.39 - 1), sig(f(B, L, Hk, 1)), sig(f(B, L, Hk, 1))
    elif layout == "rank3_one":
        g, b, w = -np.exp(f(B, L, 1) * 0.39 - 1), sig(f(B, L, Hk, 128)), sig(f(B, L, 1))
    else:
        g, b, w = -np.exp(f(B, L, Hv, 128) * 0.39 - 1), sig(f(B, L, Hv, 128)), sig(f(B, L, Hv, 128))
    seg = np.array([[0] * 70 + [1] * 130, [5] * 150 + [2] * 50])
    init = f(B, Hv, 128, 128) * 0.05
    do, df = f(B, L, Hv, 128), f(B, Hv, 128, 128)
    _, got = run_dev(q, k, v, g, b, w, do, df=df, init=init, precision="fp32",
                     segment_ids=torch.from_numpy(seg).cuda(), initial_state_segment_id=[0, 2])
    ref = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do, df, initial_state=init, segment_ids=seg,
                            initial_state_segment_id=[0, 2])
    compare(got, ref, 1e-5, f"gates {layout}")
    # batch 1's first document (id 5) differs from its initial_state_segment_id (2)
    assert np.all(got["dinit"][1] == 0.0) and np.abs(got["dinit"][0]).max() > 0


def test_backward_f16_inputs():
    """f16 q, k, v: dq and dk come back in f16 from the kernel (v is carried in
    f32 and its gradient cast back by autograd); scale 1 and no L2-norm, so the
    forward sees the f16 values exactly and the oracle runs on them."""
    B, L, Hk, Hv = 1, 200, 2, 4
    q, k, v, g, b, w = ref_inputs(31, B, L, Hk, Hv)
    qh, kh, vh = (x.astype(np.float16).astype(np.float64) for x in (q, k, v))
    do = np.random.default_rng(32).standard_normal((B, L, Hv, 128))
    _, got = run_dev(q, k, v, g, b, w, do, qkv_dtype=torch.float16, precision="fp32", scale=1.0)
    doh = do.astype(np.float16).astype(np.float64)   # the f16 output's cotangent is f16
    ref = GR.chunk_gdn2_vjp(qh, kh, vh, g, b, w, doh, scale=1.0)
    # scale 1 instead of 1/sqrt(K) makes the scores ~11x larger than in the
    # reference's cases, and the fp32 rounding of the gate gradients with them
    compare({n: got[n] for n in ("dg", "db", "dw")}, ref, 5e-5, "f16 q/k/v (f32 leaves)")
    compare({n: got[n] for n in ("dq", "dk", "dv")}, ref, 2e-3, "f16 q/k/v (f16 leaves)")


def test_backward_bf16_inputs_and_chunk_gdn():
    from deltanet_tpu_amd import chunk_gdn
    B, L, Hk, Hv = 1, 256, 2, 4
    q, k, v, g, b, w = ref_inputs(12, B, L, Hk, Hv)
    qb, kb, vb = (O.bf16_round(x).astype(np.float64) for x in (q, k, v))
    do = np.random.default_rng(13).standard_normal((B, L, Hv, 128))
    _, got = run_dev(q, k, v, g, b, w, do, qkv_dtype=torch.bfloat16, precision="fp32", qk_l2norm=True)
    # a bf16 output receives its cotangent in bf16 (as JAX's does), and the
    # gradients of bf16 leaves are bf16: they carry bf16 rounding (2^-9)
    dob = O.bf16_round(do).astype(np.float64)
    ref = GR.chunk_gdn2_vjp(qb, kb, vb, g, b, w, dob, qk_l2norm=True, qk_bf16=True)
    compare({n: got[n] for n in ("dg", "db", "dw")}, ref, 1e-5, "bf16 q/k/v, l2norm (f32 leaves)")
    compare({n: got[n] for n in ("dq", "dk", "dv")}, ref, 4e-3, "bf16 q/k/v, l2norm (bf16 leaves)")
    # chunk_gdn: scalar decay per head, b = w = beta (variants.py:17-88)
    gs = -np.exp(np.random.default_rng(14).standard_normal((B, L, Hk)) * 0.39 - 1)
    beta = sig(np.random.default_rng(15).standard_normal((B, L, Hk)))
    qt, kt, vt = (to_dev(x).requires_grad_(True) for x in (q, k, v))
    gt, bt = to_dev(gs).requires_grad_(True), to_dev(beta).requires_grad_(True)
    out = chunk_gdn(qt, kt, vt, gt, bt, precision="fp32", is_inference=False)
    (out.float() * to_dev(do)).sum().backward()
    rg = GR.chunk_gdn2_vjp(q, k, v, gs, beta, beta, do)
    # beta feeds both b and w: its gradient is the sum of both
    got2 = {"dq": as_np(qt.grad), "dk": as_np(kt.grad), "dv": as_np(vt.grad), "dg": as_np(gt.grad)}
    for n in got2:
        e = rel_l2(got2[n], rg[n])
        print(f"[measured] chunk_gdn {n}={e:.2e}", flush=True)
        assert e < 1e-5, n
    e = rel_l2(as_np(bt.grad), rg["db"] + rg["dw"])
    assert e < 1e-5, e


def test_backward_cu_seqlens_batch2():
    """cu_seqlens documents (gdn2.py:2033-2079) with B = 2 and an initial state."""
    B, L, Hk, Hv = 2, 320, 2, 4
    q, k, v, g, b, w = ref_inputs(31, B, L, Hk, Hv)
    rng = np.random.default_rng(32)
    init = rng.standard_normal((B, Hv, 128, 128)) * 0.05
    do, df = rng.standard_normal((B, L, Hv, 128)), rng.standard_normal((B, Hv, 128, 128))
    cu = [0, 70, 200, 201, 320]
    _, got = run_dev(q, k, v, g, b, w, do, df=df, init=init, precision="fp32", cu_seqlens=cu)
    ref = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do, df, initial_state=init, cu_seqlens=cu)
    compare(got, ref, 1e-5, "cu_seqlens B=2")


@pytest.mark.parametrize("variant", ["gdn", "kda", "gla", "delta_rule"])
@pytest.mark.parametrize("Hk,Hv", [(2, 2), (2, 4)])
@pytest.mark.parametrize("has_init", [False, True])
def test_backward_variants(variant, Hk, Hv, has_init):
    """The variants are adapters over chunk_gdn2 (variants.py:17-285), so they
    train through the same backward: GDN (one decay per key head, b = w =
    beta), KDA (channel decay, b = w = beta), GLA (b = 0, w = 1), DeltaNet
    (g = 0, b = w = beta).  As tests/test_matrix.py:263-336: B = 2, L = 300,
    with and without an initial state, a loss on the output and the final
    state; every gradient (and the initial state's) within rel L2 1e-4."""
    import deltanet_tpu_amd as D
    B, L = 2, 300
    rng = np.random.default_rng(40)
    q, k = 0.1 * rng.standard_normal((2, B, L, Hk, 128))
    v = 0.1 * rng.standard_normal((B, L, Hv, 128))
    g = -rng.uniform(0.1, 2.0, (B, L, Hk, 1 if variant == "gdn" else 128))
    beta = sig(0.39 * rng.standard_normal((B, L, Hk, 1)))
    init = 0.05 * rng.standard_normal((B, Hv, 128, 128)) if has_init else None
    do, df = rng.standard_normal((B, L, Hv, 128)), rng.standard_normal((B, Hv, 128, 128))
    qt, kt, vt = (to_dev(x).requires_grad_(True) for x in (q, k, v))
    gt, bt = to_dev(g).requires_grad_(True), to_dev(beta).requires_grad_(True)
    it = to_dev(init).requires_grad_(True) if has_init else None
    kw = dict(initial_state=it, output_final_state=True, precision="fp32", is_inference=False)
    zeros, ones = np.zeros((B, L, Hk, 1)), np.ones((B, L, Hv, 1))
    if variant == "gdn":
        out, fin = D.chunk_gdn(qt, kt, vt, gt, bt, **kw)
        args = (g, beta, beta)
    elif variant == "kda":
        out, fin = D.chunk_kda(qt, kt, vt, gt, bt, **kw)
        args = (g, beta, beta)
    elif variant == "gla":
        out, fin = D.chunk_gla(qt, kt, vt, gt, **kw)
        args = (g, zeros, ones)
    else:
        out, fin = D.chunk_delta_rule(qt, kt, vt, bt, **kw)
        args = (zeros, beta, beta)
    ((out.float() * to_dev(do)).sum() + (fin * to_dev(df)).sum()).backward()
    torch.cuda.synchronize()
    o_ref, f_ref = O.chunk_gdn2(q, k, v, *args, initial_state=init, output_final_state=True)
    assert rel_l2(as_np(out), o_ref) < 1e-4 and rel_l2(as_np(fin), f_ref) < 1e-4
    ref = GR.chunk_gdn2_vjp(q, k, v, *args, do, df, initial_state=init)
    got = {"dq": as_np(qt.grad), "dk": as_np(kt.grad), "dv": as_np(vt.grad)}
    if variant != "delta_rule":
        got["dg"] = as_np(gt.grad)
    if variant != "gla":
        got["db"] = as_np(bt.grad)
        ref = dict(ref, db=ref["db"] + ref["dw"])   # beta feeds both b and w
    if has_init:
        got["dinit"] = as_np(it.grad)
    compare(got, {n: ref[n] for n in got}, 1e-4, f"variant {variant} Hk={Hk} Hv={Hv} init={has_init}")


def test_backward_full_size_cfg2_vs_torch_fp32():
    """BASELINE config-2 shape (B=1, L=2048, Hk=12, Hv=24), fp32 inputs,
    segment reset at 1024: the HIP backward against torch.autograd through the
    oracle's token-serial restatement run in float32 on the GPU (the float64
    oracle is too slow at this size; the fp32 reference's own rounding over
    2048 tokens bounds the comparison at 1e-4)."""
    from deltanet_tpu_amd import chunk_gdn2
    B, L, Hk, Hv, K = 1, 2048, 12, 24, 128
    gen = torch.Generator(device="cuda").manual_seed(77)
    r = lambda *s: torch.randn(*s, device="cuda", generator=gen)
    q, k, v = r(B, L, Hk, K), r(B, L, Hk, K), r(B, L, Hv, K)
    g = -torch.exp(0.39 * r(B, L, Hk, K) - 1.0)
    b, w = torch.sigmoid(0.39 * r(B, L, Hk, K)), torch.sigmoid(0.39 * r(B, L, Hv, K))
    seg = (torch.arange(L, device="cuda") >= 1024).to(torch.int32)[None]
    do = r(B, L, Hv, K)
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v, g, b, w)]
    out = chunk_gdn2(*leaves, segment_ids=seg, is_inference=False, qk_l2norm=True, precision="fp32")
    (out * do).sum().backward()
    got = [t.grad.detach() for t in leaves]
    ref_leaves = [t.clone().requires_grad_(True) for t in (q, k, v, g, b, w)]
    qh, kh, vv, ga, ba, wa = GR.prepare_torch(*ref_leaves, qk_l2norm=True)
    o_ref, _ = GR.torch_token_serial(qh, kh, vv, ga, ba, wa, seg.cpu().numpy(), None, None)
    (o_ref * do).sum().backward()
    ref = [t.grad.detach() for t in ref_leaves]
    e_o = rel_l2(as_np(out), as_np(o_ref))
    print(f"[measured] cfg2 full size: out rel L2 {e_o:.2e}", flush=True)
    assert e_o < 1e-4
    errs = {n: rel_l2(as_np(a_), as_np(b_)) for n, a_, b_ in zip(NAMES, got, ref)}
    print("[measured] cfg2 full size grads", {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e < 1e-4, (n, e)


@pytest.mark.parametrize("saturate, tol", [(False, 1e-5), (True, 1e-3)])
def test_backward_fuse_prologue_with_guard(saturate, tol):
    """fuse_prologue + stability_guard: raw g below ln(1e-6) (decay clamped to
    -1e-6, zero gradient: gdn2.py:133-142, 1972-1974) and, with `saturate`,
    above 5 (decay saturated at -e^5 per token, zero gradient), beside
    ordinary values; raw b logits of both signs.  A per-token decay of -e^5 is
    the strong-decay regime, checked at the reference's strong-decay
    tolerance (tests/test_strong_decay.py: 1e-3 in fp32).  Exact ties (raw
    g == 5) are avoided: the reference's minimum passes half the gradient
    there, a measure-zero case."""
    B, L, Hk, Hv, K, V = 1, 320, 2, 4, 128, 128
    rng = np.random.default_rng(4242)
    f = lambda *s: rng.standard_normal(s)
    q, k, v = f(B, L, Hk, K) * 0.1, f(B, L, Hk, K) * 0.1, f(B, L, Hv, V) * 0.1
    g = f(B, L, Hk, K) * 0.39 - 1.0
    sel = rng.random(g.shape)
    g = np.where(sel < 0.15, -16.0 - np.abs(f(B, L, Hk, K)), g)           # -exp(g) > -1e-6: clamped
    if saturate:
        g = np.where(sel > 0.9, 5.5 + np.abs(f(B, L, Hk, K)), g)          # saturated at -e^5
    b = f(B, L, Hk, K) * 0.8
    w = f(B, L, Hv, V) * 0.39
    init = f(B, Hv, K, V) * 0.05
    seg = np.array([[0] * 100 + [1] * 220], dtype=np.int32)
    do, df = f(B, L, Hv, V), f(B, Hv, K, V)
    kw = dict(qk_l2norm=True, fuse_prologue=True, stability_guard=True)
    _, got = run_dev(q, k, v, g, b, w, do, df=df, init=init, precision="fp32",
                     segment_ids=torch.from_numpy(seg).cuda(), **kw)
    ref = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do, df, initial_state=init, segment_ids=seg, **kw)
    compare(got, ref, tol, f"fuse_prologue + guard, saturate={saturate}")
    assert np.all(got["dg"][g < -14.0] == 0.0) and np.all(got["dg"][g > 5.0] == 0.0)
    assert np.abs(got["dg"][(g > -3) & (g < 0)]).max() > 0


@pytest.mark.parametrize("with_init, shape, precision, fuse", [
    (False, (2, 3000, 16, 32), "bf16", False), (True, (2, 3000, 16, 32), "bf16", False),
    (True, (1, 3000, 11, 33), "bf16", False),
    # the fp32 chain kernels (fp32 LDS state) and the fused prologue, in blocks
    (True, (2, 3000, 16, 32), "fp32", False), (False, (2, 3000, 16, 32), "bf16", True)])
def test_backward_recompute_states_bit_identical(with_init, shape, precision, fuse):
    """recompute_states=True (token blocks, only block-boundary states kept,
    chunk states recomputed per block: reference gdn2.py:655-695, 1614-1630)
    gives gradients bit-identical to the single-pass backward.  B * Hv = 64
    (batch, head) pairs make a block 16 chunks (1024 tokens), so L = 3000 runs
    three blocks; document boundaries sit inside and across block edges.  With
    B * Hv = 33 a block is 32 chunks (two blocks), and the forward-only scan
    launch has 132 column-block chains, not a multiple of the 8 XCDs (its
    padding blocks exit at once)."""
    from deltanet_tpu_amd import chunk_gdn2

    B, L, Hk, Hv = shape
    rng = np.random.default_rng(77)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    q, k, v = f(B, L, Hk, 128), f(B, L, Hk, 128), f(B, L, Hv, 128)
    if fuse:   # raw pre-activation gates; w channel-wise at the value heads
        g, b, w = f(B, L, Hk, 128), f(B, L, Hk, 128), f(B, L, Hv, 128)
    else:
        g = -np.exp(0.39 * f(B, L, Hk, 128) - 1.0)
        b, w = sig(0.39 * f(B, L, Hk, 128)), sig(0.39 * f(B, L, Hv, 128))
    seg = np.zeros((B, L), np.int32)
    seg[0, 1000:] = 1
    seg[0, 1024:] = 2        # a document starting exactly at the first block edge
    if B > 1:
        seg[1, 2100:] = 1
    init = (0.05 * f(B, Hv, 128, 128)) if with_init else None
    do, df = f(B, L, Hv, 128), f(B, Hv, 128, 128)
    res = {}
    for rc in (False, True):
        ts = [to_dev(x, torch.bfloat16 if i < 3 else torch.float32).requires_grad_(True)
              for i, x in enumerate((q, k, v, g, b, w))]
        ti = to_dev(init).requires_grad_(True) if with_init else None
        out, fin = chunk_gdn2(*ts, initial_state=ti, output_final_state=True, is_inference=False,
                              segment_ids=torch.from_numpy(seg).cuda(), qk_l2norm=True, precision=precision,
                              fuse_prologue=fuse, recompute_states=rc)
        ((out.float() * to_dev(do)).sum() + (fin * to_dev(df)).sum()).backward()
        torch.cuda.synchronize()
        res[rc] = {n: as_np(t.grad) for n, t in zip(NAMES, ts)}
        if with_init:
            res[rc]["dinit"] = as_np(ti.grad)
    for n in res[False]:
        a, c = res[False][n], res[True][n]
        assert np.isfinite(a).all(), n
        assert np.array_equal(a, c), f"{n}: max diff {np.abs(a.astype(np.float64) - c).max():.3e}"
    print(f"[measured] recompute_states bit-identical over {len(res[False])} gradients", flush=True)


def test_backward_w_in_place_and_staged_agree():
    """dn_prefill_bwd_raw reads a per-value-head channel-wise w in place (no
    staged copy) and stages every other layout.  The same write gate given
    at Hv heads (read in place) and at Hk heads (staged, broadcast over the G
    value heads of a key head) must give the same gradients: dq, dk, dv, dg,
    db bit-identical, dw at Hk equal to the sum over each key head's G value
    heads of dw at Hv."""
    from deltanet_tpu_amd import chunk_gdn2

    B, L, Hk, Hv = 2, 200, 2, 4
    G = Hv // Hk
    q, k, v, g, b, _ = ref_inputs(91, B, L, Hk, Hv)
    w_hk = sig(np.random.default_rng(92).standard_normal((B, L, Hk, 128)) * 0.39)
    w_hv = np.repeat(w_hk, G, axis=2)
    do = np.random.default_rng(93).standard_normal((B, L, Hv, 128))
    grads = {}
    for name, w in (("in_place", w_hv), ("staged", w_hk)):
        _, grads[name] = run_dev(q, k, v, g, b, w, do, precision="fp32")
    for n in ("dq", "dk", "dv", "dg", "db"):
        assert np.array_equal(grads["in_place"][n], grads["staged"][n]), n
    dw_sum = grads["in_place"]["dw"].reshape(B, L, Hk, G, 128).sum(axis=3)
    assert rel_l2(grads["staged"]["dw"], dw_sum) < 1e-6


def test_backward_config3_length_bf16_vs_fp32():
    """chunk_gdn (scalar per-head decay) training at the config-3 length:
    B=1, L=8192, Hk=16, Hv=32, geometric documents.  The bf16 mode's split-bf16
    scans carry ~2^-17 relative error per step, which accumulates over the
    128 chunk steps: measured 1.2e-4 (dq, dk, dv) and 4e-6 (dg, db) against
    the fp32 mode at this length (5e-6 at L <= 512).  The bound leaves 8x."""
    from deltanet_tpu_amd import chunk_gdn

    B, L, Hk, Hv = 1, 8192, 16, 32
    gen = torch.Generator(device="cuda").manual_seed(3)
    rn = lambda *s: torch.randn(*s, device="cuda", generator=gen)
    q, k, v = rn(B, L, Hk, 128).bfloat16(), rn(B, L, Hk, 128).bfloat16(), rn(B, L, Hv, 128).bfloat16()
    g = -torch.exp(torch.rand(Hv, device="cuda", generator=gen) * np.log(16.0)) * torch.nn.functional.softplus(rn(B, L, Hv))
    beta = torch.sigmoid(rn(B, L, Hv))
    rng = np.random.default_rng(3)
    bounds = np.cumsum(np.clip(rng.geometric(1.0 / 1024, size=64), 16, L))
    seg = torch.from_numpy(np.searchsorted(bounds, np.arange(L), side="right").astype(np.int32)[None]).cuda()
    do = rn(B, L, Hv, 128).bfloat16()
    grads = {}
    for prec in ("fp32", "bf16"):
        ts = [x.detach().clone().requires_grad_(True) for x in (q, k, v, g, beta)]
        out = chunk_gdn(*ts, segment_ids=seg, is_inference=False, qk_l2norm=True, precision=prec)
        out.backward(do)
        torch.cuda.synchronize()
        grads[prec] = [as_np(t.grad.float()) for t in ts]
    errs = [rel_l2(a, r) for a, r in zip(grads["bf16"], grads["fp32"])]
    print("[measured] config-3 length bf16 vs fp32:", " ".join(f"{e:.2e}" for e in errs), flush=True)
    for n, a, e in zip(("dq", "dk", "dv", "dg", "db"), grads["bf16"], errs):
        assert np.isfinite(a).all(), n
        assert e < 1e-3, f"{n}: rel L2 {e:.2e}"


def adversarial_batch(kind, L, *, eps=1e-4, period=2, seed=42):
    """The reference's adversarial generator (tests/test_nan_adversarial.py:39-99)
    with seeded NumPy: raw gates for the fused prologue, g = -10 (decay
    -e^-10), b = 5 (beta ~ 0.993), w = 0 (0.5); q, v, do ~ N(0, 1)."""
    rng = np.random.default_rng(seed)
    B, Hk, Hv = 1, 1, 1
    q = rng.standard_normal((B, L, Hk, 128))
    v = rng.standard_normal((B, L, Hv, 128))
    do = rng.standard_normal((B, L, Hv, 128))
    w = np.zeros((B, L, Hv, 128))
    g = np.full((B, L, Hk, 128), -10.0)
    b = np.full((B, L, Hk, 128), 5.0)
    if kind == "identical":
        k = np.repeat(rng.standard_normal((B, 1, Hk, 128)), L, 1)
    elif kind == "near":
        k = np.repeat(rng.standard_normal((B, 1, Hk, 128)), L, 1) + eps * rng.standard_normal((B, L, Hk, 128))
    else:   # periodic
        k = np.tile(rng.standard_normal((B, period, Hk, 128)), (1, L // period + 1, 1, 1))[:, :L]
    return q, k, v, g, b, w, do


# tests/test_nan_adversarial.py:116-208: every output and gradient finite; the
# bf16 forward within rel L2 0.10 (periodic keys 0.05) of the token-serial
# reference; the fp32 gradients within 1e-4 (identical and near-identical keys)
@pytest.mark.parametrize("kind, L, kw", [
    ("identical", 128, {}), ("identical", 512, {}), ("identical", 1024, {}),
    ("near", 512, {"eps": 1e-4}), ("near", 512, {"eps": 1e-2}), ("near", 512, {"eps": 1e-1}),
    ("periodic", 512, {"period": 2}), ("periodic", 512, {"period": 16}), ("periodic", 512, {"period": 64})])
def test_backward_adversarial_keys(kind, L, kw):
    q, k, v, g, b, w, do = adversarial_batch(kind, L, **kw)
    opts = dict(qk_l2norm=True, fuse_prologue=True)
    o_ref, _ = O.chunk_gdn2(q, k, v, g, b, w, is_inference=False, **opts)
    out_b, got_b = run_dev(q, k, v, g, b, w, do, precision="bf16", **opts)
    assert np.isfinite(out_b).all() and all(np.isfinite(x).all() for x in got_b.values() if x is not None)
    e_o = rel_l2(out_b, o_ref)
    print(f"[measured] adversarial {kind} L={L} {kw}: bf16 out rel L2 {e_o:.2e}", flush=True)
    assert e_o < (0.05 if kind == "periodic" else 0.10)
    if kind != "periodic":
        _, got = run_dev(q, k, v, g, b, w, do, precision="fp32", **opts)
        ref = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do, **opts)
        compare(got, ref, 1e-4, f"adversarial {kind} L={L} {kw} fp32")


def test_backward_alternating_keys_vanishing_decay():
    # tests/test_nan_adversarial.py:267-312: one-hot keys of alternating sign,
    # decay -e^-10, beta = sigmoid(10), w = 0.5; forward and gradients within
    # 1e-4 (a gradient whose reference norm is below 1e-6: within 1e-6 absolute)
    B, L, Hk, Hv = 1, 512, 2, 4
    rng = np.random.default_rng(1)
    k = np.zeros((B, L, Hk, 128))
    k[:, :, :, 0] = ((-1.0) ** np.arange(L))[None, :, None]
    q = 0.1 * rng.standard_normal((B, L, Hk, 128))
    v = 0.1 * rng.standard_normal((B, L, Hv, 128))
    g = np.full((B, L, Hk, 128), -10.0)
    b = np.full((B, L, Hk, 128), 10.0)
    w = np.zeros((B, L, Hv, 128))
    do = rng.standard_normal((B, L, Hv, 128))
    opts = dict(qk_l2norm=True, fuse_prologue=True)
    out, got = run_dev(q, k, v, g, b, w, do, precision="fp32", **opts)
    o_ref, _ = O.chunk_gdn2(q, k, v, g, b, w, is_inference=False, **opts)
    ref = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do, **opts)
    assert np.isfinite(out).all()
    assert rel_l2(out, o_ref) < 1e-4
    for n in NAMES:
        assert np.isfinite(got[n]).all(), n
        if np.linalg.norm(ref[n]) > 1e-6:
            e = rel_l2(got[n], ref[n])
            print(f"[measured] alternating keys {n}={e:.2e}", flush=True)
            assert e < 1e-4, (n, e)
        else:
            assert np.abs(got[n] - ref[n]).max() < 1e-6, n


@pytest.mark.parametrize("t_cut", [100, 128])
def test_backward_causality(t_cut):
    # tests/test_causality.py:27-74: with the loss on outputs before t_cut,
    # every gradient at t >= t_cut is exactly zero, and the gradients before
    # t_cut are bit-identical when every input from t_cut on is replaced
    from deltanet_tpu_amd import chunk_gdn2
    B, L, Hk, Hv = 1, 256, 2, 4
    a1 = ref_inputs(101, B, L, Hk, Hv)
    pert = ref_inputs(202, B, L - t_cut, Hk, Hv)
    a2 = tuple(np.concatenate([x[:, :t_cut], p], 1) for x, p in zip(a1, pert))
    grads = []
    for args in (a1, a2):
        ts = [to_dev(x).requires_grad_(True) for x in args]
        o = chunk_gdn2(*ts, is_inference=False, precision="fp32", chunk_size=128)
        (o[:, :t_cut] ** 2).sum().backward()
        torch.cuda.synchronize()
        grads.append([as_np(t.grad) for t in ts])
    for n, g1, g2 in zip(NAMES, *grads):
        assert np.all(g1[:, t_cut:] == 0.0), (n, float(np.abs(g1[:, t_cut:]).max()))
        assert np.array_equal(g1[:, :t_cut], g2[:, :t_cut]), (n, float(np.abs(g1[:, :t_cut] - g2[:, :t_cut]).max()))


def test_backward_gate_pass_through_at_zero():
    # tests/test_strong_decay.py:91-109: the nonpositive gate passes the full
    # gradient at g = 0 (not half, as min(g, 0) would) and none for g > 0;
    # a third of g exactly 0, a third positive
    B, L, Hk, Hv = 1, 192, 2, 4
    q, k, v, g, b, w = ref_inputs(19, B, L, Hk, Hv)
    sel = np.random.default_rng(20).integers(0, 3, g.shape)
    g = np.where(sel == 0, 0.0, np.where(sel == 1, 0.05, g))
    do = np.random.default_rng(21).standard_normal((B, L, Hv, 128))
    _, got = run_dev(q, k, v, g, b, w, do, precision="fp32")
    ref = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do)
    compare(got, ref, 1e-5, "g = 0 pass-through")
    assert np.all(got["dg"][sel == 1] == 0.0)
    assert np.abs(got["dg"][sel == 0]).max() > 0.0   # passed through (it matches the oracle above)


def test_scale_as_array_scalar():
    # tests/test_parity.py:286-318: scale given as an array scalar gives the
    # float's result bit for bit, on the default and the fused-prologue paths
    from deltanet_tpu_amd import chunk_gdn2
    B, L, Hk, Hv = 1, 128, 2, 4
    q, k, v, g, b, w = ref_inputs(555, B, L, Hk, Hv)
    ts = [to_dev(x) for x in (q, k, v, g, b, w)]
    for fuse in (False, True):
        kw = dict(fuse_prologue=fuse, qk_l2norm=fuse, precision="fp32", is_inference=True)
        o_f = chunk_gdn2(*ts, scale=0.2, **kw)
        for s in (np.float32(0.2), torch.tensor(0.2), torch.tensor(0.2, dtype=torch.float64)):
            assert torch.equal(chunk_gdn2(*ts, scale=s, **kw), o_f), (fuse, type(s))


@pytest.mark.parametrize("pattern", ["reused", "gaps"])
def test_backward_reused_segment_ids_weak_decay(pattern):
    # tests/test_document_boundaries.py:136-180: ids reused after another
    # document, and pad gaps between documents, under weak decay (g = -0.01);
    # output and every gradient within rel L2 1e-4
    from deltanet_tpu_amd import chunk_gdn2
    B, L, Hk, Hv = 1, 256, 2, 4
    seg = np.array([[0] * 40 + [1] * 40 + [0] * 176] if pattern == "reused"
                   else [[1] * 30 + [0] * 10 + [2] * 30 + [0] * 10 + [3] * 176], np.int32)
    q, k, v, g, b, w = ref_inputs(601, B, L, Hk, Hv)
    g = np.full_like(g, -0.01)
    do = np.random.default_rng(602).standard_normal((B, L, Hv, 128))
    ts = [to_dev(x).requires_grad_(True) for x in (q, k, v, g, b, w)]
    out = chunk_gdn2(*ts, segment_ids=to_dev(seg, torch.int32), is_inference=False, precision="fp32")
    (out * to_dev(do)).sum().backward()
    torch.cuda.synchronize()
    got = {n: as_np(t.grad) for n, t in zip(NAMES, ts)}
    o_ref, _ = O.chunk_gdn2(q, k, v, g, b, w, segment_ids=seg)
    assert rel_l2(as_np(out), o_ref) < 1e-4
    compare(got, GR.chunk_gdn2_vjp(q, k, v, g, b, w, do, segment_ids=seg), 1e-4, f"segment ids {pattern}")


@pytest.mark.parametrize("L", [1, 127, 1000])
def test_backward_arbitrary_lengths(L):
    # tests/test_arbitrary_lengths.py:23-78: one token, one short of a chunk,
    # and a ragged multi-chunk length, against the gradient oracle
    B, Hk, Hv = 1, 2, 4
    q, k, v, g, b, w = ref_inputs(1010 + L, B, L, Hk, Hv)
    do = np.random.default_rng(2020 + L).standard_normal((B, L, Hv, 128))
    out, got = run_dev(q, k, v, g, b, w, do, precision="fp32")
    assert out.shape == (B, L, Hv, 128) and got["dq"].shape == (B, L, Hk, 128)
    compare(got, GR.chunk_gdn2_vjp(q, k, v, g, b, w, do), 1e-5, f"L={L}")


def matrix_gates(rng, layout, regime, B, L, Hk, Hv):
    """Gate layouts and decay regimes of tests/test_matrix.py:60-128 (gdn2)."""
    Hg = Hv if layout == "per_value_head" else Hk
    if regime == "negative":
        g = -rng.uniform(0.1, 2.0, (B, L, Hg, 128))
    elif regime == "zero":
        g = np.zeros((B, L, Hg, 128))
    else:
        g = rng.uniform(0.1, 1.0, (B, L, Hg, 128))
    s = lambda *sh: sig(0.39 * rng.standard_normal(sh))
    if layout == "channel_wise":
        return g, s(B, L, Hk, 128), s(B, L, Hv, 128)
    if layout == "per_key_head":
        return g[..., :1], s(B, L, Hk, 1), s(B, L, Hv, 128)
    if layout == "per_value_head":
        return g[..., :1], s(B, L, Hv, 1), s(B, L, Hv, 128)
    if layout == "scalar":
        return g[..., 0], s(B, L, Hk), s(B, L, Hv)
    return g[:, :, :1], s(B, L, 1, 128), s(B, L, 1, 128)   # single_head


# tests/test_matrix.py:156-246: every gate layout x decay regime x head
# ratio, two documents per row, an initial state; output and final state,
# and the gradients of every input and of the initial state for a loss on
# both, within rel L2 1e-4 of the float64 oracle
@pytest.mark.parametrize("Hk,Hv", [(2, 2), (2, 4)])
@pytest.mark.parametrize("layout", ["channel_wise", "per_key_head", "per_value_head", "scalar", "single_head"])
@pytest.mark.parametrize("regime", ["negative", "zero", "positive"])
def test_backward_gate_matrix(Hk, Hv, layout, regime):
    B, L = 2, 300
    rng = np.random.default_rng(42)
    q, k = 0.1 * rng.standard_normal((2, B, L, Hk, 128))
    v = 0.1 * rng.standard_normal((B, L, Hv, 128))
    init = 0.05 * rng.standard_normal((B, Hv, 128, 128))
    g, b, w = matrix_gates(rng, layout, regime, B, L, Hk, Hv)
    seg = np.broadcast_to(np.array([0] * (L // 2) + [1] * (L - L // 2), np.int32), (B, L)).copy()
    do, df = rng.standard_normal((B, L, Hv, 128)), rng.standard_normal((B, Hv, 128, 128))
    from deltanet_tpu_amd import chunk_gdn2
    ts = [to_dev(x).requires_grad_(True) for x in (q, k, v, g, b, w)]
    ti = to_dev(init).requires_grad_(True)
    out, fin = chunk_gdn2(*ts, initial_state=ti, segment_ids=to_dev(seg, torch.int32), output_final_state=True,
                          is_inference=False, precision="fp32")
    ((out * to_dev(do)).sum() + (fin * to_dev(df)).sum()).backward()
    torch.cuda.synchronize()
    o_ref, f_ref = O.chunk_gdn2(q, k, v, g, b, w, segment_ids=seg, initial_state=init, output_final_state=True)
    assert rel_l2(as_np(out), o_ref) < 1e-4 and rel_l2(as_np(fin), f_ref) < 1e-4
    got = {n: as_np(t.grad) for n, t in zip(NAMES, ts)}
    got["dinit"] = as_np(ti.grad)
    ref = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do, df, segment_ids=seg, initial_state=init)
    compare(got, ref, 1e-4, f"matrix {layout} {regime} Hk={Hk} Hv={Hv}")


@pytest.mark.parametrize("Hk,Hv", [(2, 2), (2, 4)])
def test_backward_chained_calls(Hk, Hv):
    # tests/test_matrix.py:339-360: the second call starts from the first
    # call's final state; the gradient of a loss on the second call's output
    # and final state reaches the first call's inputs through that state.
    # Oracle: one call over the two sequences concatenated, with no output
    # cotangent on the first
    from deltanet_tpu_amd import chunk_gdn2
    B, L = 2, 300
    rng = np.random.default_rng(1)
    ins = []
    for _ in range(2):
        q, k = 0.1 * rng.standard_normal((2, B, L, Hk, 128))
        v = 0.1 * rng.standard_normal((B, L, Hv, 128))
        g, b, w = matrix_gates(rng, "channel_wise", "negative", B, L, Hk, Hv)
        ins.append((q, k, v, g, b, w))
    do2, df = rng.standard_normal((B, L, Hv, 128)), rng.standard_normal((B, Hv, 128, 128))
    kw = dict(output_final_state=True, precision="fp32", is_inference=False)
    t1 = [to_dev(x).requires_grad_(True) for x in ins[0]]
    t2 = [to_dev(x).requires_grad_(True) for x in ins[1]]
    _, s1 = chunk_gdn2(*t1, **kw)
    o2, s2 = chunk_gdn2(*t2, initial_state=s1, **kw)
    ((o2 * to_dev(do2)).sum() + (s2 * to_dev(df)).sum()).backward()
    torch.cuda.synchronize()
    cat = [np.concatenate([a, b_], 1) for a, b_ in zip(*ins)]
    do = np.concatenate([np.zeros_like(do2), do2], 1)
    ref = GR.chunk_gdn2_vjp(*cat, do, df)
    got = {n: np.concatenate([as_np(a.grad), as_np(b_.grad)], 1) for n, a, b_ in zip(NAMES, t1, t2)}
    compare(got, ref, 1e-4, f"chained calls Hk={Hk} Hv={Hv}")


@pytest.mark.parametrize("case", ["gdn2_hv_decay_hk_erase", "gdn_hk_decay_hv_beta"])
def test_backward_mixed_gate_heads(case):
    # tests/test_variants.py:125-236: decay and erase gates at different head
    # counts; output and gradients within rel L2 1e-5, and the first token's
    # decode step against the oracle
    import deltanet_tpu_amd as D
    B, L, Hk, Hv = 1, 128, 2, 4
    rng = np.random.default_rng(710)
    q, k = 0.1 * rng.standard_normal((2, B, L, Hk, 128))
    v = 0.1 * rng.standard_normal((B, L, Hv, 128))
    do = rng.standard_normal((B, L, Hv, 128))
    S0 = np.zeros((B, Hv, 128, 128))
    qt, kt, vt = (to_dev(x).requires_grad_(True) for x in (q, k, v))
    if case == "gdn2_hv_decay_hk_erase":
        g = -np.exp(0.39 * rng.standard_normal((B, L, Hv, 1)) - 1.0)
        b = sig(0.39 * rng.standard_normal((B, L, Hk, 128)))
        w = sig(0.39 * rng.standard_normal((B, L, Hv, 128)))
        gt, bt, wt = (to_dev(x).requires_grad_(True) for x in (g, b, w))
        out = D.chunk_gdn2(qt, kt, vt, gt, bt, wt, precision="fp32", is_inference=False)
        ref = GR.chunk_gdn2_vjp(q, k, v, g, b, w, do)
        names = NAMES
        leaves = (qt, kt, vt, gt, bt, wt)
        od, sd = D.gdn2_decode_step(*(to_dev(x[:, 0]) for x in (q, k, v, g, b, w)), to_dev(S0))
        rod, rsd = O.decode_step(q[:, 0], k[:, 0], v[:, 0], g[:, 0], b[:, 0], w[:, 0], S0)
    else:
        g = -np.exp(0.39 * rng.standard_normal((B, L, Hk, 1)) - 1.0)
        beta = sig(0.39 * rng.standard_normal((B, L, Hv, 1)))
        gt, bt = to_dev(g).requires_grad_(True), to_dev(beta).requires_grad_(True)
        out = D.chunk_gdn(qt, kt, vt, gt, bt, precision="fp32", is_inference=False)
        ref = GR.chunk_gdn2_vjp(q, k, v, g, beta, beta, do)
        ref = dict(ref, db=ref["db"] + ref["dw"])
        names = ("dq", "dk", "dv", "dg", "db")
        leaves = (qt, kt, vt, gt, bt)
        od, sd = D.gdn_decode_step(*(to_dev(x[:, 0]) for x in (q, k, v, g, beta)), to_dev(S0))
        rod, rsd = O.decode_step(q[:, 0], k[:, 0], v[:, 0], g[:, 0], beta[:, 0], beta[:, 0], S0)
    (out * to_dev(do)).sum().backward()
    torch.cuda.synchronize()
    o_ref, _ = O.chunk_gdn2(q, k, v, *((g, b, w) if case.startswith("gdn2") else (g, beta, beta)))
    assert rel_l2(as_np(out), o_ref) < 1e-5
    compare({n: as_np(t.grad) for n, t in zip(names, leaves)}, {n: ref[n] for n in names}, 1e-5, case)
    assert tuple(od.shape) == (B, Hv, 128) and tuple(sd.shape) == (B, Hv, 128, 128)
    assert rel_l2(as_np(od), rod) < 1e-5 and rel_l2(as_np(sd), rsd) < 1e-5


def test_backward_fuse_prologue_scale():
    # tests/test_parity.py:259-274 (scale on the fused path), with gradients:
    # raw gates, L2-norm, scale 0.2, rel L2 1e-5
    B, L, Hk, Hv = 1, 128, 2, 4
    rng = np.random.default_rng(333)
    q, k = 0.1 * rng.standard_normal((2, B, L, Hk, 128))
    v = 0.1 * rng.standard_normal((B, L, Hv, 128))
    g = 0.39 * rng.standard_normal((B, L, Hk, 128)) - 1.0
    b = 0.39 * rng.standard_normal((B, L, Hk, 128))
    w = 0.39 * rng.standard_normal((B, L, Hv, 128))
    do = rng.standard_normal((B, L, Hv, 128))
    kw = dict(qk_l2norm=True, fuse_prologue=True, scale=0.2)
    out, got = run_dev(q, k, v, g, b, w, do, precision="fp32", **kw)
    o_ref, _ = O.chunk_gdn2(q, k, v, g, b, w, is_inference=False, **kw)
    assert rel_l2(out, o_ref) < 1e-5
    compare(got, GR.chunk_gdn2_vjp(q, k, v, g, b, w, do, **kw), 1e-5, "fuse_prologue scale=0.2")
