"""GDN-2 chunked prefill and decode step on MI355X: the host side of the
drop-in for ``deltanet_tpu.chunk_gdn2`` / ``deltanet_tpu.gdn2_decode_step``
(maelie-labs/deltanet-tpu v0.3.0, src/deltanet_tpu/gdn2.py:1772-2490).

Same signatures, shapes, return convention and ``ValueError`` texts as the
reference; tensors are ``torch`` tensors on a ROCm device instead of
``jax.Array``.  The host code only validates, picks the execution mode and
fills the C-ABI argument block: the wrapper work the reference does as XLA
passes (gate broadcast, segment canonicalisation, padding, q/k L2-norm,
value-head fusion reshapes; gdn2.py:1970-2238) happens inside the HIP kernels.
There is no CPU path: a missing HIP library or a CPU tensor raises.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import torch

from . import _lib

__all__ = ["chunk_gdn2", "gdn2_decode_step"]

_DT = {torch.float32: _lib.DN_F32, torch.bfloat16: _lib.DN_BF16, torch.float16: _lib.DN_F16}
_CHUNK = 128


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_gpu(*ts):
    dev = None
    for t in ts:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"expected a torch.Tensor, got {type(t)}")
        if t.device.type != "cuda":
            raise RuntimeError(
                "deltanet_tpu_amd runs only on a ROCm GPU (HIP kernels, no CPU fallback); "
                f"got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"all tensors must be on one device, got {dev} and {t.device}")
    return dev


def _float_arg(t):
    """Gate / value operand as a contiguous tensor of a kernel-readable dtype."""
    if t.dtype not in _DT:
        t = t.to(torch.float32)
    return t.contiguous()


def _is_integer_dtype(dt):
    return not (dt.is_floating_point or dt.is_complex or dt == torch.bool)


class _NoGrad(torch.autograd.Function):
    """Forward-only op: its backward raises like the reference's inference op
    (gdn2.py:1436-1441)."""

    @staticmethod
    def forward(ctx, msg, run, *tensors):
        ctx.msg = msg
        res = run()
        return res

    @staticmethod
    def backward(ctx, *grads):
        raise ValueError(ctx.msg)


def _maybe_guard_grad(is_inference, run, tensors):
    """Inference calls whose inputs require grad get an op whose backward
    raises (gdn2.py:1436-1441).  Training calls that need gradients never
    reach this point (they take ``_TrainFn``)."""
    if is_inference and torch.is_grad_enabled() and any(
            isinstance(t, torch.Tensor) and t.requires_grad for t in tensors):
        msg = ("chunk_gdn2: differentiation is not supported when is_inference=True; "
               "set is_inference=False for training.")
        return _NoGrad.apply(msg, run, *[t for t in tensors if isinstance(t, torch.Tensor)])
    return run()


def chunk_gdn2(
    q, k, v, g, b, w, *,
    segment_ids=None,
    cu_seqlens=None,
    initial_state=None,
    initial_state_segment_id=None,
    output_final_state: bool = False,
    chunk_size: int = 128,
    precision: str = "bf16",
    scale=None,
    qk_l2norm: bool = False,
    fallback_scan: bool = False,
    is_inference: bool = False,
    fuse_prologue: bool = False,
    recompute_states: bool = False,
    streaming_prefill: bool = False,
    prefill_block_size: int = 4096,
    stability_guard: bool = False,
    stability_tau: float = 1000.0,
    truncate_bwd_dT_bf16: bool = False,
    state_fp32_matmul: bool = False,
    mask_lambda_by_doc: bool = False,
):
    """Forward pass of chunked-WY GDN-2 on MI355X (reference: gdn2.py:1772-2286).

    Args and returns as the reference ``chunk_gdn2``.  With ``is_inference=False``
    and inputs that require grad, the call is differentiable under torch.autograd
    (backward: ``dn_prefill_bwd_raw`` at the call's ``precision``, reference custom
    VJP gdn2.py:1446-1769).
    ``recompute_states=True`` runs that backward in token blocks, keeping only
    the states at block boundaries and recomputing each block's chunk states
    (reference gdn2.py:655-695, 1614-1630): less workspace, bit-identical
    gradients.  Flags that only shape the reference's TPU fallback
    (``fallback_scan``, ``truncate_bwd_dT_bf16``) are accepted and change no
    result.  ``state_fp32_matmul=True`` runs the call at ``precision="fp32"``.
    ``mask_lambda_by_doc`` is accepted and changes no result: the forward
    accumulates the decay in double-float and the backward restarts its
    cumulative decay at every document start inside a chunk, so a strongly
    decayed document never absorbs the next one's decay (the flag's
    precision concern; checked in tests/test_precision_flags_gpu.py).
    """
    # ---- validation: same checks and messages as gdn2.py:1858-1947 ----------
    if fuse_prologue and not qk_l2norm:
        raise ValueError(
            "fuse_prologue=True requires qk_l2norm=True because L2-normalization is fused directly into the VMEM kernel prologue."
        )
    if precision is None or not isinstance(precision, str):
        raise ValueError(f"precision must be a string ('bf16' or 'fp32'), got {precision!r}.")
    precision_clean = precision.lower()
    if precision_clean not in ("bf16", "bfloat16", "fp32", "float32"):
        raise ValueError(f"Invalid precision '{precision}'; must be 'bf16' or 'fp32'.")
    if chunk_size != 128:
        raise ValueError(f"Unsupported chunk_size={chunk_size}; Pallas TPU kernel requires chunk_size=128.")
    if stability_guard and isinstance(stability_tau, (int, float)) and not stability_tau > 0:
        raise ValueError(f"stability_tau must be positive, got {stability_tau}.")
    if streaming_prefill and isinstance(prefill_block_size, int) and not prefill_block_size > 0:
        raise ValueError(f"prefill_block_size must be positive, got {prefill_block_size}.")
    if q.ndim != 4:
        raise ValueError(f"Query tensor q must be 4D (B, L, Hk, K), got shape {tuple(q.shape)}.")
    if k.ndim != 4:
        raise ValueError(f"Key tensor k must be 4D (B, L, Hk, K), got shape {tuple(k.shape)}.")
    if v.ndim != 4:
        raise ValueError(f"Value tensor v must be 4D (B, L, Hv, V), got shape {tuple(v.shape)}.")
    B, L, Hk, K = q.shape
    Hv, V = v.shape[2], v.shape[3]
    if tuple(k.shape) != (B, L, Hk, K):
        raise ValueError(f"Key tensor k shape {tuple(k.shape)} must match query q shape ({B}, {L}, {Hk}, {K}).")
    if v.shape[0] != B or v.shape[1] != L:
        raise ValueError(f"Value tensor v shape {tuple(v.shape)} must match query batch and seq dimensions ({B}, {L}).")
    if K != 128 or V != 128:
        raise ValueError(f"Unsupported head dimensions (K={K}, V={V}); Pallas TPU kernel requires K=128 and V=128.")
    if Hv % Hk != 0:
        raise ValueError(f"Value heads ({Hv}) must be divisible by key heads ({Hk}).")
    for name, t, last in (("g", g, K), ("b", b, K), ("w", w, V)):
        hname = {"g": "Hg", "b": "Hb", "w": "Hw"}[name]
        cname = {"g": "Kg", "b": "Kb", "w": "Vw"}[name]
        if t.ndim not in (3, 4):
            raise ValueError(
                f"{name} must have rank 3 (B, L, {hname}) or rank 4 (B, L, {hname}, {cname}), got rank {t.ndim} with shape {tuple(t.shape)}.")
        if t.shape[0] != B or t.shape[1] != L:
            raise ValueError(f"{name} shape {tuple(t.shape)} must match query batch and seq dimensions ({B}, {L}).")
        if t.shape[2] not in (1, Hk, Hv):
            raise ValueError(
                f"{name} head dimension ({t.shape[2]}) must match key heads ({Hk}) or value heads ({Hv}) or be 1.")
        if t.ndim == 4 and t.shape[3] not in (1, last):
            lname = "K" if name != "w" else "V"
            raise ValueError(f"{name} last dimension ({t.shape[3]}) must be 1 or {lname} ({last}).")
    if segment_ids is not None and cu_seqlens is not None:
        raise ValueError("Cannot pass both segment_ids and cu_seqlens; specify at most one.")
    if segment_ids is not None:
        seg_dt = segment_ids.dtype if isinstance(segment_ids, torch.Tensor) else np.asarray(segment_ids).dtype
        is_int = _is_integer_dtype(seg_dt) if isinstance(seg_dt, torch.dtype) else np.issubdtype(seg_dt, np.integer)
        if not is_int:
            raise ValueError(f"segment_ids must have integer dtype, got {seg_dt}.")
        if segment_ids.ndim == 1:
            if segment_ids.shape[0] != L:
                raise ValueError(f"1D segment_ids length ({segment_ids.shape[0]}) must match sequence length ({L}).")
        elif segment_ids.ndim == 2:
            if tuple(segment_ids.shape) != (B, L):
                raise ValueError(f"2D segment_ids shape {tuple(segment_ids.shape)} must match (B={B}, L={L}).")
        else:
            raise ValueError(
                f"segment_ids must be 1D (L,) or 2D (B, L), got rank {segment_ids.ndim} with shape {tuple(segment_ids.shape)}.")
    if initial_state is not None and tuple(initial_state.shape) != (B, Hv, K, V):
        raise ValueError(
            f"initial_state shape {tuple(initial_state.shape)} must match (B={B}, Hv={Hv}, K={K}, V={V}).")

    if scale is None:
        scale = 1.0 / math.sqrt(K)
    else:
        try:
            scale = float(scale)
        except (TypeError, ValueError) as e:
            raise ValueError(f"chunk_gdn2: scale must be convertible to a concrete float, got {type(scale)}: {e}")

    # ---- segment ids (gdn2.py:2033-2079) -------------------------------------
    seg_t, seg_batched = None, 0
    if segment_ids is not None:
        seg_t = segment_ids if isinstance(segment_ids, torch.Tensor) else torch.as_tensor(np.asarray(segment_ids))
        if seg_t.dtype not in (torch.int32, torch.int64):
            seg_t = seg_t.to(torch.int64)
        seg_batched = 1 if seg_t.ndim == 2 else 0
    elif cu_seqlens is not None:
        cu = cu_seqlens.detach().cpu().numpy() if isinstance(cu_seqlens, torch.Tensor) else np.asarray(cu_seqlens)
        if len(cu) == 0 or int(cu[0]) != 0:
            raise ValueError(f"cu_seqlens[0] must be 0, got {cu[0] if len(cu) else 'empty'}.")
        if int(cu[-1]) != L:
            raise ValueError(f"cu_seqlens[-1] ({int(cu[-1])}) must equal sequence length ({L}).")
        lens = np.diff(cu.astype(np.int64))
        if len(lens) > 0 and np.any(lens <= 0):
            raise ValueError(f"cu_seqlens must be strictly monotonically increasing, got {cu_seqlens}.")
        seg_t = torch.from_numpy(np.repeat(np.arange(len(lens), dtype=np.int32), lens))
        seg_batched = 0

    dev = _require_gpu(q, k, v, g, b, w, initial_state,
                       segment_ids if isinstance(segment_ids, torch.Tensor) else None)
    if seg_t is not None:
        seg_t = seg_t.to(dev).contiguous()

    fp32 = precision_clean in ("fp32", "float32") or bool(state_fp32_matmul)

    # ---- execution mode (gdn2.py:1992-2007) ----------------------------------
    gates_at_hv = ((g.shape[2] == Hv) or (b.shape[2] == Hv)) and (Hk < Hv)

    def gate(t):
        t = t.to(torch.float32).contiguous()
        if t.ndim == 3:
            t = t.unsqueeze(-1)
        return t, int(t.shape[2]), int(t.shape[3])

    g_t, g_h, g_c = gate(g)
    b_t, b_h, b_c = gate(b)
    w_t, w_h, w_c = gate(w)
    if q.dtype not in _DT or k.dtype != q.dtype:
        q = q.to(torch.float32)
        k = k.to(torch.float32)
    q = q.contiguous()
    k = k.contiguous()
    out_dtype = v.dtype
    v_in = v.contiguous() if v.dtype in (torch.float32, torch.bfloat16) else v.to(torch.float32).contiguous()

    init = None
    if initial_state is not None:
        init = initial_state.to(torch.float32).contiguous()
    init_seg = None
    if initial_state is not None and initial_state_segment_id is not None:
        s = torch.as_tensor(initial_state_segment_id, dtype=torch.int64)
        init_seg = torch.broadcast_to(s.reshape(-1) if s.ndim else s, (B,)).to(torch.int32).to(dev).contiguous()

    lib = _lib.load_library()
    out = torch.empty((B, L, Hv, V), dtype=v_in.dtype, device=dev)
    final = torch.empty((B, Hv, K, V), dtype=torch.float32, device=dev)
    st = _stream(dev)

    args = _lib.PrefillArgs()
    args.abi_version = _lib.DN_ABI_VERSION
    args.B, args.L, args.Hk, args.Hv, args.K, args.V = B, L, Hk, Hv, K, V
    args.q, args.k, args.v = _ptr(q), _ptr(k), _ptr(v_in)
    args.qk_dtype, args.v_dtype = _DT[q.dtype], _DT[v_in.dtype]
    args.g, args.g_dtype, args.g_heads, args.g_chans = _ptr(g_t), _DT[g_t.dtype], g_h, g_c
    args.b, args.b_dtype, args.b_heads, args.b_chans = _ptr(b_t), _DT[b_t.dtype], b_h, b_c
    args.w, args.w_dtype, args.w_heads, args.w_chans = _ptr(w_t), _DT[w_t.dtype], w_h, w_c
    if seg_t is not None:
        args.seg = _ptr(seg_t)
        args.seg_dtype = _lib.DN_I64 if seg_t.dtype == torch.int64 else _lib.DN_I32
        args.seg_batched = seg_batched
    args.out = _ptr(out)
    args.final_state = _ptr(final)
    args.scale = scale
    args.qk_l2norm = int(bool(qk_l2norm))
    args.fuse_prologue = int(bool(fuse_prologue))
    args.stability_guard = int(bool(stability_guard))
    args.precision = 1 if fp32 else 0
    args.gates_at_hv = int(gates_at_hv)
    args.block_tokens = 0
    args.recompute_states = int(bool(recompute_states))

    tensors = (q, k, v, g, b, w, initial_state)

    if (not is_inference) and torch.is_grad_enabled() and any(
            isinstance(t, torch.Tensor) and t.requires_grad for t in tensors):
        # training op (gdn2.py:2244-2286): differentiable through dn_prefill_bwd_raw
        out, fin = _TrainFn.apply(q, k, v_in, g_t, b_t, w_t, init, (args, seg_t, init_seg))
        o = out if out.dtype == out_dtype else out.to(out_dtype)
        return (o, fin) if output_final_state else o

    def run():
        Lp = ((L + _CHUNK - 1) // _CHUNK) * _CHUNK
        if is_inference and streaming_prefill and Lp > prefill_block_size:
            if prefill_block_size % _CHUNK != 0:
                raise ValueError(
                    f"prefill_block_size ({prefill_block_size}) must be a multiple of chunk_size ({chunk_size}).")
            blocks = [(s0, min(prefill_block_size, L - s0)) for s0 in range(0, L, prefill_block_size)]
        else:
            blocks = [(0, L)]
        ws_bytes = 0
        for s0, n in blocks:
            args.t0, args.nt = s0, n
            ws_bytes = max(ws_bytes, lib.dn_prefill_workspace_size(ctypes.byref(args)))
        if ws_bytes == 0:
            _lib.check(-1, "dn_prefill_workspace_size")
        ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
        for i, (s0, n) in enumerate(blocks):
            args.t0, args.nt = s0, n
            if i == 0:
                args.init_state = _ptr(init)
                args.init_seg = _ptr(init_seg)
            else:
                args.init_state = _ptr(final)   # carried state (aliases final_state)
                args.init_seg = None
            _lib.check(lib.dn_prefill_fwd(ctypes.byref(args), _ptr(ws), ws_bytes, st), "dn_prefill_fwd")
            if len(blocks) > 1 and stability_guard:
                _lib.check(lib.dn_state_frob_cap(_ptr(final), B * Hv, K, V, float(stability_tau), st),
                           "dn_state_frob_cap")
        if len(blocks) == 1 and stability_guard and is_inference and output_final_state:
            _lib.check(lib.dn_state_frob_cap(_ptr(final), B * Hv, K, V, float(stability_tau), st),
                       "dn_state_frob_cap")
        o = out if out.dtype == out_dtype else out.to(out_dtype)
        if output_final_state:
            return o, final
        return o

    return _maybe_guard_grad(is_inference, run, tensors)


# ---------------------------------------------------------------------------
# training path: autograd around the HIP forward and backward
# ---------------------------------------------------------------------------

class _TrainFn(torch.autograd.Function):
    """chunk_gdn2 with is_inference=False (reference custom VJP,
    gdn2.py:1446-1769).  Forward: ``dn_prefill_fwd`` on the raw inputs (the
    wrapper steps run inside the kernels, as in inference).  Backward:
    ``dn_prefill_bwd_raw`` on the same argument block, which also
    differentiates the wrapper steps (prologue, L2-norm, gate broadcast, GQA)."""

    @staticmethod
    def _args(proto, q, k, v, g, b, w, init):
        a = _lib.PrefillArgs.from_buffer_copy(proto)
        a.q, a.k, a.v, a.g, a.b, a.w = (_ptr(x) for x in (q, k, v, g, b, w))
        a.init_state = _ptr(init)
        a.t0, a.nt = 0, a.L
        return a

    @staticmethod
    def forward(ctx, q, k, v, g, b, w, init, meta):
        proto, seg_t, init_seg = meta
        dev = q.device
        a = _TrainFn._args(proto, q, k, v, g, b, w, init)
        a.init_seg = _ptr(init_seg)
        out = torch.empty((a.B, a.L, a.Hv, a.V), dtype=v.dtype, device=dev)
        fin = torch.empty((a.B, a.Hv, a.K, a.V), dtype=torch.float32, device=dev)
        a.out, a.final_state = _ptr(out), _ptr(fin)
        lib = _lib.load_library()
        nbytes = lib.dn_prefill_workspace_size(ctypes.byref(a))
        if nbytes == 0:
            _lib.check(-1, "dn_prefill_workspace_size")
        ws = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
        _lib.check(lib.dn_prefill_fwd(ctypes.byref(a), _ptr(ws), nbytes, _stream(dev)), "dn_prefill_fwd")
        ctx.save_for_backward(q, k, v, g, b, w, init)
        ctx.meta = meta
        # an unused output (usually the final state) reaches backward as None
        # instead of a materialised zero tensor; the kernels take NULL for it
        ctx.set_materialize_grads(False)
        return out, fin

    @staticmethod
    def backward(ctx, d_out, d_fin):
        q, k, v, g, b, w, init = ctx.saved_tensors
        proto, seg_t, init_seg = ctx.meta
        dev = q.device
        a = _TrainFn._args(proto, q, k, v, g, b, w, init)
        a.init_seg = _ptr(init_seg)
        # dq, dk, dv come back in the input dtypes (rounded to nearest even in
        # the kernels), the gate gradients in f32; the output cotangent is read
        # in the output's (v's) dtype
        like = lambda t, dt: torch.empty(t.shape, dtype=dt, device=dev)
        dq, dk, dv = like(q, q.dtype), like(k, k.dtype), like(v, v.dtype)
        dg, db, dw = (like(x, torch.float32) for x in (g, b, w))
        d_init = like(init, torch.float32) if init is not None else None
        d_out = torch.zeros(v.shape, dtype=v.dtype, device=dev) if d_out is None \
            else d_out.to(v.dtype).contiguous()
        d_fin = None if d_fin is None else d_fin.to(torch.float32).contiguous()
        lib = _lib.load_library()
        nbytes = lib.dn_prefill_bwd_raw_workspace_size(ctypes.byref(a))
        if nbytes == 0:
            _lib.check(-1, "dn_prefill_bwd_raw_workspace_size")
        ws = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
        _lib.check(lib.dn_prefill_bwd_raw(ctypes.byref(a), _ptr(d_out), _ptr(d_fin), _ptr(dq), _ptr(dk), _ptr(dv),
                                          _ptr(dg), _ptr(db), _ptr(dw), _ptr(d_init), _ptr(ws), nbytes,
                                          _stream(dev)), "dn_prefill_bwd_raw")
        cast = lambda d, x: d if d.dtype == x.dtype else d.to(x.dtype)
        return (cast(dq, q), cast(dk, k), cast(dv, v), dg, db, dw, d_init, None)


def _decode_gate(t, B, Hk, Hv, last, name):
    t = _float_arg(t)
    if t.ndim == 2:
        t = t.unsqueeze(-1)
    return t, int(t.shape[1]), int(t.shape[2])


def gdn2_decode_step(
    q, k, v, g, b, w, state, *,
    reset=None,
    scale=None,
    qk_l2norm: bool = False,
    state_dtype=None,
    stability_guard: bool = False,
    stability_tau: float = 1000.0,
    out_state=None,
):
    """Single-token GDN-2 decode step on MI355X (reference: gdn2.py:2289-2490).

    Returns ``(output, new_state)`` like the reference.  ``out_state`` (an
    extension) lets the caller supply the new-state buffer, e.g. ``state``
    itself for an in-place update when the dtypes match.
    """
    if stability_guard and isinstance(stability_tau, (int, float)) and not stability_tau > 0:
        raise ValueError(f"stability_tau must be positive, got {stability_tau}.")
    out_dtype = v.dtype
    orig_ndim = q.ndim
    if orig_ndim not in (3, 4):
        raise ValueError(f"Query q must have rank 3 (B, Hk, K) or rank 4 (B, 1, Hk, K), got shape {tuple(q.shape)}.")
    if k.ndim != orig_ndim:
        raise ValueError(f"Key k rank ({k.ndim}) must match query rank ({orig_ndim}).")
    if v.ndim != orig_ndim:
        raise ValueError(f"Value v rank ({v.ndim}) must match query rank ({orig_ndim}).")
    if orig_ndim == 4:
        if q.shape[1] != 1 or k.shape[1] != 1 or v.shape[1] != 1:
            raise ValueError(
                f"Decode step sequence dimension must be 1, got q={tuple(q.shape)}, k={tuple(k.shape)}, v={tuple(v.shape)}.")
        q, k, v = q[:, 0], k[:, 0], v[:, 0]
        if g.ndim in (3, 4) and g.shape[1] == 1:
            g = g[:, 0]
        if b.ndim in (3, 4) and b.shape[1] == 1:
            b = b[:, 0]
        if w.ndim in (3, 4) and w.shape[1] == 1:
            w = w[:, 0]
    B, Hk, K = q.shape
    if v.ndim != 3 or v.shape[0] != B:
        raise ValueError(f"Value tensor v batch dimension ({v.shape[0]}) must match query batch dimension ({B}).")
    Hv, V = v.shape[1], v.shape[2]
    if g.ndim in (3, 4) and g.shape[0] == B and g.shape[1] == 1 and g.shape[2] in (1, Hk, Hv):
        g = g[:, 0]
    if b.ndim in (3, 4) and b.shape[0] == B and b.shape[1] == 1 and b.shape[2] in (1, Hk, Hv):
        b = b[:, 0]
    if w.ndim in (3, 4) and w.shape[0] == B and w.shape[1] == 1 and w.shape[2] in (1, Hk, Hv):
        w = w[:, 0]
    if tuple(k.shape) != (B, Hk, K):
        raise ValueError(f"Key tensor k shape {tuple(k.shape)} must match query q shape ({B}, {Hk}, {K}).")
    if K != 128 or V != 128:
        raise ValueError(f"Unsupported head dimensions (K={K}, V={V}); requires K=128 and V=128.")
    if Hv % Hk != 0:
        raise ValueError(f"Value heads ({Hv}) must be divisible by key heads ({Hk}).")
    if tuple(state.shape) != (B, Hv, K, V):
        raise ValueError(f"state shape {tuple(state.shape)} must match ({B}, {Hv}, {K}, {V}).")
    if state_dtype is not None:
        sd = state_dtype
        if isinstance(sd, str):
            sd = {"float32": torch.float32, "fp32": torch.float32, "bfloat16": torch.bfloat16,
                  "bf16": torch.bfloat16}.get(sd.lower())
        elif not isinstance(sd, torch.dtype):
            sd = {np.dtype("float32"): torch.float32}.get(np.dtype(sd), None) if not hasattr(sd, "name") \
                else {"float32": torch.float32, "bfloat16": torch.bfloat16}.get(sd.name)
        if sd not in (torch.float32, torch.bfloat16):
            raise ValueError(f"state_dtype must be float32 or bfloat16, got {state_dtype!r}.")
        target_state_dtype = sd
    else:
        target_state_dtype = torch.float32
    for name, t, last in (("g", g, K), ("b", b, K), ("w", w, V)):
        if (t.ndim not in (2, 3) or t.shape[0] != B or t.shape[1] not in (1, Hk, Hv)
                or (t.ndim == 3 and t.shape[2] not in (1, last))):
            dim = "K" if name != "w" else "V"
            raise ValueError(f"{name} shape {tuple(t.shape)} invalid for batch={B}, Hk={Hk}, Hv={Hv}, {dim}={last}.")

    reset_t = None
    if reset is not None:
        r = reset if isinstance(reset, torch.Tensor) else torch.as_tensor(np.asarray(reset))
        if r.ndim > 0 and r.shape[0] != B:
            raise ValueError(f"reset batch dimension ({r.shape[0]}) must match input batch dimension ({B}).")
        if r.ndim > 4:
            raise ValueError(f"reset ndim ({r.ndim}) cannot exceed 4.")
        r = r.reshape(-1) if r.ndim > 0 else r.reshape(1)
        if r.numel() != 1 and r.numel() != B:
            raise ValueError(f"reset batch dimension ({r.shape[0]}) must match input batch dimension ({B}).")
        if r.numel() == B and r.dtype in (torch.bool, torch.uint8) and r.is_cuda and r.is_contiguous():
            # one byte per row, nonzero = reset: read in place (no conversion copy per step)
            reset_t = r
        else:
            reset_t = torch.broadcast_to(r.to(torch.bool), (B,)).to(torch.uint8)

    dev = _require_gpu(q, k, v, g, b, w, state)
    if reset_t is not None and (reset_t.device != dev or not reset_t.is_contiguous()):
        reset_t = reset_t.to(dev).contiguous()
    if scale is None:
        scale = 1.0 / math.sqrt(K)
    if q.dtype not in _DT or k.dtype != q.dtype:
        q = q.to(torch.float32)
        k = k.to(torch.float32)
    q, k = q.contiguous(), k.contiguous()
    v_in = _float_arg(v)
    g_t, g_h, g_c = _decode_gate(g, B, Hk, Hv, K, "g")
    b_t, b_h, b_c = _decode_gate(b, B, Hk, Hv, K, "b")
    w_t, w_h, w_c = _decode_gate(w, B, Hk, Hv, V, "w")
    s_in = state
    if s_in.dtype not in (torch.float32, torch.bfloat16):
        s_in = s_in.to(torch.float32)
    s_in = s_in.contiguous()
    if out_state is not None:
        if tuple(out_state.shape) != (B, Hv, K, V) or out_state.dtype != target_state_dtype or not out_state.is_contiguous():
            raise ValueError("out_state must be a contiguous (B, Hv, K, V) tensor of state_dtype.")
        s_out = out_state
    else:
        s_out = torch.empty((B, Hv, K, V), dtype=target_state_dtype, device=dev)
    out = torch.empty((B, Hv, V), dtype=v_in.dtype, device=dev)

    a = _lib.DecodeArgs()
    a.abi_version = _lib.DN_ABI_VERSION
    a.B, a.Hk, a.Hv, a.K, a.V = B, Hk, Hv, K, V
    a.q, a.k, a.v = _ptr(q), _ptr(k), _ptr(v_in)
    a.qk_dtype, a.v_dtype = _DT[q.dtype], _DT[v_in.dtype]
    a.g, a.g_dtype, a.g_heads, a.g_chans = _ptr(g_t), _DT[g_t.dtype], g_h, g_c
    a.b, a.b_dtype, a.b_heads, a.b_chans = _ptr(b_t), _DT[b_t.dtype], b_h, b_c
    a.w, a.w_dtype, a.w_heads, a.w_chans = _ptr(w_t), _DT[w_t.dtype], w_h, w_c
    a.state_in, a.state_in_dtype = _ptr(s_in), _DT[s_in.dtype]
    a.state_out, a.state_out_dtype = _ptr(s_out), _DT[s_out.dtype]
    a.reset = _ptr(reset_t)
    a.out = _ptr(out)
    a.scale = float(scale)
    a.qk_l2norm = int(bool(qk_l2norm))
    a.stability_guard = int(bool(stability_guard))
    a.stability_tau = float(stability_tau)
    lib = _lib.load_library()
    _lib.check(lib.dn_decode_step(ctypes.byref(a), _stream(dev)), "dn_decode_step")
    o = out if out.dtype == out_dtype else out.to(out_dtype)
    if orig_ndim == 4:
        o = o[:, None]
    return o, s_out


def gdn2_decode_steps(
    q, k, v, g, b, w, state, *,
    reset=None,
    scale=None,
    qk_l2norm: bool = False,
    state_dtype=None,
    stability_guard: bool = False,
    stability_tau: float = 1000.0,
    out_state=None,
):
    """T consecutive GDN-2 decode steps in one launch (an extension: the
    reference has the single step only, gdn2.py:2289-2490).

    q, k: (B, T, Hk, K); v: (B, T, Hv, V); g, b: (B, T, Hx) or (B, T, Hx, K)
    and w: (B, T, Hx) or (B, T, Hx, V) with Hx in {1, Hk, Hv}; state
    (B, Hv, K, V).  ``reset`` is None, (B,) (clear the state before the first
    token) or (B, T) (clear it before each marked token).  Returns
    ``(output (B, T, Hv, V), new_state)``: the recurrence of T chained
    ``gdn2_decode_step`` calls with the state read and written once.  From 6
    tokens without the stability guard the launch runs the tokens as 16-token
    chunks in the WY form on matrix cores and carries the state in fp32,
    rounding a bfloat16 ``state_dtype`` once at the end; shorter launches (and
    those with the guard) round it after every token as chained calls do.
    """
    if stability_guard and isinstance(stability_tau, (int, float)) and not stability_tau > 0:
        raise ValueError(f"stability_tau must be positive, got {stability_tau}.")
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError(f"q, k, v must have rank 4 (B, T, H, D), got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}.")
    B, T, Hk, K = q.shape
    if tuple(k.shape) != (B, T, Hk, K):
        raise ValueError(f"Key tensor k shape {tuple(k.shape)} must match query q shape ({B}, {T}, {Hk}, {K}).")
    if v.shape[0] != B or v.shape[1] != T:
        raise ValueError(f"Value tensor v shape {tuple(v.shape)} must start with (B, T) = ({B}, {T}).")
    Hv, V = v.shape[2], v.shape[3]
    if K != 128 or V != 128:
        raise ValueError(f"Unsupported head dimensions (K={K}, V={V}); requires K=128 and V=128.")
    if Hv % Hk != 0:
        raise ValueError(f"Value heads ({Hv}) must be divisible by key heads ({Hk}).")
    if T < 1:
        raise ValueError(f"T must be at least 1, got {T}.")
    if tuple(state.shape) != (B, Hv, K, V):
        raise ValueError(f"state shape {tuple(state.shape)} must match ({B}, {Hv}, {K}, {V}).")
    if state_dtype is not None:
        sd = state_dtype
        if isinstance(sd, str):
            sd = {"float32": torch.float32, "fp32": torch.float32, "bfloat16": torch.bfloat16,
                  "bf16": torch.bfloat16}.get(sd.lower())
        if sd not in (torch.float32, torch.bfloat16):
            raise ValueError(f"state_dtype must be float32 or bfloat16, got {state_dtype!r}.")
        target_state_dtype = sd
    else:
        target_state_dtype = torch.float32
    for name, t, last in (("g", g, K), ("b", b, K), ("w", w, V)):
        if (t.ndim not in (3, 4) or t.shape[0] != B or t.shape[1] != T or t.shape[2] not in (1, Hk, Hv)
                or (t.ndim == 4 and t.shape[3] not in (1, last))):
            dim = "K" if name != "w" else "V"
            raise ValueError(f"{name} shape {tuple(t.shape)} invalid for batch={B}, T={T}, Hk={Hk}, Hv={Hv}, {dim}={last}.")
    reset_t = None
    if (isinstance(reset, torch.Tensor) and tuple(reset.shape) == (B, T) and reset.dtype in (torch.bool, torch.uint8)
            and reset.is_cuda and reset.is_contiguous()):
        # one byte per (row, token), nonzero = reset: read in place
        reset_t = reset
    elif reset is not None:
        r = reset if isinstance(reset, torch.Tensor) else torch.as_tensor(np.asarray(reset))
        r = r.to(torch.bool)
        if r.ndim == 0:
            r = r.reshape(1)
        if r.ndim == 1:
            if r.numel() not in (1, B):
                raise ValueError(f"reset batch dimension ({r.shape[0]}) must match input batch dimension ({B}).")
            first = torch.broadcast_to(r, (B,))
            r = torch.zeros((B, T), dtype=torch.bool, device=r.device)
            r[:, 0] = first
        elif tuple(r.shape) != (B, T):
            raise ValueError(f"reset must have shape (B,) or (B, T) = ({B}, {T}), got {tuple(r.shape)}.")
        reset_t = r.to(torch.uint8)

    dev = _require_gpu(q, k, v, g, b, w, state)
    if reset_t is not None and (reset_t.device != dev or not reset_t.is_contiguous()):
        reset_t = reset_t.to(dev).contiguous()
    if scale is None:
        scale = 1.0 / math.sqrt(K)
    if q.dtype not in _DT or k.dtype != q.dtype:
        q = q.to(torch.float32)
        k = k.to(torch.float32)
    q, k = q.contiguous(), k.contiguous()
    v_in = _float_arg(v)
    # the kernel indexes every per-token tensor as (B*T, ...): fold T into B
    fold = lambda t: t.reshape((B * T,) + tuple(t.shape[2:]))
    g_t, g_h, g_c = _decode_gate(fold(g), B * T, Hk, Hv, K, "g")
    b_t, b_h, b_c = _decode_gate(fold(b), B * T, Hk, Hv, K, "b")
    w_t, w_h, w_c = _decode_gate(fold(w), B * T, Hk, Hv, V, "w")
    s_in = state
    if s_in.dtype not in (torch.float32, torch.bfloat16):
        s_in = s_in.to(torch.float32)
    s_in = s_in.contiguous()
    if out_state is not None:
        if tuple(out_state.shape) != (B, Hv, K, V) or out_state.dtype != target_state_dtype or not out_state.is_contiguous():
            raise ValueError("out_state must be a contiguous (B, Hv, K, V) tensor of state_dtype.")
        s_out = out_state
    else:
        s_out = torch.empty((B, Hv, K, V), dtype=target_state_dtype, device=dev)
    out = torch.empty((B, T, Hv, V), dtype=v_in.dtype, device=dev)

    a = _lib.DecodeArgs()
    a.abi_version = _lib.DN_ABI_VERSION
    a.B, a.Hk, a.Hv, a.K, a.V = B, Hk, Hv, K, V
    a.q, a.k, a.v = _ptr(q), _ptr(k), _ptr(v_in)
    a.qk_dtype, a.v_dtype = _DT[q.dtype], _DT[v_in.dtype]
    a.g, a.g_dtype, a.g_heads, a.g_chans = _ptr(g_t), _DT[g_t.dtype], g_h, g_c
    a.b, a.b_dtype, a.b_heads, a.b_chans = _ptr(b_t), _DT[b_t.dtype], b_h, b_c
    a.w, a.w_dtype, a.w_heads, a.w_chans = _ptr(w_t), _DT[w_t.dtype], w_h, w_c
    a.state_in, a.state_in_dtype = _ptr(s_in), _DT[s_in.dtype]
    a.state_out, a.state_out_dtype = _ptr(s_out), _DT[s_out.dtype]
    a.reset = _ptr(reset_t)
    a.out = _ptr(out)
    a.scale = float(scale)
    a.qk_l2norm = int(bool(qk_l2norm))
    a.stability_guard = int(bool(stability_guard))
    a.stability_tau = float(stability_tau)
    lib = _lib.load_library()
    _lib.check(lib.dn_decode_steps(ctypes.byref(a), int(T), _stream(dev)), "dn_decode_steps")
    o = out if out.dtype == v.dtype else out.to(v.dtype)
    return o, s_out

