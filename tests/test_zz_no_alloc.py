"""The allocation-free prefill entry point (dn_prefill_fwd_noalloc, scratch in a
file-scope device array) against dn_prefill_fwd with a caller workspace,
through the C-ABI: bit-identical outputs and final states, on two calls in a
row, the second with a smaller input (the scratch keeps the first call's
contents).  The refusal of oversized shapes is a host-only check
(tests/test_capi.py)."""

import ctypes
import math

import pytest
import torch

from deltanet_tpu_amd import _lib

pytestmark = pytest.mark.gpu


def _call_args(B, L, Hk, Hv, seed, precision, with_init):
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    rn = lambda *s: torch.randn(*s, device=dev, generator=gen)
    keep = {
        "q": rn(B, L, Hk, 128).to(torch.bfloat16),
        "k": rn(B, L, Hk, 128).to(torch.bfloat16),
        "v": rn(B, L, Hv, 128).to(torch.bfloat16),
        "g": -torch.exp(0.39 * rn(B, L, Hk, 128) - 1.0),
        "b": torch.sigmoid(0.39 * rn(B, L, Hk, 128)),
        "w": torch.sigmoid(0.39 * rn(B, L, Hv, 128)),
        "seg": (torch.arange(L, device=dev) >= L // 3).to(torch.int32)[None].repeat(B, 1).contiguous(),
        "init": (0.05 * rn(B, Hv, 128, 128)) if with_init else None,
    }
    a = _lib.PrefillArgs()
    a.abi_version = _lib.DN_ABI_VERSION
    a.B, a.L, a.Hk, a.Hv, a.K, a.V = B, L, Hk, Hv, 128, 128
    a.t0, a.nt = 0, L
    a.q, a.k, a.v = (keep[n].data_ptr() for n in ("q", "k", "v"))
    a.qk_dtype = a.v_dtype = _lib.DN_BF16
    a.g, a.g_dtype, a.g_heads, a.g_chans = keep["g"].data_ptr(), _lib.DN_F32, Hk, 128
    a.b, a.b_dtype, a.b_heads, a.b_chans = keep["b"].data_ptr(), _lib.DN_F32, Hk, 128
    a.w, a.w_dtype, a.w_heads, a.w_chans = keep["w"].data_ptr(), _lib.DN_F32, Hv, 128
    a.seg, a.seg_dtype, a.seg_batched = keep["seg"].data_ptr(), _lib.DN_I32, 1
    a.init_state = keep["init"].data_ptr() if with_init else None
    a.scale = 1.0 / math.sqrt(128)
    a.qk_l2norm = 1
    a.precision = precision
    return a, keep


def _run(a, keep, noalloc):
    lib = _lib.load_library()
    out = torch.full((a.B, a.L, a.Hv, 128), float("nan"), dtype=torch.bfloat16, device="cuda:0")
    fin = torch.full((a.B, a.Hv, 128, 128), float("nan"), dtype=torch.float32, device="cuda:0")
    a.out, a.final_state = out.data_ptr(), fin.data_ptr()
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.dn_prefill_fwd_noalloc(ctypes.byref(a), stream)
    else:
        n = lib.dn_prefill_workspace_size(ctypes.byref(a))
        ws = torch.empty((n,), dtype=torch.uint8, device="cuda:0")
        rc = lib.dn_prefill_fwd(ctypes.byref(a), ws.data_ptr(), n, stream)
    assert rc == 0, lib.dn_last_error()
    torch.cuda.synchronize()
    return out, fin


@pytest.mark.parametrize("precision", [0, 1])
def test_noalloc_matches_workspace_entry(precision):
    # first call: 36 (batch, head) pairs x 24 chunks (more than the scratch
    # holds at once, so the entry runs several token blocks); second call
    # smaller, with an initial state and an unaligned length
    for (B, L, Hk, Hv, seed, init) in ((3, 3072, 12, 24, 11, False), (1, 600, 4, 8, 12, True)):
        print(f"[case] precision={precision} B={B} L={L} Hk={Hk} Hv={Hv} init={init}", flush=True)
        a, keep = _call_args(B, L, Hk, Hv, seed, precision, init)
        o_ref, f_ref = _run(a, keep, noalloc=False)
        o, f = _run(a, keep, noalloc=True)
        assert torch.isfinite(o_ref.float()).all() and torch.isfinite(f_ref).all()
        assert torch.equal(o, o_ref), (o.float() - o_ref.float()).abs().max().item()
        assert torch.equal(f, f_ref), (f - f_ref).abs().max().item()

