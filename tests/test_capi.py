"""The C-ABI library loads and exports every entry point include/deltanet_amd.h
declares, and the ctypes mirrors of the argument structs have the C layout
(compiled here with gcc from the header).  No compute calls: CPU-only."""

import ctypes
import os
import re
import subprocess

import pytest

from deltanet_tpu_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "deltanet_amd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dn_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_symbols():
    assert declared_functions() == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT\s+(dn_[a-z0-9_]+)\b", out))
    missing = [f for f in declared_functions() if f not in exported]
    assert not missing, f"missing exports: {missing}"
    lib = _lib.load_library()
    assert lib.dn_abi_version() == _lib.DN_ABI_VERSION
    assert lib.dn_last_error() == b""


def test_struct_layout_matches_header(tmp_path):
    fields = {
        "dn_prefill_args": _lib.PrefillArgs,
        "dn_decode_args": _lib.DecodeArgs,
        "dn_backward_args": _lib.BackwardArgs,
    }
    src = ['#include <stdio.h>', '#include <stddef.h>', '#include "deltanet_amd.h"', "int main(void){"]
    for cname, cls in fields.items():
        src.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            src.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    src.append("return 0;}")
    c = tmp_path / "layout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(c), "-o", str(exe)], check=True)
    got = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    for line in filter(None, got):
        parts = line.split()
        cls = fields[parts[0]]
        if parts[1] == "size":
            assert ctypes.sizeof(cls) == int(parts[2]), line
        else:
            assert getattr(cls, parts[1]).offset == int(parts[2]), line


def test_invalid_args_rejected_without_gpu():
    """Argument checking happens before any HIP call, so it runs on the CPU."""
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    lib = _lib.load_library()
    a = _lib.PrefillArgs()
    a.abi_version = _lib.DN_ABI_VERSION
    a.B, a.L, a.Hk, a.Hv, a.K, a.V = 1, 128, 2, 4, 64, 64
    assert lib.dn_prefill_workspace_size(ctypes.byref(a)) == 0
    rc = lib.dn_prefill_fwd(ctypes.byref(a), None, 0, None)
    assert rc == -1 and b"128" in lib.dn_last_error()
    a.abi_version = 99
    assert lib.dn_prefill_fwd(ctypes.byref(a), None, 0, None) == -4
    d = _lib.DecodeArgs()
    d.abi_version = _lib.DN_ABI_VERSION
    d.B, d.Hk, d.Hv, d.K, d.V = 1, 2, 3, 128, 128
    assert lib.dn_decode_step(ctypes.byref(d), None) == -1
    assert lib.dn_decode_steps(ctypes.byref(d), 4, None) == -1
    d.Hv = 4
    assert lib.dn_decode_steps(ctypes.byref(d), 0, None) == -1 and b"T must be positive" in lib.dn_last_error()
    assert lib.dn_state_frob_cap(None, 1, 128, 128, 1.0, None) == -1
    bw = _lib.BackwardArgs()
    bw.abi_version = _lib.DN_ABI_VERSION
    bw.B, bw.L, bw.H, bw.K, bw.V = 1, 128, 4, 128, 128
    # missing tensor pointers: size 0 and a clear error, no HIP call
    assert lib.dn_prefill_bwd_workspace_size(ctypes.byref(bw)) == 0
    assert lib.dn_prefill_bwd(ctypes.byref(bw), None, 0, None) == -1 and b"missing" in lib.dn_last_error()
    bw.K = 64
    assert lib.dn_prefill_bwd(ctypes.byref(bw), None, 0, None) == -1 and b"128" in lib.dn_last_error()
    bw.abi_version = 99
    assert lib.dn_prefill_bwd(ctypes.byref(bw), None, 0, None) == -4
    # with (fake, never dereferenced) pointers the size is positive and a short
    # workspace is refused before any launch
    bw.abi_version, bw.K = _lib.DN_ABI_VERSION, 128
    for f in ("q", "k", "v", "g", "b", "w", "d_out", "dq", "dk", "dv", "dg", "db", "dw"):
        setattr(bw, f, 0x1000)
    need = lib.dn_prefill_bwd_workspace_size(ctypes.byref(bw))
    assert need == 4 * 2 * 4 * (9 * 64 * 128 + 4 * 64 * 64 + 2 * 128 + 3 * 128 * 128)   # bytes: 2 chunks x 4 heads
    assert lib.dn_prefill_bwd(ctypes.byref(bw), None, 0, None) == -2
    bw.d_init = 0x1000
    assert lib.dn_prefill_bwd(ctypes.byref(bw), None, 0, None) == -1 and b"init_state" in lib.dn_last_error()
    # raw-input backward: same argument block as the forward
    ra = _lib.PrefillArgs()
    ra.abi_version = _lib.DN_ABI_VERSION
    ra.B, ra.L, ra.Hk, ra.Hv, ra.K, ra.V = 1, 128, 2, 4, 128, 128
    assert lib.dn_prefill_bwd_raw_workspace_size(ctypes.byref(ra)) == 0       # no tensors
    for f in ("q", "k", "v", "g", "b", "w"):
        setattr(ra, f, 0x1000)
    ra.g_heads, ra.g_chans, ra.b_heads, ra.b_chans, ra.w_heads, ra.w_chans = 2, 128, 2, 128, 4, 128
    ra.qk_dtype, ra.v_dtype = _lib.DN_BF16, _lib.DN_BF16
    need = lib.dn_prefill_bwd_raw_workspace_size(ctypes.byref(ra))
    core = 4 * 2 * 4 * (9 * 64 * 128 + 4 * 64 * 64 + 2 * 128 + 3 * 128 * 128)
    hv_arr, hk_arr = 1 * 128 * 4 * 128 * 4, 1 * 128 * 2 * 128 * 4   # (B,L,Hv,128), (B,L,Hk,128) f32
    # seven arrays at Hv; q, k, and g, b (both at the key heads here) at Hk
    assert need == 512 + 7 * hv_arr + 4 * hk_arr + core
    ra.b_heads = 4   # b at the value heads: g and b prepared at Hv
    assert lib.dn_prefill_bwd_raw_workspace_size(ctypes.byref(ra)) == 512 + 9 * hv_arr + 2 * hk_arr + core
    ra.b_heads = 2
    fake = [0x1000] * 6 + [None]   # dq dk dv dg db dw, no d_init
    assert lib.dn_prefill_bwd_raw(ctypes.byref(ra), 0x1000, None, *fake, None, 0, None) == -2
    ra.g_heads = 3
    assert lib.dn_prefill_bwd_raw(ctypes.byref(ra), 0x1000, None, *fake, None, 0, None) == -1
    assert b"gate heads" in lib.dn_last_error()


def test_recompute_states_workspace_size():
    """recompute_states sizes the backward workspace for one token block (the
    smallest whole number of 64-token chunks giving >= 1024 (batch, head,
    chunk) units) plus one (B,H,128,128) f32 state per block boundary and one
    carried state gradient; without it, every chunk of the sequence."""
    lib = _lib.load_library()
    unit = 4 * (9 * 64 * 128 + 4 * 64 * 64 + 2 * 128 + 3 * 128 * 128)   # bytes per (batch, head, chunk)
    kk = 4 * 128 * 128
    bw = _lib.BackwardArgs()
    bw.abi_version = _lib.DN_ABI_VERSION
    for f in ("q", "k", "v", "g", "b", "w", "d_out", "dq", "dk", "dv", "dg", "db", "dw"):
        setattr(bw, f, 0x1000)
    bw.K = bw.V = 128
    for B, L, H in ((2, 3000, 32), (4, 8192, 32), (1, 2048, 24), (1, 128, 4)):
        bw.B, bw.L, bw.H = B, L, H
        NC = -(-L // 64)
        bw.recompute_states = 0
        full = lib.dn_prefill_bwd_workspace_size(ctypes.byref(bw))
        assert full == B * H * NC * unit
        bw.recompute_states = 1
        rec = lib.dn_prefill_bwd_workspace_size(ctypes.byref(bw))
        ncb = min(NC, max(1, -(-1024 // (B * H))))
        nblk = -(-NC // ncb)
        assert rec == B * H * ncb * unit + (nblk * B * H * kk if nblk > 1 else 0)
        assert rec <= full
        if nblk > 2:
            assert rec < full / 2
    # the raw entry sizes its core the same way
    ra = _lib.PrefillArgs()
    ra.abi_version = _lib.DN_ABI_VERSION
    ra.B, ra.L, ra.Hk, ra.Hv, ra.K, ra.V = 4, 8192, 16, 32, 128, 128
    for f in ("q", "k", "v", "g", "b", "w"):
        setattr(ra, f, 0x1000)
    ra.g_heads, ra.g_chans, ra.b_heads, ra.b_chans, ra.w_heads, ra.w_chans = 16, 128, 16, 128, 32, 128
    ra.qk_dtype, ra.v_dtype = _lib.DN_BF16, _lib.DN_BF16
    full = lib.dn_prefill_bwd_raw_workspace_size(ctypes.byref(ra))
    ra.recompute_states = 1
    rec = lib.dn_prefill_bwd_raw_workspace_size(ctypes.byref(ra))
    pre = (7 * 32 + 4 * 16) * 4 * 8192 * 128 * 4
    assert full - rec == (4 * 32 * 128 * unit) - (4 * 32 * 8 * unit + 16 * 4 * 32 * kk)
    assert rec > pre


def test_noalloc_entry_refuses_oversized_shape():
    """dn_prefill_fwd_noalloc refuses, before any launch, a shape whose single
    128-token block of every (batch, head) needs more scratch than
    DN_NOALLOC_SCRATCH_BYTES (64 MiB), and accepts the size check of one that
    fits (then it would launch, so only the refusal runs here)."""
    lib = _lib.load_library()
    a = _lib.PrefillArgs()
    a.abi_version = _lib.DN_ABI_VERSION
    a.B, a.L, a.Hk, a.Hv, a.K, a.V = 64, 128, 16, 32, 128, 128
    a.t0, a.nt = 0, 128
    for f in ("q", "k", "v", "g", "b", "w", "out"):
        setattr(a, f, 0x1000)
    a.qk_dtype = a.v_dtype = _lib.DN_BF16
    a.g_heads, a.g_chans, a.b_heads, a.b_chans, a.w_heads, a.w_chans = 16, 128, 16, 128, 32, 128
    a.scale = 128 ** -0.5
    assert lib.dn_prefill_fwd_noalloc(ctypes.byref(a), None) == -2
    assert b"DN_NOALLOC_SCRATCH_BYTES" in lib.dn_last_error()
    a.K = 64
    assert lib.dn_prefill_fwd_noalloc(ctypes.byref(a), None) == -1
