"""Specialisations of GDN-2 (maelie-labs/deltanet-tpu v0.3.0,
src/deltanet_tpu/variants.py): Gated DeltaNet (b = w = beta), Kimi Delta
Attention (channel decay, b = w = beta), Gated Linear Attention (b = 0, w = 1)
and DeltaNet (g = 0, b = w = beta), as thin adapters over ``chunk_gdn2`` /
``gdn2_decode_step``.  Constant gates are passed as one-element-per-token
broadcast gates, so no full-size gate tensors are materialised.
"""

from __future__ import annotations

import torch

from .gdn2 import chunk_gdn2, gdn2_decode_step

__all__ = [
    "chunk_gdn", "gdn_decode_step",
    "chunk_kda", "kda_decode_step",
    "chunk_gla", "gla_decode_step",
    "chunk_delta_rule", "delta_rule_decode_step",
]

_PREFILL_BETA_MSG = ("beta must be a per-head scalar gate with shape (B, L, H) or (B, L, H, 1); "
                     "channel-wise beta with shape {} is not supported.")
_DECODE_BETA_MSG = ("beta must be a per-head scalar gate with shape (B, H), (B, H, 1) or (B, 1, H); "
                    "channel-wise beta with shape {} is not supported.")


def _check_prefill_beta(beta):
    # variants.py:69-73
    if beta.ndim == 4 and beta.shape[-1] > 1:
        raise ValueError(_PREFILL_BETA_MSG.format(tuple(beta.shape)))


def _const_gate(ref, value):
    """(B, L, 1) gate of a constant value (broadcast over heads and channels)."""
    return torch.full((ref.shape[0], ref.shape[1], 1), value, dtype=torch.float32, device=ref.device)


def chunk_gdn(q, k, v, g, beta, *, segment_ids=None, cu_seqlens=None, initial_state=None,
              output_final_state=False, chunk_size=128, precision="bf16", scale=None, qk_l2norm=False,
              fallback_scan=False, is_inference=False, fuse_prologue=False, recompute_states=False):
    """Gated DeltaNet (scalar decay per head, shared gate beta); variants.py:17-88."""
    _check_prefill_beta(beta)
    return chunk_gdn2(q, k, v, g, beta, beta, segment_ids=segment_ids, cu_seqlens=cu_seqlens,
                      initial_state=initial_state, output_final_state=output_final_state,
                      chunk_size=chunk_size, precision=precision, scale=scale, qk_l2norm=qk_l2norm,
                      fallback_scan=fallback_scan, is_inference=is_inference,
                      fuse_prologue=fuse_prologue, recompute_states=recompute_states)


def chunk_kda(q, k, v, g, beta, *, segment_ids=None, cu_seqlens=None, initial_state=None,
              output_final_state=False, chunk_size=128, precision="bf16", scale=None, qk_l2norm=False,
              fallback_scan=False, is_inference=False, fuse_prologue=False, recompute_states=False):
    """Kimi Delta Attention (channel-wise decay, shared gate beta); variants.py:91-161."""
    _check_prefill_beta(beta)
    return chunk_gdn2(q, k, v, g, beta, beta, segment_ids=segment_ids, cu_seqlens=cu_seqlens,
                      initial_state=initial_state, output_final_state=output_final_state,
                      chunk_size=chunk_size, precision=precision, scale=scale, qk_l2norm=qk_l2norm,
                      fallback_scan=fallback_scan, is_inference=is_inference,
                      fuse_prologue=fuse_prologue, recompute_states=recompute_states)


def chunk_gla(q, k, v, g, *, segment_ids=None, cu_seqlens=None, initial_state=None,
              output_final_state=False, chunk_size=128, precision="bf16", scale=None, qk_l2norm=False,
              fallback_scan=False, is_inference=False, recompute_states=False):
    """Gated Linear Attention: GDN-2 with b = 0, w = 1; variants.py:164-221."""
    return chunk_gdn2(q, k, v, g, _const_gate(q, 0.0), _const_gate(q, 1.0), segment_ids=segment_ids,
                      cu_seqlens=cu_seqlens, initial_state=initial_state,
                      output_final_state=output_final_state, chunk_size=chunk_size, precision=precision,
                      scale=scale, qk_l2norm=qk_l2norm, fallback_scan=fallback_scan,
                      is_inference=is_inference, recompute_states=recompute_states)


def chunk_delta_rule(q, k, v, beta, *, segment_ids=None, cu_seqlens=None, initial_state=None,
                     output_final_state=False, chunk_size=128, precision="bf16", scale=None,
                     qk_l2norm=False, fallback_scan=False, is_inference=False, recompute_states=False):
    """DeltaNet: GDN-2 with g = 0 and b = w = beta; variants.py:224-285."""
    _check_prefill_beta(beta)
    return chunk_gdn2(q, k, v, _const_gate(q, 0.0), beta, beta, segment_ids=segment_ids,
                      cu_seqlens=cu_seqlens, initial_state=initial_state,
                      output_final_state=output_final_state, chunk_size=chunk_size, precision=precision,
                      scale=scale, qk_l2norm=qk_l2norm, fallback_scan=fallback_scan,
                      is_inference=is_inference, recompute_states=recompute_states)


def _validate_decode_beta(beta):
    # variants.py:288-305
    if beta.ndim == 3:
        if beta.shape[1] == 1:
            beta = beta[:, 0]
        elif beta.shape[-1] > 1:
            raise ValueError(_DECODE_BETA_MSG.format(tuple(beta.shape)))
    elif beta.ndim == 4:
        if beta.shape[-1] > 1:
            raise ValueError(_DECODE_BETA_MSG.format(tuple(beta.shape)))
        if beta.shape[1] == 1:
            beta = beta[:, 0]
    return beta


def gdn_decode_step(q, k, v, g, beta, state, *, reset=None, scale=None, qk_l2norm=False, state_dtype=None):
    """Gated DeltaNet decode step; variants.py:308-333."""
    beta = _validate_decode_beta(beta)
    return gdn2_decode_step(q, k, v, g, beta, beta, state, reset=reset, scale=scale,
                            qk_l2norm=qk_l2norm, state_dtype=state_dtype)


def kda_decode_step(q, k, v, g, beta, state, *, reset=None, scale=None, qk_l2norm=False, state_dtype=None):
    """KDA decode step; variants.py:336-361."""
    beta = _validate_decode_beta(beta)
    return gdn2_decode_step(q, k, v, g, beta, beta, state, reset=reset, scale=scale,
                            qk_l2norm=qk_l2norm, state_dtype=state_dtype)


def _const_decode_gate(ref, value):
    return torch.full((ref.shape[0], 1), value, dtype=torch.float32, device=ref.device)


def gla_decode_step(q, k, v, g, state, *, reset=None, scale=None, qk_l2norm=False, state_dtype=None):
    """GLA decode step (b = 0, w = 1); variants.py:364-389."""
    return gdn2_decode_step(q, k, v, g, _const_decode_gate(q, 0.0), _const_decode_gate(q, 1.0), state,
                            reset=reset, scale=scale, qk_l2norm=qk_l2norm, state_dtype=state_dtype)


def delta_rule_decode_step(q, k, v, beta, state, *, reset=None, scale=None, qk_l2norm=False, state_dtype=None):
    """DeltaNet decode step (g = 0); variants.py:392-417."""
    beta = _validate_decode_beta(beta)
    return gdn2_decode_step(q, k, v, _const_decode_gate(q, 0.0), beta, beta, state, reset=reset,
                            scale=scale, qk_l2norm=qk_l2norm, state_dtype=state_dtype)
