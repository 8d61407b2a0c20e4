"""API-contract checks that run before any device work (CPU-only), mirroring
the reference's tests/test_validation.py: same ValueError texts (regex-matched
as there), and a loud RuntimeError -- never a CPU fallback -- for CPU tensors."""

import pytest
import torch

from deltanet_tpu_amd import (chunk_delta_rule, chunk_gdn, chunk_gdn2, chunk_kda, delta_rule_decode_step,
                              gdn2_decode_step, gdn_decode_step, kda_decode_step)


def _inputs(B=1, L=128, Hk=2, Hv=4, K=128, V=128):
    q = torch.zeros(B, L, Hk, K)
    k = torch.zeros(B, L, Hk, K)
    v = torch.zeros(B, L, Hv, V)
    g = torch.zeros(B, L, Hk, K)
    b = torch.zeros(B, L, Hk, K)
    w = torch.zeros(B, L, Hv, V)
    return q, k, v, g, b, w


def test_invalid_precision():
    with pytest.raises(ValueError, match="Invalid precision"):
        chunk_gdn2(*_inputs(), precision="invalid_precision")


def test_precision_none_raises():
    with pytest.raises(ValueError, match="precision must be a string"):
        chunk_gdn2(*_inputs(), precision=None)


def test_unsupported_chunk_size():
    with pytest.raises(ValueError, match="Unsupported chunk_size"):
        chunk_gdn2(*_inputs(), chunk_size=64)


def test_unsupported_head_dims():
    with pytest.raises(ValueError, match="Unsupported head dimensions"):
        chunk_gdn2(*_inputs(K=64, V=64))


def test_unsupported_head_ratio():
    with pytest.raises(ValueError, match="Value heads .* must be divisible by key heads"):
        chunk_gdn2(*_inputs(Hk=2, Hv=3))


def test_invalid_cu_seqlens():
    with pytest.raises(ValueError, match="cu_seqlens.* must equal sequence length"):
        chunk_gdn2(*_inputs(), cu_seqlens=[0, 64, 100])
    with pytest.raises(ValueError, match="strictly monotonically increasing"):
        chunk_gdn2(*_inputs(), cu_seqlens=[0, 64, 32, 128])
    with pytest.raises(ValueError, match="Cannot pass both"):
        chunk_gdn2(*_inputs(), cu_seqlens=[0, 128], segment_ids=torch.zeros(128, dtype=torch.int32))


def test_wrong_k_v_shapes():
    q, k, v, g, b, w = _inputs()
    with pytest.raises(ValueError, match="Key tensor k shape"):
        chunk_gdn2(q, torch.zeros(1, 128, 3, 128), v, g, b, w)
    with pytest.raises(ValueError, match="Value tensor v shape"):
        chunk_gdn2(q, k, torch.zeros(1, 64, 4, 128), g, b, w)
    with pytest.raises(ValueError, match="must be 4D"):
        chunk_gdn2(q[0], k, v, g, b, w)


def test_wrong_gate_shapes():
    q, k, v, g, b, w = _inputs()
    with pytest.raises(ValueError, match="g last dimension"):
        chunk_gdn2(q, k, v, torch.zeros(1, 128, 2, 64), b, w)
    with pytest.raises(ValueError, match="b last dimension"):
        chunk_gdn2(q, k, v, g, torch.zeros(1, 128, 2, 64), w)
    with pytest.raises(ValueError, match="w last dimension"):
        chunk_gdn2(q, k, v, g, b, torch.zeros(1, 128, 4, 64))
    with pytest.raises(ValueError, match="head dimension"):
        chunk_gdn2(q, k, v, torch.zeros(1, 128, 3, 128), b, w)
    with pytest.raises(ValueError, match="must have rank 3"):
        chunk_gdn2(q, k, v, torch.zeros(1, 128), b, w)


def test_segment_ids_checks():
    with pytest.raises(ValueError, match="segment_ids length"):
        chunk_gdn2(*_inputs(), segment_ids=torch.zeros(64, dtype=torch.int32))
    with pytest.raises(ValueError, match="segment_ids must have integer dtype"):
        chunk_gdn2(*_inputs(), segment_ids=torch.zeros((1, 128), dtype=torch.float32))


def test_initial_state_shape_mismatch():
    with pytest.raises(ValueError, match="initial_state shape"):
        chunk_gdn2(*_inputs(), initial_state=torch.zeros(1, 2, 128, 128))


def test_fuse_prologue_requires_l2norm():
    with pytest.raises(ValueError, match="requires qk_l2norm=True"):
        chunk_gdn2(*_inputs(), fuse_prologue=True)


def test_nonpositive_stability_tau_and_block_size_raise():
    with pytest.raises(ValueError, match="stability_tau must be positive"):
        chunk_gdn2(*_inputs(), stability_guard=True, stability_tau=0.0)
    with pytest.raises(ValueError, match="prefill_block_size must be positive"):
        chunk_gdn2(*_inputs(), streaming_prefill=True, prefill_block_size=0)


def test_cpu_tensors_fail_loudly():
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        chunk_gdn2(*_inputs(), is_inference=True)
    q = torch.zeros(1, 2, 128)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        gdn2_decode_step(q, q, torch.zeros(1, 4, 128), torch.zeros(1, 2, 128), torch.zeros(1, 2, 128),
                         torch.zeros(1, 4, 128), torch.zeros(1, 4, 128, 128))


def test_decode_step_validation():
    q = torch.zeros(1, 2, 128)
    k = torch.zeros(1, 2, 128)
    v = torch.zeros(1, 4, 128)
    g = torch.zeros(1, 2, 128)
    b = torch.zeros(1, 2, 128)
    w = torch.zeros(1, 4, 128)
    state = torch.zeros(1, 4, 128, 128)
    with pytest.raises(ValueError, match="state shape"):
        gdn2_decode_step(q, k, v, g, b, w, torch.zeros(1, 2, 128, 128))
    with pytest.raises(ValueError, match="Key tensor k shape"):
        gdn2_decode_step(q, torch.zeros(1, 3, 128), v, g, b, w, state)
    with pytest.raises(ValueError, match="Value tensor v batch"):
        gdn2_decode_step(q, k, torch.zeros(2, 4, 128), g, b, w, state)
    with pytest.raises(ValueError, match="reset batch dimension"):
        gdn2_decode_step(torch.zeros(2, 2, 128), torch.zeros(2, 2, 128), torch.zeros(2, 4, 128),
                         torch.zeros(2, 2, 128), torch.zeros(2, 2, 128), torch.zeros(2, 4, 128),
                         torch.zeros(2, 4, 128, 128), reset=torch.tensor([True]))
    with pytest.raises(ValueError, match="Decode step sequence dimension must be 1"):
        gdn2_decode_step(torch.zeros(1, 2, 2, 128), torch.zeros(1, 2, 2, 128), torch.zeros(1, 2, 4, 128),
                         g, b, w, state)
    with pytest.raises(ValueError, match="invalid for batch"):
        gdn2_decode_step(q, k, v, torch.zeros(1, 3, 128), b, w, state)


def test_channel_wise_beta_in_variants_raises():
    q, k, v, g, b, w = _inputs()
    beta = torch.zeros(1, 128, 2, 128)
    with pytest.raises(ValueError, match="channel-wise beta with shape"):
        chunk_gdn(q, k, v, g, beta)
    with pytest.raises(ValueError, match="channel-wise beta with shape"):
        chunk_kda(q, k, v, g, beta)
    with pytest.raises(ValueError, match="channel-wise beta with shape"):
        chunk_delta_rule(q, k, v, beta)
    qd = torch.zeros(1, 2, 128)
    st = torch.zeros(1, 4, 128, 128)
    with pytest.raises(ValueError, match="channel-wise beta with shape"):
        gdn_decode_step(qd, qd, torch.zeros(1, 4, 128), torch.zeros(1, 2), torch.zeros(1, 2, 128), st)
    with pytest.raises(ValueError, match="channel-wise beta with shape"):
        kda_decode_step(qd, qd, torch.zeros(1, 4, 128), torch.zeros(1, 2, 128), torch.zeros(1, 2, 128), st)
    with pytest.raises(ValueError, match="channel-wise beta with shape"):
        delta_rule_decode_step(qd, qd, torch.zeros(1, 4, 128), torch.zeros(1, 2, 128), st)


def test_decode_steps_validation():
    from deltanet_tpu_amd import gdn2_decode_steps
    B, T, Hk, Hv = 2, 3, 2, 4
    q = torch.zeros(B, T, Hk, 128)
    v = torch.zeros(B, T, Hv, 128)
    g = torch.zeros(B, T, Hk, 128)
    st = torch.zeros(B, Hv, 128, 128)
    with pytest.raises(ValueError, match="rank 4"):
        gdn2_decode_steps(q[:, 0], q[:, 0], v[:, 0], g, g, v, st)
    with pytest.raises(ValueError, match="must start with"):
        gdn2_decode_steps(q, q, v[:, :2], g, g, v, st)
    with pytest.raises(ValueError, match="invalid for batch"):
        gdn2_decode_steps(q, q, v, g[:, :2], g, v, st)
    with pytest.raises(ValueError, match="reset must have shape"):
        gdn2_decode_steps(q, q, v, g, g, v, st, reset=torch.zeros(B, T + 1, dtype=torch.bool))
    with pytest.raises(ValueError, match="state shape"):
        gdn2_decode_steps(q, q, v, g, g, v, st[:1])
