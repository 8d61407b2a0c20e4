#!/usr/bin/env python3
"""Writes the golden fixtures in this directory: small seeded inputs and the
float64 oracle's outputs for them (oracle/gdn_oracle.py, the restatement of
maelie-labs/deltanet-tpu's token-serial GDN-2 recurrence, reference.py:123-161,
and of the wrapper semantics of chunk_gdn2, gdn2.py:1970-2125, and
gdn2_decode_step, gdn2.py:2393-2489).

The reference ships no golden vectors of its own, so these fixtures pin
today's oracle: tests/test_golden.py checks that the oracle still reproduces
them (CPU) and that the HIP path matches them (GPU).  Inputs are stored as
float32; q, k, v hold bf16-representable values so one fixture serves both
input dtypes; gates and initial states are bf16-representable too (so the
fixtures compress).

    python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import gdn_oracle as O  # noqa: E402


def bfr(x):
    return O.bf16_round(x).astype(np.float32)


def sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def prefill_fixture():
    rng = np.random.default_rng(20251201)
    B, L, Hk, Hv, K = 1, 160, 1, 2, 128          # 2 chunks, the second ragged
    q = bfr(rng.standard_normal((B, L, Hk, K)))
    k = bfr(rng.standard_normal((B, L, Hk, K)))
    v = bfr(rng.standard_normal((B, L, Hv, K)))
    g = bfr(-np.exp(0.39 * rng.standard_normal((B, L, Hk, K)) - 1))
    b = bfr(sig(0.39 * rng.standard_normal((B, L, Hk, K))))
    w = bfr(sig(0.39 * rng.standard_normal((B, L, Hv, K))))
    seg = np.where(np.arange(L) < 77, 3, 5).astype(np.int32)[None]       # reset at 77
    init = bfr(0.05 * rng.standard_normal((B, Hv, K, K)))
    init_seg = np.array([3], np.int32)                                    # continues doc 3
    out, fin = O.chunk_gdn2(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), g, b, w,
                            segment_ids=seg, initial_state=init, initial_state_segment_id=init_seg,
                            output_final_state=True, qk_l2norm=True, qk_dtype="fp32")
    np.savez_compressed(os.path.join(HERE, "prefill_gdn2_small.npz"), q=q, k=k, v=v, g=g, b=b, w=w, seg=seg,
                        init=init, init_seg=init_seg, out=out.astype(np.float32), final=fin.astype(np.float32))


def decode_fixture():
    rng = np.random.default_rng(20251202)
    B, Hk, Hv, K = 2, 1, 1, 128
    q = bfr(rng.standard_normal((B, 1, Hk, K)))
    k = bfr(rng.standard_normal((B, 1, Hk, K)))
    v = bfr(rng.standard_normal((B, 1, Hv, K)))
    g = bfr(-np.exp(0.39 * rng.standard_normal((B, 1, Hk, K)) - 1))
    b = bfr(sig(0.39 * rng.standard_normal((B, 1, Hk, K))))
    w = bfr(sig(0.39 * rng.standard_normal((B, 1, Hv, K))))
    state = bfr(0.05 * rng.standard_normal((B, Hv, K, K)))
    reset = np.array([0, 1], np.uint8)
    out, new = O.decode_step(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), g, b, w,
                             state.astype(np.float64), reset=reset.astype(bool), qk_l2norm=True)
    np.savez_compressed(os.path.join(HERE, "decode_gdn2_small.npz"), q=q, k=k, v=v, g=g, b=b, w=w, state=state,
                        reset=reset, out=out.astype(np.float32), new_state=new.astype(np.float32))


if __name__ == "__main__":
    prefill_fixture()
    decode_fixture()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
