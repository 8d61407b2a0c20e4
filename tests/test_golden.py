"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the float64 oracle on seeded inputs).  The CPU test pins the oracle to
the fixtures; the GPU tests check the HIP path against them, independently of
the oracle code."""

import os

import numpy as np
import pytest

from oracle import gdn_oracle as O
from tests._util import maxabs_over_rms, rel_frob

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(HERE, name)) as z:   # allow_pickle defaults to False
        return {k: z[k] for k in z.files}


def test_oracle_reproduces_prefill_fixture():
    z = load("prefill_gdn2_small.npz")
    f64 = lambda a: a.astype(np.float64)
    out, fin = O.chunk_gdn2(f64(z["q"]), f64(z["k"]), f64(z["v"]), z["g"], z["b"], z["w"], segment_ids=z["seg"],
                            initial_state=z["init"], initial_state_segment_id=z["init_seg"],
                            output_final_state=True, qk_l2norm=True, qk_dtype="fp32")
    assert maxabs_over_rms(out, z["out"]) < 1e-6
    assert rel_frob(fin, z["final"]) < 1e-6


def test_oracle_reproduces_decode_fixture():
    z = load("decode_gdn2_small.npz")
    f64 = lambda a: a.astype(np.float64)
    out, new = O.decode_step(f64(z["q"]), f64(z["k"]), f64(z["v"]), z["g"], z["b"], z["w"], f64(z["state"]),
                             reset=z["reset"].astype(bool), qk_l2norm=True)
    assert maxabs_over_rms(out, z["out"]) < 1e-6
    assert rel_frob(new, z["new_state"]) < 1e-6


@pytest.mark.gpu
@pytest.mark.parametrize("precision,in_dtype", [("fp32", "fp32"), ("bf16", "fp32"), ("bf16", "bf16")])
def test_prefill_matches_fixture(precision, in_dtype):
    import torch

    from deltanet_tpu_amd import chunk_gdn2
    from tests.gpu_common import check, to_dev

    z = load("prefill_gdn2_small.npz")
    dt = torch.bfloat16 if in_dtype == "bf16" else torch.float32
    out, fin = chunk_gdn2(to_dev(z["q"], dt), to_dev(z["k"], dt), to_dev(z["v"], dt), to_dev(z["g"]), to_dev(z["b"]),
                          to_dev(z["w"]), segment_ids=to_dev(z["seg"], torch.int32), initial_state=to_dev(z["init"]),
                          initial_state_segment_id=to_dev(z["init_seg"], torch.int32), output_final_state=True,
                          qk_l2norm=True, precision=precision, is_inference=True)
    torch.cuda.synchronize()
    check(out, z["out"].astype(np.float64), fin, z["final"].astype(np.float64), precision, in_dtype,
          f"golden prefill {precision}/{in_dtype}")


@pytest.mark.gpu
@pytest.mark.parametrize("state_dtype", ["float32", "bfloat16"])
def test_decode_matches_fixture(state_dtype):
    import torch

    from deltanet_tpu_amd import gdn2_decode_step
    from tests.gpu_common import check, to_dev

    z = load("decode_gdn2_small.npz")
    st = to_dev(z["state"])
    if state_dtype == "bfloat16":
        st = st.to(torch.bfloat16)   # the fixture's state is bf16-representable: exact
    o, new = gdn2_decode_step(to_dev(z["q"]), to_dev(z["k"]), to_dev(z["v"]), to_dev(z["g"]), to_dev(z["b"]),
                              to_dev(z["w"]), st, reset=to_dev(z["reset"], torch.bool), qk_l2norm=True,
                              state_dtype=state_dtype)
    torch.cuda.synchronize()
    prec = "fp32" if state_dtype == "float32" else "bf16"
    check(o[:, 0] if o.dim() == 4 else o, z["out"].astype(np.float64), new, z["new_state"].astype(np.float64), prec,
          "fp32", f"golden decode {state_dtype}")
