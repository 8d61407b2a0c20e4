"""HIP-graph capture of the hot path (torch.cuda.CUDAGraph over the C ABI).

Every entry point enqueues on the caller's stream, allocates nothing itself
and never synchronises, so prefill, the decode step and the multi-token
decode can be captured and replayed (launch overhead paid once).  Each graph
is replayed several times with new inputs copied into its static tensors and
eager work plus synchronisations in between; every replay must equal an
eager call bit for bit."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _fill(gen, *ts):
    for t in ts:
        t.copy_(torch.randn(t.shape, device=t.device, generator=gen).to(t.dtype))


def _capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()                     # warm-up outside the graph (library load, allocator)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        res = fn()
    return g, res


def test_prefill_graph_replay(dev):
    from deltanet_tpu_amd import chunk_gdn2
    gen = torch.Generator(device=dev).manual_seed(1)
    B, L, Hk, Hv, K = 1, 384, 2, 4, 128
    q = torch.empty(B, L, Hk, K, device=dev, dtype=torch.bfloat16)
    k, v = torch.empty_like(q), torch.empty(B, L, Hv, K, device=dev, dtype=torch.bfloat16)
    g_, b_, w_ = (torch.empty(B, L, H, K, device=dev) for H in (Hk, Hk, Hv))
    seg = (torch.arange(L, device=dev) >= 200).to(torch.int32)[None]

    def fn():
        return chunk_gdn2(q, k, v, -torch.exp(g_ * 0.39 - 1), torch.sigmoid(b_), torch.sigmoid(w_),
                          segment_ids=seg, is_inference=True, output_final_state=True, qk_l2norm=True,
                          precision="bf16")

    _fill(gen, q, k, v, g_, b_, w_)
    graph, (out_g, fin_g) = _capture(fn)
    for rep in range(3):
        _fill(gen, q, k, v, g_, b_, w_)
        graph.replay()
        torch.cuda.synchronize()
        out_e, fin_e = fn()
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e) and torch.equal(fin_g, fin_e), rep


@pytest.mark.parametrize("T", [1, 4])
def test_decode_graph_replay(dev, T):
    from deltanet_tpu_amd import gdn2_decode_step, gdn2_decode_steps
    gen = torch.Generator(device=dev).manual_seed(2)
    B, Hk, Hv, K = 8, 2, 4, 128
    lead = (B, T) if T > 1 else (B,)
    q = torch.empty(*lead, Hk, K, device=dev, dtype=torch.bfloat16)
    k, v = torch.empty_like(q), torch.empty(*lead, Hv, K, device=dev, dtype=torch.bfloat16)
    g_, b_, w_ = (torch.empty(*lead, H, K, device=dev) for H in (Hk, Hk, Hv))
    s_in = torch.empty(B, Hv, K, K, device=dev, dtype=torch.bfloat16)
    s_out = torch.empty_like(s_in)

    def fn():
        gates = (-torch.exp(g_ * 0.39 - 1), torch.sigmoid(b_), torch.sigmoid(w_))
        if T == 1:
            return gdn2_decode_step(q, k, v, *gates, s_in, qk_l2norm=True, state_dtype="bfloat16",
                                    out_state=s_out)
        return gdn2_decode_steps(q, k, v, *gates, s_in, qk_l2norm=True, state_dtype="bfloat16",
                                 out_state=s_out)

    _fill(gen, q, k, v, g_, b_, w_, s_in)
    graph, (o_g, _) = _capture(fn)
    for rep in range(3):
        _fill(gen, q, k, v, g_, b_, w_, s_in)
        graph.replay()
        torch.cuda.synchronize()
        o_rep, s_rep = o_g.clone(), s_out.clone()
        o_e, s_e = fn()
        torch.cuda.synchronize()
        assert torch.equal(o_rep, o_e) and torch.equal(s_rep, s_e), rep
