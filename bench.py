#!/usr/bin/env python3
"""Benchmark of the delta-rule recurrence core on one MI355X.

Workload (the configuration the headline metric is
quoted on): chunk_gdn2 prefill, is_inference=True, B=1, L=2048, Hk=12, Hv=24,
K=V=128, bf16 q/k/v, fp32 gates (channel-wise g, b at Hk; w at Hv), segment
ids 0 for t<1024 and 1 after, chunk 128, precision="bf16", qk_l2norm=True,
fp32 final state.  A "step" is one such call on inputs already resident in
HBM.  The same run also times the GDN-2 decode step of BASELINE.json
configs[3] (B=256, Hk=16, Hv=32, fp32 and bf16 state), which the metric's
second half ("decode step us + state HBM GB/s") refers to.

Prints ONE JSON line (see the "roofline" and "cpu_baseline" objects).
Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "deltanet-tpu_amd"))

# MI355X published peaks
PEAK_HBM_GBPS = 8000.0
PEAK_BF16_TFLOPS = 2516.6
PEAK_FP32_TFLOPS = 157.3      # dense fp32 MFMA (v_mfma_f32_*_f32)

METRIC = "prefill tokens/s + %bf16 MFMA peak; decode step µs + state HBM GB/s"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def prefill_inputs(torch, dev, B=1, L=2048, Hk=12, Hv=24, K=128, seed=2, packed=True):
    """BASELINE config 2 inputs.  packed=False leaves each input in its own
    allocation (wherever the caching allocator puts it)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    rn = lambda *s: torch.randn(*s, device=dev, generator=g)
    q = rn(B, L, Hk, K).to(torch.bfloat16)
    k = rn(B, L, Hk, K).to(torch.bfloat16)
    v = rn(B, L, Hv, K).to(torch.bfloat16)
    b = torch.sigmoid(0.39 * rn(B, L, Hk, K))
    w = torch.sigmoid(0.39 * rn(B, L, Hv, K))
    gg = -torch.exp(0.39 * rn(B, L, Hk, K) - 1.0)
    seg = (torch.arange(L, device=dev) >= 1024).to(torch.int32)[None].repeat(B, 1)
    t = (q, k, v, gg, b, w, seg)
    return _pack(torch, dev, t) if packed else t


def geometric_segments(torch, dev, gen, B, L, mean, lo=16):
    """segment_ids of documents with geometric(1/mean) lengths clipped to [lo, L]."""
    import numpy as np

    rng = np.random.default_rng(gen)
    seg = np.zeros((B, L), np.int32)
    for b in range(B):
        t, d = 0, 0
        while t < L:
            n = int(np.clip(rng.geometric(1.0 / mean), lo, L))
            seg[b, t:t + n] = d
            t += n
            d += 1
    return torch.from_numpy(seg).to(dev)


def config3_inputs(torch, dev, B=4, L=8192, Hk=16, Hv=32, K=128, seed=3):
    """BASELINE config 3 (chunk_gdn, Qwen3-Next scalar decay, packed documents)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    rn = lambda *s: torch.randn(*s, device=dev, generator=g)
    q = rn(B, L, Hk, K).to(torch.bfloat16)
    k = rn(B, L, Hk, K).to(torch.bfloat16)
    v = rn(B, L, Hv, K).to(torch.bfloat16)
    a_log = math.log(1.0) + (math.log(16.0) - math.log(1.0)) * torch.rand(Hv, device=dev, generator=g)
    gg = -torch.exp(a_log) * torch.nn.functional.softplus(rn(B, L, Hv))
    beta = torch.sigmoid(rn(B, L, Hv))
    seg = geometric_segments(torch, dev, seed, B, L, 1024)
    return _pack(torch, dev, (q, k, v, gg, beta, seg))


def config5_inputs(torch, dev, B=1, L=65536, Hk=16, Hv=32, K=128, seed=5):
    """BASELINE config 5 (streaming prefill, fused prologue: raw gates)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    rn = lambda *s: torch.randn(*s, device=dev, generator=g)
    q = rn(B, L, Hk, K).to(torch.bfloat16)
    k = rn(B, L, Hk, K).to(torch.bfloat16)
    v = rn(B, L, Hv, K).to(torch.bfloat16)
    gr, br, wr = rn(B, L, Hk, K), rn(B, L, Hk, K), rn(B, L, Hv, K)
    seg = geometric_segments(torch, dev, seed, B, L, 8192)
    return _pack(torch, dev, (q, k, v, gr, br, wr, seg))


def _pack(torch, dev, tensors):
    """Copy the inputs into contiguous views of ONE device allocation, laid out
    back to back (256-byte aligned) as a fused input projection writes them.
    Separately allocated inputs land wherever the caching allocator puts them;
    an input alone in a freshly mapped segment far from the rest measured about
    6 us slower per config-2 prefill, so the bench fixes the placement."""
    sizes = [(t.numel() * t.element_size() + 255) // 256 * 256 for t in tensors]
    arena = torch.empty(sum(sizes), dtype=torch.uint8, device=dev)
    out, off = [], 0
    for t, n in zip(tensors, sizes):
        view = arena[off:off + t.numel() * t.element_size()].view(t.dtype).view(t.shape)
        view.copy_(t)
        out.append(view)
        off += n
    return tuple(out)


def decode_inputs(torch, dev, B=256, Hk=16, Hv=32, K=128, seed=4):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    rn = lambda *s: torch.randn(*s, device=dev, generator=g)
    q = rn(B, 1, Hk, K).to(torch.bfloat16)
    k = rn(B, 1, Hk, K).to(torch.bfloat16)
    v = rn(B, 1, Hv, K).to(torch.bfloat16)
    b = torch.sigmoid(0.39 * rn(B, 1, Hk, K))
    w = torch.sigmoid(0.39 * rn(B, 1, Hv, K))
    gg = -torch.exp(0.39 * rn(B, 1, Hk, K) - 1.0)
    state = 0.02 * rn(B, Hv, K, K)
    return _pack(torch, dev, (q, k, v, gg, b, w, state))


def prefill_work(B=1, L=2048, Hk=12, Hv=24, K=128, C=128, gates="channel"):
    """Algorithmic flops / bytes of one prefill call, split by kernel
    (per-(exec head, chunk) figures of the chunked WY algorithm x the units one
    launch processes).  gates="channel": g, b of shape (B, L, Hk, K) and w of
    shape (B, L, Hv, K), fp32 (chunk_gdn2); gates="scalar": g and beta of shape
    (B, L, Hv), fp32 (chunk_gdn), so every value head is its own exec head."""
    Hx = Hv if gates == "scalar" else Hk
    Vp = (Hv // Hx) * K
    units = B * Hx * math.ceil(L / C)
    f_pre = 6 * C * C * K + C ** 3 / 3                        # A, M, W = T be ; T
    f_val = 2 * C * C * Vp                                    # U = T (w*v)
    f_chain = 4 * C * K * Vp + 2 * C * K * Vp + 2 * C * C * Vp   # W S ; ke^T Vnew ; qe S ; M Vnew
    if gates == "scalar":
        gate_k, gate_v = B * L * Hv * 4 * 2, 0                # g, beta (beta is also the write gate)
    else:
        gate_k, gate_v = 2 * B * L * Hk * K * 4, B * L * Hv * K * 4
    qkgb_bytes = B * L * 2 * Hk * K * 2 + gate_k + 4 * B * L
    vw_bytes = B * L * Hv * K * 2 + gate_v
    out_bytes = B * L * Hv * K * 2
    state_bytes = B * Hv * K * K * 4
    # k_prepass computes the value products too (U, Q, M U) and reads v and w
    return dict(units=units, flops_total=units * (f_pre + f_val + f_chain),
                prepass=dict(flops=units * (f_pre + f_val), bytes=qkgb_bytes + vw_bytes),
                chain=dict(flops=units * f_chain, bytes=state_bytes + out_bytes),
                bytes_total=qkgb_bytes + vw_bytes + out_bytes + state_bytes)


_TRACE = {"on": True}


def kernel_times(torch, fn, n, per_call=False):
    """Average device duration (us) per launch of each library kernel over n
    calls of fn (per_call: the summed duration per call of fn), from the
    profiler's activity trace (the same per-dispatch timestamps rocprofv3
    --kernel-trace reports; nothing is inserted into the stream).  None if the
    profiler is unavailable (e.g. under rocprofv3)."""
    if not _TRACE["on"]:
        return None
    try:
        from torch.profiler import ProfilerActivity, profile

        torch.cuda.synchronize()
        with profile(activities=[ProfilerActivity.CUDA]) as prof:
            for _ in range(n):
                fn()
            torch.cuda.synchronize()
        out = {}
        for e in prof.key_averages():
            k = _kname(e.key)
            if k and e.device_time_total > 0:
                tot, cnt = out.get(k, (0.0, 0))
                out[k] = (tot + e.device_time_total, cnt + e.count)
        return {k: t / (n if per_call else c) for k, (t, c) in out.items()} or None
    except Exception as ex:  # noqa: BLE001 - the bench line stands without it
        log(f"kernel trace unavailable: {ex}")
        return None


def time_calls(torch, fn, steps, warmup):
    """Wall time per call (ms), with a device synchronisation on both sides."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def roofline_of(work, t_us, name):
    """Roofline entry of kernel `name` ("prepass" | "chain") at t_us per launch."""
    wk = work[name]
    t = t_us * 1e-6
    if wk["bytes"] / (PEAK_HBM_GBPS * 1e9) >= wk["flops"] / (PEAK_BF16_TFLOPS * 1e12):
        r = {"bound": "hbm", "achieved": wk["bytes"] / t / 1e9, "peak": PEAK_HBM_GBPS, "unit": "GB/s"}
    else:
        r = {"bound": "mfma", "achieved": wk["flops"] / t / 1e12, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s"}
    r["frac"] = r["achieved"] / r["peak"]
    return r


def step_roofline(work, ms):
    t_roof = max(work["bytes_total"] / (PEAK_HBM_GBPS * 1e9), work["flops_total"] / (PEAK_BF16_TFLOPS * 1e12))
    return {"t_roof_us": round(t_roof * 1e6, 2), "frac": round(t_roof / (ms * 1e-3), 4),
            "bytes": work["bytes_total"], "flops": work["flops_total"],
            "mfma_pct_peak": round(work["flops_total"] / (ms * 1e-3) / (PEAK_BF16_TFLOPS * 1e12) * 100, 3)}


def backward_work(B=1, L=2048, H=24, K=128, V=128, C=64):
    """Algorithmic flops of dn_prefill_bwd (multiply-adds x 2), per the chunk
    form in dn_backward.hip (triangular products at half size):
    intra A, M, W, U0, Xf ~ 5 C^2 K / 2 + C^3 / 6; forward and reverse scans
    5 C K V; chunk products 5 C K V + 2 C^2 V; decay-weighted dq / dbeta / dk
    2 C^2 K."""
    units = B * H * ((L + C - 1) // C)
    mac = C * C * K * 5 + C ** 3 / 6 + 10 * C * K * V + 2 * C * C * V
    return {"flops": 2 * mac * units, "units": units}


def cpu_baseline(inputs, gpu_out, gpu_state, max_seconds=20.0):
    """The C token-serial restatement (oracle/gdn_serial.c, fp32, OpenMP over
    (batch, value head)) on this host's cores, on the bench's own config-2
    inputs, repeated for about max_seconds.  The same leg checks the bench's
    GPU output against one float64 run of the restatement on those inputs
    (max |out - ref| / rms(ref), raw and net of the half-ulp rounding a bf16
    output cannot avoid; relative Frobenius error of the final state)."""
    import numpy as np

    from oracle import c_oracle as C
    from oracle import gdn_oracle as O

    q, k, v, g, b, w, seg = (x.detach().float().cpu().numpy().astype(np.float64) for x in inputs)
    B, L = q.shape[:2]
    threads = min(os.cpu_count() or 1, 16)
    sg = O.canonical_segments(seg.astype(np.int64), B, L)
    prep = O.prepare_prefill(q, k, v, g, b, w, qk_l2norm=True, qk_dtype="bf16", broadcast=False)
    ref_o, ref_s = C.serial(*prep, sg, nthreads=threads, dtype=np.float64)
    o = gpu_out.float().cpu().numpy().astype(np.float64)
    s = gpu_state.float().cpu().numpy().astype(np.float64)
    rms = float(np.sqrt(np.mean(ref_o ** 2)))
    a = np.abs(ref_o).astype(np.float32).view(np.uint32)
    half_ulp = 0.5 * (a & 0x7F800000).view(np.float32).astype(np.float64) * 2.0 ** -7
    parity = {"out_maxabs_over_rms_raw": float(np.abs(o - ref_o).max() / rms),
              "out_maxabs_over_rms_net_of_bf16_rounding": float(np.maximum(np.abs(o - ref_o) - half_ulp, 0).max() / rms),
              "out_maxabs_over_rms_of_bf16_rounded_reference": float(np.abs(O.bf16_round(ref_o) - ref_o).max() / rms),
              "state_rel_frob": float(np.linalg.norm(s - ref_s) / np.linalg.norm(ref_s)),
              "bar": "north_star bf16: out max-abs <= 2e-2 of rms, final state rel Frobenius <= 1e-2",
              "reference": "float64 token-serial restatement (oracle/gdn_serial.c) on the same inputs"}
    t0 = time.perf_counter()
    # the wrapper work (L2-norm, gate activation) is part of the measured CPU path
    reps, tok = 0, 0
    while True:
        prep = O.prepare_prefill(q, k, v, g, b, w, qk_l2norm=True, qk_dtype="bf16", broadcast=False)
        C.serial(*prep, sg, nthreads=threads, dtype=np.float32)
        reps += 1
        tok += B * L
        if time.perf_counter() - t0 >= max_seconds or reps >= 200:
            break
    dt = time.perf_counter() - t0
    return ({"value": tok / dt, "unit": "tokens/s", "cores": threads, "kind": "port",
             "sample": f"config 2 (B=1, L=2048, Hk=12, Hv=24, the bench's own inputs) x {reps} full prefills, "
                       f"fp32 token-serial C (oracle/gdn_serial.c, OpenMP over 24 (batch, value-head) chains), "
                       f"{dt:.1f} s"}, parity)


def cpu_baselines_more(max_seconds=8.0):
    """Further CPU legs on this host, each a bounded sample (about max_seconds):
    config 1 (the reference's CPU-plumbing shape) with the C token-serial
    restatement; config 2 with the float64 NumPy chunked-WY restatement
    (oracle/gdn_oracle.py chunked_wy, one head at a time); the config-4 decode
    step with the float64 NumPy restatement on a slice of the batch."""
    import numpy as np

    from oracle import c_oracle as C
    from oracle import gdn_oracle as O

    out = []
    rng = np.random.default_rng(1)
    threads = min(os.cpu_count() or 1, 16)

    def timed(fn, unit_count):
        t0 = time.perf_counter()
        reps = 0
        while True:
            fn()
            reps += 1
            if time.perf_counter() - t0 >= max_seconds or reps >= 1000:
                break
        dt = time.perf_counter() - t0
        return reps, dt, reps * unit_count / dt

    # config 1: B=1, L=256, Hk=2, Hv=4, K=V=64, fp32
    B, L, Hk, Hv, K = 1, 256, 2, 4, 64
    f = lambda *s: rng.standard_normal(s)
    q, k, v = f(B, L, Hk, K), f(B, L, Hk, K), f(B, L, Hv, K)
    b, w = 1 / (1 + np.exp(-0.39 * f(B, L, Hk, K))), 1 / (1 + np.exp(-0.39 * f(B, L, Hv, K)))
    g = -np.exp(0.39 * f(B, L, Hk, K) - 1)
    seg = O.canonical_segments((np.arange(L) >= L // 2).astype(np.int64)[None], B, L)

    def c1():
        prep = O.prepare_prefill(q, k, v, g, b, w, qk_l2norm=True, broadcast=False)
        C.serial(*prep, seg, nthreads=1, dtype=np.float32)

    reps, dt, rate = timed(c1, B * L)
    out.append({"config": 1, "value": rate, "unit": "tokens/s", "cores": 1, "kind": "port",
                "sample": f"config 1 (B=1 L=256 Hk=2 Hv=4 K=V=64, fp32) x {reps}, C token-serial, {dt:.1f} s"})

    # config 2, NumPy chunked WY (float64), heads in turn
    B, L, Hk, Hv, K = 1, 2048, 12, 24, 128
    q, k, v = (O.bf16_round(f(*s)) for s in ((B, L, Hk, K), (B, L, Hk, K), (B, L, Hv, K)))
    b, w = 1 / (1 + np.exp(-0.39 * f(B, L, Hk, K))), 1 / (1 + np.exp(-0.39 * f(B, L, Hv, K)))
    g = -np.exp(0.39 * f(B, L, Hk, K) - 1)
    seg = O.canonical_segments((np.arange(L) >= 1024).astype(np.int64)[None], B, L)
    qh, kh, vv, ga, ba, wa = O.prepare_prefill(q, k, v, g, b, w, qk_l2norm=True, qk_dtype="bf16", broadcast=False)
    heads = {"n": 0}

    def c2():
        h = heads["n"] % Hv         # value head; its key head (q, k, g, b) is h // G
        hk = h // (Hv // Hk)
        heads["n"] += 1
        O.chunked_wy(qh[0, :, hk], kh[0, :, hk], vv[0, :, h], ga[0, :, hk], ba[0, :, hk], wa[0, :, h], seg[0])

    reps, dt, rate = timed(c2, B * L / Hv)
    out.append({"config": 2, "value": rate, "unit": "tokens/s", "cores": 1, "kind": "port",
                "sample": f"config 2 (B=1 L=2048 Hk=12 Hv=24) NumPy float64 chunked WY, {reps} (head) "
                          f"calls of the 24 a full prefill needs, {dt:.1f} s; tokens/s = reps / 24 x 2048 / s"})

    # config 4 decode, NumPy float64, 16 of the 256 batch rows per call
    Bs, Hk, Hv, K = 16, 16, 32, 128
    st = 0.02 * f(Bs, Hv, K, K)
    q, k, v = f(Bs, 1, Hk, K), f(Bs, 1, Hk, K), f(Bs, 1, Hv, K)
    b, w = 1 / (1 + np.exp(-0.39 * f(Bs, 1, Hk, K))), 1 / (1 + np.exp(-0.39 * f(Bs, 1, Hv, K)))
    g = -np.exp(0.39 * f(Bs, 1, Hk, K) - 1)

    def c4():
        O.decode_step(q, k, v, g, b, w, st, qk_l2norm=True)

    reps, dt, rate = timed(c4, Bs / 256)
    out.append({"config": 4, "value": 1e6 / rate, "unit": "us per full (B=256) decode step", "cores": 1,
                "kind": "port", "higher_is_better": False,
                "sample": f"config 4 decode step (Hk=16 Hv=32 K=V=128, fp32 state) NumPy float64 on 16 of the 256 "
                          f"batch rows x {reps}, {dt:.1f} s; scaled to the full batch"})
    return out


PROFILE_DIR = os.path.join(ROOT, "profiles")
TRAFFIC_JSON = os.path.join(PROFILE_DIR, "pmc_traffic_cfg2_cfg4.json")
KT_CMD = ("cd /tmp && export TMPDIR=/tmp && cd $GRAFT_REPO_ROOT && rocprofv3 --kernel-trace --stats "
          "--output-format csv -d gpurun_out/kt -o run -- python3 bench.py --no-cpu-baseline --steps 50 "
          "--warmup 5 --decode-steps 16 --train-steps 0 --config-steps 0 --no-kernel-trace --copy-calibration")
PMC_CMD = ("cd /tmp && export TMPDIR=/tmp && cd $GRAFT_REPO_ROOT && rocprofv3 --pmc {ctr} --output-format csv "
           "-d gpurun_out/{d} -o run -- python3 bench.py --no-cpu-baseline --steps 5 --warmup 1 "
           "--decode-steps 2 --train-steps 0 --config-steps 0 --no-kernel-trace --copy-calibration")
COPY_BYTES = 256 * 32 * 128 * 128 * 4   # the --copy-calibration copy (read and write this many bytes)


def _kname(n):
    """Short name of a library kernel from its (mangled) symbol, None for others."""
    if "copyBuffer" in n:
        return "copy (calibration)"
    import re

    m = re.search(r"(k_[a-z0-9_]+)", n)
    if not m or "dn" not in n:
        return None
    k = m.group(1)
    if k in ("k_decode", "k_decode_chunk"):
        return k + ("<bf16>" if ("DF16b" in n or "bf16" in n) else "<f32>")
    if k == "k_chain":
        t = re.search(r"k_chainILb\dE\w+?Li(\d)E", n)   # column tiles per workgroup
        if t and t.group(1) != "1":
            return f"k_chain<{t.group(1)} tiles>"
    return k


def rocprof_summary(kt_dir, f_dir, w_dir):
    """Summarise rocprofv3 CSV output of the KT_CMD / PMC_CMD runs into
    profiles/ (text for readers, JSON for bench.py's roofline.traffic)."""
    import csv
    import collections

    os.makedirs(PROFILE_DIR, exist_ok=True)
    dur = collections.defaultdict(list)
    for r in csv.DictReader(open(os.path.join(kt_dir, "run_kernel_trace.csv"))):
        k = _kname(r["Kernel_Name"])
        if k:
            dur[k].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    dur["copy (calibration)"] = [x for x in dur["copy (calibration)"] if x > 0.5 * max(dur["copy (calibration)"])]
    ctr = {}
    for d, name in ((f_dir, "FETCH_SIZE"), (w_dir, "WRITE_SIZE")):
        acc = collections.defaultdict(list)
        for r in csv.DictReader(open(os.path.join(d, "run_counter_collection.csv"))):
            k = _kname(r["Kernel_Name"])
            if k and r["Counter_Name"] == name:
                acc[k].append(float(r["Counter_Value"]) * 1024.0)   # KiB -> bytes
        # the calibration copy is the large one (torch issues small copies too)
        acc["copy (calibration)"] = [x for x in acc["copy (calibration)"] if x > 0.5 * max(acc["copy (calibration)"])]
        ctr[name] = {k: sum(v) / len(v) for k, v in acc.items()}
    f_scale = COPY_BYTES / ctr["FETCH_SIZE"]["copy (calibration)"]
    w_scale = COPY_BYTES / ctr["WRITE_SIZE"]["copy (calibration)"]
    work = prefill_work()
    out = {"fetch_scale": f_scale, "write_scale": w_scale, "kernels": {}}
    lines = ["# rocprofv3 kernel trace + PMC traffic, bench.py workload (prefill BASELINE config 2, "
             "decode config 4, 16-token decode launches at the config-4 shape)", "",
             "Kernel durations from:", "    " + KT_CMD, "",
             "HBM traffic per dispatch from two counter runs:",
             "    " + PMC_CMD.format(ctr="FETCH_SIZE", d="pmc_f"),
             "    " + PMC_CMD.format(ctr="WRITE_SIZE", d="pmc_w"),
             "summarised by:", "    python bench.py --rocprof-summary gpurun_out/kt gpurun_out/pmc_f gpurun_out/pmc_w", "",
             f"Calibration: a plain {COPY_BYTES >> 20} MiB device copy reads FETCH_SIZE x {f_scale:.3f} and "
             f"writes WRITE_SIZE x {w_scale:.3f} bytes; both factors are applied below.", "",
             "| kernel | dispatches | avg us | min us | max us | fetch MB | write MB | algorithmic MB | "
             "traffic / algorithmic |",
             "|---|---|---|---|---|---|---|---|---|"]
    # the 16-token decode launch: state in and out, plus q, k, v (bf16), g, b (fp32, Hk heads), w (fp32, Hv
    # heads) and the bf16 output of its 16 tokens
    tok16 = 256 * 16 * 128 * (2 * 16 * 2 + 32 * 2 + 2 * 16 * 4 + 32 * 4 + 32 * 2)
    alg = {"k_prepass": work["prepass"]["bytes"], "k_chain": work["chain"]["bytes"],
           "k_decode<f32>": 2 * 256 * 32 * 128 * 128 * 4, "k_decode<bf16>": 2 * 256 * 32 * 128 * 128 * 2,
           "k_decode_chunk<f32>": 2 * 256 * 32 * 128 * 128 * 4 + tok16,
           "k_decode_chunk<bf16>": 2 * 256 * 32 * 128 * 128 * 2 + tok16,
           "copy (calibration)": 2 * COPY_BYTES}
    for k in ("k_prepass", "k_chain", "k_decode<f32>", "k_decode<bf16>", "k_decode_chunk<f32>",
              "k_decode_chunk<bf16>", "copy (calibration)"):
        if k not in dur:
            continue
        v = dur[k]
        fb = ctr["FETCH_SIZE"].get(k, float("nan")) * f_scale
        wb = ctr["WRITE_SIZE"].get(k, float("nan")) * w_scale
        out["kernels"][k] = {"avg_us": sum(v) / len(v), "fetch_bytes": fb, "write_bytes": wb,
                             "traffic_bytes": fb + wb, "algorithmic_bytes": alg.get(k)}
        lines.append(f"| {k} | {len(v)} | {sum(v) / len(v):.2f} | {min(v):.2f} | {max(v):.2f} | "
                     f"{fb / 1e6:.1f} | {wb / 1e6:.1f} | {alg.get(k, 0) / 1e6:.1f} | "
                     f"{(fb + wb) / alg[k]:.2f} |")
    lines += ["", "Prefill intermediates (workspace) travel between the two launches; their round trips "
              "are the traffic above the algorithmic bytes."]
    with open(os.path.join(PROFILE_DIR, "prefill_cfg2_decode_cfg4_rocprof.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    with open(TRAFFIC_JSON, "w") as f:
        json.dump(out, f, indent=1)
    print("\n".join(lines))


CFG_CMD = ("cd /tmp && export TMPDIR=/tmp && cd $GRAFT_REPO_ROOT && rocprofv3 --kernel-trace --output-format csv "
           "-d gpurun_out/ktc -o run -- python3 bench.py --no-cpu-baseline --steps 2 --warmup 1 --decode-steps 0 "
           "--train-steps 0 --config-steps 4 --no-kernel-trace")
CFG_PMC_CMD = ("cd /tmp && export TMPDIR=/tmp && cd $GRAFT_REPO_ROOT && rocprofv3 --pmc {ctr} --output-format csv "
               "-d gpurun_out/{d} -o run -- python3 bench.py --no-cpu-baseline --steps 1 --warmup 1 --decode-steps 0 "
               "--train-steps 0 --config-steps 2 --no-kernel-trace --copy-calibration")


def _grid(r):
    return tuple(int(r[f"Grid_Size_{a}"]) // max(1, int(r[f"Workgroup_Size_{a}"])) for a in "XYZ")


def _nwg(r):
    """Workgroups of a dispatch in the counter CSV (one flattened grid size)."""
    return int(r["Grid_Size"]) // max(1, int(r["Workgroup_Size"]))


def rocprof_configs_summary(kt_dir, f_dir=None, w_dir=None):
    """profiles/prefill_cfg3_cfg5_rocprof.md from the CFG_CMD kernel trace: the
    library kernels of configs 3 and 5, told apart by their launch grids; with
    the two CFG_PMC_CMD counter runs, the HBM traffic of each grid too."""
    import csv
    import collections

    rows = collections.defaultdict(list)
    for r in csv.DictReader(open(os.path.join(kt_dir, "run_kernel_trace.csv"))):
        k = _kname(r["Kernel_Name"])
        if not k or k.startswith("copy"):
            continue
        rows[(k, _grid(r))].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    ctr = {}
    if f_dir and w_dir:
        for d, name in ((f_dir, "FETCH_SIZE"), (w_dir, "WRITE_SIZE")):
            acc = collections.defaultdict(list)
            for r in csv.DictReader(open(os.path.join(d, "run_counter_collection.csv"))):
                k = _kname(r["Kernel_Name"])
                if k and r["Counter_Name"] == name:
                    acc[k if k.startswith("copy") else (k, _nwg(r))].append(float(r["Counter_Value"]) * 1024.0)
            cp = acc.pop("copy (calibration)")
            cp = [x for x in cp if x > 0.5 * max(cp)]
            scale = COPY_BYTES / (sum(cp) / len(cp))
            ctr[name] = ({key: sum(v) / len(v) * scale for key, v in acc.items()}, scale)
    # algorithmic bytes per dispatch: config 3 in one launch, config 5 per 8192-token block
    w3 = prefill_work(B=4, L=8192, Hk=16, Hv=32, gates="scalar")
    w5 = prefill_work(B=1, L=8192, Hk=16, Hv=32)
    alg = {("k_prepass", (8192, 1, 1)): w3["prepass"]["bytes"], ("k_chain", (8, 32, 4)): w3["chain"]["bytes"],
           ("k_chain<4 tiles>", (2, 32, 4)): w3["chain"]["bytes"],
           ("k_prepass", (1024, 1, 1)): w5["prepass"]["bytes"], ("k_chain", (16, 16, 1)): w5["chain"]["bytes"]}
    # config 2's grids (B=1, Hk=12, 16 chunks) are the few dispatches of the warm-up and timed cfg-2 calls
    lines = ["# rocprofv3 kernel trace, configs 3 and 5 (bench.py other_configs)", "",
             "Command:", "    " + CFG_CMD]
    if ctr:
        lines += ["HBM traffic per dispatch from two counter runs:",
                  "    " + CFG_PMC_CMD.format(ctr="FETCH_SIZE", d="pmc_cf"),
                  "    " + CFG_PMC_CMD.format(ctr="WRITE_SIZE", d="pmc_cw"),
                  "summarised by:", "    python bench.py --rocprof-configs-summary gpurun_out/ktc gpurun_out/pmc_cf "
                  "gpurun_out/pmc_cw", "",
                  f"Calibration: a plain {COPY_BYTES >> 20} MiB device copy reads FETCH_SIZE x "
                  f"{ctr['FETCH_SIZE'][1]:.3f} and writes WRITE_SIZE x {ctr['WRITE_SIZE'][1]:.3f} bytes; both "
                  "factors are applied below."]
    else:
        lines += ["summarised by:", "    python bench.py --rocprof-configs-summary gpurun_out/ktc"]
    lines += ["", "Dispatches are grouped by kernel and launch grid (workgroups).  Config 3 (chunk_gdn, B=4, L=8192, "
              "Hv=32 exec heads) and config 5 (L=65536 streamed in 8192-token blocks, Hk=16) launch distinct grids; "
              "the config-2 calls of the same run are the 12-head grids.  Algorithmic bytes: inputs read once and "
              "outputs written once (config 5: per 8192-token block).", ""]
    if ctr:
        lines += ["| kernel | grid (workgroups) | dispatches | avg us | total us | fetch MB | write MB | "
                  "algorithmic MB | traffic / algorithmic |", "|---|---|---|---|---|---|---|---|---|"]
    else:
        lines += ["| kernel | grid (workgroups) | dispatches | avg us | total us |", "|---|---|---|---|---|"]
    for (k, grid), v in sorted(rows.items(), key=lambda kv: -sum(kv[1])):
        line = f"| {k} | {grid[0]} x {grid[1]} x {grid[2]} | {len(v)} | {sum(v) / len(v):.1f} | {sum(v):.0f} |"
        if ctr:
            nwg = grid[0] * grid[1] * grid[2]
            fb = ctr["FETCH_SIZE"][0].get((k, nwg), float("nan"))
            wb = ctr["WRITE_SIZE"][0].get((k, nwg), float("nan"))
            a = alg.get((k, grid))
            line += (f" {fb / 1e6:.1f} | {wb / 1e6:.1f} | " + (f"{a / 1e6:.1f} | {(fb + wb) / a:.2f} |" if a else
                                                               "- | - |"))
        lines.append(line)
    with open(os.path.join(PROFILE_DIR, "prefill_cfg3_cfg5_rocprof.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


BW_CMD = ("cd /tmp && export TMPDIR=/tmp && cd $GRAFT_REPO_ROOT && rocprofv3 --kernel-trace --output-format csv "
          "-d gpurun_out/bwkt -o run -- python3 bench.py --no-cpu-baseline --steps 2 --warmup 1 --decode-steps 0 "
          "--train-steps 10 --config-steps 0 --no-kernel-trace")


def rocprof_backward_summary(kt_dir):
    """profiles/backward_cfg2_rocprof.md from the BW_CMD kernel trace."""
    import csv
    import collections
    import re

    dur = collections.defaultdict(list)
    for r in csv.DictReader(open(os.path.join(kt_dir, "run_kernel_trace.csv"))):
        m = re.search(r"(k_bw_[a-z0-9_]+(?:<\d>)?)", r["Kernel_Name"])
        if m:
            dur[m.group(1)].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    core = ("k_bw_intra", "k_bw_chains", "k_bw_grads", "k_bw_dqk")
    bw = backward_work()
    t_core = sum(sum(dur[k]) / len(dur[k]) for k in core if dur.get(k))
    t_rest = sum(sum(v) / len(v) for k, v in dur.items() if k not in core)
    lines = ["# rocprofv3 kernel trace: training backward (dn_prefill_bwd_raw), config-2 shape", "",
             "Command (from the repository root on the GPU box):", "", "    " + BW_CMD, "",
             "summarised by:", "", "    python bench.py --rocprof-backward-summary gpurun_out/bwkt", "",
             "Workload: chunk_gdn2(is_inference=False) forward + backward under torch.autograd, B=1 L=2048 Hk=12 "
             "Hv=24 K=V=128 (bf16 q/k/v, fp32 gates, 2 segments, qk_l2norm); the backward runs at H=24 value heads, "
             "32 chunks of 64 tokens (768 (head, chunk) units), precision bf16: k_bw_chains (state scans, 32-column blocks), k_bw_grads and k_bw_intra's W / U0 / Xf / P run "
             "their products as split bf16 (hi/lo words, 3 v_mfma_f32_16x16x32_bf16 per product), k_bw_intra's A / M and "
             "k_bw_dqk on v_mfma_f32_16x16x4_f32.  The "
             "first four kernels are the recurrence backward (dn_prefill_bwd's kernels); the rest are the raw-input "
             "prologue recompute and the gradient sums back to the raw layouts.", "",
             "| kernel | dispatches | avg us | min us | max us |", "|---|---|---|---|---|"]
    for k in sorted(dur, key=lambda k_: (k_ not in core, core.index(k_) if k_ in core else 0, k_)):
        v = dur[k]
        lines.append(f"| {k} | {len(v)} | {sum(v) / len(v):.1f} | {min(v):.1f} | {max(v):.1f} |")
    lines += ["", f"Sum of the averages: {t_core:.0f} us for the recurrence backward (k_bw_chains runs the forward "
              f"and the reverse state scans in one launch), {t_rest:.0f} us for the prologue and layout kernels.",
              f"Algorithmic work of the recurrence backward (bench.py backward_work): {bw['flops'] / 1e9:.1f} GFLOP, "
              f"i.e. {bw['flops'] / (t_core * 1e-6) / 1e12:.1f} TFLOP/s = "
              f"{bw['flops'] / (t_core * 1e-6) / 1e12 / PEAK_FP32_TFLOPS * 100:.1f} % of the {PEAK_FP32_TFLOPS} "
              f"TFLOP/s dense fp32 MFMA peak (floor {bw['flops'] / (PEAK_FP32_TFLOPS * 1e12) * 1e6:.0f} us)."]
    with open(os.path.join(PROFILE_DIR, "backward_cfg2_rocprof.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def time_scattered(torch, dev, chunk_gdn2, args):
    """Config 2 with every input in its own allocation (the headline packs them
    into one arena, as a fused input projection would write them)."""
    sq, sk, sv, sg, sb, sw, sseg = prefill_inputs(torch, dev, packed=False)
    ms = time_calls(torch, lambda: chunk_gdn2(sq, sk, sv, sg, sb, sw, segment_ids=sseg, is_inference=True,
                                              output_final_state=True, qk_l2norm=True, precision="bf16",
                                              chunk_size=128), args.steps, args.warmup)
    log(f"prefill, scattered inputs: {ms * 1e3:.1f} us/step")
    return {"ms_per_step": round(ms, 5), "tokens_per_s": round(2048 / (ms * 1e-3), 1),
            "note": "config 2 with q, k, v, g, b, w, segment_ids each in a separate allocation"}


def main():
    if len(sys.argv) == 3 and sys.argv[1] == "--rocprof-backward-summary":
        rocprof_backward_summary(sys.argv[2])
        return
    if len(sys.argv) == 5 and sys.argv[1] == "--rocprof-summary":
        rocprof_summary(*sys.argv[2:5])
        return
    if sys.argv[1:2] == ["--rocprof-configs-summary"] and len(sys.argv) in (3, 5):
        rocprof_configs_summary(*sys.argv[2:])
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--decode-steps", type=int, default=64)
    ap.add_argument("--train-steps", type=int, default=10,
                    help="forward + backward steps timed at the config-2 shape (0 = skip)")
    ap.add_argument("--config-steps", type=int, default=12,
                    help="calls timed for configs 3 and 5 (config 5 runs a quarter of them; 0 = skip)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-kernel-trace", action="store_true",
                    help="skip the profiler activity trace (for runs under rocprofv3, which traces itself)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 1 GiB device copy (for PMC byte-counter scaling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one MI355X only; the hot path shards over (batch, head) "
              "with no communication (see DESIGN.md), so no multi-GPU figure is produced.", file=sys.stderr)
        sys.exit(2)

    import torch

    from deltanet_tpu_amd import _lib, chunk_gdn, chunk_gdn2, gdn2_decode_step, gdn2_decode_steps

    _TRACE["on"] = not args.no_kernel_trace

    dev = torch.device("cuda:0")
    q, k, v, g, b, w, seg = prefill_inputs(torch, dev)
    work = prefill_work()

    def step():
        return chunk_gdn2(q, k, v, g, b, w, segment_ids=seg, is_inference=True, output_final_state=True,
                          qk_l2norm=True, precision="bf16", chunk_size=128)

    ms_step = time_calls(torch, step, args.steps, args.warmup)
    tok_s = 2048 / (ms_step * 1e-3)
    # per-kernel device durations from the activity trace (uninstrumented);
    # the HIP-event pass is only the fallback where the trace is unavailable
    kern = kernel_times(torch, step, min(args.steps, 50))
    kern_src = "profiler activity trace (per-dispatch device timestamps, as rocprofv3 --kernel-trace)"
    if kern is None:
        _lib.profile_begin()
        for _ in range(args.steps):
            step()
        prof = _lib.profile_end()
        kern = {f"k_{name}": ms * 1e3 / n for name, (ms, n) in prof.items() if n}
        kern_src = "HIP events around each launch (instrumented: adds inter-kernel gaps)"
    log(f"prefill: {ms_step * 1e3:.1f} us/step; kernels (us): " +
        ", ".join(f"{k_}={v_:.1f}" for k_, v_ in kern.items()))

    # dominant kernel and its roofline
    dom = max(("prepass", "chain"), key=lambda n: kern.get(f"k_{n}", 0.0))
    roof = roofline_of(work, kern[f"k_{dom}"], dom)
    roof["kernel"] = f"k_{dom}"
    roof["avg_launch_us"] = round(kern[f"k_{dom}"], 2)
    roof["avg_launch_source"] = kern_src
    roof["traffic"] = None
    if os.path.exists(TRAFFIC_JSON):
        # HBM bytes per launch from the committed rocprofv3 --pmc summary
        t = json.load(open(TRAFFIC_JSON)).get("kernels", {}).get(roof["kernel"])
        if t:
            roof["traffic"] = round(t["traffic_bytes"])
            roof["traffic_source"] = os.path.relpath(TRAFFIC_JSON, ROOT)
    sroof = step_roofline(work, ms_step)

    # the same workload with every input in its own allocation (the headline
    # packs them into one arena, as a fused input projection would write them)
    scattered = None
    if not args.no_kernel_trace:   # (profiling runs keep to the headline layout)
        scattered = time_scattered(torch, dev, chunk_gdn2, args)

    # ---- configs 3 and 5 (timed lines beside the headline) ------------------
    others = {}
    if args.config_steps > 0:
        c3 = config3_inputs(torch, dev)
        w3 = prefill_work(B=4, L=8192, Hk=16, Hv=32, gates="scalar")

        def step3():
            return chunk_gdn(c3[0], c3[1], c3[2], c3[3], c3[4], segment_ids=c3[5], is_inference=True,
                             output_final_state=True, qk_l2norm=True, precision="bf16")

        ms3 = time_calls(torch, step3, args.config_steps, 2)
        others["config3"] = {"workload": "chunk_gdn prefill, BASELINE config 3: B=4 L=8192 Hk=16 Hv=32 K=V=128, "
                                         "bf16 qkv, scalar fp32 g/beta per value head, geometric(1024) packed "
                                         "documents, precision bf16, qk_l2norm, is_inference, chunk 128",
                             "ms_per_call": round(ms3, 4), "tokens_per_s": round(4 * 8192 / (ms3 * 1e-3), 1),
                             "step_roofline": step_roofline(w3, ms3),
                             "kernels_us": {k_: round(v_, 2) for k_, v_ in (kernel_times(torch, step3, 3) or {}).items()}}
        del c3
        log(f"config 3: {ms3 * 1e3:.1f} us/call")
        c5 = config5_inputs(torch, dev)
        w5 = prefill_work(B=1, L=65536, Hk=16, Hv=32)

        def step5():
            return chunk_gdn2(c5[0], c5[1], c5[2], c5[3], c5[4], c5[5], segment_ids=c5[6], is_inference=True,
                              output_final_state=True, qk_l2norm=True, fuse_prologue=True, precision="bf16",
                              streaming_prefill=True, prefill_block_size=8192)

        ms5 = time_calls(torch, step5, max(1, args.config_steps // 4), 1)
        others["config5"] = {"workload": "chunk_gdn2 streaming prefill, BASELINE config 5: B=1 L=65536 Hk=16 Hv=32 "
                                         "K=V=128, bf16 qkv, raw fp32 gates with fuse_prologue, geometric(8192) "
                                         "documents, prefill_block_size 8192, precision bf16, qk_l2norm",
                             "ms_per_call": round(ms5, 4), "tokens_per_s": round(65536 / (ms5 * 1e-3), 1),
                             "step_roofline": step_roofline(w5, ms5),
                             "kernels_us": {k_: round(v_, 2) for k_, v_ in (kernel_times(torch, step5, 1) or {}).items()}}
        del c5
        log(f"config 5: {ms5 * 1e3:.1f} us/call")
        torch.cuda.empty_cache()

    # ---- decode (config 4) ------------------------------------------------
    dq, dk, dv, dg, db, dw, st = decode_inputs(torch, dev)
    dec = {}
    # every state dtype with and without a reset vector (a device bool tensor,
    # all False, as a serving loop passes it: read in place by the kernel)
    no_reset = torch.zeros(dq.shape[0], dtype=torch.bool, device=dev)
    cases = [(sd, elt, rs) for sd, elt in (("float32", 4), ("bfloat16", 2)) for rs in (None, no_reset)]
    for sd, elt, rs in cases if args.decode_steps > 0 else ():
        s_in = st if sd == "float32" else st.to(torch.bfloat16)
        s_out = torch.empty_like(s_in)
        n = args.decode_steps
        tag = sd if rs is None else sd + "_reset"

        def dstep(a, bb):
            return gdn2_decode_step(dq, dk, dv, dg, db, dw, a, qk_l2norm=True, state_dtype=sd, out_state=bb,
                                    reset=rs)

        pair = [s_in, s_out]

        def dstep2():
            dstep(pair[0], pair[1])
            pair.reverse()

        us = time_calls(torch, dstep2, n, 5) * 1e3
        kt = kernel_times(torch, dstep2, n)
        if kt:
            kus = next(v_ for k_, v_ in kt.items() if k_.startswith("k_decode"))
        else:
            _lib.profile_begin()
            for _ in range(n):
                dstep2()
            dprof = _lib.profile_end()
            kus = dprof["decode"][0] * 1e3 / max(dprof["decode"][1], 1)
        sbytes = 2 * st.numel() * elt
        dec[tag] = {"us_per_step": round(us, 2), "kernel_us": round(kus, 2),
                    "state_GBps": round(sbytes / (kus * 1e-6) / 1e9, 1),
                    "frac_hbm_peak": round(sbytes / (kus * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)}
        log(f"decode {tag}: {us:.1f} us/step (kernel {kus:.1f} us, {dec[tag]['state_GBps']} GB/s)")

    # ---- multi-token decode (dn_decode_steps), config-4 shape, 16 tokens per launch
    dsteps = {}
    if args.decode_steps > 0:
        Tm = 16
        gm = torch.Generator(device=dev)
        gm.manual_seed(41)
        rn = lambda *s_: torch.randn(*s_, device=dev, generator=gm)
        Bm, Hkm, Hvm = dq.shape[0], dq.shape[2], dv.shape[2]
        mq, mk = rn(Bm, Tm, Hkm, 128).to(torch.bfloat16), rn(Bm, Tm, Hkm, 128).to(torch.bfloat16)
        mv = rn(Bm, Tm, Hvm, 128).to(torch.bfloat16)
        mg = -torch.exp(0.39 * rn(Bm, Tm, Hkm, 128) - 1.0)
        mb, mw = torch.sigmoid(0.39 * rn(Bm, Tm, Hkm, 128)), torch.sigmoid(0.39 * rn(Bm, Tm, Hvm, 128))
        for sd, elt in (("float32", 4), ("bfloat16", 2)):
            s_in = st if sd == "float32" else st.to(torch.bfloat16)
            pair = [s_in, torch.empty_like(s_in)]

            def mstep():
                gdn2_decode_steps(mq, mk, mv, mg, mb, mw, pair[0], qk_l2norm=True, state_dtype=sd, out_state=pair[1])
                pair.reverse()

            n = max(4, args.decode_steps // 4)
            us = time_calls(torch, mstep, n, 3) * 1e3
            kt = kernel_times(torch, mstep, n)
            kus = next((v_ for k_, v_ in (kt or {}).items() if k_.startswith("k_decode")), us)
            sbytes = 2 * st.numel() * elt
            dsteps[sd] = {"tokens_per_launch": Tm, "us_per_launch": round(us, 2), "kernel_us": round(kus, 2),
                          "kernel_us_per_token": round(kus / Tm, 2),
                          "state_GBps": round(sbytes / (kus * 1e-6) / 1e9, 1)}
            log(f"decode_steps {sd} T={Tm}: kernel {kus:.1f} us ({kus / Tm:.1f} us/token)")

    # ---- training step (forward + backward) at the config-2 shape ----------
    train = None
    if args.train_steps > 0:
        tq, tk, tv, tg, tb, tw = (x.requires_grad_(True) for x in _pack(torch, dev, (q, k, v, g, b, w)))
        tdo = torch.randn(tv.shape, device=dev, generator=torch.Generator(device=dev).manual_seed(9)).to(tv.dtype)

        leaves = (tq, tk, tv, tg, tb, tw)

        def tstep():
            # gradients are cleared each step, as optimizer.zero_grad() (set_to_none) does in a
            # training loop, so backward writes them instead of accumulating into last step's
            for x in leaves:
                x.grad = None
            o = chunk_gdn2(tq, tk, tv, tg, tb, tw, segment_ids=seg, is_inference=False, qk_l2norm=True,
                           precision="bf16", chunk_size=128)
            o.backward(tdo)

        for _ in range(3):
            tstep()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.train_steps):
            tstep()
        torch.cuda.synchronize()
        t_us = (time.perf_counter() - t0) * 1e6 / args.train_steps
        tk_us = kernel_times(torch, tstep, args.train_steps, per_call=True)
        if tk_us:
            tk_us = {n: round(v_, 1) for n, v_ in tk_us.items()}
            # the recurrence backward proper (the raw entry's prep / post kernels aside)
            bw_us = sum(tk_us.get(n, 0.0) for n in ("k_bw_intra", "k_bw_chains", "k_bw_grads", "k_bw_dqk"))
        else:
            _lib.profile_begin()
            for _ in range(args.train_steps):
                tstep()
            torch.cuda.synchronize()
            tprof = _lib.profile_end()
            tk_us = {n: round(ms * 1e3 / args.train_steps, 1) for n, (ms, c) in tprof.items() if c}
            bw_us = tk_us.get("backward", 0.0)
        bw = backward_work(H=tv.shape[2])
        bw_s = bw_us * 1e-6
        train = {"workload": "chunk_gdn2 forward + backward (is_inference=False, autograd), config-2 shape, "
                             "precision bf16 (backward: split-bf16 scans and gradient products)", "us_per_step": round(t_us, 1),
                 "kernels_us_per_step": tk_us,
                 "backward_roofline": {"bound": "mfma", "dtype": "fp32", "flops": bw["flops"],
                                       "achieved": round(bw["flops"] / bw_s / 1e12, 2) if bw_s else None,
                                       "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                                       "frac": round(bw["flops"] / bw_s / 1e12 / PEAK_FP32_TFLOPS, 4) if bw_s else None,
                                       "note": "algorithmic fp32 flops of the recurrence backward against the dense fp32 "
                                               "MFMA peak; in bf16 mode the scans, k_bw_grads and most of k_bw_intra carry "
                                               "those products as split-bf16 MFMAs (3 per product), k_bw_intra's A / M "
                                               "and k_bw_dqk as fp32"}}
        log(f"training step: {t_us:.1f} us; kernels per step (us): {tk_us}")

    copy_gbps = None
    if args.copy_calibration:
        # a plain device copy of the decode state's size: the practical
        # read + write HBM rate the decode step is compared against
        src = torch.empty(256 * 32 * 128 * 128, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(50):
            dst.copy_(src)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / 50
        copy_gbps = round(2 * src.numel() * 4 / dt / 1e9, 1)
        log(f"device copy of {src.numel() * 4 >> 20} MiB: {dt * 1e6:.1f} us, {copy_gbps} GB/s (read + write)")

    cpu, parity = None, None
    if not args.no_cpu_baseline:
        try:
            o_gpu, s_gpu = step()
            torch.cuda.synchronize()
            cpu, parity = cpu_baseline((q, k, v, g, b, w, seg), o_gpu, s_gpu, args.cpu_seconds)
            log(f"cpu baseline: {cpu['value']:.1f} tokens/s on {cpu['cores']} threads; parity {parity}")
            try:
                cpu["more"] = cpu_baselines_more()
                log(f"cpu baselines, other legs: {cpu['more']}")
            except Exception as e:  # noqa: BLE001
                log(f"further cpu legs unavailable: {e}")
        except Exception as e:  # the GPU figure stands on its own
            log(f"cpu baseline unavailable: {e}")

    line = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v, sigmoid/exp gates as BASELINE.json configs[1])",
        "config": {"workload": "chunk_gdn2 prefill, BASELINE config 2: B=1 L=2048 Hk=12 Hv=24 K=V=128, "
                               "bf16 qkv, fp32 gates, 2 segments, chunk 128, precision bf16, qk_l2norm, "
                               "is_inference, fp32 final state",
                   "B": 1, "L": 2048, "Hk": 12, "Hv": 24, "K": 128, "V": 128},
        "mfma_pct_peak": sroof["mfma_pct_peak"],
        "step_roofline": sroof,
        "kernels_us": {k_: round(v_, 2) for k_, v_ in kern.items()},
        "kernels_us_source": kern_src,
        "prefill_scattered_inputs": scattered,
        "other_configs": others,
        "roofline": roof,
        "decode": {"workload": "gdn2_decode_step, BASELINE config 4: B=256 Hk=16 Hv=32 K=V=128, bf16 qkv, "
                               "channel-wise fp32 gates, qk_l2norm", **dec},
        "decode_steps": {"workload": "gdn2_decode_steps, config-4 shape, 16 tokens per launch (chunked WY form), "
                                     "bf16 qkv, channel-wise fp32 gates, qk_l2norm", **dsteps},
        "training": train,
        "cpu_baseline": cpu,
        "parity_vs_oracle": parity,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
