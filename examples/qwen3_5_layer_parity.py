"""Qwen3.5 linear-attention layer parity on MI355X.

Runs one Qwen3.5 GatedDeltaNet layer's recurrence through this build's HIP
kernels (``chunk_gdn`` for the prefill, ``gdn_decode_step`` for the next token)
and through the PyTorch reference recurrences that ship with transformers
(``torch_chunk_gated_delta_rule`` / ``torch_recurrent_gated_delta_rule``), on
the same projected inputs, and reports rel L2 errors (reference:
examples/qwen3_5_layer_parity.py:1-288, tolerance 1e-4).

Layer weights come from a local checkpoint directory (``config.json`` plus
``model.safetensors`` or a sharded ``model.safetensors.index.json``); without
one, the layer is a seeded random initialisation of the same architecture
(transformers' Qwen3_5TextConfig defaults: 16 key heads, 32 value heads,
K = V = 128).  Nothing is downloaded.

    python examples/qwen3_5_layer_parity.py --model /path/to/Qwen3.5-2B --seq-len 128
    python examples/qwen3_5_layer_parity.py --random --hidden-size 1024
"""

from __future__ import annotations

import argparse
import json
import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "deltanet-tpu_amd"))

LAYER_PREFIXES = ("model.language_model.layers.{i}.linear_attn.", "model.layers.{i}.linear_attn.")
EXPECTED = {"in_proj_qkv.weight", "in_proj_a.weight", "in_proj_b.weight", "conv1d.weight", "A_log", "dt_bias"}


def _text_config(model_path=None, hidden_size=None):
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5Config, Qwen3_5TextConfig
    if model_path is None:
        kw = {} if hidden_size is None else {"hidden_size": hidden_size}
        return Qwen3_5TextConfig(**kw)
    with open(os.path.join(model_path, "config.json")) as f:
        raw = json.load(f)
    if "text_config" in raw:
        cfg = Qwen3_5Config.from_pretrained(model_path)
        return cfg.text_config
    return Qwen3_5TextConfig.from_pretrained(model_path)


def _checkpoint_tensors(model_path, layer_idx):
    """The layer's tensors from a local safetensors checkpoint (one file or shards)."""
    from safetensors import safe_open
    files = []
    index = os.path.join(model_path, "model.safetensors.index.json")
    if os.path.exists(index):
        with open(index) as f:
            wm = json.load(f).get("weight_map", {})
        pre = [p.format(i=layer_idx) for p in LAYER_PREFIXES]
        files = sorted({os.path.join(model_path, s) for k, s in wm.items() if any(k.startswith(x) for x in pre)})
    else:
        for name in ("model.safetensors", "model.safetensors-00001-of-00001.safetensors"):
            if os.path.exists(os.path.join(model_path, name)):
                files = [os.path.join(model_path, name)]
                break
    if not files:
        raise FileNotFoundError(f"no safetensors checkpoint under {model_path}")
    out = {}
    for fn in files:
        with safe_open(fn, framework="pt") as f:
            for key in f.keys():
                for p in LAYER_PREFIXES:
                    p = p.format(i=layer_idx)
                    if key.startswith(p):
                        out[key[len(p):]] = f.get_tensor(key)
    missing = EXPECTED - set(out)
    if missing:
        raise KeyError(f"checkpoint {model_path} lacks layer {layer_idx} tensors {sorted(missing)}")
    return out


def build_layer(model_path=None, layer_idx=0, hidden_size=None, seed=0):
    """A float32 Qwen3_5GatedDeltaNet and its text config (checkpoint or seeded random)."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5GatedDeltaNet
    cfg = _text_config(model_path, hidden_size)
    torch.manual_seed(seed)
    layer = Qwen3_5GatedDeltaNet(cfg, layer_idx=layer_idx)
    if model_path is not None:
        layer.load_state_dict(_checkpoint_tensors(model_path, layer_idx), strict=False)
    return layer.float().eval(), cfg


@torch.no_grad()
def layer_inputs(layer, x):
    """q, k (B,L,Hk,K), v (B,L,Hv,V), g, beta (B,L,Hv) exactly as the layer's
    forward derives them: projection, causal depthwise conv + SiLU, gates."""
    B, L, _ = x.shape
    mixed = layer.in_proj_qkv(x).transpose(1, 2)
    kc = layer.conv_kernel_size
    conv = F.conv1d(F.pad(mixed, (kc - 1, 0)), layer.conv1d.weight, layer.conv1d.bias, groups=layer.conv_dim)
    mixed = F.silu(conv[:, :, :L]).transpose(1, 2)
    q, k, v = torch.split(mixed, [layer.key_dim, layer.key_dim, layer.value_dim], dim=-1)
    q = q.reshape(B, L, layer.num_k_heads, layer.head_k_dim)
    k = k.reshape(B, L, layer.num_k_heads, layer.head_k_dim)
    v = v.reshape(B, L, layer.num_v_heads, layer.head_v_dim)
    beta = layer.in_proj_b(x).sigmoid()
    g = -layer.A_log.float().exp() * F.softplus(layer.in_proj_a(x).float() + layer.dt_bias)
    return q.contiguous(), k.contiguous(), v.contiguous(), g.contiguous(), beta.contiguous()


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-30))


@torch.no_grad()
def run_parity(layer, seq_len=128, batch=1, seed=42, device="cuda:0"):
    """Prefill of seq_len tokens then one decode step, HIP vs transformers' torch
    recurrences (fp32 on the CPU).  Returns the four rel L2 errors."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import (torch_chunk_gated_delta_rule,
                                                              torch_recurrent_gated_delta_rule)
    from deltanet_tpu_amd import chunk_gdn, gdn_decode_step

    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, seq_len + 1, layer.hidden_size, generator=gen)
    q, k, v, g, beta = layer_inputs(layer, x)
    rep = layer.num_v_heads // layer.num_k_heads
    qr = q.repeat_interleave(rep, dim=2) if rep > 1 else q
    kr = k.repeat_interleave(rep, dim=2) if rep > 1 else k
    P = slice(0, seq_len)
    ref_o, ref_s = torch_chunk_gated_delta_rule(qr[:, P], kr[:, P], v[:, P], g=g[:, P], beta=beta[:, P],
                                                initial_state=None, output_final_state=True,
                                                use_qk_l2norm_in_kernel=True)
    T = slice(seq_len, seq_len + 1)
    ref_do, ref_ds = torch_recurrent_gated_delta_rule(qr[:, T], kr[:, T], v[:, T], g=g[:, T], beta=beta[:, T],
                                                      initial_state=ref_s, output_final_state=True,
                                                      use_qk_l2norm_in_kernel=True)
    d = lambda t: t.to(device)
    out, st = chunk_gdn(d(q[:, P]), d(k[:, P]), d(v[:, P]), d(g[:, P]), d(beta[:, P]), output_final_state=True,
                        is_inference=True, precision="fp32", qk_l2norm=True)
    dout, dst = gdn_decode_step(d(q[:, seq_len]), d(k[:, seq_len]), d(v[:, seq_len]), d(g[:, seq_len]),
                                d(beta[:, seq_len]), st, qk_l2norm=True)
    torch.cuda.synchronize()
    return {
        "prefill_output_rel_l2": _rel(out.cpu(), ref_o),
        "prefill_final_state_rel_l2": _rel(st.cpu(), ref_s),
        "decode_output_rel_l2": _rel(dout.cpu(), ref_do[:, 0]),
        "decode_final_state_rel_l2": _rel(dst.float().cpu(), ref_ds),
    }


def main():
    ap = argparse.ArgumentParser(description="Qwen3.5 linear-attention layer parity (HIP vs PyTorch)")
    ap.add_argument("--model", default=None, help="local checkpoint directory (config.json + safetensors)")
    ap.add_argument("--random", action="store_true", help="seeded random weights of the architecture")
    ap.add_argument("--hidden-size", type=int, default=None, help="hidden size of a random layer")
    ap.add_argument("--layer", type=int, default=0)
    ap.add_argument("--seq-len", type=int, default=128)
    ap.add_argument("--output", default=None, help="write the results as JSON here")
    args = ap.parse_args()
    if args.model is None and not args.random:
        ap.error("give --model <local checkpoint dir> or --random")
    layer, cfg = build_layer(args.model, args.layer, args.hidden_size)
    print(f"layer {args.layer}: Hk={cfg.linear_num_key_heads} Hv={cfg.linear_num_value_heads} "
          f"K={cfg.linear_key_head_dim} V={cfg.linear_value_head_dim} hidden={cfg.hidden_size} "
          f"({'checkpoint ' + args.model if args.model else 'random weights'})")
    res = run_parity(layer, args.seq_len)
    for k_, v_ in res.items():
        print(f"{k_:30s} {v_:.4e}")
    import transformers
    res.update({"model": args.model or "random", "layer_idx": args.layer, "seq_len": args.seq_len,
                "transformers_version": transformers.__version__, "torch_version": torch.__version__,
                "device": torch.cuda.get_device_name(0), "precision": "fp32"})
    if args.output:
        with open(args.output, "w") as f:
            json.dump(res, f, indent=2)
    bad = {k_: v_ for k_, v_ in res.items() if k_.endswith("rel_l2") and not v_ < 1e-4}
    if bad:
        raise SystemExit(f"parity above 1e-4: {bad}")
    print("parity within 1e-4")


if __name__ == "__main__":
    main()
