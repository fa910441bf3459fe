"""AutoAWQ safetensors ingestion for the Qwen2 decode harness.

The reference reads every tensor of ``<model_dir>/*.safetensors``
(``model/loader.py:23-35``), copies them into its module buffers by name and
then concatenates Q/K/V and gate/up into fused projections
(``model/qwen2.py:255-276``, ``:79-85``, ``:174-178``).  ``load_qwen2_awq``
does the same in one pass: it reads ``config.json`` (``model/loader.py:7-14``)
into a ``Qwen2Shape``, checks every AWQ operand against the packing the
kernels read (int32 ``qweight [K, N/8]``, int32 ``qzeros [K/G, N/8]``,
fp16 ``scales [K/G, N]``, group size 128 -- ``model/qwen2.py:34-36``), and
fuses QKV (with the q/k/v biases) and gate||up by concatenating along the
packed-column axis, which keeps each sub-projection's columns (and their
nibble order) intact.  Missing or misshapen tensors raise; tensors the
harness does not use are reported in the result.

Tensor names are the Hugging Face / AutoAWQ ones the reference's module tree
matches (``model.layers.{i}.self_attn.q_proj.qweight``, ...,
``model.embed_tokens.weight``, ``model.norm.weight``, ``lm_head.weight``).
"""
from __future__ import annotations

import glob
import json
import os

import torch

from .qwen2_decode import Qwen2Shape

__all__ = ["load_config", "load_qwen2_awq", "save_qwen2_awq"]

_PROJ = {"q_proj": "self_attn", "k_proj": "self_attn", "v_proj": "self_attn", "o_proj": "self_attn",
         "gate_proj": "mlp", "up_proj": "mlp", "down_proj": "mlp"}


def load_config(model_dir: str) -> Qwen2Shape:
    """``config.json`` -> Qwen2Shape (group size from ``quantization_config``)."""
    path = os.path.join(model_dir, "config.json")
    if not os.path.exists(path):
        raise FileNotFoundError(f"Config file not found: {path}")
    with open(path, encoding="utf-8") as f:
        c = json.load(f)
    q = c.get("quantization_config", {})
    group = int(q.get("group_size", 128))
    bits = int(q.get("bits", q.get("w_bit", 4)))
    if group != 128 or bits != 4:
        raise ValueError(f"only 4-bit AWQ with group size 128 is served (got {bits} bits, group {group})")
    return Qwen2Shape(vocab_size=c["vocab_size"], hidden_size=c["hidden_size"],
                      intermediate_size=c["intermediate_size"], num_layers=c["num_hidden_layers"],
                      num_heads=c["num_attention_heads"],
                      num_kv_heads=c.get("num_key_value_heads", c["num_attention_heads"]),
                      rms_norm_eps=c.get("rms_norm_eps", 1e-6), rope_theta=c.get("rope_theta", 1e6),
                      group_size=group)


def _tensors(model_dir: str) -> dict:
    from safetensors.torch import load_file

    files = sorted(glob.glob(os.path.join(model_dir, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"No .safetensors files found in {model_dir}")
    out = {}
    for fp in files:
        out.update(load_file(fp, device="cpu"))
    return out


def _awq(t: dict, prefix: str, k: int, n: int, group: int):
    names = [f"{prefix}.qweight", f"{prefix}.qzeros", f"{prefix}.scales"]
    for nm in names:
        if nm not in t:
            raise KeyError(f"missing tensor {nm}")
    qw, qz, sc = (t.pop(nm) for nm in names)
    want = {"qweight": ((k, n // 8), torch.int32), "qzeros": ((k // group, n // 8), torch.int32),
            "scales": ((k // group, n), torch.float16)}
    for nm, v in zip(("qweight", "qzeros", "scales"), (qw, qz, sc)):
        shape, dtype = want[nm]
        if tuple(v.shape) != shape or v.dtype != dtype:
            raise ValueError(f"{prefix}.{nm}: {tuple(v.shape)} {v.dtype}, expected {shape} {dtype}")
    return qw.contiguous(), qz.contiguous(), sc.contiguous()


def _fuse(*ops):
    return tuple(torch.cat([op[i] for op in ops], dim=1).contiguous() for i in range(3))


def load_qwen2_awq(model_dir: str):
    """Returns (shape, weights, unused_tensor_names); ``weights`` feeds
    ``Qwen2AwqDecoder(shape, weights=weights)``.  Tensors stay on the CPU."""
    s = load_config(model_dir)
    t = _tensors(model_dir)
    H, I, G = s.hidden_size, s.intermediate_size, s.group_size
    hd = s.head_dim
    qn, kvn = s.num_heads * hd, s.num_kv_heads * hd

    def take(name, shape, dtype=torch.float16):
        if name not in t:
            raise KeyError(f"missing tensor {name}")
        v = t.pop(name)
        if tuple(v.shape) != tuple(shape):
            raise ValueError(f"{name}: shape {tuple(v.shape)}, expected {tuple(shape)}")
        return v.to(dtype).contiguous()

    layers = []
    for i in range(s.num_layers):
        p = f"model.layers.{i}"
        q = _awq(t, f"{p}.self_attn.q_proj", H, qn, G)
        k = _awq(t, f"{p}.self_attn.k_proj", H, kvn, G)
        v = _awq(t, f"{p}.self_attn.v_proj", H, kvn, G)
        bias = torch.cat([take(f"{p}.self_attn.{n}_proj.bias", (m,)) for n, m in (("q", qn), ("k", kvn), ("v", kvn))])
        layers.append({
            "ln1": take(f"{p}.input_layernorm.weight", (H,)),
            "ln2": take(f"{p}.post_attention_layernorm.weight", (H,)),
            "qkv": _fuse(q, k, v),
            "qkv_bias": bias,
            "o": _awq(t, f"{p}.self_attn.o_proj", qn, H, G),
            "gate_up": _fuse(_awq(t, f"{p}.mlp.gate_proj", H, I, G), _awq(t, f"{p}.mlp.up_proj", H, I, G)),
            "down": _awq(t, f"{p}.mlp.down_proj", I, H, G),
        })
    embed = take("model.embed_tokens.weight", (s.vocab_size, H))
    lm_head = take("lm_head.weight", (s.vocab_size, H)) if "lm_head.weight" in t else embed  # tied
    weights = {"embed": embed, "lm_head": lm_head, "final_norm": take("model.norm.weight", (H,)),
               "layers": layers}
    return s, weights, sorted(t)


def save_qwen2_awq(model_dir: str, shape: Qwen2Shape, weights: dict, shard_layers: int = 0) -> None:
    """Writes ``weights`` (the harness's fused form) back as an AutoAWQ-named
    checkpoint: ``config.json`` plus ``*.safetensors`` with the per-projection
    tensors (fused QKV / gate||up split at their column boundaries).  For
    tests and for producing fixtures; ``shard_layers`` > 0 writes that many
    layers per file."""
    from safetensors.torch import save_file

    os.makedirs(model_dir, exist_ok=True)
    H, I = shape.hidden_size, shape.intermediate_size
    hd = shape.head_dim
    qn, kvn = shape.num_heads * hd, shape.num_kv_heads * hd
    cfg = {"architectures": ["Qwen2ForCausalLM"], "vocab_size": shape.vocab_size, "hidden_size": H,
           "intermediate_size": I, "num_hidden_layers": shape.num_layers,
           "num_attention_heads": shape.num_heads, "num_key_value_heads": shape.num_kv_heads,
           "rms_norm_eps": shape.rms_norm_eps, "rope_theta": shape.rope_theta,
           "tie_word_embeddings": False,
           "quantization_config": {"quant_method": "awq", "bits": 4, "group_size": 128, "zero_point": True,
                                   "version": "gemm"}}
    with open(os.path.join(model_dir, "config.json"), "w", encoding="utf-8") as f:
        json.dump(cfg, f, indent=1)

    def split(op, cols):
        out, c0 = [], 0
        for c in cols:
            out.append((op[0][:, c0 // 8:(c0 + c) // 8], op[1][:, c0 // 8:(c0 + c) // 8], op[2][:, c0:c0 + c]))
            c0 += c
        return out

    def put(d, prefix, op):
        d[f"{prefix}.qweight"], d[f"{prefix}.qzeros"], d[f"{prefix}.scales"] = (x.contiguous().cpu() for x in op)

    shards, cur = [], {}
    for i, lw in enumerate(weights["layers"]):
        p = f"model.layers.{i}"
        q, k, v = split(lw["qkv"], (qn, kvn, kvn))
        for nm, op in (("q", q), ("k", k), ("v", v)):
            put(cur, f"{p}.self_attn.{nm}_proj", op)
        b = lw["qkv_bias"].cpu()
        cur[f"{p}.self_attn.q_proj.bias"] = b[:qn].contiguous()
        cur[f"{p}.self_attn.k_proj.bias"] = b[qn:qn + kvn].contiguous()
        cur[f"{p}.self_attn.v_proj.bias"] = b[qn + kvn:].contiguous()
        put(cur, f"{p}.self_attn.o_proj", lw["o"])
        g, u = split(lw["gate_up"], (I, I))
        put(cur, f"{p}.mlp.gate_proj", g)
        put(cur, f"{p}.mlp.up_proj", u)
        put(cur, f"{p}.mlp.down_proj", lw["down"])
        cur[f"{p}.input_layernorm.weight"] = lw["ln1"].cpu().contiguous()
        cur[f"{p}.post_attention_layernorm.weight"] = lw["ln2"].cpu().contiguous()
        if shard_layers and (i + 1) % shard_layers == 0:
            shards.append(cur)
            cur = {}
    cur["model.embed_tokens.weight"] = weights["embed"].cpu().contiguous()
    cur["model.norm.weight"] = weights["final_norm"].cpu().contiguous()
    cur["lm_head.weight"] = weights["lm_head"].cpu().contiguous()
    shards.append(cur)
    for j, d in enumerate(shards):
        save_file(d, os.path.join(model_dir, f"model-{j + 1:05d}-of-{len(shards):05d}.safetensors"))
