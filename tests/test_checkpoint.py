"""AutoAWQ safetensors ingestion (``engine/awq_checkpoint.py``): the names,
shapes and fusion of the reference's loader (``model/loader.py:23-35``,
``model/qwen2.py:79-85,174-178,255-276``).  CPU only."""
import json
import os

import numpy as np
import pytest
import torch

from engine.awq_checkpoint import load_config, load_qwen2_awq, save_qwen2_awq
from engine.qwen2_decode import Qwen2Shape
from oracle import awq_oracle as O

TINY = Qwen2Shape(vocab_size=96, hidden_size=256, intermediate_size=384, num_layers=3, num_heads=4,
                  num_kv_heads=2)


def _awq(k, n, g):
    return (torch.randint(-2**31, 2**31 - 1, (k, n // 8), generator=g, dtype=torch.int32),
            torch.randint(-2**31, 2**31 - 1, (k // 128, n // 8), generator=g, dtype=torch.int32),
            (torch.rand((k // 128, n), generator=g) * 0.018 + 0.002).half())


def _weights(s, seed=0):
    g = torch.Generator().manual_seed(seed)
    H, I = s.hidden_size, s.intermediate_size
    qkv_n = (s.num_heads + 2 * s.num_kv_heads) * s.head_dim
    return {"embed": torch.randn((s.vocab_size, H), generator=g).half(),
            "lm_head": torch.randn((s.vocab_size, H), generator=g).half(),
            "final_norm": torch.randn(H, generator=g).half(),
            "layers": [{"ln1": torch.randn(H, generator=g).half(), "ln2": torch.randn(H, generator=g).half(),
                        "qkv": _awq(H, qkv_n, g), "qkv_bias": torch.randn(qkv_n, generator=g).half(),
                        "o": _awq(H, H, g), "gate_up": _awq(H, 2 * I, g), "down": _awq(I, H, g)}
                       for _ in range(s.num_layers)]}


def _eq(a, b):
    if isinstance(a, tuple):
        return all(torch.equal(x, y) for x, y in zip(a, b))
    return torch.equal(a, b)


def test_round_trip_sharded(tmp_path):
    w = _weights(TINY)
    save_qwen2_awq(str(tmp_path), TINY, w, shard_layers=2)
    assert len([f for f in os.listdir(tmp_path) if f.endswith(".safetensors")]) == 2
    s, w2, unused = load_qwen2_awq(str(tmp_path))
    assert s == TINY and unused == []
    for key in ("embed", "lm_head", "final_norm"):
        assert torch.equal(w[key], w2[key])
    for a, b in zip(w["layers"], w2["layers"]):
        for key in a:
            assert _eq(a[key], b[key]), key


def test_fusion_keeps_logical_columns(tmp_path):
    """The fused QKV / gate||up operands dequantise to the column
    concatenation of the per-projection weights (what the reference's
    torch.cat of packed tensors means, model/qwen2.py:79-85,174-178)."""
    w = _weights(TINY, seed=1)
    save_qwen2_awq(str(tmp_path), TINY, w)
    from safetensors.torch import load_file

    f = load_file(os.path.join(tmp_path, "model-00001-of-00001.safetensors"))
    _, w2, _ = load_qwen2_awq(str(tmp_path))
    p = "model.layers.1"
    parts = [tuple(f[f"{p}.self_attn.{n}_proj.{t}"].numpy() for t in ("qweight", "qzeros", "scales"))
             for n in ("q", "k", "v")]
    dense = np.concatenate([O.dequant_awq(*pp) for pp in parts], axis=1)
    fused = O.dequant_awq(*(x.numpy() for x in w2["layers"][1]["qkv"]))
    assert np.array_equal(dense.view(np.uint16), fused.view(np.uint16))
    parts = [tuple(f[f"{p}.mlp.{n}_proj.{t}"].numpy() for t in ("qweight", "qzeros", "scales"))
             for n in ("gate", "up")]
    codes = np.concatenate([O.unpack_awq(pp[0]) for pp in parts], axis=1)
    assert np.array_equal(codes, O.unpack_awq(w2["layers"][1]["gate_up"][0].numpy()))


def test_missing_and_misshapen_tensors_raise(tmp_path):
    from safetensors.torch import load_file, save_file

    w = _weights(TINY, seed=2)
    save_qwen2_awq(str(tmp_path), TINY, w)
    fp = os.path.join(tmp_path, "model-00001-of-00001.safetensors")
    t = load_file(fp)
    bad = dict(t)
    del bad["model.layers.2.mlp.down_proj.scales"]
    save_file(bad, fp)
    with pytest.raises(KeyError, match="down_proj.scales"):
        load_qwen2_awq(str(tmp_path))
    bad = dict(t)
    bad["model.layers.0.self_attn.o_proj.qweight"] = bad["model.layers.0.self_attn.o_proj.qweight"][:, :-1].contiguous()
    save_file(bad, fp)
    with pytest.raises(ValueError, match="o_proj.qweight"):
        load_qwen2_awq(str(tmp_path))
    bad = dict(t)
    bad["model.layers.0.mlp.up_proj.scales"] = bad["model.layers.0.mlp.up_proj.scales"].float()
    save_file(bad, fp)
    with pytest.raises(ValueError, match="up_proj.scales"):
        load_qwen2_awq(str(tmp_path))


def test_config_rejects_other_quantisation(tmp_path):
    save_qwen2_awq(str(tmp_path), TINY, _weights(TINY))
    cp = os.path.join(tmp_path, "config.json")
    c = json.load(open(cp))
    assert load_config(str(tmp_path)) == TINY
    c["quantization_config"]["group_size"] = 64
    json.dump(c, open(cp, "w"))
    with pytest.raises(ValueError, match="group size"):
        load_config(str(tmp_path))
