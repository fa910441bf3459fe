"""End-to-end decoding at the Qwen2-7B shape (28 layers, the greedy decode workload) against an
independent model: HuggingFace transformers' ``Qwen2ForCausalLM`` (the
canonical implementation of the architecture the reference reproduces in
``model/qwen2.py``), in fp32 with eager attention, loaded with the oracle's
exactly dequantised weights ``fp16((q - z) * s)`` of the harness's AWQ
layers.  None of the harness's code (RMSNorm, RoPE, GQA attention, bias and
residual placement, QKV / gate||up split) is shared with it.

* tiny and full-width (hidden 3584, intermediate 18944, vocab 152064, 28 / 4
  heads) models of two layers: prefill and teacher-forced decode logits
  within max relative error 1e-2 of the HuggingFace logits;
* the full 28-layer Qwen2-7B shape at the decode workload's own size (a
  1024-token prompt, 128 greedy tokens): the graph-replayed greedy tokens
  equal the eager loop's (same kernels, same order: bitwise), and every logit
  of the prefill and of each eager decode step is finite.
"""
import numpy as np
import pytest
import torch

from engine.qwen2_decode import QWEN2_7B, Qwen2AwqDecoder, Qwen2Shape
from oracle import awq_oracle as O

pytestmark = pytest.mark.gpu

TINY = Qwen2Shape(vocab_size=512, hidden_size=256, intermediate_size=512, num_layers=2, num_heads=4,
                  num_kv_heads=2)
QWEN2_7B_2L = Qwen2Shape(num_layers=2)


def _dense_t(op, dev):
    """Oracle dequantisation of an AWQ (qweight, qzeros, scales) triple, as an
    fp32 nn.Linear weight [N, K]."""
    qw, qz, sc = (t.cpu().numpy() for t in op)
    return torch.from_numpy(O.dequant_awq(qw, qz, sc).astype(np.float32)).to(dev).t().contiguous()


def _hf_model(m: Qwen2AwqDecoder, dev):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    s = m.s
    cfg = Qwen2Config(vocab_size=s.vocab_size, hidden_size=s.hidden_size, intermediate_size=s.intermediate_size,
                      num_hidden_layers=s.num_layers, num_attention_heads=s.num_heads,
                      num_key_value_heads=s.num_kv_heads, max_position_embeddings=m.max_seq_len,
                      rope_theta=s.rope_theta, rms_norm_eps=s.rms_norm_eps, tie_word_embeddings=False)
    with torch.device(dev):
        hf = Qwen2ForCausalLM._from_config(cfg, attn_implementation="eager", dtype=torch.float32)
    nh, kvh, hd, inter = s.num_heads, s.num_kv_heads, s.head_dim, s.intermediate_size
    q_end, k_end = nh * hd, (nh + kvh) * hd
    sd = {"model.embed_tokens.weight": m.embed.float(), "lm_head.weight": m.lm_head.float(),
          "model.norm.weight": m.final_norm.float()}
    for i, p in enumerate(m.layers):
        pre = f"model.layers.{i}."
        qkv, b = _dense_t(p["qkv"], dev), p["qkv_bias"].float()
        gu = _dense_t(p["gate_up"], dev)
        sd.update({
            pre + "self_attn.q_proj.weight": qkv[:q_end], pre + "self_attn.q_proj.bias": b[:q_end],
            pre + "self_attn.k_proj.weight": qkv[q_end:k_end], pre + "self_attn.k_proj.bias": b[q_end:k_end],
            pre + "self_attn.v_proj.weight": qkv[k_end:], pre + "self_attn.v_proj.bias": b[k_end:],
            pre + "self_attn.o_proj.weight": _dense_t(p["o"], dev),
            pre + "mlp.gate_proj.weight": gu[:inter], pre + "mlp.up_proj.weight": gu[inter:],
            pre + "mlp.down_proj.weight": _dense_t(p["down"], dev),
            pre + "input_layernorm.weight": p["ln1"].float(), pre + "post_attention_layernorm.weight": p["ln2"].float(),
        })
        del qkv, gu
    missing, unexpected = hf.load_state_dict(sd, strict=False)
    assert not missing and not unexpected, (missing, unexpected)
    return hf.eval()


def _hf_last_logits(hf, ids, dev):
    with torch.no_grad():
        return hf(torch.tensor([ids], device=dev)).logits[0, -1].float()


def _close(y, y_ref, what):
    y, y_ref = y.double().cpu().numpy(), y_ref.double().cpu().numpy()
    err = O.max_rel_err(y, y_ref)
    print(f"{what}: max rel err {err:.2e}", flush=True)
    assert np.isfinite(y).all() and err <= 1e-2, f"{what}: max rel err {err:.3e}"


@pytest.mark.parametrize("shape,prompt_len,steps", [(TINY, 20, 6), (QWEN2_7B_2L, 16, 3)],
                         ids=["tiny", "qwen2_7b_width_2_layers"])
def test_logits_match_huggingface_qwen2(gpu, shape, prompt_len, steps):
    m = Qwen2AwqDecoder(shape, max_seq_len=64, seed=31, device=gpu)
    print(f"e2e vs HF: building the reference for hidden {shape.hidden_size}", flush=True)
    hf = _hf_model(m, gpu)
    prompt = torch.randint(0, shape.vocab_size, (prompt_len,), generator=torch.Generator().manual_seed(33))
    ids = prompt.tolist()
    _close(m.prefill(prompt), _hf_last_logits(hf, ids, gpu), f"hidden {shape.hidden_size} prefill")
    for step in range(steps):
        tok = int(torch.argmax(_hf_last_logits(hf, ids, gpu)))     # teacher forcing: the reference's token
        lg = m.decode_logits(torch.tensor(tok), len(ids))
        ids.append(tok)
        _close(lg, _hf_last_logits(hf, ids, gpu), f"hidden {shape.hidden_size} decode step {step}")
    del hf
    torch.cuda.empty_cache()


def test_qwen2_7b_full_graph_replay_equals_eager(gpu):
    """The end-to-end decode workload at its own size: the 28-layer Qwen2-7B
    shape, a 1024-token random prompt and 128 greedy tokens.  The
    graph-replayed greedy decoding equals the eager loop token for token, no
    step produced an out-of-vocabulary token (generate raises on the device
    flag), and every logit is finite."""
    prompt_len, new_tokens = 1024, 128
    m = Qwen2AwqDecoder(QWEN2_7B, max_seq_len=prompt_len + new_tokens, seed=41, device=gpu)
    prompt = torch.randint(0, QWEN2_7B.vocab_size, (prompt_len,), generator=torch.Generator().manual_seed(43))
    print(f"e2e qwen2-7b: graph generate, prompt {prompt_len}, {new_tokens} tokens", flush=True)
    r = m.generate(prompt, new_tokens)
    out = r["tokens"].tolist()
    print(f"e2e qwen2-7b: {r['decode_tokens_per_s']:.1f} tokens/s; eager loop", flush=True)
    assert len(out) == new_tokens and all(0 <= t < QWEN2_7B.vocab_size for t in out)
    m.k_cache.zero_()
    m.v_cache.zero_()
    lg = m.prefill(prompt)
    assert torch.isfinite(lg).all()
    toks = [int(torch.argmax(lg))]
    for i in range(new_tokens - 1):
        lg = m.decode_logits(torch.tensor(toks[-1]), prompt_len + i)
        assert torch.isfinite(lg).all(), f"step {i}"
        toks.append(int(torch.argmax(lg)))
    assert out == toks
    del m
    torch.cuda.empty_cache()
