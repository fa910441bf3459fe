"""End-to-end Qwen2-shaped greedy decoding on this build's kernels.

Mirrors the reference model and engine (``model/qwen2.py``, ``model/config.py``,
``inference/kv_cache.py``, ``inference/engine.py``) with random-init weights
(no checkpoint exists offline): every linear layer is an AWQ int4 projection
run by ``kernels.awq_gemm.awq_gemm_forward`` (fused QKV with the q/k/v biases,
``model/qwen2.py:79-85,104-113``; fused gate||up, ``:174-188``), the logits
come from the fp16 lm_head GEMV (``kernels.lm_head``, ``:253,280``), and the
non-GEMM work -- embedding, RMSNorm (``:15-22``), rotate-half RoPE
(``kernels/rope.py:41-57``), GQA attention over a static KV cache -- is
plain torch (attention in fp32 on contiguous operands).  The QKV bias and
the residual adds after o_proj and down_proj run in the GEMM's epilogue,
and SiLU * up reads the fused gate||up output in one kernel
(``kernels.silu_mul``).  Logits are computed for the last position only, where the
reference computes them for every position and keeps the last
(``inference/engine.py:93,127``).

One decode step is captured into a HIP graph once and replayed: the token
and position live in device buffers that the step itself advances, so
``generate`` issues one graph replay per token and no host synchronisation
(the reference captures a graph but never replays it, ``inference/engine.py:35-62``
vs ``:114-139``).
"""
from __future__ import annotations

import dataclasses
import math
import time

import torch

from kernels.awq_gemm import awq_gemm_forward, awq_gemm_forward_ex
from kernels.lm_head import lm_head_forward
from kernels.silu_mul import silu_mul_gate_up

__all__ = ["Qwen2Shape", "QWEN2_7B", "Qwen2AwqDecoder"]


@dataclasses.dataclass(frozen=True)
class Qwen2Shape:
    """The model dimensions (``model/config.py``)."""

    vocab_size: int = 152064
    hidden_size: int = 3584
    intermediate_size: int = 18944
    num_layers: int = 28
    num_heads: int = 28
    num_kv_heads: int = 4
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    group_size: int = 128

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads


QWEN2_7B = Qwen2Shape()


def _awq_tensors(k: int, n: int, gen: torch.Generator, dev: torch.device):
    """Random AWQ int4 operands: uniform codes and zeros, scales U[0.002, 0.02]."""
    qw = torch.randint(-2**31, 2**31 - 1, (k, n // 8), generator=gen, device=dev, dtype=torch.int32)
    qz = torch.randint(-2**31, 2**31 - 1, (k // 128, n // 8), generator=gen, device=dev, dtype=torch.int32)
    sc = (torch.rand((k // 128, n), generator=gen, device=dev) * 0.018 + 0.002).half()
    return qw, qz, sc


def _rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float()).half()


def _greedy_token(logits: torch.Tensor) -> torch.Tensor:
    """Index of the first largest logit, as an int64 [1] tensor, without a
    reduction that spans workgroups.  A whole-vector ``torch.argmax`` over a
    vocabulary-sized tensor is a multi-workgroup reduction whose captured
    graph holds a memset node, and such nodes have given wrong results on
    graph replays after the first (an out-of-range token follows).  Here each
    256-logit row is reduced on its own, then the row maxima (a few hundred
    values, one workgroup) -- the same first-maximum index as torch.argmax."""
    v = logits.reshape(-1)
    pad = (-v.numel()) % 256
    if pad:
        v = torch.nn.functional.pad(v, (0, pad), value=float("-inf"))
    vals, idx = v.view(-1, 256).max(dim=1)
    row = torch.argmax(vals).view(1)
    return row * 256 + idx.index_select(0, row)


def _checked_token(tok: torch.Tensor, vocab_size: int, bad: torch.Tensor) -> torch.Tensor:
    """``tok`` clamped into ``[0, vocab_size)``, counting out-of-range tokens
    in the device flag ``bad`` (int32 [1]).  The decode step feeds the token
    it generates straight into the embedding lookup of the next step, inside
    a replayed graph with no host check in between: an index past the table
    would make that lookup read outside it.  Clamped, the lookup stays in
    range, and ``generate`` raises from the flag after the replays.  Both
    operations are elementwise on one element: graph-safe, no host sync."""
    bad.add_(torch.logical_or(tok < 0, tok >= vocab_size).to(torch.int32))
    return tok.clamp(0, vocab_size - 1)


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


class Qwen2AwqDecoder:
    """Random-init Qwen2-shaped model; ``layers`` dicts hold the packed operands."""

    def __init__(self, shape: Qwen2Shape = QWEN2_7B, max_seq_len: int = 2048, seed: int = 0,
                 device: torch.device | str = "cuda:0", weights: dict | None = None):
        """Random-init weights (seeded), or `weights` as produced by
        ``engine.awq_checkpoint.load_qwen2_awq`` (embed, lm_head, final_norm,
        layers: list of dicts with ln1, ln2, qkv, qkv_bias, o, gate_up, down;
        the AWQ entries are (qweight, qzeros, scales) tuples)."""
        self.s = shape
        self.dev = torch.device(device)
        self.max_seq_len = max_seq_len
        H, I = shape.hidden_size, shape.intermediate_size
        qkv_n = (shape.num_heads + 2 * shape.num_kv_heads) * shape.head_dim
        if weights is not None:
            mv = lambda t: t.to(self.dev)  # noqa: E731
            self.embed = mv(weights["embed"])
            self.lm_head = mv(weights["lm_head"])
            self.final_norm = mv(weights["final_norm"])
            self.layers = [{k: (tuple(mv(t) for t in v) if isinstance(v, tuple) else mv(v)) for k, v in lw.items()}
                           for lw in weights["layers"]]
        else:
            g = torch.Generator(device=self.dev)
            g.manual_seed(seed)
            self.embed = (torch.randn((shape.vocab_size, H), generator=g, device=self.dev) * 0.02).half()
            self.lm_head = (torch.randn((shape.vocab_size, H), generator=g, device=self.dev) * 0.02).half()
            self.final_norm = torch.ones(H, dtype=torch.float16, device=self.dev)
            self.layers = []
            for _ in range(shape.num_layers):
                self.layers.append({
                    "ln1": (1.0 + 0.1 * torch.randn(H, generator=g, device=self.dev)).half(),
                    "ln2": (1.0 + 0.1 * torch.randn(H, generator=g, device=self.dev)).half(),
                    "qkv": _awq_tensors(H, qkv_n, g, self.dev),
                    "qkv_bias": (torch.randn(qkv_n, generator=g, device=self.dev) * 0.02).half(),
                    "o": _awq_tensors(H, H, g, self.dev),
                    "gate_up": _awq_tensors(H, 2 * I, g, self.dev),
                    "down": _awq_tensors(I, H, g, self.dev),
                })
        if len(self.layers) != shape.num_layers:
            raise ValueError(f"{len(self.layers)} layers of weights for a {shape.num_layers}-layer shape")
        hd = shape.head_dim
        inv = 1.0 / (shape.rope_theta ** (torch.arange(0, hd, 2, device=self.dev, dtype=torch.float32) / hd))
        t = torch.arange(max_seq_len, device=self.dev, dtype=torch.float32)
        f = torch.outer(t, inv)
        self.cos = torch.cat((f, f), dim=-1).cos()   # [max_seq_len, head_dim]
        self.sin = torch.cat((f, f), dim=-1).sin()
        L, KV = shape.num_layers, shape.num_kv_heads
        self.k_cache = torch.zeros((L, KV, max_seq_len, hd), dtype=torch.float16, device=self.dev)
        self.v_cache = torch.zeros_like(self.k_cache)
        self._graph = None

    # ---- linear layers: the path this build replaces -------------------------
    def linear(self, x: torch.Tensor, op, bias: torch.Tensor | None = None,
               residual: torch.Tensor | None = None) -> torch.Tensor:
        """AWQ projection; ``bias`` and ``residual`` are added in the GEMM's
        epilogue, rounded as torch's fp16 ``residual + (x @ W + bias)``."""
        if bias is None and residual is None:
            return awq_gemm_forward(x, *op)
        return awq_gemm_forward_ex(x, *op, bias=bias, residual=residual)

    # ---- one decoder layer over positions `pos` (device int64 [S]) -------------
    def _layer(self, li: int, h: torch.Tensor, pos: torch.Tensor, causal: bool) -> torch.Tensor:
        s = self.s
        p = self.layers[li]
        S = h.shape[0]
        nh, kvh, hd = s.num_heads, s.num_kv_heads, s.head_dim
        x = _rmsnorm(h, p["ln1"], s.rms_norm_eps)
        qkv = self.linear(x, p["qkv"], bias=p["qkv_bias"])
        q = qkv[:, :nh * hd].view(S, nh, hd).float()
        k = qkv[:, nh * hd:(nh + kvh) * hd].view(S, kvh, hd).float()
        v = qkv[:, (nh + kvh) * hd:].view(S, kvh, hd)
        cos = self.cos.index_select(0, pos).unsqueeze(1)
        sin = self.sin.index_select(0, pos).unsqueeze(1)
        q = q * cos + _rotate_half(q) * sin
        k = k * cos + _rotate_half(k) * sin
        self.k_cache[li].index_copy_(1, pos, k.half().transpose(0, 1))
        self.v_cache[li].index_copy_(1, pos, v.transpose(0, 1))
        groups = nh // kvh
        if causal:
            # prefill from position 0: the S new keys are the whole cache prefix
            T = S
            kk = self.k_cache[li, :, :T].float()
            vv = self.v_cache[li, :, :T].float()
            mask = torch.ones((S, T), dtype=torch.bool, device=self.dev).triu(1)
        else:
            T = self.max_seq_len
            kk = self.k_cache[li].float()
            vv = self.v_cache[li].float()
            mask = (torch.arange(T, device=self.dev).unsqueeze(0) > pos.unsqueeze(1))   # [S, T]
        qg = q.transpose(0, 1).reshape(kvh, groups * S, hd)                   # heads of one kv group together
        scores = torch.matmul(qg, kk.transpose(1, 2).contiguous()) / math.sqrt(hd)   # [kvh, groups*S, T]
        scores = scores.view(kvh, groups, S, T).masked_fill(mask, float("-inf"))
        probs = torch.softmax(scores, dim=-1).view(kvh, groups * S, T)
        att = torch.matmul(probs, vv.contiguous()).view(nh, S, hd)            # [nh, S, hd]
        att = att.transpose(0, 1).reshape(S, nh * hd).half()
        h = self.linear(att, p["o"], residual=h)
        x = _rmsnorm(h, p["ln2"], s.rms_norm_eps)
        inter = silu_mul_gate_up(self.linear(x, p["gate_up"]))
        return self.linear(inter, p["down"], residual=h)

    def _forward(self, ids: torch.Tensor, pos: torch.Tensor, causal: bool) -> torch.Tensor:
        h = torch.nn.functional.embedding(ids, self.embed)
        for li in range(self.s.num_layers):
            h = self._layer(li, h, pos, causal)
        last = _rmsnorm(h[-1:], self.final_norm, self.s.rms_norm_eps)
        return lm_head_forward(last, self.lm_head)[0]          # logits of the last position [vocab]

    # ---- public API ------------------------------------------------------------
    @torch.no_grad()
    def prefill(self, prompt: torch.Tensor) -> torch.Tensor:
        """Process prompt ids [S] from position 0; returns the last position's logits."""
        S = prompt.shape[0]
        if S > self.max_seq_len:
            raise ValueError(f"prompt of {S} tokens exceeds max_seq_len {self.max_seq_len}")
        pos = torch.arange(S, device=self.dev)
        return self._forward(prompt.to(self.dev), pos, causal=True)

    @torch.no_grad()
    def decode_logits(self, token: torch.Tensor, pos: int) -> torch.Tensor:
        """One eager decode step: logits after feeding `token` at position `pos`."""
        return self._forward(token.view(1).to(self.dev), torch.tensor([pos], device=self.dev), causal=False)

    @torch.no_grad()
    def _capture(self):
        self._tok = torch.zeros(1, dtype=torch.int64, device=self.dev)
        self._pos = torch.zeros(1, dtype=torch.int64, device=self.dev)
        self._out = torch.zeros(self.max_seq_len, dtype=torch.int64, device=self.dev)
        self._bad = torch.zeros(1, dtype=torch.int32, device=self.dev)

        def step():
            logits = self._forward(self._tok, self._pos, causal=False)
            nxt = _checked_token(_greedy_token(logits), self.s.vocab_size, self._bad)
            self._out.index_copy_(0, self._pos, nxt)       # out[p] = token generated at position p + 1
            self._tok.copy_(nxt)
            self._pos.add_(1)

        # warm-up outside the capture (workspace sizing, library loading), then undo its effects
        self._tok.zero_()
        self._pos.fill_(self.max_seq_len - 1)
        step()
        torch.cuda.synchronize(self.dev)
        side = torch.cuda.Stream(self.dev)
        side.wait_stream(torch.cuda.current_stream(self.dev))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            step()
        torch.cuda.current_stream(self.dev).wait_stream(side)
        self._graph = g

    @torch.no_grad()
    def generate(self, prompt: torch.Tensor, new_tokens: int) -> dict:
        """Greedy decoding: prefill the prompt, then `new_tokens` graph-replayed
        decode steps.  Returns the tokens and the timings."""
        S = prompt.shape[0]
        if S + new_tokens > self.max_seq_len:
            raise ValueError("prompt + new tokens exceed max_seq_len")
        if self._graph is None:
            self._capture()
        self.k_cache.zero_()
        self.v_cache.zero_()
        self._bad.zero_()
        torch.cuda.synchronize(self.dev)
        t0 = time.perf_counter()
        logits = self.prefill(prompt)
        first = torch.argmax(logits).view(1)
        self._tok.copy_(first)
        self._pos.fill_(S)
        torch.cuda.synchronize(self.dev)
        t1 = time.perf_counter()
        for _ in range(new_tokens - 1):
            self._graph.replay()
        torch.cuda.synchronize(self.dev)
        t2 = time.perf_counter()
        if int(self._bad.item()) != 0:
            raise RuntimeError(f"{int(self._bad.item())} decode step(s) produced a token outside the vocabulary "
                               f"[0, {self.s.vocab_size}); the lookups were clamped, the tokens are not valid")
        tokens = torch.cat([first, self._out[S:S + new_tokens - 1]]).cpu()
        decode_s = t2 - t1
        return {"tokens": tokens, "prefill_s": t1 - t0, "decode_s": decode_s,
                "decode_tokens_per_s": (new_tokens - 1) / decode_s if decode_s > 0 else float("inf")}
