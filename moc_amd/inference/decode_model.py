"""End-to-end single-token decode of a LLaMA-style decoder whose FFNs are
InferenceMoCSwiGLUFFN (the model and method of the reference's
benchmarks/inference/benchmark_decode.py:101-420,461-617).

Rows (benchmark_decode.py:46-76): "dense" (dense_baseline), "global_moc"
(gate GEMV -> Top-K -> selected Up/Down, K = 1024) and "moc_2_8" (fused
gate/up + top-2-of-8 -> selected Down).  A step embeds one token, runs every
layer (x + attn(norm(x)), x + ffn(norm(x))) against a static KV cache and
returns the logits; the token is the argmax of the logits, outside the step.

Scopes: "eager" (every kernel launched from Python), "layer_graph" (each
decoder layer captured in its own HIP graph over persistent activation
buffers, replayed layer by layer; embedding and LM head eager: the per-layer
graph runners of benchmark_decode.py:461-499) and "whole_graph" (the whole
step captured once in a HIP graph over persistent token/position buffers and
replayed per token: benchmark_decode.py:549-617).  The reference's
torch.compile scope (:423-459) is not offered: Inductor would generate
Triton kernels for the host's attention, which this build does not use.

Attention, RMSNorm, RoPE, the embedding and the LM head are stock PyTorch
(the host of the FFN).  Attention keeps K transposed in its cache
([1, heads, head_dim, max_seq]) and V as [1, heads, max_seq, head_dim], so
both attention products are batched products of contiguous operands; the
softmax runs in f32.
"""
from __future__ import annotations

import math
import statistics
from dataclasses import dataclass
from typing import Callable

import torch
import torch.nn as nn

from .inference_ffn import InferenceMoCSwiGLUFFN

HIDDEN = 2048
INTERMEDIATE = 5464
NUM_HEADS = 16
NUM_LAYERS = 24
PROMPT_LEN = 128
GEN_LEN = 128
VOCAB_SIZE = 32000
GLOBAL_K = 1024

# row -> FFN mode (benchmark_decode.py:46-76)
ROWS = {
    "dense": "dense_baseline",
    "global_moc": "moc_inference_optimized_global_after_gate_native",
    "moc_2_8": "moc_inference_grouped_top2of8",
}


@dataclass(frozen=True)
class DecodeConfig:
    hidden: int = HIDDEN
    intermediate: int = INTERMEDIATE
    heads: int = NUM_HEADS
    layers: int = NUM_LAYERS
    vocab: int = VOCAB_SIZE
    k: int = GLOBAL_K            # global MoC; MoC 2:8 keeps intermediate / 4
    max_seq: int = PROMPT_LEN + GEN_LEN


class RMSNorm(nn.Module):
    """x / rms(x) in f32, cast back, times the weight (benchmark_decode.py:101-109)."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)).to(x.dtype) * self.weight


def rope_tables(head_dim: int, max_len: int, theta: float = 10000.0):
    """cos, sin [max_len, head_dim / 2] of the position angles p * theta^(-2i/d)."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    ang = torch.outer(torch.arange(max_len, dtype=torch.float32), inv)
    return ang.cos(), ang.sin()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate the pairs (x[2i], x[2i+1]) of the last dim by the angles in
    cos/sin (broadcast over the leading dims; benchmark_decode.py:119-125)."""
    a, b = x[..., 0::2], x[..., 1::2]
    return torch.stack((a * cos - b * sin, a * sin + b * cos), dim=-1).flatten(-2)


class StaticKVAttention(nn.Module):
    def __init__(self, hidden: int, heads: int, max_seq: int):
        super().__init__()
        self.hidden, self.heads, self.head_dim, self.max_seq = hidden, heads, hidden // heads, max_seq
        self.qkv_proj = nn.Linear(hidden, 3 * hidden, bias=False)
        self.out_proj = nn.Linear(hidden, hidden, bias=False)
        cos, sin = rope_tables(self.head_dim, max_seq)
        self.register_buffer("rope_cos", cos, persistent=False)
        self.register_buffer("rope_sin", sin, persistent=False)
        self.register_buffer("mask", torch.full((max_seq, max_seq), float("-inf")).triu(1),
                             persistent=False)
        self.k_t: torch.Tensor | None = None  # [1, heads, head_dim, max_seq]
        self.v: torch.Tensor | None = None    # [1, heads, max_seq, head_dim]

    def allocate_cache(self) -> None:
        w = self.qkv_proj.weight
        self.k_t = torch.zeros(1, self.heads, self.head_dim, self.max_seq, device=w.device, dtype=w.dtype)
        self.v = torch.zeros(1, self.heads, self.max_seq, self.head_dim, device=w.device, dtype=w.dtype)

    def reset_cache(self) -> None:
        self.k_t.zero_()
        self.v.zero_()

    def _qkv(self, x: torch.Tensor):
        b, n, _ = x.shape
        qkv = self.qkv_proj(x).view(b, n, 3, self.heads, self.head_dim)
        return [t.transpose(1, 2) for t in qkv.unbind(2)]  # [b, heads, n, head_dim] each

    def _attend(self, q: torch.Tensor, k_t: torch.Tensor, v: torch.Tensor, mask: torch.Tensor):
        s = torch.matmul(q.contiguous(), k_t).float() * (1.0 / math.sqrt(self.head_dim)) + mask
        p = torch.softmax(s, dim=-1).to(v.dtype)
        return torch.matmul(p, v)

    def forward_prompt(self, x: torch.Tensor) -> torch.Tensor:
        b, n, h = x.shape
        q, k, v = self._qkv(x)
        cos, sin = self.rope_cos[:n].to(x.dtype), self.rope_sin[:n].to(x.dtype)
        q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
        self.k_t[:, :, :, :n].copy_(k.transpose(-1, -2))
        self.v[:, :, :n].copy_(v)
        y = self._attend(q, self.k_t[:, :, :, :n].contiguous(), self.v[:, :, :n].contiguous(),
                         self.mask[:n, :n])
        return self.out_proj(y.transpose(1, 2).reshape(b, n, h))

    def forward_step(self, x: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """One token at position `pos` (a 0-dim int64 tensor, so the step can
        be captured once and replayed for every position)."""
        b, _, h = x.shape
        q, k, v = self._qkv(x)
        p1 = pos.view(1)
        cos = self.rope_cos.index_select(0, p1).to(x.dtype)
        sin = self.rope_sin.index_select(0, p1).to(x.dtype)
        q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
        self.k_t.index_copy_(3, p1, k.transpose(-1, -2))
        self.v.index_copy_(2, p1, v)
        y = self._attend(q, self.k_t, self.v, self.mask.index_select(0, p1))
        return self.out_proj(y.transpose(1, 2).reshape(b, 1, h))


class DecoderLayer(nn.Module):
    def __init__(self, row: str, cfg: DecodeConfig, fuse: bool = True):
        super().__init__()
        self.mode = ROWS[row]
        # MoC decode: ffn_norm and the residual add run inside the FFN's two
        # kernels (InferenceMoCSwiGLUFFN.fused_decode_residual)
        self.fuse = fuse and row in ("global_moc", "moc_2_8")
        grouped = row == "moc_2_8"
        k = cfg.intermediate * 2 // 8 if grouped else cfg.k
        self.attn_norm = RMSNorm(cfg.hidden)
        self.attn = StaticKVAttention(cfg.hidden, cfg.heads, cfg.max_seq)
        self.ffn_norm = RMSNorm(cfg.hidden)
        self.ffn = InferenceMoCSwiGLUFFN(cfg.hidden, cfg.intermediate, k,
                                         grouped_a=2 if grouped else None,
                                         grouped_b=8 if grouped else None)

    def _ffn(self, x: torch.Tensor) -> torch.Tensor:
        b, n, h = x.shape
        return self.ffn(x.reshape(b * n, h), mode=self.mode).reshape(b, n, h)

    def forward_prompt(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.attn.forward_prompt(self.attn_norm(x))
        return x + self._ffn(self.ffn_norm(x))

    def forward_step(self, x: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        x = x + self.attn.forward_step(self.attn_norm(x), pos)
        if self.fuse and x.is_cuda:
            b, n, h = x.shape
            return self.ffn.fused_decode_residual(x.reshape(b * n, h), self.ffn_norm.weight,
                                                  self.ffn_norm.eps).reshape(b, n, h)
        return x + self._ffn(self.ffn_norm(x))


class DecoderModel(nn.Module):
    def __init__(self, row: str, cfg: DecodeConfig = DecodeConfig(), fuse: bool = True):
        super().__init__()
        if row not in ROWS:
            raise ValueError(f"unknown decode row {row!r}; expected one of {sorted(ROWS)}")
        self.row, self.cfg = row, cfg
        self.embed = nn.Embedding(cfg.vocab, cfg.hidden)
        self.layers = nn.ModuleList(DecoderLayer(row, cfg, fuse) for _ in range(cfg.layers))
        self.final_norm = RMSNorm(cfg.hidden)
        self.lm_head = nn.Linear(cfg.hidden, cfg.vocab, bias=False)

    def init_weights(self, seed: int = 1234, std: float = 0.02) -> "DecoderModel":
        """Seeded N(0, std) weights for every linear and the embedding."""
        gen = torch.Generator(device=self.embed.weight.device).manual_seed(seed)
        with torch.no_grad():
            for m in self.modules():
                if isinstance(m, (nn.Linear, nn.Embedding)):
                    w = torch.randn(m.weight.shape, generator=gen, device=m.weight.device) * std
                    m.weight.copy_(w.to(m.weight.dtype))
        return self

    def allocate_cache(self) -> None:
        for layer in self.layers:
            layer.attn.allocate_cache()

    def reset_cache(self) -> None:
        for layer in self.layers:
            layer.attn.reset_cache()

    def freeze_for_compile(self) -> None:
        for layer in self.layers:
            layer.ffn.freeze_for_compile()

    @torch.no_grad()
    def forward_prompt(self, tokens: torch.Tensor) -> torch.Tensor:
        x = self.embed(tokens)
        for layer in self.layers:
            x = layer.forward_prompt(x)
        return self.lm_head(self.final_norm(x))

    @torch.no_grad()
    def forward_step(self, tokens: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        x = self.embed(tokens)
        for layer in self.layers:
            x = layer.forward_step(x, pos)
        return self.lm_head(self.final_norm(x))


def make_step(model: DecoderModel, scope: str) -> Callable[[torch.Tensor, int], torch.Tensor]:
    """A callable (token ids [1, 1], position) -> logits [1, 1, vocab].
    "whole_graph" captures one step (after warm-up launches on a side
    stream) over persistent token/position buffers."""
    dev = model.embed.weight.device
    pos = torch.zeros((), dtype=torch.int64, device=dev)
    if scope == "eager":
        def step(tokens: torch.Tensor, p: int) -> torch.Tensor:
            pos.fill_(p)
            return model.forward_step(tokens, pos)
        return step
    if scope == "layer_graph":
        return _layer_graph_step(model, pos)
    if scope != "whole_graph":
        raise ValueError(f"unknown scope {scope!r}")
    model.freeze_for_compile()
    tok = torch.zeros(1, 1, dtype=torch.int64, device=dev)
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for _ in range(3):
            model.forward_step(tok, pos)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        logits = model.forward_step(tok, pos)

    def step(tokens: torch.Tensor, p: int) -> torch.Tensor:
        tok.copy_(tokens)
        pos.fill_(p)
        graph.replay()
        return logits

    step.graph = graph
    return step


def _layer_graph_step(model: DecoderModel, pos: torch.Tensor) -> Callable[[torch.Tensor, int], torch.Tensor]:
    """One HIP graph per decoder layer: layer i reads xs[i] and writes
    xs[i + 1]; the graphs share one memory pool and replay in order."""
    dev = model.embed.weight.device
    model.freeze_for_compile()
    h = model.cfg.hidden
    xs = [torch.zeros(1, 1, h, dtype=model.embed.weight.dtype, device=dev)
          for _ in range(len(model.layers) + 1)]

    def run_layer(i, layer):
        xs[i + 1].copy_(layer.forward_step(xs[i], pos))

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side), torch.no_grad():
        for _ in range(3):
            for i, layer in enumerate(model.layers):
                run_layer(i, layer)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    pool = torch.cuda.graph_pool_handle()
    graphs = []
    with torch.no_grad():
        for i, layer in enumerate(model.layers):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                run_layer(i, layer)
            graphs.append(g)

    @torch.no_grad()
    def step(tokens: torch.Tensor, p: int) -> torch.Tensor:
        pos.fill_(p)
        xs[0].copy_(model.embed(tokens))
        for g in graphs:
            g.replay()
        return model.lm_head(model.final_norm(xs[-1]))

    step.graphs = graphs
    return step


@torch.no_grad()
def run_decode(model: DecoderModel, prompt: torch.Tensor, gen_len: int,
               step: Callable[[torch.Tensor, int], torch.Tensor]) -> tuple[float, torch.Tensor]:
    """Prompt forward, then gen_len greedy steps timed between HIP events
    (benchmark_decode.py:366-385); returns (ms, generated token ids)."""
    model.reset_cache()
    cur = model.forward_prompt(prompt)[:, -1:, :].argmax(dim=-1)
    torch.cuda.synchronize()
    out = torch.empty(1, gen_len, dtype=torch.int64, device=prompt.device)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = prompt.shape[1]
    a.record()
    for i in range(gen_len):
        cur = step(cur, n + i).argmax(dim=-1)
        out[:, i:i + 1].copy_(cur)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b), out


def measure_decode(row: str, *, num_layers: int = NUM_LAYERS, prompt_len: int = PROMPT_LEN,
                   gen_len: int = GEN_LEN, scope: str = "whole_graph", warmup: int = 1,
                   runs: int = 3, seed: int = 1234, device: str = "cuda", fuse: bool = True) -> dict:
    """ms/token of greedy decode for one row (benchmark_decode.py:397-420),
    on a seeded random model and a seeded random prompt (no dataset here)."""
    cfg = DecodeConfig(layers=num_layers, max_seq=prompt_len + gen_len)
    model = DecoderModel(row, cfg, fuse).to(device, torch.bfloat16)
    model.init_weights(seed)
    model.allocate_cache()
    gen = torch.Generator(device=device).manual_seed(seed + 1)
    prompt = torch.randint(0, cfg.vocab, (1, prompt_len), generator=gen, device=device)
    step = make_step(model, scope)
    for _ in range(warmup):
        run_decode(model, prompt, gen_len, step)
    samples = [run_decode(model, prompt, gen_len, step)[0] for _ in range(runs)]
    med = statistics.median(samples)
    return {"row": row, "scope": scope, "fused_ffn_norm_residual": model.layers[0].fuse,
            "layers": num_layers, "prompt_len": prompt_len,
            "gen_len": gen_len, "ms_per_token": round(med / gen_len, 4),
            "tokens_per_s": round(gen_len / (med * 1e-3), 1),
            "total_ms": [round(s, 3) for s in samples]}
