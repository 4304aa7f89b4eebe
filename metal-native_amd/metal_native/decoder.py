"""Synthetic Qwen2.5-7B-shaped decoder whose every linear layer runs on the
quantized-linear kernels.

The reference's counterpart is its numpy MiniGPT example
(examples/llm_generation.py) and the prefill/decode split of PhasePipeline
(src/inference/phase_pipeline.mm:42-51); neither quantizes.  Here every
projection is an int4 g128 ``dequant_matmul``:

* q/k/v: one fused call over the concatenated weight rows, with the bias
  epilogue (Qwen2 attention projections carry biases);
* o_proj;
* gate/up: one fused call with the SwiGLU epilogue (gate rows, then up rows);
* down_proj and the lm_head.

Residual add + RMSNorm runs inside the following GEMV (the row-block
kernel's staging), rotary embedding + KV-cache write + single-token
grouped-query attention is one glue kernel (mq_glue.hip); the
embedding lookup and the greedy argmax are PyTorch ops on the same stream in
``step``; ``step_chain`` (the timed decode loop) replaces them with one fused
argmax + next-position + embedding-lookup kernel.
The decode step has static shapes (the position is a device tensor), so a
whole step is captured in a HIP graph and replayed token after token.
``reference_step`` restates the step in plain fp32 PyTorch for the tests.

Weights are random (no checkpoints are available): int4 nibbles U{0..15},
scales U(0.005, 0.02), integer zero-points U{0..15} mapped to the reference's
already-scaled zeros ``half((zp - 8) * s)``; embeddings, norms and biases
fp16 ~ N(0, 0.02).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import ops


@dataclass
class DecoderConfig:
    layers: int = 28
    d: int = 3584
    heads: int = 28
    kv_heads: int = 4
    head_dim: int = 128
    ffn: int = 18944
    vocab: int = 152064
    group_size: int = 128
    max_len: int = 512 + 64
    rope_theta: float = 1.0e6
    eps: float = 1e-6


def qwen25_7b(max_len: int = 512 + 64) -> DecoderConfig:
    return DecoderConfig(max_len=max_len)


class QLinear:
    """int4 g128 weights ``[N, K/2]`` + fp16 scales/zeros ``[N, K/g]``."""

    def __init__(self, wp: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, group_size: int,
                 bias: torch.Tensor | None = None):
        self.wp, self.scales, self.zeros, self.g, self.bias = wp, scales, zeros, group_size, bias

    @staticmethod
    def random(n: int, k: int, g: int, gen: torch.Generator, device, bias: bool = False) -> "QLinear":
        G = (k + g - 1) // g
        wp = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=device, generator=gen)
        s = (torch.rand((n, G), device=device, generator=gen) * 0.015 + 0.005).half()
        zp = torch.randint(0, 16, (n, G), device=device, generator=gen).float()
        z = ((zp - 8.0) * s.float()).half()
        b = (torch.randn(n, device=device, generator=gen) * 0.02).half() if bias else None
        return QLinear(wp, s, z, g, b)

    def operands(self):
        """(weights_packed, scales, zeros, group_size, quant_type) for the ops."""
        return self.wp, self.scales, self.zeros, self.g, "int4"

    def __call__(self, x: torch.Tensor, epilogue: str | None = None) -> torch.Tensor:
        if self.bias is not None and epilogue is None:
            return ops.dequant_matmul(x, self.wp, self.scales, self.zeros, self.g, "int4",
                                      epilogue="bias", bias=self.bias)
        return ops.dequant_matmul(x, self.wp, self.scales, self.zeros, self.g, "int4", epilogue=epilogue)


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float()).half()


def rope_tables(cfg: DecoderConfig, device) -> tuple[torch.Tensor, torch.Tensor]:
    half = cfg.head_dim // 2
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, half, device=device, dtype=torch.float32) / half))
    t = torch.arange(cfg.max_len, device=device, dtype=torch.float32)
    f = torch.outer(t, inv)
    emb = torch.cat([f, f], dim=-1)
    return emb.cos(), emb.sin()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [H, Dh] fp16, cos/sin [Dh] fp32 (rotate-half convention)."""
    xf = x.float()
    h = xf.shape[-1] // 2
    rot = torch.cat([-xf[..., h:], xf[..., :h]], dim=-1)
    return (xf * cos + rot * sin).half()


class SyntheticDecoder:
    def __init__(self, cfg: DecoderConfig, device, seed: int = 0, prefilled: int = 512):
        self.cfg = cfg
        self.device = torch.device(device)
        gen = torch.Generator(device=self.device)
        gen.manual_seed(seed)
        d, g = cfg.d, cfg.group_size
        nq, nkv = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
        rn = lambda *s: (torch.randn(*s, device=self.device, generator=gen) * 0.02).half()
        self.embed = rn(cfg.vocab, d)
        self.layers = []
        for _ in range(cfg.layers):
            self.layers.append({
                "ln1": rn(d), "ln2": rn(d),
                "qkv": QLinear.random(nq + 2 * nkv, d, g, gen, self.device, bias=True),
                "o": QLinear.random(d, nq, g, gen, self.device),
                "gate_up": QLinear.random(2 * cfg.ffn, d, g, gen, self.device),
                "down": QLinear.random(d, cfg.ffn, g, gen, self.device),
            })
        self.norm = rn(d)
        self.lm_head = QLinear.random(cfg.vocab, d, g, gen, self.device)
        self.cos, self.sin = rope_tables(cfg, self.device)
        # KV cache [layers, 2, kv_heads, max_len, head_dim]; the first `prefilled`
        # positions hold random keys/values (the benchmark's 512-token cache)
        self.kv = torch.zeros((cfg.layers, 2, cfg.kv_heads, cfg.max_len, cfg.head_dim),
                              dtype=torch.float16, device=self.device)
        if prefilled:
            self.kv[:, :, :, :prefilled] = (torch.randn((cfg.layers, 2, cfg.kv_heads, prefilled, cfg.head_dim),
                                                        device=self.device, generator=gen)).half()
        self.prefilled = prefilled
        self.positions = torch.arange(cfg.max_len, device=self.device)
        # two residual-stream buffers (the fused norm + GEMV writes out of place)
        self.resid = torch.zeros((2, 1, d), dtype=torch.float16, device=self.device)
        # greedy decode chain: the next step's embedding row and the tail workspace
        self.x0 = torch.zeros((1, d), dtype=torch.float16, device=self.device)
        self.tail_ws = ops.argmax_embed_workspace(cfg.vocab, self.device)

    # one decode step: token [1] int64, pos [1] int64 (device tensors) -> next token [1]
    def step(self, token: torch.Tensor, pos: torch.Tensor, return_logits: bool = False,
             x_in: torch.Tensor | None = None):
        """Five launches per layer: QKV with the residual add + RMSNorm fused
        into it (+bias), RoPE + cache write + attention (one kernel), o_proj,
        gate/up with the residual add + RMSNorm fused (+SwiGLU), down.  The
        residual stream alternates between two buffers (the fused kernel
        reads x and writes the new residual elsewhere)."""
        cfg = self.cfg
        H, KVH, Dh = cfg.heads, cfg.kv_heads, cfg.head_dim
        scale = 1.0 / math.sqrt(Dh)
        x = self.embed.index_select(0, token) if x_in is None else x_in   # [1, d] residual stream
        bufs = (self.resid[0], self.resid[1])
        cur = 0
        delta = None
        for li, L in enumerate(self.layers):
            qkv = ops.rmsnorm_dequant_matmul(x, delta, L["ln1"], cfg.eps, bufs[cur], *L["qkv"].operands(),
                                             epilogue="bias", bias=L["qkv"].bias)
            x = bufs[cur]
            cur ^= 1
            a = ops.attention_decode_rope(qkv, self.cos, self.sin, pos, self.kv[li, 0], self.kv[li, 1], H, KVH, Dh,
                                          scale)
            act = ops.rmsnorm_dequant_matmul(x, L["o"](a), L["ln2"], cfg.eps, bufs[cur], *L["gate_up"].operands(),
                                             epilogue="swiglu")
            x = bufs[cur]
            cur ^= 1
            delta = L["down"](act)
        logits = ops.rmsnorm_dequant_matmul(x, delta, self.norm, cfg.eps, bufs[cur], *self.lm_head.operands())
        if x_in is not None:
            return logits
        nxt = torch.argmax(logits.float(), dim=-1)
        return (nxt, logits) if return_logits else nxt

    def start_chain(self, token: torch.Tensor) -> None:
        """Stage the embedding row of ``token`` for ``step_chain``."""
        self.x0.copy_(self.embed.index_select(0, token))

    def step_chain(self, token: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """One greedy step fed by the staged row ``x0``; in place afterwards:
        ``token`` = the next token, ``pos`` + 1 and ``x0`` = its embedding row
        (one fused argmax + lookup kernel).  Returns the logits."""
        logits = self.step(token, pos, x_in=self.x0)
        ops.argmax_embed(logits, self.embed, token, pos, self.x0, self.tail_ws)
        return logits

    def reference_step(self, token: int, pos: int, dequant, probe=None) -> torch.Tensor:
        """The same step in fp32 torch with weights from ``dequant(qlinear) ->
        fp16 [N, K]`` (e.g. the CPU oracle); returns logits [vocab] (fp32).
        Rounds to fp16 where the kernel path does (projection outputs,
        residual stream, norms), so the two agree within the matmul tolerance.
        ``probe(name, layer, qlinear, x, y)``, when given, sees every linear's
        fp16 input and fp32 output (bias included) of the reference chain."""
        cfg = self.cfg
        H, KVH, Dh = cfg.heads, cfg.kv_heads, cfg.head_dim
        grp = H // KVH
        dev = self.device
        def lin(ql, x, name="", li=-1):
            y = x.float() @ dequant(ql).to(dev).float().t()
            if probe is not None:
                probe(name, li, ql, x, y + (ql.bias.float() if name == "qkv" else 0.0))
            return y

        x = self.embed[token:token + 1]
        cos, sin = self.cos[pos], self.sin[pos]
        scale = 1.0 / math.sqrt(Dh)
        kv = self.kv.clone()
        for li, L in enumerate(self.layers):
            h = rms_norm(x, L["ln1"], cfg.eps)
            qkv = (lin(L["qkv"], h, "qkv", li) + L["qkv"].bias.float()).half()[0]
            q = apply_rope(qkv[:H * Dh].view(H, Dh), cos, sin)
            k = apply_rope(qkv[H * Dh:(H + KVH) * Dh].view(KVH, Dh), cos, sin)
            v = qkv[(H + KVH) * Dh:].view(KVH, Dh)
            kv[li, 0, :, pos] = k
            kv[li, 1, :, pos] = v
            kc, vc = kv[li, 0, :, :pos + 1].float(), kv[li, 1, :, :pos + 1].float()
            s = torch.matmul(q.view(KVH, grp, Dh).float(), kc.transpose(1, 2)) * scale
            a = torch.matmul(torch.softmax(s, dim=-1), vc).half().reshape(1, H * Dh)
            x = x + lin(L["o"], a, "o", li).half()
            h = rms_norm(x, L["ln2"], cfg.eps)
            gu = lin(L["gate_up"], h, "gate_up", li).half().float()
            gate, up = gu[:, :cfg.ffn], gu[:, cfg.ffn:]
            act = (gate / (1.0 + torch.exp(-gate)) * up).half()
            x = x + lin(L["down"], act, "down", li).half()
        return lin(self.lm_head, rms_norm(x, self.norm, cfg.eps), "lm_head")[0]


def decode_tokens_per_second(model: SyntheticDecoder, n_tokens: int = 64, warmup: int = 3) -> dict:
    """Greedy-decode ``n_tokens`` tokens after the prefilled cache, each step a
    replay of one captured HIP graph; returns tokens/s and ms/token."""
    if model.prefilled + n_tokens > model.cfg.max_len:
        raise ValueError(f"decode_tokens_per_second: {model.prefilled} prefilled + {n_tokens} tokens exceed the "
                         f"KV cache of {model.cfg.max_len} positions")
    dev = model.device
    tok = torch.zeros(1, dtype=torch.int64, device=dev)
    pos = torch.full((1,), model.prefilled, dtype=torch.int64, device=dev)
    stream = torch.cuda.Stream(dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        for _ in range(warmup):  # eager warm-up: kernels loaded, workspaces allocated
            model.step(tok, pos)
        model.start_chain(tok)
        model.step_chain(tok, pos)   # eager warm-up of the chained step
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        model.step_chain(tok, pos)   # next token, position and embedding row updated in place
    pos.fill_(model.prefilled)
    graph.replay()  # one untimed replay
    pos.fill_(model.prefilled)
    torch.cuda.synchronize(dev)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(n_tokens):
        graph.replay()
    t1.record()
    torch.cuda.synchronize(dev)
    ms = t0.elapsed_time(t1)
    return {"tokens": n_tokens, "ms_per_token": ms / n_tokens, "tokens_per_s": n_tokens / (ms / 1000.0),
            "final_pos": int(pos.item())}
