"""Qwen-style decoder for the end-to-end run with ChronoQuant caches.

The reference's end-to-end scripts drive an mlx_lm Qwen model whose
attention modules call mlx_lm's `scaled_dot_product_attention` with the
layer's cache; patch.apply() rebinds that symbol so ChronoQuant caches take
the fused path (patch.py:18-33), and create_full_throttle_caches() fills the
cache slots (patch.py:91-104).  This module is that model on PyTorch-ROCm:
Qwen3-style blocks (RMSNorm, q/k RMSNorm per head, RoPE on half-split
dims, SwiGLU MLP, untied LM head) whose attention calls this module's
`scaled_dot_product_attention`, the binding apply() replaces.  Keys are
cached after RoPE, as in mlx_lm.

Dense projections are torch matmuls (hipBLASLt), with the q/k/v and the
gate/up projections each fused into one matrix (rows: query heads, key
heads, value heads; gate, up); with FUSED_OPS a single input row (a decode
step) takes the library's GEMV, which streams each weight once.  The attention and the KV cache are the
library's, and so are the elementwise ops when FUSED_OPS is set (the
default): residual add + RMSNorm, the QKV split with q/k RMSNorm and RoPE,
and the SwiGLU gate (models/fused.py).  FUSED_OPS = False runs the same
math as torch ops, the reference the fused ops are tested against.
Weights are random N(0, 0.02) (no checkpoint is available offline).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from .. import patch as _patch
from ..cache import ChronoQuantCache
from ..host import scaled_dot_product_attention  # rebound by patch.apply()
from . import fused

FUSED_OPS = True  # library kernels for the elementwise ops (False: torch ops)


@dataclass
class ModelArgs:
    hidden_size: int = 4096
    num_hidden_layers: int = 32
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 12288
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    vocab_size: int = 151936
    max_position: int = 40960


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x):
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (y * self.weight.float()).to(x.dtype)


class Rope(nn.Module):
    """Rotary embedding on half-split dims (non-interleaved), base theta."""

    def __init__(self, dim: int, theta: float, max_position: int):
        super().__init__()
        inv = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim))
        ang = torch.arange(max_position, dtype=torch.float64)[:, None] * inv[None, :]
        self.register_buffer("cos", torch.cos(ang).float(), persistent=False)
        self.register_buffer("sin", torch.sin(ang).float(), persistent=False)

    def forward(self, x, positions):
        """x [B, H, L, D]; positions [L] (int64) or [B, L] on x's device."""
        cos, sin = self.cos[positions], self.sin[positions]
        if cos.dim() == 2:
            cos, sin = cos[None, None], sin[None, None]
        else:
            cos, sin = cos[:, None], sin[:, None]
        xf = x.float()
        h = x.shape[-1] // 2
        x1, x2 = xf[..., :h], xf[..., h:]
        return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1).to(x.dtype)


class Attention(nn.Module):
    def __init__(self, a: ModelArgs, rope: Rope):
        super().__init__()
        self.nh, self.nkv, self.hd = a.num_attention_heads, a.num_key_value_heads, a.head_dim
        self.scale = a.head_dim ** -0.5
        self.qkv_proj = nn.Linear(a.hidden_size, (self.nh + 2 * self.nkv) * self.hd, bias=False)
        self.o_proj = nn.Linear(self.nh * self.hd, a.hidden_size, bias=False)
        self.q_norm = RMSNorm(self.hd, a.rms_norm_eps)
        self.k_norm = RMSNorm(self.hd, a.rms_norm_eps)
        self.rope = rope

    def _qkv_torch(self, qkv, positions):
        B, L, _ = qkv.shape
        nq, nk = self.nh * self.hd, self.nkv * self.hd
        q = self.q_norm(qkv[..., :nq].view(B, L, self.nh, self.hd)).transpose(1, 2)
        k = self.k_norm(qkv[..., nq:nq + nk].reshape(B, L, self.nkv, self.hd)).transpose(1, 2)
        v = qkv[..., nq + nk:].reshape(B, L, self.nkv, self.hd).transpose(1, 2)
        return self.rope(q, positions), self.rope(k, positions), v

    def forward(self, x, positions, mask, cache, qkv=None):
        """qkv: the fused QKV projection of x when the caller computed it
        (then x is unused)."""
        if qkv is None:
            qkv = fused.linear(x, self.qkv_proj.weight) if FUSED_OPS else self.qkv_proj(x)
        B, L, _ = qkv.shape
        q = None
        if FUSED_OPS and L == 1 and isinstance(cache, ChronoQuantCache) and _patch._patched:
            # a decode token: norm, RoPE and the cache append in one launch
            # (the patched SDPA reads the cache, not the keys / values)
            q = cache.fused_decode_append(qkv, self.nh, self.q_norm.weight, self.k_norm.weight,
                                          self.rope.cos, self.rope.sin, positions,
                                          self.q_norm.eps)
            keys = values = None
        if q is None:
            if FUSED_OPS:
                q, k, v = fused.qkv_norm_rope(qkv, self.nh, self.nkv, self.q_norm.weight,
                                              self.k_norm.weight, self.rope.cos, self.rope.sin,
                                              positions, self.q_norm.eps)
            else:
                q, k, v = self._qkv_torch(qkv, positions)
            keys, values = cache.update_and_fetch(k, v)
        out = scaled_dot_product_attention(q, keys, values, cache=cache, scale=self.scale,
                                           mask=mask)
        out = out.transpose(1, 2).reshape(B, L, self.nh * self.hd)
        return fused.linear(out, self.o_proj.weight) if FUSED_OPS else self.o_proj(out)


class MLP(nn.Module):
    def __init__(self, a: ModelArgs):
        super().__init__()
        self.inter = a.intermediate_size
        self.gate_up_proj = nn.Linear(a.hidden_size, 2 * a.intermediate_size, bias=False)
        self.down_proj = nn.Linear(a.intermediate_size, a.hidden_size, bias=False)

    def forward(self, x):
        if FUSED_OPS:
            gu = fused.linear(x, self.gate_up_proj.weight)
            return fused.linear(fused.silu_mul(gu), self.down_proj.weight)
        gu = self.gate_up_proj(x)
        return self.down_proj(F.silu(gu[..., :self.inter]) * gu[..., self.inter:])


class Block(nn.Module):
    def __init__(self, a: ModelArgs, rope: Rope):
        super().__init__()
        self.self_attn = Attention(a, rope)
        self.mlp = MLP(a)
        self.input_layernorm = RMSNorm(a.hidden_size, a.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(a.hidden_size, a.rms_norm_eps)

    def forward(self, x, positions, mask, cache):
        h = x + self.self_attn(self.input_layernorm(x), positions, mask, cache)
        return h + self.mlp(self.post_attention_layernorm(h))


class Model(nn.Module):
    def __init__(self, a: ModelArgs):
        super().__init__()
        self.args = a
        self.rope = Rope(a.head_dim, a.rope_theta, a.max_position)
        self.embed_tokens = nn.Embedding(a.vocab_size, a.hidden_size)
        self.layers = nn.ModuleList([Block(a, self.rope) for _ in range(a.num_hidden_layers)])
        self.norm = RMSNorm(a.hidden_size, a.rms_norm_eps)
        self.lm_head = nn.Linear(a.hidden_size, a.vocab_size, bias=False)

    def forward(self, tokens, cache, positions=None, last_only: bool = False):
        """tokens [B, L]; positions [L] (default: the caches' offset onward)
        or [B, L] device tensor (graph-captured decode).  last_only: logits of
        the last position only."""
        B, L = tokens.shape
        if positions is None:
            off = cache[0].offset
            positions = torch.arange(off, off + L, device=tokens.device)
        mask = "causal" if L > 1 else None
        x = self.embed_tokens(tokens)
        if FUSED_OPS and B * L == 1:
            return self._forward_one(x, positions, cache)
        if not FUSED_OPS:
            for layer, c in zip(self.layers, cache):
                x = layer(x, positions, mask, c)
            if last_only:
                x = x[:, -1:]
            return self.lm_head(self.norm(x))
        # fused: each residual add is folded into the RMSNorm that follows it
        eps = self.norm.eps
        y = fused.rms_norm(x, self.layers[0].input_layernorm.weight, eps)
        n = len(self.layers)
        for i, (layer, c) in enumerate(zip(self.layers, cache)):
            a = layer.self_attn(y, positions, mask, c)
            h, y = fused.add_rms_norm(a, x, layer.post_attention_layernorm.weight, eps)
            m = layer.mlp(y)
            w_next = self.layers[i + 1].input_layernorm.weight if i + 1 < n else self.norm.weight
            if last_only and i + 1 == n:
                m, h = m[:, -1:], h[:, -1:]
            x, y = fused.add_rms_norm(m, h, w_next, eps)
        return fused.linear(y, self.lm_head.weight)

    def _forward_one(self, x, positions, cache):
        """One token (a decode step) with the fused ops: every RMSNorm and
        residual add runs inside the projection that consumes it
        (fused.linear_rms_norm) and the SwiGLU gate inside the down projection
        (fused.linear_silu).  The residual stream: x_i (layer input), h_i =
        x_i + attn_i, x_{i+1} = h_i + mlp_i."""
        eps = self.norm.eps
        inp, res = x, None  # x_i = inp + res (res None: x_i = inp)
        for layer, c in zip(self.layers, cache):
            attn, mlp = layer.self_attn, layer.mlp
            qkv, xi = fused.linear_rms_norm(inp, res, layer.input_layernorm.weight, eps,
                                            attn.qkv_proj.weight, want_h=res is not None)
            if res is None:
                xi = inp
            a = attn(None, positions, None, c, qkv=qkv)
            gu, h = fused.linear_rms_norm(a, xi, layer.post_attention_layernorm.weight, eps,
                                          mlp.gate_up_proj.weight, want_h=True)
            inp, res = fused.linear_silu(gu, mlp.down_proj.weight), h
        logits, _ = fused.linear_rms_norm(inp, res, self.norm.weight, eps, self.lm_head.weight)
        return logits


def random_model(args: ModelArgs | None = None, device="cuda", dtype=torch.bfloat16,
                 seed: int = 0, std: float = 0.02) -> Model:
    """Model with every matrix drawn from N(0, std) (norm weights 1)."""
    args = args or ModelArgs()
    with torch.device("meta"):
        m = Model(args).to(dtype)  # parameters materialise directly in dtype
    m = m.to_empty(device=device)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.normal_(0.0, std, generator=g)
    m = m.eval()
    # the rotary tables are fp32 (the cast above applied to every buffer)
    m.rope = Rope(args.head_dim, args.rope_theta, args.max_position).to(device)
    for blk in m.layers:
        blk.self_attn.rope = m.rope
    return m


class GraphDecoder:
    """Greedy decode steps of `model` captured once as a HIP graph.

    The caches take their positions from one device tensor (ChronoQuantCache.
    bind_device_position), so the captured step (embedding, every layer's
    append + fused decode attention, LM head, argmax, position advance)
    replays unchanged at successive positions; the host only advances the
    caches' offsets.
    """

    def __init__(self, model: Model, caches: list, batch: int, max_len: int):
        dev = next(model.parameters()).device
        self.model, self.caches = model, caches
        self.pos = torch.tensor([caches[0].offset] * batch, dtype=torch.int32, device=dev)
        self.tok = torch.zeros(batch, 1, dtype=torch.long, device=dev)
        # one length vector pos + 1 for all layers, computed by the first
        lens = torch.empty_like(self.pos)
        for i, c in enumerate(caches):
            c.bind_device_position(self.pos, max_len, lengths=lens, update_lengths=i == 0)
        self.graph = None

    def _step(self):
        logits = self.model(self.tok, self.caches, positions=self.pos.long()[:, None])
        nxt = logits[:, -1].argmax(-1, keepdim=True)
        self.tok.copy_(nxt)
        self.pos.add_(1)
        return nxt

    def capture(self, first_token: torch.Tensor):
        """Warm up once on the stream the graph is then captured on
        (allocations, among them the stream's decode workspace, happen
        outside the graph; the warm-up writes the first decode position,
        which the first replay rewrites identically), then capture one
        step."""
        pos0 = self.pos.clone()
        self.tok.copy_(first_token)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side), torch.no_grad():
            self._step()
        torch.cuda.current_stream().wait_stream(side)
        self.pos.copy_(pos0)
        self.tok.copy_(first_token)
        side.wait_stream(torch.cuda.current_stream())
        self.graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(self.graph, stream=side):
            self.out = self._step()
        torch.cuda.current_stream().wait_stream(side)
        self.pos.copy_(pos0)
        self.tok.copy_(first_token)

    def step(self) -> torch.Tensor:
        """One greedy token (the tensor is overwritten by the next step)."""
        self.graph.replay()
        for c in self.caches:
            c.advance(1)
        return self.out

    def release(self):
        for c in self.caches:
            c.bind_device_position(None)


@torch.no_grad()
def generate(model: Model, caches: list, prompt: torch.Tensor, n_new: int,
             prefill_chunk: int = 512, graph: bool = True):
    """Greedy generation: the prompt in prefill_chunk-token chunks, then n_new
    tokens.  Returns (new tokens [B, n_new], prefill seconds, decode seconds)."""
    import time
    B, P = prompt.shape
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits = None
    for s in range(0, P, prefill_chunk):
        logits = model(prompt[:, s:s + prefill_chunk], caches, last_only=True)
    first = logits[:, -1].argmax(-1, keepdim=True)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    out = [first]
    if graph:
        dec = GraphDecoder(model, caches, B, P + n_new)
        dec.capture(first)
        torch.cuda.synchronize()
        t1 = time.perf_counter()  # capture is set-up, not decode time
        for _ in range(n_new - 1):
            out.append(dec.step().clone())
        torch.cuda.synchronize()
        dec.release()
    else:
        tok = first
        for _ in range(n_new - 1):
            tok = model(tok, caches)[:, -1].argmax(-1, keepdim=True)
            out.append(tok)
        torch.cuda.synchronize()
    t2 = time.perf_counter()
    return torch.cat(out, dim=1), t1 - t0, t2 - t1
