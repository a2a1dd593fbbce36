"""Qwen2 forward on flat token batches, driving the HIP path.

Mirrors the reference model (nanoserve/qwen2.py:29-174, layers.py): module
names match HuggingFace (model.layers.N.self_attn.q_proj, ...), activations
are flat [num_tokens, hidden] with no padding, the rotary cos/sin lookup is
done once per forward for all layers, and logits are computed only for the
rows the sampler needs.  Each attention layer runs, in order (qwen2.py:46-66):

    projections -> fused rotary + cache write (ns_rope_reshape_and_cache)
                -> paged attention (attn_fn, ns_paged_attention) -> o_proj

Linear layers are nn.Linear or, after `quantize_model`, Int4Linear
(ns_int4_linear).  `fuse_projections()` concatenates q/k/v into one
projection and gate/up into another (row concatenation, so INT4 groups are
unchanged), which turns 5 GEMM launches per layer into 2; q, k and v are then
column views of the fused output, which the rotary kernel reads in place.  A
fused INT4 q|k|v projection keeps each head's rows in rotary-pair order and
runs rotary and the cache write in its own epilogue
(ns_int4_linear_rope_cache), so projection, rotary and cache write are one
launch.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from .quant import Int4Linear, int4_qkv_rope_cache
from .rotary import RotaryEmbedding, rope_reshape_and_cache


@dataclass
class Qwen2Config:
    """Field names as transformers' Qwen2Config; defaults are Qwen2.5-0.5B."""

    vocab_size: int = 151936
    hidden_size: int = 896
    intermediate_size: int = 4864
    num_hidden_layers: int = 24
    num_attention_heads: int = 14
    num_key_value_heads: int = 2
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1000000.0
    max_position_embeddings: int = 32768
    tie_word_embeddings: bool = True

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps) * weight (reference layers.py:25-47, fused torch kernel)."""

    def __init__(self, hidden_size: int, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.rms_norm(x, (x.shape[-1],), self.weight, self.variance_epsilon)


def _linear(mod: nn.Module, x: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
    """mod(x) (+ residual): INT4 projections add the residual inside their launch."""
    if isinstance(mod, Int4Linear):
        return mod(x, residual=residual)
    y = mod(x)
    return y if residual is None else residual + y


def _concat_linears(parts: list[nn.Module]) -> nn.Module:
    """One linear whose output rows are the parts' rows in order."""
    if all(isinstance(p, Int4Linear) for p in parts):
        p0 = parts[0]
        out_f = sum(p.out_features for p in parts)
        m = Int4Linear(p0.in_features, out_f, p0.bias is not None, p0.group_size, p0.compute_dtype,
                       p0.qweight.device)
        m.qweight.copy_(torch.cat([p.qweight for p in parts]))
        m.scales.copy_(torch.cat([p.scales for p in parts]))
        m.zeros.copy_(torch.cat([p.zeros for p in parts]))
        if p0.bias is not None:
            m.bias.data.copy_(torch.cat([p.bias.data for p in parts]))
        return m
    if all(isinstance(p, nn.Linear) for p in parts):
        p0 = parts[0]
        w = torch.cat([p.weight.data for p in parts])
        m = nn.Linear(p0.in_features, w.shape[0], bias=p0.bias is not None, device=w.device, dtype=w.dtype)
        m.weight.data.copy_(w)
        if p0.bias is not None:
            m.bias.data.copy_(torch.cat([p.bias.data for p in parts]))
        return m
    raise TypeError("cannot fuse a mix of linear types")


class Qwen2Attention(nn.Module):
    def __init__(self, cfg: Qwen2Config, layer_idx: int, linear_cls=nn.Linear) -> None:
        super().__init__()
        self.layer_idx = layer_idx
        self.num_heads = cfg.num_attention_heads
        self.num_kv_heads = cfg.num_key_value_heads
        self.head_dim = cfg.head_dim
        self.scale = self.head_dim ** -0.5
        hd = self.head_dim
        # Qwen2 puts biases on q/k/v but not on o (qwen2.py:40-44).
        self.q_proj = linear_cls(cfg.hidden_size, self.num_heads * hd, bias=True)
        self.k_proj = linear_cls(cfg.hidden_size, self.num_kv_heads * hd, bias=True)
        self.v_proj = linear_cls(cfg.hidden_size, self.num_kv_heads * hd, bias=True)
        self.o_proj = linear_cls(self.num_heads * hd, cfg.hidden_size, bias=False)
        self.qkv_proj: nn.Module | None = None

    def fuse(self) -> None:
        qkv = _concat_linears([self.q_proj, self.k_proj, self.v_proj])
        if isinstance(qkv, Int4Linear) and self.head_dim % 16 == 0:
            # Rows in rotary-pair order: rotary and the cache write run in the
            # projection's epilogue (ns_int4_linear_rope_cache).
            qkv = Int4Linear.rope_pairs(qkv, self.num_heads, self.num_kv_heads, self.head_dim)
        self.qkv_proj = qkv
        del self.q_proj, self.k_proj, self.v_proj

    def forward(self, hidden, cos, sin, kv_cache, md, attn_fn, residual=None, norm=None):
        """o_proj(attention(norm(hidden))) (+ residual).  `norm` (the layer's
        input RMSNorm) runs inside the fused INT4 q|k|v launch when it can."""
        T = hidden.shape[0]
        Hq, Hkv, D = self.num_heads, self.num_kv_heads, self.head_dim
        if norm is not None and not (isinstance(self.qkv_proj, Int4Linear) and self.qkv_proj.fuses_norm):
            hidden, norm = norm(hidden), None
        kc, vc = kv_cache.k_cache[self.layer_idx], kv_cache.v_cache[self.layer_idx]
        if isinstance(self.qkv_proj, Int4Linear) and self.qkv_proj.rope_heads is not None:
            q = int4_qkv_rope_cache(hidden, self.qkv_proj, cos, sin, kc, vc, md.slot_mapping, norm=norm)
            out = attn_fn(q, kc, vc, md, self.scale)
            return _linear(self.o_proj, out.view(T, Hq * D), residual)
        if self.qkv_proj is not None:
            qkv = self.qkv_proj(hidden, norm=norm) if norm is not None else self.qkv_proj(hidden)
            q = qkv[:, :Hq * D].view(T, Hq, D)
            k = qkv[:, Hq * D:(Hq + Hkv) * D].view(T, Hkv, D)
            v = qkv[:, (Hq + Hkv) * D:].view(T, Hkv, D)
        else:
            q = self.q_proj(hidden).view(T, Hq, D)
            k = self.k_proj(hidden).view(T, Hkv, D)
            v = self.v_proj(hidden).view(T, Hkv, D)
        # Rotary on q and k, then k and v into the cache before attention reads
        # it (a prefill chunk attends to the keys it just produced).
        q = rope_reshape_and_cache(q, k, v, cos, sin, kc, vc, md.slot_mapping)
        out = attn_fn(q, kc, vc, md, self.scale)
        return _linear(self.o_proj, out.view(T, Hq * D), residual)


class Qwen2MLP(nn.Module):
    """down(silu(gate(x)) * up(x)) (reference layers.py:98-109)."""

    def __init__(self, cfg: Qwen2Config, linear_cls=nn.Linear) -> None:
        super().__init__()
        self.intermediate_size = cfg.intermediate_size
        self.gate_proj = linear_cls(cfg.hidden_size, cfg.intermediate_size, bias=False)
        self.up_proj = linear_cls(cfg.hidden_size, cfg.intermediate_size, bias=False)
        self.down_proj = linear_cls(cfg.intermediate_size, cfg.hidden_size, bias=False)
        self.gate_up_proj: nn.Module | None = None

    def fuse(self) -> None:
        if isinstance(self.gate_proj, Int4Linear) and isinstance(self.up_proj, Int4Linear):
            # One launch computes silu(gate) * up from interleaved rows.
            self.gate_up_proj = Int4Linear.gate_up_pairs(self.gate_proj, self.up_proj)
        else:
            self.gate_up_proj = _concat_linears([self.gate_proj, self.up_proj])
        del self.gate_proj, self.up_proj

    def forward(self, x, residual=None, norm=None):
        """down(silu(gate(norm(x))) * up(norm(x))) (+ residual); the RMSNorm runs
        inside the fused INT4 gate|up launch when it can."""
        gu = self.gate_up_proj
        if isinstance(gu, Int4Linear) and gu.silu_mul:
            act = gu(x, norm=norm)  # normalises first when the layer does not fuse it
        else:
            if norm is not None:
                x = norm(x)
            if gu is not None:
                y = gu(x)
                g, u = y[:, :self.intermediate_size], y[:, self.intermediate_size:]
            else:
                g, u = self.gate_proj(x), self.up_proj(x)
            act = F.silu(g) * u
        return _linear(self.down_proj, act, residual)


class Qwen2DecoderLayer(nn.Module):
    def __init__(self, cfg: Qwen2Config, layer_idx: int, linear_cls=nn.Linear) -> None:
        super().__init__()
        self.self_attn = Qwen2Attention(cfg, layer_idx, linear_cls)
        self.mlp = Qwen2MLP(cfg, linear_cls)
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)

    def forward(self, hidden, cos, sin, kv_cache, md, attn_fn):
        h = self.self_attn(hidden, cos, sin, kv_cache, md, attn_fn, residual=hidden, norm=self.input_layernorm)
        return self.mlp(h, residual=h, norm=self.post_attention_layernorm)


class Qwen2Model(nn.Module):
    def __init__(self, cfg: Qwen2Config, linear_cls=nn.Linear, max_position: int = 4096) -> None:
        super().__init__()
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList([Qwen2DecoderLayer(cfg, i, linear_cls) for i in range(cfg.num_hidden_layers)])
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        # Sized to the serving length, like the reference (qwen2.py:92-98).
        self.rotary = RotaryEmbedding(cfg.head_dim, max_position, base=cfg.rope_theta)

    def forward(self, input_ids, positions, kv_cache, md, attn_fn):
        hidden = self.embed_tokens(input_ids)
        if self.rotary.cos_cached.device != positions.device:
            self.rotary.to(positions.device)  # float32 tables follow the model's device
        # One cos/sin lookup for all layers (qwen2.py:105-113), and the
        # attention backend's per-step preparation (the HIP backend's decode
        # plan), also shared by all layers.
        cos, sin = self.rotary.cos_sin(positions, hidden.dtype)
        prepare = getattr(attn_fn, "prepare", None)
        if prepare is not None:
            prepare(md, kv_cache.k_cache[0])
        for layer in self.layers:
            hidden = layer(hidden, cos, sin, kv_cache, md, attn_fn)
        return self.norm(hidden)


class Qwen2ForCausalLM(nn.Module):
    def __init__(self, cfg: Qwen2Config, linear_cls=nn.Linear, max_position: int = 4096) -> None:
        super().__init__()
        self.config = cfg
        self.model = Qwen2Model(cfg, linear_cls, max_position)
        # lm_head stays in the model dtype under quantisation (quant.py skip list).
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        if cfg.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight

    def forward(self, input_ids, positions, kv_cache, md, attn_fn):
        return self.model(input_ids, positions, kv_cache, md, attn_fn)

    def compute_logits(self, hidden: torch.Tensor, indices: torch.Tensor | None = None) -> torch.Tensor:
        if indices is not None:
            hidden = hidden.index_select(0, indices)
        return self.lm_head(hidden)

    def fuse_projections(self) -> "Qwen2ForCausalLM":
        for layer in self.model.layers:
            layer.self_attn.fuse()
            layer.mlp.fuse()
        return self

    @property
    def num_layers(self) -> int:
        return self.config.num_hidden_layers

    @property
    def num_kv_heads(self) -> int:
        return self.config.num_key_value_heads

    @property
    def head_dim(self) -> int:
        return self.config.head_dim


@torch.no_grad()
def random_init_(model: nn.Module, std: float = 0.02, seed: int = 0) -> nn.Module:
    """N(0, std) for every linear and embedding weight, zero biases, unit norms (HF's init)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    for name, p in model.named_parameters():
        if name.endswith("layernorm.weight") or name.endswith("norm.weight"):
            p.fill_(1.0)
        elif name.endswith(".bias"):
            p.zero_()
        else:
            p.copy_(torch.randn(p.shape, generator=g) * std)
    return model
