"""CPU oracle for one Qwen2 forward over a paged cache -- TEST INFRASTRUCTURE ONLY.

Restates the reference forward (nanoserve/qwen2.py:46-113, layers.py:25-109)
in float32 on the CPU from the model's weights (INT4 projections dequantised
by oracle.quant to the model dtype, as the reference QuantLinear does), with
the oracle's own rotary (oracle.rope), cache write and gather+SDPA attention
(oracle.paged_attention).  Only tests/ use it, as the checker.

Its pieces are pinned where they live (rotary, cache write, attention,
dequantiser); the composition -- norm, residuals, SwiGLU, layer order, cos/sin
shared by all layers, logits of the selected rows -- is the reference's
forward, and the GPU tests compare against it at fp16 tolerance (and
within-GPU invariants: incremental == one-shot, batchmate independence).
"""

from __future__ import annotations

import torch

from .paged_attention import paged_attention_ref, reshape_and_cache_ref
from .quant import dequantize_int4_ref
from .rope import rope_apply_ref, rope_cos_sin_ref, rope_table_ref


def _weight(module, dtype_name: str) -> tuple[torch.Tensor, torch.Tensor | None]:
    """(W [out, in] float32 holding model-dtype values, bias or None) of a linear-like module."""
    if hasattr(module, "qweight"):
        w = dequantize_int4_ref(module.qweight.cpu().numpy(), module.scales.cpu().numpy(),
                                module.zeros.cpu().numpy(), module.group_size, dtype_name)
        w = torch.from_numpy(w)
    else:
        w = module.weight.detach().cpu().float()
    b = None if module.bias is None else module.bias.detach().cpu().float()
    return w, b


def _rope_pair_order_ref(heads: int, D: int) -> list[int]:
    """Stored row r of a rope-paired q|k|v weight holds original row order[r]:
    16-row tile i of each head holds dims [8i, 8i+8) then [D/2 + 8i, D/2 + 8i + 8)
    (the layout ns_int4_linear_rope_cache documents; restated here, not imported)."""
    return [h * D + (8 * i + j if j < 8 else D // 2 + 8 * i + (j - 8))
            for h in range(heads) for i in range(D // 16) for j in range(16)]


def _qkv_weight(module, dtype_name: str):
    """(W, b) of a fused q|k|v module in q|k|v row order."""
    w, b = _weight(module, dtype_name)
    heads = getattr(module, "rope_heads", None)
    if heads is not None:
        Hq, Hkv, D = heads
        order = torch.tensor(_rope_pair_order_ref(Hq + 2 * Hkv, D))
        inv = torch.empty_like(order)
        inv[order] = torch.arange(order.numel())
        w = w[inv]
        b = None if b is None else b[inv]
    return w, b


def _rms(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


@torch.inference_mode()
def qwen2_forward_ref(model, input_ids, positions, k_caches, v_caches, md, sample_idx=None):
    """Returns (logits of sample_idx rows or all rows, new k_caches, new v_caches), all float32 on CPU.

    `model` is a nanoserve_amd Qwen2ForCausalLM (fused or not); only its
    weights and config are read.  Caches are lists of per-layer CPU tensors
    in the model dtype; the returned caches are new tensors.
    """
    cfg = model.config
    dt = model.model.embed_tokens.weight.dtype
    name = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}[dt]
    Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    ids = input_ids.detach().cpu().long()
    pos = positions.detach().cpu().long()
    T = ids.shape[0]
    emb = model.model.embed_tokens.weight.detach().cpu().float()
    h = emb[ids]
    ct, st = rope_table_ref(D, int(pos.max()) + 1, cfg.rope_theta)
    cos, sin = rope_cos_sin_ref(ct, st, pos, dt)
    cos, sin = cos.float(), sin.float()
    kcs, vcs = [], []
    for li, layer in enumerate(model.model.layers):
        att, mlp = layer.self_attn, layer.mlp
        x = _rms(h, layer.input_layernorm.weight.detach().cpu().float(), cfg.rms_norm_eps)
        if att.qkv_proj is not None:
            w, b = _qkv_weight(att.qkv_proj, name)
            qkv = x @ w.T + b
            q, k, v = qkv[:, :Hq * D], qkv[:, Hq * D:(Hq + Hkv) * D], qkv[:, (Hq + Hkv) * D:]
        else:
            q, k, v = [(lambda wb: x @ wb[0].T + wb[1])(_weight(p, name))
                       for p in (att.q_proj, att.k_proj, att.v_proj)]
        q, k, v = q.reshape(T, Hq, D), k.reshape(T, Hkv, D), v.reshape(T, Hkv, D)
        q, k = rope_apply_ref(q, k, cos, sin)
        kc, vc = reshape_and_cache_ref(k, v, k_caches[li], v_caches[li], md.slot_mapping)
        kcs.append(kc)
        vcs.append(vc)
        o = paged_attention_ref(q, kc.float(), vc.float(), md, att.scale)
        wo, _ = _weight(att.o_proj, name)
        h = h + o.reshape(T, Hq * D) @ wo.T
        x = _rms(h, layer.post_attention_layernorm.weight.detach().cpu().float(), cfg.rms_norm_eps)
        if mlp.gate_up_proj is not None:
            w, _ = _weight(mlp.gate_up_proj, name)
            gu = x @ w.T
            if getattr(mlp.gate_up_proj, "silu_mul", False):  # rows interleaved (gate_j, up_j)
                g, u = gu[:, 0::2], gu[:, 1::2]
            else:
                g, u = gu[:, :cfg.intermediate_size], gu[:, cfg.intermediate_size:]
        else:
            g, u = x @ _weight(mlp.gate_proj, name)[0].T, x @ _weight(mlp.up_proj, name)[0].T
        wd, _ = _weight(mlp.down_proj, name)
        h = h + (torch.nn.functional.silu(g) * u) @ wd.T
    h = _rms(h, model.model.norm.weight.detach().cpu().float(), cfg.rms_norm_eps)
    if sample_idx is not None:
        h = h[sample_idx.detach().cpu().long()]
    logits = h @ model.lm_head.weight.detach().cpu().float().T
    return logits, kcs, vcs


def relative_error(got: torch.Tensor, want: torch.Tensor) -> float:
    """max |got - want| / max |want| (the scale-free error the model tests bound)."""
    g, w = got.detach().cpu().double(), want.detach().cpu().double()
    return float((g - w).abs().max() / w.abs().max().clamp_min(1e-30))

