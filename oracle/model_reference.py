"""Restatement of the reference's Qwen2 forward on the CPU (test infrastructure only).

Follows Qwen2Paged.forward (src/tinybatch/model.py:101-158) op for op on a
state dict that uses the reference's names (model.py:97-98,111-151):
RMSNorm in fp32 (model.py:65-69), RoPE recomputed from positions in fp32
(model.py:72-80), separate q/k/v projections with biases, the paged write and
per-sequence attention of oracle.reference_path (kv_cache.py:25-45,
model.py:127-147), o_proj, SwiGLU MLP, final norm over every row, logits of
each sequence's last token (model.py:153-158).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import reference_path as ref


def rms_norm(x, weight, eps):
    dtype = x.dtype
    x = x.float()
    x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return (x * weight.float()).to(dtype)


def rope(x, positions, theta):
    head_dim = x.shape[-1]
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    freqs = positions.float()[:, None] * inv_freq[None, :]
    cos, sin = freqs.cos()[:, None, :], freqs.sin()[:, None, :]
    x1, x2 = x.float().chunk(2, dim=-1)
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)


@torch.inference_mode()
def forward(w: dict, cfg, token_ids, positions, seq_slices, block_tables, context_lens, pools,
            block_size: int) -> torch.Tensor:
    """Logits [n_seqs, vocab] (fp32). ``pools`` are the per-layer CPU pools, updated in place."""
    h = F.embedding(token_ids, w["model.embed_tokens.weight"])
    for layer in range(cfg.n_layers):
        p = f"model.layers.{layer}."
        x = rms_norm(h, w[p + "input_layernorm.weight"], cfg.rms_eps)
        q = F.linear(x, w[p + "self_attn.q_proj.weight"], w[p + "self_attn.q_proj.bias"])
        k = F.linear(x, w[p + "self_attn.k_proj.weight"], w[p + "self_attn.k_proj.bias"])
        v = F.linear(x, w[p + "self_attn.v_proj.weight"], w[p + "self_attn.v_proj.bias"])
        q = q.view(-1, cfg.n_heads, cfg.head_dim)
        k = k.view(-1, cfg.n_kv_heads, cfg.head_dim)
        v = v.view(-1, cfg.n_kv_heads, cfg.head_dim)
        q, k = rope(q, positions, cfg.rope_theta), rope(k, positions, cfg.rope_theta)
        ref.kv_write(pools[layer], k, v, positions, seq_slices, block_tables, block_size)
        attn = ref.attention(q, pools[layer], seq_slices, block_tables, context_lens, cfg.n_heads, cfg.n_kv_heads)
        h = h + F.linear(attn, w[p + "self_attn.o_proj.weight"])
        x = rms_norm(h, w[p + "post_attention_layernorm.weight"], cfg.rms_eps)
        gate = F.linear(x, w[p + "mlp.gate_proj.weight"])
        up = F.linear(x, w[p + "mlp.up_proj.weight"])
        h = h + F.linear(F.silu(gate) * up, w[p + "mlp.down_proj.weight"])
    h = rms_norm(h, w["model.norm.weight"], cfg.rms_eps)
    last = torch.tensor([e - 1 for _, e in seq_slices])
    return F.linear(h[last], w["lm_head.weight"]).float()
