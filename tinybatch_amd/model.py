"""Random-initialised Qwen2 forward pass over the paged KV cache (GPU).

Counterpart of Qwen2Paged (reference src/tinybatch/model.py:111-158) with the
attention region (model.py:127-147) replaced by the paged data path:
kv_cache.write (K1, slot-mapped append) and kv_cache.attention (K2, fused
paged attention over every sequence of the flat batch in one launch). The
rest follows the reference layer by layer: RMSNorm computed in fp32
(model.py:65-69), rotate-half RoPE in fp32 (model.py:72-80), q/k/v
projections with biases, o_proj, SwiGLU MLP, residuals, final norm, tied LM
head on the last token of each sequence (model.py:153-158).

MI355X-side choices: q/k/v are one GEMM over a concatenated weight (and
gate/up another); the residual add + RMSNorm, the RoPE of q and k and the
SwiGLU gate are one fused kernel each (layer_ops) instead of chains of tensor
ops; the RoPE tables are built once for every position up to max_position;
the LM head runs on the last rows only. With ``fused_rope`` (the default) the
RoPE of q and k is folded into the paged kernels (K1 rotates k on its way to
the pool, K2 rotates q as it loads it) instead of a launch of its own. With
``fused_mlp`` (the default) decode-sized batches of 16-bit rows take the
weight-streaming projections: o_proj and down_proj as split-K partials that
the residual add + RMSNorm launch after them adds up, gate/up fused with the
SwiGLU gate.

Weights are drawn from a seeded generator (no checkpoint exists offline):
N(0, 0.02) for embeddings, projections and biases, ones for the norms.
``reference_weights`` returns them under the reference's state-dict names.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import layer_ops, ops
from .kv_cache import PagedKVCache


@dataclass
class ModelConfig:
    n_layers: int
    n_heads: int
    n_kv_heads: int
    d_model: int
    head_dim: int
    d_ff: int
    vocab_size: int
    rms_eps: float
    rope_theta: float
    tie_embeddings: bool
    max_position: int

    @staticmethod
    def qwen2_0_5b() -> "ModelConfig":
        """Qwen2.5-0.5B dimensions (494,032,768 parameters with tied embeddings);
        rope_theta / rms_eps are Qwen2.5's published 1e6 / 1e-6."""
        return ModelConfig(n_layers=24, n_heads=14, n_kv_heads=2, d_model=896, head_dim=64, d_ff=4864,
                           vocab_size=151936, rms_eps=1e-6, rope_theta=1e6, tie_embeddings=True,
                           max_position=32768)

    def num_params(self) -> int:
        qkv = (self.n_heads + 2 * self.n_kv_heads) * self.head_dim
        per_layer = (self.d_model * qkv + qkv + self.n_heads * self.head_dim * self.d_model
                     + 3 * self.d_model * self.d_ff + 2 * self.d_model)
        head = 0 if self.tie_embeddings else self.vocab_size * self.d_model
        return self.vocab_size * self.d_model + self.n_layers * per_layer + self.d_model + head


def rope_tables(head_dim: int, theta: float, max_position: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """cos / sin [max_position, head_dim/2] with the reference's fp32 arithmetic (model.py:74-76)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device).float() / head_dim))
    freqs = torch.arange(max_position, device=device).float()[:, None] * inv_freq[None, :]
    return freqs.cos(), freqs.sin()


class Qwen2Paged:
    """Weights + forward; inference only."""

    def __init__(self, cfg: ModelConfig, device: torch.device, dtype: torch.dtype, seed: int = 0):
        self.cfg, self.device, self.dtype = cfg, torch.device(device), dtype
        g = torch.Generator(device=self.device).manual_seed(seed)

        def rnd(*shape):
            return (torch.randn(*shape, generator=g, device=self.device, dtype=torch.float32) * 0.02).to(dtype)

        c = cfg
        qkv = (c.n_heads + 2 * c.n_kv_heads) * c.head_dim
        self.embed = rnd(c.vocab_size, c.d_model)
        self.lm_head = self.embed if c.tie_embeddings else rnd(c.vocab_size, c.d_model)
        self.layers = []
        for _ in range(c.n_layers):
            self.layers.append({
                "ln1": torch.ones(c.d_model, device=self.device, dtype=dtype),
                "w_qkv": rnd(qkv, c.d_model), "b_qkv": rnd(qkv),
                "w_o": rnd(c.d_model, c.n_heads * c.head_dim),
                "ln2": torch.ones(c.d_model, device=self.device, dtype=dtype),
                "w_gu": rnd(2 * c.d_ff, c.d_model),
                "w_down": rnd(c.d_model, c.d_ff),
            })
        self.norm = torch.ones(c.d_model, device=self.device, dtype=dtype)
        self.cos, self.sin = rope_tables(c.head_dim, c.rope_theta, c.max_position, self.device)
        self.rope = ops.Rope(self.cos, self.sin)
        self.fused_rope = True
        self.fused_mlp = True

    def reference_weights(self) -> dict[str, torch.Tensor]:
        """The weights under the reference's state-dict names (model.py:97-98,111-151)."""
        c = self.cfg
        hq, hk = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
        w = {"model.embed_tokens.weight": self.embed, "model.norm.weight": self.norm, "lm_head.weight": self.lm_head}
        for i, L in enumerate(self.layers):
            p = f"model.layers.{i}."
            w[p + "input_layernorm.weight"] = L["ln1"]
            w[p + "post_attention_layernorm.weight"] = L["ln2"]
            for name, lo, hi in (("q", 0, hq), ("k", hq, hq + hk), ("v", hq + hk, hq + 2 * hk)):
                w[p + f"self_attn.{name}_proj.weight"] = L["w_qkv"][lo:hi]
                w[p + f"self_attn.{name}_proj.bias"] = L["b_qkv"][lo:hi]
            w[p + "self_attn.o_proj.weight"] = L["w_o"]
            w[p + "mlp.gate_proj.weight"] = L["w_gu"][:c.d_ff]
            w[p + "mlp.up_proj.weight"] = L["w_gu"][c.d_ff:]
            w[p + "mlp.down_proj.weight"] = L["w_down"]
        return w

    # Split-K ranges of the partial projections: o_proj (K = d_model) and
    # down_proj (K = d_ff), measured at the 0.5B shapes for 1..32 rows.
    O_SPLITS, DOWN_SPLITS = 4, 8

    @staticmethod
    def _streamed(x: torch.Tensor) -> bool:
        """Decode-sized batches of 16-bit rows take the weight-streaming kernels
        (measured faster than the library GEMM at these shapes for up to 32 rows)."""
        return x.shape[0] <= 32 and x.dtype in (torch.float16, torch.bfloat16)

    def _proj(self, x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None = None) -> torch.Tensor:
        """q/k/v and o projections: tb_linear for decode-sized batches, F.linear otherwise."""
        if self._streamed(x):
            return layer_ops.linear(x, w, b)
        return F.linear(x, w, b)

    def run_layers(self, token_ids: torch.Tensor, positions: torch.Tensor, attention,
                   fused_rope: bool = False) -> torch.Tensor:
        """Hidden states after the final norm, [T, d_model]. ``attention(layer, q, k, v)``
        appends the step's K/V and returns attn_out [T, Hq*D] (model.py:127-147); with
        ``fused_rope`` q and k are the projections before RoPE (views of the qkv rows)
        and ``attention`` must rotate them."""
        c = self.cfg
        T = token_ids.shape[0]
        hq, hk = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
        h = F.embedding(token_ids, self.embed)                       # the residual stream
        x = layer_ops.rms_norm(h, self.layers[0]["ln1"], c.rms_eps)
        for i, L in enumerate(self.layers):
            qkv = self._proj(x, L["w_qkv"], L["b_qkv"])
            if fused_rope:
                q = qkv[:, :hq].view(T, c.n_heads, c.head_dim)
                k = qkv[:, hq:hq + hk].view(T, c.n_kv_heads, c.head_dim)
            else:
                q, k = layer_ops.rope_qk(qkv, positions, self.cos, self.sin, c.n_heads, c.n_kv_heads, c.head_dim)
            v = qkv[:, hq + hk:].view(T, c.n_kv_heads, c.head_dim)
            attn = attention(i, q, k, v)
            nxt = self.layers[i + 1]["ln1"] if i + 1 < len(self.layers) else self.norm
            if self.fused_mlp and self._streamed(x):
                parts = layer_ops.linear_partials(attn, L["w_o"], self.O_SPLITS)
                x = layer_ops.rms_norm_partials(parts, L["ln2"], c.rms_eps, residual=h)
                act = layer_ops.linear_silu_mul(x, L["w_gu"])
                parts = layer_ops.linear_partials(act, L["w_down"], self.DOWN_SPLITS)
                x = layer_ops.rms_norm_partials(parts, nxt, c.rms_eps, residual=h)
                continue
            x = layer_ops.rms_norm(self._proj(attn, L["w_o"]), L["ln2"], c.rms_eps, residual=h)
            act = layer_ops.silu_mul(F.linear(x, L["w_gu"]), c.d_ff)
            x = layer_ops.rms_norm(F.linear(act, L["w_down"]), nxt, c.rms_eps, residual=h)
        return x

    @torch.inference_mode()
    def forward(self, token_ids: torch.Tensor, positions: torch.Tensor, seq_slices: list[tuple[int, int]],
                block_tables: list[list[int]], context_lens: list[int], kv_cache: PagedKVCache) -> torch.Tensor:
        """Logits [n_seqs, vocab] (fp32) for the last token of each sequence (model.py:101-158)."""
        rope = self.rope if self.fused_rope else None

        def attention(i, q, k, v):   # the append (kv_cache.write) folded into attention where it can be
            return kv_cache.append_attention(i, q, k, v, positions, seq_slices, block_tables, context_lens,
                                             rope=rope)

        x = self.run_layers(token_ids, positions, attention, fused_rope=self.fused_rope)
        last = torch.tensor([e - 1 for _, e in seq_slices], device=x.device)
        return F.linear(x[last], self.lm_head).float()
