"""Restatement of the reference's CPU data path (test infrastructure only).

Follows the reference op for op, so that its numerics (and its cost, when
bench.py times it) are those of tinybatch's own CPU path:
* kv_write   — PagedKVCache.write, src/tinybatch/kv_cache.py:25-38
* kv_gather  — PagedKVCache.gather, src/tinybatch/kv_cache.py:40-45
* attention  — the per-sequence region of Qwen2Paged.forward,
               src/tinybatch/model.py:130-147 (gather, repeat_interleave,
               is_causal branch or boolean offset mask, SDPA, output rows)
All tensors live on the CPU; the dtype is the model dtype (fp32 / fp16 / bf16).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def kv_write(pool: torch.Tensor, k: torch.Tensor, v: torch.Tensor, positions: torch.Tensor,
             seq_slices, block_tables, block_size: int) -> None:
    """Scatter new K/V rows of every sequence into its blocks (kv_cache.py:32-38)."""
    for (start, end), table in zip(seq_slices, block_tables):
        p = positions[start:end]
        phys = torch.tensor(table, device=k.device)[torch.div(p, block_size, rounding_mode="floor")]
        within = p % block_size
        pool[phys, 0, :, within] = k[start:end]
        pool[phys, 1, :, within] = v[start:end]


def kv_gather(pool: torch.Tensor, table, context_len: int):
    """Contiguous [ctx, kv_heads, head_dim] K and V of one sequence (kv_cache.py:42-45)."""
    blocks = pool[torch.tensor(table, device=pool.device)]                  # [nb, 2, kvh, bs, hd]
    kv = blocks.permute(1, 0, 3, 2, 4).reshape(2, -1, blocks.shape[2], blocks.shape[4])
    return kv[0, :context_len], kv[1, :context_len]


def attention(q: torch.Tensor, pool: torch.Tensor, seq_slices, block_tables, context_lens,
              num_heads: int, num_kv_heads: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """attn_out [T, num_heads*head_dim] of the flat batch (model.py:131-147).

    q: [T, num_heads, head_dim] (post-RoPE). Rows outside every slice keep the
    contents of ``out`` (the reference allocates it with torch.empty).
    """
    T, _, head_dim = q.shape
    if out is None:
        out = torch.zeros(T, num_heads * head_dim, dtype=q.dtype, device=q.device)
    group = num_heads // num_kv_heads
    for (start, end), table, ctx in zip(seq_slices, block_tables, context_lens):
        keys, vals = kv_gather(pool, table, ctx)                             # [ctx, kvh, hd]
        qi = q[start:end].transpose(0, 1)                                    # [h, q_len, hd]
        ki = keys.repeat_interleave(group, dim=1).transpose(0, 1)            # [h, ctx, hd]
        vi = vals.repeat_interleave(group, dim=1).transpose(0, 1)
        n_new = end - start
        if n_new == ctx:
            o = F.scaled_dot_product_attention(qi, ki, vi, is_causal=True)
        else:
            allowed = torch.zeros(n_new, ctx, dtype=torch.bool, device=q.device)
            first = ctx - n_new
            for i in range(n_new):
                allowed[i, : first + i + 1] = True
            o = F.scaled_dot_product_attention(qi, ki, vi, attn_mask=allowed)
        out[start:end] = o.transpose(0, 1).reshape(n_new, -1)
    return out


def decode_step(pool: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cached_lens,
                block_tables, num_heads: int, num_kv_heads: int, block_size: int) -> torch.Tensor:
    """One decode step of a batch (one new token per sequence, engine.py:114-120):
    the token at position cached_len is written, then attends to cached_len+1 positions."""
    B = q.shape[0]
    positions = torch.tensor(list(cached_lens), dtype=torch.int64)
    slices = [(b, b + 1) for b in range(B)]
    kv_write(pool, k, v, positions, slices, block_tables, block_size)
    ctx = [int(c) + 1 for c in cached_lens]
    return attention(q, pool, slices, block_tables, ctx, num_heads, num_kv_heads)
