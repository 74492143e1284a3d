"""Float64 brute force and closed forms used to pin the oracle (test infrastructure only).

Written independently of reference_path: the pool is addressed through the
flat index (((blk*2 + kv)*Hkv + h)*BS + s)*D + d of the layout documented in
src/tinybatch/kv_cache.py:1-7, and attention is the textbook definition with
explicit loops:
    O[r, h] = sum_{j <= ctx - q_len + i} softmax_j(q[r,h] . k_{h // rep, j} * scale) v_{h // rep, j}
(the rule of src/tinybatch/model.py:135-146; scale = 1/sqrt(D) as
scaled_dot_product_attention's default).
"""
from __future__ import annotations

import math

import numpy as np


def flat_index(blk, kv, h, s, d, Hkv, BS, D):
    return (((blk * 2 + kv) * Hkv + h) * BS + s) * D + d


def write_closed_form(pool_flat: np.ndarray, k: np.ndarray, v: np.ndarray, positions, seq_slices,
                      block_tables, Hkv: int, BS: int, D: int) -> np.ndarray:
    """Sequential scatter, last writer wins; returns a new flat pool."""
    out = pool_flat.copy()
    dd = np.arange(D)
    for (s, e), table in zip(seq_slices, block_tables):
        for t in range(s, e):
            pos = int(positions[t])
            blk, off = table[pos // BS], pos % BS
            for h in range(Hkv):
                out[flat_index(blk, 0, h, off, dd, Hkv, BS, D)] = k[t, h]
                out[flat_index(blk, 1, h, off, dd, Hkv, BS, D)] = v[t, h]
    return out


def gather_closed_form(pool_flat: np.ndarray, table, ctx: int, Hkv: int, BS: int, D: int):
    """K, V [ctx, Hkv, D] read one element row at a time through the table."""
    K = np.empty((ctx, Hkv, D), dtype=pool_flat.dtype)
    V = np.empty_like(K)
    dd = np.arange(D)
    for t in range(ctx):
        blk, off = table[t // BS], t % BS
        for h in range(Hkv):
            K[t, h] = pool_flat[flat_index(blk, 0, h, off, dd, Hkv, BS, D)]
            V[t, h] = pool_flat[flat_index(blk, 1, h, off, dd, Hkv, BS, D)]
    return K, V


def attention_f64(q: np.ndarray, pool_flat: np.ndarray, seq_slices, block_tables, context_lens,
                  Hq: int, Hkv: int, BS: int, D: int, scale: float | None = None) -> np.ndarray:
    """out [T, Hq*D] in float64 (rows outside every slice are zero)."""
    T = q.shape[0]
    rep = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = np.zeros((T, Hq * D), dtype=np.float64)
    pf = pool_flat.astype(np.float64)
    for (s, e), table, ctx in zip(seq_slices, block_tables, context_lens):
        K, V = gather_closed_form(pf, table, ctx, Hkv, BS, D)
        q_len = e - s
        for i in range(q_len):
            limit = ctx - q_len + i          # last visible position
            for h in range(Hq):
                g = h // rep
                qv = q[s + i, h].astype(np.float64)
                scores = (K[: limit + 1, g] @ qv) * scale
                scores -= scores.max()
                p = np.exp(scores)
                out[s + i, h * D:(h + 1) * D] = (p[:, None] * V[: limit + 1, g]).sum(0) / p.sum()
    return out


def copy_closed_form(pool_flat: np.ndarray, src, dst, block_elems: int) -> np.ndarray:
    out = pool_flat.copy()
    for s, d in zip(src, dst):
        out[d * block_elems:(d + 1) * block_elems] = pool_flat[s * block_elems:(s + 1) * block_elems]
    return out
