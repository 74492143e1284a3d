"""Writes tests/golden/qwen_fp32_b8_decode.npz from the CPU oracle (run from the repo root).

Workload qwen-fp32-b8 (tinybatch_amd.workloads): Qwen2.5-0.5B layer geometry,
fp32, 8 sequences, one decode step (append one token per sequence, then paged
attention). The fixture stores the step's small inputs, a checksum of the
seeded pool, the oracle's attention output and the float64 brute-force output;
the pool itself is regenerated from the seed.
"""
import hashlib
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import brute, reference_path as ref  # noqa: E402
from tinybatch_amd.workloads import make_decode_workload  # noqa: E402

OUT = os.path.join(ROOT, "tests", "golden", "qwen_fp32_b8_decode.npz")


def pool_digest(pool: torch.Tensor) -> str:
    return hashlib.sha256(pool.contiguous().numpy().tobytes()).hexdigest()


def main():
    wl = make_decode_workload("qwen-fp32-b8")
    digest_before = pool_digest(wl.pool)
    pool = wl.pool.clone()
    out = ref.decode_step(pool, wl.q, wl.k_new, wl.v_new, wl.cached_lens, wl.block_tables,
                          wl.num_heads, wl.num_kv_heads, wl.block_size)
    exact = brute.attention_f64(wl.q.numpy(), pool.numpy().reshape(-1), wl.seq_slices, wl.block_tables,
                                wl.context_lens, wl.num_heads, wl.num_kv_heads, wl.block_size, wl.head_dim)
    assert np.abs(out.numpy() - exact).max() < 1e-5
    tables = np.full((wl.batch, max(len(t) for t in wl.block_tables)), -1, dtype=np.int32)
    for b, t in enumerate(wl.block_tables):
        tables[b, :len(t)] = t
    np.savez_compressed(
        OUT, seed=np.int64(wl.seed), cached_lens=np.asarray(wl.cached_lens, np.int32), block_tables=tables,
        q=wl.q.numpy(), k_new=wl.k_new.numpy(), v_new=wl.v_new.numpy(),
        pool_sha256_before=np.array(digest_before), pool_sha256_after=np.array(pool_digest(pool)),
        attn_out=out.numpy(), attn_out_f64=exact)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
