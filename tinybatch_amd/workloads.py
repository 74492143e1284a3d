"""Seeded synthetic workloads of the paged data path (bench and tests).

Shapes follow the layer geometries the data path is measured on:
* ``qwen-fp32-b8``    Qwen2.5-0.5B layer (14 query / 2 KV heads, head_dim 64),
  block 16, fp32, 8 sequences with U{16..256} cached tokens, 512-block pool.
* ``qwen-fp16-b64``   same geometry in fp16, 64 sequences with U{512..4096}
  cached tokens, 32768-block pool.
* ``llama-bf16-b256`` Llama-3-8B layer (32 / 8 heads, head_dim 128), bf16, 256
  sequences with log-normal cached lengths (median 8192, sigma 0.5) clipped to
  [1024, 32768], pool sized to fit every sequence.
* ``llama-bf16-b256-s1`` the same with sigma 1.0: a heavier tail, many contexts
  at the 32768 clip (the distribution's sigma is not given; 0.5 and 1.0 are
  both measured).
Each decode step appends one token per sequence at position L (the cached
length) and then attends over ctx = L + 1 positions, as LLMEngine.step does
for running sequences (reference src/tinybatch/engine.py:114-120).

Draw order from one CPU torch.Generator seeded per workload: cached lengths,
block permutation, q, new k, new v, then the pool (N(0,1), drawn in fp32 and
cast). A pool too large to draw on the CPU in reasonable time is drawn on the
GPU from its own seeded generator instead (``pool_device``).
Block tables are consecutive chunks of one random permutation of the pool.

``qwen-bf16-mixed`` is one mixed engine step (``make_mixed_workload``): Qwen
geometry in bf16, eight fresh 512-token prefills (q_len = ctx = 512, the
is_causal branch) scheduled before 56 decodes (the engine's token order,
reference src/tinybatch/engine.py:104-120). 32 decodes have U{256..2048}
cached tokens; 24 share one 32-block (512-token) prompt prefix, as prefix-cache
hits do (reference src/tinybatch/block_manager.py:94-104), and have
U{512..2048} cached tokens so that the prefix fits. Plus a compaction round of
1024 block copies (distinct sources in use, destinations free).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass
class DecodeWorkload:
    name: str
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    dtype: torch.dtype
    num_blocks: int
    cached_lens: list[int]
    block_tables: list[list[int]]
    q: torch.Tensor          # [B, Hq, D]
    k_new: torch.Tensor      # [B, Hkv, D]
    v_new: torch.Tensor      # [B, Hkv, D]
    pool: torch.Tensor       # [NB, 2, Hkv, BS, D]
    seed: int

    @property
    def batch(self) -> int:
        return len(self.cached_lens)

    @property
    def context_lens(self) -> list[int]:
        return [c + 1 for c in self.cached_lens]

    @property
    def positions(self) -> list[int]:
        return list(self.cached_lens)

    @property
    def seq_slices(self) -> list[tuple[int, int]]:
        return [(b, b + 1) for b in range(self.batch)]

    def algorithmic_bytes(self) -> dict:
        """Logical bytes of one append + decode-attention layer step (no cache credit).

        append: read k,v + write the pool rows + 4 B slot per token;
        attention: every visible K and V row once, q and out once, the block-table
        entries used and the context lengths.
        """
        b = torch.tensor([], dtype=self.dtype).element_size()
        B, Hq, Hkv, D, BS = self.batch, self.num_heads, self.num_kv_heads, self.head_dim, self.block_size
        ctx = self.context_lens
        append = B * 2 * Hkv * D * b * 2 + 4 * B
        attn = (sum(ctx) * 2 * Hkv * D * b + 2 * B * Hq * D * b
                + 4 * sum((c + BS - 1) // BS for c in ctx) + 4 * B)
        return {"append": append, "attention": attn, "total": append + attn}

    def flops(self) -> int:
        return 4 * self.num_heads * self.head_dim * sum(self.context_lens)


SPECS = {
    "qwen-fp32-b8": dict(Hq=14, Hkv=2, D=64, BS=16, dtype=torch.float32, B=8, lens=("uniform", 16, 256),
                         num_blocks=512, seed=1),
    "qwen-fp16-b64": dict(Hq=14, Hkv=2, D=64, BS=16, dtype=torch.float16, B=64, lens=("uniform", 512, 4096),
                          num_blocks=32768, seed=2),
    "llama-bf16-b256": dict(Hq=32, Hkv=8, D=128, BS=16, dtype=torch.bfloat16, B=256,
                            lens=("lognormal", 8192, 0.5, 1024, 32768), num_blocks=None, seed=3),
    "llama-bf16-b256-s1": dict(Hq=32, Hkv=8, D=128, BS=16, dtype=torch.bfloat16, B=256,
                               lens=("lognormal", 8192, 1.0, 1024, 32768), num_blocks=None, seed=5),
}


def _cached_lengths(gen: torch.Generator, B: int, spec) -> list[int]:
    if spec[0] == "uniform":
        lo, hi = spec[1], spec[2]
        return torch.randint(lo, hi + 1, (B,), generator=gen).tolist()
    median, sigma, lo, hi = spec[1:]
    z = torch.randn(B, generator=gen, dtype=torch.float64)
    vals = torch.exp(math.log(median) + sigma * z).round().clamp(lo, hi)
    return [int(x) for x in vals.tolist()]


def make_decode_workload(name: str, *, pool_device: str | torch.device = "cpu", seed: int | None = None,
                         batch: int | None = None) -> DecodeWorkload:
    spec = SPECS[name]
    seed = spec["seed"] if seed is None else seed
    gen = torch.Generator().manual_seed(seed)
    B = spec["B"] if batch is None else batch
    Hq, Hkv, D, BS, dt = spec["Hq"], spec["Hkv"], spec["D"], spec["BS"], spec["dtype"]
    cached = _cached_lengths(gen, B, spec["lens"])
    need = [(c + 1 + BS - 1) // BS for c in cached]      # blocks for ctx = L + 1
    NB = spec["num_blocks"] or sum(need)
    if sum(need) > NB:
        raise ValueError(f"{name}: sequences need {sum(need)} blocks, pool has {NB}")
    perm = torch.randperm(NB, generator=gen).tolist()
    tables, at = [], 0
    for n in need:
        tables.append(perm[at:at + n])
        at += n
    q = torch.randn(B, Hq, D, generator=gen).to(dt)
    k_new = torch.randn(B, Hkv, D, generator=gen).to(dt)
    v_new = torch.randn(B, Hkv, D, generator=gen).to(dt)
    shape = (NB, 2, Hkv, BS, D)
    pool_device = torch.device(pool_device)
    if pool_device.type == "cpu":
        pool = torch.randn(*shape, generator=gen).to(dt)
    else:
        g2 = torch.Generator(device=pool_device).manual_seed(seed + 1000)
        pool = torch.empty(shape, dtype=dt, device=pool_device)
        flat = pool.view(-1)
        step = 1 << 28
        for s in range(0, flat.numel(), step):
            n = min(step, flat.numel() - s)
            flat[s:s + n] = torch.randn(n, generator=g2, device=pool_device, dtype=torch.float32).to(dt)
    return DecodeWorkload(name=name, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, block_size=BS, dtype=dt,
                          num_blocks=NB, cached_lens=cached, block_tables=tables, q=q, k_new=k_new,
                          v_new=v_new, pool=pool, seed=seed)


@dataclass
class MixedWorkload:
    name: str
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    dtype: torch.dtype
    num_blocks: int
    q_lens: list[int]
    context_lens: list[int]
    block_tables: list[list[int]]
    q: torch.Tensor          # [T, Hq, D]
    k_new: torch.Tensor      # [T, Hkv, D]
    v_new: torch.Tensor      # [T, Hkv, D]
    pool: torch.Tensor       # [NB, 2, Hkv, BS, D]
    copy_src: list[int]
    copy_dst: list[int]
    shared_prefix: list[int]
    num_prefill: int
    seed: int

    @property
    def batch(self) -> int:
        return len(self.q_lens)

    @property
    def num_tokens(self) -> int:
        return sum(self.q_lens)

    @property
    def seq_slices(self) -> list[tuple[int, int]]:
        out, at = [], 0
        for n in self.q_lens:
            out.append((at, at + n))
            at += n
        return out

    @property
    def positions(self) -> list[int]:
        pos = []
        for n, c in zip(self.q_lens, self.context_lens):
            pos.extend(range(c - n, c))
        return pos

    def part(self, which: str) -> "MixedWorkload":
        """The prefill-only or decode-only sub-batch (same pool, same tables)."""
        sel = range(self.num_prefill) if which == "prefill" else range(self.num_prefill, self.batch)
        sl = self.seq_slices
        rows = torch.cat([torch.arange(sl[i][0], sl[i][1]) for i in sel])
        return MixedWorkload(
            name=f"{self.name}:{which}", num_heads=self.num_heads, num_kv_heads=self.num_kv_heads,
            head_dim=self.head_dim, block_size=self.block_size, dtype=self.dtype, num_blocks=self.num_blocks,
            q_lens=[self.q_lens[i] for i in sel], context_lens=[self.context_lens[i] for i in sel],
            block_tables=[self.block_tables[i] for i in sel], q=self.q[rows], k_new=self.k_new[rows],
            v_new=self.v_new[rows], pool=self.pool, copy_src=self.copy_src, copy_dst=self.copy_dst,
            shared_prefix=self.shared_prefix, num_prefill=self.num_prefill if which == "prefill" else 0,
            seed=self.seed)

    def algorithmic_bytes(self) -> dict:
        """append: read k,v + write the pool rows + slots; attention: every visible
        K/V row of every sequence once (shared prefix counted per sequence, as
        logical bytes), q and out of every row, block-table entries, context
        lengths; copy: read + write of every copied block."""
        b = torch.tensor([], dtype=self.dtype).element_size()
        Hq, Hkv, D, BS = self.num_heads, self.num_kv_heads, self.head_dim, self.block_size
        T = self.num_tokens
        append = T * 2 * Hkv * D * b * 2 + 4 * T
        attn = (sum(self.context_lens) * 2 * Hkv * D * b + 2 * T * Hq * D * b
                + 4 * sum((c + BS - 1) // BS for c in self.context_lens) + 4 * self.batch)
        copy = 2 * len(self.copy_src) * 2 * Hkv * BS * D * b
        return {"append": append, "attention": attn, "copy": copy}

    def unique_kv_bytes(self) -> int:
        """K/V bytes of distinct blocks the attention reads (shared prefix once)."""
        b = torch.tensor([], dtype=self.dtype).element_size()
        used = set()
        for t, c in zip(self.block_tables, self.context_lens):
            used.update(t[:(c + self.block_size - 1) // self.block_size])
        return len(used) * 2 * self.num_kv_heads * self.block_size * self.head_dim * b

    def flops(self) -> int:
        """Attention flops: 2 (QK) + 2 (PV) per head, dim and visible (row, key) pair."""
        pairs = 0
        for n, c in zip(self.q_lens, self.context_lens):
            first = c - n
            pairs += sum(first + i + 1 for i in range(n))
        return 4 * self.num_heads * self.head_dim * pairs


def make_mixed_workload(name: str = "qwen-bf16-mixed", *, seed: int = 4, num_blocks: int = 32768,
                        num_copies: int = 1024) -> MixedWorkload:
    if name != "qwen-bf16-mixed":
        raise KeyError(name)
    gen = torch.Generator().manual_seed(seed)
    Hq, Hkv, D, BS, dt = 14, 2, 64, 16, torch.bfloat16
    n_pre, pre_len, n_dec, n_share, prefix_blocks = 8, 512, 32, 24, 32
    cached_dec = torch.randint(256, 2049, (n_dec,), generator=gen).tolist()
    cached_share = torch.randint(prefix_blocks * BS, 2049, (n_share,), generator=gen).tolist()
    perm = torch.randperm(num_blocks, generator=gen).tolist()
    at = 0

    def take(n):
        nonlocal at
        ids = perm[at:at + n]
        at += n
        return ids

    tables, q_lens, ctx = [], [], []
    for _ in range(n_pre):
        tables.append(take(pre_len // BS))
        q_lens.append(pre_len)
        ctx.append(pre_len)
    for c in cached_dec:
        tables.append(take((c + 1 + BS - 1) // BS))
        q_lens.append(1)
        ctx.append(c + 1)
    prefix = take(prefix_blocks)
    for c in cached_share:
        tables.append(prefix + take((c + 1 + BS - 1) // BS - prefix_blocks))
        q_lens.append(1)
        ctx.append(c + 1)
    in_use = perm[:at]
    if at + num_copies > num_blocks:
        raise ValueError("pool too small for the copy round")
    dst = take(num_copies)
    src_idx = torch.randperm(len(in_use), generator=gen)[:num_copies].tolist()
    src = [in_use[i] for i in src_idx]
    T = sum(q_lens)
    q = torch.randn(T, Hq, D, generator=gen).to(dt)
    k_new = torch.randn(T, Hkv, D, generator=gen).to(dt)
    v_new = torch.randn(T, Hkv, D, generator=gen).to(dt)
    pool = torch.randn(num_blocks, 2, Hkv, BS, D, generator=gen).to(dt)
    return MixedWorkload(name=name, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, block_size=BS, dtype=dt,
                         num_blocks=num_blocks, q_lens=q_lens, context_lens=ctx, block_tables=tables, q=q,
                         k_new=k_new, v_new=v_new, pool=pool, copy_src=src, copy_dst=dst,
                         shared_prefix=prefix, num_prefill=n_pre, seed=seed)


@dataclass
class ServingWorkload:
    """Continuous-batching workload of requests (token ids), all arriving at t = 0."""
    name: str
    prompts: list[list[int]]
    max_new_tokens: list[int]
    shared_prefix_len: int
    sharing: list[bool]
    seed: int


def make_serving_workload(name: str = "qwen2-0.5b-e2e", *, seed: int = 5, vocab_size: int = 151936,
                          num_requests: int = 32, share_frac: float = 0.75, prefix_len: int = 400,
                          max_prompt: int = 512, min_prompt: int = 32, out_lo: int = 16,
                          out_hi: int = 256) -> ServingWorkload:
    """Random-token requests: ``share_frac`` of them (chosen by a seeded
    permutation) start with one common ``prefix_len``-token prefix and have
    lengths U{prefix_len+1..max_prompt}; the rest U{min_prompt..max_prompt};
    output lengths U{out_lo..out_hi} (greedy, no stop tokens)."""
    if name != "qwen2-0.5b-e2e":
        raise KeyError(name)
    gen = torch.Generator().manual_seed(seed)
    n_share = round(share_frac * num_requests)
    order = torch.randperm(num_requests, generator=gen).tolist()
    sharing = [False] * num_requests
    for i in order[:n_share]:
        sharing[i] = True
    prefix = torch.randint(0, vocab_size, (prefix_len,), generator=gen).tolist()
    prompts, outs = [], []
    for i in range(num_requests):
        if sharing[i]:
            n = int(torch.randint(prefix_len + 1, max_prompt + 1, (1,), generator=gen))
            prompts.append(prefix + torch.randint(0, vocab_size, (n - prefix_len,), generator=gen).tolist())
        else:
            n = int(torch.randint(min_prompt, max_prompt + 1, (1,), generator=gen))
            prompts.append(torch.randint(0, vocab_size, (n,), generator=gen).tolist())
        outs.append(int(torch.randint(out_lo, out_hi + 1, (1,), generator=gen)))
    return ServingWorkload(name=name, prompts=prompts, max_new_tokens=outs, shared_prefix_len=prefix_len,
                           sharing=sharing, seed=seed)
