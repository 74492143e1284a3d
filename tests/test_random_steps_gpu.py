"""Seeded random steps through every attention path, against the oracle.

Each case draws its geometry (query / kv heads, head dim), dtype, block size and
step shape from a seed, prints them before it runs, and checks: the pool after
the step bit-exact against the oracle's append (kv_cache.py:25-38), the
attention within rtol = atol = 2e-2 of the oracle in the same dtype
(model.py:130-147), every output finite, and the in-launch merges' error count
zero. The new rows' slots hold NaN before each fused call, so a row read from
the pool instead of from k / v shows up.

- decode steps through tb_paged_decode with a random kernel variant (waves per
  workgroup) and plan unit cost, fused append or not: contexts uniform, tiny,
  whole blocks, or one long sequence among short ones;
- whole-prefill steps through tb_paged_prefill: random cached prefixes (first
  new row anywhere in a tile), new-row counts, contexts up to the kernel's limit,
  fused append or not;
- mixed steps (prefills, cached-prefix tails and decode rows, in the
  reference's token order) through the drop-in cache's append_attention, which
  picks the kernels (one launch, split step, or append then attention) itself.
"""
import numpy as np
import pytest
import torch

from oracle import reference_path as ref
from tinybatch_amd import ops
from tinybatch_amd.kv_cache import PagedKVCache
from tinybatch_amd.metadata import build_step_metadata

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
TOL = dict(atol=2e-2, rtol=2e-2)
GEOMS = [(14, 2, 64), (32, 8, 128), (8, 8, 64), (16, 2, 64), (4, 2, 128), (12, 4, 64)]
DTYPES = [torch.float16, torch.bfloat16]
WAVES = {64: [4, 6, 8], 128: [3, 4]}


def _bits(t):
    return t.contiguous().view(torch.int16)


def _say(msg):
    print(msg, flush=True)


def _pool_and_tables(g, ctx, NB_extra, Hkv, BS, D, dtype):
    need = [(c + BS - 1) // BS for c in ctx]
    NB = sum(need) + NB_extra
    pool = torch.randn(NB, 2, Hkv, BS, D, generator=g).to(dtype)
    perm = torch.randperm(NB, generator=g).tolist()
    tables, at = [], 0
    for n in need:
        tables.append(perm[at:at + n])
        at += n
    for t, c in zip(tables, ctx):       # stale slots past every context, unused blocks: NaN
        if c % BS:
            pool[t[-1], :, :, c % BS:] = float("nan")
    for b in perm[at:]:
        pool[b] = float("nan")
    return pool, tables, NB


def _stale_new_slots(pool, positions, slices, tables, BS):
    stale = pool.clone()
    for (b, e), table in zip(slices, tables):
        for p in positions[b:e]:
            stale[table[p // BS], :, :, p % BS] = float("nan")
    return stale


def _errors():
    return ops.decode_device(DEV).errors()


def _decode_contexts(rng, B, BS):
    kind = int(rng.integers(4))
    if kind == 0:
        ctx = rng.integers(1, 3000, B)
    elif kind == 1:
        ctx = rng.integers(1, 41, B)
    elif kind == 2:
        ctx = BS * rng.integers(1, 61, B)
    else:
        ctx = rng.integers(1, 200, B)
        ctx[int(rng.integers(B))] = int(rng.integers(4000, 9000))
    return ["uniform", "tiny", "whole blocks", "one long"][kind], [int(c) for c in ctx]


@pytest.mark.parametrize("seed", range(16))
def test_random_decode_steps(seed):
    rng = np.random.default_rng(7000 + seed)
    Hq, Hkv, D = GEOMS[int(rng.integers(len(GEOMS)))]
    dtype = DTYPES[int(rng.integers(2))]
    BS = [16, 32, 64][int(rng.integers(3))]
    B = int(rng.integers(1, 49))
    kind, ctx = _decode_contexts(rng, B, BS)
    waves = WAVES[D][int(rng.integers(len(WAVES[D])))]
    unit_cost = int(rng.integers(0, 13))
    fused = bool(rng.integers(2))
    _say(f"[decode seed {seed}] Hq={Hq} Hkv={Hkv} D={D} {dtype} BS={BS} B={B} ctx={kind} (max {max(ctx)}) "
         f"waves={waves} unit_cost={unit_cost} fused={fused}")
    g = torch.Generator().manual_seed(seed)
    pool, tables, NB = _pool_and_tables(g, ctx, 3, Hkv, BS, D, dtype)
    q = torch.randn(B, Hq, D, generator=g).to(dtype)
    k = torch.randn(B, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, Hkv, D, generator=g).to(dtype)
    want_pool = pool.clone()
    want = ref.decode_step(want_pool, q, k, v, [c - 1 for c in ctx], tables, Hq, Hkv, BS)

    meta = build_step_metadata([c - 1 for c in ctx], [(b, b + 1) for b in range(B)], tables, ctx, block_size=BS,
                               num_blocks=NB, partition_tokens=ops.partition_tokens(dtype, D))
    assert ops.attach_decode_plan(meta, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, dtype=dtype, device=DEV,
                                  waves=waves, unit_cost=unit_cost)
    meta = meta.to(DEV)
    positions = [c - 1 for c in ctx]
    slices = [(b, b + 1) for b in range(B)]
    dpool = (_stale_new_slots(pool, positions, slices, tables, BS) if fused else pool).to(DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    if fused:
        out = ops.paged_attention(qd, dpool, meta, num_heads=Hq, k_new=kd, v_new=vd)
    else:
        ops.kv_append(dpool, kd, vd, meta.slot_mapping)
        out = ops.paged_attention(qd, dpool, meta, num_heads=Hq)
    torch.cuda.synchronize()
    assert torch.equal(_bits(dpool.cpu()), _bits(want_pool)), "pool differs (append)"
    got = out.cpu()
    assert torch.isfinite(got).all()
    torch.testing.assert_close(got.float(), want.float(), **TOL)
    assert _errors() == 0


@pytest.mark.parametrize("seed", range(12))
def test_random_whole_prefill_steps(seed):
    rng = np.random.default_rng(8000 + seed)
    Hq, Hkv, D = GEOMS[int(rng.integers(len(GEOMS)))]
    dtype = DTYPES[int(rng.integers(2))]
    BS = [16, 32, 64][int(rng.integers(3))]
    route = ops.prefill_route(dtype, Hq, Hkv, D, DEV)
    assert route is not None
    n = int(rng.integers(1, 7))
    qlens, cached = [], []
    for _ in range(n):
        ql = int(rng.integers(16, min(400, route.max_context) + 1))
        qlens.append(ql)
        cached.append(int(rng.integers(0, route.max_context - ql + 1)) if rng.integers(2) else 0)
    fused = bool(rng.integers(2))
    _say(f"[prefill seed {seed}] Hq={Hq} Hkv={Hkv} D={D} {dtype} BS={BS} new rows={qlens} cached={cached} "
         f"fused={fused}")
    g = torch.Generator().manual_seed(100 + seed)
    ctx = [c + q_ for c, q_ in zip(cached, qlens)]
    pool, tables, NB = _pool_and_tables(g, ctx, 3, Hkv, BS, D, dtype)
    slices, positions, t = [], [], 0
    for c, ql in zip(cached, qlens):
        slices.append((t, t + ql))
        positions.extend(range(c, c + ql))
        t += ql
    q = torch.randn(t, Hq, D, generator=g).to(dtype)
    k = torch.randn(t, Hkv, D, generator=g).to(dtype)
    v = torch.randn(t, Hkv, D, generator=g).to(dtype)
    want_pool = pool.clone()
    ref.kv_write(want_pool, k, v, torch.tensor(positions, dtype=torch.int64), slices, tables, BS)
    want = ref.attention(q, want_pool, slices, tables, ctx, Hq, Hkv)

    meta = build_step_metadata(positions, slices, tables, ctx, block_size=BS, num_blocks=NB,
                               partition_tokens=ops.partition_tokens(dtype, D),
                               rows_per_item=ops.rows_per_item(dtype, Hq, Hkv), tile_prefill=True,
                               prefill_route=route).to(DEV)
    assert meta.num_prefill_work and not meta.num_work_items and not meta.num_prefill_tiles
    dpool = (_stale_new_slots(pool, positions, slices, tables, BS) if fused else pool).to(DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    if fused:
        out = ops.paged_attention(qd, dpool, meta, num_heads=Hq, k_new=kd, v_new=vd)
    else:
        ops.kv_append(dpool, kd, vd, meta.slot_mapping)
        out = ops.paged_attention(qd, dpool, meta, num_heads=Hq)
    torch.cuda.synchronize()
    assert torch.equal(_bits(dpool.cpu()), _bits(want_pool)), "pool differs (append)"
    got = out.cpu()
    assert torch.isfinite(got).all()
    torch.testing.assert_close(got.float(), want.float(), **TOL)


@pytest.mark.parametrize("seed", range(10))
def test_random_mixed_steps_through_the_drop_in_cache(seed):
    rng = np.random.default_rng(9000 + seed)
    Hq, Hkv, D = GEOMS[int(rng.integers(len(GEOMS)))]
    dtype = DTYPES[int(rng.integers(2))]
    BS = [16, 32][int(rng.integers(2))]
    seqs = []                                 # (cached, new rows): prefills first, then decode rows
    for _ in range(int(rng.integers(0, 5))):
        ql = int(rng.integers(2, 300))
        seqs.append((int(rng.integers(0, 400)) if rng.integers(2) else 0, ql))
    n_dec = int(rng.integers(1 if not seqs else 0, 41))
    long_dec = bool(rng.integers(2))
    for _ in range(n_dec):
        seqs.append((int(rng.integers(1000, 3000) if long_dec else rng.integers(0, 600)), 1))
    _say(f"[mixed seed {seed}] Hq={Hq} Hkv={Hkv} D={D} {dtype} BS={BS} prefills={[s for s in seqs if s[1] > 1]} "
         f"decode rows={n_dec} ({'long' if long_dec else 'short'} contexts)")
    g = torch.Generator().manual_seed(200 + seed)
    ctx = [c + ql for c, ql in seqs]
    pool, tables, NB = _pool_and_tables(g, ctx, 3, Hkv, BS, D, dtype)
    slices, positions, t = [], [], 0
    for c, ql in seqs:
        slices.append((t, t + ql))
        positions.extend(range(c, c + ql))
        t += ql
    q = torch.randn(t, Hq, D, generator=g).to(dtype)
    k = torch.randn(t, Hkv, D, generator=g).to(dtype)
    v = torch.randn(t, Hkv, D, generator=g).to(dtype)
    want_pool = pool.clone()
    ref.kv_write(want_pool, k, v, torch.tensor(positions, dtype=torch.int64), slices, tables, BS)
    want = ref.attention(q, want_pool, slices, tables, ctx, Hq, Hkv)

    cache = PagedKVCache(1, NB, BS, Hkv, D, DEV, dtype)
    cache.pools[0].copy_(_stale_new_slots(pool, positions, slices, tables, BS))
    out = cache.append_attention(0, q.to(DEV), k.to(DEV), v.to(DEV), torch.tensor(positions, device=DEV), slices,
                                 tables, ctx, num_heads=Hq)
    torch.cuda.synchronize()
    assert torch.equal(_bits(cache.pools[0].cpu()), _bits(want_pool)), "pool differs (append)"
    got = out.cpu()
    assert torch.isfinite(got).all()
    torch.testing.assert_close(got.float(), want.float(), **TOL)
    assert _errors() == 0
