"""tb_build_decode_plan (host code, no GPU), checked through the properties the
decode kernel relies on: every 16-position tile of every (sequence, kv head)
unit appears exactly once (pads, flagged, only as the second tile of a pair;
every worker's count even); each entry addresses the right pool block (block
sizes 16..64), with the tile's valid rows, the unit's last-tile flag and the
context; a worker's tiles of one unit are consecutive and in order; all the
workers holding a unit run on one XCD (worker k on XCD (k / waves) % num_xcds)
and are consecutive there, their piece indices 0.. in that order, the wave of
piece 0 recorded, and partial slots [base, base + pieces) distinct across units;
a unit one worker holds is written whole (-1); each XCD's workers get even
shares of its weight (tiles + unit_cost per unit); block ids outside the pool
and short tables are IndexError; more than 255 pieces for a unit is declined."""
import numpy as np
import pytest

from tinybatch_amd.metadata import build_decode_plan

E_LAST, E_NULL = 1 << 28, 1 << 29


def tables_for(ctx, bs, rng):
    need = [(c + bs - 1) // bs for c in ctx]
    nb = sum(need) + 7
    perm = rng.permutation(nb)
    t = np.full((len(ctx), max(need)), -1, dtype=np.int32)
    at = 0
    for b, n in enumerate(need):
        t[b, :n] = perm[at:at + n]
        at += n
    return t, nb


def decode(plan, workers, stride):
    counts = plan[:workers]
    ents = plan[(workers + 3) // 4 * 4:].reshape(-1, 4)[:workers * stride].reshape(workers, stride, 4)
    return counts, ents


def check_plan(ctx, hkv, D, bs, G, nx, waves, uc, seed=0):
    rng = np.random.default_rng(seed)
    tables, nb = tables_for(ctx, bs, rng)
    got = build_decode_plan(ctx, tables, block_size=bs, num_blocks=nb, num_kv_heads=hkv, head_dim=D, workgroups=G,
                            num_xcds=nx, waves=waves, unit_cost=uc)
    assert got is not None
    plan, w, stride, pieces = got
    assert w == waves and stride % 2 == 0
    W = G * waves
    counts, ents = decode(plan, W, stride)
    tb = 32 * D
    tile_bytes = tb * (bs // 16)
    blk_bytes = 2 * hkv * tile_bytes
    seen = {}
    holders = {}                                  # unit -> list of (kk, worker, idx, base, np, w0)
    for k in range(W):
        n = int(counts[k])
        assert 0 <= n <= stride and n % 2 == 0
        prev = None
        for i in range(n):
            x, y, z, ww = (int(v) for v in ents[k, i])
            b, h = y & 0xFFFFF, (y >> 20) & 15
            if y & E_NULL:
                assert i % 2 == 1 and prev is not None and prev[0] == (b, h)   # a pad ends an odd segment
                continue
            u = (b, h)
            off = (x & 0xFFFFFFFF) << 8
            blk, rem = divmod(off, blk_bytes)
            hh, rem = divmod(rem, tile_bytes)
            sub, rem = divmod(rem, tb)
            assert hh == h and rem == 0
            t = None
            for tt in range((ctx[b] + 15) // 16):
                if tables[b, 16 * tt // bs] == blk and (16 * tt % bs) // 16 == sub:
                    t = tt
            assert t is not None, "entry addresses a block the unit does not own"
            assert (u, t) not in seen
            seen[(u, t)] = k
            nt = (ctx[b] + 15) // 16
            assert ((y >> 24) & 15) + 1 == min(16, ctx[b] - 16 * t)
            assert bool(y & E_LAST) == (t == nt - 1)
            assert (z & 0xFFFFFF) == ctx[b]
            if prev is not None and prev[0] == u:
                assert t == prev[1] + 1                  # consecutive tiles of a unit
            prev = (u, t)
            kk = (k // waves // nx) * waves + k % waves  # the worker's index on its XCD
            rec = (kk, k, (z >> 24) & 0xFF, ww)
            lst = holders.setdefault(u, [])
            if not lst or lst[-1][1] != k:
                lst.append(rec)
    for b, c in enumerate(ctx):
        for h in range(hkv):
            for t in range((c + 15) // 16):
                assert ((b, h), t) in seen, "a tile is missing"
    slots = set()
    for u, lst in holders.items():
        xcds = {(k // waves) % nx for _, k, _, _ in lst}
        assert len(xcds) == 1                          # a unit's partials stay on one XCD
        kks = [r[0] for r in lst]
        assert kks == list(range(kks[0], kks[0] + len(kks)))
        if len(lst) == 1:
            assert lst[0][3] == -1                     # written whole
            continue
        np_ = len(lst)
        for i, (kk, k, idx, ww) in enumerate(lst):
            assert idx == i and ww != -1
            assert ((ww >> 20) & 0xFF) + 1 == np_ and (ww >> 28) & 15 == kks[0] % waves
        base = lst[0][3] & 0xFFFFF
        assert all((r[3] & 0xFFFFF) == base for r in lst)
        rng_ = set(range(base, base + np_))
        assert not (rng_ & slots)
        slots |= rng_
    assert len(slots) <= pieces
    # balance: each XCD's workers cut its weight evenly
    for x in range(nx):
        us = {u for u, lst in holders.items() if (lst[0][1] // waves) % nx == x}
        weight = sum((ctx[b] + 15) // 16 + uc for b, h in us)
        nwg = len(range(x, G, nx))
        share = weight / (nwg * waves)
        for k in range(W):
            if (k // waves) % nx != x:
                continue
            real = sum(1 for i in range(int(counts[k])) if not (int(ents[k, i, 1]) & E_NULL))
            assert real <= share + 1 + 1e-9
    return plan, holders


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("D,waves", [(64, 8), (64, 4), (128, 4), (128, 3)])
def test_random_steps(seed, D, waves):
    rng = np.random.default_rng(100 + seed)
    B = int(rng.integers(40, 90))
    ctx = rng.integers(1, 3000, B).tolist()
    check_plan(ctx, 2 if D == 64 else 8, D, 16, 64, 8, waves, int(rng.integers(0, 9)), seed=seed)


@pytest.mark.parametrize("bs", [16, 32, 64])
def test_block_sizes(bs):
    ctx = [1, 15, 16, 17, 31, 32, 33, 64, 65, 700, 1024, 5000] * 4
    check_plan(ctx, 2, 64, bs, 64, 8, 4, 4, seed=bs)


def test_headline_shape_is_balanced_and_every_unit_splits():
    from tinybatch_amd.workloads import make_decode_workload

    wl = make_decode_workload("qwen-fp16-b64")
    _, holders = check_plan(wl.context_lens, 2, 64, 16, 256, 8, 8, 8)
    assert all(len(v) > 1 for v in holders.values())   # 128 units over 2048 workers


def test_many_pieces_and_the_255_limit():
    ctx = [60000, 300, 200]
    tables, nb = tables_for(ctx, 16, np.random.default_rng(1))
    # 8 waves x 32 workgroups per XCD: the long units would need 256 pieces
    assert build_decode_plan(ctx, tables, block_size=16, num_blocks=nb, num_kv_heads=2, head_dim=64,
                             workgroups=256, num_xcds=8, waves=8, unit_cost=0) is None
    _, holders = check_plan(ctx, 2, 64, 16, 256, 8, 4, 0)
    assert max(len(v) for v in holders.values()) == 128


def test_block_outside_the_pool_and_short_tables():
    ctx = [40, 50]
    tables, nb = tables_for(ctx, 16, np.random.default_rng(2))
    bad = tables.copy()
    bad[1, 1] = nb
    with pytest.raises(IndexError):
        build_decode_plan(ctx, bad, block_size=16, num_blocks=nb, num_kv_heads=2, head_dim=64, workgroups=16,
                          num_xcds=8, waves=4)
    with pytest.raises(IndexError):
        build_decode_plan([40, 90], tables, block_size=16, num_blocks=nb, num_kv_heads=2, head_dim=64,
                          workgroups=16, num_xcds=8, waves=4)


def test_unsupported_geometries_and_variants():
    ctx = [100, 200]
    tables, nb = tables_for(ctx, 16, np.random.default_rng(3))
    assert build_decode_plan(ctx, tables, block_size=16, num_blocks=nb, num_kv_heads=2, head_dim=96,
                             workgroups=16, num_xcds=8) is None
    with pytest.raises(ValueError):
        build_decode_plan(ctx, tables, block_size=16, num_blocks=nb, num_kv_heads=2, head_dim=64, workgroups=16,
                          num_xcds=8, waves=5)
    with pytest.raises(ValueError):
        build_decode_plan([0, 10], tables, block_size=16, num_blocks=nb, num_kv_heads=2, head_dim=64,
                          workgroups=16, num_xcds=8)


def test_the_decode_kernel_is_chosen_for_large_decode_steps():
    import torch

    from tinybatch_amd import ops
    from tinybatch_amd.metadata import build_step_metadata
    from tinybatch_amd.workloads import make_decode_workload

    wl = make_decode_workload("qwen-fp16-b64")
    meta = build_step_metadata(wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens, block_size=16,
                               num_blocks=wl.num_blocks, partition_tokens=256)
    assert ops.decode_kernel_preferred(meta, num_kv_heads=2, head_dim=64, dtype=torch.float16)
    assert not ops.decode_kernel_preferred(meta, num_kv_heads=2, head_dim=64, dtype=torch.float32)
    small = make_decode_workload("qwen-fp16-b64", batch=8)   # 16 units: XCDs would idle
    meta = build_step_metadata(small.positions, small.seq_slices, small.block_tables, small.context_lens,
                               block_size=16, num_blocks=small.num_blocks, partition_tokens=256)
    assert not ops.decode_kernel_preferred(meta, num_kv_heads=2, head_dim=64, dtype=torch.float16)


def expand_on_host(counts, segs, tables, *, bs, hkv, D, workers, stride):
    """The descriptors of tb_build_decode_segments expanded as tb_expand_decode_plan
    does on the device (a restatement in numpy, for the host-side check)."""
    plan = np.zeros((workers + 3) // 4 * 4 + (workers * stride + 64) * 4, dtype=np.int32)
    plan[:counts.size] = counts
    ents = plan[(workers + 3) // 4 * 4:].reshape(-1, 4)
    tb = 32 * D
    tile_bytes = tb * (bs // 16)
    blk_bytes = 2 * hkv * tile_bytes
    for k, pos_first, bh, tu0, info, ctx, piece, e3 in segs.tolist():
        n, unit_end = info & 0x3FFFFFFF, bool(info & (1 << 30))
        b, h = bh & 0xFFFFF, bh >> 20
        for i in range(n + (n & 1)):
            pad = i >= n
            tu = tu0 + (n - 1 if pad else i)
            pos0 = 16 * tu
            off = int(tables[b, pos0 // bs]) * blk_bytes + h * tile_bytes + ((pos0 % bs) // 16) * tb
            rows = min(16, ctx - pos0)
            y = b | (h << 20) | ((rows - 1) << 24) | (E_LAST if (not pad and unit_end and i == n - 1) else 0) \
                | (E_NULL if pad else 0)
            ents[k * stride + pos_first + i] = [np.int64(off >> 8).astype(np.int32), y, ctx | (piece << 24), e3]
    return plan


@pytest.mark.parametrize("ctx,hkv,D,bs,waves", [
    ([2631, 2025, 2714, 2772, 17, 1, 16, 33] * 3, 2, 64, 16, 4),
    ([900 + 37 * i for i in range(40)], 2, 64, 32, 8),
    ([5000, 1200, 30000, 64, 1024], 8, 128, 16, 4),
    ([1, 2, 3, 15, 16, 17, 31, 32, 33], 2, 64, 64, 6),
])
def test_segments_expand_to_the_host_plan(ctx, hkv, D, bs, waves):
    """tb_build_decode_segments' counts and descriptors, expanded entry by entry, give
    exactly the words of tb_build_decode_plan (the device builds the same plan)."""
    from tinybatch_amd.metadata import build_decode_segments

    rng = np.random.default_rng(3)
    tables, nb = tables_for(ctx, bs, rng)
    G, nx = 32, 8
    host = build_decode_plan(ctx, tables, block_size=bs, num_blocks=nb, num_kv_heads=hkv, head_dim=D, workgroups=G,
                             num_xcds=nx, waves=waves)
    seg = build_decode_segments(ctx, tables, block_size=bs, num_kv_heads=hkv, head_dim=D, workgroups=G,
                                num_xcds=nx, waves=waves)
    plan, w, stride, pieces = host
    counts, segs, w2, stride2, pieces2 = seg
    assert (w, stride, pieces) == (w2, stride2, pieces2)
    assert segs.shape[0] <= len(ctx) * hkv + G * waves
    got = expand_on_host(counts, segs, tables, bs=bs, hkv=hkv, D=D, workers=G * waves, stride=stride)
    W = G * waves
    np.testing.assert_array_equal(got[:W], plan[:W])
    cw, cs = decode(plan, W, stride)
    gw, gs = decode(got, W, stride)
    for k in range(W):
        n = int(cw[k])
        np.testing.assert_array_equal(gs[k, :n], cs[k, :n])


def test_segments_carry_the_shared_newest_mark():
    from tinybatch_amd.metadata import build_decode_segments

    rng = np.random.default_rng(4)
    ctx = [40, 40]
    tables, nb = tables_for(ctx, 16, rng)
    tables[1, 2] = tables[0, 2]                       # both newest positions (39) in one block, offset 7
    counts = build_decode_segments(ctx, tables, block_size=16, num_kv_heads=2, head_dim=64, workgroups=8,
                                   num_xcds=8, waves=4)[0]
    assert np.all(counts[:32] & (1 << 30))
    host = build_decode_plan(ctx, tables, block_size=16, num_blocks=nb, num_kv_heads=2, head_dim=64, workgroups=8,
                             num_xcds=8, waves=4)[0]
    np.testing.assert_array_equal(counts[:32], host[:32])


def _max_entries(ctx, hkv, D, uc, waves=4):
    tables, nb = tables_for(ctx, 16, np.random.default_rng(7))
    plan, w, stride, _ = build_decode_plan(ctx, tables, block_size=16, num_blocks=nb, num_kv_heads=hkv, head_dim=D,
                                           workgroups=256, num_xcds=8, waves=waves, unit_cost=uc)
    return int(decode(plan, 256 * w, stride)[0].max() & 0x3FFFFFFF)


def test_unit_cost_is_lowered_only_when_it_empties_the_busiest_worker():
    """tb_decode_unit_cost against the built plans' own counts: the headline step (64
    sequences of 513..4096 positions) gets 18 entries per busiest worker at cost 6
    against 20 at the default 8, so 6; the 56 decode rows of the mixed step tie (the
    default stays); the Llama-geometry step saves < 5% (the default stays)."""
    from tinybatch_amd.metadata import decode_defaults, decode_unit_cost
    from tinybatch_amd.workloads import make_decode_workload, make_mixed_workload

    mixed = make_mixed_workload()
    cases = [
        ("headline", make_decode_workload("qwen-fp16-b64").context_lens, 2, 64, 6),
        ("mixed", [c for c, q in zip(mixed.context_lens, mixed.q_lens) if q == 1], 2, 64, 8),
    ]
    rng = np.random.default_rng(11)
    cases.append(("llama", (rng.integers(256, 4096, 256) + 1).tolist(), 8, 128, None))
    for name, ctx, hkv, D, want in cases:
        dflt = decode_defaults(D)[1]
        got = decode_unit_cost(ctx, num_kv_heads=hkv, head_dim=D, workgroups=256, num_xcds=8, waves=4)
        me, me_lower = _max_entries(ctx, hkv, D, dflt), _max_entries(ctx, hkv, D, dflt - 2)
        assert got in (dflt, dflt - 2), name
        assert (got == dflt - 2) == (me_lower * 20 <= me * 19), name
        if want is not None:
            assert got == want, name
    assert _max_entries(cases[0][1], 2, 64, 6) == 18 and _max_entries(cases[0][1], 2, 64, 8) == 20
