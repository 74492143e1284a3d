"""tb_build_decode_plan (host code, no GPU): every 16-position tile of every
(sequence, kv head) unit belongs to exactly one segment; the workers are the
waves of the workgroups (worker k on XCD (k / waves) % num_xcds); all segments
of a unit belong to workers of one XCD; each XCD's workers get equal shares of
its tiles (within one tile); the plan carries each segment's context length and
the pool block of every tile in worker order (block_tables gathered); a unit
held by one segment writes its output directly (slot -1); the pieces of a unit
cut into several segments are grouped per workgroup (consecutive, one leader
carrying the member and group counts, LDS indices in workgroup order), and a
unit over several workgroups has one distinct partial slot per group, numbered
from its first slot; limits are reported as TB_ERR_UNSUPPORTED and answered
with more workgroups; a block id outside the pool is TB_ERR_INDEX."""
import ctypes

import numpy as np
import pytest

from tinybatch_amd import _lib
from tinybatch_amd.metadata import build_decode_plan, decode_limits

TILE = 16


def tables_for(ctx, bs, rng=None, nb=None):
    """Distinct random blocks for every sequence (or blocks in order)."""
    need = [(c + bs - 1) // bs for c in ctx]
    width = max(need) if need else 1
    total = sum(need)
    nb = nb or total + 3
    perm = (rng.permutation(nb) if rng is not None else np.arange(nb))[:total]
    t = np.full((len(ctx), width), -1, dtype=np.int32)
    at = 0
    for b, n in enumerate(need):
        t[b, :n] = perm[at:at + n]
        at += n
    return t, nb


def c_plan(ctx, hkv, G, nx, waves=4, tmax=1 << 20, smax=1 << 20, bs=16, tables=None, nb=None, group=True):
    ctx = np.ascontiguousarray(ctx, dtype=np.int32)
    if tables is None:
        tables, nb = tables_for(ctx, bs)
    tables = np.ascontiguousarray(tables, dtype=np.int32)
    vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    L = _lib.lib()
    nbytes = int(L.tb_decode_plan_bytes(vp(ctx), len(ctx), hkv, G, waves))
    if nbytes == 0:
        return _lib.TB_ERR_INVALID_ARG, None
    plan = np.zeros(nbytes // 4, dtype=np.int32)
    st = L.tb_build_decode_plan(vp(ctx), len(ctx), hkv, vp(tables), tables.shape[1], bs, nb, G, waves, nx, tmax,
                                smax, int(group), vp(plan), nbytes)
    return st, plan


def parse(plan):
    W, S, U, pieces, nx, waves, T = (int(x) for x in plan[:7])
    workers = plan[8:8 + 4 * W].reshape(W, 4)
    off = 8 + 4 * W
    segs = plan[off:off + 8 * S].reshape(S, 8)
    units = plan[off + 8 * S:off + 8 * S + 2 * U].reshape(U, 2)
    tiles = plan[off + 8 * S + 2 * U:off + 8 * S + 2 * U + T]
    return W, S, U, pieces, nx, waves, T, workers, segs, units, tiles


def check(ctx, hkv, G, nx, waves=4, bs=16, seed=0, group=True):
    rng = np.random.default_rng(seed)
    tables, nb = tables_for(ctx, bs, rng)
    st, plan = c_plan(ctx, hkv, G, nx, waves=waves, bs=bs, tables=tables, nb=nb, group=group)
    assert st == 0
    assert plan[7] == int(group)
    W, S, U, pieces, nx_, waves_, T, workers, segs, units, tiles = parse(plan)
    assert (W, U, nx_, waves_) == (G * waves, len(ctx) * hkv, nx, waves)
    ntile = [(c + TILE - 1) // TILE for c in ctx for _ in range(hkv)]
    assert T == sum(ntile)
    covered = [np.zeros(t, dtype=np.int32) for t in ntile]
    per_w = np.zeros(W, dtype=np.int64)
    seg_w = np.full(S, -1, dtype=np.int64)
    at_seg = at_tile = 0
    for k in range(W):
        s0, ns, t0, nt = workers[k]
        assert s0 == at_seg and t0 == at_tile        # workers' records are back to back
        seg_w[s0:s0 + ns] = k
        at_seg += ns
        at_tile += nt
        got = 0
        for (u, a, e, slot, c, *_) in segs[s0:s0 + ns]:
            b = u // hkv
            assert c == ctx[b]                         # the segment's context length
            # the blocks of the segment's tiles, gathered from the tables in order
            want = [tables[b, (TILE * t) // bs] for t in range(a, e)]
            assert tiles[t0 + got:t0 + got + e - a].tolist() == want
            got += e - a
        assert got == nt
        per_w[k] = nt
    assert at_seg == S and at_tile == T
    for (u, a, e, slot, *_) in segs:
        assert 0 <= u < U and 0 <= a < e <= ntile[u]
        covered[u][a:e] += 1
    assert all(np.all(c == 1) for c in covered), "a tile missing or covered twice"
    # one XCD per unit; even shares over each XCD's workers
    xcd = lambda k: (k // waves) % nx
    xcd_of = {}
    for (u, *_), k in zip(segs, seg_w):
        assert xcd_of.setdefault(int(u), xcd(k)) == xcd(k)
    for x in range(nx):
        share = per_w[[k for k in range(W) if xcd(k) == x]]
        assert share.max() - share.min() <= 1
    # pieces: a unit held by several segments; grouped, its pieces in one workgroup form a
    # group (consecutive in the workgroup's order: each wave's first, then last segment);
    # ungrouped, every piece is a group of its own
    nseg_u = np.bincount(segs[:, 0], minlength=U)
    groups = {}                                       # unit -> [(workgroup, [segments])]
    for g in range(G):
        order = []
        for w in range(waves):
            s0, ns = workers[g * waves + w][:2]
            ends = [s0] if ns == 1 else ([s0, s0 + ns - 1] if ns > 1 else [])
            for sg in range(s0, s0 + ns):
                u = segs[sg, 0]
                if sg not in ends:
                    assert nseg_u[u] == 1             # a worker's middle segments hold whole units
            order += [sg for sg in ends if nseg_u[segs[sg, 0]] > 1]
        for k, sg in enumerate(order):
            assert segs[sg, 5] == k                   # LDS index of the piece's state
            u = segs[sg, 0]
            if not group or k == 0 or segs[order[k - 1], 0] != u:
                groups.setdefault(int(u), []).append((g, [sg]))
            else:
                groups[int(u)][-1][1].append(sg)
    total = 0
    for u in range(U):
        mine = np.nonzero(segs[:, 0] == u)[0]
        np_u, base = units[u]
        if nseg_u[u] == 1:
            assert (np_u, base) == (0, -1) and segs[mine[0], 3] == -1 and segs[mine[0], 5] == -1
            continue
        gl = groups[u]
        assert sum(len(m) for _, m in gl) == len(mine)
        if group:
            assert len({g for g, _ in gl}) == len(gl)     # one group per workgroup
        slots = []
        for g, members in gl:
            lead, rest = members[0], members[1:]
            assert segs[lead, 6] == len(members) | (len(gl) << 8)
            assert all(segs[sg, 6] == 0 for sg in rest)
            assert len({segs[sg, 3] for sg in members}) == 1
            slots.append(int(segs[lead, 3]))
        if len(gl) == 1:
            assert (np_u, base) == (1, -1) and slots == [-1]
        else:
            assert np_u == len(gl) and sorted(slots) == list(range(base, base + np_u))
            assert all(segs[sg, 7] == base for sg in mine)
            total += np_u
    assert pieces == total
    return per_w, units


@pytest.mark.parametrize("seed", range(8))
def test_random_steps(seed):
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 80))
    ctx = rng.integers(1, 5000, B).tolist()
    hkv = int(rng.choice([1, 2, 8]))
    nx = int(rng.choice([1, 2, 8]))
    G = nx * int(rng.integers(1, 40))
    check(ctx, hkv, G, nx, waves=int(rng.choice([1, 4, 8])), bs=int(rng.choice([16, 32])), seed=seed,
          group=seed % 2 == 0)


def test_headline_shape_is_balanced_per_xcd():
    rng = np.random.default_rng(2)
    ctx = (rng.integers(512, 4097, 64) + 1).tolist()
    per_w, units = check(ctx, 2, 256, 8)
    # the XCDs' totals (longest first onto the least loaded) are within one unit of each other
    tot = [per_w[[k for k in range(len(per_w)) if (k // 4) % 8 == x]].sum() for x in range(8)]
    assert max(tot) - min(tot) <= max((c + 15) // 16 for c in ctx)


@pytest.mark.parametrize("bs", [16, 32, 64])
def test_block_sizes_gather_the_right_blocks(bs):
    check([1, 15, 16, 17, 100, 257, 1000], 2, 8, 2, bs=bs, seed=bs)


def test_tiny_contexts_many_units():
    check([1] * 300, 2, 64, 8)
    check([17, 1, 16, 33], 8, 256, 8)     # fewer tiles than workgroups: some workgroups idle


def test_limits_answered_with_more_workgroups():
    ctx = [30000] * 64
    st, _ = c_plan(ctx, 8, 256, 8, tmax=512)
    assert st == _lib.TB_ERR_UNSUPPORTED
    tables, nb = tables_for(ctx, 16)
    got = build_decode_plan(ctx, tables, block_size=16, num_blocks=nb, num_heads=32, num_kv_heads=8, head_dim=128,
                            workgroups=256, num_xcds=8)
    assert got is not None and got[1] > 256
    assert decode_limits(14, 2, 64) is not None and decode_limits(32, 2, 64) is None   # 16 heads per kv head


def test_bad_arguments():
    st, _ = c_plan([5, 0], 2, 8, 8, tables=np.zeros((2, 1), np.int32), nb=4)
    assert st == _lib.TB_ERR_INVALID_ARG                      # a context of 0 positions
    st, _ = c_plan([5], 2, 12, 8)
    assert st == _lib.TB_ERR_INVALID_ARG                      # workgroups not a multiple of the XCDs
    st, _ = c_plan([40], 2, 8, 8, tables=np.array([[0, 1]], np.int32), nb=4)
    assert st == _lib.TB_ERR_INVALID_ARG                      # more positions than the table row holds
    st, _ = c_plan([20], 2, 8, 8, tables=np.array([[0, 7]], np.int32), nb=4)
    assert st == _lib.TB_ERR_INDEX                            # a block outside the pool


def test_the_decode_kernel_is_chosen_for_large_decode_steps():
    """ops.decode_kernel_preferred: decode-only fp16 / bf16 steps of at least
    DECODE_KERNEL_MIN_BYTES of K/V (2 tensors x kv heads x head_dim x 2 bytes per position)."""
    import torch

    from tinybatch_amd import ops
    from tinybatch_amd.metadata import build_step_metadata

    def step(ctx, hkv=8, d=128, rows_are_seqs=True):
        tables, nb = tables_for(ctx, 16)
        pos = [c - 1 for c in ctx]
        slices = [(b, b + 1) for b in range(len(ctx))]
        if not rows_are_seqs:                   # one sequence with two rows: not a decode-only step
            pos = [ctx[0] - 2, ctx[0] - 1] + pos[1:]
            slices = [(0, 2)] + [(b + 1, b + 2) for b in range(1, len(ctx))]
        return build_step_metadata(pos, slices, tables, ctx, block_size=16, num_blocks=nb, partition_tokens=256)

    per_pos = 2 * 8 * 128 * 2
    at = ops.DECODE_KERNEL_MIN_BYTES // per_pos
    big = step([at // 4 + 1] * 4)
    small = step([at // 4 - 1] * 4)
    kw = dict(num_kv_heads=8, head_dim=128)
    assert ops.decode_kernel_preferred(big, dtype=torch.bfloat16, **kw)
    assert not ops.decode_kernel_preferred(small, dtype=torch.bfloat16, **kw)
    assert not ops.decode_kernel_preferred(big, dtype=torch.float32, **kw)
    assert not ops.decode_kernel_preferred(step([at // 4 + 1] * 4, rows_are_seqs=False), dtype=torch.float16, **kw)
