"""tb_build_decode_plan (host code, no GPU): every 16-position tile of every
(sequence, kv head) unit belongs to exactly one segment; all segments of a
unit belong to workgroups of one XCD (g % num_xcds); each XCD's workgroups
get equal shares of its tiles (within one tile); a unit held by one segment
writes its output directly (slot -1), a unit cut into several has one
distinct partial slot per segment, numbered from its first slot; limits are
reported as TB_ERR_UNSUPPORTED and answered with more workgroups."""
import ctypes

import numpy as np
import pytest

from tinybatch_amd import _lib
from tinybatch_amd.metadata import build_decode_plan, decode_limits


def c_plan(ctx, hkv, G, nx, tmax=1 << 20, smax=1 << 20):
    ctx = np.ascontiguousarray(ctx, dtype=np.int32)
    L = _lib.lib()
    nbytes = int(L.tb_decode_plan_bytes(len(ctx), hkv, G))
    plan = np.zeros(nbytes // 4, dtype=np.int32)
    st = L.tb_build_decode_plan(ctx.ctypes.data_as(ctypes.c_void_p), len(ctx), hkv, G, nx, tmax, smax,
                                plan.ctypes.data_as(ctypes.c_void_p), nbytes)
    return st, plan


def parse(plan):
    G, S, U, pieces, nx = (int(x) for x in plan[:5])
    wg_first = plan[8:8 + G + 1]
    off = 8 + (G + 1 + 3) // 4 * 4
    segs = plan[off:off + 4 * S].reshape(S, 4)
    units = plan[off + 4 * S:off + 4 * S + 2 * U].reshape(U, 2)
    return G, S, U, pieces, nx, wg_first, segs, units


def check(ctx, hkv, G, nx):
    st, plan = c_plan(ctx, hkv, G, nx)
    assert st == 0
    G_, S, U, pieces, nx_, wg_first, segs, units = parse(plan)
    assert (G_, U, nx_) == (G, len(ctx) * hkv, nx)
    tiles = [(c + 15) // 16 for c in ctx for _ in range(hkv)]
    covered = [np.zeros(t, dtype=np.int32) for t in tiles]
    seg_wg = np.zeros(S, dtype=np.int64)
    assert wg_first[0] == 0 and wg_first[G] == S and np.all(np.diff(wg_first) >= 0)
    for g in range(G):
        seg_wg[wg_first[g]:wg_first[g + 1]] = g
    per_wg = np.zeros(G, dtype=np.int64)
    for (u, t0, t1, slot), g in zip(segs, seg_wg):
        assert 0 <= u < U and 0 <= t0 < t1 <= tiles[u]
        covered[u][t0:t1] += 1
        per_wg[g] += t1 - t0
    assert all(np.all(c == 1) for c in covered), "a tile missing or covered twice"
    # one XCD per unit; even shares per XCD
    xcd_of = {}
    for (u, *_), g in zip(segs, seg_wg):
        assert xcd_of.setdefault(int(u), g % nx) == g % nx
    for x in range(nx):
        share = per_wg[x::nx]
        assert share.max() - share.min() <= 1
    # pieces and slots
    total = 0
    for u in range(U):
        mine = segs[segs[:, 0] == u]
        np_u, base = units[u]
        assert np_u == len(mine)
        if np_u == 1:
            assert base == -1 and mine[0, 3] == -1
        else:
            assert sorted(mine[:, 3].tolist()) == list(range(base, base + np_u))
            total += np_u
    assert pieces == total
    return per_wg, units


@pytest.mark.parametrize("seed", range(8))
def test_random_steps(seed):
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 80))
    ctx = rng.integers(1, 5000, B).tolist()
    hkv = int(rng.choice([1, 2, 8]))
    nx = int(rng.choice([1, 2, 8]))
    G = nx * int(rng.integers(1, 40))
    check(ctx, hkv, G, nx)


def test_headline_shape_is_balanced_per_xcd():
    rng = np.random.default_rng(2)
    ctx = (rng.integers(512, 4097, 64) + 1).tolist()
    per_wg, units = check(ctx, 2, 256, 8)
    # the XCDs' totals (longest first onto the least loaded) are within one unit of each other
    tot = [per_wg[x::8].sum() for x in range(8)]
    assert max(tot) - min(tot) <= max((c + 15) // 16 for c in ctx)


def test_tiny_contexts_many_units():
    check([1] * 300, 2, 64, 8)
    check([17, 1, 16, 33], 8, 256, 8)     # fewer tiles than workgroups: some workgroups idle


def test_limits_answered_with_more_workgroups():
    ctx = [30000] * 64
    st, _ = c_plan(ctx, 8, 256, 8, tmax=1024)
    assert st == _lib.TB_ERR_UNSUPPORTED
    got = build_decode_plan(ctx, 32, 8, 128, 256, 8)
    assert got is not None and got[1] > 256
    assert decode_limits(14, 2, 64) is not None and decode_limits(32, 2, 64) is None   # 16 heads per kv head


def test_bad_arguments():
    st, _ = c_plan([5, 0], 2, 8, 8)
    assert st == _lib.TB_ERR_INVALID_ARG                      # a context of 0 positions
    st, _ = c_plan([5], 2, 12, 8)
    assert st == _lib.TB_ERR_INVALID_ARG                      # workgroups not a multiple of the XCDs
