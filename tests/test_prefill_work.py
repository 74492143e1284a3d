"""tb_build_prefill_work (host code, no GPU): every (sequence, kv head, pair of
16-row blocks p and nb-1-p) appears exactly once, with the sequence's first row,
index, pos0 and new rows; the entries of one (sequence, kv head) sit at list
positions of one residue modulo the XCD count (while the list allows) and the
XCDs' loads are even; the most tiles one entry holds is the later block's range;
contexts past the kernel's limit and bad rows are refused; metadata routing takes
whole prefill sequences out of tiles, work items and partition slots."""
import numpy as np
import pytest
import torch

from tinybatch_amd import ops
from tinybatch_amd.metadata import PrefillRoute, build_prefill_work, build_step_metadata


def check(first, seqs, pos0, rows, hkv, xcds):
    work, tiles = build_prefill_work(first, seqs, pos0, rows, num_kv_heads=hkv, head_dim=64, num_xcds=xcds)
    want = set()
    for f, s, p0, n in zip(first, seqs, pos0, rows):
        nb = (n + 15) // 16
        for p in range((nb + 1) // 2):
            for h in range(hkv):
                want.add((f, s, p0, n | (p << 16) | (h << 24)))
    got = [tuple(int(x) for x in w) for w in work]
    assert len(got) == len(want) and set(got) == want
    # the largest range: positions 0 .. the later block's last row
    rng = max(p0 + min(n, 16 * ((n + 15) // 16 - ((w >> 16) & 0xFF))) for (_, _, p0, w), n in
              ((g, g[3] & 0xFFFF) for g in got))
    assert tiles == (rng + 15) // 16
    return got


def test_every_pair_once_and_xcd_groups():
    rng = np.random.default_rng(0)
    B = 12
    rows = rng.integers(16, 500, B).tolist()
    pos0 = rng.integers(0, 40, B).tolist()
    first = np.concatenate([[0], np.cumsum(rows)[:-1]]).tolist()
    got = check(first, list(range(B)), pos0, rows, 2, 8)
    # a (sequence, kv head)'s entries share a residue mod 8 except where a lent slot broke it
    res = {}
    for i, (_, s, _, w) in enumerate(got):
        res.setdefault((s, (w >> 24) & 0x7F), []).append(i % 8)
    kept = sum(max(np.bincount(v)) for v in res.values())
    assert kept >= 0.85 * len(got)


def test_one_xcd_and_lone_middle_blocks():
    got = check([0, 33, 50], [0, 1, 2], [0, 7, 100], [33, 17, 16], 4, 1)
    assert len(got) == (2 + 1 + 1) * 4


def test_the_headline_prefill_step_lands_whole_groups_on_xcds():
    rows = [512] * 8
    first = [512 * i for i in range(8)]
    got = check(first, list(range(8)), [0] * 8, rows, 2, 8)
    assert len(got) == 256
    for key in {(s, (w >> 24) & 0x7F) for _, s, _, w in got}:
        idx = [i for i, (_, s, _, w) in enumerate(got) if (s, (w >> 24) & 0x7F) == key]
        assert len({i % 8 for i in idx}) == 1       # 16 workgroups of one sequence and kv head: one XCD


def test_limits_and_bad_rows():
    lim = 16 * 35                                    # 36 tiles of LDS at head dim 64, one spare
    build_prefill_work([0], [0], [lim - 100], [100], num_kv_heads=2, head_dim=64)
    with pytest.raises(RuntimeError):
        build_prefill_work([0], [0], [lim - 99], [100], num_kv_heads=2, head_dim=64)
    with pytest.raises(ValueError):
        build_prefill_work([0], [0], [0], [0], num_kv_heads=2, head_dim=64)
    with pytest.raises(RuntimeError):
        build_prefill_work([0], [0], [0], [16], num_kv_heads=2, head_dim=96)


def test_metadata_routes_whole_prefill_sequences():
    # two prefills (one past the limit keeps its tiles), one decode row
    route = PrefillRoute(num_kv_heads=2, head_dim=64, max_context=560, num_xcds=8)
    q_lens, cached = [100, 600, 1], [20, 0, 300]
    tables, at, slices, t, pos = [], 0, [], 0, []
    for n, c in zip(q_lens, cached):
        nb = (c + n + 15) // 16
        tables.append(list(range(at, at + nb)))
        at += nb
        slices.append((t, t + n))
        t += n
        pos.extend(range(c, c + n))
    ctx = [c + n for c, n in zip(cached, q_lens)]
    meta = build_step_metadata(pos, slices, tables, ctx, block_size=16, num_blocks=at, partition_tokens=256,
                               tile_prefill=True, prefill_route=route)
    assert meta.num_prefill_work == 4 * 2            # 7 blocks -> 4 pairs, 2 kv heads
    assert int(meta.prefill_work_np[:, 0].max()) == 0 and int(meta.prefill_work_np[:, 2].max()) == 20
    assert meta.num_prefill_tiles > 0                # the 600-row sequence
    assert all(int(r) != 0 for r in meta.prefill_tiles_np[:, 1])   # no tile of sequence 0
    assert np.all(meta.row_part_off_np[1:101] == 0)  # its rows own no partition slots
    rows_in_items = set(int(w[0]) for w in meta.work_np)
    assert rows_in_items == {700}                    # the decode row only
    assert ops.prefill_route(torch.float32, 14, 2, 64) is None
    assert ops.prefill_route(torch.bfloat16, 18, 2, 64) is None   # 9 query heads per kv head
