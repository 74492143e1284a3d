"""Host-side step metadata: slot mapping, work list and the reference's error behaviour."""
import numpy as np
import pytest
import torch

from tinybatch_amd.metadata import (TILE_PARTITION, TILE_ROWS, build_step_metadata, decode_staging_offsets,
                                    pack_decode_step, pack_step)


def _mixed():
    # seq0: prefill of 5 (ctx 5); seq1: decode at position 9 (ctx 10); seq2: tail prefill 3 of ctx 7
    positions = [0, 1, 2, 3, 4, 9, 4, 5, 6]
    slices = [(0, 5), (5, 6), (6, 9)]
    tables = [[7, 3], [1, 4, 0], [5, 6]]
    ctx = [5, 10, 7]
    return positions, slices, tables, ctx


def test_slot_mapping_follows_table_rule():
    pos, sl, tb, ctx = _mixed()
    m = build_step_metadata(pos, sl, tb, ctx, block_size=4, num_blocks=8, partition_tokens=64)
    want = []
    for (s, e), t in zip(sl, tb):
        for i in range(s, e):
            want.append(t[pos[i] // 4] * 4 + pos[i] % 4)
    assert m.slot_mapping_np.tolist() == want


def test_work_items_cover_every_row_and_partition():
    pos, sl, tb, ctx = _mixed()
    m = build_step_metadata(pos, sl, tb, ctx, block_size=4, num_blocks=8, partition_tokens=4)
    items = []
    for (s, e), c in zip(sl, ctx):
        n = e - s
        for i in range(n):
            row_ctx = c - n + i + 1
            for p in range((row_ctx + 3) // 4):
                items.append((s + i, sl.index((s, e)), p, row_ctx))
    got = [tuple(x) for x in m.work_np.tolist()]
    assert sorted(got) == sorted(items)
    # issued shortest partition first, row order among equals
    lengths = [min(4, rc - 4 * p) for _, _, p, rc in got]
    assert lengths == sorted(lengths)
    assert got == sorted(items, key=lambda it: min(4, it[3] - 4 * it[2]))
    counts = np.diff(m.row_part_off_np)
    for r in range(len(pos)):
        assert counts[r] == sum(1 for it in items if it[0] == r)
    assert m.max_parts_per_row == max(counts)
    assert not m.decode_only


def test_duplicate_slots_keep_the_last_writer():
    # two sequences rewrite the same slot (fully cached prompt sharing one block)
    m = build_step_metadata([3, 3], [(0, 1), (1, 2)], [[2], [2]], [4, 4], block_size=4, num_blocks=4,
                            partition_tokens=64)
    assert m.slot_mapping_np.tolist() == [-1, 11]


def test_short_table_raises_index_error_like_the_reference():
    with pytest.raises(IndexError):
        build_step_metadata([8], [(0, 1)], [[0, 1]], [9], block_size=4, num_blocks=4, partition_tokens=64)
    # write path alone (no context lengths) also checks the position
    with pytest.raises(IndexError):
        build_step_metadata([8], [(0, 1)], [[0, 1]], None, block_size=4, num_blocks=4, partition_tokens=64)


def test_block_outside_pool_raises_index_error():
    with pytest.raises(IndexError):
        build_step_metadata([0], [(0, 1)], [[9]], [1], block_size=4, num_blocks=4, partition_tokens=64)


def test_context_shorter_than_new_tokens_rejected():
    with pytest.raises(ValueError):
        build_step_metadata([0, 1], [(0, 2)], [[0]], [1], block_size=4, num_blocks=4, partition_tokens=64)


def test_decode_only_flag_and_device_tensor_positions():
    m = build_step_metadata(torch.tensor([5, 17]), [(0, 1), (1, 2)], [[0, 1], [2, 3, 4, 5, 6]], [6, 18],
                            block_size=4, num_blocks=8, partition_tokens=64)
    assert m.decode_only
    assert m.slot_mapping_np.tolist() == [1 * 4 + 1, 6 * 4 + 1]


def test_off_by_one_of_block_multiple_prompt_is_refused():
    """A 16-token prompt owns exactly one block of 16; its first decode writes
    position 16, which needs a second block (the engine must reserve it)."""
    with pytest.raises(IndexError):
        build_step_metadata([16], [(0, 1)], [[3]], [17], block_size=16, num_blocks=8, partition_tokens=256)


def test_row_groups_cover_each_row_partition_once():
    # seq0: 40-row prefill (ctx 40); seq1: decode; seq2: 9-row tail of ctx 70
    q = [40, 1, 9]
    ctx = [40, 77, 70]
    positions, slices, t = [], [], 0
    for n, c in zip(q, ctx):
        positions += list(range(c - n, c))
        slices.append((t, t + n)); t += n
    tables = [list(range(0, 3)), list(range(3, 8)), list(range(8, 13))]
    m = build_step_metadata(positions, slices, tables, ctx, block_size=16, num_blocks=16,
                            partition_tokens=32, rows_per_item=4)
    seen = {}
    for row0, seq, z, rc in m.work_np.tolist():
        part, nrows = z & 0xFFFFFF, (z >> 24) + 1
        assert 1 <= nrows <= 4
        s, e = slices[seq]
        assert s <= row0 and row0 + nrows <= e
        parts = {-(-(m.row_ctx_np[r]) // 32) for r in range(row0, row0 + nrows)}
        assert len(parts) == 1                               # equal partition counts in a group
        for i in range(nrows):
            assert m.row_ctx_np[row0 + i] == rc + i
            seen[(row0 + i, part)] = seen.get((row0 + i, part), 0) + 1
    want = {(r, p) for r in range(t) for p in range(-(-int(m.row_ctx_np[r]) // 32))}
    assert set(seen) == want and all(v == 1 for v in seen.values())
    assert m.total_partitions == len(want)


def test_prefill_tiles_cover_tiled_rows_most_positions_first():
    # seq0: prefill 150 (tiles 64, 64, 22); seq1: decode; seq2: tail 20 of ctx 520; seq3: tail 8 (row groups)
    q = [150, 1, 20, 8]
    ctx = [150, 33, 520, 300]
    positions, slices, t = [], [], 0
    for n, c in zip(q, ctx):
        positions += list(range(c - n, c))
        slices.append((t, t + n)); t += n
    need = [(c + 15) // 16 for c in ctx]
    tables, at = [], 0
    for n in need:
        tables.append(list(range(at, at + n))); at += n
    P, TP = 256, TILE_PARTITION
    m = build_step_metadata(positions, slices, tables, ctx, block_size=16, num_blocks=at,
                            partition_tokens=P, rows_per_item=2, tile_prefill=True)
    items = [tuple(x) for x in m.prefill_tiles_np.tolist()]
    want = [(0, 0, 64, 0), (64, 0, 64, 64), (128, 0, 22, 128), (151, 2, 20, 500)]
    assert sorted(items) == sorted(want)
    covered = [min(TP, p0 + (z & 0xFF) - (z >> 8) * TP) for _, _, z, p0 in items]
    assert covered == sorted(covered, reverse=True)
    tiled = {r for r0, _, z, _ in items for r in range(r0, r0 + (z & 0xFF))}
    worked = {int(r) + i for r, _, z, _ in m.work_np.tolist() for i in range((z >> 24) + 1)}
    assert tiled.isdisjoint(worked) and tiled | worked == set(range(t))
    counts = np.diff(m.row_part_off_np)
    for r in range(t):   # tile rows count tile partitions, work-item rows count P-position ones
        assert counts[r] == -(-int(m.row_ctx_np[r]) // (TP if r in tiled else P))
    assert m.total_partitions == int(counts.sum())
    assert m.split_rows_np[:, 0].tolist() == [r for r in range(t) if counts[r] > 1]
    for r, pbeg, n, z in m.split_rows_np.tolist():   # combine records: first slot and count
        assert (pbeg, n, z) == (m.row_part_off_np[r], counts[r], 0)
    # fp32 metadata (no tiles) keeps every row in work items
    m32 = build_step_metadata(positions, slices, tables, ctx, block_size=16, num_blocks=at,
                              partition_tokens=P)
    assert m32.num_prefill_tiles == 0 and m32.num_work_items == m32.total_partitions


def test_tile_constants_match_the_header():
    import os
    import re
    hdr = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                            "tinybatch_amd.h")).read()
    assert int(re.search(r"#define TB_PREFILL_TILE_ROWS (\d+)", hdr).group(1)) == TILE_ROWS
    assert int(re.search(r"#define TB_PREFILL_TILE_PARTITION (\d+)", hdr).group(1)) == TILE_PARTITION


def test_long_prefill_tiles_span_tile_partitions():
    n = 2100
    m = build_step_metadata(list(range(n)), [(0, n)], [list(range((n + 15) // 16))], [n], block_size=16,
                            num_blocks=200, partition_tokens=256, rows_per_item=2, tile_prefill=True)
    items = m.prefill_tiles_np.tolist()
    ntiles = -(-n // TILE_ROWS)
    want = sum(-(-min(n, 64 * (t + 1)) // TILE_PARTITION) for t in range(ntiles))
    assert len(items) == want
    assert m.max_parts_per_row == 3
    assert m.split_rows_np[:, 0].tolist() == [r for r in range(n) if r + 1 > TILE_PARTITION]


def _decode_case(rng, B, BS, NB, extra_blocks=0):
    ctx = [int(c) for c in rng.integers(1, 3000, B)]
    ctx[:4] = [1, BS, BS + 1, 256][:B]
    perm = rng.permutation(NB).tolist()
    tables, at = [], 0
    for c in ctx:
        nb = (c + BS - 1) // BS + int(rng.integers(0, extra_blocks + 1))   # reserved blocks past the context
        tables.append(perm[at:at + nb]); at += nb
    return ctx, tables


def _read_parts(h, o, Bp, max_nb, ctx, BS):
    """What the kernels read of a packed decode step: every slot, the table entries
    inside each context, the work items, offsets, split rows and counts."""
    W, S = int(h[o[5]]), int(h[o[5] + 1])
    tab = h[o[1]:o[1] + Bp * max_nb].reshape(Bp, max_nb)
    used = [tab[b, :(c + BS - 1) // BS].tolist() for b, c in enumerate(ctx)]
    return (h[o[0]:o[0] + Bp].tolist(), used, h[o[2]:o[2] + 4 * W].tolist(), h[o[3]:o[3] + Bp + 1].tolist(),
            h[o[4]:o[4] + 4 * S].tolist(), h[o[5]:o[5] + 4].tolist())


@pytest.mark.parametrize("BS,B,Bp", [(16, 32, 32), (16, 5, 8), (4, 9, 16), (32, 1, 1), (8, 64, 96)])
def test_pack_decode_step_matches_the_general_builder(BS, B, Bp):
    """The decode fast path writes what build_step_metadata + pack_step write
    (stale staging contents beneath), work items in the same order."""
    rng = np.random.default_rng(BS * 1000 + B)
    NB, P, max_len = 16384, 256, 4096
    max_nb, max_parts = max_len // BS, max_len // P
    ctx, tables = _decode_case(rng, B, BS, NB, extra_blocks=2)
    o = decode_staging_offsets(Bp, max_nb, max_parts)
    fast = rng.integers(-5, 10**6, int(o[-1])).astype(np.int32)       # stale contents
    ref = fast.copy()
    assert pack_decode_step(fast, o, Bp, max_nb, ctx, tables, block_size=BS, num_blocks=NB, partition_tokens=P)
    meta = build_step_metadata([c - 1 for c in ctx], [(i, i + 1) for i in range(B)], tables, ctx,
                               block_size=BS, num_blocks=NB, partition_tokens=P)
    pack_step(ref, o, Bp, max_nb, meta)
    assert _read_parts(fast, o, Bp, max_nb, ctx, BS) == _read_parts(ref, o, Bp, max_nb, ctx, BS)


def test_pack_decode_step_rejects_what_the_builder_rejects():
    o = decode_staging_offsets(4, 8, 2)
    h = np.zeros(int(o[-1]), np.int32)
    kw = dict(block_size=16, num_blocks=10, partition_tokens=256)
    with pytest.raises(IndexError):                      # table shorter than the context
        pack_decode_step(h, o, 4, 8, [17], [[3]], **kw)
    with pytest.raises(IndexError):                      # block outside the pool
        pack_decode_step(h, o, 4, 8, [5], [[10]], **kw)
    with pytest.raises(IndexError):
        pack_decode_step(h, o, 4, 8, [5], [[-1]], **kw)
    with pytest.raises(ValueError):                      # no position to attend to
        pack_decode_step(h, o, 4, 8, [0], [[1]], **kw)
    with pytest.raises(ValueError):                      # longer than the staging tables
        pack_decode_step(h, o, 4, 8, [129], [list(range(9))], **dict(kw, num_blocks=20))
    # two rows writing one slot: left to the general builder's last-writer rule
    assert not pack_decode_step(h, o, 4, 8, [5, 5], [[2], [2]], **kw)


def _split_case(order="pre-dec"):
    # two whole prefills (64 and 33 new rows) and three decode rows, in row order
    BS = 16
    pre = [(64, [1, 2, 3, 4]), (33, [5, 6, 7])]
    dec = [(40, [8, 9, 10]), (17, [11, 12]), (100, [13, 14, 15, 16, 17, 18, 19])]
    seqs = pre + [("d", c, t) for c, t in dec] if order == "pre-dec" else [("d", c, t) for c, t in dec] + pre
    positions, slices, tables, ctx, r = [], [], [], [], 0
    for s in seqs:
        if s[0] == "d":
            _, c, t = s
            positions.append(c - 1)
            slices.append((r, r + 1))
            r += 1
        else:
            n, t = s
            c = n
            positions.extend(range(n))
            slices.append((r, r + n))
            r += n
        tables.append(t)
        ctx.append(c)
    return positions, slices, tables, ctx, BS


@pytest.mark.parametrize("order", ["pre-dec", "dec-pre"])
def test_split_step_parts_rebase_each_side(order):
    from tinybatch_amd.metadata import PrefillRoute, split_step_parts

    positions, slices, tables, ctx, BS = _split_case(order)
    route = PrefillRoute(num_kv_heads=2, head_dim=64, max_context=560)
    parts = split_step_parts(positions, slices, tables, ctx, block_size=BS, num_blocks=32, partition_tokens=256,
                             rows_per_item=2, prefill_route=route)
    assert parts is not None and len(parts) == 2
    T = len(positions)
    assert parts[0][0] == 0 and parts[-1][1] == T and parts[0][1] == parts[1][0]   # the rows, once each
    full = build_step_metadata(positions, slices, tables, ctx, block_size=BS, num_blocks=32, partition_tokens=256)
    for r0, r1, m in parts:
        assert m.num_tokens == r1 - r0
        # the sub-step's slots are the whole step's slots of the same rows
        assert np.array_equal(m.slot_mapping_np, full.slot_mapping_np[r0:r1])
        if m.decode_only:
            assert m.rows_are_seqs and m.num_seqs == 3
            assert np.array_equal(m.row_ctx_np, full.row_ctx_np[r0:r1])
        else:
            assert m.num_work_items == 0 and m.num_prefill_tiles == 0 and m.num_prefill_work > 0


def test_split_step_parts_refuse_other_shapes():
    from tinybatch_amd.metadata import PrefillRoute, split_step_parts

    positions, slices, tables, ctx, BS = _split_case()
    kw = dict(block_size=BS, num_blocks=32, partition_tokens=256, rows_per_item=2)
    route = PrefillRoute(num_kv_heads=2, head_dim=64, max_context=560)
    # a prefill longer than the kernel serves
    assert split_step_parts(positions, slices, tables, ctx, prefill_route=route._replace(max_context=48), **kw) is None
    # decode rows on both sides of the prefills
    p2, s2, t2, c2, _ = _split_case()
    order = [2, 0, 1, 3, 4]
    rows, sl, r = [], [], 0
    for i in order:
        b, e = s2[i]
        rows.extend(p2[b:e])
        sl.append((r, r + e - b))
        r += e - b
    assert split_step_parts(rows, sl, [t2[i] for i in order], [c2[i] for i in order], prefill_route=route,
                            **kw) is None
    # a short tail of new rows (not a whole prefill, not a decode row)
    assert split_step_parts(positions[:67] + [70, 71] + positions[97:], [(0, 64), (64, 67)] + [(67, 69)] +
                            [(69 + i, 70 + i) for i in range(3)], [tables[0], tables[1], [20, 21, 22, 23, 24]] +
                            tables[2:], [64, 3, 72] + ctx[2:], prefill_route=route, **kw) is None
    # no decode rows, or no prefills: nothing to split
    assert split_step_parts(positions[:97], slices[:2], tables[:2], ctx[:2], prefill_route=route, **kw) is None
    assert split_step_parts(positions[97:], [(i, i + 1) for i in range(3)], tables[2:], ctx[2:],
                            prefill_route=route, **kw) is None
