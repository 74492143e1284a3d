"""Block-table contract of the host BlockManager (the reference's
tests/test_block_manager.py scenarios, restated) plus compaction."""
import pytest

from tinybatch_amd.block_manager import BlockManager, OutOfBlocks


def bm_(num_blocks=8, block_size=4, prefix=True):
    return BlockManager(num_blocks, block_size, enable_prefix_caching=prefix)


def test_prompt_takes_ceil_blocks_lifo_from_the_top():
    bm = bm_()
    table, cached = bm.allocate_prompt(list(range(10)))
    assert table == [7, 6, 5] and cached == 0          # free ids are popped from the end
    assert bm.num_free() == 5


def test_free_returns_uncached_blocks():
    bm = bm_(prefix=False)
    table, _ = bm.allocate_prompt(list(range(10)))
    bm.free_table(table)
    assert bm.num_free() == 8


def test_exhausted_pool_raises():
    with pytest.raises(OutOfBlocks):
        bm_(num_blocks=2, prefix=False).allocate_prompt(list(range(100)))


def test_append_slot_grows_only_at_block_boundaries():
    bm = bm_()
    seq = list(range(4))
    table, _ = bm.allocate_prompt(seq)
    assert bm.append_slot(table, seq) and len(table) == 2     # index 4 opens block 2
    seq.append(9)
    assert not bm.append_slot(table, seq) and len(table) == 2


def test_prefix_hit_shares_physical_blocks():
    bm = bm_()
    t1, c1 = bm.allocate_prompt(list(range(8)))
    t2, c2 = bm.allocate_prompt(list(range(8)) + [50, 51])
    assert (c1, c2) == (0, 8) and t2[:2] == t1[:2]
    assert bm.blocks[t1[0]].ref_count == 2 and bm.hit_rate() == 2 / 4


def test_prefix_match_stops_at_first_divergent_block():
    bm = bm_()
    bm.allocate_prompt([1, 2, 3, 4, 5, 6, 7, 8])
    assert bm.allocate_prompt([1, 2, 3, 4, 0, 0, 0, 0])[1] == 4
    # a later block equal to a cached one does not match once the prefix broke
    assert bm.allocate_prompt([0, 0, 0, 0, 5, 6, 7, 8])[1] == 0


def test_shared_block_survives_until_last_owner_frees():
    bm = bm_()
    t1, _ = bm.allocate_prompt(list(range(8)))
    t2, _ = bm.allocate_prompt(list(range(8)))
    bm.free_table(t1)
    assert bm.blocks[t1[0]].ref_count == 1
    bm.free_table(t2)
    assert bm.blocks[t1[0]].ref_count == 0
    with pytest.raises(AssertionError):
        bm.free_table(t2)                                    # double free


def test_unreferenced_cached_blocks_are_evicted_lru():
    bm = bm_(num_blocks=4)
    t1, _ = bm.allocate_prompt(list(range(8)))
    bm.free_table(t1)
    assert bm.num_free() == 4                                # evictable counts as free
    t2, cached = bm.allocate_prompt(list(range(100, 116)))
    assert len(t2) == 4 and cached == 0
    bm.free_table(t2)
    assert bm.allocate_prompt(list(range(8)))[1] == 0        # the old prefix is gone


def test_disabled_prefix_cache_never_hits():
    bm = bm_(prefix=False)
    bm.allocate_prompt(list(range(8)))
    assert bm.allocate_prompt(list(range(8)))[1] == 0


def test_block_filled_by_decode_is_published():
    bm = bm_()
    seq = [1, 2, 3]
    table, _ = bm.allocate_prompt(seq)
    for tok in (4, 5):
        bm.append_slot(table, seq)
        seq.append(tok)
    assert bm.allocate_prompt([1, 2, 3, 4, 9])[1] == 4


def test_compact_moves_live_blocks_down_and_remaps_tables_and_cache():
    bm = bm_(num_blocks=16)
    a, _ = bm.allocate_prompt(list(range(8)))            # ids 15, 14 (cached)
    b, _ = bm.allocate_prompt(list(range(100, 106)))     # ids 13, 12
    c, _ = bm.allocate_prompt(list(range(200, 210)))     # ids 11, 10, 9
    bm.free_table(b)                                      # 13 cached -> evictable; 12 (partial) -> free
    before = {tuple(t) for t in (a, c)}
    src, dst = bm.compact([a, c])
    live = sorted(set(a) | set(c) | {bid for bid in bm.evictable})
    assert live == list(range(len(live)))                 # dense at the bottom
    assert len(src) == len(dst) and not set(src) & set(dst)
    assert all(d < len(live) for d in dst)
    # the tables still describe the same blocks (through the copy)
    m = dict(zip(src, dst))
    assert {tuple(m.get(x, x) for x in t) for t in before} == {tuple(a), tuple(c)}
    # the prefix cache follows the moved blocks
    assert bm.allocate_prompt(list(range(8)))[0][:2] == a[:2]
    # allocation continues right above the live blocks
    t, _ = bm.allocate_prompt([7])
    assert t == [len(live)]
