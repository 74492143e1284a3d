"""tb_build_step_metadata (the C ABI's host-side builder) against
metadata.build_step_metadata: the same arrays, bit for bit, on the shapes of
the fp32 and fp16 decode workloads, the Llama-geometry decode, the mixed step
with prefill tiles, and seeded random steps (prefill tails, decode rows,
grouped rows, shared and repeated written blocks, rows outside every
sequence). No GPU: the builder is host code."""
import ctypes

import numpy as np
import pytest
import torch

from tinybatch_amd import _lib
from tinybatch_amd.metadata import build_step_metadata
from tinybatch_amd.workloads import SPECS, _cached_lengths, make_decode_workload, make_mixed_workload


def _i32(a):
    a = np.ascontiguousarray(a, dtype=np.int32)
    return a, a.ctypes.data_as(ctypes.c_void_p)


def c_build(qlens, ctx, tables, num_blocks, bs, P, rows=1, tiles=False, num_tokens=None, positions=None,
            caps=None):
    B = len(qlens)
    qsl = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    T = int(qsl[-1]) if num_tokens is None else num_tokens
    max_nb = max(1, max((len(t) for t in tables), default=1))
    tab = np.zeros((max(B, 1), max_nb), dtype=np.int32)
    for b, t in enumerate(tables):
        tab[b, :len(t)] = t
    L = _lib.lib()
    counts = np.zeros(5, dtype=np.int64)
    qsl_a, qsl_p = _i32(qsl)
    ctx_a, ctx_p = _i32(ctx if B else [0])
    st = L.tb_step_metadata_counts(qsl_p, B, ctx_p, T, bs, P, rows, int(tiles), counts.ctypes.data_as(ctypes.c_void_p))
    if st != 0:
        return st, None
    W, N, S = (int(x) for x in counts[:3])
    cw, cn, cs = caps or (W, N, S)
    slot = np.zeros(T, np.int32)
    rpo = np.zeros(T + 1, np.int32)
    work = np.zeros((max(cw, 1), 4), np.int32)
    tl = np.zeros((max(cn, 1), 4), np.int32)
    sp = np.zeros((max(cs, 1), 4), np.int32)
    counts2 = np.zeros(6, dtype=np.int64)
    pos_p = None
    if positions is not None:
        pos_a = np.ascontiguousarray(positions, dtype=np.int64)
        pos_p = pos_a.ctypes.data_as(ctypes.c_void_p)
    vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    st = L.tb_build_step_metadata(qsl_p, B, ctx_p, pos_p, T, vp(tab), max_nb, num_blocks, bs, P, rows, int(tiles),
                                  vp(slot), vp(rpo), vp(work), cw, vp(tl), cn, vp(sp), cs, vp(counts2))
    return st, dict(slot=slot, rpo=rpo, work=work[:W], tiles=tl[:N], split=sp[:S], counts=counts2)


def compare(qlens, ctx, tables, num_blocks, bs, P, rows=1, tiles=False, num_tokens=None):
    pos, slices, at = [], [], 0
    for n, c in zip(qlens, ctx):
        slices.append((at, at + n))
        pos.extend(range(c - n, c))
        at += n
    T = at if num_tokens is None else num_tokens
    pos_full = pos + [0] * (T - len(pos))
    m = build_step_metadata(pos_full, slices, tables, ctx, block_size=bs, num_blocks=num_blocks,
                            partition_tokens=P, rows_per_item=rows, tile_prefill=tiles, num_tokens=T)
    st, got = c_build(qlens, ctx, tables, num_blocks, bs, P, rows, tiles, num_tokens=T,
                      positions=pos_full)
    assert st == 0
    np.testing.assert_array_equal(got["slot"], m.slot_mapping_np)
    np.testing.assert_array_equal(got["rpo"], m.row_part_off_np)
    np.testing.assert_array_equal(got["work"], m.work_np.reshape(-1, 4))
    np.testing.assert_array_equal(got["tiles"], m.prefill_tiles_np.reshape(-1, 4))
    np.testing.assert_array_equal(got["split"], m.split_rows_np.reshape(-1, 4))
    superseded = sum(int(m.slot_mapping_np[r] < 0) for b, e in slices for r in range(b, e))
    assert got["counts"].tolist() == [m.num_work_items, m.num_prefill_tiles, m.num_split_rows,
                                      m.total_partitions, m.max_parts_per_row, superseded]
    return m


@pytest.mark.parametrize("name,P", [("qwen-fp32-b8", 64), ("qwen-fp32-b8", 256), ("qwen-fp16-b64", 256)])
def test_decode_workloads(name, P):
    wl = make_decode_workload(name)
    compare([1] * wl.batch, wl.context_lens, wl.block_tables, wl.num_blocks, wl.block_size, P)


def test_llama_geometry_decode_tables():
    spec = SPECS["llama-bf16-b256"]
    gen = torch.Generator().manual_seed(spec["seed"])
    cached = _cached_lengths(gen, spec["B"], spec["lens"])
    need = [(c + 1 + 15) // 16 for c in cached]
    perm = torch.randperm(sum(need), generator=gen).tolist()
    tables, at = [], 0
    for n in need:
        tables.append(perm[at:at + n])
        at += n
    m = compare([1] * len(cached), [c + 1 for c in cached], tables, sum(need), 16, 256)
    assert m.num_work_items > 8000


@pytest.mark.parametrize("rows,tiles", [(2, True), (2, False), (1, True)])
def test_mixed_step(rows, tiles):
    wl = make_mixed_workload()
    m = compare(wl.q_lens, wl.context_lens, wl.block_tables, wl.num_blocks, wl.block_size, 256, rows, tiles)
    assert (m.num_prefill_tiles > 0) == tiles


@pytest.mark.parametrize("seed", range(12))
def test_random_steps(seed):
    rng = np.random.default_rng(seed)
    bs = int(rng.choice([4, 8, 16, 32, 64]))
    P = bs * int(rng.integers(1, 9)) * (4 if bs <= 8 else 1)
    B = int(rng.integers(1, 12))
    qlens, ctx = [], []
    for _ in range(B):
        kind = rng.integers(0, 4)
        if kind == 0:                      # decode row
            q, c = 1, int(rng.integers(1, 600))
        elif kind == 1:                    # whole prompt
            q = int(rng.integers(1, 300)); c = q
        elif kind == 2:                    # cached-prefix tail
            q = int(rng.integers(1, 120)); c = q + int(rng.integers(0, 700))
        else:                              # no rows this step
            q, c = 0, int(rng.integers(1, 50))
        qlens.append(q)
        ctx.append(c)
    need = [(c + bs - 1) // bs for c in ctx]
    NB = sum(need) + 8
    perm = rng.permutation(NB).tolist()
    tables, at = [], 0
    for n in need:
        tables.append(perm[at:at + n] + perm[:int(rng.integers(0, 3))])   # some padding entries
        at += n
    # shared written blocks: another sequence's newest block (last writer wins)
    for _ in range(int(rng.integers(0, 3))):
        a, b = rng.integers(0, B, 2)
        if a != b and qlens[a] and qlens[b]:
            tables[b][(ctx[b] - 1) // bs] = tables[a][(ctx[a] - 1) // bs]
    # a table that names one block twice among its written positions
    b = int(rng.integers(0, B))
    if qlens[b] and (ctx[b] - 1) // bs > (ctx[b] - qlens[b]) // bs:
        tables[b][(ctx[b] - 1) // bs] = tables[b][(ctx[b] - qlens[b]) // bs]
    rows = int(rng.choice([1, 2, 4, 16]))
    extra = int(rng.integers(0, 3))
    compare(qlens, ctx, tables, NB, bs, P, rows, bool(rng.integers(0, 2)), num_tokens=sum(qlens) + extra)


def test_shared_written_slot_keeps_the_last_writer():
    m = compare([1, 1, 1], [20, 40, 36], [[3, 6], [1, 2, 4], [0, 5, 6]], 12, 16, 256)
    assert m.slot_mapping_np.tolist() == [-1, 4 * 16 + 7, 6 * 16 + 3]


def test_errors_mirror_the_reference():
    # a table shorter than its context: IndexError in the reference (kv_cache.py:35)
    st, _ = c_build([1], [40], [[1, 2]], 8, 16, 256)
    assert st == _lib.TB_ERR_INDEX
    # a block id outside the pool
    st, _ = c_build([1], [20], [[1, 9]], 8, 16, 256)
    assert st == _lib.TB_ERR_INDEX
    # positions that are not ctx - q_len + i
    st, _ = c_build([2], [20], [[1, 2]], 8, 16, 256, positions=[18, 18])
    assert st == _lib.TB_ERR_INVALID_ARG
    # a context shorter than the new rows
    st, _ = c_build([3], [2], [[1]], 8, 16, 256)
    assert st == _lib.TB_ERR_INVALID_ARG
    # capacities below the counts: rejected, counts still reported
    st, got = c_build([1, 1], [300, 600], [[0] * 19, [1] * 38], 8, 16, 256, caps=(1, 0, 2))
    assert st == _lib.TB_ERR_INVALID_ARG and got["counts"][0] == 5


def test_superseded_rows_are_counted():
    # two decode rows whose newest positions share one slot (block 3 offset 4 in both
    # tables): the first row's slot is -1 and counts[5] reports it, the sign a fused
    # append cannot serve the step (the reference lets the last writer win,
    # kv_cache.py:33-38)
    st, got = c_build([1, 1], [21, 21], [[0, 3], [1, 3]], 8, 16, 256)
    assert st == 0
    assert got["slot"].tolist() == [-1, 3 * 16 + 4]
    assert int(got["counts"][5]) == 1
    # distinct slots: nothing superseded
    st, got = c_build([1, 1], [21, 21], [[0, 3], [1, 2]], 8, 16, 256)
    assert st == 0 and int(got["counts"][5]) == 0
