"""tb_build_xcd_slot_map (host code, no GPU): the grid of tb_paged_attention_merged.
Every (work item, kv head) appears in exactly one slot; every item of a row
group (the items sharing their first row) of one kv head sits in slots of one
XCD (slot s on XCD s % num_xcds), in item order; the rest hold -1; the XCDs'
item counts differ by at most the largest row group."""
import numpy as np
import pytest

from tinybatch_amd.metadata import build_step_metadata, build_xcd_slot_map


def check(work, n, hkv, nx):
    m = build_xcd_slot_map(work, n, hkv, nx)
    assert m.size % nx == 0
    vals = m[m >= 0]
    assert sorted(vals.tolist()) == list(range(n * hkv))
    xcd_of = {}
    first_row = np.asarray(work)[:n, 0]
    per_x = np.zeros(nx, dtype=np.int64)
    last_in_x = [-1] * nx
    for s, v in enumerate(m.tolist()):
        if v < 0:
            continue
        x = s % nx
        item, kvh = divmod(v, hkv)
        assert xcd_of.setdefault((int(first_row[item]), kvh), x) == x
        assert v > last_in_x[x]                   # ascending within an XCD
        last_in_x[x] = v
        per_x[x] += 1
    group = np.bincount(first_row).max() if n else 0
    assert per_x.max() - per_x.min() <= group
    assert m.size == nx * per_x.max()
    return m


def decode_step(ctx, bs=16, P=256):
    need = [(c + bs - 1) // bs for c in ctx]
    tables = np.zeros((len(ctx), max(need)), dtype=np.int32)
    at = 0
    for b, k in enumerate(need):
        tables[b, :k] = np.arange(at, at + k)
        at += k
    return build_step_metadata([c - 1 for c in ctx], [(b, b + 1) for b in range(len(ctx))], tables, ctx,
                               block_size=bs, num_blocks=at + 1, partition_tokens=P)


@pytest.mark.parametrize("seed", range(6))
def test_random_decode_steps(seed):
    rng = np.random.default_rng(seed)
    ctx = rng.integers(1, 5000, int(rng.integers(1, 90))).tolist()
    meta = decode_step(ctx)
    for hkv in (1, 2, 8):
        for nx in (1, 4, 8):
            check(meta.work_np, meta.num_work_items, hkv, nx)


def test_headline_shape_balance():
    rng = np.random.default_rng(1)
    meta = decode_step((rng.integers(512, 4097, 64) + 1).tolist())
    m = check(meta.work_np, meta.num_work_items, 2, 8)
    assert m.size <= 8 * (-(-meta.num_work_items * 2 // 8) + 2)     # within two items of perfect balance


def test_items_out_of_row_order_and_empty():
    w = np.array([[5, 0, 1, 9], [2, 0, 0, 9], [5, 0, 0, 9], [2, 0, 1, 9]], dtype=np.int32)
    check(w, 4, 2, 8)
    assert build_xcd_slot_map(np.zeros((0, 4), np.int32), 0, 2, 8).size == 0


def test_attach_refuses_rows_of_more_than_255_partitions():
    """The merged launch counts a row's partitions in 8-bit per-XCD fields: a step with a
    row of 256 or more partitions gets no slot map (its split rows go to the combine
    kernel), one of 255 does."""
    import torch

    from tinybatch_amd.metadata import attach_xcd_slot_map

    for ctx, want in ((256 * 255, True), (256 * 255 + 1, False), (256 * 400, False)):
        blocks = (ctx + 15) // 16
        meta = build_step_metadata([ctx - 1, 9], [(0, 1), (1, 2)], [list(range(blocks)), [0]], [ctx, 10],
                                   block_size=16, num_blocks=blocks, partition_tokens=256)
        assert meta.max_parts_per_row == (ctx + 255) // 256
        assert attach_xcd_slot_map(meta, num_heads=14, num_kv_heads=2, dtype=torch.float16, num_xcds=8) is want
