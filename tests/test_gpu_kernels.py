"""Parity of the HIP kernels (through the C ABI) with the CPU oracle.

Bars: append / gather / copy bit-exact; attention max-abs <= 1e-5 at fp32 and
rtol = atol = 2e-2 at fp16 / bf16, against the oracle in the same dtype.
"""
import math

import numpy as np
import pytest
import torch

from oracle import reference_path as ref
from tinybatch_amd import ops
from tinybatch_amd.kv_cache import PagedKVCache
from tinybatch_amd.metadata import build_step_metadata
from tinybatch_amd.workloads import make_decode_workload

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
TOL = {torch.float32: dict(atol=1e-5, rtol=0.0), torch.float16: dict(atol=2e-2, rtol=2e-2),
       torch.bfloat16: dict(atol=2e-2, rtol=2e-2)}


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().view(torch.int32 if t.element_size() == 4 else torch.int16)


def _meta(positions, slices, tables, ctx, BS, NB, P=256, rows=1, tiles=False):
    return build_step_metadata(positions, slices, tables, ctx, block_size=BS, num_blocks=NB,
                               partition_tokens=P, rows_per_item=rows, tile_prefill=tiles).to(DEV)


def _mixed_case(seed, Hq, Hkv, D, BS, dtype, qlens, cached, NB=None, nan_tail=False):
    g = torch.Generator().manual_seed(seed)
    need = [(c + n + BS - 1) // BS for c, n in zip(cached, qlens)]
    NB = NB or sum(need) + 3
    pool = torch.randn(NB, 2, Hkv, BS, D, generator=g).to(dtype)
    perm = torch.randperm(NB, generator=g).tolist()
    tables, slices, ctx, pos, at, t = [], [], [], [], 0, 0
    for c, n, nb in zip(cached, qlens, need):
        tables.append(perm[at:at + nb]); at += nb
        slices.append((t, t + n)); t += n
        ctx.append(c + n)
        pos.extend(range(c, c + n))
    if nan_tail:
        # stale slots past every context hold NaN; they must never reach the output
        for table, c in zip(tables, ctx):
            last = table[-1]
            off = c % BS
            if off:
                pool[last, :, :, off:] = float("nan")
        for b in perm[at:]:
            pool[b] = float("nan")
    q = torch.randn(t, Hq, D, generator=g).to(dtype)
    k = torch.randn(t, Hkv, D, generator=g).to(dtype)
    v = torch.randn(t, Hkv, D, generator=g).to(dtype)
    return dict(pool=pool, tables=tables, slices=slices, ctx=ctx, pos=pos, q=q, k=k, v=v, NB=NB)


# ---------------------------------------------------------------- K1 append
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_append_bit_exact_mixed_batch(dtype):
    c = _mixed_case(1, 8, 2, 64, 16, dtype, qlens=[5, 1, 17, 1], cached=[0, 40, 3, 15])
    want = c["pool"].clone()
    ref.kv_write(want, c["k"], c["v"], torch.tensor(c["pos"]), c["slices"], c["tables"], 16)
    pool = c["pool"].to(DEV)
    meta = _meta(c["pos"], c["slices"], c["tables"], c["ctx"], 16, c["NB"])
    ops.kv_append(pool, c["k"].to(DEV), c["v"].to(DEV), meta.slot_mapping)
    torch.cuda.synchronize()
    assert torch.equal(_bits(pool.cpu()), _bits(want))


def test_append_through_drop_in_write_config_shapes():
    for name in ("qwen-fp32-b8", "qwen-fp16-b64"):
        wl = make_decode_workload(name)
        want = wl.pool.clone()
        ref.kv_write(want, wl.k_new, wl.v_new, torch.tensor(wl.positions), wl.seq_slices, wl.block_tables, 16)
        cache = PagedKVCache(1, wl.num_blocks, 16, wl.num_kv_heads, wl.head_dim, DEV, wl.dtype)
        cache.pools[0].copy_(wl.pool.to(DEV))
        cache.write(0, wl.k_new.to(DEV), wl.v_new.to(DEV), torch.tensor(wl.positions, device=DEV),
                    wl.seq_slices, wl.block_tables)
        torch.cuda.synchronize()
        assert torch.equal(_bits(cache.pools[0].cpu()), _bits(want)), name


def test_append_duplicate_slot_last_writer_wins():
    dtype = torch.float16
    pool = torch.zeros(4, 2, 2, 4, 64, dtype=dtype)
    k = torch.randn(2, 2, 64).to(dtype)
    v = torch.randn(2, 2, 64).to(dtype)
    want = pool.clone()
    ref.kv_write(want, k, v, torch.tensor([3, 3]), [(0, 1), (1, 2)], [[2], [2]], 4)
    gp = pool.to(DEV)
    meta = _meta([3, 3], [(0, 1), (1, 2)], [[2], [2]], [4, 4], 4, 4, P=64)
    ops.kv_append(gp, k.to(DEV), v.to(DEV), meta.slot_mapping)
    torch.cuda.synchronize()
    assert torch.equal(_bits(gp.cpu()), _bits(want))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_rows_sharing_a_slot_last_writer_wins(dtype):
    """Rows 0 and 2 of a decode step have their newest positions on one pool slot
    (block 6, offset 3). The reference writes the whole batch first, row 2 last,
    and both rows then read row 2's K/V there (kv_cache.py:33-38). The fused
    append cannot give that and is refused; append + attention match the oracle."""
    g = torch.Generator().manual_seed(21)
    Hq, Hkv, D, BS, NB = 8, 2, 64, 16, 12
    pool = torch.randn(NB, 2, Hkv, BS, D, generator=g).to(dtype)
    tables = [[3, 6], [1, 2, 4], [0, 5, 6]]
    ctx = [20, 40, 36]                        # newest positions 19, 39, 35: slots 6*16+3, 4*16+7, 6*16+3
    pos = [c - 1 for c in ctx]
    slices = [(i, i + 1) for i in range(3)]
    q = torch.randn(3, Hq, D, generator=g).to(dtype)
    k = torch.randn(3, Hkv, D, generator=g).to(dtype)
    v = torch.randn(3, Hkv, D, generator=g).to(dtype)
    want_pool = pool.clone()
    ref.kv_write(want_pool, k, v, torch.tensor(pos), slices, tables, BS)
    want = ref.attention(q, want_pool, slices, tables, ctx, Hq, Hkv)
    meta = _meta(pos, slices, tables, ctx, BS, NB, P=ops.partition_tokens(dtype, D))
    assert meta.slot_mapping_np.tolist() == [-1, 4 * 16 + 7, 6 * 16 + 3]
    gp = pool.to(DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    with pytest.raises(ValueError, match="one pool slot"):
        ops.paged_attention(qd, gp, meta, num_heads=Hq, k_new=kd, v_new=vd)
    ops.kv_append(gp, kd, vd, meta.slot_mapping)
    out = ops.paged_attention(qd, gp, meta, num_heads=Hq)
    torch.cuda.synchronize()
    assert torch.equal(_bits(gp.cpu()), _bits(want_pool))
    torch.testing.assert_close(out.cpu().float(), want.float(), **TOL[dtype])


# ---------------------------------------------------------------- gather
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gather_bit_exact(dtype):
    c = _mixed_case(2, 8, 4, 128, 16, dtype, qlens=[1, 1], cached=[37, 130])
    cache = PagedKVCache(1, c["NB"], 16, 4, 128, DEV, dtype)
    cache.pools[0].copy_(c["pool"].to(DEV))
    for table, ctx in zip(c["tables"], c["ctx"]):
        k, v = cache.gather(0, table, ctx)
        K, V = ref.kv_gather(c["pool"], table, ctx)
        assert torch.equal(_bits(k.cpu()), _bits(K)) and torch.equal(_bits(v.cpu()), _bits(V))


# ---------------------------------------------------------------- K2 attention
def _attention_vs_oracle(c, Hq, Hkv, dtype, P=256, rows=None):
    """Every work shape: one row per item, (16-bit) the widest row group, and
    (16-bit) prefill tiles for sequences with many new rows."""
    want = ref.attention(c["q"], c["pool"], c["slices"], c["tables"], c["ctx"], Hq, Hkv)
    widest = ops.rows_per_item(dtype, Hq, Hkv)
    shapes = [(1, False), (widest, False)] if rows is None else [(rows, False)]
    if rows is None and dtype != torch.float32:
        shapes.append((widest, True))
    for r, tiles in sorted(set(shapes)):
        meta = _meta(c["pos"], c["slices"], c["tables"], c["ctx"], c["pool"].shape[3], c["NB"], P=P, rows=r,
                     tiles=tiles)
        out = ops.paged_attention(c["q"].to(DEV), c["pool"].to(DEV), meta, num_heads=Hq)
        torch.cuda.synchronize()
        got = out.cpu()
        case = f"rows per item {r}, tiles {tiles} ({meta.num_prefill_tiles})"
        assert torch.isfinite(got).all(), case
        torch.testing.assert_close(got.float(), want.float(), **TOL[dtype], msg=lambda m: f"{case}: {m}")
    return got, want


def test_decode_config1_fp32_within_1e5():
    wl = make_decode_workload("qwen-fp32-b8")
    want = ref.decode_step(wl.pool.clone(), wl.q, wl.k_new, wl.v_new, wl.cached_lens, wl.block_tables,
                           14, 2, 16)
    cache = PagedKVCache(1, wl.num_blocks, 16, 2, 64, DEV, torch.float32)
    cache.pools[0].copy_(wl.pool.to(DEV))
    pos = torch.tensor(wl.positions, device=DEV)
    cache.write(0, wl.k_new.to(DEV), wl.v_new.to(DEV), pos, wl.seq_slices, wl.block_tables)
    got = cache.attention(0, wl.q.to(DEV), pos, wl.seq_slices, wl.block_tables, wl.context_lens)
    torch.cuda.synchronize()
    assert (got.cpu() - want).abs().max().item() <= 1e-5


@pytest.mark.parametrize("fused", [False, True])
def test_decode_config2_fp16_full_size(fused):
    wl = make_decode_workload("qwen-fp16-b64")
    pool_ref = wl.pool.clone()
    want = ref.decode_step(pool_ref, wl.q, wl.k_new, wl.v_new, wl.cached_lens, wl.block_tables, 14, 2, 16)
    pool = wl.pool.to(DEV)
    meta = _meta(wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens, 16, wl.num_blocks)
    q, k, v = wl.q.to(DEV), wl.k_new.to(DEV), wl.v_new.to(DEV)
    if fused:
        out = ops.paged_attention(q, pool, meta, num_heads=14, k_new=k, v_new=v)
    else:
        ops.kv_append(pool, k, v, meta.slot_mapping)
        out = ops.paged_attention(q, pool, meta, num_heads=14)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu().float(), want.float(), **TOL[torch.float16])
    # the appended rows land bit-exactly in both modes
    assert torch.equal(_bits(pool.cpu()), _bits(pool_ref))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Hq,Hkv,D", [(14, 2, 64), (32, 8, 128), (4, 4, 64), (28, 2, 128), (6, 1, 64)])
def test_mixed_batch_attention_shapes(dtype, Hq, Hkv, D):
    c = _mixed_case(3, Hq, Hkv, D, 16, dtype, qlens=[1, 7, 1, 20, 1], cached=[600, 0, 15, 300, 1])
    _attention_vs_oracle(c, Hq, Hkv, dtype)


@pytest.mark.parametrize("BS,P", [(4, 128), (8, 256), (32, 512), (64, 1024)])
def test_block_sizes_and_partitions(BS, P):
    c = _mixed_case(4, 14, 2, 64, BS, torch.float32, qlens=[1, 3, 1], cached=[700, 90, 2])
    _attention_vs_oracle(c, 14, 2, torch.float32, P=P)


def test_stale_nan_slots_never_reach_output():
    c = _mixed_case(5, 14, 2, 64, 16, torch.float16, qlens=[1, 1, 5], cached=[33, 300, 10], nan_tail=True)
    _attention_vs_oracle(c, 14, 2, torch.float16)


def test_permuted_blocks_identical_output():
    c = _mixed_case(6, 8, 2, 64, 16, torch.bfloat16, qlens=[1, 1], cached=[500, 77])
    meta = _meta(c["pos"], c["slices"], c["tables"], c["ctx"], 16, c["NB"])
    out1 = ops.paged_attention(c["q"].to(DEV), c["pool"].to(DEV), meta, num_heads=8)
    perm = torch.randperm(c["NB"], generator=torch.Generator().manual_seed(1))
    pool2 = torch.empty_like(c["pool"])
    pool2[perm] = c["pool"]
    tables2 = [[int(perm[b]) for b in t] for t in c["tables"]]
    meta2 = _meta(c["pos"], c["slices"], tables2, c["ctx"], 16, c["NB"])
    out2 = ops.paged_attention(c["q"].to(DEV), pool2.to(DEV), meta2, num_heads=8)
    torch.cuda.synchronize()
    assert torch.equal(out1.cpu(), out2.cpu())


def test_long_context_split_into_many_partitions():
    c = _mixed_case(7, 32, 8, 128, 16, torch.bfloat16, qlens=[1, 1], cached=[20000, 4095])
    _attention_vs_oracle(c, 32, 8, torch.bfloat16)


def test_config3_subset_bf16():
    """Llama-3-8B decode geometry; the pool is drawn on the GPU, 8 sequences checked."""
    wl = make_decode_workload("llama-bf16-b256", pool_device=DEV, batch=8)
    meta = _meta(wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens, 16, wl.num_blocks)
    pool = wl.pool
    out = ops.paged_attention(wl.q.to(DEV), pool, meta, num_heads=32, k_new=wl.k_new.to(DEV),
                              v_new=wl.v_new.to(DEV))
    torch.cuda.synchronize()
    pool_cpu = pool.cpu()
    want = ref.attention(wl.q, pool_cpu, wl.seq_slices, wl.block_tables, wl.context_lens, 32, 8)
    torch.testing.assert_close(out.cpu().float(), want.float(), **TOL[torch.bfloat16])


# ---------------------------------------------------------------- K3 copy
def test_block_copy_all_layers_bit_exact():
    cache = PagedKVCache(3, 64, 16, 2, 64, DEV, torch.bfloat16)
    g = torch.Generator().manual_seed(8)
    host = torch.randn(3, 64, 2, 2, 16, 64, generator=g).to(torch.bfloat16)
    cache.storage.copy_(host.to(DEV))
    src, dst = [1, 5, 9, 33], [40, 2, 63, 0]
    cache.copy_blocks(src, dst)
    torch.cuda.synchronize()
    want = host.clone()
    for layer in range(3):
        for s, d in zip(src, dst):
            want[layer, d] = host[layer, s]
    assert torch.equal(_bits(cache.storage.cpu()), _bits(want))


def test_block_copy_rejects_overlapping_pairs():
    cache = PagedKVCache(1, 8, 16, 2, 64, DEV, torch.float16)
    with pytest.raises(ValueError):
        cache.copy_blocks([1, 2], [2, 3])
    with pytest.raises(IndexError):
        cache.copy_blocks([1], [8])


def test_swap_out_swap_in_roundtrip_pinned_host():
    cache = PagedKVCache(2, 32, 16, 2, 64, DEV, torch.float16)
    host = torch.randn(2, 32, 2, 2, 16, 64).to(torch.float16)
    cache.storage.copy_(host.to(DEV))
    blocks = [3, 17, 30]
    staging = [torch.empty(3, 2, 2, 16, 64, dtype=torch.float16, pin_memory=True) for _ in range(2)]
    cache.swap_out(blocks, staging)
    torch.cuda.synchronize()
    for layer in range(2):
        assert torch.equal(_bits(staging[layer]), _bits(host[layer, blocks]))
    cache.storage.zero_()
    cache.swap_in(staging, [0, 1, 2])
    torch.cuda.synchronize()
    for layer in range(2):
        assert torch.equal(_bits(cache.storage[layer, :3].cpu()), _bits(host[layer, blocks]))


def test_consecutive_calls_of_different_shapes_share_workspace():
    """Split rows of one call must not be disturbed by an earlier call of another
    shape that used the same partials buffer."""
    cases = [(14, 2, 64, torch.bfloat16), (32, 8, 128, torch.float32), (14, 2, 64, torch.float16),
             (32, 8, 128, torch.bfloat16), (8, 1, 128, torch.float16)]
    for i, (Hq, Hkv, D, dt) in enumerate(cases * 2):
        c = _mixed_case(20 + i, Hq, Hkv, D, 16, dt, qlens=[1, 3, 9, 1], cached=[700, 260, 300, 40])
        _attention_vs_oracle(c, Hq, Hkv, dt)


@pytest.mark.parametrize("BS", [4, 8, 32, 64])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_block_sizes_16bit(BS, dtype):
    c = _mixed_case(9, 14, 2, 64, BS, dtype, qlens=[1, 3, 1], cached=[700, 90, 2])
    _attention_vs_oracle(c, 14, 2, dtype)
    c = _mixed_case(10, 16, 4, 128, BS, dtype, qlens=[1, 2], cached=[333, 1000])
    _attention_vs_oracle(c, 16, 4, dtype)


@pytest.mark.parametrize("BS", [4, 8, 16, 64])
@pytest.mark.parametrize("dtype,Hq,Hkv,D", [(torch.float16, 14, 2, 64), (torch.bfloat16, 16, 4, 128)])
def test_fused_decode_append_block_sizes(BS, dtype, Hq, Hkv, D):
    """Fused append + attention on both address paths (block tables read per lane for
    BS < 16, per 16-position tile otherwise); the newest position may sit in any
    wave, partition and block offset."""
    cached = [0, 1, 15, 63, 64, 255, 256, 700, 1023, 2047]
    c = _mixed_case(30 + BS, Hq, Hkv, D, BS, dtype, qlens=[1] * len(cached), cached=cached)
    pool_ref = c["pool"].clone()
    want = ref.decode_step(pool_ref, c["q"], c["k"], c["v"], cached, c["tables"], Hq, Hkv, BS)
    pool = c["pool"].to(DEV)
    meta = _meta(c["pos"], c["slices"], c["tables"], c["ctx"], BS, c["NB"])
    out = ops.paged_attention(c["q"].to(DEV), pool, meta, num_heads=Hq, k_new=c["k"].to(DEV), v_new=c["v"].to(DEV))
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu().float(), want.float(), **TOL[dtype])
    assert torch.equal(_bits(pool.cpu()), _bits(pool_ref))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_split_rows_merge_the_same_bits_every_call(dtype):
    """Rows over up to 20 partitions (two batches of the combine) and short rows
    in one step; repeated calls give the same bits (the merge order is fixed)."""
    Hq, Hkv, D = 16, 4, 128
    c = _mixed_case(12, Hq, Hkv, D, 16, dtype, qlens=[1, 1, 1, 3], cached=[5000, 300, 2600, 1500])
    meta = _meta(c["pos"], c["slices"], c["tables"], c["ctx"], 16, c["NB"])
    assert meta.max_parts_per_row == 20 and meta.num_split_rows == 6
    q, pool = c["q"].to(DEV), c["pool"].to(DEV)
    outs = [ops.paged_attention(q, pool, meta, num_heads=Hq).cpu() for _ in range(3)]
    assert all(torch.equal(_bits(outs[0]), _bits(o)) for o in outs[1:])
    _attention_vs_oracle(c, Hq, Hkv, dtype)


def test_golden_fixture_decode_fp32():
    """GPU decode step of the committed fixture (inputs regenerated from its seed)."""
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "qwen_fp32_b8_decode.npz"))
    wl = make_decode_workload("qwen-fp32-b8")
    pool = wl.pool.to(DEV)
    meta = _meta(wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens, 16, wl.num_blocks)
    out = ops.paged_attention(wl.q.to(DEV), pool, meta, num_heads=14, k_new=wl.k_new.to(DEV), v_new=wl.v_new.to(DEV))
    torch.cuda.synchronize()
    assert np.abs(out.cpu().numpy() - g["attn_out_f64"]).max() <= 1e-5
    assert np.abs(out.cpu().numpy() - g["attn_out"]).max() <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Hq,Hkv,D", [(14, 2, 64), (32, 8, 128), (8, 8, 64)])
def test_prefill_rows_grouped(dtype, Hq, Hkv, D):
    """Full prefills (q_len == ctx, the is_causal branch), a cached-prefix tail
    (1 < q_len < ctx) and decodes in one batch; rows straddle partition edges."""
    c = _mixed_case(11, Hq, Hkv, D, 16, dtype, qlens=[300, 1, 37, 260, 1, 3], cached=[0, 700, 220, 0, 40, 509])
    _attention_vs_oracle(c, Hq, Hkv, dtype)


def test_prefill_config4_shape_bf16():
    """Eight 512-token prefills next to 56 decodes, Qwen geometry, bf16."""
    qlens = [512] * 8 + [1] * 56
    g = torch.Generator().manual_seed(12)
    cached = [0] * 8 + torch.randint(256, 2049, (56,), generator=g).tolist()
    c = _mixed_case(12, 14, 2, 64, 16, torch.bfloat16, qlens=qlens, cached=cached)
    _attention_vs_oracle(c, 14, 2, torch.bfloat16)


def test_mixed_step_config4_append_attention_copy():
    """The mixed engine step at full size: 8 x 512-token prefills + 56 decodes
    (24 share a 32-block prefix) in bf16 — append bit-exact, attention within
    2e-2 with grouped prefill rows, then the 1024-block compaction copy bit-exact."""
    from tinybatch_amd.workloads import make_mixed_workload
    wl = make_mixed_workload()
    BS = wl.block_size
    pos = torch.tensor(wl.positions, dtype=torch.int64)
    want_pool = wl.pool.clone()
    ref.kv_write(want_pool, wl.k_new, wl.v_new, pos, wl.seq_slices, wl.block_tables, BS)
    want = ref.attention(wl.q, want_pool, wl.seq_slices, wl.block_tables, wl.context_lens,
                         wl.num_heads, wl.num_kv_heads)
    rows = ops.rows_per_item(wl.dtype, wl.num_heads, wl.num_kv_heads)
    assert rows == 2
    meta = _meta(wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens, BS, wl.num_blocks, rows=rows,
                 tiles=True)
    assert meta.num_prefill_tiles == 8 * 512 // 64            # one 1024-position partition each
    pool = wl.pool.to(DEV)
    ops.kv_append(pool, wl.k_new.to(DEV), wl.v_new.to(DEV), meta.slot_mapping)
    out = ops.paged_attention(wl.q.to(DEV), pool, meta, num_heads=wl.num_heads)
    torch.cuda.synchronize()
    assert torch.equal(_bits(pool.cpu()), _bits(want_pool))
    torch.testing.assert_close(out.cpu().float(), want.float(), **TOL[torch.bfloat16])
    # compaction round: live blocks move to free ids
    ops.block_copy([pool], wl.copy_src, wl.copy_dst)
    torch.cuda.synchronize()
    want_pool[wl.copy_dst] = want_pool[wl.copy_src]
    assert torch.equal(_bits(pool.cpu()), _bits(want_pool))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Hq,Hkv,D", [(14, 2, 64), (32, 8, 128), (4, 4, 64)])
def test_prefill_tiles_ragged_and_tails(dtype, Hq, Hkv, D):
    """Tiles with partial last tiles (q_len not a multiple of 64), prefill tails
    after a cached prefix (pos0 > 0, chunks straddling the diagonal), block
    sizes other than 16 through the chunk walk, next to decode rows."""
    for BS, seed in ((16, 21), (4, 22), (64, 23)):
        c = _mixed_case(seed, Hq, Hkv, D, BS, dtype, qlens=[16, 1, 130, 64, 77, 1, 200],
                        cached=[0, 300, 0, 5, 600, 17, 2000])
        meta = _meta(c["pos"], c["slices"], c["tables"], c["ctx"], BS, c["NB"], tiles=True)
        # one item per (tile of 64 rows, 1024-position partition its last row reaches)
        assert meta.num_prefill_tiles == 1 + 3 + 1 + (1 + 1) + 4 * 3
        _attention_vs_oracle(c, Hq, Hkv, dtype)


def test_prefill_tiles_through_the_drop_in_cache():
    """PagedKVCache.write + attention (16-bit pools use tiles for prefills)."""
    Hq, Hkv, D, BS = 14, 2, 64, 16
    c = _mixed_case(24, Hq, Hkv, D, BS, torch.bfloat16, qlens=[96, 1, 40], cached=[0, 70, 400])
    cache = PagedKVCache(1, c["NB"], BS, Hkv, D, DEV, torch.bfloat16)
    cache.pools[0].copy_(c["pool"])
    pos = torch.tensor(c["pos"], device=DEV)
    cache.write(0, c["k"].to(DEV), c["v"].to(DEV), pos, c["slices"], c["tables"])
    out = cache.attention(0, c["q"].to(DEV), pos, c["slices"], c["tables"], c["ctx"])
    torch.cuda.synchronize()
    want_pool = c["pool"].clone()
    ref.kv_write(want_pool, c["k"], c["v"], torch.tensor(c["pos"]), c["slices"], c["tables"], BS)
    want = ref.attention(c["q"], want_pool, c["slices"], c["tables"], c["ctx"], Hq, Hkv)
    assert cache.step_metadata(pos, c["slices"], c["tables"], c["ctx"], 2).num_prefill_tiles == 2 + 1
    torch.testing.assert_close(out.cpu().float(), want.float(), **TOL[torch.bfloat16])


def test_prefill_tiles_split_over_tile_partitions_bf16():
    """A 1500-row prefill and a 300-row tail at positions 2000..2299: tile rows
    reach several 1024-position partitions and merge through the combine pass."""
    c = _mixed_case(25, 14, 2, 64, 16, torch.bfloat16, qlens=[1500, 1, 300], cached=[0, 3000, 2000])
    meta = _meta(c["pos"], c["slices"], c["tables"], c["ctx"], 16, c["NB"], rows=2, tiles=True)
    counts = np.diff(meta.row_part_off_np)
    assert counts[1500] == 12                       # the decode row: 256-position partitions
    assert counts[1501:].max() == 3 and counts[:1500].max() == 2   # tile rows: 1024-position ones
    _attention_vs_oracle(c, 14, 2, torch.bfloat16)


@pytest.mark.parametrize("BS", [8, 16])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mixed_step_one_launch_tiles_and_decode_items(BS, dtype):
    """A step with prefill tiles (rows of the 40- and 100-token sequences) and
    decode items (single rows, a 33-row tail) runs as one launch of the
    combined kernel; both block-id paths (block size 8: per-lane lookups; 16:
    wave-uniform tiles); tolerance 2e-2 against the oracle."""
    c = _mixed_case(41 + BS, 14, 2, 64, BS, dtype, qlens=[40, 1, 1, 100, 33, 1], cached=[0, 300, 2000, 200, 700, 17])
    _attention_vs_oracle(c, 14, 2, dtype)
