"""tb_paged_prefill (whole prefill sequences; a workgroup per sequence, kv head and
pair of 16-row blocks holds the K/V range in LDS, shared by the kv head's query
heads) against the oracle through the C ABI. Bar: attention within 2e-2 at fp16 /
bf16 against the oracle in the same dtype.

Cases: 1 to 8 query heads per kv head at head dim 64, 1 to 4 at 128;
block sizes 16 to 64; new-row counts that are not multiples of 16 (a lone middle
block, a last block of one row); cached prefixes (pos0 > 0); contexts at the
longest the kernel serves; stale NaN slots past every context; a step mixing these
sequences with decode rows and with sequences past the kernel's limit (which keep
the tiles); the config-4 mixed step, also split into its prefill and decode sides
(with and without the appends folded into both kernels); fused RoPE equal to
rotating q first; the fused append (new rows read from k / v and stored: the pool
bit-exact against the oracle's append) and what it refuses."""
import pytest
import torch

from oracle import reference_path as ref
from tinybatch_amd import layer_ops, ops
from tinybatch_amd.metadata import build_step_metadata
from tinybatch_amd.model import rope_tables

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
TOL = dict(atol=2e-2, rtol=2e-2)


def _bits(t):
    return t.contiguous().view(torch.int16)


def case(seed, Hq, Hkv, D, BS, dtype, qlens, cached, nan_tail=True):
    g = torch.Generator().manual_seed(seed)
    need = [(c + n + BS - 1) // BS for c, n in zip(cached, qlens)]
    NB = sum(need) + 3
    pool = torch.randn(NB, 2, Hkv, BS, D, generator=g).to(dtype)
    perm = torch.randperm(NB, generator=g).tolist()
    tables, slices, ctx, pos, at, t = [], [], [], [], 0, 0
    for c, n, nb in zip(cached, qlens, need):
        tables.append(perm[at:at + nb])
        at += nb
        slices.append((t, t + n))
        t += n
        ctx.append(c + n)
        pos.extend(range(c, c + n))
    if nan_tail:   # stale slots past every context, and unused blocks, hold NaN
        for table, c in zip(tables, ctx):
            if c % BS:
                pool[table[-1], :, :, c % BS:] = float("nan")
        for b in perm[at:]:
            pool[b] = float("nan")
    q = torch.randn(t, Hq, D, generator=g).to(dtype)
    return dict(pool=pool, tables=tables, slices=slices, ctx=ctx, pos=pos, q=q, NB=NB, Hq=Hq, Hkv=Hkv, D=D, BS=BS,
                dtype=dtype)


def metadata(c, route=True):
    dt, Hq, Hkv, D = c["dtype"], c["Hq"], c["Hkv"], c["D"]
    r = ops.prefill_route(dt, Hq, Hkv, D) if route else None
    assert not route or r is not None
    return build_step_metadata(c["pos"], c["slices"], c["tables"], c["ctx"], block_size=c["BS"], num_blocks=c["NB"],
                               partition_tokens=ops.partition_tokens(dt, D),
                               rows_per_item=ops.rows_per_item(dt, Hq, Hkv), tile_prefill=True,
                               prefill_route=r).to(DEV)


def check(c, min_work=1):
    want = ref.attention(c["q"], c["pool"], c["slices"], c["tables"], c["ctx"], c["Hq"], c["Hkv"])
    meta = metadata(c)
    assert meta.num_prefill_work >= min_work
    out = ops.paged_attention(c["q"].to(DEV), c["pool"].to(DEV), meta, num_heads=c["Hq"])
    torch.cuda.synchronize()
    got = out.cpu()
    assert torch.isfinite(got).all()
    torch.testing.assert_close(got.float(), want.float(), **TOL)
    return meta


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Hq,Hkv,D", [(14, 2, 64), (8, 8, 64), (16, 2, 64), (8, 2, 64), (16, 8, 64), (6, 2, 64),
                                      (10, 2, 64), (12, 2, 64), (32, 8, 128), (4, 2, 128), (8, 8, 128),
                                      (12, 4, 128)])
@pytest.mark.parametrize("BS", [16, 64])
def test_geometries_rows_and_prefixes(Hq, Hkv, D, BS, dtype):
    # new rows 16 .. 100 (lone middle blocks, a last block of one row), cached
    # prefixes, and two decode rows in the same step (work items)
    lim = ops.prefill_route(dtype, Hq, Hkv, D).max_context
    qlens = [16, 17, 33, 100, 1, 49, 1]
    cached = [0, 5, 64, lim - 100 - 13, 300, 160, 40]
    c = case(Hq * 10 + D + BS, Hq, Hkv, D, BS, dtype, qlens, cached)
    meta = check(c)
    assert meta.num_work_items > 0                     # the decode rows
    assert meta.num_prefill_tiles == 0                 # every long run of rows went to the new kernel


@pytest.mark.parametrize("D", [64, 128])
def test_contexts_at_the_limit_and_past_it(D):
    lim = ops.prefill_route(torch.bfloat16, 14 if D == 64 else 32, 2 if D == 64 else 8, D).max_context
    # one context at the limit from position 0, one at the limit after a prefix,
    # one past it (tiles), one short
    c = case(D, 14 if D == 64 else 32, 2 if D == 64 else 8, D, 32, torch.bfloat16,
             qlens=[lim, lim - 48, lim + 40, 16], cached=[0, 48, 0, 7])
    meta = check(c)
    assert meta.num_prefill_tiles > 0                  # the sequence past the limit keeps the tiles


def test_block_size_32_and_a_lone_sequence():
    c = case(3, 14, 2, 64, 32, torch.float16, qlens=[65], cached=[130])
    check(c)


def test_config4_mixed_step():
    from tinybatch_amd.workloads import make_mixed_workload

    wl = make_mixed_workload()
    c = dict(pool=wl.pool, tables=wl.block_tables, slices=wl.seq_slices, ctx=wl.context_lens,
             pos=list(wl.positions),
             q=wl.q, NB=wl.num_blocks, Hq=14, Hkv=2, D=64, BS=16, dtype=torch.bfloat16)
    meta = check(c)
    assert meta.num_prefill_work == 8 * 16 * 2          # 8 sequences x 16 block pairs x 2 kv heads


def test_config4_split_step_against_the_oracle_and_the_one_launch():
    """The config-4 step (8 whole prefills, then 56 decode rows) as two sub-steps
    (ops.attach_split_parts: tb_paged_prefill on the prefill rows, the streaming
    decode kernel on the decode rows): within the bar of the oracle, and of the
    one launch of tiles and decode items the same metadata runs without its parts;
    the drop-in cache takes the split by itself."""
    from tinybatch_amd.kv_cache import PagedKVCache
    from tinybatch_amd.workloads import make_mixed_workload

    wl = make_mixed_workload()
    dt, Hq, Hkv, D = wl.dtype, wl.num_heads, wl.num_kv_heads, wl.head_dim
    want = ref.attention(wl.q, wl.pool, wl.seq_slices, wl.block_tables, wl.context_lens, Hq, Hkv)
    meta = build_step_metadata(wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens, block_size=16,
                               num_blocks=wl.num_blocks, partition_tokens=ops.partition_tokens(dt, D),
                               rows_per_item=ops.rows_per_item(dt, Hq, Hkv), tile_prefill=True)
    assert ops.attach_split_parts(meta, wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens, num_heads=Hq,
                                  num_kv_heads=Hkv, head_dim=D, dtype=dt, device=DEV)
    (r0, r1, pre), (d0, d1, dec) = meta.parts
    assert (r0, r1, d0, d1) == (0, 4096, 4096, 4152) and dec.decode_segments_np is not None and pre.num_prefill_work
    meta.to(DEV)
    q, pool = wl.q.to(DEV), wl.pool.to(DEV)
    split = ops.paged_attention(q, pool, meta, num_heads=Hq)
    parts, meta.parts = meta.parts, None
    one = ops.paged_attention(q, pool, meta, num_heads=Hq)
    meta.parts = parts
    cache = PagedKVCache(1, wl.num_blocks, 16, Hkv, D, DEV, dt)
    cache.pools[0].copy_(pool)
    drop_in = cache.attention(0, q, torch.tensor(wl.positions, device=DEV), wl.seq_slices, wl.block_tables,
                              wl.context_lens, num_heads=Hq)
    torch.cuda.synchronize()
    assert cache._meta_cache[0]["meta"].parts is not None
    for got in (split, one, drop_in):
        assert torch.isfinite(got.cpu()).all()
        torch.testing.assert_close(got.cpu().float(), want.float(), **TOL)
    torch.testing.assert_close(split.cpu().float(), one.cpu().float(), **TOL)
    assert torch.equal(_bits(split.cpu()), _bits(drop_in.cpu()))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_rope_equals_rotating_first(dtype):
    c = case(21, 14, 2, 64, 16, dtype, qlens=[40, 96, 1], cached=[3, 100, 50], nan_tail=False)
    cos, sin = rope_tables(64, 1e6, 8192, DEV)
    meta = metadata(c)
    q = c["q"].to(DEV)
    pool = c["pool"].to(DEV)
    out_a = ops.paged_attention(q, pool, meta, num_heads=14, rope=ops.Rope(cos, sin))
    T = q.shape[0]
    pos = torch.tensor(c["pos"], dtype=torch.int64, device=DEV)
    zeros = torch.zeros(T, 2 * 2 * 64, dtype=dtype, device=DEV)
    qr, _ = layer_ops.rope_qk(torch.cat([q.reshape(T, -1), zeros], 1).contiguous(), pos, cos, sin, 14, 2, 64)
    out_b = ops.paged_attention(qr.contiguous(), pool, meta, num_heads=14)
    torch.cuda.synchronize()
    assert torch.equal(_bits(out_a), _bits(out_b))


@pytest.mark.parametrize("BS", [16, 32])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cached", [[0, 32, 0, 64], [0, 37, 5, 71]])
def test_fused_append_stores_the_new_rows_and_reads_them_from_k_v(BS, dtype, cached):
    """k_new / v_new given: the kernel reads each sequence's new rows from them (the
    pool's new slots hold NaN before the call) and stores them: the pool afterwards
    equals the oracle's append bit for bit, the attention is within the bar of the
    oracle on that pool. New rows 16 .. 100 after cached prefixes of 0 .. 71
    positions, also ones whose first new row lies inside a 16-position tile (the
    tile's earlier rows then come from the pool)."""
    qlens = [17, 100, 33, 16]
    c = case(BS + 7, 14, 2, 64, BS, dtype, qlens, cached)
    g = torch.Generator().manual_seed(BS)
    T = sum(qlens)
    k = torch.randn(T, 2, 64, generator=g).to(dtype)
    v = torch.randn(T, 2, 64, generator=g).to(dtype)
    pos = torch.tensor(c["pos"], dtype=torch.int64)
    want_pool = c["pool"].clone()
    ref.kv_write(want_pool, k, v, pos, c["slices"], c["tables"], BS)
    want = ref.attention(c["q"], want_pool, c["slices"], c["tables"], c["ctx"], 14, 2)
    stale = c["pool"].clone()
    for (b, e), table, p0 in zip(c["slices"], c["tables"], cached):   # the new slots: NaN before the call
        for i in range(e - b):
            p = p0 + i
            stale[table[p // BS], :, :, p % BS] = float("nan")
    meta = metadata(c)
    assert meta.num_prefill_work and not meta.num_work_items and not meta.num_prefill_tiles
    pool = stale.to(DEV)
    out = ops.paged_attention(c["q"].to(DEV), pool, meta, num_heads=14, k_new=k.to(DEV), v_new=v.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(_bits(pool.cpu()), _bits(want_pool))
    got = out.cpu()
    assert torch.isfinite(got).all()
    torch.testing.assert_close(got.float(), want.float(), **TOL)


@pytest.mark.parametrize("D,Hq,Hkv", [(64, 14, 2), (128, 16, 4)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_append_with_rope_equals_rotating_then_appending(D, Hq, Hkv, dtype):
    """RoPE in the fused append (the reference rotates k, then writes it,
    model.py:125,128): the kernel rotates the new K rows in LDS, stores them and
    attends with them; pool and output equal, bit for bit, the rotating append
    kernel followed by the unfused call (new rows also starting inside a tile)."""
    qlens, cached = [40, 17, 100], [0, 9, 48]
    c = case(31 + D, Hq, Hkv, D, 16, dtype, qlens, cached)
    g = torch.Generator().manual_seed(D)
    T = sum(qlens)
    k = torch.randn(T, Hkv, D, generator=g).to(dtype).to(DEV)
    v = torch.randn(T, Hkv, D, generator=g).to(dtype).to(DEV)
    cos, sin = rope_tables(D, 1e6, 512, DEV)
    rope = ops.Rope(cos, sin)
    meta = metadata(c)
    q = c["q"].to(DEV)
    pool_a = c["pool"].to(DEV)
    out_a = ops.paged_attention(q, pool_a, meta, num_heads=Hq, k_new=k, v_new=v, rope=rope)
    pool_b = c["pool"].to(DEV)
    pos = torch.tensor(c["pos"], dtype=torch.int64, device=DEV)
    ops.kv_append(pool_b, k, v, meta.slot_mapping, rope=rope, positions=pos)
    out_b = ops.paged_attention(q, pool_b, meta, num_heads=Hq, rope=rope)
    torch.cuda.synchronize()
    assert torch.equal(_bits(pool_a.cpu()), _bits(pool_b.cpu()))
    assert torch.equal(_bits(out_a.cpu()), _bits(out_b.cpu()))
    # and against the oracle: rotate q and the new k on the host, append, attend
    qkv = torch.cat([q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1)], 1)
    qr, kr = layer_ops.rope_qk(qkv.contiguous(), pos, cos, sin, Hq, Hkv, D)
    want_pool = c["pool"].clone()
    ref.kv_write(want_pool, kr.cpu(), v.cpu(), pos.cpu(), c["slices"], c["tables"], 16)
    want = ref.attention(qr.cpu(), want_pool, c["slices"], c["tables"], c["ctx"], Hq, Hkv)
    assert torch.equal(_bits(pool_a.cpu()), _bits(want_pool))
    torch.testing.assert_close(out_a.cpu().float(), want.float(), **TOL)


def test_config4_split_step_appending_in_both_kernels():
    """The config-4 step split into its sides, each kernel appending its own rows
    (no kv_append): the pool equals the oracle's append bit for bit, the
    attention is within the bar of the oracle on that pool."""
    from tinybatch_amd.workloads import make_mixed_workload

    wl = make_mixed_workload()
    dt, Hq, Hkv, D = wl.dtype, wl.num_heads, wl.num_kv_heads, wl.head_dim
    want_pool = wl.pool.clone()
    ref.kv_write(want_pool, wl.k_new, wl.v_new, torch.tensor(wl.positions, dtype=torch.int64), wl.seq_slices,
                 wl.block_tables, 16)
    want = ref.attention(wl.q, want_pool, wl.seq_slices, wl.block_tables, wl.context_lens, Hq, Hkv)
    meta = build_step_metadata(wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens, block_size=16,
                               num_blocks=wl.num_blocks, partition_tokens=ops.partition_tokens(dt, D),
                               rows_per_item=ops.rows_per_item(dt, Hq, Hkv), tile_prefill=True)
    assert ops.attach_split_parts(meta, wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens, num_heads=Hq,
                                  num_kv_heads=Hkv, head_dim=D, dtype=dt, device=DEV)
    meta.to(DEV)
    pool = wl.pool.to(DEV)
    out = ops.paged_attention(wl.q.to(DEV), pool, meta, num_heads=Hq, k_new=wl.k_new.to(DEV),
                              v_new=wl.v_new.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(_bits(pool.cpu()), _bits(want_pool))
    torch.testing.assert_close(out.cpu().float(), want.float(), **TOL)


def test_split_step_refuses_a_slot_shared_across_its_parts():
    """A prefill row and a decode row of one split step write the same pool slot: each
    part's own slot mapping cannot see it, so the fused append is refused on the whole
    step's mapping (the reference's last writer wins, kv_cache.py:33-38) before any
    launch; without k_new the step runs."""
    g = torch.Generator().manual_seed(11)
    Hq, Hkv, D, BS, dt = 14, 2, 64, 16, torch.bfloat16
    n_dec, dec_ctx = 16, 2048 + 5                     # 16 x 2 units, 32 Ki positions: the decode kernel's side
    nb_dec = (dec_ctx + BS - 1) // BS
    NB = 2 + n_dec * nb_dec
    pool = torch.randn(NB, 2, Hkv, BS, D, generator=g).to(dt)
    pre_table = [0, 1]                                # 32 new rows at positions 0..31
    tables = [pre_table] + [list(range(2 + i * nb_dec, 2 + (i + 1) * nb_dec)) for i in range(n_dec)]
    tables[1][-1] = 1                                 # decode row 0's newest slot: block 1, offset 4 = position 20
    slices, pos, ctx = [(0, 32)], list(range(32)), [32]
    for i in range(n_dec):
        slices.append((32 + i, 33 + i))
        pos.append(dec_ctx - 1)
        ctx.append(dec_ctx)
    T = 32 + n_dec
    meta = build_step_metadata(pos, slices, tables, ctx, block_size=BS, num_blocks=NB,
                               partition_tokens=ops.partition_tokens(dt, D),
                               rows_per_item=ops.rows_per_item(dt, Hq, Hkv), tile_prefill=True)
    assert meta.slot_mapping_np[20] == -1             # the prefill row is superseded by the decode row
    assert ops.attach_split_parts(meta, pos, slices, tables, ctx, num_heads=Hq, num_kv_heads=Hkv, head_dim=D,
                                  dtype=dt, device=DEV)
    for _, _, m in meta.parts:                        # neither part's own mapping sees the shared slot
        assert not ((m.slot_mapping_np < 0) & (m.row_ctx_np > 0)).any()
    meta.to(DEV)
    q = torch.randn(T, Hq, D, generator=g).to(dt).to(DEV)
    k = torch.randn(T, Hkv, D, generator=g).to(dt).to(DEV)
    dpool = pool.to(DEV)
    before = dpool.clone()
    with pytest.raises(ValueError, match="write one pool slot"):
        ops.paged_attention(q, dpool, meta, num_heads=Hq, k_new=k, v_new=k)
    torch.cuda.synchronize()
    assert torch.equal(_bits(dpool), _bits(before))   # nothing launched
