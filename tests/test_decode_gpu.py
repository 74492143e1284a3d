"""The decode kernel (tb_paged_decode: one workgroup per CU, every wave streaming
its share of the step's 16-position tiles, partials merged inside the launch)
against the oracle, through the C ABI.

Bars: appended rows bit-exact; attention rtol = atol = 2e-2 at fp16 / bf16
against the oracle in the same dtype. Also: every compiled variant (waves per
workgroup), steps with fewer tiles than workers, the same bits from repeated
calls and from fused RoPE against rotating first; no unit ever merged across
XCDs."""
import numpy as np
import pytest
import torch

from oracle import reference_path as ref
from tinybatch_amd import layer_ops, ops
from tinybatch_amd.metadata import build_step_metadata
from tinybatch_amd.model import rope_tables
from tinybatch_amd.workloads import make_decode_workload

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
TOL = dict(atol=2e-2, rtol=2e-2)


def _bits(t):
    return t.contiguous().view(torch.int16)


def decode_meta(ctx, tables, NB, BS, Hq, Hkv, D, dtype, waves=None, unit_cost=None):
    B = len(ctx)
    meta = build_step_metadata([c - 1 for c in ctx], [(b, b + 1) for b in range(B)], tables, ctx, block_size=BS,
                               num_blocks=NB, partition_tokens=ops.partition_tokens(dtype, D))
    assert ops.attach_decode_plan(meta, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, dtype=dtype, device=DEV,
                                  waves=waves, unit_cost=unit_cost)
    return meta.to(DEV)


def case(seed, B, Hq, Hkv, D, BS, dtype, ctx=None, nan_stale=True):
    g = torch.Generator().manual_seed(seed)
    if ctx is None:
        ctx = torch.randint(1, 2500, (B,), generator=g).tolist()
    need = [(c + BS - 1) // BS for c in ctx]
    NB = sum(need) + 5
    pool = torch.randn(NB, 2, Hkv, BS, D, generator=g).to(dtype)
    perm = torch.randperm(NB, generator=g).tolist()
    tables, at = [], 0
    for n in need:
        tables.append(perm[at:at + n])
        at += n
    if nan_stale:   # positions past each context, and unused blocks, hold NaN
        for t, c in zip(tables, ctx):
            if c % BS:
                pool[t[-1], :, :, c % BS:] = float("nan")
        for blk in perm[at:]:
            pool[blk] = float("nan")
    q = torch.randn(len(ctx), Hq, D, generator=g).to(dtype)
    k = torch.randn(len(ctx), Hkv, D, generator=g).to(dtype)
    v = torch.randn(len(ctx), Hkv, D, generator=g).to(dtype)
    return dict(pool=pool, tables=tables, ctx=ctx, q=q, k=k, v=v, NB=NB, BS=BS, Hq=Hq, Hkv=Hkv, D=D, dtype=dtype)


def oracle(c):
    pool = c["pool"].clone()
    out = ref.decode_step(pool, c["q"], c["k"], c["v"], [x - 1 for x in c["ctx"]], c["tables"], c["Hq"], c["Hkv"],
                          c["BS"])
    return out, pool


def run(c, fused=True, waves=None, unit_cost=None):
    meta = decode_meta(c["ctx"], c["tables"], c["NB"], c["BS"], c["Hq"], c["Hkv"], c["D"], c["dtype"], waves,
                       unit_cost)
    pool = c["pool"].to(DEV)
    q, k, v = c["q"].to(DEV), c["k"].to(DEV), c["v"].to(DEV)
    if fused:
        out = ops.paged_attention(q, pool, meta, num_heads=c["Hq"], k_new=k, v_new=v)
    else:
        ops.kv_append(pool, k, v, meta.slot_mapping)
        out = ops.paged_attention(q, pool, meta, num_heads=c["Hq"])
    torch.cuda.synchronize()
    return out.cpu(), pool.cpu(), meta


def check(c, fused=True, waves=None):
    want, want_pool = oracle(c)
    got, pool, meta = run(c, fused, waves)
    assert torch.equal(_bits(pool), _bits(want_pool)), "pool differs (append)"
    torch.testing.assert_close(got.float(), want.float(), **TOL)
    return got, meta


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("fused", [True, False])
def test_headline_shape(dtype, fused):
    wl = make_decode_workload("qwen-fp16-b64")
    c = dict(pool=wl.pool.to(dtype), tables=wl.block_tables, ctx=wl.context_lens, q=wl.q.to(dtype),
             k=wl.k_new.to(dtype), v=wl.v_new.to(dtype), NB=wl.num_blocks, BS=16, Hq=14, Hkv=2, D=64, dtype=dtype)
    _, meta = check(c, fused)
    assert meta.decode_pieces > 0                  # units cut over workgroups: partials merged


@pytest.mark.parametrize("D,Hq,Hkv", [(64, 14, 2), (128, 32, 8)])
def test_plans_of_every_unit_cost_agree_with_the_oracle(D, Hq, Hkv):
    """The plan's unit cost moves the workers' cut points (and so the pieces, the pads
    and the merges): every cost gives the oracle's attention and the bit-exact append."""
    c = case(90 + D, 48 if D == 64 else 12, Hq, Hkv, D, 16, torch.bfloat16)
    want, want_pool = oracle(c)
    for uc in (0, 3, 6, 8, 12):
        got, pool, meta = run(c, True, None, uc)
        assert meta.decode_unit_cost == uc
        assert torch.equal(_bits(pool), _bits(want_pool)), f"unit cost {uc}: pool differs (append)"
        torch.testing.assert_close(got.float(), want.float(), **TOL, msg=f"unit cost {uc}")


def test_llama_geometry_subset():
    wl = make_decode_workload("llama-bf16-b256", batch=8)
    c = dict(pool=wl.pool, tables=wl.block_tables, ctx=wl.context_lens, q=wl.q, k=wl.k_new, v=wl.v_new,
             NB=wl.num_blocks, BS=16, Hq=32, Hkv=8, D=128, dtype=torch.bfloat16)
    check(c, fused=True)


@pytest.mark.parametrize("Hq,Hkv,D", [(14, 2, 64), (8, 8, 64), (16, 2, 64), (4, 2, 128), (32, 8, 128), (7, 7, 128)])
@pytest.mark.parametrize("BS", [16, 64])
def test_geometries_and_block_sizes(Hq, Hkv, D, BS):
    c = case(Hq * 100 + BS, 21, Hq, Hkv, D, BS, torch.bfloat16)
    check(c, fused=True)


def test_short_and_block_multiple_contexts():
    ctx = [1, 2, 15, 16, 17, 31, 32, 33, 48, 64, 65, 1, 700, 16 * 37]
    for BS in (16, 32):
        check(case(7, len(ctx), 14, 2, 64, BS, torch.float16, ctx=ctx), fused=True)
        check(case(8, len(ctx), 14, 2, 64, BS, torch.float16, ctx=ctx), fused=False)


def test_long_sequences_over_many_workgroups():
    """Units cut over up to 128 workers (4 waves per workgroup)."""
    c = case(9, 4, 14, 2, 64, 16, torch.bfloat16, ctx=[60000, 31000, 900, 5])
    _, meta = check(c, fused=True, waves=4)
    assert meta.decode_pieces > 100


@pytest.mark.parametrize("D,waves", [(64, 8), (64, 6), (64, 4), (128, 4), (128, 3)])
def test_every_variant(D, waves):
    Hq, Hkv = (14, 2) if D == 64 else (32, 8)
    c = case(15 + waves, 48, Hq, Hkv, D, 16, torch.bfloat16)
    _, meta = check(c, fused=True, waves=waves)
    assert meta.decode_waves == waves and meta.decode_pieces > 0


def test_fewer_tiles_than_workers():
    """A step far smaller than the grid: most workers idle, units over consecutive workers."""
    for seed, ctx in ((16, [40, 33, 17, 1, 64]), (17, [300] * 12), (18, [2000, 20])):
        check(case(seed, len(ctx), 14, 2, 64, 16, torch.float16, ctx=ctx), fused=True)


def test_repeated_calls_same_bits_and_no_cross_xcd_merges():
    c = case(11, 64, 14, 2, 64, 16, torch.float16, nan_stale=False)
    meta = decode_meta(c["ctx"], c["tables"], c["NB"], 16, 14, 2, 64, torch.float16)
    pool = c["pool"].to(DEV)
    q = c["q"].to(DEV)
    outs = [ops.paged_attention(q, pool, meta, num_heads=14).clone() for _ in range(3)]
    small = case(12, 3, 14, 2, 64, 16, torch.float16)     # a smaller step between: counters reset
    check(small, fused=False)
    outs.append(ops.paged_attention(q, pool, meta, num_heads=14))
    torch.cuda.synchronize()
    assert all(torch.equal(_bits(o), _bits(outs[0])) for o in outs[1:])
    assert int(ops.decode_device(DEV).violations.item()) == 0


def test_workspace_contents_before_the_call_never_reach_the_output():
    # every partial slot holds a NaN bit pattern before each call: the merges must
    # read only what this launch wrote (the last arriving group's own partial too)
    c = case(13, 64, 14, 2, 64, 16, torch.float16, nan_stale=False)
    want, want_pool = oracle(c)
    meta = decode_meta(c["ctx"], c["tables"], c["NB"], 16, 14, 2, 64, torch.float16)
    bufs = ops.DecodeBuffers(DEV, ops.decode_workspace_bytes(meta, 14, 2, 64), meta.decode_units)
    q, k, v = c["q"].to(DEV), c["k"].to(DEV), c["v"].to(DEV)
    outs = []
    for _ in range(3):
        pool = c["pool"].to(DEV)
        bufs.pieces.fill_(0xFF)
        outs.append(ops.paged_decode(q, pool, meta, num_heads=14, k_new=k, v_new=v, workspace=bufs).cpu())
        assert torch.equal(_bits(pool.cpu()), _bits(want_pool))
    for o in outs:
        torch.testing.assert_close(o.float(), want.float(), **TOL)
        assert torch.equal(_bits(o), _bits(outs[0]))


def test_drop_in_cache_runs_the_decode_kernel_on_large_steps():
    # the reference's call sequence (write, then attention) and the fused
    # decode_step both attach the streaming kernel's plan on the headline step
    from tinybatch_amd.kv_cache import PagedKVCache

    wl = make_decode_workload("qwen-fp16-b64")
    c = dict(pool=wl.pool, tables=wl.block_tables, ctx=wl.context_lens, q=wl.q, k=wl.k_new, v=wl.v_new,
             NB=wl.num_blocks, BS=16, Hq=14, Hkv=2, D=64, dtype=torch.float16)
    want, want_pool = oracle(c)
    B = len(c["ctx"])
    pos = torch.tensor([x - 1 for x in c["ctx"]], dtype=torch.int64, device=DEV)
    slices = [(b, b + 1) for b in range(B)]
    q, k, v = c["q"].to(DEV), c["k"].to(DEV), c["v"].to(DEV)
    for fused in (False, True):
        cache = PagedKVCache(1, c["NB"], 16, 2, 64, DEV, torch.float16)
        cache.pools[0].copy_(c["pool"].to(DEV))
        if fused:
            meta = cache.step_metadata(pos, slices, c["tables"], c["ctx"], num_heads=14)
            out = cache.decode_step(0, q, k, v, meta)
        else:
            cache.write(0, k, v, pos, slices, c["tables"])
            out = cache.attention(0, q, pos, slices, c["tables"], c["ctx"])
            meta = cache.step_metadata(pos, slices, c["tables"], c["ctx"], cache.rows_per_item(14), num_heads=14)
        torch.cuda.synchronize()
        assert meta.decode_plan is not None, f"fused={fused}: the step did not take the decode kernel"
        assert torch.equal(_bits(cache.pools[0].cpu()), _bits(want_pool)), f"fused={fused}"
        torch.testing.assert_close(out.cpu().float(), want.float(), **TOL)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_rope_equals_rotating_first(dtype):
    c = case(13, 24, 14, 2, 64, 16, dtype, nan_stale=False)
    cos, sin = rope_tables(64, 1e6, 8192, DEV)
    rope = ops.Rope(cos, sin)
    pos = torch.tensor([x - 1 for x in c["ctx"]], dtype=torch.int64, device=DEV)
    meta = decode_meta(c["ctx"], c["tables"], c["NB"], 16, 14, 2, 64, dtype)
    q, k, v = c["q"].to(DEV), c["k"].to(DEV), c["v"].to(DEV)
    pool_a = c["pool"].to(DEV)
    out_a = ops.paged_attention(q, pool_a, meta, num_heads=14, k_new=k, v_new=v, rope=rope)
    # rotate first (the separate RoPE kernel), then the same call without rope
    qkv = torch.cat([q.reshape(len(c["ctx"]), -1), k.reshape(len(c["ctx"]), -1), v.reshape(len(c["ctx"]), -1)], 1)
    qr, kr = layer_ops.rope_qk(qkv.contiguous(), pos, cos, sin, 14, 2, 64)
    pool_b = c["pool"].to(DEV)
    out_b = ops.paged_attention(qr.contiguous(), pool_b, meta, num_heads=14, k_new=kr.contiguous(), v_new=v)
    torch.cuda.synchronize()
    assert torch.equal(_bits(pool_a), _bits(pool_b))
    assert torch.equal(_bits(out_a), _bits(out_b))


def test_shared_slot_refused_by_the_fused_append():
    c = case(14, 3, 14, 2, 64, 16, torch.float16, ctx=[20, 40, 36], nan_stale=False)
    c["tables"][2][2] = c["tables"][0][1]                     # rows 0 and 2 write one slot
    meta = decode_meta(c["ctx"], c["tables"], c["NB"], 16, 14, 2, 64, torch.float16)
    with pytest.raises(ValueError, match="one pool slot"):
        ops.paged_attention(c["q"].to(DEV), c["pool"].to(DEV), meta, num_heads=14, k_new=c["k"].to(DEV),
                            v_new=c["v"].to(DEV))


def _c_decode(c, meta, q, pool, out, k, v, bufs, violations, plan=None):
    """tb_paged_decode through the C ABI with a private error counter and buffers."""
    from tinybatch_amd import _lib

    plan = meta.decode_plan if plan is None else plan
    D, Hq, Hkv = c["D"], c["Hq"], c["Hkv"]
    return _lib.lib().tb_paged_decode(
        q.data_ptr(), Hq * D, pool.data_ptr(), pool.shape[0], out.data_ptr(), Hq * D, len(c["ctx"]),
        plan.data_ptr(), meta.decode_workgroups, meta.decode_waves, meta.decode_stride, Hq, Hkv, D, c["BS"],
        float(D ** -0.5), _lib.DTYPE_CODE[c["dtype"]], None if k is None else k.data_ptr(), Hkv * D,
        None if v is None else v.data_ptr(), Hkv * D, bufs.pieces.data_ptr(), bufs.pieces.numel(),
        meta.decode_pieces, bufs.arrivals.data_ptr(), bufs.units, violations.data_ptr(), None, None, 0,
        _lib.stream_handle(DEV))


def test_c_abi_refuses_a_fused_call_on_a_plan_with_a_shared_newest_slot():
    """Two rows whose newest positions share a pool slot: the plan builder marks every
    count word, and a fused tb_paged_decode on it counts one error and writes nothing
    (the reference's last writer wins, kv_cache.py:33-38); the same plan without k_new,
    after the slot-mapped append, serves the step."""
    c = case(21, 40, 14, 2, 64, 16, torch.float16, ctx=[900 + 37 * i for i in range(40)], nan_stale=False)
    c["tables"][5][-1] = c["tables"][2][-1]
    c["ctx"][5] = (len(c["tables"][5]) - 1) * 16 + (c["ctx"][2] - 1) % 16 + 1   # row 5's newest slot = row 2's
    meta = decode_meta(c["ctx"], c["tables"], c["NB"], 16, 14, 2, 64, torch.float16)
    workers = meta.decode_workgroups * meta.decode_waves
    assert np.all(meta.decode_plan[:workers].cpu().numpy() & (1 << 30))   # TB_DECODE_SHARED_NEWEST
    q, k, v = c["q"].to(DEV), c["k"].to(DEV), c["v"].to(DEV)
    pool = c["pool"].to(DEV)
    out = torch.full((40, 14 * 64), 7.0, dtype=torch.float16, device=DEV)
    bufs = ops.DecodeBuffers(DEV, ops.decode_workspace_bytes(meta, 14, 2, 64), meta.decode_units)
    viol = torch.zeros(1, dtype=torch.int32, device=DEV)
    assert _c_decode(c, meta, q, pool, out, k, v, bufs, viol) == 0
    torch.cuda.synchronize()
    assert int(viol.item()) == 1
    assert torch.equal(_bits(pool.cpu()), _bits(c["pool"])) and bool((out == 7.0).all())
    # unfused: the append (last writer wins) and then attention from the pool
    want, want_pool = oracle(c)
    ops.kv_append(pool, k, v, meta.slot_mapping)
    assert _c_decode(c, meta, q, pool, out, None, None, bufs, viol) == 0
    torch.cuda.synchronize()
    assert int(viol.item()) == 1
    assert torch.equal(_bits(pool.cpu()), _bits(want_pool))
    torch.testing.assert_close(out.cpu().float(), want.float(), **TOL)


def test_malformed_plan_count_is_counted():
    """A worker count the plan builder never writes (odd, or past the stride): that
    worker streams nothing and the call's error count says so, instead of rows left
    silently unwritten."""
    c = case(22, 64, 14, 2, 64, 16, torch.float16, nan_stale=False)
    meta = decode_meta(c["ctx"], c["tables"], c["NB"], 16, 14, 2, 64, torch.float16)
    q = c["q"].to(DEV)
    pool = c["pool"].to(DEV)
    out = torch.empty(64, 14 * 64, dtype=torch.float16, device=DEV)
    workers = meta.decode_workgroups * meta.decode_waves
    plan_host = meta.decode_plan.cpu().numpy()
    for bad in (int(plan_host[0]) + 1, meta.decode_stride + 2):
        host = plan_host.copy()
        host[0] = bad
        plan = torch.from_numpy(host).to(DEV)
        bufs = ops.DecodeBuffers(DEV, ops.decode_workspace_bytes(meta, 14, 2, 64), meta.decode_units)
        viol = torch.zeros(1, dtype=torch.int32, device=DEV)
        assert _c_decode(c, meta, q, pool, out, None, None, bufs, viol, plan=plan) == 0
        torch.cuda.synchronize()
        assert int(viol.item()) == 1, bad
    # the valid plan, fresh counters: no error
    bufs = ops.DecodeBuffers(DEV, ops.decode_workspace_bytes(meta, 14, 2, 64), meta.decode_units)
    viol = torch.zeros(1, dtype=torch.int32, device=DEV)
    assert _c_decode(c, meta, q, pool, out, None, None, bufs, viol) == 0
    torch.cuda.synchronize()
    assert int(viol.item()) == 0 and workers > 0


@pytest.mark.parametrize("name,batch,waves", [("qwen-fp16-b64", 0, 4), ("qwen-fp16-b64", 0, 8),
                                              ("llama-bf16-b256", 48, 4)])
def test_device_built_plan_equals_the_host_plan(name, batch, waves):
    """The plan the device writes from the segment descriptors (tb_expand_decode_plan)
    is the host builder's, word for word: count words and every worker's entries."""
    from tinybatch_amd.metadata import attach_decode_plan as attach

    wl = make_decode_workload(name, **({"batch": batch} if batch else {}))
    dd = ops.decode_device(DEV)
    metas = []
    for on_device in (False, True):
        meta = build_step_metadata(wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens,
                                   block_size=16, num_blocks=wl.num_blocks,
                                   partition_tokens=ops.partition_tokens(wl.dtype, wl.head_dim))
        assert attach(meta, num_heads=wl.num_heads, num_kv_heads=wl.num_kv_heads, head_dim=wl.head_dim,
                      dtype=wl.dtype, workgroups=dd.workgroups, num_xcds=dd.num_xcds, waves=waves,
                      on_device=on_device)
        metas.append(meta.to(DEV))
    torch.cuda.synchronize()
    host, dev = (m.decode_plan.cpu().numpy() for m in metas)
    W = dd.workgroups * waves
    stride = metas[0].decode_stride
    assert metas[1].decode_stride == stride and metas[1].decode_pieces == metas[0].decode_pieces
    np.testing.assert_array_equal(dev[:W], host[:W])
    base = (W + 3) // 4 * 4
    he = host[base:base + W * stride * 4].reshape(W, stride, 4)
    de = dev[base:base + W * stride * 4].reshape(W, stride, 4)
    for k in range(W):
        n = int(host[k]) & 0x3FFFFFFF
        np.testing.assert_array_equal(de[k, :n], he[k, :n])
    assert dd.errors() == 0


def test_device_built_plan_counts_bad_block_ids_instead_of_reading_outside_the_pool():
    """A table entry outside the pool reaching tb_expand_decode_plan (the host builders
    raise IndexError first): counted in the error word and replaced by block 0."""
    from tinybatch_amd import _lib
    from tinybatch_amd.metadata import build_decode_segments

    ctx = [100, 70]
    tables = np.array([[3, 4, 5, 6, 7, 8, 9], [0, 1, 2, 10, 11, 0, 0]], dtype=np.int32)
    counts, segs, waves, stride, pieces = build_decode_segments(ctx, tables, block_size=16, num_kv_heads=2,
                                                                 head_dim=64, workgroups=8, num_xcds=8, waves=4)
    bad = tables.copy()
    bad[1, 2] = 1 << 20                                     # outside a 12-block pool
    W = 32
    plan = torch.zeros(int(_lib.lib().tb_decode_plan_words(W, stride)), dtype=torch.int32, device=DEV)
    segs_d = torch.from_numpy(segs).to(DEV)
    tab_d = torch.from_numpy(bad).to(DEV)
    errs = torch.zeros(1, dtype=torch.int32, device=DEV)
    assert _lib.lib().tb_expand_decode_plan(segs_d.data_ptr(), segs.shape[0], tab_d.data_ptr(), 7, 16, 12, 2, 64, W,
                                            stride, plan.data_ptr(), errs.data_ptr(), _lib.stream_handle(DEV)) == 0
    torch.cuda.synchronize()
    # the tile in block index 2 of both kv heads' units (and a pad that repeats it) is counted
    assert int(errs.item()) >= 2
    base = (W + 3) // 4 * 4
    host = plan.cpu().numpy()
    ents = host[base:base + W * stride * 4].reshape(W, stride, 4)
    blk_bytes = 2 * 2 * 16 * 64 * 2
    for k in range(W):
        n = int(host[k]) & 0x3FFFFFFF
        assert np.all((ents[k, :n, 0].astype(np.int64) << 8) < 12 * blk_bytes)   # inside the pool
