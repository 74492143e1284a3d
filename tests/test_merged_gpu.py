"""tb_paged_attention_merged (split rows merged inside the launch of the work-item
kernel) through the C ABI: the same bits as tb_paged_attention with its combine
kernel, and the oracle's result (rtol = atol = 2e-2 at fp16 / bf16); appended rows
bit-exact; no row group merged across XCDs."""
import pytest
import torch

from oracle import reference_path as ref
from tinybatch_amd import ops
from tinybatch_amd.metadata import build_step_metadata
from tinybatch_amd.model import rope_tables
from tinybatch_amd.workloads import make_decode_workload

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
TOL = dict(atol=2e-2, rtol=2e-2)


def _bits(t):
    return t.contiguous().view(torch.int16)


def case(seed, B, Hq, Hkv, D, BS, dtype, lo=1, hi=3000):
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(lo, hi, (B,), generator=g).tolist()
    need = [(c + BS - 1) // BS for c in ctx]
    NB = sum(need) + 3
    perm = torch.randperm(NB, generator=g).tolist()
    tables, at = [], 0
    for n in need:
        tables.append(perm[at:at + n])
        at += n
    pool = torch.randn(NB, 2, Hkv, BS, D, generator=g).to(dtype)
    q = torch.randn(B, Hq, D, generator=g).to(dtype)
    k = torch.randn(B, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, Hkv, D, generator=g).to(dtype)
    return dict(ctx=ctx, tables=tables, NB=NB, pool=pool, q=q, k=k, v=v, Hq=Hq, Hkv=Hkv, D=D, BS=BS, dtype=dtype)


def run(c, merged, fused=True, rope=None):
    meta = build_step_metadata([x - 1 for x in c["ctx"]], [(b, b + 1) for b in range(len(c["ctx"]))], c["tables"],
                               c["ctx"], block_size=c["BS"], num_blocks=c["NB"],
                               partition_tokens=ops.partition_tokens(c["dtype"], c["D"]))
    if merged:
        assert ops.attach_xcd_slot_map(meta, num_heads=c["Hq"], num_kv_heads=c["Hkv"], dtype=c["dtype"], device=DEV)
    meta.to(DEV)
    pool = c["pool"].to(DEV)
    q, k, v = c["q"].to(DEV), c["k"].to(DEV), c["v"].to(DEV)
    if fused:
        out = ops.paged_attention(q, pool, meta, num_heads=c["Hq"], k_new=k, v_new=v, rope=rope)
    else:
        ops.kv_append(pool, k, v, meta.slot_mapping)
        out = ops.paged_attention(q, pool, meta, num_heads=c["Hq"], rope=rope)
    torch.cuda.synchronize()
    return out.cpu(), pool.cpu()


def check(c, fused=True):
    if not ops.decode_device(DEV).merge_in_kernel:
        pytest.skip("this GPU does not run workgroup g on XCD g mod the XCD count")
    got, pool = run(c, True, fused)
    base, base_pool = run(c, False, fused)
    assert torch.equal(_bits(got), _bits(base)), "merged launch differs from the combine kernel"
    assert torch.equal(_bits(pool), _bits(base_pool))
    want_pool = c["pool"].clone()
    want = ref.decode_step(want_pool, c["q"], c["k"], c["v"], [x - 1 for x in c["ctx"]], c["tables"], c["Hq"],
                           c["Hkv"], c["BS"])
    assert torch.equal(_bits(pool), _bits(want_pool)), "pool differs (append)"
    torch.testing.assert_close(got.float(), want.float(), **TOL)
    assert int(ops.decode_device(DEV).violations.item()) == 0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_headline_shape(dtype):
    wl = make_decode_workload("qwen-fp16-b64")
    c = dict(ctx=wl.context_lens, tables=wl.block_tables, NB=wl.num_blocks, pool=wl.pool.to(dtype), q=wl.q.to(dtype),
             k=wl.k_new.to(dtype), v=wl.v_new.to(dtype), Hq=14, Hkv=2, D=64, BS=16, dtype=dtype)
    check(c)


@pytest.mark.parametrize("Hq,Hkv,D,BS", [(14, 2, 64, 16), (32, 8, 128, 16), (8, 8, 64, 32), (16, 1, 128, 64),
                                         (12, 4, 64, 4)])
def test_geometries(Hq, Hkv, D, BS):
    check(case(Hq * D + BS, 37, Hq, Hkv, D, BS, torch.bfloat16))


def test_unfused_and_long_rows():
    check(case(3, 9, 14, 2, 64, 16, torch.float16, lo=4000, hi=9000), fused=False)


def test_repeated_calls_leave_counters_zero():
    c = case(4, 20, 14, 2, 64, 16, torch.bfloat16)
    if not ops.decode_device(DEV).merge_in_kernel:
        pytest.skip("this GPU does not run workgroup g on XCD g mod the XCD count")
    outs = [run(c, True, fused=False)[0] for _ in range(3)]
    assert all(torch.equal(_bits(o), _bits(outs[0])) for o in outs)
    assert int(ops.decode_device(DEV).violations.item()) == 0


def test_fused_rope():
    c = case(5, 24, 14, 2, 64, 16, torch.bfloat16)
    if not ops.decode_device(DEV).merge_in_kernel:
        pytest.skip("this GPU does not run workgroup g on XCD g mod the XCD count")
    cos, sin = rope_tables(64, 1e6, 8192, DEV)
    rope = ops.Rope(cos, sin)
    a, pa = run(c, True, rope=rope)
    b, pb = run(c, False, rope=rope)
    assert torch.equal(_bits(a), _bits(b)) and torch.equal(_bits(pa), _bits(pb))
