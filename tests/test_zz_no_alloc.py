"""tb_paged_attention_noalloc (the allocation-free entry point, partials in the
library's static per-GPU scratch) against tb_paged_attention with a caller
workspace: the same kernels, so the same bits, on two calls in a row, the
second smaller than the first (the scratch keeps the first call's partials,
which the second must not read); the call makes no allocation through torch's
allocator (its allocation count is unchanged across it); and the call captured
in a HIP graph gives the same bits on every replay, with other work between."""
import pytest
import torch

from tinybatch_amd import ops
from tinybatch_amd.metadata import build_step_metadata
from tinybatch_amd.workloads import make_decode_workload

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _bits(t):
    return t.contiguous().view(torch.int16)


def _both(wl, fused: bool):
    meta = build_step_metadata(wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens,
                               block_size=wl.block_size, num_blocks=wl.num_blocks,
                               partition_tokens=ops.partition_tokens(wl.dtype, wl.head_dim)).to(DEV)
    assert meta.max_parts_per_row > 1          # the partials (scratch) are in use
    pools = [wl.pool.to(DEV), wl.pool.to(DEV)]
    q = wl.q.to(DEV)
    kv = dict(k_new=wl.k_new.to(DEV), v_new=wl.v_new.to(DEV)) if fused else {}
    outs = [torch.full((wl.batch, wl.num_heads * wl.head_dim), float("nan"), dtype=wl.dtype, device=DEV)
            for _ in range(2)]
    ops.paged_attention(q, pools[0], meta, num_heads=wl.num_heads, out=outs[0], **kv)
    torch.cuda.synchronize()
    allocs = torch.cuda.memory_stats(DEV)["allocation.all.allocated"]
    ops.paged_attention(q, pools[1], meta, num_heads=wl.num_heads, out=outs[1], noalloc=True, **kv)
    torch.cuda.synchronize()
    assert torch.cuda.memory_stats(DEV)["allocation.all.allocated"] == allocs
    return outs, pools


def test_noalloc_entry_point_matches_the_workspace_one_on_two_calls():
    # first call: the 64-sequence fp16 decode step (fused append), 582 partitions
    wl = make_decode_workload("qwen-fp16-b64")
    outs, pools = _both(wl, fused=True)
    assert torch.equal(_bits(outs[0]), _bits(outs[1]))
    assert torch.equal(_bits(pools[0]), _bits(pools[1]))
    # second call, smaller: 6 sequences of another draw, separate append
    wl = make_decode_workload("qwen-fp16-b64", seed=9, batch=6)
    outs2, _ = _both(wl, fused=False)
    assert torch.equal(_bits(outs2[0]), _bits(outs2[1]))
    assert not torch.isnan(outs2[1].float()).any()


def test_noalloc_needs_an_output_buffer():
    wl = make_decode_workload("qwen-fp16-b64", batch=2)
    meta = build_step_metadata(wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens,
                               block_size=wl.block_size, num_blocks=wl.num_blocks,
                               partition_tokens=ops.partition_tokens(wl.dtype, wl.head_dim)).to(DEV)
    with pytest.raises(ValueError, match="output buffer"):
        ops.paged_attention(wl.q.to(DEV), wl.pool.to(DEV), meta, num_heads=wl.num_heads, noalloc=True)


def test_noalloc_call_replays_from_a_captured_graph():
    wl = make_decode_workload("qwen-fp16-b64", seed=5, batch=16)
    meta = build_step_metadata(wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens,
                               block_size=wl.block_size, num_blocks=wl.num_blocks,
                               partition_tokens=ops.partition_tokens(wl.dtype, wl.head_dim)).to(DEV)
    assert meta.max_parts_per_row > 1
    pool, q = wl.pool.to(DEV), wl.q.to(DEV)
    want = ops.paged_attention(q, pool, meta, num_heads=wl.num_heads)
    out = torch.full((wl.batch, wl.num_heads * wl.head_dim), float("nan"), dtype=wl.dtype, device=DEV)
    ops.paged_attention(q, pool, meta, num_heads=wl.num_heads, out=out, noalloc=True)   # eager, before capture
    torch.cuda.synchronize()
    assert torch.equal(_bits(out), _bits(want))
    g = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream(device=DEV)
    stream.wait_stream(torch.cuda.current_stream(DEV))
    with torch.cuda.graph(g, stream=stream):
        ops.paged_attention(q, pool, meta, num_heads=wl.num_heads, out=out, noalloc=True)
    for i in range(4):
        out.fill_(float("nan"))                    # eager work between the replays
        other = ops.paged_attention(q, pool, meta, num_heads=wl.num_heads)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(_bits(out), _bits(want)), f"replay {i}"
        assert torch.equal(_bits(other), _bits(want))
