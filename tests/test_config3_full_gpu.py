"""The Llama-3-8B-geometry decode step at its full size on the GPU: 32 query /
8 KV heads, head_dim 128, bf16, 256 sequences with log-normal contexts (median
8192, sigma 0.5 or 1.0, clipped to [1024, 32768]), one pool sized to fit every
sequence (135,657 blocks of 64 KiB, 8.9 GB, at sigma 0.5; 175,571 blocks, 11.5
GB, 13 contexts at the 32768 clip, at sigma 1.0), values N(0,1) drawn on the GPU.

The whole batch runs through the fused append + attention launch, once through
the work items and once through the streaming decode kernel (its plan built on
the device; the second append writes the same rows again). Sixteen
sequences are then checked against the oracle: their blocks before the step
(and after it) are brought back to the host, their tables remapped onto a
compact pool, and the oracle's append + attention run there. Byte offsets of
blocks with ids >= 65536 lie past 4 GiB of the pool (the kernels' 64-bit
addressing); the selection includes the sequence holding the pool's last
block and the longest and shortest contexts. Bars: the appended rows bit-exact,
attention rtol = atol = 2e-2 (reference pool layout: kv_cache.py:17-20).
"""
import pytest
import torch

from oracle import reference_path as ref
from tinybatch_amd import ops
from tinybatch_amd.metadata import build_step_metadata
from tinybatch_amd.workloads import make_decode_workload

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


@pytest.mark.parametrize("name", ["llama-bf16-b256", "llama-bf16-b256-s1"])
def test_config3_full_pool_fused_decode_bf16(name):
    wl = make_decode_workload(name, pool_device=DEV)
    blk_bytes = wl.pool[0].numel() * wl.pool.element_size()
    past_4g = (1 << 32) // blk_bytes
    assert wl.num_blocks > past_4g and wl.batch == 256
    print(f"[config3] NB={wl.num_blocks} ({wl.num_blocks * blk_bytes / 1e9:.2f} GB), blocks >= {past_4g} "
          f"lie past 4 GiB", flush=True)

    ctx = wl.context_lens
    order = sorted(range(wl.batch), key=lambda b: ctx[b])
    last_owner = next(b for b, t in enumerate(wl.block_tables) if wl.num_blocks - 1 in t)
    g = torch.Generator().manual_seed(31)
    pick = {order[0], order[1], order[-1], order[-2], last_owner}
    pick |= set([b for b in range(wl.batch) if ctx[b] == max(ctx)][:6])      # contexts at the clip (sigma 1.0)
    for b in torch.randperm(wl.batch, generator=g).tolist():
        if len(pick) >= 16:
            break
        pick.add(b)
    pick = sorted(pick)
    assert sum(max(wl.block_tables[b]) >= past_4g for b in pick) >= 8

    # the selected sequences' blocks, before the step, on the host
    used = [wl.block_tables[b] for b in pick]
    flat = torch.tensor(sum(used, []), dtype=torch.int64, device=DEV)
    before = wl.pool.index_select(0, flat).cpu()

    outs = {}
    for kernel in ("items", "decode"):
        meta = build_step_metadata(wl.positions, wl.seq_slices, wl.block_tables, ctx, block_size=wl.block_size,
                                   num_blocks=wl.num_blocks,
                                   partition_tokens=ops.partition_tokens(wl.dtype, wl.head_dim))
        if kernel == "decode":
            assert ops.attach_decode_plan(meta, num_heads=wl.num_heads, num_kv_heads=wl.num_kv_heads,
                                          head_dim=wl.head_dim, dtype=wl.dtype, device=DEV)
        meta.to(DEV)
        out = ops.paged_attention(wl.q.to(DEV), wl.pool, meta, num_heads=wl.num_heads, k_new=wl.k_new.to(DEV),
                                  v_new=wl.v_new.to(DEV))
        outs[kernel] = out[torch.tensor(pick, device=DEV)].cpu()
    after = wl.pool.index_select(0, flat).cpu()
    torch.cuda.synchronize()
    assert ops.decode_device(DEV).errors() == 0

    # the oracle on a compact pool holding just these blocks
    tables, at = [], 0
    for t in used:
        tables.append(list(range(at, at + len(t))))
        at += len(t)
    want_pool = before.clone()
    sel = torch.tensor(pick)
    want = ref.decode_step(want_pool, wl.q[sel], wl.k_new[sel], wl.v_new[sel], [wl.cached_lens[b] for b in pick],
                           tables, wl.num_heads, wl.num_kv_heads, wl.block_size)
    assert torch.equal(after.view(torch.int16), want_pool.view(torch.int16)), "appended rows differ"
    assert not torch.equal(before.view(torch.int16), after.view(torch.int16))
    for kernel, got in outs.items():
        err = (got.float() - want.float()).abs().max().item()
        print(f"[config3] {name} {kernel}: {len(pick)} sequences, contexts {min(ctx[b] for b in pick)}.."
              f"{max(ctx[b] for b in pick)}: attention max|err| {err:.3e}", flush=True)
        torch.testing.assert_close(got.float(), want.float(), atol=2e-2, rtol=2e-2)
