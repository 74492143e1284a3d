"""The engine on the GPU against the oracle: model forward logits, and whole
continuous-batching runs (prefix hits, block-multiple prompts, mixed steps)
token for token against the same schedule driven through the CPU restatement."""
import pytest
import torch

from oracle import model_reference as mref
from tinybatch_amd import ops
from tinybatch_amd.block_manager import BlockManager
from tinybatch_amd.config import EngineConfig
from tinybatch_amd.engine import LLMEngine
from tinybatch_amd.kv_cache import PagedKVCache
from tinybatch_amd.model import ModelConfig, Qwen2Paged
from tinybatch_amd.scheduler import Request, Scheduler

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def small_cfg(layers=2, heads=2, kv_heads=1, vocab=300):
    return ModelConfig(n_layers=layers, n_heads=heads, n_kv_heads=kv_heads, d_model=64 * heads, head_dim=64,
                       d_ff=256, vocab_size=vocab, rms_eps=1e-6, rope_theta=1e6, tie_embeddings=True,
                       max_position=2048)


def cpu_weights(model):
    return {k: v.detach().float().cpu() for k, v in model.reference_weights().items()}


def test_forward_logits_match_oracle_fp32_mixed_step():
    mc = small_cfg(layers=3, heads=4, kv_heads=2)
    model = Qwen2Paged(mc, DEV, torch.float32, seed=1)
    w = cpu_weights(model)
    BS, NB = 16, 64
    cache = PagedKVCache(mc.n_layers, NB, BS, mc.n_kv_heads, mc.head_dim, DEV, torch.float32)
    pools = [torch.zeros(NB, 2, mc.n_kv_heads, BS, mc.head_dim) for _ in range(mc.n_layers)]
    g = torch.Generator().manual_seed(2)
    # step 1: two prefills (one of exactly two blocks); step 2: both decode + a new prefill
    tables = [[5, 9, 2], [11, 3, 6], [7, 1, 0, 4]]   # the 32-token prompt has its decode block
    p0 = torch.randint(0, mc.vocab_size, (40,), generator=g).tolist()
    p1 = torch.randint(0, mc.vocab_size, (32,), generator=g).tolist()
    p2 = torch.randint(0, mc.vocab_size, (50,), generator=g).tolist()
    steps = [
        (p0 + p1, list(range(40)) + list(range(32)), [(0, 40), (40, 72)], tables[:2], [40, 32]),
        (p2 + [7, 8], list(range(50)) + [40, 32], [(0, 50), (50, 51), (51, 52)], [tables[2]] + tables[:2],
         [50, 41, 33]),
    ]
    for ids, pos, slices, tbls, ctx in steps:
        ids_t, pos_t = torch.tensor(ids), torch.tensor(pos)
        got = model.forward(ids_t.to(DEV), pos_t.to(DEV), slices, tbls, ctx, cache)
        want = mref.forward(w, mc, ids_t, pos_t, slices, tbls, ctx, pools, BS)
        torch.cuda.synchronize()
        torch.testing.assert_close(got.cpu(), want, atol=2e-4, rtol=2e-4)
    for layer in range(mc.n_layers):
        torch.testing.assert_close(cache.pools[layer].cpu(), pools[layer], atol=1e-5, rtol=1e-5)


def test_fused_mlp_bf16_forward_as_close_to_the_oracle_as_the_library_path():
    """Decode-sized bf16 batches (<= 32 rows) with the split-K o/down
    projections and gate/up + SwiGLU fused (fused_mlp) against the same model
    on the library GEMMs: both against the fp32 oracle of the same bf16
    weights, the fused path no further off than twice the library path."""
    mc = small_cfg(layers=2, heads=4, kv_heads=2)
    model = Qwen2Paged(mc, DEV, torch.bfloat16, seed=11)
    w = cpu_weights(model)
    BS, NB = 16, 32
    g = torch.Generator().manual_seed(12)
    tables = [[5, 9], [11, 3]]
    p0 = torch.randint(0, mc.vocab_size, (20,), generator=g).tolist()
    p1 = torch.randint(0, mc.vocab_size, (10,), generator=g).tolist()
    steps = [(p0 + p1, list(range(20)) + list(range(10)), [(0, 20), (20, 30)], [20, 10]),
             ([7, 8], [20, 10], [(0, 1), (1, 2)], [21, 11])]
    pools = [torch.zeros(NB, 2, mc.n_kv_heads, BS, mc.head_dim) for _ in range(mc.n_layers)]
    want = [mref.forward(w, mc, torch.tensor(ids), torch.tensor(pos), sl, tables, ctx, pools, BS)
            for ids, pos, sl, ctx in steps]
    errs = {}
    for fused in (False, True):
        model.fused_mlp = fused
        cache = PagedKVCache(mc.n_layers, NB, BS, mc.n_kv_heads, mc.head_dim, DEV, torch.bfloat16)
        errs[fused] = 0.0
        for (ids, pos, sl, ctx), ref in zip(steps, want):
            got = model.forward(torch.tensor(ids, device=DEV), torch.tensor(pos, device=DEV), sl, tables, ctx, cache)
            errs[fused] = max(errs[fused], float((got.cpu() - ref).abs().max()))
    scale = max(float(r.abs().max()) for r in want)
    assert errs[False] < 0.05 * scale, errs
    assert errs[True] <= 2 * errs[False] + 1e-3 * scale, errs


def oracle_generate(model, ecfg, prompts, max_new):
    """The engine loop with the CPU restatement as the forward pass."""
    mc = model.cfg
    w = cpu_weights(model)
    bm = BlockManager(ecfg.num_blocks, ecfg.block_size, ecfg.enable_prefix_caching)
    sch = Scheduler(ecfg, bm)
    pools = [torch.zeros(ecfg.num_blocks, 2, mc.n_kv_heads, ecfg.block_size, mc.head_dim)
             for _ in range(mc.n_layers)]
    reqs = [Request(prompt_token_ids=list(p), max_new_tokens=m) for p, m in zip(prompts, max_new)]
    for r in reqs:
        sch.add(r)
    while sch.has_work():
        b = sch.schedule()
        ordered = b.prefill + b.decode
        ids, pos, slices, tables, ctx = LLMEngine.build_step(b.prefill, b.decode)
        logits = mref.forward(w, mc, torch.tensor(ids), torch.tensor(pos), slices, tables, ctx, pools,
                              ecfg.block_size)
        for r, t in zip(ordered, logits.argmax(-1).tolist()):
            r.output_token_ids.append(int(t))
            if len(r.output_token_ids) >= r.max_new_tokens:
                sch.finish(r)
    return [r.output_token_ids for r in reqs], bm.hit_rate()


@pytest.mark.parametrize("graphs", [True, False])
def test_engine_generation_matches_oracle_token_for_token_fp32(graphs):
    """Eager steps, and decode steps replayed from captured graphs (batch buckets
    1, 2, 4, 5 with padded rows), against the oracle-driven schedule."""
    mc = small_cfg(layers=2, heads=4, kv_heads=2)
    ecfg = EngineConfig(dtype="float32", num_blocks=96, block_size=16, max_batch_tokens=160, max_running=5,
                        decode_graphs=graphs)
    model = Qwen2Paged(mc, DEV, torch.float32, seed=3)
    g = torch.Generator().manual_seed(4)
    shared = torch.randint(0, mc.vocab_size, (48,), generator=g).tolist()      # three full blocks
    prompts = [shared + torch.randint(0, mc.vocab_size, (n,), generator=g).tolist() for n in (5, 17, 0)]
    prompts += [torch.randint(0, mc.vocab_size, (n,), generator=g).tolist() for n in (32, 9, 70)]
    max_new = [12, 7, 20, 15, 30, 9]
    eng = LLMEngine(ecfg, model=model)
    reqs = [eng.add_request(p, max_new_tokens=m) for p, m in zip(prompts, max_new)]
    while eng.has_work():
        eng.step()
    want, hit_rate = oracle_generate(model, ecfg, prompts, max_new)
    assert [r.output_token_ids for r in reqs] == want
    assert eng.block_manager.hit_rate() == hit_rate > 0
    assert [len(r.output_token_ids) for r in reqs] == max_new
    assert (eng.graph_steps > 0) == graphs


def test_engine_qwen_dims_bf16_runs_with_prefix_hits():
    """0.5B dimensions in bf16 (two layers to keep it short): the tiled prefill,
    the row-group work items and decode all run inside one engine."""
    mc = ModelConfig.qwen2_0_5b()
    mc.n_layers = 2
    ecfg = EngineConfig(num_blocks=256, max_batch_tokens=2048, max_running=8)
    eng = LLMEngine(ecfg, model_config=mc)
    g = torch.Generator().manual_seed(5)
    prefix = torch.randint(0, mc.vocab_size, (400,), generator=g).tolist()
    prompts = [prefix + torch.randint(0, mc.vocab_size, (n,), generator=g).tolist() for n in (1, 60, 111)]
    prompts += [torch.randint(0, mc.vocab_size, (n,), generator=g).tolist() for n in (32, 512)]
    outs = eng.generate(prompts, max_new_tokens=6)
    assert [len(o) for o in outs] == [6] * 5
    assert eng.block_manager.hit_rate() > 0
    assert all(0 <= t < mc.vocab_size for o in outs for t in o)


def test_decode_graph_replays_match_eager_steps_bf16():
    """The same decode steps through a captured graph and eagerly (fused vs
    separate append, padded bucket rows): identical K/V written and next tokens
    within bf16 noise of each other's logits."""
    from tinybatch_amd.decode_graphs import DecodeGraphs
    mc = small_cfg(layers=2, heads=14, kv_heads=2, vocab=500)
    model = Qwen2Paged(mc, DEV, torch.bfloat16, seed=7)
    BS, NB = 16, 128
    caches = [PagedKVCache(mc.n_layers, NB, BS, mc.n_kv_heads, mc.head_dim, DEV, torch.bfloat16) for _ in range(2)]
    g = torch.Generator().manual_seed(8)
    lens = [37, 300, 16, 64, 129]
    tables, at = [], 0
    for n in lens:
        k = n // BS + 1
        tables.append(list(range(at, at + k))); at += k
    prompts = [torch.randint(0, mc.vocab_size, (n,), generator=g).tolist() for n in lens]
    ids = torch.tensor(sum(prompts, []), device=DEV)
    pos = torch.tensor(sum([list(range(n)) for n in lens], []), device=DEV)
    slices, at = [], 0
    for n in lens:
        slices.append((at, at + n)); at += n
    for cache in caches:                                     # the same prefill into both caches
        model.forward(ids, pos, slices, tables, lens, cache)
    graphs = DecodeGraphs(model, caches[1], max_batch=8, max_model_len=1024)
    toks = [p[-1] for p in prompts]
    ctx = list(lens)
    for _ in range(3):
        positions = list(ctx)
        ctx = [c + 1 for c in ctx]
        eager = model.forward(torch.tensor(toks, device=DEV), torch.tensor(positions, device=DEV),
                              [(i, i + 1) for i in range(len(toks))], tables, ctx, caches[0])
        got = graphs.run(toks, positions, tables, ctx)
        top2 = eager.topk(2, dim=-1)
        for b, t in enumerate(got):
            if t != int(top2.indices[b, 0]):                 # only a near tie may differ
                assert float(top2.values[b, 0] - eager[b, t]) < 0.05
        toks = got
    torch.cuda.synchronize()
    for layer in range(mc.n_layers):
        a, b = caches[0].pools[layer], caches[1].pools[layer]
        assert torch.equal(a[:sum(len(t) for t in tables)].view(torch.int16)[:, 1],
                           b[:sum(len(t) for t in tables)].view(torch.int16)[:, 1]) or \
            torch.allclose(a.float(), b.float(), atol=2e-2, rtol=2e-2)


def _prefilled_caches(model, mc, lens, n, BS=16, NB=256, seed=8):
    g = torch.Generator().manual_seed(seed)
    tables, at = [], 0
    for L in lens:
        k = L // BS + 1
        tables.append(list(range(at, at + k)))
        at += k
    prompts = [torch.randint(0, mc.vocab_size, (L,), generator=g).tolist() for L in lens]
    ids = torch.tensor(sum(prompts, []), device=DEV)
    pos = torch.tensor(sum([list(range(L)) for L in lens], []), device=DEV)
    slices, at = [], 0
    for L in lens:
        slices.append((at, at + L))
        at += L
    caches = [PagedKVCache(mc.n_layers, NB, BS, mc.n_kv_heads, mc.head_dim, DEV, model.dtype) for _ in range(n)]
    for cache in caches:
        model.forward(ids, pos, slices, tables, lens, cache)
    return caches, tables, prompts


def test_merged_decode_graphs_equal_the_work_item_graphs_bf16():
    """Captured decode steps on the merged launch (split rows merged inside the
    attention launch, slot map in the staging buffer) against the same steps on
    the work items and their combine launch: identical token ids and identical
    pools, step after step, and no merge errors."""
    from tinybatch_amd.decode_graphs import DecodeGraphs
    if not ops.decode_device(DEV).merge_in_kernel:
        pytest.skip("the device's workgroup placement does not allow in-launch merges")
    mc = small_cfg(layers=2, heads=14, kv_heads=2, vocab=500)
    model = Qwen2Paged(mc, DEV, torch.bfloat16, seed=7)
    P = ops.partition_tokens(torch.bfloat16, mc.head_dim)
    lens = [37, 3 * P + 5, 16, P + 1, 129, 2 * P]
    caches, tables, prompts = _prefilled_caches(model, mc, lens, 2)
    merged = DecodeGraphs(model, caches[0], max_batch=8, max_model_len=4 * P)
    items = DecodeGraphs(model, caches[1], max_batch=8, max_model_len=4 * P)
    items.merged = False                         # before the first capture
    assert merged.merged and merged.slots > 0
    toks, ctx = [p[-1] for p in prompts], list(lens)
    for _ in range(4):
        positions = list(ctx)
        ctx = [c + 1 for c in ctx]
        a = merged.run(toks, positions, tables, ctx)
        b = items.run(toks, positions, tables, ctx)
        assert a == b
        toks = a
    torch.cuda.synchronize()
    assert ops.decode_device(DEV).errors() == 0 and merged.merged
    n = sum(len(t) for t in tables)
    for layer in range(mc.n_layers):
        assert torch.equal(caches[0].pools[layer][:n].view(torch.int16), caches[1].pools[layer][:n].view(torch.int16))


def test_engine_recomputes_captured_steps_after_a_merge_error():
    """A merge error reported by a captured (pipelined) decode step: the engine runs
    that step and the one queued from its ids again, eagerly, the graphs move to the
    work items, and every request ends with the tokens of an undisturbed run."""
    if not ops.decode_device(DEV).merge_in_kernel:
        pytest.skip("the device's workgroup placement does not allow in-launch merges")
    mc = small_cfg(layers=2, heads=14, kv_heads=2, vocab=500)
    P = ops.partition_tokens(torch.bfloat16, mc.head_dim)
    g = torch.Generator().manual_seed(11)
    prompts = [torch.randint(0, mc.vocab_size, (n,), generator=g).tolist() for n in (P + 40, 2 * P + 3, 70, 300)]
    budget = 12

    def run(inject_at):
        ecfg = EngineConfig(dtype="bfloat16", num_blocks=256, block_size=16, max_batch_tokens=4096, max_running=8,
                            max_model_len=4 * P, decode_graphs=True, pipeline_decode=True)
        eng = LLMEngine(ecfg, model=Qwen2Paged(mc, DEV, torch.bfloat16, seed=9))
        reqs = [eng.add_request(p, max_new_tokens=budget) for p in prompts]
        assert eng.graphs.merged
        while eng.has_work():
            if eng.pipelined_steps == inject_at:
                ops.decode_device(DEV).violations.fill_(1)   # as a merge across two XCDs would count
            eng.step()
        return eng, [list(r.output_token_ids) for r in reqs]

    clean, want = run(inject_at=-1)
    assert clean.merge_failures == 0 and clean.pipelined_steps > 4
    dd = ops.decode_device(DEV)
    try:
        hit, got = run(inject_at=3)
        assert hit.merge_failures == 1 and not hit.graphs.merged and not dd.merge_in_kernel
        assert got == want
        assert dd.errors() == 0
    finally:
        dd.merge_in_kernel = True                               # later tests keep in-launch merges
        dd.violations.zero_()


@pytest.mark.parametrize("graphs", [True, False])
def test_swap_preemption_gives_the_tokens_of_an_unpressured_run(graphs):
    """preemption="swap" under block pressure: victims' blocks go to pinned host
    memory (K3 gather) and come back into other block ids (K3 scatter); greedy
    outputs are those of a run with room for everything (block ids never change
    what attention computes). Recompute preemption regenerates the same tokens."""
    mc = small_cfg(layers=2, heads=4, kv_heads=2)
    model = Qwen2Paged(mc, DEV, torch.float32, seed=11)
    g = torch.Generator().manual_seed(12)
    prompts = [torch.randint(0, mc.vocab_size, (n,), generator=g).tolist() for n in (40, 33, 50, 20, 47)]
    max_new = [40, 45, 30, 50, 38]

    def run(num_blocks, preemption):
        ecfg = EngineConfig(dtype="float32", num_blocks=num_blocks, block_size=16, max_batch_tokens=256,
                            max_running=5, decode_graphs=graphs, preemption=preemption)
        eng = LLMEngine(ecfg, model=model)
        reqs = [eng.add_request(p, max_new_tokens=m) for p, m in zip(prompts, max_new)]
        while eng.has_work():
            eng.step()
        return [r.output_token_ids for r in reqs], eng, reqs

    want, eng, _ = run(96, "swap")
    assert eng.swap_outs == 0
    got, eng, reqs = run(16, "swap")
    assert got == want
    assert eng.swap_outs > 0 and eng.swap_ins == eng.swap_outs and not eng.scheduler.swapped
    assert sum(r.preemptions for r in reqs) == eng.swap_outs
    got_rc, eng_rc, reqs_rc = run(16, "recompute")
    assert got_rc == want and sum(r.preemptions for r in reqs_rc) > 0


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_pipelined_decode_streams_match_synchronous_steps(dtype):
    """Decode steps queued ahead of their tokens (pipeline_decode) give every
    request the same token stream, finished flags included, as synchronous
    steps: with budget ends, a request arriving mid-run (the pipeline drains
    for its prefill) and a stop token that ends requests while a later step
    is already queued for them."""
    mc = small_cfg(layers=2, heads=4, kv_heads=2)
    model = Qwen2Paged(mc, DEV, getattr(torch, dtype), seed=21)
    g = torch.Generator().manual_seed(22)
    prompts = [torch.randint(0, mc.vocab_size, (n,), generator=g).tolist() for n in (30, 17, 45, 8)]
    late = torch.randint(0, mc.vocab_size, (25,), generator=g).tolist()
    max_new = [40, 12, 33, 25]

    def run(pipeline, stop=()):
        ecfg = EngineConfig(dtype=dtype, num_blocks=128, block_size=16, max_batch_tokens=256, max_running=8,
                            pipeline_decode=pipeline, stop_token_ids=tuple(stop))
        eng = LLMEngine(ecfg, model=model)
        reqs = [eng.add_request(p, max_new_tokens=m) for p, m in zip(prompts, max_new)]
        streams, calls = {}, 0
        while eng.has_work():
            for o in eng.step():
                streams.setdefault(o.req_id, []).append((o.token_id, o.finished))
            calls += 1
            if calls == 6:
                reqs.append(eng.add_request(late, max_new_tokens=20))
        assert eng._inflight is None and not any(-1 in r.output_token_ids for r in reqs)
        return [r.output_token_ids for r in reqs], [streams[r.req_id] for r in reqs], eng

    want, want_streams, e0 = run(False)
    got, got_streams, e1 = run(True)
    assert e0.pipelined_steps == 0 and e1.pipelined_steps > 20
    assert got == want and got_streams == want_streams
    assert [len(t) for t in want] == max_new + [20]
    assert all(s[-1][1] and not any(f for _, f in s[:-1]) for s in want_streams)
    # a stop token taken from the middle of one request's output
    stop = want[2][len(want[2]) // 2]
    want_s, want_streams_s, _ = run(False, (stop,))
    got_s, got_streams_s, e2 = run(True, (stop,))
    assert got_s == want_s and got_streams_s == want_streams_s and e2.pipelined_steps > 0
    assert any(t[-1] == stop and len(t) < m for t, m in zip(want_s, max_new + [20]))


def test_decode_graphs_refuse_a_step_with_a_shared_slot():
    """The captured step appends inside attention, each row its own K/V; a step
    whose rows share their newest slot is not queued (launch returns None) and
    the engine runs it with the separate append."""
    from tinybatch_amd.decode_graphs import DecodeGraphs

    mc = small_cfg(layers=2, heads=4, kv_heads=2)
    model = Qwen2Paged(mc, DEV, torch.bfloat16, seed=5)
    cache = PagedKVCache(mc.n_layers, 16, 16, mc.n_kv_heads, mc.head_dim, DEV, torch.bfloat16)
    graphs = DecodeGraphs(model, cache, max_batch=4, max_model_len=128)
    ctx = [20, 36]
    assert graphs.launch([1, 2], [19, 35], [[3, 6], [0, 5, 6]], ctx) is None
    assert graphs.run([1, 2], [19, 35], [[3, 6], [0, 5, 6]], ctx) is None
    ids = graphs.run([1, 2], [19, 35], [[3, 6], [0, 5, 7]], ctx)
    assert len(ids) == 2 and all(0 <= t < mc.vocab_size for t in ids)


def test_merge_error_recomputes_the_step_without_in_launch_merges():
    """A nonzero in-launch merge error count (as a unit merged across two XCDs would
    leave) seen at an eager step's token copy: the engine switches merges off for the
    device and recomputes the step through the work items, so the tokens equal a clean
    run's; PagedKVCache.check raises on the same count."""
    from tinybatch_amd import ops

    mc = small_cfg(layers=2, heads=4, kv_heads=2)
    ecfg = EngineConfig(dtype="float32", num_blocks=96, block_size=16, max_batch_tokens=160, max_running=5,
                        decode_graphs=False)
    model = Qwen2Paged(mc, DEV, torch.float32, seed=3)
    g = torch.Generator().manual_seed(9)
    prompts = [torch.randint(0, mc.vocab_size, (n,), generator=g).tolist() for n in (20, 33, 7)]
    clean = LLMEngine(ecfg, model=model).generate(prompts, max_new_tokens=5)
    dd = ops.decode_device(DEV)
    assert dd.merge_in_kernel
    try:
        cache = PagedKVCache(1, 8, 16, 2, 64, DEV, torch.float16)
        dd.violations.fill_(1)
        with pytest.raises(RuntimeError, match="merge errors"):
            cache.check()
        eng = LLMEngine(ecfg, model=model)
        got = eng.generate(prompts, max_new_tokens=5)          # the first step sees the count
        assert eng.merge_failures == 1 and not dd.merge_in_kernel
        assert dd.errors() == 0
        assert got == clean
        cache.check()                                           # nothing left to report
    finally:
        dd.merge_in_kernel = True                               # later tests keep the decode kernel
        dd.violations.zero_()


def test_engine_prefill_steps_take_the_whole_sequence_prefill_kernel():
    """The engine's metadata is built with its query heads, so a prefill-only bf16 step
    routes its whole sequences to tb_paged_prefill (work list, no tiles or items)."""
    mc = small_cfg(layers=2, heads=4, kv_heads=2)
    ecfg = EngineConfig(dtype="bfloat16", num_blocks=96, block_size=16, max_batch_tokens=512, max_running=4,
                        decode_graphs=False)
    eng = LLMEngine(ecfg, model=Qwen2Paged(mc, DEV, torch.bfloat16, seed=3))
    g = torch.Generator().manual_seed(10)
    for n in (40, 64, 100):
        eng.add_request(torch.randint(0, mc.vocab_size, (n,), generator=g).tolist(), max_new_tokens=2)
    eng.step()                                                  # the three prefills
    assert eng.last_step_prefills == 3
    meta = eng.kv_cache._meta_cache[0]["meta"]
    assert meta.num_prefill_work > 0 and meta.num_work_items == 0 and meta.num_prefill_tiles == 0
    while eng.has_work():
        eng.step()
