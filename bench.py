"""Benchmark of the paged KV-cache decode step on one MI355X.

One step = one decode iteration of a 24-layer model's attention data path:
for every layer pool, append one new K/V row per sequence and run paged decode
attention over the whole context (the fused K1+K2 launch the engine uses for
decode-only steps). Workload "qwen-fp16-b64": Qwen2.5-0.5B layer geometry
(14/2 heads, head_dim 64, block 16), fp16, 64 sequences with U{512..4096}
cached tokens, 32768-block pool per layer. Inputs are resident in HBM before
the timed region; the 24 distinct layer pools (6 GiB) keep the working set far
above the 256 MB Infinity Cache. The step is captured once in a HIP graph and
replayed; HIP events on the capturing stream bracket the timed replays.

value = algorithmic bytes of all layers / wall time of the step (GB/s).
Algorithmic bytes per layer: append (read k,v; write the pool rows; 4-byte
slots) + attention (every visible K and V row once, q and out once, the
block-table entries used, the context lengths); no credit for cache hits.

Prints ONE JSON line (rank 0, N = 1 only).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "paged decode attn+append HBM GB/s (% of peak) at 1 GPU; e2e decode tok/s"


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(wl, reps: int, budget_s: float) -> dict:
    """The oracle (op-for-op restatement of the reference CPU path) on the same
    workload, one layer step per rep, on the host's cores."""
    import torch

    from oracle import reference_path as ref

    threads = len(os.sched_getaffinity(0))
    threads = min(threads, 16)        # the GPU box grants 16 cores per GPU
    torch.set_num_threads(threads)
    times = []
    t_start = time.perf_counter()
    for _ in range(reps):
        pool = wl.pool  # the append rewrites the same rows each rep (idempotent)
        t0 = time.perf_counter()
        ref.decode_step(pool, wl.q, wl.k_new, wl.v_new, wl.cached_lens, wl.block_tables,
                        wl.num_heads, wl.num_kv_heads, wl.block_size)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s:
            break
    times.sort()
    med = times[len(times) // 2]
    gbs = wl.algorithmic_bytes()["total"] / med / 1e9
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{len(times)} one-layer decode steps of {wl.name} (B={wl.batch}), median "
                      f"{med * 1e3:.1f} ms, torch CPU ({cpu_model()})"}


def cpu_baseline_mixed(wl, reps: int, budget_s: float) -> dict:
    """The oracle on the mixed step, on the host's cores: the prefill rows' attention
    alone (the line's value, TFLOP/s) and the whole layer step (append of all 4152
    new rows, then attention of every row: 8 causal prefills and 56 decodes)."""
    import torch

    from oracle import reference_path as ref

    threads = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(threads)
    pre = wl.part("prefill")
    pos = torch.tensor(wl.positions, dtype=torch.int64)

    def timed(fn):
        times, t_start = [], time.perf_counter()
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
            if time.perf_counter() - t_start > budget_s / 2:
                break
        times.sort()
        return times[len(times) // 2], len(times)

    t_pre, n_pre = timed(lambda: ref.attention(pre.q, pre.pool, pre.seq_slices, pre.block_tables,
                                               pre.context_lens, pre.num_heads, pre.num_kv_heads))

    def whole():
        ref.kv_write(wl.pool, wl.k_new, wl.v_new, pos, wl.seq_slices, wl.block_tables, wl.block_size)
        ref.attention(wl.q, wl.pool, wl.seq_slices, wl.block_tables, wl.context_lens, wl.num_heads,
                      wl.num_kv_heads)

    t_all, n_all = timed(whole)
    b = wl.algorithmic_bytes()
    return {"value": round(pre.flops() / t_pre / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "step_ms": round(t_all * 1e3, 2),
            "step_algorithmic_GBps": round((b["append"] + b["attention"]) / t_all / 1e9, 4),
            "sample": f"prefill attention of the 8 x 512 rows: {n_pre} reps, median {t_pre * 1e3:.1f} ms; "
                      f"whole layer step (append + attention of {wl.num_tokens} rows): {n_all} reps, median "
                      f"{t_all * 1e3:.1f} ms; torch CPU ({cpu_model()})"}


def cpu_baseline_e2e(weights: dict, mc, wl, reps: int, budget_s: float) -> dict:
    """The oracle's Qwen2 forward (the reference's Qwen2Paged.forward restated op for op,
    per-sequence gather + SDPA included) on the host cores: decode steps of the serving
    workload's 32 requests at their first output position (context = prompt + 1), with
    the model's own weights and dtype. Reports output tokens per second of those steps
    (one token per request per step)."""
    import torch

    from oracle import model_reference as mref

    threads = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(threads)
    BS = 16
    ctx = [len(p) + 1 for p in wl.prompts]
    B = len(ctx)
    tables, at = [], 0
    for c in ctx:                                  # private blocks per request (no sharing on this path)
        n = (c + BS - 1) // BS
        tables.append(list(range(at, at + n)))
        at += n
    dt = next(iter(weights.values())).dtype
    pools = [torch.zeros(at, 2, mc.n_kv_heads, BS, mc.head_dim, dtype=dt) for _ in range(mc.n_layers)]
    ids = torch.tensor([p[-1] for p in wl.prompts])
    pos = torch.tensor([c - 1 for c in ctx])
    slices = [(i, i + 1) for i in range(B)]

    def step():
        mref.forward(weights, mc, ids, pos, slices, tables, ctx, pools, BS)

    step()                                         # warm-up (allocator, kernels)
    times, t_start = [], time.perf_counter()
    for _ in range(max(reps, 1)):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s:
            break
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(B / med, 2), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{len(times)} decode steps of the {B} requests (contexts {min(ctx)}..{max(ctx)}, "
                      f"{mc.n_layers} layers, {str(dt).replace('torch.', '')} weights), median {med * 1e3:.1f} ms "
                      f"per step; torch CPU ({cpu_model()})"}


def kernel_source_hash() -> str:
    """sha256 (first 16 hex digits) of the code of the HIP sources and the C header,
    comments and white space left out: the kernels a profile was measured on (an edit
    of a comment does not void a profile, any edit of code does)."""
    import hashlib
    import re

    def code(path):
        with open(path) as f:
            text = re.sub(r"//[^\n]*|/\*.*?\*/", " ", f.read(), flags=re.S)
        return " ".join(text.split()).encode()

    h = hashlib.sha256()
    csrc = os.path.join(ROOT, "tinybatch_amd", "csrc")
    for name in sorted(os.listdir(csrc)):
        if name.endswith((".hip", ".h", ".cpp")):
            h.update(name.encode() + b"\0" + code(os.path.join(csrc, name)))
    h.update(code(os.path.join(ROOT, "include", "tinybatch_amd.h")))
    return h.hexdigest()[:16]


def load_traffic(workload: str, mode: str):
    """HBM bytes per call measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, calibrated
    against a plain device copy) in the committed profile summary, or None when there is
    none or it was measured on other kernel sources than these (its kernel_source_sha)."""
    path = os.path.join(ROOT, "profiles", f"paged_decode_{workload}_{mode}.md")
    if not os.path.exists(path):
        return None
    traffic = sha = None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_call:"):
                traffic = int(line.split(":", 1)[1])
            elif line.startswith("kernel_source_sha:"):
                sha = line.split(":", 1)[1].strip()
    if sha != kernel_source_hash():
        _log(f"profile {os.path.basename(path)} was measured on other kernel sources; traffic not reported")
        return None
    return traffic


def time_step(step, dev, args) -> tuple[float, bool]:
    """ms per call of ``step``: one eager warm-up, capture into a HIP graph (unless
    --no-graph), W untimed and K timed replays bracketed by events on the stream
    the work runs on."""
    import torch

    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        step()                                   # eager warm-up (also exercises every launch)
    torch.cuda.synchronize()
    graph = None
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            step()
        torch.cuda.synchronize()

    def run_once():
        # replays and eager launches both go to `stream`, the stream the events are recorded on
        with torch.cuda.stream(stream):
            if graph is not None:
                graph.replay()
            else:
                step()

    for _ in range(args.warmup):
        run_once()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        ev0.record(stream)
    for _ in range(args.steps):
        run_once()
    with torch.cuda.stream(stream):
        ev1.record(stream)
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / args.steps, graph is not None


MFMA_PEAK_TFLOPS_16 = 2500.0


def bench_mixed(args, dev) -> int:
    """The mixed step (run_mixed) as its own JSON line."""
    print(json.dumps(run_mixed(args, dev, with_cpu=not args.no_cpu)), flush=True)
    return 0


def run_mixed(args, dev, with_cpu: bool = True) -> dict:
    """Mixed engine step (8 x 512-token prefills + 56 decodes, shared prefix) and a
    1024-block compaction round, on rotating layer pools. Times the whole layer
    step (append + attention), the prefill rows alone (MFMA-bound: reported in
    TFLOP/s against the dense 16-bit MFMA peak), the decode rows alone (GB/s)
    and the block copy over every layer pool in one launch (GB/s)."""
    import torch

    from tinybatch_amd import ops
    from tinybatch_amd.metadata import build_step_metadata
    from tinybatch_amd.workloads import make_mixed_workload

    t0 = time.perf_counter()
    wl = make_mixed_workload()
    _log(f"workload {wl.name}: T={wl.num_tokens} seqs={wl.batch} ({time.perf_counter() - t0:.1f}s)")
    L = args.layers or 24
    storage = torch.empty((L,) + tuple(wl.pool.shape), dtype=wl.dtype, device=dev)
    src = wl.pool.to(dev)
    for l in range(L):
        storage[l].copy_(src)
    del src
    pools = [storage[l] for l in range(L)]
    P = args.partition or ops.partition_tokens(wl.dtype, wl.head_dim)
    rows = ops.rows_per_item(wl.dtype, wl.num_heads, wl.num_kv_heads)
    Hq = wl.num_heads
    results = {}
    dec_kernel = "paged_attn_mfma_kernel (work items)"
    step_kernels = "paged_step_mfma_kernel (prefill tiles and decode items in one launch)"
    for which, w in (("step", wl), ("prefill", wl.part("prefill")), ("decode", wl.part("decode"))):
        # whole prefill sequences go to tb_paged_prefill in a prefill-only step; a
        # step with decode rows keeps the one launch of tiles and decode items
        route = None if (which != "prefill" or args.no_tiles or args.no_stream_prefill) else ops.prefill_route(
            wl.dtype, wl.num_heads, wl.num_kv_heads, wl.head_dim, dev)
        meta = build_step_metadata(w.positions, w.seq_slices, w.block_tables, w.context_lens,
                                   block_size=w.block_size, num_blocks=w.num_blocks, partition_tokens=P,
                                   rows_per_item=rows, tile_prefill=not args.no_tiles, prefill_route=route)
        split = which == "step" and not args.no_split_step and ops.attach_split_parts(
            meta, w.positions, w.seq_slices, w.block_tables, w.context_lens, num_heads=Hq,
            num_kv_heads=wl.num_kv_heads, head_dim=wl.head_dim, dtype=wl.dtype, device=dev, rows=rows)
        if split:
            step_kernels = ("paged_prefill_stream_kernel + paged_stream_kernel (split step, each appending "
                            "its own rows)")
        if which == "decode" and not args.no_decode_stream and ops.decode_kernel_preferred(
                meta, num_kv_heads=wl.num_kv_heads, head_dim=wl.head_dim, dtype=wl.dtype):
            if ops.attach_decode_plan(meta, num_heads=Hq, num_kv_heads=wl.num_kv_heads, head_dim=wl.head_dim,
                                      dtype=wl.dtype, device=dev,
                                      unit_cost=args.unit_cost if args.unit_cost >= 0 else None):
                dec_kernel = "paged_stream_kernel"
        meta = meta.to(dev)
        q, k, v = w.q.to(dev), w.k_new.to(dev), w.v_new.to(dev)
        out = torch.empty(w.num_tokens, Hq * w.head_dim, dtype=w.dtype, device=dev)
        ws = ops.workspace_for(meta, Hq, w.head_dim, dev)
        append = which == "step"
        # a split step appends inside its two kernels (each side its own rows); the one
        # launch of tiles and items needs the append kernel first
        fuse = append and split

        def step(meta=meta, q=q, k=k, v=v, out=out, ws=ws, append=append, fuse=fuse):
            for pool in pools:
                if append and not fuse:
                    ops.kv_append(pool, k, v, meta.slot_mapping)
                ops.paged_attention(q, pool, meta, num_heads=Hq, out=out, workspace=ws,
                                    k_new=k if fuse else None, v_new=v if fuse else None)

        ms, graph = time_step(step, dev, args)
        results[which] = (ms / L, w)
        _log(f"{which}: {ms / L * 1e3:.2f} us per layer")
    # the append kernel alone: the step's 4152 new K/V rows into every layer pool
    meta = build_step_metadata(wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens,
                               block_size=wl.block_size, num_blocks=wl.num_blocks, partition_tokens=P).to(dev)
    k_all, v_all = wl.k_new.to(dev), wl.v_new.to(dev)

    def append_only():
        for pool in pools:
            ops.kv_append(pool, k_all, v_all, meta.slot_mapping)

    ms_append, _ = time_step(append_only, dev, args)
    _log(f"append: {ms_append / L * 1e3:.2f} us per layer")
    plan = ops.BlockCopyPlan(pools, wl.copy_src, wl.copy_dst)
    ms_copy, _ = time_step(plan.launch, dev, args)
    _log(f"copy: {ms_copy * 1e3:.2f} us for {L} layer pools")
    cpu = None
    if with_cpu:
        _log("timing the CPU baseline (oracle) ...")
        cpu = cpu_baseline_mixed(wl, args.cpu_reps, args.cpu_budget)

    step_ms, _ = results["step"]
    b = wl.algorithmic_bytes()
    step_gbs = (b["append"] + b["attention"]) / (step_ms * 1e-3) / 1e9
    pre_ms, pre = results["prefill"]
    pre_tflops = pre.flops() / (pre_ms * 1e-3) / 1e12
    dec_ms, dec = results["decode"]
    dec_gbs = dec.algorithmic_bytes()["attention"] / (dec_ms * 1e-3) / 1e9
    copy_gbs = b["copy"] * L / (ms_copy * 1e-3) / 1e9
    append_gbs = b["append"] / (ms_append / L * 1e-3) / 1e9
    line = {
        "metric": "mixed step: prefill attention TFLOP/s (MFMA), decode attention and block copy GB/s",
        "value": round(pre_tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(step_ms * L, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) pool, q, k, v; seeded random block tables, one shared prefix)",
        "config": {"workload": f"{wl.name}: 8 x 512-token prefills + 56 decodes (24 share a 32-block "
                               f"prefix) per layer, {L} layer pools; 1024-block copy over all pools",
                   "tokens": wl.num_tokens, "layers": L, "partition_tokens": P, "rows_per_item": rows,
                   "prefill_tiles": not args.no_tiles, "graph": graph, "step_kernels": step_kernels},
        "step_us_per_layer": round(step_ms * 1e3, 3),
        "step_algorithmic_GBps": round(step_gbs, 2),
        "prefill_us_per_layer": round(pre_ms * 1e3, 3),
        "decode_us_per_layer": round(dec_ms * 1e3, 3),
        "decode_kv_bytes_logical": dec.algorithmic_bytes()["attention"],
        "decode_kv_bytes_unique": dec.unique_kv_bytes(),
        "copy_us_all_layers": round(ms_copy * 1e3, 3),
        "roofline": {"bound": "mfma", "achieved": round(pre_tflops, 2), "peak": MFMA_PEAK_TFLOPS_16,
                     "unit": "TFLOP/s", "frac": round(pre_tflops / MFMA_PEAK_TFLOPS_16, 4), "traffic": None,
                     "kernel": ("paged_attn_mfma_kernel + combine_partials_kernel" if args.no_tiles
                                else "paged_prefill_mfma_kernel" if args.no_stream_prefill
                                else "paged_prefill_stream_kernel") + " (prefill rows)"},
        "decode_roofline": {"bound": "hbm", "achieved": round(dec_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(dec_gbs / HBM_PEAK_GBS, 4), "kernel": dec_kernel},
        "copy_roofline": {"bound": "hbm", "achieved": round(copy_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(copy_gbs / HBM_PEAK_GBS, 4), "kernel": "block_copy_kernel"},
        "append_us_per_layer": round(ms_append / L * 1e3, 3),
        "append_roofline": {"bound": "hbm", "achieved": round(append_gbs, 2), "peak": HBM_PEAK_GBS,
                            "unit": "GB/s", "frac": round(append_gbs / HBM_PEAK_GBS, 4),
                            "bytes_per_layer": b["append"], "kernel": "kv_append_kernel"},
        "cpu_baseline": cpu,
    }
    del storage, pools
    torch.cuda.empty_cache()
    return line


def run_e2e(dev, warmup: int, cpu: dict | None = None) -> dict:
    """Continuous batching of 32 random-token requests on a random-init Qwen2 at
    0.5B dimensions (bf16), 75% sharing a 400-token prefix, greedy outputs of
    U{16..256} tokens, everything submitted at t = 0. Returns output tokens per
    second of wall time, decode-only-step token rate, TTFT mean / p99 (first
    token time - submit time, the reference's engine.py:131-132) and the run's
    configuration. With ``cpu`` ({"reps", "budget"}) also the oracle's decode-step
    rate on the host cores (cpu_baseline_e2e) under "cpu_baseline"."""
    import statistics

    import torch

    from tinybatch_amd.config import EngineConfig
    from tinybatch_amd.engine import LLMEngine
    from tinybatch_amd.model import ModelConfig, Qwen2Paged
    from tinybatch_amd.workloads import make_serving_workload

    mc = ModelConfig.qwen2_0_5b()
    ecfg = EngineConfig(num_blocks=4096, block_size=16, max_batch_tokens=2048, max_running=32, seed=0)
    t0 = time.perf_counter()
    model = Qwen2Paged(mc, dev, torch.bfloat16, seed=0)
    torch.cuda.synchronize()
    _log(f"model {mc.num_params()} params ({time.perf_counter() - t0:.1f}s)")
    wl = make_serving_workload()

    def run(prompts, outs):
        eng = LLMEngine(ecfg, model=model)
        if eng.graphs is not None:
            eng.graphs.capture_all()               # before the clock starts
        torch.cuda.synchronize()
        start = time.perf_counter()
        reqs = [eng.add_request(p, max_new_tokens=m) for p, m in zip(prompts, outs)]
        for r in reqs:
            r.arrival_time = start
        dec_time = dec_tokens = 0.0
        while eng.has_work():
            ts = time.perf_counter()
            outs_ = eng.step()
            dt = time.perf_counter() - ts
            if outs_ and eng.last_step_prefills == 0:   # decode-only step
                dec_time += dt
                dec_tokens += len(outs_)
        wall = time.perf_counter() - start
        return eng, reqs, wall, dec_tokens, dec_time

    for _ in range(max(warmup, 1)):                # untimed: kernels, GEMM heuristics, allocator
        run(wl.prompts[:4], [8] * 4)
    eng, reqs, wall, dec_tokens, dec_time = run(wl.prompts, wl.max_new_tokens)
    out_tokens = sum(len(r.output_token_ids) for r in reqs)
    ttft = sorted(r.first_token_time - r.arrival_time for r in reqs)
    res = {
        "tok_s": round(out_tokens / wall, 1), "output_tokens": out_tokens, "wall_s": round(wall, 4),
        "steps": eng.steps, "graph_steps": eng.graph_steps, "pipelined_steps": eng.pipelined_steps,
        "decode_only_tok_s": round(dec_tokens / dec_time, 1) if dec_time else None,
        "ttft_mean_ms": round(statistics.mean(ttft) * 1e3, 2),
        "ttft_p99_ms": round(ttft[int(0.99 * (len(ttft) - 1))] * 1e3, 2),
        "prefix_hit_rate": round(eng.block_manager.hit_rate(), 3),
        "preemptions": sum(r.preemptions for r in reqs),
        "workload": f"{wl.name}: 32 requests, prompts U{{32..512}} (sharing ones U{{401..512}}), "
                    f"outputs U{{16..256}}, greedy",
        "config": {"params": mc.num_params(), "layers": mc.n_layers, "num_blocks": ecfg.num_blocks,
                   "max_batch_tokens": ecfg.max_batch_tokens, "max_running": ecfg.max_running,
                   "rope_theta": mc.rope_theta, "rms_eps": mc.rms_eps},
    }
    res["cpu_baseline"] = None
    if cpu is not None:
        _log("timing the e2e CPU baseline (oracle forward) ...")
        w = {k: v.detach().cpu() for k, v in model.reference_weights().items()}
        res["cpu_baseline"] = cpu_baseline_e2e(w, mc, wl, cpu["reps"], cpu["budget"])
        del w
    del eng, model
    torch.cuda.empty_cache()
    return res


def bench_e2e(args, dev) -> int:
    """The end-to-end serving workload alone (run_e2e) as its own JSON line."""
    r = run_e2e(dev, args.warmup, None if args.no_cpu else {"reps": args.cpu_reps, "budget": args.cpu_budget})
    line = {
        "metric": "e2e decode tok/s (continuous batching, random-init Qwen2 0.5B dims)",
        "value": r["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": r["steps"], "warmup": args.warmup,
        "ms_per_step": round(r["wall_s"] / max(r["steps"], 1) * 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random token ids; seeded random-init weights; 24/32 requests share a 400-token prefix)",
        "config": dict(workload=r["workload"], **r["config"]),
        **{k: r[k] for k in ("output_tokens", "wall_s", "decode_only_tok_s", "ttft_mean_ms", "ttft_p99_ms",
                              "prefix_hit_rate", "preemptions", "graph_steps", "pipelined_steps")},
        "cpu_baseline": r["cpu_baseline"],
    }
    print(json.dumps(line), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="qwen-fp16-b64")
    ap.add_argument("--layers", type=int, default=0, help="layer pools to rotate (0 = auto)")
    ap.add_argument("--batch", type=int, default=0, help="decode workloads: the first N sequences only")
    ap.add_argument("--mode", choices=["fused", "split"], default="fused")
    ap.add_argument("--kernel", choices=["auto", "decode", "items"], default="auto",
                    help="decode: streaming decode kernel (tb_paged_decode); items: work-item kernel; "
                         "auto: the decode kernel for steps of >= ops.DECODE_KERNEL_MIN_BYTES of K/V")
    ap.add_argument("--decode-waves", type=int, default=0,
                    help="decode kernel: waves per workgroup (a compiled variant; 0 = the library's default)")
    ap.add_argument("--unit-cost", type=int, default=-1,
                    help="decode kernel: tile-equivalents a unit adds to its worker's share (-1 = default)")
    ap.add_argument("--combine", action="store_true",
                    help="work-item kernel: merge split rows with the separate combine kernel, not inside the launch")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-decode-stream", action="store_true",
                    help="mixed workload: the decode rows through work items even where the streaming "
                         "decode kernel is preferred")
    ap.add_argument("--no-split-step", action="store_true",
                    help="mixed workload: the whole step as one launch of prefill tiles and decode items, not "
                         "tb_paged_prefill + the streaming decode kernel on their own rows")
    ap.add_argument("--no-stream-prefill", action="store_true",
                    help="mixed workload: prefill sequences through the tile kernel, not tb_paged_prefill")
    ap.add_argument("--cpu-reps", type=int, default=5)
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline (profiling runs)")
    ap.add_argument("--no-e2e", action="store_true",
                    help="headline: skip the end-to-end serving run whose tok/s and TTFT join the line")
    ap.add_argument("--no-extra", action="store_true",
                    help="headline: skip the Llama-geometry and mixed-step sub-objects of the line")
    ap.add_argument("--partition", type=int, default=0)
    ap.add_argument("--no-tiles", action="store_true", help="mixed step: prefill rows as row groups, not tiles")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB five times (HBM counter calibration)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}, "
              f"WORLD_SIZE={world}", file=sys.stderr)
        return 2

    import torch

    from tinybatch_amd import _lib

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    _lib.lib()

    if args.calibrate_copy:
        n = args.calibrate_copy << 20
        a_buf = torch.ones(n // 4, dtype=torch.float32, device=dev)
        b_buf = torch.empty_like(a_buf)
        for _ in range(5):
            b_buf.copy_(a_buf)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "device copy", "bytes_read_per_launch": n,
                          "bytes_written_per_launch": n, "launches": 5}), flush=True)
        return 0

    if args.workload == "qwen-bf16-mixed":
        return bench_mixed(args, dev)
    if args.workload == "qwen2-0.5b-e2e":
        return bench_e2e(args, dev)

    line = run_decode(args, dev, args.workload, batch=args.batch, with_cpu=not args.no_cpu)
    if args.workload == "qwen-fp16-b64" and not args.batch and not args.no_extra:
        # the other configurations in the same invocation, each with its own roofline
        # and CPU baseline: the Llama-geometry decode at sigma 0.5 and 1.0, the mixed step
        sub = argparse.Namespace(**vars(args))
        sub.layers, sub.partition, sub.decode_waves, sub.unit_cost, sub.kernel = 0, 0, 0, -1, "auto"
        for key, name in (("llama", "llama-bf16-b256"), ("llama_sigma1", "llama-bf16-b256-s1")):
            _log(f"{name} ...")
            line[key] = run_decode(sub, dev, name, with_cpu=not args.no_cpu)
        _log("mixed step ...")
        sub.no_tiles = sub.no_stream_prefill = sub.no_split_step = sub.no_decode_stream = False
        line["mixed"] = run_mixed(sub, dev, with_cpu=not args.no_cpu)
    if not args.no_e2e and args.workload == "qwen-fp16-b64" and not args.batch:
        # the metric's second half: the serving workload through the engine, same invocation
        _log("end-to-end serving run ...")
        e2e = run_e2e(dev, 1, None if args.no_cpu else {"reps": 3, "budget": 10.0})
        _log(f"e2e: {e2e['tok_s']} tok/s, TTFT mean {e2e['ttft_mean_ms']} ms, p99 {e2e['ttft_p99_ms']} ms")
        line["e2e_tok_s"] = e2e["tok_s"]
        line["ttft_mean_ms"] = e2e["ttft_mean_ms"]
        line["ttft_p99_ms"] = e2e["ttft_p99_ms"]
        line["e2e"] = e2e
    print(json.dumps(line), flush=True)
    return 0


def host_step_cost(wl, dev, reps: int = 5) -> dict:
    """Host work of one decode step's metadata, median over ``reps``: the step arrays from
    the host lists (build_step_metadata), the decode plan's tile assignment
    (tb_build_decode_segments), and the upload with the device-side plan expansion
    (meta.to, synchronised); for comparison the plan built entry by entry on the host
    (tb_build_decode_plan) and uploaded whole."""
    import torch

    from tinybatch_amd import ops
    from tinybatch_amd.metadata import build_step_metadata

    P = ops.partition_tokens(wl.dtype, wl.head_dim)
    kw = dict(num_heads=wl.num_heads, num_kv_heads=wl.num_kv_heads, head_dim=wl.head_dim, dtype=wl.dtype,
              device=dev)
    res = {k: [] for k in ("metadata", "plan", "upload", "plan_host", "upload_host")}
    for _ in range(reps + 1):
        t0 = time.perf_counter()
        meta = build_step_metadata(wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens,
                                   block_size=wl.block_size, num_blocks=wl.num_blocks, partition_tokens=P)
        t1 = time.perf_counter()
        ops.attach_decode_plan(meta, **kw)
        t2 = time.perf_counter()
        meta.to(dev)
        torch.cuda.synchronize()
        t3 = time.perf_counter()
        meta2 = build_step_metadata(wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens,
                                    block_size=wl.block_size, num_blocks=wl.num_blocks, partition_tokens=P)
        t4 = time.perf_counter()
        ops.attach_decode_plan(meta2, on_device=False, **kw)
        t5 = time.perf_counter()
        meta2.to(dev)
        torch.cuda.synchronize()
        t6 = time.perf_counter()
        for k, v in (("metadata", t1 - t0), ("plan", t2 - t1), ("upload", t3 - t2), ("plan_host", t5 - t4),
                     ("upload_host", t6 - t5)):
            res[k].append(v * 1e3)
    med = {k: round(sorted(v[1:])[len(v[1:]) // 2], 3) for k, v in res.items()}   # first rep: warm-up
    return {"metadata_ms": med["metadata"], "plan_ms": med["plan"], "upload_and_device_plan_ms": med["upload"],
            "host_built_plan_ms": med["plan_host"], "host_built_plan_upload_ms": med["upload_host"],
            "plan_bytes_host_built": int(meta2.decode_plan.numel() * 4) if meta2.decode_plan is not None else 0,
            "reps": reps}


def run_decode(args, dev, name: str, *, batch: int = 0, with_cpu: bool = True) -> dict:
    """One decode workload: append + paged attention per layer pool, captured in a graph
    and timed (time_step); returns the bench line's fields for it (metric, value in
    algorithmic GB/s, roofline per call, CPU baseline, the host cost of a step's
    metadata and plan)."""
    import torch

    from tinybatch_amd import ops
    from tinybatch_amd.metadata import build_step_metadata
    from tinybatch_amd.workloads import make_decode_workload

    big = name.startswith("llama")
    t0 = time.perf_counter()
    wl = make_decode_workload(name, pool_device=(dev if big else "cpu"), **({"batch": batch} if batch else {}))
    _log(f"workload {wl.name}: B={wl.batch} NB={wl.num_blocks} mean ctx={sum(wl.context_lens)/wl.batch:.0f} "
         f"({time.perf_counter() - t0:.1f}s)")
    pool_bytes = wl.pool.numel() * wl.pool.element_size()
    # 24 layer pools (a Qwen2.5-0.5B model's worth) unless one pool alone dwarfs the Infinity Cache
    L = args.layers or (24 if pool_bytes * 24 <= (64 << 30) else 2)
    storage = torch.empty((L,) + tuple(wl.pool.shape), dtype=wl.dtype, device=dev)
    src = wl.pool if wl.pool.is_cuda else wl.pool.to(dev)
    for l in range(L):
        storage[l].copy_(src)
    del src
    if wl.pool.is_cuda:
        wl.pool = None                                         # the draw lives on in the layer pools
    pools = [storage[l] for l in range(L)]
    P = args.partition or ops.partition_tokens(wl.dtype, wl.head_dim)
    meta = build_step_metadata(wl.positions, wl.seq_slices, wl.block_tables, wl.context_lens,
                               block_size=wl.block_size, num_blocks=wl.num_blocks, partition_tokens=P)
    want_decode = args.kernel == "decode" or (args.kernel == "auto" and ops.decode_kernel_preferred(
        meta, num_kv_heads=wl.num_kv_heads, head_dim=wl.head_dim, dtype=wl.dtype))
    decode_kernel = want_decode and ops.attach_decode_plan(
        meta, num_heads=wl.num_heads, num_kv_heads=wl.num_kv_heads, head_dim=wl.head_dim, dtype=wl.dtype, device=dev,
        waves=args.decode_waves or None, unit_cost=args.unit_cost if args.unit_cost >= 0 else None)
    # work items: split rows merged inside the launch where the device allows it
    merged = (not decode_kernel and not args.combine and ops.attach_xcd_slot_map(
        meta, num_heads=wl.num_heads, num_kv_heads=wl.num_kv_heads, dtype=wl.dtype, device=dev))
    meta.to(dev)
    q = wl.q.to(dev)
    k = wl.k_new.to(dev)
    v = wl.v_new.to(dev)
    out = torch.empty(wl.batch, wl.num_heads * wl.head_dim, dtype=wl.dtype, device=dev)
    ws = ops.workspace_for(meta, wl.num_heads, wl.head_dim, dev)
    fused = args.mode == "fused"

    def step():
        for pool in pools:
            if fused:
                ops.paged_attention(q, pool, meta, num_heads=wl.num_heads, out=out, k_new=k, v_new=v, workspace=ws)
            else:
                ops.kv_append(pool, k, v, meta.slot_mapping)
                ops.paged_attention(q, pool, meta, num_heads=wl.num_heads, out=out, workspace=ws)

    ms, graph = time_step(step, dev, args)
    _log(f"{L} layers x {args.steps} steps: {ms:.4f} ms/step")

    bytes_layer = wl.algorithmic_bytes()
    total_bytes = bytes_layer["total"] * L
    gbs = total_bytes / (ms * 1e-3) / 1e9
    # one tb_paged_attention call per layer (attention kernel + its combine kernel; plus the
    # append kernel in split mode): the time per call is the step time over the layers
    per_launch_ms = ms / L
    achieved = bytes_layer["total"] / (per_launch_ms * 1e-3) / 1e9
    traffic = load_traffic(wl.name, args.mode)
    if decode_kernel or merged:
        viol = int(ops.decode_device(dev).violations.item())
        if viol:
            raise RuntimeError(f"{viol} in-launch merge errors: the workgroup placement assumption failed")
    host = None
    if decode_kernel:
        _log("host cost of a step's metadata and plan ...")
        host = host_step_cost(wl, dev)
        # the model's attention time per step: Qwen2.5-0.5B has 24 layers, Llama-3-8B 32
        model_layers = 32 if big else 24
        attn_ms = per_launch_ms * model_layers
        host["model_layers"] = model_layers
        host["attention_ms_per_step"] = round(attn_ms, 4)
        host["plan_frac_of_attention"] = round((host["plan_ms"] + host["upload_and_device_plan_ms"]) / attn_ms, 4)
        host["host_built_plan_frac_of_attention"] = round(
            (host["host_built_plan_ms"] + host["host_built_plan_upload_ms"]) / attn_ms, 4)
    del storage, pools
    torch.cuda.empty_cache()

    cpu = None
    if with_cpu:
        _log("timing the CPU baseline (oracle) ...")
        if big:
            wl_cpu = make_decode_workload(name, pool_device="cpu", batch=16)
        else:
            wl_cpu = wl
        cpu = cpu_baseline(wl_cpu, args.cpu_reps, args.cpu_budget)
        if big:
            cpu["sample"] += " (first 16 sequences of the workload)"

    if decode_kernel:
        kernel = "paged_stream_kernel"
    else:
        attn = "paged_attn_valu_kernel" if wl.dtype == torch.float32 else "paged_attn_mfma_kernel"
        kernel = attn if merged else attn + " + combine_partials_kernel"
    kernel += "" if fused else " + kv_append_kernel"
    return {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}[wl.dtype],
        "data": "synthetic (seeded N(0,1) pool, q, k, v; seeded random block tables)",
        "config": {
            "workload": f"{wl.name}: decode step, append 1 token/seq + paged attention, {L} layer pools",
            "batch": wl.batch, "num_heads": wl.num_heads, "num_kv_heads": wl.num_kv_heads,
            "head_dim": wl.head_dim, "block_size": wl.block_size, "num_blocks": wl.num_blocks,
            "mean_context": round(sum(wl.context_lens) / wl.batch, 1), "max_context": max(wl.context_lens),
            "layers": L, "mode": args.mode, "graph": graph,
            "kernel": (f"decode ({meta.decode_waves} waves per workgroup, unit cost {meta.decode_unit_cost})"
                       if decode_kernel else
                       ("items, split rows merged in the launch" if merged else "items")),
            "partition_tokens": P,
            "bytes_per_layer_step": bytes_layer["total"],
        },
        "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": kernel,
            "avg_launch_us": round(per_launch_ms * 1e3, 3),
        },
        "host_step": host,
        "cpu_baseline": cpu,
    }


if __name__ == "__main__":
    sys.exit(main())
