"""Continuous-batching scheduler (the reference's tests/test_scheduler.py
scenarios, restated) and the decode-slot reservation at context_len - 1."""
from tinybatch_amd.block_manager import BlockManager
from tinybatch_amd.config import EngineConfig
from tinybatch_amd.scheduler import Request, Scheduler, Status


def sched(max_batch_tokens=64, num_blocks=16, block_size=4, max_running=8, prefix=False, preemption="recompute"):
    cfg = EngineConfig(max_batch_tokens=max_batch_tokens, num_blocks=num_blocks, block_size=block_size,
                       max_running=max_running, enable_prefix_caching=prefix, preemption=preemption)
    return Scheduler(cfg, BlockManager(num_blocks, block_size, prefix))


def req(n, max_new=32, base=0):
    return Request(prompt_token_ids=list(range(base, base + n)), max_new_tokens=max_new)


def run_step(s):
    """What the engine does after a forward: every scheduled sequence gets one token."""
    b = s.schedule()
    for r in b.prefill + b.decode:
        r.output_token_ids.append(0)
    return b


def test_token_budget_limits_admission():
    s = sched(max_batch_tokens=20)
    for _ in range(3):
        s.add(req(12))
    assert len(run_step(s).prefill) == 1
    b = run_step(s)
    assert len(b.decode) == 1 and len(b.prefill) == 1


def test_new_request_joins_while_others_decode():
    s = sched()
    a = req(8)
    s.add(a)
    run_step(s)
    b = req(8)
    s.add(b)
    batch = run_step(s)
    assert a in batch.decode and b in batch.prefill


def test_finish_returns_blocks():
    s = sched()
    a = req(8)
    s.add(a)
    run_step(s)
    free = s.bm.num_free()
    s.finish(a)
    assert s.bm.num_free() > free and a.status is Status.FINISHED


def test_youngest_is_preempted_under_memory_pressure():
    s = sched(num_blocks=4, block_size=4)
    a, b = req(8, max_new=64), req(7, max_new=64)
    s.add(a)
    s.add(b)
    run_step(s)
    assert len(s.running) == 2
    for _ in range(12):
        run_step(s)
        if b.status is Status.WAITING:
            break
    assert b.status is Status.WAITING and b.preemptions >= 1 and b.output_token_ids == []
    assert a.status is Status.RUNNING
    assert s.waiting[0] is b                                 # back at the head of the queue


def test_swap_preemption_keeps_tokens_and_resumes_first():
    """preemption="swap": the victim keeps its tokens, its written blocks are listed
    for a swap-out in the step that preempts it, nothing new is admitted while it
    waits, and it resumes in fresh blocks listed for a swap-in."""
    s = sched(num_blocks=4, block_size=4, preemption="swap")
    a, b = req(8, max_new=64), req(7, max_new=64, base=100)
    s.add(a)
    s.add(b)
    run_step(s)
    swap_out = None
    for _ in range(12):
        batch = run_step(s)
        if b.status is Status.SWAPPED:
            swap_out = batch.swap_out
            break
    assert b.status is Status.SWAPPED and b.preemptions == 1 and b.block_table == []
    kept = list(b.output_token_ids)
    assert len(kept) >= 1                                    # the sampled tokens survive the preemption
    written = b.context_len() - 1                            # positions 0 .. context_len - 2 hold K/V
    assert [r for r, _ in swap_out] == [b] and len(swap_out[0][1]) == -(-written // 4) == b.swap_blocks
    assert a in batch.decode and b not in batch.decode
    s.add(req(3, base=200))
    batch = run_step(s)                                      # still short of blocks: b waits, so does the new one
    assert not batch.prefill and b.status is Status.SWAPPED
    s.finish(a)
    batch = run_step(s)
    assert [r for r, _ in batch.swap_in] == [b] and b in batch.decode   # b first; the new one may follow
    blocks = batch.swap_in[0][1]
    assert len(blocks) == b.swap_blocks and b.block_table[:len(blocks)] == blocks
    assert b.output_token_ids[:len(kept)] == kept and b.status is Status.RUNNING
    # room for the position the step writes (run_step has appended its sampled token since)
    assert len(b.block_table) * 4 >= b.context_len() - 1
    used = set(b.block_table) | {x for r in batch.prefill for x in r.block_table}
    assert len(s.bm.free_ids) + len(s.bm.evictable) + len(used) == 4


def test_decode_slot_covers_the_written_position():
    """A prompt of exactly one block: its first decode writes position 4, which
    must have a block (the reference reserves one position late here)."""
    bs = 4
    s = sched(block_size=bs)
    a = req(4)
    s.add(a)
    run_step(s)                                              # prefill; first output token sampled
    for _ in range(9):
        b = s.schedule()
        assert a in b.decode
        pos = a.context_len() - 1                           # the position this step writes
        assert pos // bs < len(a.block_table)
        assert len(a.block_table) == pos // bs + 1           # and no block beyond it
        a.output_token_ids.append(0)


def test_fully_cached_prompt_recomputes_its_last_token():
    s = sched(prefix=True)
    p = list(range(8))
    a = Request(prompt_token_ids=p, max_new_tokens=4)
    s.add(a)
    run_step(s)
    b = Request(prompt_token_ids=p, max_new_tokens=4)
    s.add(b)
    run_step(s)
    assert b.num_cached_tokens == 7 and b.block_table[:2] == a.block_table[:2]
