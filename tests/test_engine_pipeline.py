"""Host logic of pipelined decode steps (no GPU): the engine's scheduling,
placeholders, budget ends, stop tokens and drains around a stand-in for the
decode graphs whose "model" is a fixed function of (input token, position).
Pipelined and synchronous engines must give every request the same token
stream, finished flags included, through admissions, preemptions and stops."""
import pytest

from tinybatch_amd.block_manager import BlockManager
from tinybatch_amd.config import EngineConfig
from tinybatch_amd.engine import LLMEngine
from tinybatch_amd.scheduler import Scheduler

V = 97


def rule(token: int, position: int) -> int:
    return (token * 31 + position * 7 + 3) % V


class StandInGraphs:
    """launch/collect/run of DecodeGraphs on the host: row i's input token is the
    previous launch's id of row src[i] where src[i] >= 0."""

    def __init__(self, refuse=()):
        self.prev: list[int] = []
        self.launches = 0
        self.calls = 0
        self.refuse = set(refuse)   # launch calls refused as a step with two rows on one slot

    def bucket(self, B):
        return next((b for b in (1, 2, 4, 8) if b >= B), None)

    def launch(self, tokens, positions, block_tables, context_lens, src_rows=None):
        self.calls += 1
        if self.calls in self.refuse:
            return None
        src = src_rows if src_rows is not None else [-1] * len(tokens)
        inputs = [self.prev[s] if s >= 0 else t for t, s in zip(tokens, src)]
        assert all(t >= 0 for t in inputs), "a placeholder reached the model"
        assert all(p == c - 1 for p, c in zip(positions, context_lens))
        self.prev = [rule(t, p) for t, p in zip(inputs, positions)]
        self.launches += 1
        return list(self.prev)

    def collect(self, handle):
        return list(handle)

    def run(self, tokens, positions, block_tables, context_lens):
        h = self.launch(tokens, positions, block_tables, context_lens)
        return None if h is None else self.collect(h)


def make_engine(pipeline: bool, *, num_blocks=64, stop=(), max_running=4, refuse=()):
    cfg = EngineConfig(num_blocks=num_blocks, block_size=4, max_batch_tokens=48, max_running=max_running,
                       pipeline_decode=pipeline, stop_token_ids=tuple(stop))
    eng = LLMEngine.__new__(LLMEngine)          # no model, cache or device: the steps are stood in for
    eng.cfg = cfg
    eng.block_manager = BlockManager(cfg.num_blocks, cfg.block_size, cfg.enable_prefix_caching)
    eng.scheduler = Scheduler(cfg, eng.block_manager)
    eng.eos_ids = set(cfg.stop_token_ids)
    eng.steps = eng.last_step_prefills = eng.graph_steps = eng.pipelined_steps = 0
    eng.swap_outs = eng.swap_ins = 0
    eng._swap_reads = []
    eng._inflight = None
    eng.graphs = StandInGraphs(refuse)
    eng.eager_steps = 0

    def forward_eager(ordered, ids, pos, slices, tables, ctx):
        # LLMEngine._forward_eager with the model replaced by the rule
        eng.eager_steps += 1
        return [rule(ids[e - 1], pos[e - 1]) for s, e in slices]

    eng._forward_eager = forward_eager
    return eng


def run(eng, prompts, max_new, late=None):
    reqs = [eng.add_request(p, max_new_tokens=m) for p, m in zip(prompts, max_new)]
    streams, calls = {}, 0
    while eng.has_work():
        for o in eng.step():
            streams.setdefault(o.req_id, []).append((o.token_id, o.finished))
        calls += 1
        if late and calls == late[0]:
            reqs.append(eng.add_request(late[1], max_new_tokens=late[2]))
    assert eng._inflight is None
    eng.requests = reqs
    return [r.output_token_ids for r in reqs], [streams[r.req_id] for r in reqs]


PROMPTS = [[5, 6, 7, 8, 9], [11, 12], [13, 14, 15, 16, 17, 18, 19, 20, 21], [22, 23, 24]]
MAX_NEW = [17, 6, 23, 12]


@pytest.mark.parametrize("late", [None, (4, [40, 41, 42, 43, 44, 45], 9)])
def test_pipelined_streams_equal_synchronous_ones(late):
    want = run(make_engine(False), PROMPTS, MAX_NEW, late)
    eng = make_engine(True)
    got = run(eng, PROMPTS, MAX_NEW, late)
    assert got == want
    assert eng.pipelined_steps > 10
    for stream in want[1]:
        assert stream[-1][1] and not any(f for _, f in stream[:-1])   # finished exactly once, last


def test_stop_tokens_end_requests_with_a_step_already_queued():
    tokens, _ = run(make_engine(False), PROMPTS, MAX_NEW)
    stop = tokens[2][9]                            # mid-stream for the longest request
    want = run(make_engine(False, stop=[stop]), PROMPTS, MAX_NEW)
    eng = make_engine(True, stop=[stop])
    got = run(eng, PROMPTS, MAX_NEW)
    assert got == want and eng.pipelined_steps > 0
    assert any(t and t[-1] == stop and len(t) < m for t, m in zip(want[0], MAX_NEW))
    # every block is back: the stopped requests' queued step wrote into blocks they gave up
    assert eng.block_manager.num_free() == make_engine(False).block_manager.num_free()


def test_block_pressure_drains_to_synchronous_steps():
    # 10 blocks of 4 tokens for requests growing to 8..32 tokens: decode steps meet
    # the free-block condition only part of the time, and recompute preemptions happen
    want = run(make_engine(False, num_blocks=10), PROMPTS, MAX_NEW)
    eng = make_engine(True, num_blocks=10)
    got = run(eng, PROMPTS, MAX_NEW)
    assert got == want
    assert 0 < eng.pipelined_steps < eng.steps
    assert sum(r.preemptions for r in eng.requests) > 0


@pytest.mark.parametrize("back", [1, 2, 3])
def test_stop_token_at_the_end_of_a_budget(back):
    """A stop token among a request's last budgeted tokens: with back = 2 the
    request's budget ends with the step queued after the stop's step (finished at
    that launch), so collecting the stop must not finish it a second time."""
    tokens, _ = run(make_engine(False), PROMPTS, MAX_NEW)
    for r in range(len(PROMPTS)):
        stop = tokens[r][MAX_NEW[r] - back]
        want = run(make_engine(False, stop=[stop]), PROMPTS, MAX_NEW)
        eng = make_engine(True, stop=[stop])
        got = run(eng, PROMPTS, MAX_NEW)
        assert got == want, f"request {r}, stop {stop}"
        assert eng.block_manager.num_free() == make_engine(False).block_manager.num_free()


@pytest.mark.parametrize("pipeline", [False, True])
def test_steps_the_graphs_refuse_run_eagerly(pipeline):
    """A decode step whose rows share a pool slot is refused by the graphs (their
    fused append cannot give the reference's last-writer-wins result): the engine
    then runs the step's rows eagerly, draining a queued step first, with the
    same token streams."""
    want = run(make_engine(False), PROMPTS, MAX_NEW)
    eng = make_engine(pipeline, refuse=(3, 7, 8, 15))
    got = run(eng, PROMPTS, MAX_NEW)
    assert got == want
    assert eng.graphs.calls > 15 and eng.eager_steps >= 4 + 1   # the refused steps and the first prefill
