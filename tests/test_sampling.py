"""Sampling of the next token (reference src/tinybatch/engine.py:145-159):
greedy argmax at temperature 0, otherwise a draw from softmax(logits / T),
restricted with top-p to the tokens whose probability mass *before* them (in
descending order) is below p, renormalised.

Logits are the logs of chosen probabilities, so every expected distribution
is a closed form: p^(1/T) renormalised for a temperature; for top-p, the
nucleus is read off the cumulative sums of the chosen probabilities. Seeded
draws are compared with those distributions within 5 binomial standard
deviations, and tokens outside a nucleus must never be drawn.
"""
import math

import torch

from tinybatch_amd.engine import LLMEngine
from tinybatch_amd.scheduler import Request

P = [0.5, 0.3, 0.15, 0.05]
N = 20000


def draws(temperature: float, top_p: float) -> list[int]:
    logits = torch.tensor([[math.log(p) for p in P]], dtype=torch.float32)
    req = Request(prompt_token_ids=[1], max_new_tokens=1, temperature=temperature, top_p=top_p)
    torch.manual_seed(0)
    counts = [0] * len(P)
    for _ in range(N):
        counts[LLMEngine._sample(None, logits, [req])[0]] += 1
    return counts


def assert_matches(counts, want):
    for c, p in zip(counts, want):
        if p == 0.0:
            assert c == 0
        else:
            sd = math.sqrt(N * p * (1 - p))
            assert abs(c - N * p) <= 5 * sd, (counts, want)


def test_greedy_takes_the_first_maximum():
    logits = torch.tensor([[0.1, 2.0, 2.0, -1.0], [3.0, 3.0, 3.0, 3.0]])
    reqs = [Request(prompt_token_ids=[1], max_new_tokens=1) for _ in range(2)]
    assert LLMEngine._sample(None, logits, reqs) == [1, 0]


def test_temperature_one_draws_the_softmax():
    assert_matches(draws(1.0, 1.0), P)


def test_temperature_half_squares_the_probabilities():
    w = [p ** 2 for p in P]
    assert_matches(draws(0.5, 1.0), [x / sum(w) for x in w])


def test_top_p_keeps_tokens_whose_preceding_mass_is_below_p():
    # mass before each token: 0, 0.5, 0.8, 0.95
    assert_matches(draws(1.0, 0.8), [0.5 / 0.8, 0.3 / 0.8, 0.0, 0.0])          # 0.8 is not below 0.8
    assert_matches(draws(1.0, 0.81), [p / 0.95 for p in P[:3]] + [0.0])
    assert_matches(draws(1.0, 0.3), [1.0, 0.0, 0.0, 0.0])


def test_rows_mix_greedy_and_sampled():
    logits = torch.tensor([[math.log(p) for p in P], [0.0, 5.0, 0.0, 0.0]])
    reqs = [Request(prompt_token_ids=[1], max_new_tokens=1, temperature=1.0, top_p=0.5),
            Request(prompt_token_ids=[1], max_new_tokens=1)]
    torch.manual_seed(1)
    for _ in range(50):
        assert LLMEngine._sample(None, logits, reqs) == [0, 1]
