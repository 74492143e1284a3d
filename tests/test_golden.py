"""The committed golden fixture (qwen-fp32-b8 decode step) against the oracle and the workload generator."""
import hashlib
import os

import numpy as np
import torch

from oracle import reference_path as ref
from tinybatch_amd.workloads import make_decode_workload

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "qwen_fp32_b8_decode.npz")


def test_generator_reproduces_fixture_inputs():
    g = np.load(FIXTURE)
    wl = make_decode_workload("qwen-fp32-b8")
    assert int(g["seed"]) == wl.seed
    assert g["cached_lens"].tolist() == wl.cached_lens
    for b, t in enumerate(wl.block_tables):
        assert g["block_tables"][b, :len(t)].tolist() == t
    assert np.array_equal(g["q"], wl.q.numpy()) and np.array_equal(g["k_new"], wl.k_new.numpy())
    assert hashlib.sha256(wl.pool.numpy().tobytes()).hexdigest() == str(g["pool_sha256_before"])


def test_oracle_matches_fixture_and_f64():
    g = np.load(FIXTURE)
    wl = make_decode_workload("qwen-fp32-b8")
    pool = wl.pool.clone()
    out = ref.decode_step(pool, wl.q, wl.k_new, wl.v_new, wl.cached_lens, wl.block_tables, 14, 2, 16)
    assert np.abs(out.numpy() - g["attn_out"]).max() <= 1e-6
    assert np.abs(g["attn_out"] - g["attn_out_f64"]).max() < 1e-5
    assert hashlib.sha256(pool.numpy().tobytes()).hexdigest() == str(g["pool_sha256_after"])
