"""bench.py's contract on the CPU: one GPU only (--gpus N > 1 exits with a message),
no CPU fallback for the measured path, and the end-to-end CPU baseline (the oracle's
model forward over the serving workload's decode step) on a small model."""
import os
import subprocess
import sys
from types import SimpleNamespace

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def _run(*args):
    env = dict(os.environ, WORLD_SIZE="1")
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          env=env, timeout=300)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _run("--gpus", "2")
    assert r.returncode == 2 and r.stdout == ""
    assert "one GPU" in r.stderr


def test_no_gpu_no_measurement():
    if torch.cuda.is_available():
        return
    r = _run("--steps", "1", "--warmup", "0")
    assert r.returncode == 2 and r.stdout == ""
    assert "needs a GPU" in r.stderr


def test_e2e_cpu_baseline_times_the_oracle_forward():
    import bench

    mc = SimpleNamespace(n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16, d_model=64, d_ff=128, vocab_size=50,
                         rms_eps=1e-6, rope_theta=1e4)
    g = torch.Generator().manual_seed(0)
    r = lambda *s: torch.randn(*s, generator=g) * 0.1
    w = {"model.embed_tokens.weight": r(50, 64), "model.norm.weight": torch.ones(64), "lm_head.weight": r(50, 64)}
    for i in range(2):
        p = f"model.layers.{i}."
        w[p + "input_layernorm.weight"] = torch.ones(64)
        w[p + "post_attention_layernorm.weight"] = torch.ones(64)
        for n, o in (("q", 64), ("k", 32), ("v", 32)):
            w[p + f"self_attn.{n}_proj.weight"] = r(o, 64)
            w[p + f"self_attn.{n}_proj.bias"] = r(o)
        w[p + "self_attn.o_proj.weight"] = r(64, 64)
        w[p + "mlp.gate_proj.weight"] = r(128, 64)
        w[p + "mlp.up_proj.weight"] = r(128, 64)
        w[p + "mlp.down_proj.weight"] = r(64, 128)
    wl = SimpleNamespace(prompts=[[1, 2, 3] * 10, [4] * 17, [5, 6] * 40])   # contexts 31, 18, 81
    out = bench.cpu_baseline_e2e(w, mc, wl, reps=2, budget_s=5.0)
    assert out["unit"] == "tok/s" and out["kind"] == "port" and out["value"] > 0
    assert out["cores"] >= 1 and "3 requests" in out["sample"] and "contexts 18..81" in out["sample"]
