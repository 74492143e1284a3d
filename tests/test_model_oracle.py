"""Pins of the model restatement (oracle/model_reference.py) on the CPU.

The reference's own correctness oracle is HF transformers' Qwen2 (its
tests/test_correctness.py builds Qwen2ForCausalLM); here the same class is
built from a locally constructed Qwen2Config with random weights (nothing is
fetched), and the restatement must reproduce its logits on full prefills.
RoPE and RMSNorm are also pinned by properties that fix them independently.
"""
import math

import pytest
import torch

from oracle import model_reference as mref
from tinybatch_amd.model import ModelConfig

transformers = pytest.importorskip("transformers")


def _hf_model(layers=2, d=128, heads=2, kv_heads=1, ff=256, vocab=300, seed=0):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    torch.manual_seed(seed)
    hcfg = Qwen2Config(vocab_size=vocab, hidden_size=d, intermediate_size=ff, num_hidden_layers=layers,
                       num_attention_heads=heads, num_key_value_heads=kv_heads, rms_norm_eps=1e-6,
                       rope_theta=1e6, tie_word_embeddings=True, max_position_embeddings=1024)
    m = Qwen2ForCausalLM(hcfg).eval()
    with torch.no_grad():   # HF zero-initialises biases and ones the norms: randomise both
        for name, p in m.named_parameters():
            if name.endswith("bias") or "norm" in name:
                p.add_(torch.randn_like(p) * 0.1)
    w = {k: v.detach().clone() for k, v in m.state_dict().items()}
    w.setdefault("lm_head.weight", w["model.embed_tokens.weight"])
    cfg = ModelConfig(n_layers=layers, n_heads=heads, n_kv_heads=kv_heads, d_model=d, head_dim=d // heads,
                      d_ff=ff, vocab_size=vocab, rms_eps=1e-6, rope_theta=1e6, tie_embeddings=True,
                      max_position=1024)
    return m, w, cfg


def _paged(cfg, lens, bs=16):
    nb = sum(-(-n // bs) for n in lens) + 2
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(5)).tolist()
    tables, at = [], 0
    for n in lens:
        k = -(-n // bs)
        tables.append(perm[at:at + k]); at += k
    pools = [torch.zeros(nb, 2, cfg.n_kv_heads, bs, cfg.head_dim) for _ in range(cfg.n_layers)]
    return tables, pools


def test_restated_forward_matches_hf_qwen2_on_prefills():
    m, w, cfg = _hf_model()
    g = torch.Generator().manual_seed(1)
    lens = [37, 5, 64]
    seqs = [torch.randint(0, cfg.vocab_size, (n,), generator=g) for n in lens]
    tables, pools = _paged(cfg, lens)
    slices, at = [], 0
    for n in lens:
        slices.append((at, at + n)); at += n
    ids = torch.cat(seqs)
    pos = torch.cat([torch.arange(n) for n in lens])
    got = mref.forward(w, cfg, ids, pos, slices, tables, lens, pools, 16)
    with torch.no_grad():
        want = torch.stack([m(s[None]).logits[0, -1] for s in seqs])
    torch.testing.assert_close(got, want.float(), atol=1e-4, rtol=1e-4)


def test_restated_forward_matches_hf_on_decode_after_prefill():
    """Prefill, then one decode step per sequence through the paged pools, equals
    HF on the whole sequence: the cached K/V and the offset mask line up."""
    m, w, cfg = _hf_model(layers=3, heads=4, kv_heads=2, d=128, seed=3)
    g = torch.Generator().manual_seed(2)
    lens = [20, 33]
    seqs = [torch.randint(0, cfg.vocab_size, (n + 1,), generator=g) for n in lens]
    tables, pools = _paged(cfg, [n + 1 for n in lens])
    slices, at = [], 0
    for n in lens:
        slices.append((at, at + n)); at += n
    mref.forward(w, cfg, torch.cat([s[:-1] for s in seqs]), torch.cat([torch.arange(n) for n in lens]),
                 slices, tables, lens, pools, 16)
    got = mref.forward(w, cfg, torch.stack([s[-1] for s in seqs]), torch.tensor(lens),
                       [(0, 1), (1, 2)], tables, [n + 1 for n in lens], pools, 16)
    with torch.no_grad():
        want = torch.stack([m(s[None]).logits[0, -1] for s in seqs])
    torch.testing.assert_close(got, want.float(), atol=1e-4, rtol=1e-4)


def test_rope_depends_on_relative_position_only():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 1, 64, generator=g, dtype=torch.float64).float()
    k = torch.randn(1, 1, 64, generator=g, dtype=torch.float64).float()
    dots = []
    for p in (0, 7, 300):
        qa = mref.rope(q, torch.tensor([p + 11]), 1e4)
        ka = mref.rope(k, torch.tensor([p]), 1e4)
        dots.append(float((qa * ka).sum()))
    assert max(dots) - min(dots) < 1e-3
    assert torch.allclose(mref.rope(q, torch.tensor([0]), 1e4), q)            # position 0 is identity
    assert math.isclose(float(mref.rope(q, torch.tensor([123]), 1e4).norm()), float(q.norm()), rel_tol=1e-5)


def test_rms_norm_unit_rms():
    x = torch.randn(5, 96, generator=torch.Generator().manual_seed(4)) * 7
    y = mref.rms_norm(x, torch.ones(96), 0.0)
    torch.testing.assert_close(y.pow(2).mean(-1), torch.ones(5), atol=1e-5, rtol=0)
