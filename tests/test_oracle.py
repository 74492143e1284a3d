"""Pins the CPU oracle (oracle/reference_path.py) before anything is compared with it.

Each check uses an independent formulation (flat-index closed forms, a float64
brute force with explicit loops, torch's SDPA with an explicit mask, special
cases whose answer is known) so that a plausible mistake in the restatement
fails at least one of them; the planted-mistake tests prove that.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import brute, reference_path as ref


def _case(seed=0, Hq=4, Hkv=2, D=16, BS=4, NB=40, qlens=(1, 3, 1, 5), cached=(6, 0, 9, 2),
          dtype=torch.float32):
    """A small mixed batch: sequence b has cached[b] old tokens and qlens[b] new ones."""
    g = torch.Generator().manual_seed(seed)
    pool = torch.randn(NB, 2, Hkv, BS, D, generator=g).to(dtype)
    perm = torch.randperm(NB, generator=g).tolist()
    tables, slices, ctx, positions, at, t = [], [], [], [], 0, 0
    for c, n in zip(cached, qlens):
        total = c + n
        nb = (total + BS - 1) // BS
        tables.append(perm[at:at + nb]); at += nb
        slices.append((t, t + n)); t += n
        ctx.append(total)
        positions.extend(range(c, total))
    T = t
    q = torch.randn(T, Hq, D, generator=g).to(dtype)
    k = torch.randn(T, Hkv, D, generator=g).to(dtype)
    v = torch.randn(T, Hkv, D, generator=g).to(dtype)
    return dict(pool=pool, tables=tables, slices=slices, ctx=ctx, positions=torch.tensor(positions),
                q=q, k=k, v=v, Hq=Hq, Hkv=Hkv, D=D, BS=BS, NB=NB)


def test_write_matches_closed_form_and_leaves_other_bytes():
    c = _case()
    before = c["pool"].clone()
    ref.kv_write(c["pool"], c["k"], c["v"], c["positions"], c["slices"], c["tables"], c["BS"])
    want = brute.write_closed_form(before.numpy().reshape(-1), c["k"].numpy(), c["v"].numpy(),
                                   c["positions"].numpy(), c["slices"], c["tables"], c["Hkv"], c["BS"], c["D"])
    got = c["pool"].numpy().reshape(-1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    changed = (got.view(np.uint32) != before.numpy().reshape(-1).view(np.uint32)).sum()
    assert changed == len(c["positions"]) * 2 * c["Hkv"] * c["D"]


def test_gather_matches_closed_form():
    c = _case()
    for table, ctx in zip(c["tables"], c["ctx"]):
        k, v = ref.kv_gather(c["pool"], table, ctx)
        K, V = brute.gather_closed_form(c["pool"].numpy().reshape(-1), table, ctx, c["Hkv"], c["BS"], c["D"])
        assert np.array_equal(k.numpy(), K) and np.array_equal(v.numpy(), V)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_attention_matches_f64_brute_force(seed):
    c = _case(seed=seed)
    ref.kv_write(c["pool"], c["k"], c["v"], c["positions"], c["slices"], c["tables"], c["BS"])
    got = ref.attention(c["q"], c["pool"], c["slices"], c["tables"], c["ctx"], c["Hq"], c["Hkv"])
    want = brute.attention_f64(c["q"].numpy(), c["pool"].numpy().reshape(-1), c["slices"], c["tables"],
                               c["ctx"], c["Hq"], c["Hkv"], c["BS"], c["D"])
    assert np.abs(got.numpy() - want).max() < 1e-5


def test_attention_matches_sdpa_with_explicit_full_mask():
    """Library routine on the whole sequence with a mask built from the rule j <= ctx-q_len+i."""
    c = _case(seed=3, qlens=(4,), cached=(7,), Hq=6, Hkv=3)
    got = ref.attention(c["q"], c["pool"], c["slices"], c["tables"], c["ctx"], c["Hq"], c["Hkv"])
    K, V = brute.gather_closed_form(c["pool"].numpy().reshape(-1), c["tables"][0], c["ctx"][0], 3, c["BS"], c["D"])
    K, V = torch.from_numpy(K), torch.from_numpy(V)
    ctx, n = c["ctx"][0], 4
    i = torch.arange(n)[:, None]
    j = torch.arange(ctx)[None, :]
    mask = j <= (ctx - n + i)
    heads = []
    for h in range(6):
        heads.append(F.scaled_dot_product_attention(c["q"][:, h][None], K[:, h // 2][None], V[:, h // 2][None],
                                                    attn_mask=mask[None])[0])
    want = torch.stack(heads, 1).reshape(n, -1)
    assert torch.allclose(got, want, atol=1e-6, rtol=0)


def test_single_position_context_returns_v0():
    c = _case(qlens=(1,), cached=(0,))
    ref.kv_write(c["pool"], c["k"], c["v"], c["positions"], c["slices"], c["tables"], c["BS"])
    got = ref.attention(c["q"], c["pool"], c["slices"], c["tables"], c["ctx"], c["Hq"], c["Hkv"])
    rep = c["Hq"] // c["Hkv"]
    for h in range(c["Hq"]):
        assert torch.allclose(got[0, h * c["D"]:(h + 1) * c["D"]], c["v"][0, h // rep], atol=1e-7)


def test_identical_keys_give_mean_of_values():
    c = _case(qlens=(1,), cached=(11,))
    pool = c["pool"]
    for b in c["tables"][0]:
        pool[b, 0] = 0.5          # every key equal -> uniform softmax
    got = ref.attention(c["q"], pool, c["slices"], c["tables"], c["ctx"], c["Hq"], c["Hkv"])
    _, V = brute.gather_closed_form(pool.numpy().reshape(-1), c["tables"][0], c["ctx"][0], c["Hkv"], c["BS"], c["D"])
    rep = c["Hq"] // c["Hkv"]
    for h in range(c["Hq"]):
        assert np.allclose(got[0, h * c["D"]:(h + 1) * c["D"]].numpy(), V[:, h // rep].mean(0), atol=1e-6)


def test_full_prefill_branch_equals_offset_mask_rule():
    """q_len == ctx takes the is_causal branch; it must equal the general mask rule."""
    c = _case(qlens=(9,), cached=(0,))
    ref.kv_write(c["pool"], c["k"], c["v"], c["positions"], c["slices"], c["tables"], c["BS"])
    got = ref.attention(c["q"], c["pool"], c["slices"], c["tables"], c["ctx"], c["Hq"], c["Hkv"])
    want = brute.attention_f64(c["q"].numpy(), c["pool"].numpy().reshape(-1), c["slices"], c["tables"],
                               c["ctx"], c["Hq"], c["Hkv"], c["BS"], c["D"])
    assert np.abs(got.numpy() - want).max() < 1e-5


def test_rep_one_is_plain_mha():
    c = _case(Hq=3, Hkv=3, qlens=(2, 1), cached=(5, 3))
    got = ref.attention(c["q"], c["pool"], c["slices"], c["tables"], c["ctx"], 3, 3)
    want = brute.attention_f64(c["q"].numpy(), c["pool"].numpy().reshape(-1), c["slices"], c["tables"],
                               c["ctx"], 3, 3, c["BS"], c["D"])
    assert np.abs(got.numpy() - want).max() < 1e-5


def test_permuting_physical_blocks_does_not_change_output():
    c = _case(seed=5)
    out1 = ref.attention(c["q"], c["pool"], c["slices"], c["tables"], c["ctx"], c["Hq"], c["Hkv"])
    g = torch.Generator().manual_seed(9)
    perm = torch.randperm(c["NB"], generator=g)
    pool2 = torch.empty_like(c["pool"])
    pool2[perm] = c["pool"]                      # block b moves to perm[b]
    tables2 = [[int(perm[b]) for b in t] for t in c["tables"]]
    out2 = ref.attention(c["q"], pool2, c["slices"], tables2, c["ctx"], c["Hq"], c["Hkv"])
    assert torch.equal(out1, out2)


# ---- planted mistakes: each altered oracle must fail the brute-force check ----

def _planted_attention(q, pool, slices, tables, ctxs, Hq, Hkv, mistake):
    T, _, D = q.shape
    out = torch.zeros(T, Hq * D)
    rep = Hq // Hkv
    for (s, e), table, ctx in zip(slices, tables, ctxs):
        keys, vals = ref.kv_gather(pool, table, ctx)
        if mistake == "head_map_mod":
            idx = torch.arange(Hq) % Hkv          # h % Hkv instead of h // rep
        else:
            idx = torch.arange(Hq) // rep
        ki, vi = keys[:, idx].transpose(0, 1), vals[:, idx].transpose(0, 1)
        qi = q[s:e].transpose(0, 1)
        n = e - s
        i = torch.arange(n)[:, None]
        j = torch.arange(ctx)[None, :]
        shift = 1 if mistake == "mask_off_by_one" else 0
        mask = j <= (ctx - n + i - shift)
        mask[:, 0] = True
        scale = 1.0 if mistake == "no_scale" else 1.0 / math.sqrt(D)
        o = F.scaled_dot_product_attention(qi, ki, vi, attn_mask=mask, scale=scale)
        out[s:e] = o.transpose(0, 1).reshape(n, -1)
    return out


@pytest.mark.parametrize("mistake", ["head_map_mod", "mask_off_by_one", "no_scale"])
def test_planted_mistakes_are_caught(mistake):
    c = _case(seed=7, Hq=6, Hkv=2)
    want = brute.attention_f64(c["q"].numpy(), c["pool"].numpy().reshape(-1), c["slices"], c["tables"],
                               c["ctx"], c["Hq"], c["Hkv"], c["BS"], c["D"])
    good = _planted_attention(c["q"], c["pool"], c["slices"], c["tables"], c["ctx"], 6, 2, "none")
    bad = _planted_attention(c["q"], c["pool"], c["slices"], c["tables"], c["ctx"], 6, 2, mistake)
    assert np.abs(good.numpy() - want).max() < 1e-5
    assert np.abs(bad.numpy() - want).max() > 1e-2


def test_copy_closed_form_roundtrip():
    c = _case()
    flat = c["pool"].numpy().reshape(-1)
    be = 2 * c["Hkv"] * c["BS"] * c["D"]
    out = brute.copy_closed_form(flat, [1, 2], [7, 9], be)
    assert np.array_equal(out[7 * be:8 * be], flat[1 * be:2 * be])
    assert np.array_equal(out[:7 * be], flat[:7 * be])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_low_precision_oracle_within_tolerance_of_f64(dtype):
    """The oracle in fp16/bf16 (the reference's own numerics) stays within 2e-2 of exact."""
    c = _case(seed=11, dtype=dtype, qlens=(1, 1, 4), cached=(30, 17, 12), NB=60)
    got = ref.attention(c["q"], c["pool"], c["slices"], c["tables"], c["ctx"], c["Hq"], c["Hkv"])
    want = brute.attention_f64(c["q"].float().numpy(), c["pool"].float().numpy().reshape(-1), c["slices"],
                               c["tables"], c["ctx"], c["Hq"], c["Hkv"], c["BS"], c["D"])
    assert np.allclose(got.float().numpy(), want, atol=2e-2, rtol=2e-2)
