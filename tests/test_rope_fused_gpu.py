"""RoPE folded into the paged kernels (tb_kv_append_rope, tb_paged_attention's
rope tables): the fused paths give exactly the bits of rotating first with
tb_rope_qk (the reference's _rope arithmetic, model.py:72-80) and then
appending / attending, on every kernel (decode rows, row groups, prefill
tiles, fp32, fused decode append at both address paths); the rotated rows
stay within the oracle's tolerance of its own RoPE."""
import pytest
import torch

from oracle import model_reference as mref
from oracle import reference_path as ref
from tinybatch_amd import layer_ops, ops
from tinybatch_amd.metadata import build_step_metadata
from tinybatch_amd.model import ModelConfig, Qwen2Paged, rope_tables
from tinybatch_amd.kv_cache import PagedKVCache

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
TOL = {torch.float32: dict(atol=1e-5, rtol=0.0), torch.float16: dict(atol=2e-2, rtol=2e-2),
       torch.bfloat16: dict(atol=2e-2, rtol=2e-2)}
THETA = 1e6


def _bits(t):
    return t.contiguous().view(torch.int32 if t.element_size() == 4 else torch.int16)


def _tables(d, max_pos=8192):
    cos, sin = rope_tables(d, THETA, max_pos, DEV)
    return cos, sin, ops.Rope(cos, sin)


def _rotated(x, pos, cos, sin):
    """x [T, H, D] rotated with tb_rope_qk (x as the q heads of qkv rows)."""
    T, H, D = x.shape
    qkv = torch.cat([x.reshape(T, H * D), torch.zeros(T, 2 * D, dtype=x.dtype, device=x.device)], dim=1)
    q, _ = layer_ops.rope_qk(qkv.contiguous(), pos, cos, sin, H, 1, D)
    return q


def _case(seed, Hq, Hkv, D, BS, dtype, qlens, cached):
    g = torch.Generator().manual_seed(seed)
    need = [(c + n + BS - 1) // BS for c, n in zip(cached, qlens)]
    NB = sum(need) + 3
    pool = torch.randn(NB, 2, Hkv, BS, D, generator=g).to(dtype)
    perm = torch.randperm(NB, generator=g).tolist()
    tables, slices, ctx, pos, at, t = [], [], [], [], 0, 0
    for c, n, nb in zip(cached, qlens, need):
        tables.append(perm[at:at + nb]); at += nb
        slices.append((t, t + n)); t += n
        ctx.append(c + n)
        pos.extend(range(c, c + n))
    q = torch.randn(t, Hq, D, generator=g).to(dtype)
    k = torch.randn(t, Hkv, D, generator=g).to(dtype)
    v = torch.randn(t, Hkv, D, generator=g).to(dtype)
    return dict(pool=pool, tables=tables, slices=slices, ctx=ctx, pos=pos, q=q, k=k, v=v, NB=NB, BS=BS)


def _meta(c, rows=1, tiles=False):
    return build_step_metadata(c["pos"], c["slices"], c["tables"], c["ctx"], block_size=c["BS"], num_blocks=c["NB"],
                               partition_tokens=256, rows_per_item=rows, tile_prefill=tiles).to(DEV)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Hkv,D", [(2, 64), (8, 128)])
def test_append_rope_bits_of_rotate_then_append(dtype, Hkv, D):
    c = _case(1, Hkv, Hkv, D, 16, dtype, qlens=[5, 1, 17, 1], cached=[0, 4000, 3, 15])
    cos, sin, rope = _tables(D)
    pos = torch.tensor(c["pos"], device=DEV)
    meta = _meta(c)
    k, v = c["k"].to(DEV), c["v"].to(DEV)
    pool_a, pool_b = c["pool"].to(DEV), c["pool"].to(DEV)
    k_rot = _rotated(k, pos, cos, sin)
    ops.kv_append(pool_a, k_rot, v, meta.slot_mapping)
    ops.kv_append(pool_b, k, v, meta.slot_mapping, rope=rope, positions=pos)
    torch.cuda.synchronize()
    assert torch.equal(_bits(pool_a.cpu()), _bits(pool_b.cpu()))
    # the rotated rows against the oracle's RoPE (fp32: the tables' angle rounding, about pos * 2^-24)
    want = mref.rope(c["k"], torch.tensor(c["pos"]), THETA)
    tol = dict(atol=2e-3, rtol=0) if dtype == torch.float32 else TOL[dtype]
    torch.testing.assert_close(k_rot.cpu().float(), want.float(), **tol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Hq,Hkv,D", [(14, 2, 64), (32, 8, 128)])
def test_attention_rope_bits_of_rotate_then_attend(dtype, Hq, Hkv, D):
    c = _case(2, Hq, Hkv, D, 16, dtype, qlens=[1, 7, 1, 40, 1], cached=[600, 0, 15, 300, 3000])
    cos, sin, rope = _tables(D)
    q, pool = c["q"].to(DEV), c["pool"].to(DEV)
    q_rot = _rotated(q, torch.tensor(c["pos"], device=DEV), cos, sin)
    widest = ops.rows_per_item(dtype, Hq, Hkv)
    shapes = [(1, False), (widest, False)] + ([(widest, True)] if dtype != torch.float32 else [])
    for rows, tiles in shapes:
        meta = _meta(c, rows, tiles)
        a = ops.paged_attention(q_rot, pool, meta, num_heads=Hq)
        b = ops.paged_attention(q, pool, meta, num_heads=Hq, rope=rope)
        torch.cuda.synchronize()
        assert torch.equal(_bits(a.cpu()), _bits(b.cpu())), f"rows {rows} tiles {tiles}"
    # and the rotated query attends like the oracle's
    want = ref.attention(q_rot.cpu(), c["pool"], c["slices"], c["tables"], c["ctx"], Hq, Hkv)
    torch.testing.assert_close(b.cpu().float(), want.float(), **TOL[dtype])


@pytest.mark.parametrize("BS", [4, 16])
@pytest.mark.parametrize("dtype,Hq,Hkv,D", [(torch.float32, 14, 2, 64), (torch.float16, 14, 2, 64),
                                            (torch.bfloat16, 16, 4, 128)])
def test_fused_decode_rope_bits(BS, dtype, Hq, Hkv, D):
    cached = [0, 1, 15, 255, 256, 700, 2047]
    c = _case(3 + BS, Hq, Hkv, D, BS, dtype, qlens=[1] * len(cached), cached=cached)
    cos, sin, rope = _tables(D)
    pos = torch.tensor(c["pos"], device=DEV)
    q, k, v = c["q"].to(DEV), c["k"].to(DEV), c["v"].to(DEV)
    meta = _meta(c)
    pool_a, pool_b = c["pool"].to(DEV), c["pool"].to(DEV)
    a = ops.paged_attention(_rotated(q, pos, cos, sin), pool_a, meta, num_heads=Hq,
                            k_new=_rotated(k, pos, cos, sin), v_new=v)
    b = ops.paged_attention(q, pool_b, meta, num_heads=Hq, k_new=k, v_new=v, rope=rope)
    torch.cuda.synchronize()
    assert torch.equal(_bits(a.cpu()), _bits(b.cpu()))
    assert torch.equal(_bits(pool_a.cpu()), _bits(pool_b.cpu()))


def test_model_forward_same_logits_and_pools_with_fused_rope():
    mc = ModelConfig(n_layers=2, n_heads=4, n_kv_heads=2, d_model=256, head_dim=64, d_ff=256, vocab_size=300,
                     rms_eps=1e-6, rope_theta=THETA, tie_embeddings=True, max_position=2048)
    model = Qwen2Paged(mc, DEV, torch.bfloat16, seed=3)
    g = torch.Generator().manual_seed(4)
    tables = [[5, 9, 2, 8], [11, 3, 6]]
    lens = [50, 20]
    toks = torch.randint(0, mc.vocab_size, (sum(lens),), generator=g).to(DEV)
    pos = torch.cat([torch.arange(n) for n in lens]).to(DEV)
    slices = [(0, 50), (50, 70)]
    out = []
    for fused in (False, True):
        cache = PagedKVCache(mc.n_layers, 16, 16, mc.n_kv_heads, mc.head_dim, DEV, torch.bfloat16)
        model.fused_rope = fused
        logits = model.forward(toks, pos, slices, tables, lens, cache)
        torch.cuda.synchronize()
        out.append((logits.cpu(), [p.cpu() for p in cache.pools]))
    assert torch.equal(out[0][0], out[1][0])
    assert all(torch.equal(_bits(x), _bits(y)) for x, y in zip(out[0][1], out[1][1]))
