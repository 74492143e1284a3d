"""The fused layer kernels against the oracle's restatement of the reference
ops (oracle/model_reference.py, CPU): RMSNorm with and without the residual
add, RoPE of q and k from qkv rows, SiLU * up; the weight-streaming
projections against float32 products of the same 16-bit inputs."""
import pytest
import torch
import torch.nn.functional as F

from oracle import model_reference as mref
from tinybatch_amd import layer_ops
from tinybatch_amd.model import rope_tables

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
TOL = {torch.float32: dict(atol=1e-5, rtol=1e-5), torch.bfloat16: dict(atol=2e-2, rtol=2e-2),
       torch.float16: dict(atol=2e-3, rtol=2e-3)}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dim", [896, 4096, 100])
def test_rms_norm_with_and_without_residual(dtype, dim):
    g = torch.Generator().manual_seed(dim)
    x = (torch.randn(37, dim, generator=g) * 3).to(dtype)
    r = torch.randn(37, dim, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(dim, generator=g)).to(dtype)
    got = layer_ops.rms_norm(x.to(DEV), w.to(DEV), 1e-6)
    torch.testing.assert_close(got.cpu().float(), mref.rms_norm(x, w, 1e-6).float(), **TOL[dtype])
    res = r.to(DEV)
    got = layer_ops.rms_norm(x.to(DEV), w.to(DEV), 1e-6, residual=res)
    h = r + x                                                    # the tensor add of the reference layer
    assert torch.equal(res.cpu(), h)                             # same rounding as the tensor add
    torch.testing.assert_close(got.cpu().float(), mref.rms_norm(h, w, 1e-6).float(), **TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (32, 8, 128)])
def test_rope_qk_from_qkv_rows(dtype, hq, hkv, d):
    """fp32 tolerance: the angle pos * inv_freq is rounded to fp32 (and cos/sin
    evaluated) by each platform's own routines, so the GPU table and the CPU
    oracle differ by about pos * 2^-24 rad; small positions pin the kernel's
    arithmetic tightly, large ones within that angle error."""
    g = torch.Generator().manual_seed(hq)
    T = 29
    qkv = torch.randn(T, (hq + 2 * hkv) * d, generator=g).to(dtype)
    cos, sin = rope_tables(d, 1e6, 8192, DEV)
    for hi, atol in ((64, 2e-5), (5000, 2e-3)):
        pos = torch.randint(0, hi, (T,), generator=g)
        q, k = layer_ops.rope_qk(qkv.to(DEV), pos.to(DEV), cos, sin, hq, hkv, d)
        want_q = mref.rope(qkv[:, :hq * d].view(T, hq, d), pos, 1e6)
        want_k = mref.rope(qkv[:, hq * d:(hq + hkv) * d].view(T, hkv, d), pos, 1e6)
        tol = dict(atol=atol, rtol=0) if dtype == torch.float32 else TOL[dtype]
        torch.testing.assert_close(q.cpu().float(), want_q.float(), **tol)
        torch.testing.assert_close(k.cpu().float(), want_k.float(), **tol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_silu_mul(dtype):
    g = torch.Generator().manual_seed(9)
    gu = (torch.randn(13, 2 * 4864, generator=g) * 4).to(dtype)
    got = layer_ops.silu_mul(gu.to(DEV), 4864)
    want = F.silu(gu[:, :4864]) * gu[:, 4864:]                   # the reference's two tensor ops
    torch.testing.assert_close(got.cpu().float(), want.float(), **TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,k", [(1152, 896), (896, 896), (9728, 896), (896, 4864), (48, 64)])
def test_linear_against_fp32_matmul(dtype, n, k):
    """tb_linear against a float32 matmul of the same 16-bit inputs: one rounding
    of an fp32 accumulation (bias included), rows 1 .. 64, strided rows."""
    g = torch.Generator().manual_seed(n + k)
    w = (torch.randn(n, k, generator=g) * 0.05).to(dtype)
    b = (torch.randn(n, generator=g) * 0.05).to(dtype)
    for rows in (1, 7, 16, 33, 64):
        xs = torch.randn(rows, k + 32, generator=g).to(dtype)[:, 16:16 + k]   # strided rows
        want = xs.float() @ w.float().t() + b.float()
        got = layer_ops.linear(xs.to(DEV), w.to(DEV), b.to(DEV))
        torch.testing.assert_close(got.cpu().float(), want, atol=1e-2, rtol=1e-2)
        got = layer_ops.linear(xs.to(DEV), w.to(DEV))
        torch.testing.assert_close(got.cpu().float(), want - b.float(), atol=1e-2, rtol=1e-2)
    with pytest.raises(RuntimeError):   # more than 64 rows: not this kernel's shape
        layer_ops.linear(torch.zeros(65, k, dtype=dtype, device=DEV), w.to(DEV))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,k,splits", [(896, 896, 4), (896, 4864, 8), (48, 64, 2), (64, 96, 3)])
def test_linear_partials_are_the_products_of_their_k_ranges(dtype, n, k, splits):
    """tb_linear_partials: piece s is the fp32 product over k-slices
    [s*S/splits, (s+1)*S/splits) of the 16-bit inputs (S = k/32), so the pieces
    sum to the whole product; rows 1..32, strided rows, both tile shapes."""
    g = torch.Generator().manual_seed(n + k + splits)
    w = (torch.randn(n, k, generator=g) * 0.05).to(dtype)
    S = k // 32
    for rows in (1, 9, 16, 32):
        xs = torch.randn(rows, k + 32, generator=g).to(dtype)[:, 16:16 + k]     # strided rows
        parts = layer_ops.linear_partials(xs.to(DEV), w.to(DEV), splits).cpu()
        assert parts.shape == (splits, rows, n) and parts.dtype == torch.float32
        for s in range(splits):
            lo, hi = 32 * (s * S // splits), 32 * ((s + 1) * S // splits)
            want = xs[:, lo:hi].float() @ w[:, lo:hi].float().t()
            torch.testing.assert_close(parts[s], want, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d_ff,k", [(4864, 896), (48, 64), (64, 1024)])
def test_linear_silu_mul_rounds_like_linear_then_silu_mul(dtype, d_ff, k):
    """gate/up fused with the SwiGLU gate. Integer-valued inputs make every
    product and sum exact in any order, which pins the epilogue bit for bit:
    T(gate) and T(up) rounded once, then tb_silu_mul's arithmetic (and
    tb_linear's one rounding of the same sums). Random inputs stay within the
    dtype's tolerance of silu(gate) * up from one fp32 product. Up to 16 rows:
    8 features per workgroup (gate and up rows in one tile); above: d_ff 4864
    four tiles per workgroup, 48 two; k 1024: two staging passes at 33+ rows."""
    g = torch.Generator().manual_seed(d_ff + k)
    wi = torch.randint(-2, 3, (2 * d_ff, k), generator=g).to(dtype)
    w = (torch.randn(2 * d_ff, k, generator=g) * 0.05).to(dtype)
    wid, wd = wi.to(DEV), w.to(DEV)
    for rows in (1, 7, 16, 33, 64):
        xi = torch.randint(-2, 3, (rows, k), generator=g).to(dtype)
        exact = (xi.float() @ wi.float().t()).to(dtype)             # exact integer sums, one rounding
        got = layer_ops.linear_silu_mul(xi.to(DEV), wid)
        want = layer_ops.silu_mul(exact.to(DEV), d_ff)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), rows
        assert torch.equal(layer_ops.linear(xi.to(DEV), wid).cpu().view(torch.int16), exact.view(torch.int16)), rows
        x = torch.randn(rows, k, generator=g).to(dtype)
        got = layer_ops.linear_silu_mul(x.to(DEV), wd)
        gu = (x.float() @ w.float().t()).to(dtype)                  # F.linear: one rounding
        want = F.silu(gu[:, :d_ff]) * gu[:, d_ff:]
        torch.testing.assert_close(got.cpu().float(), want.float(), **TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dim,splits", [(896, 4), (896, 8), (4096, 1), (136, 2)])
def test_rms_norm_partials(dtype, dim, splits):
    """x = one rounding of the fp32 pieces added in split order; the residual
    sum is bit-exact (the tensor add of the reference layer) and the norm
    within tolerance of the oracle's RMSNorm; 37 rows (not a multiple of the
    four rows per workgroup)."""
    g = torch.Generator().manual_seed(dim + splits)
    rows = 37
    parts = torch.randn(splits, rows, dim, generator=g) * 2
    r = torch.randn(rows, dim, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(dim, generator=g)).to(dtype)
    acc = parts[0].clone()
    for s in range(1, splits):
        acc = acc + parts[s]
    x = acc.to(dtype)
    res = r.to(DEV)
    got = layer_ops.rms_norm_partials(parts.to(DEV), w.to(DEV), 1e-6, residual=res)
    h = r + x
    assert torch.equal(res.cpu(), h)
    torch.testing.assert_close(got.cpu().float(), mref.rms_norm(h, w, 1e-6).float(), **TOL[dtype])
    got = layer_ops.rms_norm_partials(parts.to(DEV), w.to(DEV), 1e-6)
    torch.testing.assert_close(got.cpu().float(), mref.rms_norm(x, w, 1e-6).float(), **TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 5, 16, 32])
def test_linear_argmax_is_the_argmax_of_the_rounded_logits(dtype, rows):
    """The LM head with greedy sampling fused: the index torch.argmax picks from
    tb_linear's rounded logits (the same sums), on a 151936-wide head (two and
    four tiles per workgroup), with ties (the first index wins), a NaN column
    (NaN is the maximum, as in torch.argmax), an all-zero head (index 0)."""
    g = torch.Generator(device=DEV).manual_seed(rows)
    V, K = 151936, 896
    w = (torch.randn(V, K, generator=g, device=DEV) * 0.05).to(dtype)
    x = torch.randn(rows, K, generator=g, device=DEV).to(dtype)
    want = layer_ops.linear(x, w).argmax(dim=-1)
    got = layer_ops.linear_argmax(x, w)
    assert torch.equal(got, want)
    # the pick holds the largest fp32 logit up to the logits' rounding
    ref = x.float() @ w.float().t()
    assert float((ref.max(-1).values - ref.gather(1, got[:, None])[:, 0]).abs().max()) < 0.1
    # ties: a copy of every row's winning column placed earlier wins
    w2 = w.clone()
    w2[3] = w[int(got[0])]
    w2[int(got[0])] = w[int(got[0])]
    got2 = layer_ops.linear_argmax(x[:1], w2)
    assert int(got2[0]) == 3 == int(layer_ops.linear(x[:1], w2).argmax(-1)[0])
    # a NaN column is the maximum of every row
    w2[77777] = float("nan")
    assert torch.equal(layer_ops.linear_argmax(x, w2), torch.full((rows,), 77777, device=DEV))
    assert torch.equal(layer_ops.linear(x, w2).argmax(-1), torch.full((rows,), 77777, device=DEV))
    # all logits zero: the first index
    assert torch.equal(layer_ops.linear_argmax(x, torch.zeros_like(w)), torch.zeros(rows, dtype=torch.int64, device=DEV))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_norm_kernels_agree_bit_for_bit(dtype):
    """tb_rms_norm and tb_rms_norm_partials (one piece holding x) on integer-valued
    rows, whose sums of squares are exact in any order: the same bits, i.e. the
    same mean rounding and the same two single-rounded products per element
    (a contraction of the last product with the rounding to fp16 had made
    rare elements differ by one ulp between the kernels)."""
    g = torch.Generator().manual_seed(11)
    k = 896
    w = (1 + 0.1 * torch.randn(k, generator=g)).to(dtype).to(DEV)
    for rows in (1, 16, 17, 37):
        x = torch.randint(-3, 4, (rows, k), generator=g).to(dtype).to(DEV)
        r = torch.randint(-3, 4, (rows, k), generator=g).to(dtype).to(DEV)
        ra, rb = r.clone(), r.clone()
        a = layer_ops.rms_norm(x, w, 1e-6, residual=ra)
        b = layer_ops.rms_norm_partials(x.float()[None].contiguous(), w, 1e-6, residual=rb)
        assert torch.equal(ra, rb)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), rows
