"""GPU parity of the decoder's fused kernels (cq_rms_norm, cq_add_rms_norm,
cq_qkv_norm_rope, cq_silu_mul, and the one-row projections cq_gemv,
cq_gemv_rms_norm, cq_gemv_silu) against torch fp32
statements of the same math, rounded once to the tensor dtype, plus closed
forms: a constant row normalises to the weight, position 0 is the identity
rotation, a rotation keeps each pair's norm, out-of-range positions give NaN.

Bar: within one ulp of the dtype everywhere (fp32: 2^-18 relative), and
for 16-bit dtypes at least 99% of elements bit-identical (the kernels and torch differ only in fp32
summation order and the rsqrt/exp rounding, which moves a 16-bit result
across a rounding boundary rarely).
"""
import math

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

ULP = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 2.0 ** -18}
TINY = {torch.bfloat16: 1e-38, torch.float16: 2.0 ** -24, torch.float32: 1e-38}  # subnormal step


def _assert_ulp(got, ref, what="", mag=None):
    """mag: the magnitude the rounding error scales with, when it is not the
    result's own (a rotation x1 c - x2 s cancels; its error scales with the
    pair's norm)."""
    assert got.dtype == ref.dtype and got.shape == ref.shape, what
    g, r = got.float(), ref.float()
    tol = ULP[ref.dtype] * (r.abs() if mag is None else torch.maximum(r.abs(), mag)) \
        + TINY[ref.dtype]
    bad = ((g - r).abs() > tol) & ~(torch.isnan(g) & torch.isnan(r))
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond one ulp, e.g. " \
                          f"{g[bad][:4].tolist()} vs {r[bad][:4].tolist()}"
    if ref.dtype != torch.float32:
        same = (got.view(torch.int16) == ref.view(torch.int16)).float().mean().item()
        assert same >= 0.99, f"{what}: only {same:.4f} bit-identical"


def _rms_ref(h, w, eps):
    hf = h.float()
    return (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + eps) * w.float()).to(h.dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,dim", [(1, 4096), (7, 5120), (300, 128), (3, 100), (2, 8192),
                                      (2, 8200), (5, 2048), (4, 6000)])
def test_rms_norm(dtype, rows, dim):
    from chronoquant_mlx_amd.models import fused
    g = torch.Generator(device="cuda").manual_seed(rows * 7 + dim)
    x = (torch.randn(rows, dim, device="cuda", generator=g) * 3).to(dtype)
    w = (1 + 0.1 * torch.randn(dim, device="cuda", generator=g)).to(dtype)
    _assert_ulp(fused.rms_norm(x, w, 1e-6), _rms_ref(x, w, 1e-6), f"{rows}x{dim} {dtype}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rms_norm_constant_row_gives_weight(dtype):
    # x = c everywhere: mean(x^2) = c^2, so y = w * c / sqrt(c^2 + eps) = w (eps -> 0)
    from chronoquant_mlx_amd.models import fused
    w = torch.linspace(-2, 2, 4096, device="cuda").to(dtype)
    x = torch.full((3, 4096), 0.75, device="cuda").to(dtype)
    x[1] = -1.5
    y = fused.rms_norm(x, w, 0.0)
    assert torch.equal(y[0], w) and torch.equal(y[2], w) and torch.equal(y[1], -w)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,dim", [(1, 4096), (33, 4096), (2, 100)])
def test_add_rms_norm(dtype, rows, dim):
    from chronoquant_mlx_amd.models import fused
    g = torch.Generator(device="cuda").manual_seed(dim + rows)
    x = torch.randn(rows, dim, device="cuda", generator=g).to(dtype)
    r = (torch.randn(rows, dim, device="cuda", generator=g) * 4).to(dtype)
    w = (1 + 0.1 * torch.randn(dim, device="cuda", generator=g)).to(dtype)
    h, y = fused.add_rms_norm(x, r, w, 1e-6)
    assert torch.equal(h, x + r)  # torch adds in fp32 and rounds once, as the kernel does
    _assert_ulp(y, _rms_ref(x + r, w, 1e-6), f"add {rows}x{dim}")


def _rope_tables(max_pos, theta=1e6, D=128):
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    ang = torch.arange(max_pos, dtype=torch.float64)[:, None] * inv[None, :]
    return torch.cos(ang).float().cuda(), torch.sin(ang).float().cuda()


def _qkv_ref(qkv, nq, nkv, qw, kw, cos, sin, positions, eps):
    B, L, _ = qkv.shape
    D = 128
    heads = qkv.view(B, L, nq + 2 * nkv, D)

    def norm_rope(x, w):  # x [B, L, H, D]
        if w is not None:
            x = _rms_ref(x, w, eps)
        x = x.transpose(1, 2).float()
        c, s = cos[positions], sin[positions]
        c, s = (c[None, None], s[None, None]) if c.dim() == 2 else (c[:, None], s[:, None])
        x1, x2 = x[..., :64], x[..., 64:]
        return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], -1).to(qkv.dtype)

    q = norm_rope(heads[:, :, :nq], qw)
    k = norm_rope(heads[:, :, nq:nq + nkv], kw)
    v = heads[:, :, nq + nkv:].transpose(1, 2).contiguous()
    return q, k, v


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("B,L,nq,nkv,pos2d", [(1, 1, 32, 8, False), (1, 300, 32, 8, False),
                                              (3, 5, 8, 2, True), (2, 1, 40, 8, True)])
def test_qkv_norm_rope(dtype, B, L, nq, nkv, pos2d):
    from chronoquant_mlx_amd.models import fused
    g = torch.Generator(device="cuda").manual_seed(B * 100 + L)
    cos, sin = _rope_tables(4096)
    qkv = torch.randn(B, L, (nq + 2 * nkv) * 128, device="cuda", generator=g).to(dtype)
    qw = (1 + 0.1 * torch.randn(128, device="cuda", generator=g)).to(dtype)
    kw = (1 + 0.1 * torch.randn(128, device="cuda", generator=g)).to(dtype)
    if pos2d:
        positions = torch.stack([torch.arange(L) + 37 * b + 900 for b in range(B)]).cuda()
    else:
        positions = torch.arange(L, device="cuda") + 1000
    q, k, v = fused.qkv_norm_rope(qkv, nq, nkv, qw, kw, cos, sin, positions, 1e-6)
    rq, rk, rv = _qkv_ref(qkv, nq, nkv, qw, kw, cos, sin, positions, 1e-6)
    assert q.shape == (B, nq, L, 128) and k.shape == v.shape == (B, nkv, L, 128)
    assert torch.equal(v, rv)

    def pair_norm(t):
        t = t.float()
        n = (t[..., :64] ** 2 + t[..., 64:] ** 2).sqrt()
        return torch.cat([n, n], -1)
    _assert_ulp(q, rq, "q", mag=pair_norm(rq))
    _assert_ulp(k, rk, "k", mag=pair_norm(rk))


def test_qkv_rope_closed_forms():
    from chronoquant_mlx_amd.models import fused
    cos, sin = _rope_tables(64)
    g = torch.Generator(device="cuda").manual_seed(5)
    qkv = torch.randn(1, 3, 6 * 128, device="cuda", generator=g)
    positions = torch.tensor([0, 17, 64], device="cuda")  # 64 is past the tables
    q, k, v = fused.qkv_norm_rope(qkv, 4, 1, None, None, cos, sin, positions, 1e-6)
    x = qkv.view(1, 3, 6, 128)
    # position 0: cos 1, sin 0, the identity
    assert torch.equal(q[0, :, 0], x[0, 0, :4])
    # a rotation keeps each (j, j + 64) pair's norm
    pair = lambda t: t[..., :64] ** 2 + t[..., 64:] ** 2
    torch.testing.assert_close(pair(q[0, :, 1]), pair(x[0, 1, :4]), rtol=1e-5, atol=1e-6)
    # out of range: NaN instead of a read past the tables; values still copied
    assert torch.isnan(q[0, :, 2]).all() and torch.isnan(k[0, :, 2]).all()
    assert torch.equal(v[0, 0], x[0, :, 5])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,n", [(1, 12288), (37, 1024), (4, 100)])
def test_silu_mul(dtype, rows, n):
    from chronoquant_mlx_amd.models import fused
    g = torch.Generator(device="cuda").manual_seed(n + rows)
    gu = (torch.randn(rows, 2 * n, device="cuda", generator=g) * 3).to(dtype)
    ref = F.silu(gu[:, :n]) * gu[:, n:]
    _assert_ulp(fused.silu_mul(gu), ref, f"silu {rows}x{n}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,k", [(4096, 4096), (6144, 4096), (4096, 12288), (13, 72), (9, 520),
                                 (1000, 4104)])
def test_gemv(dtype, n, k):
    # One input row through cq_gemv against the fp32 product rounded once.
    # The fp32 sums differ only in order (k terms), so the rounded results
    # agree to one ulp of the result plus the fp32 summation error bound.
    from chronoquant_mlx_amd.models import fused
    g = torch.Generator(device="cuda").manual_seed(n * 7 + k)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(dtype)
    x = torch.randn(1, 1, k, device="cuda", generator=g).to(dtype)
    got = fused.linear(x, w)
    exact = x.float().reshape(1, k) @ w.float().t()
    ref = exact.to(dtype).reshape(1, 1, n)
    mag = (x.float().abs().reshape(1, k) @ w.float().abs().t()).reshape(1, 1, n)
    err = (got.float() - ref.float()).abs()
    tol = ULP[dtype] * ref.float().abs() + k * 2.0 ** -23 * mag + TINY[dtype]
    assert (err <= tol).all(), (err - tol).max().item()
    assert got.shape == (1, 1, n) and got.dtype == dtype


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,k,with_res", [(6144, 4096, False), (24576, 4096, True), (13, 72, True),
                                          (100, 8192, True)])
def test_gemv_rms_norm(dtype, n, k, with_res):
    # One launch of "h = x + residual; y = W rms_norm(h)" against the unfused
    # library ops (cq_add_rms_norm / cq_rms_norm, then cq_gemv): h bit-exact;
    # y equal except where the two kernels' fp32 sums of squares round the
    # inverse norm to neighbouring values (a rare 1-ulp change of a normed
    # element, which moves y by at most |w| ulp(x) over k terms).
    from chronoquant_mlx_amd.models import fused
    g = torch.Generator(device="cuda").manual_seed(n + 3 * k)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(dtype)
    x = torch.randn(1, 1, k, device="cuda", generator=g).to(dtype)
    res = torch.randn(1, 1, k, device="cuda", generator=g).to(dtype) if with_res else None
    nw = (1 + 0.1 * torch.randn(k, device="cuda", generator=g)).to(dtype)
    y, h = fused.linear_rms_norm(x, res, nw, 1e-6, w, want_h=with_res)
    if with_res:
        h_ref, xn = fused.add_rms_norm(x, res, nw, 1e-6)
        assert torch.equal(h.view(torch.int16), h_ref.view(torch.int16))
    else:
        assert h is None
        xn = fused.rms_norm(x, nw, 1e-6)
    ref = fused.linear(xn, w)
    mag = (xn.float().abs().reshape(1, k) @ w.float().abs().t()).reshape(1, 1, n)
    tol = 2 * ULP[dtype] * ref.float().abs() + ULP[dtype] * mag + TINY[dtype]
    assert ((y.float() - ref.float()).abs() <= tol).all()
    same = (y.view(torch.int16) == ref.view(torch.int16)).float().mean().item()
    assert same >= 0.95, same


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,k", [(4096, 12288), (17, 64)])
def test_gemv_silu(dtype, n, k):
    # One launch of "y = W silu_mul(gate | up)" against cq_silu_mul then
    # cq_gemv: the gate values are the same rounded numbers, so y agrees
    # bit for bit.
    from chronoquant_mlx_amd.models import fused
    g = torch.Generator(device="cuda").manual_seed(n + k)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(dtype)
    gu = (torch.randn(1, 1, 2 * k, device="cuda", generator=g) * 2).to(dtype)
    y = fused.linear_silu(gu, w)
    ref = fused.linear(fused.silu_mul(gu), w)
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


def test_argument_errors():
    from chronoquant_mlx_amd._lib import ChronoQuantError
    from chronoquant_mlx_amd.models import fused
    x = torch.randn(2, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        fused.rms_norm(x, torch.ones(63, device="cuda", dtype=torch.bfloat16), 1e-6)
    cos, sin = _rope_tables(8)
    with pytest.raises(ChronoQuantError):  # head_dim 64 is not served
        qkv = torch.randn(1, 1, 3 * 128, device="cuda")
        from chronoquant_mlx_amd import _lib
        q = torch.empty(1, 1, 1, 128, device="cuda")
        _lib.call("cq_qkv_norm_rope", qkv.data_ptr(), None, None, q.data_ptr(), q.data_ptr(),
                  q.data_ptr(), cos.data_ptr(), sin.data_ptr(), 8,
                  torch.zeros(1, dtype=torch.int64, device="cuda").data_ptr(), 0, 1, 1, 1, 1, 64,
                  1e-6, 2, 0)


def test_fused_model_matches_torch_ops():
    # The decoder with fused ops against the same decoder running torch ops:
    # layer 0's attention output within the attention bar (its inputs agree to
    # an ulp), and the logits close (deeper layers quantise slightly different
    # K/V, so they are compared loosely).
    from chronoquant_mlx_amd import create_full_throttle_caches, patch
    from chronoquant_mlx_amd.models import qwen
    from chronoquant_mlx_amd.models.qwen import ModelArgs, random_model
    args = ModelArgs(hidden_size=512, num_hidden_layers=2, num_attention_heads=8,
                     num_key_value_heads=2, head_dim=128, intermediate_size=1024,
                     vocab_size=1000, max_position=4096)
    model = random_model(args, seed=3)
    prompt = torch.randint(0, 1000, (1, 200), generator=torch.Generator().manual_seed(6)).cuda()
    outs, logits = [], []
    hook = model.layers[0].self_attn.register_forward_hook(
        lambda m, i, o: outs.append(o.detach().float().clone()))
    patch.apply()
    try:
        with torch.no_grad():
            for fused_ops in (True, False):
                qwen.FUSED_OPS = fused_ops
                caches = create_full_throttle_caches(model)
                lg = model(prompt, caches).float()
                lg2 = model(prompt[:, -1:], caches).float()  # one decode step
                logits.append(torch.cat([lg, lg2], 1))
    finally:
        qwen.FUSED_OPS = True
        patch.revert()
        hook.remove()
    got, ref = outs[0], outs[2]
    assert ((got - ref).abs() <= 2e-3 + 1e-2 * ref.abs()).all()
    rel = ((logits[0] - logits[1]).norm() / logits[1].norm()).item()
    assert rel <= 2e-2, rel
    assert math.isfinite(rel)
