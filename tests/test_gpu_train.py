"""Backward and optimizer kernels of the C5 training step through the C-ABI,
against torch float64 autograd on the CPU (the gradient the jitted
value_and_grad of temp/dp_train.py:67-76 computes, in exact arithmetic).

Float tolerances: fp32 I/O paths are held to fp32 rounding of the fp64
result (relative to the scale of the quantity); bf16 paths to bf16 rounding
(2^-8 relative) plus the fp32 accumulation terms."""

import math

import numpy as np
import pytest
import torch

from oracle import bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K(cuda):
    from mi355x_pjrt import kernels

    kernels.lib()
    return kernels


def _f64(t):
    return t.detach().to("cpu", torch.float64)


def _rel(got, want):
    got, want = _f64(got), _f64(want)
    return float((got - want).norm() / max(float(want.norm()), 1e-30))


# ------------------------------------------------------------------ GELU backward
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gelu_tanh_bwd(K, dtype):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4099, generator=g) * 3
    x[:8] = torch.tensor([0.0, -0.0, 10.0, -10.0, 30.0, -30.0, 1e-20, -1e-3])
    dy = torch.randn(4099, generator=g)
    xd, dyd = x.to(dtype).cuda(), dy.to(dtype).cuda()
    got = K.gelu_tanh_bwd(xd, dyd)
    xr = _f64(xd).requires_grad_(True)
    torch.nn.functional.gelu(xr, approximate="tanh").backward(_f64(dyd))
    want = xr.grad
    if dtype == torch.float32:
        np.testing.assert_allclose(_f64(got), want, rtol=2e-5, atol=2e-6 * float(want.abs().max()))
    else:
        np.testing.assert_allclose(_f64(got), want, rtol=2 ** -7, atol=1e-6)
    # the bf16 vector path (length a multiple of 8, aligned)
    x8 = xd[:4096]
    got8 = K.gelu_tanh_bwd(x8, dyd[:4096])
    np.testing.assert_array_equal(_f64(got8), _f64(got[:4096]))


# ------------------------------------------------------------------ library GEMM
def _gemm_err(got, a, b, ref):
    """max |got - ref| relative to sum_k |a||b| (the fp32 accumulation bound)."""
    scale = _f64(a).abs() @ _f64(b).abs()
    return float(((_f64(got) - ref).abs() / (scale + 1e-30)).max())


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_gemm_blas_layouts(K, ta, tb, out_dtype):
    """Every operand orientation the step uses (A or B stored transposed),
    bf16 operands, fp32 / bf16 output, against float64."""
    g = torch.Generator().manual_seed(int(ta) * 2 + int(tb))
    M, N, Kd = 200, 136, 328
    a_st = torch.randn(Kd, M, generator=g) if ta else torch.randn(M, Kd, generator=g)
    b_st = torch.randn(N, Kd, generator=g) if tb else torch.randn(Kd, N, generator=g)
    a = (a_st.bfloat16().cuda().t() if ta else a_st.bfloat16().cuda())
    b = (b_st.bfloat16().cuda().t() if tb else b_st.bfloat16().cuda())
    got = K.gemm_blas(a, b, out_dtype=out_dtype)
    ref = _f64(a) @ _f64(b)
    tol = 1e-5 if out_dtype == torch.float32 else 2 ** -8
    if out_dtype == torch.float32:
        assert _gemm_err(got, a, b, ref) < tol
    else:
        np.testing.assert_allclose(_f64(got), ref, rtol=2 ** -8, atol=1e-5 * float((_f64(a).abs() @ _f64(b).abs()).max()))


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("M,N,Kd", [(77, 1001, 133), (1, 9, 5), (130, 3, 1031)])
def test_gemm_blas_ragged(K, M, N, Kd, ta, tb, out_dtype):
    """Sizes and row strides that are no multiple of the kernels' vector
    widths (the vocabulary axis of the logits GEMMs is one), against float64."""
    g = torch.Generator().manual_seed(M * 7 + N + Kd + 2 * int(ta) + int(tb))
    a_st = torch.randn(Kd, M, generator=g) if ta else torch.randn(M, Kd, generator=g)
    b_st = torch.randn(N, Kd, generator=g) if tb else torch.randn(Kd, N, generator=g)
    a = (a_st.bfloat16().cuda().t() if ta else a_st.bfloat16().cuda())
    b = (b_st.bfloat16().cuda().t() if tb else b_st.bfloat16().cuda())
    got = K.gemm_blas(a, b, out_dtype=out_dtype)
    ref = _f64(a) @ _f64(b)
    scale = float((_f64(a).abs() @ _f64(b).abs()).max())
    if out_dtype == torch.float32:
        assert float((_f64(got) - ref).abs().max()) < 1e-5 * scale
    else:
        np.testing.assert_allclose(_f64(got), ref, rtol=2 ** -8, atol=1e-5 * scale)
    assert torch.equal(got, K.gemm_blas(a, b, out_dtype=out_dtype))


def test_gemm_blas_batched_alpha_beta_and_f32(K):
    g = torch.Generator().manual_seed(9)
    a = torch.randn(3, 40, 24, generator=g).cuda()
    b = torch.randn(3, 24, 56, generator=g).cuda()
    c0 = torch.randn(3, 40, 56, generator=g).cuda()
    got = K.gemm_blas(a, b, out=c0.clone(), alpha=0.5, beta=2.0)
    ref = 0.5 * (_f64(a) @ _f64(b)) + 2.0 * _f64(c0)
    assert float((_f64(got) - ref).abs().max()) < 1e-4


@pytest.mark.parametrize("M,N,Kd,splits", [(768, 3072, 8192, 4), (96, 64, 512, 8), (64, 32, 64, 1)])
def test_gemm_blas_splitk(K, M, N, Kd, splits):
    """Weight-gradient form (A = Xᵀ stored [K, M]): split-K agrees with the
    plain GEMM to fp32 accumulation and is bit-reproducible."""
    g = torch.Generator().manual_seed(M + N + splits)
    x = (torch.randn(Kd, M, generator=g)).bfloat16().cuda()
    dy = torch.randn(Kd, N, generator=g).bfloat16().cuda()
    a = x.t()
    got = K.gemm_blas_splitk(a, dy, splits)
    if M * N * Kd <= 96 * 64 * 512:
        ref = _f64(a) @ _f64(dy)
    else:
        ref = _f64(K.gemm_blas(a, dy, out_dtype=torch.float32))
    scale = float((_f64(x).abs().t() @ _f64(dy).abs()).max())
    assert float((_f64(got) - ref).abs().max()) < 2e-6 * scale
    assert torch.equal(got, K.gemm_blas_splitk(a, dy, splits))


@pytest.mark.parametrize("M,N,Kd,splits", [(768, 3072, 8192, 4), (3072, 768, 8192, 2), (768, 768, 8192, 8),
                                            (96, 64, 512, 8), (64, 32, 64, 1)])
def test_gemm_splitk(K, M, N, Kd, splits):
    """Hand-written split-K (mk_gemm_splitk) on the weight-gradient form
    (A = Xᵀ stored [K, M], B = dY [K, N]): within fp32 accumulation of the
    float64 product and bit-reproducible."""
    print(f"case: mk_gemm_splitk M={M} N={N} K={Kd} splits={splits}", flush=True)
    g = torch.Generator().manual_seed(M + N + splits)
    x = (torch.randn(Kd, M, generator=g)).bfloat16().cuda()
    dy = torch.randn(Kd, N, generator=g).bfloat16().cuda()
    a = x.t()
    got = K.gemm_splitk(a, dy, splits)
    ref = _f64(a) @ _f64(dy)
    scale = float((_f64(x).abs().t() @ _f64(dy).abs()).max())
    assert float((_f64(got) - ref).abs().max()) < 2e-6 * scale
    assert torch.equal(got, K.gemm_splitk(a, dy, splits))


# ------------------------------------------------------------------ row adds
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 13), (8192, 768), (33, 2304)])
def test_add_rows(K, dtype, rows, cols):
    g = torch.Generator().manual_seed(rows * 31 + cols)
    a, b = (torch.randn(rows, cols, generator=g).to(dtype).cuda() for _ in range(2))
    bias = torch.randn(cols, generator=g).to(dtype).cuda()
    exact = _f64(a) + _f64(b) + _f64(bias)
    tol = dict(rtol=0, atol=1e-6) if dtype == torch.float32 else dict(rtol=2 ** -8, atol=1e-6)
    got = K.add_rows(a, b, bias)
    np.testing.assert_allclose(_f64(got), exact, **tol)
    # the kernel adds left to right in fp32 and rounds once: bit-exact with the same order on the CPU
    af, bf, cf = (t.cpu().float() for t in (a, b, bias))
    np.testing.assert_array_equal(_f64(got), _f64(((af + bf) + cf).to(dtype)))
    np.testing.assert_array_equal(_f64(K.add_rows(a, None, bias)), _f64((af + cf).to(dtype)))
    np.testing.assert_array_equal(_f64(K.add_rows(a, b)), _f64((af + bf).to(dtype)))
    # in place over a, as the step's residual adds run
    a2 = a.clone()
    K.add_rows(a2, b, bias, out=a2)
    np.testing.assert_array_equal(_f64(a2), _f64(got))


# ------------------------------------------------------------------ fused forward rows
@pytest.mark.parametrize("rows,cols", [(8192, 768), (37, 100), (5, 2048), (3, 260)])
def test_add_layernorm(K, rows, cols):
    """The stored sum equals mk_add_rows bit for bit; the LayerNorm of it is
    within bf16 rounding of the float64 LayerNorm of the rounded sum (and of
    mk_layernorm on that sum)."""
    g = torch.Generator().manual_seed(rows + cols)
    a, b = ((torch.randn(rows, cols, generator=g) * 2).bfloat16().cuda() for _ in range(2))
    bias = (0.1 * torch.randn(cols, generator=g)).bfloat16().cuda()
    gamma = (1 + 0.1 * torch.randn(cols, generator=g)).bfloat16().cuda()
    beta = (0.1 * torch.randn(cols, generator=g)).bfloat16().cuda()
    s, y = K.add_layernorm(a, b, bias, gamma, beta, 1e-5)
    assert torch.equal(s, K.add_rows(a, b, bias))
    want = torch.nn.functional.layer_norm(_f64(s), (cols,), _f64(gamma), _f64(beta), 1e-5)
    np.testing.assert_allclose(_f64(y), want, rtol=2 ** -7, atol=2 ** -8)
    y2 = K.layernorm(s, gamma, beta, 1e-5)
    assert float((_f64(y) - _f64(y2)).abs().max()) <= 2 ** -7 * float(_f64(y2).abs().max())
    # no second operand, no bias
    s1, y1 = K.add_layernorm(a, None, None, gamma, beta, 1e-5)
    assert torch.equal(s1, a)


@pytest.mark.parametrize("rows,cols,off", [(8192, 768, 0), (37, 100, 0), (5, 4096, 0), (3, 768, 1)])
def test_add_layernorm_f32_rows(K, rows, cols, off):
    """fp32 rows (mk_add_layernorm_typed): the stored sum is the fp32 a + b
    bit for bit, and the LayerNorm (fp32 or bf16) is mk_layernorm_typed of
    that sum bit for bit (same kernel arithmetic; off = 1 starts the operands
    off their 16-byte alignment, the streaming kernel)."""
    g = torch.Generator().manual_seed(rows * 5 + cols + off)

    def dev(t):
        flat = torch.zeros(t.numel() + off, dtype=t.dtype)
        flat[off:] = t.reshape(-1)
        return flat.cuda()[off:].view(t.shape)
    a, b = (dev(torch.randn(rows, cols, generator=g) * 2) for _ in range(2))
    gamma = dev(1 + 0.1 * torch.randn(cols, generator=g))
    beta = dev(0.1 * torch.randn(cols, generator=g))
    for od in (torch.float32, torch.bfloat16):
        s, y = K.add_layernorm(a, b, None, gamma, beta, 1e-5, out_dtype=od)
        assert s.dtype == torch.float32 and y.dtype == od
        assert torch.equal(s, a + b)
        if off == 0:  # (the plain LayerNorm of the aligned sum takes the other kernel when off > 0)
            assert torch.equal(y, K.layernorm(s, gamma, beta, 1e-5, out_dtype=od))
        want = torch.nn.functional.layer_norm(_f64(s), (cols,), _f64(gamma), _f64(beta), 1e-5)
        tol = 2 ** -7 if od == torch.bfloat16 else 1e-5
        assert float((_f64(y) - want).abs().max()) <= tol * (float(want.abs().max()) + 1)


@pytest.mark.parametrize("rows,cols", [(8192, 3072), (33, 100)])
def test_bias_gelu(K, rows, cols):
    """pre equals mk_add_rows and y equals mk_gelu_tanh of pre, bit for bit
    (the second shape takes the two-pass path); in place over x."""
    g = torch.Generator().manual_seed(rows * 7 + cols)
    x = (torch.randn(rows, cols, generator=g) * 2).bfloat16().cuda()
    bias = (0.5 * torch.randn(cols, generator=g)).bfloat16().cuda()
    pre, y = K.bias_gelu(x, bias)
    want_pre = K.add_rows(x, None, bias)
    assert torch.equal(pre, want_pre)
    assert torch.equal(y, K.gelu_tanh(want_pre))
    x2 = x.clone()
    K.bias_gelu(x2, bias, pre_out=x2)
    assert torch.equal(x2, pre)


# ------------------------------------------------------------------ column sums
@pytest.mark.parametrize("rows,cols", [(1, 1), (19, 768), (8192, 768), (8, 786432), (1000, 257)])
def test_col_sum(K, rows, cols):
    g = torch.Generator().manual_seed(rows + cols)
    x = torch.randn(rows, cols, generator=g)
    for dtype in (torch.float32, torch.bfloat16):
        xd = x.to(dtype).cuda()
        got = K.col_sum(xd)
        want = _f64(xd).sum(0)
        scale = _f64(xd).abs().sum(0)
        assert float(((_f64(got) - want).abs() / (scale + 1e-30)).max()) < 1e-6
    # deterministic: same bits twice
    a, b = K.col_sum(xd), K.col_sum(xd)
    assert torch.equal(a, b)


# ------------------------------------------------------------------ LayerNorm backward
@pytest.mark.parametrize("cols", [1, 100, 768, 1000, 2048])
def test_layernorm_bwd_f32(K, cols):
    g = torch.Generator().manual_seed(cols)
    rows = 37
    x = torch.randn(rows, cols, generator=g) * 2 + 0.5
    gamma = torch.randn(cols, generator=g)
    beta = torch.randn(cols, generator=g)
    dy = torch.randn(rows, cols, generator=g)
    dx, dgam, dbet = K.layernorm_bwd(x.cuda(), gamma.cuda(), dy.cuda(), 1e-5)
    xr = x.double().requires_grad_(True)
    gr = gamma.double().requires_grad_(True)
    br = beta.double().requires_grad_(True)
    torch.nn.functional.layer_norm(xr, (cols,), gr, br, 1e-5).backward(dy.double())
    # dx is rstd times an O(|dy gamma|) combination: fp32 rounding relative to
    # that scale (a one-column row has dx = 0 exactly)
    rstd = 1 / torch.sqrt(x.double().var(-1, unbiased=False, keepdim=True) + 1e-5)
    scale = float((rstd * (dy.double() * gamma.double()).abs()).max())
    assert float((_f64(dx) - xr.grad).abs().max()) < 5e-5 * scale
    assert _rel(dgam, gr.grad) < 2e-5 or cols == 1
    assert float((_f64(dgam) - gr.grad).abs().max()) < 1e-5 * float((dy.double() * (x.double() - x.double().mean(-1, keepdim=True)) * rstd).abs().sum(0).max() + 1)
    assert _rel(dbet, br.grad) < 2e-6


def test_layernorm_bwd_bf16_c5_rows(K):
    g = torch.Generator().manual_seed(7)
    rows, cols = 8192, 768
    x = (torch.randn(rows, cols, generator=g) * 1.5).bfloat16()
    gamma = (1 + 0.1 * torch.randn(cols, generator=g)).bfloat16()
    dy = torch.randn(rows, cols, generator=g).bfloat16()
    dx, dgam, dbet = K.layernorm_bwd(x.cuda(), gamma.cuda(), dy.cuda(), 1e-5)
    xr = x.double().requires_grad_(True)
    gr = gamma.double().requires_grad_(True)
    br = torch.zeros(cols, dtype=torch.float64, requires_grad=True)
    torch.nn.functional.layer_norm(xr, (cols,), gr, br, 1e-5).backward(dy.double())
    assert _rel(dx, xr.grad) < 6e-3  # bf16 output rounding
    assert _rel(dgam, gr.grad) < 1e-5
    assert _rel(dbet, br.grad) < 1e-6
    # dx alone (no parameter gradients, no workspace needed)
    dx2, _, _ = K.layernorm_bwd(x.cuda(), gamma.cuda(), dy.cuda(), 1e-5, want_params=False)
    assert torch.equal(dx2, dx)


@pytest.mark.parametrize("dtype,rows,cols", [(torch.bfloat16, 8192, 768), (torch.bfloat16, 50, 1000),
                                             (torch.float32, 8192, 768), (torch.float32, 37, 1000),
                                             (torch.float32, 9, 2048),
                                             (torch.bfloat16, 5, 100)])
def test_layernorm_bwd_residual_and_colsum(K, dtype, rows, cols):
    """dx = dres + LN'(dy) in place over dres, with dgamma, dbeta and the
    column sums of dx from the same pass (the pre-LN residual block)."""
    g = torch.Generator().manual_seed(rows * 3 + cols)
    x = (torch.randn(rows, cols, generator=g) * 1.5 + 0.2).to(dtype)
    gamma = (1 + 0.1 * torch.randn(cols, generator=g)).to(dtype)
    dy = torch.randn(rows, cols, generator=g).to(dtype)
    dres = torch.randn(rows, cols, generator=g).to(dtype)
    buf = dres.cuda()
    d16 = torch.empty(rows, cols, dtype=torch.bfloat16, device="cuda") if dtype == torch.float32 else None
    dx, dgam, dbet, csum = K.layernorm_bwd(x.cuda(), gamma.cuda(), dy.cuda(), 1e-5, dx=buf, dres=buf,
                                           want_colsum=True, dx_bf16=d16)
    assert dx.data_ptr() == buf.data_ptr()
    if d16 is not None:  # the bf16 copy is the RNE rounding of the stored fp32 dx
        assert torch.equal(d16.cpu(), dx.cpu().bfloat16())
    xr = x.double().requires_grad_(True)
    gr = gamma.double().requires_grad_(True)
    br = torch.zeros(cols, dtype=torch.float64, requires_grad=True)
    torch.nn.functional.layer_norm(xr, (cols,), gr, br, 1e-5).backward(dy.double())
    want = xr.grad + dres.double()
    tol = 6e-3 if dtype == torch.bfloat16 else 2e-5
    assert _rel(dx, want) < tol
    assert _rel(dgam, gr.grad) < 1e-5
    assert _rel(dbet, br.grad) < 1e-6
    # column sums of the stored dx, to its rounding
    assert _rel(csum, want.sum(0)) < (1e-2 if dtype == torch.bfloat16 else 2e-5)
    np.testing.assert_allclose(_f64(csum), _f64(dx).sum(0), rtol=0,
                               atol=(2 ** -8 if dtype == torch.bfloat16 else 1e-5) * float(_f64(dx).abs().sum(0).max()))
    # deterministic
    buf2 = dres.cuda()
    _, _, _, csum2 = K.layernorm_bwd(x.cuda(), gamma.cuda(), dy.cuda(), 1e-5, dx=buf2, dres=buf2, want_colsum=True)
    assert torch.equal(buf2, dx) and torch.equal(csum2, csum)


@pytest.mark.parametrize("dtype,rows,cols", [(torch.bfloat16, 8192, 3072), (torch.bfloat16, 33, 100),
                                             (torch.float32, 300, 256), (torch.bfloat16, 7, 13)])
def test_gelu_tanh_bwd_colsum(K, dtype, rows, cols):
    g = torch.Generator().manual_seed(rows + cols)
    x = (torch.randn(rows, cols, generator=g) * 2).to(dtype).cuda()
    dy = torch.randn(rows, cols, generator=g).to(dtype).cuda()
    dx, csum = K.gelu_tanh_bwd_colsum(x, dy)
    np.testing.assert_array_equal(_f64(dx), _f64(K.gelu_tanh_bwd(x, dy)))  # same values as the plain pass
    want = _f64(dx).sum(0)
    scale = _f64(dx).abs().sum(0)
    tol = 2 ** -7 if dtype == torch.bfloat16 else 1e-6  # bf16: the sum runs over the unrounded products
    assert float(((_f64(csum) - want).abs() / (scale + 1e-30)).max()) < tol
    # in place over dy
    dy2 = dy.clone()
    dx2, csum2 = K.gelu_tanh_bwd_colsum(x, dy2, out=dy2)
    assert torch.equal(dx2, dx) and torch.equal(csum2, csum)


# ------------------------------------------------------------------ softmax cross-entropy
@pytest.mark.parametrize("rows,cols", [(64, 257), (5, 1), (3, 50257)])
def test_softmax_xent_f32(K, rows, cols):
    g = torch.Generator().manual_seed(rows * cols)
    x = torch.randn(rows, cols, generator=g) * 4
    lab = torch.randint(0, cols, (rows,), generator=g, dtype=torch.int32)
    loss, dl = K.softmax_xent(x.cuda(), lab.cuda(), 1.0 / rows)
    xr = x.double().requires_grad_(True)
    ref = torch.nn.functional.cross_entropy(xr, lab.long(), reduction="none")
    ref.mean().backward()
    np.testing.assert_allclose(_f64(loss), _f64(ref), rtol=1e-5, atol=1e-5)
    assert _rel(dl, xr.grad) < 1e-5


def test_softmax_xent_bf16_in_place(K):
    g = torch.Generator().manual_seed(3)
    rows, cols = 16, 50257
    x = (torch.randn(rows, cols, generator=g) * 3).bfloat16()
    lab = torch.randint(0, cols, (rows,), generator=g, dtype=torch.int64)
    xd = x.cuda()
    loss, dl = K.softmax_xent(xd, lab.cuda(), 1.0 / rows, dlogits=xd)
    assert dl.data_ptr() == xd.data_ptr()
    xr = x.double().requires_grad_(True)
    ref = torch.nn.functional.cross_entropy(xr, lab, reduction="none")
    ref.mean().backward()
    np.testing.assert_allclose(_f64(loss), _f64(ref), rtol=1e-5, atol=1e-5)
    assert _rel(dl, xr.grad) < 4e-3


@pytest.mark.parametrize("rows,cols", [(9, 1), (5, 7), (6, 9), (33, 1000), (7, 4099), (3, 32773), (2, 65536),
                                       (2, 70001)])
def test_softmax_xent_bf16_shapes(K, rows, cols):
    """Register-resident rows (unaligned head / tail, every vector-count
    bucket) and the streaming kernel past 64K columns; -inf logits and an
    out-of-range label, above and below (loss = logsumexp, gradient without
    the one-hot term)."""
    g = torch.Generator().manual_seed(rows + cols)
    x = (torch.randn(rows, cols, generator=g) * 3).bfloat16()
    if cols > 3:
        x[0, 1] = float("-inf")
        x[-1, -2] = float("-inf")
    lab = torch.randint(0, cols, (rows,), generator=g, dtype=torch.int32)
    lab[-1] = cols  # out of range, above and below
    if rows > 1:
        lab[0] = -1
    loss, dl = K.softmax_xent(x.cuda(), lab.cuda(), 1.0 / rows)
    xr = x.double()
    lse = torch.logsumexp(xr, -1)
    p = torch.softmax(xr, -1)
    onehot = torch.zeros_like(p)
    ok = (lab >= 0) & (lab < cols)
    onehot[torch.arange(rows)[ok], lab[ok].long()] = 1.0
    want_grad = (p - onehot) / rows
    want_loss = lse - torch.where(ok, xr[torch.arange(rows), lab.clamp(0, cols - 1).long()], 0.0)
    np.testing.assert_allclose(_f64(loss), want_loss, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(_f64(dl), want_grad, rtol=2 ** -7, atol=1e-30)


@pytest.mark.parametrize("rows,cols", [(7, 1000), (5, 20011), (4, 50257), (2, 70001)])
def test_softmax_xent_f32_logits_bf16_dlogits(K, rows, cols):
    """fp32 logits with a bf16 gradient (mk_softmax_xent_typed): registers
    for up to 24 elements per thread, the two-pass streaming kernel above;
    the loss as the fp32 kernel's to 1e-5 relative, the gradient within
    one bf16 ulp of the float64 value; out-of-range labels (-1 and cols)."""
    g = torch.Generator().manual_seed(rows * 7 + cols)
    x = torch.randn(rows, cols, generator=g) * 3
    x[0, 1] = float("-inf")
    lab = torch.randint(0, cols, (rows,), generator=g, dtype=torch.int32)
    lab[-1] = cols
    lab[0] = -1
    dl = torch.empty(rows, cols, dtype=torch.bfloat16, device="cuda")
    loss, dl = K.softmax_xent(x.cuda(), lab.cuda(), 1.0 / rows, dlogits=dl)
    xr = x.double()
    lse = torch.logsumexp(xr, -1)
    ok = (lab >= 0) & (lab < cols)
    want_loss = lse - torch.where(ok, xr[torch.arange(rows), lab.clamp(0, cols - 1).long()], 0.0)
    np.testing.assert_allclose(_f64(loss), want_loss, rtol=1e-5, atol=1e-5)
    p = torch.softmax(xr, -1)
    onehot = torch.zeros_like(p)
    onehot[torch.arange(rows)[ok], lab[ok].long()] = 1.0
    want = ((p - onehot) / rows).numpy()
    got = bf16.from_bf16_bits(dl.cpu().view(torch.int16).numpy().view(np.uint16)).astype(np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-38))) - 7)
    assert np.all(np.abs(got - want) <= ulp + 1e-7 * np.abs(want).max())


@pytest.mark.parametrize("cols,ld_in,ld_out", [(50257, 50260, 50264), (50257, 50264, 50264), (4096, 4100, 4104),
                                              (4099, 4104, 4104), (70001, 70004, 70008)])
def test_softmax_xent_strided_f32_logits_bf16_dlogits(K, cols, ld_in, ld_out):
    """Padded row pitches (mk_softmax_xent_strided): fp32 logits rows ld_in
    apart with NaN in the padding (never read), bf16 dlogits rows ld_out
    apart whose padding must stay untouched; 16-byte aligned rows take the
    vector kernel (a partial last vector when cols % 4 != 0), 70001 columns
    the streaming kernel.  Loss to 1e-5 of float64, gradient within one bf16
    ulp, out-of-range labels -1 and cols."""
    rows = 6
    print(f"case: xent strided cols={cols} ld_in={ld_in} ld_out={ld_out}", flush=True)
    g = torch.Generator().manual_seed(cols + ld_in)
    x = torch.randn(rows, cols, generator=g) * 3
    x[1, 2] = float("-inf")
    lab = torch.randint(0, cols, (rows,), generator=g, dtype=torch.int32)
    lab[-1] = cols
    lab[0] = -1
    lab[2] = cols - 1
    xbuf = torch.full((rows, ld_in), float("nan"), dtype=torch.float32, device="cuda")
    xbuf[:, :cols] = x.cuda()
    dbuf = torch.full((rows, ld_out), -7.0, dtype=torch.bfloat16, device="cuda")
    loss, dl = K.softmax_xent(xbuf[:, :cols], lab.cuda(), 1.0 / rows, dlogits=dbuf[:, :cols])
    xr = x.double()
    lse = torch.logsumexp(xr, -1)
    ok = (lab >= 0) & (lab < cols)
    want_loss = lse - torch.where(ok, xr[torch.arange(rows), lab.clamp(0, cols - 1).long()], 0.0)
    np.testing.assert_allclose(_f64(loss), want_loss, rtol=1e-5, atol=1e-5)
    p = torch.softmax(xr, -1)
    onehot = torch.zeros_like(p)
    onehot[torch.arange(rows)[ok], lab[ok].long()] = 1.0
    want = ((p - onehot) / rows).numpy()
    got = bf16.from_bf16_bits(dbuf[:, :cols].cpu().view(torch.int16).numpy().view(np.uint16)).astype(np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-38))) - 7)
    assert np.all(np.abs(got - want) <= ulp + 1e-7 * np.abs(want).max())
    assert bool((dbuf[:, cols:].float() == -7.0).all())
    if cols % 4 == 0:
        # packed rows of a multiple of 4 columns take the same vector kernel:
        # the same bits (other widths run the element-wise kernels, whose
        # sums of exponentials are ordered differently)
        dl2 = torch.empty(rows, cols, dtype=torch.bfloat16, device="cuda")
        loss2, dl2 = K.softmax_xent(x.cuda(), lab.cuda(), 1.0 / rows, dlogits=dl2)
        assert torch.equal(loss2, loss)
        assert torch.equal(dl2, dbuf[:, :cols])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_softmax_xent_strided_same_type_in_place(K, dtype):
    """bf16 (register-resident kernel) and fp32 logits with a padded row pitch,
    the gradient written in place over them: same bits as the packed rows,
    padding untouched."""
    rows, cols, ld = 5, 50257, 50264
    g = torch.Generator().manual_seed(17)
    x = (torch.randn(rows, cols, generator=g) * 3).to(dtype)
    lab = torch.randint(0, cols, (rows,), generator=g, dtype=torch.int64)
    buf = torch.full((rows, ld), -7.0, dtype=dtype, device="cuda")
    buf[:, :cols] = x.cuda()
    v = buf[:, :cols]
    loss, dl = K.softmax_xent(v, lab.cuda(), 1.0 / rows, dlogits=v)
    xd = x.cuda()
    loss2, dl2 = K.softmax_xent(xd, lab.cuda(), 1.0 / rows, dlogits=xd)
    assert torch.equal(loss, loss2)
    assert torch.equal(buf[:, :cols], dl2)
    assert bool((buf[:, cols:].float() == -7.0).all())


def test_softmax_xent_bf16_dlogits_offset_view(K):
    """dlogits in a different 16-byte phase from logits (an offset view):
    the launcher must not use the register-resident kernel's vector stores,
    whose offsets follow the logits' phase."""
    g = torch.Generator().manual_seed(11)
    rows, cols = 6, 4099
    x = (torch.randn(rows, cols, generator=g) * 3).bfloat16()
    lab = torch.randint(0, cols, (rows,), generator=g, dtype=torch.int32)
    buf = torch.zeros(rows * cols + 8, dtype=torch.bfloat16, device="cuda")
    for off in (1, 3):
        buf.zero_()
        xd = x.cuda()
        dl = buf[off:off + rows * cols].view(rows, cols)
        assert (dl.data_ptr() - xd.data_ptr()) % 16 != 0
        loss, dl = K.softmax_xent(xd, lab.cuda(), 1.0 / rows, dlogits=dl)
        xr = x.double().requires_grad_(True)
        ref = torch.nn.functional.cross_entropy(xr, lab.long(), reduction="none")
        ref.mean().backward()
        np.testing.assert_allclose(_f64(loss), _f64(ref), rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(_f64(dl), _f64(xr.grad), rtol=2 ** -7, atol=1e-30)
        assert float(buf[:off].abs().sum()) == 0.0 and float(buf[off + rows * cols:].abs().sum()) == 0.0


# ------------------------------------------------------------------ Adam
def _adam_ref(p, g, m, v, lr, b1, b2, eps, bc1, bc2):
    m = b1 * m + (1 - b1) * g
    v = b2 * v + (1 - b2) * g * g
    return p - lr * (m / bc1) / (np.sqrt(v / bc2) + eps), m, v


@pytest.mark.parametrize("n", [100003, 100000])  # scalar kernel; four-wide kernel (n % 4 == 0)
def test_adam_update_f32_and_master(K, n):
    rng = np.random.default_rng(0)
    p = rng.standard_normal(n).astype(np.float32)
    g = rng.standard_normal(n).astype(np.float32)
    m = (rng.standard_normal(n) * 0.1).astype(np.float32)
    v = np.abs(rng.standard_normal(n) * 0.01).astype(np.float32)
    hp = dict(lr=1e-3, b1=0.9, b2=0.999, eps=1e-8, bc1=1 - 0.9 ** 3, bc2=1 - 0.999 ** 3)
    wp, wm, wv = _adam_ref(p.astype(np.float64), g.astype(np.float64), m.astype(np.float64),
                           v.astype(np.float64), **hp)
    pd, gd, md, vd = (torch.from_numpy(a.copy()).cuda() for a in (p, g, m, v))
    K.adam_update(pd, gd, md, vd, **hp)
    # fp32 rounding of each update, bounded by the magnitudes of its terms
    # (m = b1 m + (1-b1) g can cancel, so a relative bound on m alone is wrong)
    e32 = 2.0 ** -23
    m64, g64, v64, p64 = (a.astype(np.float64) for a in (m, g, v, p))
    m_scale = np.abs(hp["b1"] * m64) + np.abs((1 - hp["b1"]) * g64)
    assert np.all(np.abs(md.cpu().numpy() - wm) <= 3 * e32 * m_scale + 1e-30)
    assert np.all(np.abs(vd.cpu().numpy() - wv) <= 4 * e32 * wv + 1e-30)
    step = hp["lr"] * (np.abs(wm) / hp["bc1"] + 3 * e32 * m_scale / hp["bc1"]) / (np.sqrt(wv / hp["bc2"]) + hp["eps"])
    assert np.all(np.abs(pd.cpu().numpy() - wp) <= 2 * e32 * np.abs(p64) + 8 * e32 * step + 1e-30)
    # bf16 parameter with an fp32 master copy and a bf16 gradient
    master = torch.from_numpy(p.copy()).cuda()
    pb = master.bfloat16()
    gb = torch.from_numpy(g).bfloat16().cuda()
    md, vd = torch.from_numpy(m.copy()).cuda(), torch.from_numpy(v.copy()).cuda()
    K.adam_update(pb, gb, md, vd, master=master, **hp)
    wp2, _, _ = _adam_ref(p.astype(np.float64), gb.cpu().double().numpy(), m.astype(np.float64),
                          v.astype(np.float64), **hp)
    assert np.all(np.abs(master.cpu().numpy() - wp2) <= 2 * e32 * np.abs(p64) + 8 * e32 * step * 2 + 1e-30)
    assert torch.equal(pb, master.bfloat16())


def test_adam_update_dev_matches_host_scalars(K):
    """lr, bc1, bc2 from a device buffer give the same bits as the same
    values passed as host scalars (both rounded once to fp32)."""
    rng = np.random.default_rng(1)
    n = 70001
    p, g, m = (rng.standard_normal(n).astype(np.float32) for _ in range(3))
    v = np.abs(rng.standard_normal(n)).astype(np.float32) * 0.01
    lr, b1, b2, eps, t = 3e-4, 0.9, 0.95, 1e-8, 7
    bc1, bc2 = 1 - b1 ** t, 1 - b2 ** t
    a = [torch.from_numpy(x.copy()).cuda() for x in (p, g, m, v)]
    b = [torch.from_numpy(x.copy()).cuda() for x in (p, g, m, v)]
    K.adam_update(a[0], a[1], a[2], a[3], lr, b1, b2, eps, bc1, bc2)
    hyper = torch.tensor([lr, bc1, bc2], dtype=torch.float32).cuda()
    K.adam_update_dev(b[0], b[1], b[2], b[3], hyper, b1, b2, eps)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


# ------------------------------------------------------------------ attention backward
def _attn_ref(q, k, v, scale, causal):
    s = (q @ k.transpose(-1, -2)) * scale
    if causal:
        Sq, Sk = s.shape[-2:]
        mask = torch.ones(Sq, Sk, dtype=torch.bool).tril()
        s = s.masked_fill(~mask, float("-inf"))
    return torch.softmax(s, -1) @ v


@pytest.mark.parametrize("B,H,S,D,causal", [(2, 3, 128, 64, True), (1, 2, 100, 128, True),
                                            (2, 2, 96, 64, False), (1, 1, 1, 64, True)])
def test_sdpa_bwd(K, B, H, S, D, causal):
    g = torch.Generator().manual_seed(S + D)
    q, k, v = ((torch.randn(B, H, S, D, generator=g) * (1.0 if i < 2 else 0.5)).bfloat16() for i in range(3))
    do = torch.randn(B, H, S, D, generator=g).bfloat16()
    scale = 1 / math.sqrt(D)
    qd, kd, vd, dod = (t.cuda() for t in (q, k, v, do))
    lse = torch.empty(B, H, S, dtype=torch.float32, device="cuda")
    o = K.sdpa_fwd(qd, kd, vd, scale, causal, lse=lse)
    dq, dk, dv = K.sdpa_bwd(qd, kd, vd, o, dod, lse, scale, causal)
    qr, kr, vr = (t.double().requires_grad_(True) for t in (q, k, v))
    _attn_ref(qr, kr, vr, scale, causal).backward(do.double())
    # bf16 operands, bf16 P / dS and bf16 outputs: relative L2 error of a few
    # 2^-8.  With one key dq = dk = 0 exactly (dP equals D), so the error is
    # measured against max(|grad|, 1e-3 |dO|) rather than |grad| alone.
    floor = 1e-3 * float(do.double().norm())
    for got, want, name in ((dq, qr.grad, "dq"), (dk, kr.grad, "dk"), (dv, vr.grad, "dv")):
        err = float((_f64(got) - want).norm()) / max(float(want.norm()), floor)
        assert err < 2.5e-2, (name, err)


def _bwd_vs_float64(K, B, H, Sq, Sk, D, causal, seed):
    """mk_sdpa_bwd on bf16 inputs with o, lse of the float64 forward, against
    float64 autograd; returns the GPU gradients."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Sq, D, generator=g).bfloat16()
    k = torch.randn(B, H, Sk, D, generator=g).bfloat16()
    v = (torch.randn(B, H, Sk, D, generator=g) * 0.5).bfloat16()
    do = torch.randn(B, H, Sq, D, generator=g).bfloat16()
    scale = 1 / math.sqrt(D)
    qr, kr, vr = (t.double().requires_grad_(True) for t in (q, k, v))
    s = (qr @ kr.transpose(-1, -2)) * scale
    if causal:
        s = s.masked_fill(~torch.ones(Sq, Sk, dtype=torch.bool).tril(), float("-inf"))
    o = torch.softmax(s, -1) @ vr
    o.backward(do.double())
    lse = torch.logsumexp(s.detach(), -1).float().cuda()
    dq, dk, dv = K.sdpa_bwd(q.cuda(), k.cuda(), v.cuda(), o.detach().bfloat16().cuda(), do.cuda(), lse, scale, causal)
    floor = 1e-3 * float(do.double().norm())
    for got, want, name in ((dq, qr.grad, "dq"), (dk, kr.grad, "dk"), (dv, vr.grad, "dv")):
        err = float((_f64(got) - want).norm()) / max(float(want.norm()), floor)
        assert err < 2.5e-2, (name, err)
        assert bool(torch.isfinite(got).all()), name
    return dq, dk, dv


# flash path (D 64 / 128): ragged tiles, Sq != Sk both ways, the C5 sequence
# length; D 96: the materialised path
@pytest.mark.parametrize("B,H,Sq,Sk,D,causal", [
    (1, 2, 1024, 1024, 64, True), (1, 1, 200, 200, 64, True), (2, 1, 300, 300, 128, False),
    (1, 2, 70, 200, 64, False), (1, 1, 200, 70, 64, True), (1, 1, 70, 200, 128, True),
    (1, 1, 129, 129, 128, True), (1, 2, 65, 33, 64, False), (1, 2, 100, 100, 96, True)])
def test_sdpa_bwd_vs_float64(K, B, H, Sq, Sk, D, causal):
    print(f"case: sdpa_bwd B{B} H{H} Sq{Sq} Sk{Sk} D{D} causal={causal}", flush=True)
    _bwd_vs_float64(K, B, H, Sq, Sk, D, causal, seed=Sq * 7 + Sk + D)


def test_sdpa_bwd_deterministic(K):
    """No atomics: two runs give identical bits."""
    g = torch.Generator().manual_seed(4)
    B, H, S, D = 2, 3, 320, 64
    q, k, v, do = (torch.randn(B, H, S, D, generator=g).bfloat16().cuda() for _ in range(4))
    lse = torch.empty(B, H, S, dtype=torch.float32, device="cuda")
    o = K.sdpa_fwd(q, k, v, 0.125, True, lse=lse)
    r1 = K.sdpa_bwd(q, k, v, o, do, lse, 0.125, True)
    r2 = K.sdpa_bwd(q, k, v, o, do, lse, 0.125, True)
    for a, b in zip(r1, r2):
        assert torch.equal(a, b)


def test_sdpa_bwd_strided_head_split(K):
    """q, k, v as column slices of one [B*S, 3*H*D] projection (the GPT-2
    layout), dq/dk/dv written into the same layout."""
    g = torch.Generator().manual_seed(11)
    B, S, H, D = 2, 64, 2, 64
    qkv = (torch.randn(B, S, 3, H, D, generator=g) * 0.7).bfloat16()
    do = torch.randn(B, S, H, D, generator=g).bfloat16()
    dev = qkv.cuda()
    q, k, v = (dev[:, :, i].permute(0, 2, 1, 3) for i in range(3))
    dod = do.cuda().permute(0, 2, 1, 3)
    lse = torch.empty(B, H, S, dtype=torch.float32, device="cuda")
    o = K.sdpa_fwd(q, k, v, 0.125, True, lse=lse)
    dqkv = torch.empty_like(dev)
    dq, dk, dv = (dqkv[:, :, i].permute(0, 2, 1, 3) for i in range(3))
    K.sdpa_bwd(q, k, v, o, dod, lse, 0.125, True, dq=dq, dk=dk, dv=dv)
    qr, kr, vr = (qkv[:, :, i].permute(0, 2, 1, 3).double().requires_grad_(True) for i in range(3))
    _attn_ref(qr, kr, vr, 0.125, True).backward(do.permute(0, 2, 1, 3).double())
    for i, r in enumerate((qr, kr, vr)):
        assert _rel(dqkv[:, :, i].permute(0, 2, 1, 3), r.grad) < 2.5e-2
