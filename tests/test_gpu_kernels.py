"""Kernel parity on the MI355X: every mk_* entry point, called through the
C-ABI (ctypes), against the CPU oracle on the same seeded inputs.

Bars: integer / index / copy work bit-exact; fp32
within 1e-5 relative (stated per test in its norm-scaled form); bf16 outputs
within one bf16 ulp of the float64 oracle rounded once; attention within
2e-2 absolute (the north_star bar) and a tighter relative bound.
Full benchmark sizes are used where the oracle finishes in seconds; the
attention sweep at full size is checked on sampled rows plus closed forms.
"""

import math

import numpy as np
import pytest
import torch

from oracle import bf16, inputs, native, ops

pytestmark = pytest.mark.gpu


def dev_bf16(bits, device="cuda"):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def host_bf16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.fixture(scope="module")
def K(cuda):
    from mi355x_pjrt import kernels

    kernels.lib()  # raises if the HIP library is missing: no fallback
    return kernels


# ------------------------------------------------------------------ C2c / C2d reduce + argmax
def test_row_reduce_sum_c2_full(K):
    x = inputs.c2_reduce()["x"]
    print("case: row_reduce sum [65536,1024] bf16", flush=True)
    y = K.row_reduce(dev_bf16(x), "sum").cpu().numpy().astype(np.float64)
    ref = native.row_sum_bf16(x)
    norm = native.row_sum_bf16(bf16.to_bf16_bits(np.abs(bf16.from_bf16_bits(x))))
    # fp32 summation error is bounded relative to sum |x_i| (norm-scaled 1e-5)
    assert np.max(np.abs(y - ref) / norm) < 1e-5
    assert np.median(np.abs(y - ref) / np.maximum(np.abs(ref), 1.0)) < 1e-6


def test_row_reduce_ops_and_nan(K):
    rng = np.random.default_rng(0)
    for cols in (1, 7, 64, 1000, 1024, 4104):
        x = rng.standard_normal((37, cols)).astype(np.float32)
        x[3, cols // 2] = np.nan
        xd = torch.from_numpy(x).cuda()
        for op in ("sum", "max", "min", "prod"):
            xx = x if op != "prod" else np.clip(x, 0.9, 1.1)
            xd2 = torch.from_numpy(np.ascontiguousarray(xx)).cuda()
            got = K.row_reduce(xd2 if op == "prod" else xd, op).cpu().numpy()
            want = ops.reduce_rows(xx, op)
            np.testing.assert_allclose(got, want, rtol=2e-5, atol=1e-5, equal_nan=True, err_msg=f"{op} {cols}")
        got = K.row_reduce(xd, "sum", init=2.5).cpu().numpy()
        np.testing.assert_allclose(got, ops.reduce_rows(x, "sum", 2.5), rtol=2e-5, atol=1e-4)


@pytest.mark.parametrize("is_min", [False, True])
def test_row_argmax_c2_full_bit_exact(K, is_min):
    x = inputs.c2_reduce()["x"]
    print(f"case: argmax is_min={is_min} [65536,1024] bf16", flush=True)
    idx, vals = K.row_argmax(dev_bf16(x), is_min=is_min)
    ri, rv = native.argmax_rows_bf16(x, is_min)
    np.testing.assert_array_equal(idx.cpu().numpy(), ri)
    np.testing.assert_array_equal(host_bf16(vals), rv)


def test_row_argmax_ties_nan_dtypes(K):
    rng = np.random.default_rng(1)
    for cols in (1, 3, 8, 1024, 1030):
        x = rng.integers(-2, 3, size=(257, cols)).astype(np.float32)
        x[rng.random(x.shape) < 0.01] = np.nan
        x[0, :] = 1.0
        x[1, :] = -0.0
        x[1, cols - 1] = 0.0
        xb = bf16.to_bf16_bits(x)
        for is_min in (False, True):
            wi, _ = native.argmax_rows_bf16(xb, is_min)
            gi, _ = K.row_argmax(dev_bf16(xb), is_min=is_min)
            np.testing.assert_array_equal(gi.cpu().numpy(), wi, err_msg=f"bf16 cols={cols}")
            gi32, gv32 = K.row_argmax(torch.from_numpy(x).cuda(), is_min=is_min, index_dtype=torch.int64)
            wi32, wv32 = ops.argmax_rows(x, is_min)
            np.testing.assert_array_equal(gi32.cpu().numpy(), wi32, err_msg=f"f32 cols={cols}")
            np.testing.assert_array_equal(gv32.cpu().numpy().view(np.uint32), wv32.view(np.uint32))


def _argmax_ref_bits(bits, is_min, to_f32):
    """Reference on raw 16-bit patterns: the pairwise-reducer oracle on the
    exact fp32 values, values returned as the winner's own bits."""
    idx, _ = ops.argmax_rows(to_f32(bits), is_min)
    return idx, bits[np.arange(bits.shape[0]), idx]


@pytest.mark.parametrize("fmt", ["bf16", "f16"])
def test_row_argmax_special_bit_patterns(K, fmt):
    """16-bit keyed path: NaNs of both signs and several payloads (all beat
    every number; the first NaN wins), +-inf, +-0 ties, subnormals, lowest
    index on ties; int32 and int64 indices; values bit-exact."""
    rng = np.random.default_rng(17)
    if fmt == "bf16":
        specials = np.array([0x7F80, 0xFF80, 0x7FC0, 0xFFC0, 0x7F81, 0xFFFF, 0x0000, 0x8000, 0x0001, 0x8001,
                             0x3F80, 0xBF80], np.uint16)
        to_f32, to_t = bf16.from_bf16_bits, (lambda b: dev_bf16(b))
    else:
        specials = np.array([0x7C00, 0xFC00, 0x7E00, 0xFE00, 0x7C01, 0xFFFF, 0x0000, 0x8000, 0x0001, 0x8001,
                             0x3C00, 0xBC00], np.uint16)
        to_f32 = lambda b: b.view(np.float16).astype(np.float32)
        to_t = lambda b: torch.from_numpy(b.view(np.float16)).cuda()
    for cols in (8, 64, 1024, 4096):
        bits = rng.choice(specials, size=(300, cols)).astype(np.uint16)
        bits[0] = specials[6]                       # all +0
        bits[1] = specials[7]; bits[1, cols // 2] = specials[6]   # -0 / +0 tie -> index 0
        bits[2] = specials[0]; bits[2, 3 % cols] = specials[3]    # +inf row with one negative NaN
        finite = (to_f32(specials) == to_f32(specials))
        bits[3] = rng.choice(specials[finite], size=cols)          # no NaN at all
        for is_min in (False, True):
            want_i, want_v = _argmax_ref_bits(bits, is_min, to_f32)
            for it in (torch.int32, torch.int64):
                gi, gv = K.row_argmax(to_t(bits), is_min=is_min, index_dtype=it)
                np.testing.assert_array_equal(gi.cpu().numpy(), want_i, err_msg=f"{fmt} cols={cols} min={is_min}")
                got_v = gv.cpu().view(torch.int16).numpy().view(np.uint16)
                np.testing.assert_array_equal(got_v, want_v, err_msg=f"{fmt} values cols={cols}")


# ------------------------------------------------------------------ C2a LayerNorm / C2b GELU
def _ulp_check(got_bits, want_bits, exact_frac=0.999):
    d = bf16.bf16_ulp_distance(got_bits, want_bits)
    assert d.max() <= 1, f"max ulp distance {d.max()}"
    assert np.mean(d == 0) >= exact_frac, f"exact fraction {np.mean(d == 0)}"


def _bf16_close(got_bits, want, scale, rel=1e-5, exact_frac=0.999):
    """bf16 result vs float64 truth: |got - want| <= 1 bf16 ulp of want plus
    rel * scale, where scale is the magnitude of the fp32 terms that formed
    the value (cancellation makes tiny results legitimately inexact)."""
    got = bf16.from_bf16_bits(got_bits).astype(np.float64)
    want = np.asarray(want, dtype=np.float64)
    with np.errstate(divide="ignore"):
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-38))) - 7)
    err = np.abs(got - want)
    bad = err > ulp + rel * scale
    assert not bad.any(), f"{bad.sum()} elements out of bound; worst err {err[bad].max()}"
    exact = np.mean(got_bits == bf16.to_bf16_bits_f64(want))
    assert exact >= exact_frac, f"exact fraction {exact}"


def _ln_scale(x, g, b):
    x = np.asarray(x, np.float64)
    xh = np.abs(x - x.mean(-1, keepdims=True)) / np.sqrt(x.var(-1, keepdims=True) + 1e-5)
    return (xh + 1.0) * np.abs(np.asarray(g, np.float64)) + np.abs(np.asarray(b, np.float64))


def test_layernorm_c2_full(K):
    d = inputs.c2_layernorm()
    print("case: layernorm [8192,4096] bf16", flush=True)
    y = host_bf16(K.layernorm(dev_bf16(d["x"]), dev_bf16(d["gamma"]), dev_bf16(d["beta"]), 1e-5))
    x, g, b = (bf16.from_bf16_bits(d[n]) for n in ("x", "gamma", "beta"))
    for r0 in range(0, 8192, 2048):
        sl = slice(r0, r0 + 2048)
        _bf16_close(y[sl], ops.layernorm(x[sl], g, b, 1e-5), _ln_scale(x[sl], g, b))


@pytest.mark.parametrize("cols", [1, 100, 768, 4096, 4104, 6000, 12288, 16384, 16392])
def test_layernorm_widths_f32_bf16(K, cols):
    rng = np.random.default_rng(cols)
    x = (rng.standard_normal((19, cols)) * 3 + 1).astype(np.float32)
    g = rng.standard_normal(cols).astype(np.float32)
    b = rng.standard_normal(cols).astype(np.float32)
    got = K.layernorm(torch.from_numpy(x).cuda(), torch.from_numpy(g).cuda(), torch.from_numpy(b).cuda()).cpu().numpy()
    want = ops.layernorm(x, g, b)
    scale = np.abs(g)[None, :] * 8 + np.abs(b)[None, :]
    assert np.max(np.abs(got - want) / (scale + 1e-30)) < 1e-5
    xb = bf16.to_bf16_bits(x)
    gb, bb = bf16.to_bf16_bits(g), bf16.to_bf16_bits(b)
    got = host_bf16(K.layernorm(dev_bf16(xb), dev_bf16(gb), dev_bf16(bb)))
    xf, gf, bf_ = (bf16.from_bf16_bits(a) for a in (xb, gb, bb))
    _bf16_close(got, ops.layernorm(xf, gf, bf_), _ln_scale(xf, gf, bf_), exact_frac=0.98)


@pytest.mark.parametrize("cols,off", [(1, 0), (100, 0), (768, 0), (1000, 0), (2048, 0), (4096, 0), (768, 3)])
def test_layernorm_f32_rows_bf16_out(K, cols, off):
    """fp32 rows, bf16 result (mk_layernorm_typed): the same arithmetic as the
    fp32 kernel, so each element is the round-to-nearest-even bf16 of the fp32
    kernel's result (bit for bit), and within bf16 rounding of the oracle.
    off > 0 starts x and y off their 16-byte alignment (the streaming kernel)."""
    rng = np.random.default_rng(cols + 7 * off)
    rows = 8192 if cols == 768 and off == 0 else 23
    x = (rng.standard_normal((rows, cols)) * 3 + 1).astype(np.float32)
    g = rng.standard_normal(cols).astype(np.float32)
    b = rng.standard_normal(cols).astype(np.float32)
    print(f"case: layernorm f32 -> bf16 [{rows},{cols}] off={off}", flush=True)
    xd = torch.from_numpy(np.concatenate([np.zeros(off, np.float32), x.ravel()])).cuda()[off:].view(rows, cols)
    gd, bd = torch.from_numpy(g).cuda(), torch.from_numpy(b).cuda()
    y16 = K.layernorm(xd, gd, bd, out_dtype=torch.bfloat16)
    assert y16.dtype == torch.bfloat16 and y16.shape == (rows, cols)
    y32 = K.layernorm(xd, gd, bd).cpu().numpy()
    got = host_bf16(y16)
    if off == 0 and cols % 4 == 0 and cols <= 2048:
        np.testing.assert_array_equal(got, bf16.to_bf16_bits(y32))
    want = ops.layernorm(x, g, b)
    _bf16_close(got, want, np.abs(g)[None, :] * 8 + np.abs(b)[None, :], exact_frac=0.98)
    # the unaligned output rows take the streaming kernel
    if off:
        yb = torch.empty(rows * cols + 1, dtype=torch.bfloat16, device="cuda")[1:].view(rows, cols)
        rc = K.lib().mk_layernorm_typed(None, 11, 13, rows, cols, K._ptr(xd), K._ptr(gd), K._ptr(bd), 1e-5,
                                        K._ptr(yb))
        assert rc == 0
        np.testing.assert_array_equal(host_bf16(yb), got)


def test_layernorm_typed_rejects_bf16_to_f32(K):
    x = torch.zeros(4, 8, dtype=torch.bfloat16, device="cuda")
    y = torch.zeros(4, 8, dtype=torch.float32, device="cuda")
    rc = K.lib().mk_layernorm_typed(None, 13, 11, 4, 8, K._ptr(x), None, None, 1e-5, K._ptr(y))
    assert rc != 0


def test_gelu_c2_full(K):
    x = inputs.c2_gelu()["x"]
    print("case: gelu_tanh [8192,16384] bf16", flush=True)
    y = host_bf16(K.gelu_tanh(dev_bf16(x)))
    for r0 in range(0, x.shape[0], 1024):  # oracle in row chunks to bound host memory
        want = ops.round_to(ops.gelu_tanh(bf16.from_bf16_bits(x[r0:r0 + 1024])), "bf16")
        _ulp_check(y[r0:r0 + 1024], want)


def test_gelu_special_values_and_ragged(K):
    vals = np.array([0.0, -0.0, 1.0, -1.0, 3.0, -3.0, 10.0, -10.0, 30.0, -30.0, 1e-20, np.inf,
                     -np.inf, np.nan, 88.0, -88.0, 0.5, -0.5, 1e4], dtype=np.float32)
    got = K.gelu_tanh(torch.from_numpy(vals).cuda()).cpu().numpy()
    want = ops.gelu_tanh(vals.astype(np.float64))
    fin = np.isfinite(want)
    np.testing.assert_allclose(got[fin], want[fin], rtol=2e-6, atol=1e-30)
    assert np.isnan(got[13]) and got[11] == np.inf
    x = bf16.to_bf16_bits(np.random.default_rng(2).standard_normal(1001).astype(np.float32))
    _ulp_check(host_bf16(K.gelu_tanh(dev_bf16(x))), ops.round_to(ops.gelu_tanh(bf16.from_bf16_bits(x)), "bf16"), 0.99)


def test_softmax_rows(K):
    rng = np.random.default_rng(3)
    for cols in (5, 64, 1024, 3000):
        x = (rng.standard_normal((9, cols)) * 4).astype(np.float32)
        got = K.softmax_rows(torch.from_numpy(x).cuda()).cpu().numpy()
        np.testing.assert_allclose(got, ops.softmax_rows(x), rtol=1e-5, atol=1e-7)


# ------------------------------------------------------------------ C4 gather / scatter-add
def test_gather_c4_full_bit_exact(K):
    d = inputs.c4_indexing()
    print("case: gather ids[32,2048] table[50257,768] bf16", flush=True)
    out = host_bf16(K.gather_rows(dev_bf16(d["table_bf16"]), torch.from_numpy(d["ids"]).cuda()))
    assert out.shape == (32, 2048, 768)
    np.testing.assert_array_equal(out.reshape(-1, 768), native.gather_rows(d["table_bf16"], d["ids"]))


def test_gather_clamp_and_odd_rows(K):
    table = np.arange(7 * 6, dtype=np.float32).reshape(7, 6)  # 24-byte rows: 4-byte path
    ids = np.array([0, 6, -5, 99, 3], dtype=np.int64)
    got = K.gather_rows(torch.from_numpy(table).cuda(), torch.from_numpy(ids).cuda()).cpu().numpy()
    np.testing.assert_array_equal(got, ops.gather_rows(table, ids))


def test_scatter_add_c4_full_bit_exact(K):
    d = inputs.c4_indexing()
    ids = d["ids"].reshape(-1)
    print("case: scatter-add [65536,768] -> [50257,768] fp32", flush=True)
    table_d = torch.from_numpy(d["table_f32"]).cuda()
    out = K.scatter_add_rows(table_d, torch.from_numpy(ids).cuda(), torch.from_numpy(d["grads"]).cuda())
    want = native.scatter_add_f32(d["table_f32"], ids, d["grads"])
    np.testing.assert_array_equal(out.cpu().numpy(), want)
    # into zeros, in place
    z = torch.zeros((50257, 768), dtype=torch.float32, device="cuda")
    K.scatter_add_rows(z, torch.from_numpy(ids).cuda(), torch.from_numpy(d["grads"]).cuda(), out=z)
    want0 = native.scatter_add_f32(np.zeros((50257, 768), np.float32), ids, d["grads"])
    np.testing.assert_array_equal(z.cpu().numpy(), want0)


def test_scatter_add_edge_cases(K):
    rng = np.random.default_rng(4)
    table = rng.standard_normal((300, 12)).astype(np.float32)
    cases = {
        "oob": rng.integers(-50, 350, size=2000).astype(np.int32),
        "all_same": np.full(5000, 17, dtype=np.int32),           # one bucket of 5000
        "skewed": (rng.zipf(1.5, size=4000) % 300).astype(np.int32),
        "single": np.array([5], dtype=np.int32),
        "empty": np.zeros(0, dtype=np.int32),
    }
    for name, ids in cases.items():
        upd = (rng.standard_normal((ids.size, 12)) * 100).astype(np.float32)
        got = K.scatter_add_rows(torch.from_numpy(table).cuda(), torch.from_numpy(ids).cuda(),
                                 torch.from_numpy(upd).cuda()).cpu().numpy()
        np.testing.assert_array_equal(got, native.scatter_add_f32(table, ids, upd), err_msg=name)
    # tables on both sides of the 16-bit key limit of the three-launch sort
    # (n_rows < 65535; larger tables take the multi-pass radix sort), with
    # out-of-range ids and a hot row
    for n_rows in (65534, 65535, 70001):
        print(f"case: scatter-add rows={n_rows}", flush=True)
        tb = rng.standard_normal((n_rows, 4)).astype(np.float32)
        ids = np.concatenate([rng.integers(-10, n_rows + 10, size=20000), np.full(3000, n_rows - 1)])
        ids = rng.permutation(ids).astype(np.int32)
        upd = rng.standard_normal((ids.size, 4)).astype(np.float32)
        got = K.scatter_add_rows(torch.from_numpy(tb).cuda(), torch.from_numpy(ids).cuda(),
                                 torch.from_numpy(upd).cuda()).cpu().numpy()
        np.testing.assert_array_equal(got, native.scatter_add_f32(tb, ids, upd), err_msg=f"rows={n_rows}")
    # int64 ids, ragged row length (scalar path), bf16 rows rounded after every add
    ids = rng.integers(0, 40, size=700)
    tb = bf16.to_bf16_bits(rng.standard_normal((40, 9)).astype(np.float32))
    ub = bf16.to_bf16_bits(rng.standard_normal((700, 9)).astype(np.float32))
    got = host_bf16(K.scatter_add_rows(dev_bf16(tb), torch.from_numpy(ids).cuda(), dev_bf16(ub)))
    np.testing.assert_array_equal(got, native.scatter_add_bf16(tb, ids.astype(np.int32), ub))


def test_scatter_add_wide_rows_edge_cases(K):
    """Wide fp32 rows (256..1024 floats, the vector accumulate kernels with
    one to four float4 per lane) bit-exact against the in-order oracle:
    out-of-range ids, one hot row taking 20000 updates, Zipf-skewed ids,
    int64 ids, fewer rows than ids, a single id, no ids, and in place."""
    rng = np.random.default_rng(9)
    for n_rows, row_len, ids, idx_dtype, in_place in [
        (3001, 256, rng.integers(-100, 3100, size=9000), np.int32, False),
        (3001, 256, np.full(20000, 1234), np.int32, False),
        (3001, 512, (rng.zipf(1.3, size=30000) % 3001), np.int64, False),
        (100, 800, rng.integers(0, 100, size=5000), np.int32, True),
        (777, 1024, rng.integers(0, 777, size=1), np.int64, False),
        (777, 1024, np.zeros(0), np.int32, False),
    ]:
        print(f"case: scatter-add wide rows rows={n_rows} len={row_len} ids={ids.size} in_place={in_place}",
              flush=True)
        ids = ids.astype(idx_dtype)
        table = rng.standard_normal((n_rows, row_len)).astype(np.float32)
        upd = (rng.standard_normal((ids.size, row_len)) * 10).astype(np.float32)
        t = torch.from_numpy(table).cuda()
        got = K.scatter_add_rows(t, torch.from_numpy(ids).cuda(), torch.from_numpy(upd).cuda(),
                                 out=t if in_place else None).cpu().numpy()
        np.testing.assert_array_equal(got, native.scatter_add_f32(table, ids.astype(np.int64).clip(-2**31, 2**31 - 1)
                                                                  .astype(np.int32), upd))


# ------------------------------------------------------------------ C3 attention
def _sdpa_case(K, B, H, S, D, causal, seed, Sk=None, qk_std=1 / math.sqrt(128), k_ramp=0):
    rng = np.random.default_rng(seed)
    Sk = Sk or S
    s = 1 / math.sqrt(128)
    qq = rng.standard_normal((B, H, S, D)) * qk_std
    kk = rng.standard_normal((B, H, Sk, D)) * qk_std
    if k_ramp:  # q, k > 0 and |k_j| grows like j / k_ramp: the row max keeps rising
        qq = np.abs(qq)
        kk = np.abs(kk) * (1 + np.arange(Sk) / k_ramp)[None, None, :, None]
    q = bf16.to_bf16_bits(qq.astype(np.float32))
    k = bf16.to_bf16_bits(kk.astype(np.float32))
    v = bf16.to_bf16_bits((rng.standard_normal((B, H, Sk, D)) * s).astype(np.float32))
    scale = 1 / math.sqrt(D)
    lse = torch.empty((B, H, S), dtype=torch.float32, device="cuda")
    o = host_bf16(K.sdpa_fwd(dev_bf16(q), dev_bf16(k), dev_bf16(v), scale, causal, lse=lse))
    qf, kf, vf = (bf16.from_bf16_bits(a) for a in (q, k, v))
    want = ops.sdpa(qf, kf, vf, scale, causal)
    got = bf16.from_bf16_bits(o).astype(np.float64)
    err = np.abs(got - want)
    assert err.max() <= 2e-2, err.max()                       # north_star bar
    assert err.max() <= 2e-2 * np.abs(want).max(), (err.max(), np.abs(want).max())
    # the kernel's row sum adds the bf16-rounded probabilities (the values
    # its P.V product uses, as XLA's bf16 softmax does): bf16 keeps 8
    # significant bits, so each carries <= 2^-8 relative rounding and
    # log(sum) is within ln(1 + 2^-8) < 2^-8 of the exact lse; the fp32
    # scores add ~2e-5 relative to the lse's own magnitude
    np.testing.assert_allclose(lse.cpu().numpy(), ops.sdpa_lse(qf, kf, scale, causal), atol=2.0 ** -8, rtol=2e-5)
    return got, want


@pytest.mark.parametrize("S,D,causal", [(64, 128, True), (128, 128, True), (512, 128, True),
                                        (512, 128, False), (100, 128, True), (257, 64, True),
                                        (1024, 64, False), (33, 64, False)])
def test_sdpa_small_vs_oracle(K, S, D, causal):
    print(f"case: sdpa S={S} D={D} causal={causal}", flush=True)
    _sdpa_case(K, 2, 3, S, D, causal, seed=S + D)


def test_sdpa_cross_lengths(K):
    _sdpa_case(K, 1, 2, 96, 128, False, seed=5, Sk=300)
    _sdpa_case(K, 1, 2, 300, 64, True, seed=6, Sk=320)


@pytest.mark.parametrize("causal", [True, False])
def test_sdpa_large_scores_rescale(K, causal):
    """Scores with a wide spread (q, k ~ N(0, 1)) and scores that keep growing
    along the keys, by ~15 (k_ramp 8) and ~4 (k_ramp 32) log2 units per
    64-key tile: the running max is raised on many tiles (O and l rescaled),
    and between raises p reaches up to 2^8 against a stale max."""
    print(f"case: sdpa large scores causal={causal}", flush=True)
    _sdpa_case(K, 1, 2, 1024, 128, causal, seed=21, qk_std=1.0)
    for D in (64, 128):
        _sdpa_case(K, 1, 2, 700, D, causal, seed=22, qk_std=0.5, k_ramp=8)
        _sdpa_case(K, 1, 2, 700, D, causal, seed=23, qk_std=0.5, k_ramp=32)


@pytest.mark.parametrize("S,Sk,causal,ramp", [(300, None, True, 0), (320, 1000, False, 0), (700, None, True, 8),
                                               (700, None, False, 32), (64, None, True, 0)])
def test_sdpa_wide_kernel_d64(K, S, Sk, causal, ramp):
    """head_dim 64 with at least 512 workgroups of 256 query rows (B2 H128):
    the wide-wave kernel (64 query rows per wave, 32-key half steps).
    Ragged query and key lengths, cross lengths, the causal diagonal and
    rising scores that raise the running max on many half steps."""
    print(f"case: sdpa wide D=64 S={S} Sk={Sk} causal={causal} ramp={ramp}", flush=True)
    _sdpa_case(K, 2, 128, S, 64, causal, seed=S + (Sk or 0) + ramp, Sk=Sk,
               qk_std=0.5 if ramp else 1 / math.sqrt(128), k_ramp=ramp)


def test_sdpa_wide_kernel_d64_long_sampled_rows(K):
    """B4 H16 S8192 D64 causal (the wide kernel at a benchmark length): row 0
    equals V[0] exactly; 4 (b,h) pairs x ~40 rows against the float64 oracle."""
    B, H, S, D = 4, 16, 8192, 64
    rng = np.random.default_rng(31)
    x = [bf16.to_bf16_bits((rng.standard_normal((B, H, S, D)) / 8).astype(np.float32)) for _ in range(3)]
    print("case: sdpa wide D=64 B4 H16 S8192 causal", flush=True)
    o = host_bf16(K.sdpa_fwd(*(dev_bf16(a) for a in x), 0.125, True))
    np.testing.assert_array_equal(o[:, :, 0, :], x[2][:, :, 0, :])
    rows = np.array(sorted(set([1, 31, 32, 63, 64, 255, 256, 4095, 4096, S - 2, S - 1] +
                               list(rng.integers(0, S, 30)))))
    for b, h in [(0, 0), (1, 7), (2, 12), (3, 15)]:
        qf, kf, vf = (bf16.from_bf16_bits(a[b, h]).astype(np.float64) for a in x)
        sc = (qf[rows] @ kf.T) * 0.125
        sc[np.arange(S)[None, :] > rows[:, None]] = -np.inf
        p = np.exp(sc - sc.max(axis=1, keepdims=True))
        want = (p @ vf) / p.sum(axis=1, keepdims=True)
        got = bf16.from_bf16_bits(o[b, h, rows]).astype(np.float64)
        assert np.abs(got - want).max() <= 2e-3, (b, h, np.abs(got - want).max())


@pytest.mark.parametrize("D", [64, 128])
def test_sdpa_strided_views(K, D):
    """[B, S, H, D] storage (the layout a head split produces) passed as a
    permuted view: no copy, strides folded into addressing."""
    rng = np.random.default_rng(9)
    B, S, H = 2, 200, 4
    x = [bf16.to_bf16_bits((rng.standard_normal((B, S, H, D)) / 8).astype(np.float32)) for _ in range(3)]
    q, k, v = (dev_bf16(a).permute(0, 2, 1, 3) for a in x)
    o = host_bf16(K.sdpa_fwd(q, k, v, 0.125, True))
    want = ops.sdpa(*(bf16.from_bf16_bits(a).transpose(0, 2, 1, 3) for a in x), 0.125, True)
    assert np.abs(bf16.from_bf16_bits(o) - want).max() < 2e-3


@pytest.mark.parametrize("S", [512, 1024, 2048, 4096, 8192, 16384])
def test_sdpa_c3_full_size_sampled_rows(K, S):
    """C3 at its benchmark shape, every length of the sweep: the kernel runs
    on all [4,16,S,128].  Row 0 must equal V[0] exactly (a single visible
    key).  For S <= 2048 every row of every (b,h) is checked against the
    float64 oracle; above, 8 (b,h) pairs including the last are checked on
    ~70 rows each (each row needs only its prefix), the last row among them."""
    d = inputs.c3_sdpa(S)
    print(f"case: sdpa C3 full S={S}", flush=True)
    qd, kd, vd = dev_bf16(d["q"]), dev_bf16(d["k"]), dev_bf16(d["v"])
    scale = 1 / math.sqrt(128)
    # NaN-filled output: every query tile of every (b, h) must be written
    # (S >= 8192 runs the XCD-grouped tile order)
    out = torch.full_like(qd, float("nan"))
    o = host_bf16(K.sdpa_fwd(qd, kd, vd, scale, True, out=out))
    assert bool(torch.isfinite(out).all())
    np.testing.assert_array_equal(o[:, :, 0, :], d["v"][:, :, 0, :])
    if S <= 2048:
        pairs = [(b, h) for b in range(4) for h in range(16)]
        rows = np.arange(S)
    else:
        pairs = [(0, 0), (0, 15), (1, 3), (1, 7), (2, 9), (2, 12), (3, 0), (3, 15)]
        rng = np.random.default_rng(10 + S)
        rows = np.array(sorted(set([1, 63, 64, 127, 128, 255, 256, S // 2 - 1, S // 2, S - 2, S - 1] +
                                   list(rng.integers(0, S, 60)))))
    worst = 0.0
    for b, h in pairs:
        qf = bf16.from_bf16_bits(d["q"][b, h]).astype(np.float64)
        kf = bf16.from_bf16_bits(d["k"][b, h]).astype(np.float64)
        vf = bf16.from_bf16_bits(d["v"][b, h]).astype(np.float64)
        for r0 in range(0, len(rows), 256):
            rr = rows[r0:r0 + 256]
            kmax = int(rr.max()) + 1
            sc = (qf[rr] @ kf[:kmax].T) * scale
            sc[np.arange(kmax)[None, :] > rr[:, None]] = -np.inf
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            want = (p @ vf[:kmax]) / p.sum(axis=1, keepdims=True)
            # the kernel multiplies bf16-rounded probabilities (relative
            # error <= 2^-9 each, so the normalised weights move by <= 2^-8
            # of themselves) and rounds O to bf16 (<= 2^-9 relative)
            wabs = (p @ np.abs(vf[:kmax])) / p.sum(axis=1, keepdims=True)
            got = bf16.from_bf16_bits(o[b, h, rr]).astype(np.float64)
            e = np.abs(got - want)
            worst = max(worst, float(e.max()))
            assert e.max() <= 2e-2, (b, h, e.max())        # north_star bar
            bad = e > 2.0 ** -8 * wabs + 2.0 ** -9 * np.abs(want) + 1e-6
            assert not bad.any(), (b, h, rr[np.nonzero(bad)[0][:5]], e[bad][:5])
    print(f"case: sdpa C3 full S={S} max abs err {worst:.2e} over {len(pairs)} (b,h) x {len(rows)} rows", flush=True)


def test_sdpa_noncausal_long_grouped_order(K):
    """Non-causal B1 H16 S8192 D128: 512 workgroups of 256 rows, so the
    8-wave kernel runs its XCD-grouped tile order with ascending query
    tiles.  Every row is written (NaN-filled output) and sampled rows of
    four heads, spread over query tiles, match the float64 oracle."""
    B, H, S, D = 1, 16, 8192, 128
    rng = np.random.default_rng(77)
    x = [bf16.to_bf16_bits((rng.standard_normal((B, H, S, D)) / math.sqrt(D)).astype(np.float32)) for _ in range(3)]
    print("case: sdpa non-causal B1 H16 S8192 D128", flush=True)
    qd, kd, vd = (dev_bf16(a) for a in x)
    out = torch.full_like(qd, float("nan"))
    K.sdpa_fwd(qd, kd, vd, 1 / math.sqrt(D), False, out=out)
    assert bool(torch.isfinite(out).all())
    o = host_bf16(out)
    rows = np.array([0, 255, 256, 4095, 4096, 8191] + list(rng.integers(0, S, 26)))
    for h in (0, 5, 10, 15):
        qf, kf, vf = (bf16.from_bf16_bits(a[0, h]).astype(np.float64) for a in x)
        sc = (qf[rows] @ kf.T) / math.sqrt(D)
        p = np.exp(sc - sc.max(axis=1, keepdims=True))
        want = (p @ vf) / p.sum(axis=1, keepdims=True)
        got = bf16.from_bf16_bits(o[0, h, rows]).astype(np.float64)
        assert np.abs(got - want).max() <= 2e-2, (h, np.abs(got - want).max())


def test_sdpa_prefix_mean_closed_form(K):
    """Q = 0 makes every visible key equally likely: O[i] = mean(V[0..i])."""
    S = 4096
    v = inputs.c3_sdpa(S, batch=1, heads=2)["v"]
    vd = dev_bf16(v)
    q = torch.zeros_like(vd)
    o = bf16.from_bf16_bits(host_bf16(K.sdpa_fwd(q, vd, vd, 0.0883883, True))).astype(np.float64)
    want = np.cumsum(bf16.from_bf16_bits(v).astype(np.float64), axis=2) / np.arange(1, S + 1)[None, None, :, None]
    err = np.abs(o - want) / (np.abs(want) + 1e-3)
    assert err.max() < 1e-2


# ------------------------------------------------------------------ a4 GEMM
def test_gemm_c1_mlp_fp32(K):
    d = inputs.c1_mlp()
    print("case: C1 MLP fp32 via mk_gemm (bias, bias+relu epilogues)", flush=True)
    t = {k: torch.from_numpy(v).cuda() for k, v in d.items()}
    h = K.gemm(t["x"], t["w1"], bias=t["b1"], relu=True)
    y = K.gemm(h, t["w2"], bias=t["b2"]).cpu().numpy()
    want = ops.mlp_forward(d["x"], d["w1"], d["b1"], d["w2"], d["b2"])
    hh = np.maximum(np.abs(d["x"]).astype(np.float64) @ np.abs(d["w1"]) + np.abs(d["b1"]), 0)
    norm = hh @ np.abs(d["w2"]) + np.abs(d["b2"])
    assert np.max(np.abs(y - want) / norm) < 1e-5


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gemm_layouts_ragged(K, ta, tb, dtype):
    rng = np.random.default_rng(11)
    for (M, N, Kd) in [(100, 70, 33), (256, 384, 512), (1, 129, 8), (130, 1, 64)]:
        a = rng.standard_normal((M, Kd)).astype(np.float32)
        b = rng.standard_normal((Kd, N)).astype(np.float32)
        if dtype == torch.bfloat16:
            a, b = bf16.round_bf16(a), bf16.round_bf16(b)
        at = torch.from_numpy(np.ascontiguousarray(a.T)).cuda().to(dtype).t() if ta else torch.from_numpy(a).cuda().to(dtype)
        bt = torch.from_numpy(np.ascontiguousarray(b.T)).cuda().to(dtype).t() if tb else torch.from_numpy(b).cuda().to(dtype)
        got = K.gemm(at, bt, out_dtype=torch.float32).cpu().numpy()
        want = a.astype(np.float64) @ b
        norm = np.abs(a).astype(np.float64) @ np.abs(b)
        assert np.max(np.abs(got - want) / (norm + 1e-30)) < 1e-5, (M, N, Kd)


def test_gemm_batched_bf16_out(K):
    rng = np.random.default_rng(12)
    a = bf16.round_bf16(rng.standard_normal((3, 64, 96)).astype(np.float32))
    b = bf16.round_bf16(rng.standard_normal((3, 96, 80)).astype(np.float32))
    got = K.gemm(torch.from_numpy(a).cuda().bfloat16(), torch.from_numpy(b).cuda().bfloat16(),
                 out_dtype=torch.bfloat16)
    want = ops.round_to(np.matmul(a.astype(np.float64), b), "bf16")
    d = bf16.bf16_ulp_distance(host_bf16(got), want)
    assert d.max() <= 1


def _bf16_out_ok(got_bits, want, norm):
    """bf16 GEMM output bar: within one ulp of the float64 value rounded once,
    or, where the sum cancels to far below its terms, within the fp32
    accumulation bound (1e-5 of sum |a||b|) of the float64 value."""
    ulp = bf16.bf16_ulp_distance(got_bits, ops.round_to(want, "bf16"))
    err = np.abs(bf16.from_bf16_bits(got_bits).astype(np.float64) - want)
    return bool(np.all((ulp <= 1) | (err <= 1e-5 * norm)))


def _bf16_operand(x, transposed):
    """bf16 device view of x, stored transposed (unit stride along rows) when asked."""
    if transposed:
        return dev_bf16(bf16.to_bf16_bits(np.ascontiguousarray(x.T))).t()
    return dev_bf16(bf16.to_bf16_bits(x))


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_tiled_bf16_shapes(K, ta, tb):
    """bf16 products big enough for the 256-row tiled kernel: ragged M, N and
    K (multiples of 8, partial 64-deep k tiles), both column tile widths, and
    shapes whose strides send them to the general kernel (N = 777 with a
    row-contiguous B).  fp32 out within 1e-5 norm-scaled; bf16 out within one
    ulp of the float64 product rounded once."""
    rng = np.random.default_rng(21)
    for (M, N, Kd) in [(264, 264, 200), (520, 136, 72), (256, 1000, 64), (300, 777, 136), (769, 384, 1032)]:
        print(f"case: tiled gemm ta={ta} tb={tb} M={M} N={N} K={Kd}", flush=True)
        a = bf16.round_bf16(rng.standard_normal((M, Kd)).astype(np.float32))
        b = bf16.round_bf16(rng.standard_normal((Kd, N)).astype(np.float32))
        at, bt = _bf16_operand(a, ta), _bf16_operand(b, tb)
        want = a.astype(np.float64) @ b
        norm = np.abs(a).astype(np.float64) @ np.abs(b)
        got = K.gemm(at, bt, out_dtype=torch.float32).cpu().numpy()
        assert np.max(np.abs(got - want) / (norm + 1e-30)) < 1e-5, (M, N, Kd)
        gb = host_bf16(K.gemm(at, bt, out_dtype=torch.bfloat16))
        assert _bf16_out_ok(gb, want, norm), (M, N, Kd)


def test_gemm_tiled_epilogues_and_layouts(K):
    """Tiled kernel epilogues: bias, bias + ReLU, f16 out, C rows that are not
    16-byte multiples (element stores), batched operands with padded leading
    and batch strides, and a B shared by every batch (batch stride 0)."""
    rng = np.random.default_rng(22)
    M, N, Kd = 392, 520, 264
    a = bf16.round_bf16(rng.standard_normal((M, Kd)).astype(np.float32))
    b = bf16.round_bf16(rng.standard_normal((Kd, N)).astype(np.float32))
    bias = bf16.round_bf16(rng.standard_normal(N).astype(np.float32))
    prod = a.astype(np.float64) @ b
    norm = np.abs(a).astype(np.float64) @ np.abs(b) + np.abs(bias)
    at, bt = _bf16_operand(a, False), _bf16_operand(b, False)
    bias_d = dev_bf16(bf16.to_bf16_bits(bias))
    print("case: tiled gemm bias / relu epilogues, bf16 out", flush=True)
    for relu in (False, True):
        want = prod + bias
        if relu:
            want = np.maximum(want, 0)
        got = host_bf16(K.gemm(at, bt, out_dtype=torch.bfloat16, bias=bias_d, relu=relu))
        assert _bf16_out_ok(got, want, norm), relu
    print("case: tiled gemm f16 out, bias", flush=True)
    bias_h = torch.from_numpy(bias).cuda().half()
    gh = K.gemm(at, bt, out_dtype=torch.float16, bias=bias_h).cpu().numpy().astype(np.float64)
    want = prod + bias.astype(np.float16).astype(np.float64)
    # f16 keeps 11 bits: half an ulp is 2^-11 relative, plus the fp32 bound
    assert np.all(np.abs(gh - want) <= np.abs(want) * 2.0**-11 + 1e-5 * norm)
    print("case: tiled gemm C rows 2 bytes off 16-byte alignment (element stores)", flush=True)
    wide = torch.full((M, N + 3), -7.0, dtype=torch.bfloat16, device="cuda")
    K.gemm(at, bt, out_dtype=torch.bfloat16, out=wide[:, :N])
    wh = host_bf16(wide)
    assert _bf16_out_ok(wh[:, :N], prod, norm)
    assert np.all(bf16.from_bf16_bits(wh[:, N:]) == -7.0)  # padding untouched
    print("case: tiled gemm batched, padded strides, shared B", flush=True)
    a3 = bf16.round_bf16(rng.standard_normal((3, M, Kd)).astype(np.float32))
    buf = torch.zeros((3, M + 8, Kd + 16), dtype=torch.bfloat16, device="cuda")
    buf[:, :M, :Kd] = dev_bf16(bf16.to_bf16_bits(a3))
    got3 = K.gemm(buf[:, :M, :Kd], bt, out_dtype=torch.float32).cpu().numpy()
    want3 = np.matmul(a3.astype(np.float64), b)
    norm3 = np.matmul(np.abs(a3).astype(np.float64), np.abs(b))
    assert np.max(np.abs(got3 - want3) / (norm3 + 1e-30)) < 1e-5


def test_gemm_tiled_f32_out_unaligned_rows(K):
    """fp32 C whose rows are not 16-byte aligned (odd N, as a vocabulary
    projection has): the tile goes out through LDS, a pass of rows at a time,
    one C row segment per wave.  Shapes that select each tile size (256 x 256,
    128 x 192, 128 x 128 on 256 CUs), with an fp32 bias, written into a wider
    buffer whose padding columns must stay untouched; within 1e-5 of the
    float64 product, scaled by the product of magnitudes."""
    rng = np.random.default_rng(23)
    for (M, N, Kd) in [(3072, 4099, 64), (2048, 2051, 136), (520, 517, 72)]:
        print(f"case: tiled gemm fp32 out M={M} N={N} K={Kd}", flush=True)
        a = bf16.round_bf16(rng.standard_normal((M, Kd)).astype(np.float32))
        b = bf16.round_bf16(rng.standard_normal((Kd, N)).astype(np.float32))
        bias = bf16.round_bf16(rng.standard_normal(N).astype(np.float32))
        at, bt = _bf16_operand(a, False), _bf16_operand(b, True)
        want = a.astype(np.float64) @ b + bias
        norm = np.abs(a).astype(np.float64) @ np.abs(b) + np.abs(bias)
        wide = torch.full((M, N + 3), -7.0, dtype=torch.float32, device="cuda")
        K.gemm(at, bt, out_dtype=torch.float32, bias=torch.from_numpy(bias).cuda(), out=wide[:, :N])
        got = wide.cpu().numpy()
        assert np.max(np.abs(got[:, :N] - want) / (norm + 1e-30)) < 1e-5, (M, N, Kd)
        assert np.all(got[:, N:] == -7.0)


def _nan_padded(x, pad_cols, transposed):
    """bf16 device view of x ([rows, cols]) whose storage rows are padded with
    NaN to a multiple of 8 columns (+ pad_cols); transposed: the storage holds
    x.T padded the same way and the view is its transpose."""
    src = np.ascontiguousarray(x.T) if transposed else x
    r, c = src.shape
    cp = (c + 7) // 8 * 8 + pad_cols
    buf = torch.full((r, cp), float("nan"), dtype=torch.bfloat16, device="cuda")
    buf[:, :c] = dev_bf16(bf16.to_bf16_bits(src))
    v = buf[:, :c]
    return v.t() if transposed else v


def test_gemm_tiled_ragged_k_and_rows(K):
    """The tiled kernel on extents that are not multiples of 8, with NaN in
    every storage element past them: a k-contiguous operand whose K % 8 != 0
    (the chunk straddling K is cleared past K in LDS), an m- or n-contiguous
    operand whose M or N % 8 != 0 (the straddling chunk only reaches C rows or
    columns that are never stored), and both at once.  No NaN may leak; fp32
    out within 1e-5 of the float64 product scaled by the product of
    magnitudes, bf16 out within one ulp of it rounded once; repeat calls are
    bit-identical."""
    rng = np.random.default_rng(31)
    # (M, N, K, A stored transposed (m-contiguous), B stored transposed (k-contiguous))
    cases = [(264, 392, 203, False, True), (261, 384, 136, True, True), (264, 389, 200, False, False),
             (517, 389, 197, True, False), (300, 260, 1001, False, True), (256, 256, 67, False, True)]
    for (M, N, Kd, ta, tb) in cases:
        print(f"case: tiled gemm ragged M={M} N={N} K={Kd} ta={ta} tb={tb}", flush=True)
        a = bf16.round_bf16(rng.standard_normal((M, Kd)).astype(np.float32))
        b = bf16.round_bf16(rng.standard_normal((Kd, N)).astype(np.float32))
        at = _nan_padded(a, 8, ta)
        bt = _nan_padded(b, 8, tb)
        want = a.astype(np.float64) @ b
        norm = np.abs(a).astype(np.float64) @ np.abs(b)
        got_t = K.gemm(at, bt, out_dtype=torch.float32)
        got = got_t.cpu().numpy()
        assert np.isfinite(got).all(), (M, N, Kd)
        assert np.max(np.abs(got - want) / (norm + 1e-30)) < 1e-5, (M, N, Kd)
        assert torch.equal(got_t, K.gemm(at, bt, out_dtype=torch.float32))
        gb_t = K.gemm(at, bt, out_dtype=torch.bfloat16)
        gb = host_bf16(gb_t)
        assert _bf16_out_ok(gb, want, norm), (M, N, Kd)
        # C rows 16-byte aligned with N not a multiple of the store chunk:
        # the straddling chunk is stored column by column, the pitch's
        # padding stays untouched, the values are the dense call's
        pitch = (N + 7) // 8 * 8 + 8
        for dt, dense in ((torch.float32, got_t), (torch.bfloat16, gb_t)):
            wide = torch.full((M, pitch), -7.0, dtype=dt, device="cuda")
            K.gemm(at, bt, out_dtype=dt, out=wide[:, :N])
            assert torch.equal(wide[:, :N], dense), (M, N, Kd, dt)
            assert bool((wide[:, N:].float() == -7.0).all()), (M, N, Kd, dt)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_gemm_splitk_uneven_slices(K, out_dtype):
    """Split-K whose K the slice count does not divide (mk_gemm_splitk_typed:
    slices a multiple of 8 apart, a shorter last one, K % 8 != 0 cleared in
    the last slice), in the two vocabulary-product forms: a k-contiguous A
    with NaN past K against a row-major B (dX = dlogits W), and an
    m-contiguous A (dW = dlogitsᵀ X).  fp32 / bf16 out against the float64
    product; bit-identical on repeat and to the same call with the slices'
    results summed in order on the host."""
    rng = np.random.default_rng(32)
    for (M, N, Kd, ta, splits) in [(256, 768, 4099, False, 4), (264, 384, 1003, True, 3), (384, 256, 2050, False, 8)]:
        print(f"case: splitk uneven M={M} N={N} K={Kd} ta={ta} splits={splits} out={out_dtype}", flush=True)
        a = bf16.round_bf16(rng.standard_normal((M, Kd)).astype(np.float32))
        b = bf16.round_bf16(rng.standard_normal((Kd, N)).astype(np.float32))
        at = _nan_padded(a, 8, ta)
        bt = dev_bf16(bf16.to_bf16_bits(b))
        want = a.astype(np.float64) @ b
        norm = np.abs(a).astype(np.float64) @ np.abs(b)
        got_t = K.gemm_splitk(at, bt, splits, out_dtype=out_dtype)
        assert torch.equal(got_t, K.gemm_splitk(at, bt, splits, out_dtype=out_dtype))
        if out_dtype == torch.float32:
            got = got_t.cpu().numpy()
            assert np.isfinite(got).all()
            assert np.max(np.abs(got - want) / (norm + 1e-30)) < 2e-5, (M, N, Kd)
            # the slices' own products (fp32, tiled kernel) summed in slice order
            ks = ((Kd + splits - 1) // splits + 7) // 8 * 8
            acc = None
            for si in range(splits):
                k0, k1 = si * ks, min(Kd, (si + 1) * ks)
                part = K.gemm(at[:, k0:k1], bt[k0:k1, :], out_dtype=torch.float32)
                acc = part if acc is None else acc + part
            assert torch.equal(got_t, acc)
        else:
            gb = host_bf16(got_t)
            assert _bf16_out_ok(gb, want, norm), (M, N, Kd)


@pytest.mark.parametrize("relu", [False, True])
def test_gemm_fp32_bias_bf16_out(K, relu):
    """Epilogue 5 / 6: an fp32 bias (+ ReLU) added to the fp32 accumulator and
    rounded once to bf16 -- bit for bit the fp32-output product with the same
    bias, rounded to bf16 afterwards (the module's f32 add then convert), on
    the tiled kernel, the general kernel and the split-K sum."""
    rng = np.random.default_rng(55 + relu)
    for (M, N, Kd, splits) in [(512, 2304, 768, 1), (40, 72, 96, 1), (256, 768, 2048, 4)]:
        print(f"case: fp32 bias bf16 out M={M} N={N} K={Kd} splits={splits} relu={relu}", flush=True)
        a = dev_bf16(bf16.to_bf16_bits(rng.standard_normal((M, Kd)).astype(np.float32)))
        b = dev_bf16(bf16.to_bf16_bits(rng.standard_normal((Kd, N)).astype(np.float32)))
        bias = torch.from_numpy(rng.standard_normal(N).astype(np.float32) * 3).cuda()
        if splits == 1:
            ref = K.gemm(a, b, out_dtype=torch.float32, bias=bias, relu=relu)
            got = K.gemm(a, b, out_dtype=torch.bfloat16, bias=bias, relu=relu)
        else:
            ref = K.gemm_splitk(a, b, splits, out_dtype=torch.float32, bias=bias, relu=relu)
            got = K.gemm_splitk(a, b, splits, out_dtype=torch.bfloat16, bias=bias, relu=relu)
        assert got.dtype == torch.bfloat16
        assert torch.equal(got, ref.bfloat16()), (M, N, Kd, splits)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_gemm_bias_gelu(K, out_dtype):
    """mk_gemm_bias_gelu: C is mk_gemm's product + bias bit for bit, and Y is
    mk_gelu_tanh of C as stored, rounded to bf16 (bit for bit), including the
    chunk that straddles N (N = 1004 in rows padded to 1008)."""
    rng = np.random.default_rng(77)
    for (M, N, Kd, pitch) in [(8192, 3072, 768, 3072), (512, 1000, 256, 1000), (384, 1004, 192, 1008)]:
        print(f"case: gemm_bias_gelu M={M} N={N} K={Kd} pitch={pitch} out={out_dtype}", flush=True)
        a = dev_bf16(bf16.to_bf16_bits(rng.standard_normal((M, Kd)).astype(np.float32)))
        # B's rows padded like C's (the tiled kernel's 16-byte aligned rows)
        b = dev_bf16(bf16.to_bf16_bits((rng.standard_normal((Kd, pitch)) * 0.05).astype(np.float32)))[:, :N]
        bias = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).cuda().to(out_dtype)
        c = torch.full((M, pitch), float("nan"), dtype=out_dtype, device="cuda")
        y = torch.full((M, pitch), float("nan"), dtype=torch.bfloat16, device="cuda")
        K.gemm_bias_gelu(a, b, bias, out=c[:, :N], y=y[:, :N])
        want_c = K.gemm(a, b, out_dtype=out_dtype, bias=bias)
        assert torch.equal(c[:, :N], want_c)
        want_y = K.gelu_tanh(want_c.contiguous())
        assert torch.equal(y[:, :N], want_y.bfloat16())
        if pitch > N:  # the padding columns stay untouched
            assert torch.isnan(c[:, N:].float()).all() and torch.isnan(y[:, N:].float()).all()


def test_gemm_gelu_bwd(K):
    """mk_gemm_gelu_bwd: dx is mk_gelu_tanh_bwd(pre, mk_gemm's bf16 product)
    bit for bit, including the chunk that straddles N (rows padded to 1008)
    and the rows past the last whole tile; the column sums equal the float64
    sums of the stored dx to fp32 rounding, bit for bit on repeat."""
    rng = np.random.default_rng(78)
    for (M, N, Kd, pitch, tb) in [(8192, 3072, 768, 3072, True), (300, 1000, 256, 1000, False),
                                  (384, 1004, 192, 1008, True)]:
        print(f"case: gemm_gelu_bwd M={M} N={N} K={Kd} pitch={pitch} b_kc={tb}", flush=True)
        a = dev_bf16(bf16.to_bf16_bits(rng.standard_normal((M, Kd)).astype(np.float32)))
        if tb:  # B read k-contiguous (the transposed weight of the step)
            b = dev_bf16(bf16.to_bf16_bits((rng.standard_normal((pitch, Kd)) * 0.05).astype(np.float32)))[:N].t()
        else:
            b = dev_bf16(bf16.to_bf16_bits((rng.standard_normal((Kd, pitch)) * 0.05).astype(np.float32)))[:, :N]
        pre = dev_bf16(bf16.to_bf16_bits((rng.standard_normal((M, pitch)) * 2).astype(np.float32)))[:, :N]
        dx = torch.full((M, pitch), float("nan"), dtype=torch.bfloat16, device="cuda")
        got, cs = K.gemm_gelu_bwd(a, b, pre, out=dx[:, :N])
        dy = K.gemm(a, b, out_dtype=torch.bfloat16)
        want = K.gelu_tanh_bwd(pre.contiguous(), dy.contiguous())
        assert torch.equal(dx[:, :N], want)
        if pitch > N:
            assert torch.isnan(dx[:, N:].float()).all()
        ref = dx[:, :N].double().sum(0)
        scale = dx[:, :N].double().abs().sum(0)
        assert float(((cs.double() - ref).abs() / (scale + 1e-30)).max()) < 1e-5
        _, cs2 = K.gemm_gelu_bwd(a, b, pre, out=dx[:, :N])
        assert torch.equal(cs, cs2)


def test_gemm_bias_gelu_needs_the_tiled_kernel(K):
    a = torch.zeros(64, 64, dtype=torch.bfloat16, device="cuda")
    b = torch.zeros(64, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(Exception, match="mk_gemm_bias_gelu"):
        K.gemm_bias_gelu(a, b)


# ------------------------------------------------------------------ a6 iota, a12 layout, misc
def test_iota_convert_fill_copy(K):
    it = K.iota((3, 5, 7), 1).cpu().numpy()
    np.testing.assert_array_equal(it, ops.iota((3, 5, 7), 1))
    itf = K.iota((4, 9), 1, dtype=torch.float32).cpu().numpy()
    np.testing.assert_array_equal(itf, ops.iota((4, 9), 1, np.float32))
    x = np.random.default_rng(13).standard_normal(1000).astype(np.float32) * 100
    got = host_bf16(K.convert(torch.from_numpy(x).cuda(), torch.bfloat16))
    np.testing.assert_array_equal(got, bf16.to_bf16_bits(x))
    gi = K.convert(torch.from_numpy(x).cuda(), torch.int32).cpu().numpy()
    np.testing.assert_array_equal(gi, x.astype(np.int32))
    f = K.fill(torch.empty(1001, dtype=torch.int32, device="cuda"), 0xDEADBEEF).cpu().numpy()
    assert np.all(f.view(np.uint32) == 0xDEADBEEF)
    a = torch.arange(2 * 3 * 4, dtype=torch.float32, device="cuda").reshape(2, 3, 4)
    np.testing.assert_array_equal(K.copy_strided(a.permute(2, 0, 1)).cpu().numpy(),
                                  np.arange(24, dtype=np.float32).reshape(2, 3, 4).transpose(2, 0, 1))
    col = torch.arange(5, dtype=torch.float32, device="cuda").reshape(5, 1)
    np.testing.assert_array_equal(K.copy_strided(col.expand(5, 3)).cpu().numpy(),
                                  np.broadcast_to(np.arange(5, dtype=np.float32).reshape(5, 1), (5, 3)))


def test_ew_program_ragged_rows(K):
    """Rows whose length is not a multiple of 4 (a 50257-wide vocabulary):
    groups of 4 along a row with a partial last group, no 4-wide access; a
    transposed input, a broadcast column, bf16 output, and a rank-1 tensor
    (which passes the alignment test with no outer stride to reject it)."""
    E = K.EW
    rng = np.random.default_rng(15)
    for rows, cols in ((9, 257), (3, 50257), (1, 7), (5, 1)):
        print(f"case: ew ragged {rows}x{cols}", flush=True)
        x = rng.standard_normal((cols, rows)).astype(np.float32)  # read transposed
        c = rng.standard_normal((rows, 1)).astype(np.float32)
        xd = torch.from_numpy(x).cuda().t()
        cd = torch.from_numpy(c).cuda()
        prog = [(E["SUB"], 2, 0, 1), (E["MUL"], 3, 2, 2)]  # (x - c)^2: IEEE ops, one bf16 rounding
        got = host_bf16(K.ew_program((rows, cols), [xd, cd], prog, [], 3, torch.bfloat16))
        d = (x.T - c).astype(np.float32)
        want = bf16.to_bf16_bits((d * d).astype(np.float32))
        np.testing.assert_array_equal(got, want)
    for n in (1001, 3, 4096 + 2):
        print(f"case: ew ragged rank-1 n={n}", flush=True)
        a = rng.standard_normal(n).astype(np.float32)
        guard = torch.full((n + 64,), 7.0, device="cuda")
        out = guard[:n]
        got = K.ew_program((n,), [torch.from_numpy(a).cuda()], [(E["ADD"], 1, 0, 0)], [], 1, torch.float32,
                           out=out)
        np.testing.assert_array_equal(got.cpu().numpy(), a + a)
        assert torch.all(guard[n:] == 7.0).item()


def test_ew_program_vec_kernel_matches_one_element_kernel(K):
    """The 4-lane interpreter (innermost dim a multiple of 4) and the
    one-element interpreter (innermost dim 3) run the same program on the
    same elements: the outputs must agree bit for bit.  The programs touch
    the transcendental, division, compare/select/clamp, integer and rounding
    opcodes, with values that include 0, negatives, NaN and infinities; the
    first names registers up to 20 (the 32-register form of the 4-lane
    kernel), the second stays below 16 (the 16-register form)."""
    E = K.EW
    rng = np.random.default_rng(16)
    n = 4 * 3 * 1000
    x = rng.standard_normal(n).astype(np.float32) * 3
    y = rng.standard_normal(n).astype(np.float32)
    x[:8] = [0.0, -0.0, np.nan, np.inf, -np.inf, 1e-40, -1e30, 88.5]
    y[:8] = [0.0, 2.0, 1.0, -np.inf, np.nan, -1e-40, 0.5, -3.0]
    i = rng.integers(-1000, 1000, n).astype(np.int32)
    prog = [
        (E["EXP"], 3, 0, 0), (E["LOG"], 4, 3, 0), (E["TANH"], 5, 1, 0), (E["DIV"], 6, 0, 1),
        (E["POW"], 7, 3, 1), (E["ERF"], 8, 0, 0), (E["LOGISTIC"], 9, 1, 0), (E["RSQRT"], 10, 3, 0),
        (E["CMP_GT"], 11, 0, 1), (E["SELECT"], 12, 11, 5 | (6 << 16)), (E["CLAMP"], 13, 8, 9 | (5 << 16)),
        (E["ROUND_BF16"], 14, 7, 0), (E["ADD"], 15, 12, 13), (E["MUL"], 15, 15, 14), (E["SUB"], 15, 15, 10),
        (E["MAX"], 15, 15, 4), (E["MUL_S32"], 16, 2, 2), (E["ADD_S32"], 16, 16, 2), (E["S32_TO_F32"], 17, 16, 0),
        (E["FLOOR"], 18, 6, 0), (E["SIGN"], 19, 1, 0), (E["CONST"], 20, 0, 0), (E["MUL"], 18, 18, 20),
        (E["ADD"], 15, 15, 17), (E["ADD"], 15, 15, 18), (E["ADD"], 15, 15, 19),
    ]
    prog16 = [
        (E["EXP"], 3, 0, 0), (E["LOG"], 4, 3, 0), (E["TANH"], 5, 1, 0), (E["DIV"], 6, 0, 1),
        (E["POW"], 7, 3, 1), (E["ERF"], 8, 0, 0), (E["CMP_GT"], 9, 0, 1), (E["SELECT"], 10, 9, 5 | (6 << 16)),
        (E["CLAMP"], 11, 8, 7 | (5 << 16)), (E["ADD"], 12, 10, 11), (E["MUL_S32"], 13, 2, 2),
        (E["S32_TO_F32"], 14, 13, 0), (E["ADD"], 15, 12, 14), (E["MAX"], 15, 15, 4),
    ]
    xs, ys, is_ = (torch.from_numpy(a).cuda() for a in (x, y, i))
    for name, pr, cst in (("32-register", prog, [1e-3]), ("16-register", prog16, [])):
        outs = []
        for shape in ((n // 12, 12), (n // 3, 3)):
            print(f"case: ew vec vs one-element, {name} program, shape {shape}", flush=True)
            ins = [t.reshape(shape) for t in (xs, ys, is_)]
            outs.append(K.ew_program(shape, ins, pr, cst, 15, torch.float32).reshape(-1).cpu().numpy())
        np.testing.assert_array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
        assert np.isfinite(outs[0]).sum() > n // 2


@pytest.mark.parametrize("shape", [(512, 768), (37, 3)])
def test_ew_program_multi_outputs(K, shape):
    """Three outputs of one program (an Adam-shaped update: m' = b1 m +
    (1-b1) g, v' = b2 v + (1-b2) g g, p' = p - lr m' / (sqrt(v') + eps),
    lr a broadcast scalar) equal the three single-output programs bit for
    bit, also written in place over p, m and v (f32) and with p' in bf16;
    shapes for the 4-lane and one-element kernels."""
    E = K.EW
    rng = np.random.default_rng(21)
    p, g, m, v = (rng.standard_normal(shape).astype(np.float32) for _ in range(4))
    v = np.abs(v)
    lr = np.array([1e-3], np.float32)
    cst = [0.9, 0.1, 0.999, 0.001, 1e-8]
    # registers: 0 p, 1 g, 2 m, 3 v, 4 lr
    prog = [(E["CONST"], 5, 0, 0), (E["MUL"], 5, 5, 2), (E["CONST"], 6, 1, 0), (E["MUL"], 6, 6, 1),
            (E["ADD"], 7, 5, 6),                                   # m'
            (E["CONST"], 5, 2, 0), (E["MUL"], 5, 5, 3), (E["MUL"], 6, 1, 1), (E["CONST"], 8, 3, 0),
            (E["MUL"], 6, 6, 8), (E["ADD"], 9, 5, 6),              # v'
            (E["SQRT"], 10, 9, 0), (E["CONST"], 11, 4, 0), (E["ADD"], 10, 10, 11), (E["MUL"], 12, 4, 7),
            (E["DIV"], 12, 12, 10), (E["SUB"], 13, 0, 12)]         # p'
    ins = [torch.from_numpy(a).cuda() for a in (p, g, m, v)] + [torch.from_numpy(lr).cuda().reshape((1,) * len(shape))]
    print(f"case: ew multi-output {shape}", flush=True)
    singles = [K.ew_program(shape, ins, prog, cst, r, torch.float32).cpu().numpy() for r in (13, 7, 9)]
    outs = [torch.empty(shape, device="cuda") for _ in range(3)]
    K.ew_program_multi(shape, ins, prog, cst, [13, 7, 9], outs)
    for a, b in zip(outs, singles):
        np.testing.assert_array_equal(a.cpu().numpy().view(np.uint32), b.view(np.uint32))
    # in place: p', m', v' over p, m, v
    pd, md, vd = ins[0].clone(), ins[2].clone(), ins[3].clone()
    K.ew_program_multi(shape, [pd, ins[1], md, vd, ins[4]], prog, cst, [13, 7, 9], [pd, md, vd])
    for a, b in zip((pd, md, vd), singles):
        np.testing.assert_array_equal(a.cpu().numpy().view(np.uint32), b.view(np.uint32))
    # mixed output types
    pb = torch.empty(shape, dtype=torch.bfloat16, device="cuda")
    mo = torch.empty(shape, device="cuda")
    K.ew_program_multi(shape, ins, prog, cst, [13, 7], [pb, mo])
    np.testing.assert_array_equal(host_bf16(pb), bf16.to_bf16_bits(singles[0]))
    np.testing.assert_array_equal(mo.cpu().numpy().view(np.uint32), singles[1].view(np.uint32))


def test_ew_program_fused_chain(K):
    """relu(x * w + b) with a broadcast row vector, plus a select/compare chain."""
    E = K.EW
    rng = np.random.default_rng(14)
    x = rng.standard_normal((33, 70)).astype(np.float32)
    w = rng.standard_normal((70,)).astype(np.float32)
    b = rng.standard_normal((33, 1)).astype(np.float32)
    xd, wd, bd = (torch.from_numpy(a).cuda() for a in (x, w, b))
    prog = [(E["MUL"], 3, 0, 1), (E["ADD"], 3, 3, 2), (E["CONST"], 4, 0, 0), (E["MAX"], 5, 3, 4)]
    got = K.ew_program((33, 70), [xd, wd, bd], prog, [0.0], 5, torch.float32).cpu().numpy()
    np.testing.assert_allclose(got, np.maximum(x * w + b, 0), rtol=1e-6, atol=1e-6)
    # where(x > 0, x, -inf) in bf16 out
    prog = [(E["CONST"], 1, 0, 0), (E["CMP_GT"], 2, 0, 1), (E["CONST"], 3, 1, 0),
            (E["SELECT"], 4, 2, 0 | (3 << 16))]
    got = host_bf16(K.ew_program((33, 70), [xd], prog, [0.0, -np.inf], 4, torch.bfloat16))
    np.testing.assert_array_equal(got, bf16.to_bf16_bits(np.where(x > 0, x, -np.inf).astype(np.float32)))
