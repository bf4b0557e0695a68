"""Pins for the CPU oracle (runs without a GPU).

The reference ships no golden vectors or known-answer tests for this path
(its only KATs are the out-of-scope collective smokes), so each oracle
function is pinned here by what the mathematics fixes: closed forms,
invariants, special cases that reduce to an independent library routine
(torch's CPU float64 kernels, math.fsum), and brute force on tiny inputs.
Each check is chosen so that a plausible slip in the oracle (a dropped term,
a wrong sign or index, a transposed operand, a wrong tie rule) fails it.
"""

import math
import struct

import numpy as np
import pytest
import torch

from oracle import bf16, inputs, native, ops


# ------------------------------------------------------------------ bf16 rounding
def _nearest_bf16_bruteforce(f: float) -> int:
    """Nearest bf16 by comparing the two truncation neighbours in float64,
    ties to the even mantissa — a definition, not the bit trick."""
    u = struct.unpack("<I", struct.pack("<f", f))[0]
    lo = u >> 16
    hi = lo + 1
    fl = struct.unpack("<f", struct.pack("<I", lo << 16))[0]
    fh = struct.unpack("<f", struct.pack("<I", (hi & 0xFFFF) << 16))[0] if (hi & 0x7F80) != 0x7F80 or (lo & 0x7F80) == 0x7F00 else math.copysign(math.inf, f)
    dl, dh = abs(f - fl), abs(fh - f)
    if dl < dh:
        return lo
    if dh < dl:
        return hi & 0xFFFF
    return lo if lo % 2 == 0 else hi & 0xFFFF


def test_bf16_known_values():
    vals = np.array([0.0, -0.0, 1.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, 1.0 + 2**-7, -2.5,
                     3.140625, 65504.0, np.inf, -np.inf], dtype=np.float32)
    # hand-derived: 1+2^-8 is a tie -> even (0x3F80); 1+3*2^-8 is a tie -> even (0x3F82)
    want = [0x0000, 0x8000, 0x3F80, 0x3F80, 0x3F82, 0x3F81, 0xC020, 0x4049, 0x4780,
            0x7F80, 0xFF80]
    assert list(bf16.to_bf16_bits(vals)) == want


def test_bf16_rne_matches_bruteforce_nearest():
    rng = np.random.default_rng(7)
    f = rng.standard_normal(4000).astype(np.float32) * np.float32(1e3)
    # add exact halfway cases: low 16 bits == 0x8000
    u = rng.integers(0x00800000, 0x7F000000, size=500, dtype=np.uint32)
    ties = ((u & 0xFFFF0000) | 0x8000).view(np.float32)
    f = np.concatenate([f, ties, -ties])
    got = bf16.to_bf16_bits(f)
    want = np.array([_nearest_bf16_bruteforce(float(x)) for x in f], dtype=np.uint16)
    np.testing.assert_array_equal(got, want)


def test_bf16_roundtrip_all_patterns_and_nan():
    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = bf16.from_bf16_bits(allbits)
    back = bf16.to_bf16_bits(f)
    finite = ~np.isnan(f)
    np.testing.assert_array_equal(back[finite], allbits[finite])
    # NaNs stay NaN (quiet bit set), never become Inf as structural.mm:33-38 would
    assert np.all(np.isnan(bf16.from_bf16_bits(back[~finite])))
    assert bf16.to_bf16_bits(np.array([struct.unpack('<f', struct.pack('<I', 0x7F800001))[0]],
                                      dtype=np.float32))[0] != 0x7F80


def test_bf16_single_rounding_from_f64():
    # x just above a bf16 tie that float32 rounding lands exactly on
    base = 1.0 + 2**-8                      # exact tie between 0x3F80 and 0x3F81
    x = np.array([base + 2**-40, base - 2**-40, -(base + 2**-40)])
    got = bf16.to_bf16_bits_f64(x)
    assert list(got) == [0x3F81, 0x3F80, 0xBF81]
    rng = np.random.default_rng(3)
    y = rng.standard_normal(2000)
    # away from ties the single- and double-rounded results coincide
    assert np.mean(bf16.to_bf16_bits_f64(y) == bf16.to_bf16_bits(y.astype(np.float32))) > 0.999


# ------------------------------------------------------------------ dot_general
def test_dot_general_bruteforce_tiny():
    rng = np.random.default_rng(0)
    a = rng.standard_normal((3, 7))
    b = rng.standard_normal((7, 5))
    got = ops.dot_general(a, b, lhs_contract=[1], rhs_contract=[0])
    want = [[sum(a[i, k] * b[k, j] for k in range(7)) for j in range(5)] for i in range(3)]
    np.testing.assert_allclose(got, want, rtol=1e-13, atol=1e-13)


def test_dot_general_dimension_numbers():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((2, 3, 5, 4))   # [B,H,S,D]
    k = rng.standard_normal((2, 3, 6, 4))
    s = ops.dot_general(q, k, lhs_batch=[0, 1], rhs_batch=[0, 1], lhs_contract=[3], rhs_contract=[3])
    assert s.shape == (2, 3, 5, 6)
    np.testing.assert_allclose(s, np.einsum("bhqd,bhkd->bhqk", q, k), rtol=1e-12)
    # contraction over lhs dim 0 (transposed operand)
    a = rng.standard_normal((4, 3))
    b = rng.standard_normal((4, 2))
    np.testing.assert_allclose(ops.dot_general(a, b, lhs_contract=[0], rhs_contract=[0]), a.T @ b)


def test_dot_general_identity_and_zero_rows_exact():
    rng = np.random.default_rng(2)
    a = rng.standard_normal((8, 8)).astype(np.float32)
    np.testing.assert_array_equal(ops.dot_general(a, np.eye(8), lhs_contract=[1], rhs_contract=[0]), a)
    z = a.copy()
    z[3] = 0
    assert np.all(ops.dot_general(z, a, lhs_contract=[1], rhs_contract=[0])[3] == 0)


def test_mlp_forward_matches_torch_f64():
    rng = np.random.default_rng(4)
    x, w1, b1 = rng.standard_normal((5, 6)), rng.standard_normal((6, 7)), rng.standard_normal(7)
    w2, b2 = rng.standard_normal((7, 3)), rng.standard_normal(3)
    t = lambda a: torch.from_numpy(a)
    want = torch.relu(t(x) @ t(w1) + t(b1)) @ t(w2) + t(b2)
    np.testing.assert_allclose(ops.mlp_forward(x, w1, b1, w2, b2), want.numpy(), rtol=1e-12)


# ------------------------------------------------------------------ attention
def _sdpa_loops(q, k, v, scale, causal):
    S, D = q.shape
    out = np.zeros_like(q)
    for i in range(S):
        keys = range(i + 1) if causal else range(k.shape[0])
        s = [scale * sum(q[i, d] * k[j, d] for d in range(D)) for j in keys]
        m = max(s)
        e = [math.exp(x - m) for x in s]
        z = sum(e)
        for d in range(D):
            out[i, d] = sum(e[t] * v[j, d] for t, j in enumerate(keys)) / z
    return out


@pytest.mark.parametrize("causal", [True, False])
def test_sdpa_bruteforce_tiny(causal):
    rng = np.random.default_rng(5)
    q, k, v = (rng.standard_normal((6, 4)) for _ in range(3))
    np.testing.assert_allclose(ops.sdpa(q, k, v, 0.5, causal), _sdpa_loops(q, k, v, 0.5, causal),
                               rtol=1e-12, atol=1e-12)


def test_sdpa_closed_forms():
    rng = np.random.default_rng(6)
    B, H, S, D = 2, 3, 33, 8
    q, k, v = (rng.standard_normal((B, H, S, D)) for _ in range(3))
    o = ops.sdpa(q, k, v, 0.3, causal=True)
    # row 0 sees only key 0
    np.testing.assert_array_equal(o[:, :, 0, :], v[:, :, 0, :])
    # Q = 0 -> uniform weights over the visible prefix -> prefix mean of V
    o0 = ops.sdpa(np.zeros_like(q), k, v, 0.3, causal=True)
    prefix_mean = np.cumsum(v, axis=2) / np.arange(1, S + 1)[None, None, :, None]
    np.testing.assert_allclose(o0, prefix_mean, rtol=1e-12, atol=1e-12)
    # the last row sees every key: equals non-causal attention for that query
    full = ops.sdpa(q, k, v, 0.3, causal=False)
    np.testing.assert_allclose(o[:, :, -1], full[:, :, -1], rtol=1e-12)
    # heads are independent: permuting heads permutes outputs
    perm = [2, 0, 1]
    np.testing.assert_allclose(ops.sdpa(q[:, perm], k[:, perm], v[:, perm], 0.3), o[:, perm])


def test_sdpa_matches_torch_f64():
    rng = np.random.default_rng(8)
    q, k, v = (rng.standard_normal((1, 2, 17, 8)) for _ in range(3))
    t = [torch.from_numpy(a) for a in (q, k, v)]
    want = torch.nn.functional.scaled_dot_product_attention(*t, is_causal=True, scale=0.25)
    np.testing.assert_allclose(ops.sdpa(q, k, v, 0.25, causal=True), want.numpy(), rtol=1e-10)
    lse = ops.sdpa_lse(q, k, 0.25)
    s = np.einsum("bhqd,bhkd->bhqk", q, k) * 0.25
    s = np.where(np.tril(np.ones((17, 17), bool)), s, -np.inf)
    np.testing.assert_allclose(lse, np.log(np.sum(np.exp(s), axis=-1)), rtol=1e-12)


# ------------------------------------------------------------------ GELU / LayerNorm / softmax
def test_gelu_tanh_identities_and_torch():
    x = np.linspace(-12, 12, 4001)
    g = ops.gelu_tanh(x)
    # gelu(x) - gelu(-x) = x exactly in real arithmetic (tanh is odd)
    np.testing.assert_allclose(g - ops.gelu_tanh(-x), x, rtol=0, atol=1e-12)
    assert ops.gelu_tanh(np.array([0.0]))[0] == 0.0
    np.testing.assert_allclose(ops.gelu_tanh(np.array([30.0])), [30.0])
    assert abs(ops.gelu_tanh(np.array([-30.0]))[0]) < 1e-30
    # slope 1/2 at 0
    h = 1e-6
    assert abs((ops.gelu_tanh(np.array([h]))[0] - ops.gelu_tanh(np.array([-h]))[0]) / (2 * h) - 0.5) < 1e-9
    want = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    np.testing.assert_allclose(g, want, rtol=1e-12, atol=1e-15)
    # and it stays within 5e-4 of the exact erf GELU
    exact = 0.5 * x * (1 + np.vectorize(math.erf)(x / math.sqrt(2)))
    assert np.max(np.abs(g - exact)) < 5e-4


def test_layernorm_invariants_and_torch():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((7, 64))
    gm, bt = rng.standard_normal(64), rng.standard_normal(64)
    y = ops.layernorm(x, gm, bt, 1e-5)
    want = torch.nn.functional.layer_norm(torch.from_numpy(x), (64,), torch.from_numpy(gm),
                                          torch.from_numpy(bt), 1e-5).numpy()
    np.testing.assert_allclose(y, want, rtol=1e-10, atol=1e-12)
    # constant row -> beta exactly
    c = np.full((2, 64), 3.25)
    np.testing.assert_array_equal(ops.layernorm(c, gm, bt), np.broadcast_to(bt, (2, 64)))
    # shift invariance
    np.testing.assert_allclose(ops.layernorm(x + 100.0, gm, bt), y, atol=1e-9)
    # gamma = 1, beta = 0: zero mean, variance var/(var+eps)
    z = ops.layernorm(x, None, None, 0.0)
    np.testing.assert_allclose(z.mean(-1), 0, atol=1e-12)
    np.testing.assert_allclose(z.var(-1), 1, atol=1e-12)


def test_softmax_rows():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((5, 9))
    p = ops.softmax_rows(x)
    np.testing.assert_allclose(p.sum(-1), 1, atol=1e-15)
    np.testing.assert_allclose(ops.softmax_rows(x + 7.0), p, atol=1e-15)
    np.testing.assert_allclose(p, torch.softmax(torch.from_numpy(x), -1).numpy(), rtol=1e-12)


# ------------------------------------------------------------------ reduce / argmax
def test_reduce_rows_exact_cases():
    ones = np.ones((3, 1024), dtype=np.float32)
    assert list(ops.reduce_rows(ones, "sum")) == [1024.0] * 3
    rng = np.random.default_rng(11)
    x = rng.standard_normal((4, 513))
    np.testing.assert_allclose(ops.reduce_rows(x, "sum"), [math.fsum(r) for r in x], rtol=1e-13)
    y = x.copy()
    y[1, 7] = np.nan
    assert np.isnan(ops.reduce_rows(y, "max")[1]) and np.isnan(ops.reduce_rows(y, "min")[1])
    assert ops.reduce_rows(x, "max")[0] == max(x[0]) and ops.reduce_rows(x, "prod", 2.0)[2] == 2.0 * np.prod(x[2])


@pytest.mark.parametrize("is_min", [False, True])
def test_argmax_matches_pairwise_reducer(is_min):
    rng = np.random.default_rng(12)
    # few distinct values -> many ties; sprinkle NaNs and signed zeros
    x = rng.integers(-3, 4, size=(300, 37)).astype(np.float32)
    x[rng.random(x.shape) < 0.02] = np.nan
    x[5, :] = 0.0
    x[5, 3] = -0.0
    x[6, :] = 2.0                                  # all equal -> index 0
    got_i, got_v = ops.argmax_rows(x, is_min)
    for r in range(x.shape[0]):
        wi, wv = ops.argmax_reducer_pairwise(x[r], is_min)
        assert got_i[r] == wi, (r, x[r])
        assert (math.isnan(wv) and math.isnan(got_v[r])) or got_v[r] == wv
    assert got_i[6] == 0


def test_native_oracle_matches_numpy_oracle():
    rng = np.random.default_rng(13)
    xb = bf16.to_bf16_bits(rng.standard_normal((200, 1024)).astype(np.float32))
    xb[3, 100] = 0x7FC0          # NaN
    xb[4, :] = xb[4, 0]          # all equal
    for is_min in (False, True):
        i1, v1 = native.argmax_rows_bf16(xb, is_min)
        i2, _ = ops.argmax_rows(bf16.from_bf16_bits(xb), is_min)
        np.testing.assert_array_equal(i1, i2)
        np.testing.assert_array_equal(v1, xb[np.arange(200), i1])
    np.testing.assert_array_equal(native.row_sum_bf16(xb[:10]),
                                  [math.fsum(r) for r in bf16.from_bf16_bits(xb[:10]).astype(np.float64)])


# ------------------------------------------------------------------ gather / scatter / iota
def test_gather_rows_clamp():
    table = np.arange(20, dtype=np.float32).reshape(5, 4)
    ids = np.array([0, 4, -3, 9, 2], dtype=np.int32)
    want = np.stack([table[min(max(i, 0), 4)] for i in ids])
    np.testing.assert_array_equal(ops.gather_rows(table, ids), want)
    np.testing.assert_array_equal(native.gather_rows(table, ids), want)


def test_scatter_add_sequential_forms():
    rng = np.random.default_rng(14)
    table = rng.standard_normal((9, 5)).astype(np.float32)
    ids = rng.integers(-2, 11, size=40).astype(np.int32)
    upd = (rng.standard_normal((40, 5)) * 1e3).astype(np.float32)
    a = ops.scatter_add_rows_f32(table, ids, upd)
    b = ops.scatter_add_rows_loop(table, ids, upd)
    c = native.scatter_add_f32(table, ids, upd)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(a, c)
    # unique in-range ids -> a plain elementwise add
    uid = np.array([3, 0, 7], dtype=np.int32)
    np.testing.assert_array_equal(ops.scatter_add_rows_f32(table, uid, upd[:3])[uid], table[uid] + upd[:3])
    # all updates to one row -> the sequential fp32 prefix sum
    same = np.full(40, 2, dtype=np.int32)
    seq = table[2].copy()
    for i in range(40):
        seq = (seq + upd[i]).astype(np.float32)
    np.testing.assert_array_equal(native.scatter_add_f32(table, same, upd)[2], seq)
    # order matters in fp32: reversing the updates changes some bits
    rev = native.scatter_add_f32(table, same[::-1].copy(), upd[::-1].copy())[2]
    assert not np.array_equal(rev, seq)


def test_scatter_add_bf16_rounds_every_add():
    rng = np.random.default_rng(15)
    tb = bf16.to_bf16_bits(rng.standard_normal((6, 8)).astype(np.float32))
    ids = rng.integers(0, 6, size=30).astype(np.int32)
    ub = bf16.to_bf16_bits(rng.standard_normal((30, 8)).astype(np.float32))
    got = native.scatter_add_bf16(tb, ids, ub)
    want = ops.scatter_add_rows_loop(bf16.from_bf16_bits(tb), ids, bf16.from_bf16_bits(ub),
                                     round_fn=bf16.round_bf16)
    np.testing.assert_array_equal(bf16.from_bf16_bits(got), want)


def test_iota():
    it = ops.iota((3, 4, 5), 1)
    for i in range(3):
        for j in range(4):
            for k in range(5):
                assert it[i, j, k] == j


def test_inputs_are_deterministic():
    a = inputs.c3_sdpa(64, batch=1, heads=2)
    b = inputs.c3_sdpa(64, batch=1, heads=2)
    for key in a:
        np.testing.assert_array_equal(a[key], b[key])
    assert a["q"].dtype == np.uint16 and a["q"].shape == (1, 2, 64, 128)


# ------------------------------------------------------------------ C5 training-step oracle
def _tiny_gpt2_params(rng, V=11, S=4, d=8, L=1, F=32):
    p = {"wte": rng.standard_normal((V, d)) * 0.5, "wpe": rng.standard_normal((S, d)) * 0.5}
    for l in range(L):
        q = f"h{l}."
        p.update({q + "ln1_g": 1 + 0.1 * rng.standard_normal(d), q + "ln1_b": 0.1 * rng.standard_normal(d),
                  q + "w_qkv": rng.standard_normal((d, 3 * d)) * 0.4, q + "b_qkv": 0.1 * rng.standard_normal(3 * d),
                  q + "w_o": rng.standard_normal((d, d)) * 0.4, q + "b_o": 0.1 * rng.standard_normal(d),
                  q + "ln2_g": 1 + 0.1 * rng.standard_normal(d), q + "ln2_b": 0.1 * rng.standard_normal(d),
                  q + "w_fc": rng.standard_normal((d, F)) * 0.4, q + "b_fc": 0.1 * rng.standard_normal(F),
                  q + "w_pr": rng.standard_normal((F, d)) * 0.3, q + "b_pr": 0.1 * rng.standard_normal(d)})
    p.update({"lnf_g": 1 + 0.1 * rng.standard_normal(d), "lnf_b": 0.1 * rng.standard_normal(d)})
    return p


def test_gpt2_ref_gradients_match_finite_differences():
    """oracle/gpt2_ref.py: the float64 autograd gradients of every parameter
    agree with central finite differences of the loss (torch gradcheck), and
    loss_and_grads returns exactly those gradients."""
    from oracle import gpt2_ref

    rng = np.random.default_rng(0)
    p = _tiny_gpt2_params(rng)
    ids = rng.integers(0, 11, (2, 4))
    labels = rng.integers(0, 11, (2, 4))
    names = sorted(p)
    ts = tuple(torch.tensor(p[n], dtype=torch.float64, requires_grad=True) for n in names)

    def f(*args):
        return gpt2_ref.forward_loss(dict(zip(names, args)), ids, labels, 1, 2)

    assert torch.autograd.gradcheck(f, ts, eps=1e-6, atol=1e-6, rtol=1e-4)
    loss, grads = gpt2_ref.loss_and_grads(p, ids, labels, 1, 2)
    auto = torch.autograd.grad(f(*ts), ts)
    for n, g in zip(names, auto):
        np.testing.assert_array_equal(grads[n], g.numpy())
    assert loss == float(f(*ts).detach())


def test_gpt2_ref_zero_head_gives_uniform_loss():
    """With the (tied) embedding table all zero every logit is 0: the loss is
    ln(V) for any labels, and the head's bias gradient dL/d lnf_b is 0."""
    from oracle import gpt2_ref

    rng = np.random.default_rng(1)
    p = _tiny_gpt2_params(rng)
    p["wte"] = np.zeros_like(p["wte"])
    ids = rng.integers(0, 11, (2, 4))
    labels = rng.integers(0, 11, (2, 4))
    loss, grads = gpt2_ref.loss_and_grads(p, ids, labels, 1, 2)
    assert abs(loss - math.log(11)) < 1e-14
    np.testing.assert_array_equal(grads["lnf_b"], 0.0)


def test_gpt2_ref_adam_first_step_closed_form():
    """From m = v = 0 at t = 1 the bias corrections cancel: p - lr g / (|g| + eps)."""
    from oracle import gpt2_ref

    rng = np.random.default_rng(2)
    p, g = rng.standard_normal(1000), rng.standard_normal(1000)
    lr, eps = 1e-3, 1e-8
    p1, m1, v1 = gpt2_ref.adam(p, g, np.zeros(1000), np.zeros(1000), 1, lr, eps=eps)
    np.testing.assert_allclose(p1, p - lr * g / (np.abs(g) + eps), rtol=1e-14, atol=1e-18)
    np.testing.assert_allclose(m1, 0.1 * g, rtol=1e-15)
    np.testing.assert_allclose(v1, 0.001 * g * g, rtol=1e-13)
