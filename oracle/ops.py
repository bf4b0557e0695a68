"""numpy restatements of the hot-path ops (oracle; test infrastructure only).

Floating-point functions compute in float64 from the exact values of their
(bf16 / fp32) inputs and return float64; the caller rounds once to the
output dtype (to_bf16_bits / astype(float32)).  Integer and indexing
functions are exact.  Each function cites the reference call site whose
semantics it restates; numerical semantics follow the StableHLO spec and
JAX's lowering, because the reference delegates the math to MPSGraph.
"""

from __future__ import annotations

import math

import numpy as np

from . import bf16 as _bf16

# ----------------------------------------------------------------- a4 dot_general


def dot_general(lhs, rhs, lhs_batch=(), rhs_batch=(), lhs_contract=(), rhs_contract=()):
    """StableHLO dot_general in float64.

    Follows the canonicalisation of src/jam/ops/linalg.mm:47-105: permute each
    operand to [batch..., free..., contract...] / [batch..., contract...,
    free...], multiply, and lay the result out as [batch..., lhs free...,
    rhs free...] (the StableHLO result order)."""
    a = np.asarray(lhs, dtype=np.float64)
    b = np.asarray(rhs, dtype=np.float64)
    lb, rb, lc, rc = map(list, (lhs_batch, rhs_batch, lhs_contract, rhs_contract))
    lf = [d for d in range(a.ndim) if d not in lb and d not in lc]
    rf = [d for d in range(b.ndim) if d not in rb and d not in rc]
    at = np.transpose(a, lb + lf + lc)
    bt = np.transpose(b, rb + rc + rf)
    nb = int(np.prod([a.shape[d] for d in lb])) if lb else 1
    m = int(np.prod([a.shape[d] for d in lf])) if lf else 1
    k = int(np.prod([a.shape[d] for d in lc])) if lc else 1
    n = int(np.prod([b.shape[d] for d in rf])) if rf else 1
    out = np.matmul(at.reshape(nb, m, k), bt.reshape(nb, k, n))
    shape = [a.shape[d] for d in lb] + [a.shape[d] for d in lf] + [b.shape[d] for d in rf]
    return out.reshape(shape)


def mlp_forward(x, w1, b1, w2, b2):
    """Config C1: relu(x @ W1 + b1) @ W2 + b2 in float64 (the jnp MLP of
    docs/ops.md:79 "MLP forward")."""
    h = dot_general(x, w1, lhs_contract=[1], rhs_contract=[0]) + np.asarray(b1, np.float64)
    h = np.maximum(h, 0.0)
    return dot_general(h, w2, lhs_contract=[1], rhs_contract=[0]) + np.asarray(b2, np.float64)


# ----------------------------------------------------------------- a5/a6 attention


def sdpa(q, k, v, scale, causal=True):
    """Scaled-dot-product attention in float64 over [..., S, D] operands.

    Restates the jnp pattern the reference lowers op by op: einsum
    (linalg.mm:98) -> * scale -> where(tril mask) (shape.mm:249-256 iota,
    binary.mm:84-109 compare, binary.mm:77-82 select) -> softmax
    (elementwise.mm:71-89) -> einsum.  The causal mask is jnp.tril of the
    [Sq, Sk] score matrix: key j is visible to query i iff j <= i.  A row
    with no visible key gives NaN, as softmax over all -inf does."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * scale
    if causal:
        sq, sk = s.shape[-2], s.shape[-1]
        mask = np.tril(np.ones((sq, sk), dtype=bool))
        s = np.where(mask, s, -np.inf)
    m = np.max(s, axis=-1, keepdims=True)
    with np.errstate(invalid="ignore"):
        p = np.exp(s - m)
        p = p / np.sum(p, axis=-1, keepdims=True)
    return np.matmul(p, v)


def sdpa_lse(q, k, scale, causal=True):
    """Natural-log log-sum-exp of the scaled, masked score rows (float64)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * scale
    if causal:
        sq, sk = s.shape[-2], s.shape[-1]
        s = np.where(np.tril(np.ones((sq, sk), dtype=bool)), s, -np.inf)
    m = np.max(s, axis=-1)
    return m + np.log(np.sum(np.exp(s - m[..., None]), axis=-1))


def softmax_rows(x):
    """softmax along the last axis (elementwise.mm:87 softMaxWithTensor)."""
    x = np.asarray(x, dtype=np.float64)
    m = np.max(x, axis=-1, keepdims=True)
    e = np.exp(x - m)
    return e / np.sum(e, axis=-1, keepdims=True)


# ----------------------------------------------------------------- a7 elementwise

GELU_C = math.sqrt(2.0 / math.pi)


def gelu_tanh(x):
    """jax.nn.gelu(approximate=True) on float32-upcast input, float64:
    0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))  (docs/ops.md:79)."""
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + np.tanh(GELU_C * (x + 0.044715 * x ** 3)))


def layernorm(x, gamma=None, beta=None, eps=1e-5):
    """LayerNorm over the last axis with biased variance, float64 two-pass
    (the reduce + elementwise "LayerNorm" composition, docs/ops.md:79):
    (x - mean) / sqrt(var + eps) * gamma + beta."""
    x = np.asarray(x, dtype=np.float64)
    mean = np.mean(x, axis=-1, keepdims=True)
    var = np.mean((x - mean) ** 2, axis=-1, keepdims=True)
    y = (x - mean) / np.sqrt(var + eps)
    if gamma is not None:
        y = y * np.asarray(gamma, dtype=np.float64)
    if beta is not None:
        y = y + np.asarray(beta, dtype=np.float64)
    return y


# ----------------------------------------------------------------- a8/a9 reduce, argmax

REDUCE_OPS = ("sum", "max", "min", "prod")


def reduce_rows(x, op="sum", init=None):
    """StableHLO reduce over the last axis in float64 (reduce.mm:79-108, whose
    generic path ignores the init operand; StableHLO folds it in, and so do
    we).  max/min propagate NaN."""
    x = np.asarray(x, dtype=np.float64)
    if op == "sum":
        r = np.sum(x, axis=-1)
        return r if init is None else r + init
    if op == "prod":
        r = np.prod(x, axis=-1)
        return r if init is None else r * init
    if op == "max":
        r = np.max(x, axis=-1)  # np.max propagates NaN
        return r if init is None else np.maximum(r, init)
    if op == "min":
        r = np.min(x, axis=-1)
        return r if init is None else np.minimum(r, init)
    raise ValueError(op)


def argmax_rows(x, is_min=False):
    """Exact row argmax / argmin with the semantics of the variadic reduce
    JAX emits for jnp.argmax / jnp.argmin (matched by DetectArgReduce,
    reduce.mm:29-43, emitted at reduce.mm:61-77): the larger (smaller) value
    wins, NaN beats every number, ties go to the lower index; -0.0 == +0.0.

    numpy's argmax/argmin implement exactly this order (first occurrence of
    the extremum, NaN treated as the extremum); the pins in tests compare it
    with a brute-force pairwise reducer.  Returns (index int64, value)."""
    x = np.asarray(x)
    idx = np.argmin(x, axis=-1) if is_min else np.argmax(x, axis=-1)
    val = np.take_along_axis(x, idx[..., None], axis=-1)[..., 0]
    return idx.astype(np.int64), val


def argmax_reducer_pairwise(values, is_min=False):
    """Literal pairwise form of JAX's argmax reducer body for one row
    (value_a, index_a) x (value_b, index_b) -> winner, folded left to right.
    Used only to pin argmax_rows on small inputs."""
    best_v, best_i = None, None
    for i, v in enumerate(values):
        v = float(v)
        if best_i is None:
            best_v, best_i = v, i
            continue
        a_nan, b_nan = math.isnan(v), math.isnan(best_v)
        if a_nan or b_nan:
            take = a_nan and not b_nan
        elif v == best_v:
            take = False  # equal: the earlier (lower) index stays
        else:
            take = (v < best_v) if is_min else (v > best_v)
        if take:
            best_v, best_i = v, i
    return best_i, best_v


# ----------------------------------------------------------------- C5 loss


def softmax_xent(logits, labels, grad_scale):
    """Per-row softmax cross-entropy and its logit gradient in float64: the
    loss rows and d(mean loss)/d logits of the jitted step's
    optax-style loss (temp/dp_train.py:67-70 value_and_grad of a mean loss),
    loss_r = logsumexp(x_r) - x_r[label_r], dlogits = (softmax(x_r) -
    onehot(label_r)) * grad_scale.  An out-of-range label has no target term
    (loss = logsumexp, gradient = softmax * grad_scale), as the one-hot form
    sum(select(iota == label, x, 0)) of the jitted module gives."""
    x = np.asarray(logits, dtype=np.float64)
    lab = np.asarray(labels).astype(np.int64).reshape(-1)
    m = np.max(x, axis=-1, keepdims=True)
    e = np.exp(x - m)
    s = e.sum(axis=-1, keepdims=True)
    lse = (m + np.log(s))[:, 0]
    ok = (lab >= 0) & (lab < x.shape[-1])
    picked = np.where(ok, x[np.arange(x.shape[0]), np.clip(lab, 0, x.shape[-1] - 1)], 0.0)
    grad = e / s
    grad[np.arange(x.shape[0])[ok], lab[ok]] -= 1.0
    return lse - picked, grad * grad_scale


# ----------------------------------------------------------------- a10/a11 gather, scatter


def gather_rows(table, ids):
    """Embedding gather: table[clamp(ids, 0, n-1)] — gather_scatter.mm:135-207,
    index clamp at 180-183 (StableHLO gather clamps start indices)."""
    table = np.asarray(table)
    ids = np.asarray(ids).astype(np.int64)
    return table[np.clip(ids, 0, table.shape[0] - 1)]


def scatter_add_rows_f32(table, ids, updates):
    """Sequential fp32 scatter-add: for i = 0, 1, ...: table[ids[i]] += updates[i],
    each add rounded to fp32, out-of-range ids dropped (StableHLO scatter /
    JAX FILL_OR_DROP).  np.add.at applies the updates unbuffered in index
    order, which is this sequential order.  Replaces the order-unspecified
    scatterNDWithDataTensor mode:Add of gather_scatter.mm:322-327."""
    out = np.array(table, dtype=np.float32, copy=True)
    ids = np.asarray(ids).reshape(-1).astype(np.int64)
    upd = np.asarray(updates, dtype=np.float32).reshape(ids.shape[0], out.shape[1])
    keep = (ids >= 0) & (ids < out.shape[0])
    np.add.at(out, ids[keep], upd[keep])
    return out


def scatter_add_rows_loop(table, ids, updates, round_fn=None):
    """Literal per-update loop (pins scatter_add_rows_f32 on small inputs and
    restates the bf16 variant: round_fn applied after every add)."""
    out = np.array(table, dtype=np.float32, copy=True)
    ids = np.asarray(ids).reshape(-1).astype(np.int64)
    upd = np.asarray(updates, dtype=np.float32).reshape(ids.shape[0], out.shape[1])
    for i, r in enumerate(ids):
        if 0 <= r < out.shape[0]:
            s = (out[r] + upd[i]).astype(np.float32)
            out[r] = round_fn(s) if round_fn is not None else s
    return out


# ----------------------------------------------------------------- a6 iota


def iota(shape, dim, dtype=np.int32):
    """StableHLO iota: out[idx] = idx[dim] (shape.mm:249-256)."""
    shape = tuple(int(s) for s in shape)
    ar = np.arange(shape[dim], dtype=np.int64)
    view = [1] * len(shape)
    view[dim] = shape[dim]
    return np.broadcast_to(ar.reshape(view), shape).astype(dtype)


def round_to(x, dtype):
    """Single rounding of float64 results to the output dtype; bf16 comes back
    as uint16 bits."""
    if dtype == "bf16":
        return _bf16.to_bf16_bits_f64(x)
    return np.asarray(x).astype(dtype)
