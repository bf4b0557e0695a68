"""StableHLO text of the C5 training step as one jitted module: the mean
softmax cross-entropy of a pre-LayerNorm GPT-2 decoder, its gradients with
respect to every parameter, and the Adam update of temp/dp_train.py:67-76
(``loss, grads = jax.value_and_grad(loss_fn)(params, batch)`` followed by
the per-parameter update of lines 71-75).

JAX is not installed in this image, so the module is written by a small
graph builder with reverse-mode differentiation: every differentiable op
records its vector-Jacobian product, and ``Builder.grad`` walks the record
backwards emitting the transposed ops, the way ``jax.grad`` produces the
backward half of a jitted step.  The ops and text forms are the ones the
other modules here use (``jax.jit(...).lower(...).as_text()`` pretty form).
Mixed precision as a bf16 JAX model runs it: parameters, optimizer state and
every elementwise / reduction op in fp32, the matrix products on bf16
operands with fp32 results (``preferred_element_type=float32``).

Inputs, in order: the parameters (``GPT2Config.param_shapes`` order, fp32),
then Adam's m and v for each (same order), then ids and labels (i32 [B, S]),
then three f32 scalars: lr, 1 / (1 - b1^t), 1 / (1 - b2^t).  Outputs: the
loss, the updated parameters, m and v (same order), and, when asked for, the
gradients (same order).
"""

from __future__ import annotations

import math


def _t(shape, dt):
    return "tensor<" + "".join(f"{d}x" for d in shape) + dt + ">"


class V:
    """An SSA value of the module being built."""

    __slots__ = ("name", "shape", "dt", "needs_grad")

    def __init__(self, name, shape, dt, needs_grad=False):
        self.name, self.shape, self.dt, self.needs_grad = name, tuple(shape), dt, needs_grad

    @property
    def type(self):
        return _t(self.shape, self.dt)


class Builder:
    def __init__(self):
        self.lines: list[str] = []
        self.args: list[V] = []
        self.n = 0
        self.tape: list[tuple] = []  # (out, inputs, vjp(g) -> cotangents per input)

    # ------------------------------------------------------------------ plumbing
    def arg(self, shape, dt, needs_grad=False) -> V:
        v = V(f"%arg{len(self.args)}", shape, dt, needs_grad)
        self.args.append(v)
        return v

    def _new(self, shape, dt, inputs=()) -> V:
        v = V(f"%{self.n}", shape, dt, any(i.needs_grad for i in inputs))
        self.n += 1
        return v

    def _emit(self, text):
        self.lines.append("    " + text)

    def _record(self, out, inputs, vjp):
        if out.needs_grad:
            self.tape.append((out, inputs, vjp))
        return out

    # ------------------------------------------------------------------ constants
    def scalar(self, x, dt="f32") -> V:
        v = V(f"%cst_{self.n}", (), dt)
        self.n += 1
        if dt == "f32" and math.isinf(x):
            lit = "0xFF800000" if x < 0 else "0x7F800000"
        elif dt in ("f32", "bf16"):
            lit = f"{x:.9e}"
        else:
            lit = str(int(x))
        self._emit(f"{v.name} = stablehlo.constant dense<{lit}> : {v.type}")
        return v

    def full(self, x, shape, dt="f32") -> V:
        return self.bcast(self.scalar(x, dt), shape, ())

    # ------------------------------------------------------------------ shape ops
    def bcast(self, x: V, shape, dims) -> V:
        """broadcast_in_dim: x's dim k becomes result dim dims[k]."""
        shape, dims = tuple(shape), tuple(dims)
        out = self._new(shape, x.dt, (x,))
        self._emit(f"{out.name} = stablehlo.broadcast_in_dim {x.name}, dims = [{', '.join(map(str, dims))}] : "
                   f"({x.type}) -> {out.type}")

        def vjp(g):
            # sum over result dims that x does not map, and over dims x has
            # as size 1 but the result widened; then reshape to x
            summed = [d for d in range(len(shape)) if d not in dims or
                      (x.shape[dims.index(d)] == 1 and shape[d] != 1)]
            r = self.reduce_sum(g, summed) if summed else g
            return [self.reshape(r, x.shape) if r.shape != x.shape else r]
        return self._record(out, [x], vjp)

    def reshape(self, x: V, shape) -> V:
        out = self._new(shape, x.dt, (x,))
        self._emit(f"{out.name} = stablehlo.reshape {x.name} : ({x.type}) -> {out.type}")
        return self._record(out, [x], lambda g: [self.reshape(g, x.shape)])

    def transpose(self, x: V, perm) -> V:
        perm = tuple(perm)
        out = self._new(tuple(x.shape[p] for p in perm), x.dt, (x,))
        self._emit(f"{out.name} = stablehlo.transpose {x.name}, dims = [{', '.join(map(str, perm))}] : "
                   f"({x.type}) -> {out.type}")
        inv = tuple(perm.index(k) for k in range(len(perm)))
        return self._record(out, [x], lambda g: [self.transpose(g, inv)])

    def slice(self, x: V, starts, limits) -> V:
        out = self._new(tuple(l - s for s, l in zip(starts, limits)), x.dt, (x,))
        spec = ", ".join(f"{s}:{l}" for s, l in zip(starts, limits))
        self._emit(f"{out.name} = stablehlo.slice {x.name} [{spec}] : ({x.type}) -> {out.type}")

        def vjp(g):
            # the rows around the slice get zero cotangent (slices here cut
            # the leading dim only)
            assert all(s == 0 and l == n for s, l, n in zip(starts[1:], limits[1:], x.shape[1:]))
            parts = []
            if starts[0] > 0:
                parts.append(self.full(0.0, (starts[0],) + x.shape[1:], g.dt))
            parts.append(g)
            if limits[0] < x.shape[0]:
                parts.append(self.full(0.0, (x.shape[0] - limits[0],) + x.shape[1:], g.dt))
            return [self.concat(parts, 0) if len(parts) > 1 else g]
        return self._record(out, [x], vjp)

    def concat(self, xs, dim) -> V:
        shape = list(xs[0].shape)
        shape[dim] = sum(x.shape[dim] for x in xs)
        out = self._new(shape, xs[0].dt, xs)
        self._emit(f"{out.name} = stablehlo.concatenate {', '.join(x.name for x in xs)}, dim = {dim} : "
                   f"({', '.join(x.type for x in xs)}) -> {out.type}")
        return out  # only built on cotangents here (not differentiated)

    def split(self, x: V, dim, sizes):
        """Consecutive slices of x along `dim`; the cotangent of x is the
        concatenation of theirs (zeros for an unused part)."""
        outs, off = [], 0
        for n in sizes:
            starts = [0] * len(x.shape)
            limits = list(x.shape)
            starts[dim], limits[dim] = off, off + n
            o = self._new(tuple(l - s for s, l in zip(starts, limits)), x.dt, (x,))
            spec = ", ".join(f"{s}:{l}" for s, l in zip(starts, limits))
            self._emit(f"{o.name} = stablehlo.slice {x.name} [{spec}] : ({x.type}) -> {o.type}")
            outs.append(o)
            off += n
        # one record for the group: the cotangents of the parts are gathered
        # by grad() before this entry is reached (it follows every part)
        self._split_groups = getattr(self, "_split_groups", {})
        gid = len(self._split_groups)
        self._split_groups[gid] = (x, dim, outs)
        if x.needs_grad:
            for o in outs:
                o.needs_grad = True
            self.tape.append((None, [x], ("split", gid)))
        return outs

    # ------------------------------------------------------------------ elementwise
    def _binary(self, op, a: V, b: V, vjp) -> V:
        assert a.shape == b.shape and a.dt == b.dt, (op, a.shape, b.shape, a.dt, b.dt)
        out = self._new(a.shape, a.dt, (a, b))
        self._emit(f"{out.name} = stablehlo.{op} {a.name}, {b.name} : {out.type}")
        return self._record(out, [a, b], vjp)

    def add(self, a, b):
        return self._binary("add", a, b, lambda g: [g, g])

    def sub(self, a, b):
        return self._binary("subtract", a, b, lambda g: [g, self.neg(g)])

    def mul(self, a, b):
        return self._binary("multiply", a, b, lambda g: [self.mul(g, b), self.mul(g, a)])

    def div(self, a, b):
        out = None

        def vjp(g):
            return [self.div(g, b), self.neg(self.mul(g, self.div(out, b)))]
        out = self._binary("divide", a, b, vjp)
        return out

    def _unary(self, op, x: V, vjp, dt=None) -> V:
        out = self._new(x.shape, dt or x.dt, (x,))
        if dt and dt != x.dt:
            self._emit(f"{out.name} = stablehlo.{op} {x.name} : ({x.type}) -> {out.type}")
        else:
            self._emit(f"{out.name} = stablehlo.{op} {x.name} : {out.type}")
        return self._record(out, [x], vjp)

    def neg(self, x):
        return self._unary("negate", x, lambda g: [self.neg(g)])

    def exp(self, x):
        out = None
        out = self._unary("exponential", x, lambda g: [self.mul(g, out)])
        return out

    def log(self, x):
        return self._unary("log", x, lambda g: [self.div(g, x)])

    def tanh(self, x):
        out = None

        def vjp(g):
            one = self.full(1.0, x.shape)
            return [self.mul(g, self.sub(one, self.mul(out, out)))]
        out = self._unary("tanh", x, vjp)
        return out

    def rsqrt(self, x):
        out = None

        def vjp(g):
            c = self.full(-0.5, x.shape)
            return [self.mul(self.mul(g, c), self.mul(out, self.mul(out, out)))]
        out = self._unary("rsqrt", x, vjp)
        return out

    def sqrt(self, x):
        return self._unary("sqrt", x, None)

    def convert(self, x: V, dt) -> V:
        if x.dt == dt:
            return x
        return self._unary("convert", x, lambda g: [self.convert(g, x.dt)], dt)

    def stop(self, x: V) -> V:
        """x without a gradient path (jax.lax.stop_gradient)."""
        return V(x.name, x.shape, x.dt, False)

    def select(self, p: V, a: V, b: V) -> V:
        out = self._new(a.shape, a.dt, (a, b))
        self._emit(f"{out.name} = stablehlo.select {p.name}, {a.name}, {b.name} : {p.type}, {out.type}")

        def vjp(g):
            z = self.full(0.0, g.shape, g.dt)
            return [self.select(p, g, z), self.select(p, z, g)]
        return self._record(out, [a, b], vjp)

    def iota(self, shape, dim, dt="i32") -> V:
        out = self._new(shape, dt)
        self._emit(f"{out.name} = stablehlo.iota dim = {dim} : {out.type}")
        return out

    def compare(self, a: V, b: V, direction, kind="SIGNED") -> V:
        out = self._new(a.shape, "i1")
        self._emit(f"{out.name} = stablehlo.compare  {direction}, {a.name}, {b.name},  {kind} : "
                   f"({a.type}, {b.type}) -> {out.type}")
        return out

    # ------------------------------------------------------------------ reductions
    def _reduce(self, x: V, dims, body, init) -> V:
        dims = tuple(sorted(dims))
        shape = tuple(n for d, n in enumerate(x.shape) if d not in dims)
        out = self._new(shape, x.dt, (x,))
        c = self.scalar(init, x.dt)
        self._emit(f"{out.name} = stablehlo.reduce({x.name} init: {c.name}) applies stablehlo.{body} across "
                   f"dimensions = [{', '.join(map(str, dims))}] : ({x.type}, {c.type}) -> {out.type}")
        return out, dims

    def reduce_sum(self, x: V, dims) -> V:
        out, dims = self._reduce(x, dims, "add", 0.0)
        keep = tuple(d for d in range(len(x.shape)) if d not in dims)
        return self._record(out, [x], lambda g: [self.bcast(g, x.shape, keep)])

    def reduce_max(self, x: V, dims) -> V:
        """Not differentiated (used behind stop_gradient, as jax.nn.softmax
        and logsumexp do)."""
        out, _ = self._reduce(self.stop(x), dims, "maximum", -math.inf)
        return out

    def softmax_last(self, x: V) -> V:
        """jax.nn.softmax over the last axis: the forward as it lowers
        (max behind stop_gradient, exp, sum, divide) and its custom JVP rule
        y * (x' - sum(y * x')) transposed, so the backward is
        y g - y bcast(sum(y g)) with y g formed once (what jax.grad emits for
        jax.nn.softmax after CSE)."""
        r = len(x.shape) - 1
        keep = tuple(range(r))
        xs = self.stop(x)
        m = self.reduce_max(xs, [r])
        e = self.exp(self.sub(xs, self.bcast(m, x.shape, keep)))
        z = self.reduce_sum(e, [r])
        y = self.div(e, self.bcast(z, x.shape, keep))
        y.needs_grad = x.needs_grad

        def vjp(g):
            ys = self.stop(y)
            yg = self.mul(g, ys)
            t = self.reduce_sum(yg, [r])
            return [self.sub(yg, self.mul(ys, self.bcast(t, x.shape, keep)))]
        return self._record(y, [x], vjp)

    # ------------------------------------------------------------------ products
    def dot(self, a: V, b: V, lc, rc, lb=(), rb=(), out_dt="f32") -> V:
        """dot_general; result dims: batch, a's free dims, b's free dims."""
        fa = [d for d in range(len(a.shape)) if d not in lc and d not in lb]
        fb = [d for d in range(len(b.shape)) if d not in rc and d not in rb]
        shape = [a.shape[d] for d in lb] + [a.shape[d] for d in fa] + [b.shape[d] for d in fb]
        out = self._new(shape, out_dt, (a, b))
        bt = f"batching_dims = [{', '.join(map(str, lb))}] x [{', '.join(map(str, rb))}], " if lb else ""
        self._emit(f"{out.name} = stablehlo.dot_general {a.name}, {b.name}, {bt}contracting_dims = "
                   f"[{', '.join(map(str, lc))}] x [{', '.join(map(str, rc))}], precision = [DEFAULT, DEFAULT] : "
                   f"({a.type}, {b.type}) -> {out.type}")
        return out

    def mm(self, a: V, b: V, kind="nn") -> V:
        """2-D matrix product on bf16 operands, fp32 result: kind nn = a·b,
        nt = a·bᵀ."""
        ab, bb = self.convert(self.stop(a), "bf16"), self.convert(self.stop(b), "bf16")
        rc = [0] if kind == "nn" else [1]
        out = self.dot(ab, bb, [1], rc)
        out.needs_grad = a.needs_grad or b.needs_grad

        def vjp(g):
            gb16 = self.convert(self.stop(g), "bf16")
            # da = g·bᵀ (nn) or g·b (nt); db = aᵀ·g (nn) or gᵀ·a (nt)
            da = self.dot(gb16, bb, [1], [1] if kind == "nn" else [0]) if a.needs_grad else None
            if not b.needs_grad:
                db = None
            elif kind == "nn":
                db = self.dot(ab, gb16, [0], [0])
            else:
                db = self.dot(gb16, ab, [0], [0])
            return [da, db]
        return self._record(out, [a, b], vjp)

    def bmm(self, a: V, b: V, lc, rc) -> V:
        """Batched (dims 0, 1) product of two rank-4 bf16-operand tensors,
        fp32 result; a, b are fp32 values converted here."""
        ab, bb = self.convert(self.stop(a), "bf16"), self.convert(self.stop(b), "bf16")
        out = self.dot(ab, bb, [lc], [rc], [0, 1], [0, 1])
        out.needs_grad = a.needs_grad or b.needs_grad
        fa = 3 if lc == 2 else 2  # a's free dim
        fb = 3 if rc == 2 else 2

        def vjp(g):
            gb16 = self.convert(self.stop(g), "bf16")
            # out[b,h,i,j] = sum_k a[.., i|k ..] b[.., k|j ..]: g's dim 2 is a's
            # free dim, dim 3 is b's free dim
            da = self.dot(gb16, bb, [3], [fb], [0, 1], [0, 1])  # [B,H, a_free, a_contract]
            if fa == 3:  # a was [B,H,k,i]: da computed as [B,H,i,k]
                da = self.transpose(da, (0, 1, 3, 2))
            db = self.dot(gb16, ab, [2], [fa], [0, 1], [0, 1])  # [B,H, b_free, b_contract]
            if fb == 2:  # b was [B,H,j,k]: db computed as [B,H,j,k] -> already (free, contract)
                pass
            else:  # b was [B,H,k,j]
                db = self.transpose(db, (0, 1, 3, 2))
            return [da if a.needs_grad else None, db if b.needs_grad else None]
        return self._record(out, [a, b], vjp)

    # ------------------------------------------------------------------ indexing
    def gather_rows(self, table: V, ids: V) -> V:
        """table[ids] for i32 ids [n] (row gather, like jnp indexing)."""
        n = ids.shape[0]
        ie = self._new((n, 1), ids.dt)
        self._emit(f"{ie.name} = stablehlo.broadcast_in_dim {ids.name}, dims = [0] : ({ids.type}) -> {ie.type}")
        out = self._new((n,) + table.shape[1:], table.dt, (table,))
        self._emit(f'{out.name} = "stablehlo.gather"({table.name}, {ie.name}) <{{dimension_numbers = '
                   f"#stablehlo.gather<offset_dims = [1], collapsed_slice_dims = [0], start_index_map = [0], "
                   f"index_vector_dim = 1>, indices_are_sorted = false, slice_sizes = array<i64: 1, "
                   f"{', '.join(map(str, table.shape[1:]))}>}}> : ({table.type}, {ie.type}) -> {out.type}")

        def vjp(g):
            z = self.full(0.0, table.shape, g.dt)
            return [self.scatter_add_rows(z, ie, g)]
        return self._record(out, [table], vjp)

    def scatter_add_rows(self, table: V, ie: V, upd: V) -> V:
        out = self._new(table.shape, table.dt)
        self._emit(f'{out.name} = "stablehlo.scatter"({table.name}, {ie.name}, {upd.name}) <{{indices_are_sorted '
                   f"= false, scatter_dimension_numbers = #stablehlo.scatter<update_window_dims = [1], "
                   f"inserted_window_dims = [0], scatter_dims_to_operand_dims = [0], index_vector_dim = 1>, "
                   f"unique_indices = false}}> ({{")
        self._emit(f"^bb0(%sa{self.n}: tensor<{table.dt}>, %sb{self.n}: tensor<{table.dt}>):")
        self._emit(f"  %ss{self.n} = stablehlo.add %sa{self.n}, %sb{self.n} : tensor<{table.dt}>")
        self._emit(f"  stablehlo.return %ss{self.n} : tensor<{table.dt}>")
        self._emit(f"}}) : ({table.type}, {ie.type}, {upd.type}) -> {out.type}")
        self.n += 1
        return out

    # ------------------------------------------------------------------ reverse mode
    def grad(self, loss: V, wrt):
        """Cotangents of the scalar `loss` with respect to each value in
        `wrt` (zeros where no path exists), emitted after the forward ops."""
        cot = {loss.name: self.full(1.0, loss.shape, loss.dt)}

        def acc(v, ct):
            if ct is None or not v.needs_grad:
                return
            if ct.shape != v.shape:
                ct = self.reshape(ct, v.shape)
            cot[v.name] = self.add(cot[v.name], ct) if v.name in cot else ct

        for out, inputs, vjp in reversed(self.tape):
            if out is None:  # split group: concatenate the parts' cotangents
                x, dim, outs = self._split_groups[vjp[1]]
                if not any(o.name in cot for o in outs):
                    continue
                parts = [cot.get(o.name) or self.full(0.0, o.shape, x.dt) for o in outs]
                acc(x, self.concat(parts, dim))
                continue
            g = cot.get(out.name)
            if g is None:
                continue
            for v, ct in zip(inputs, vjp(g)):
                acc(v, ct)
        # the backward ops are not differentiated again
        return [cot.get(v.name) or self.full(0.0, v.shape, v.dt) for v in wrt]

    # ------------------------------------------------------------------ text
    def module(self, name, outputs) -> str:
        sig = ", ".join(f"{a.name}: {a.type}" for a in self.args)
        res = ", ".join(f'{o.type} {{jax.result_info = ""}}' for o in outputs)
        ret = f"    return {', '.join(o.name for o in outputs)} : {', '.join(o.type for o in outputs)}"
        return (f"module @{name} attributes {{mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32}} {{\n"
                f"  func.func public @main({sig}) -> ({res}) {{\n" + "\n".join(self.lines) + "\n" + ret +
                "\n  }\n}\n")


def gpt2_train_step(cfg, b1=0.9, b2=0.999, eps=1e-8, return_grads=False) -> str:
    """The module described in the file's docstring for a GPT2Config."""
    B, S, d, H, L, Vv = cfg.batch, cfg.seq, cfg.d_model, cfg.n_head, cfg.n_layer, cfg.vocab
    hd, T = d // H, cfg.batch * cfg.seq
    shapes = cfg.param_shapes()
    g = Builder()
    P = {n: g.arg(s, "f32", needs_grad=True) for n, s in shapes}
    M = {n: g.arg(s, "f32") for n, s in shapes}
    Vs = {n: g.arg(s, "f32") for n, s in shapes}
    ids = g.arg((B, S), "i32")
    labels = g.arg((B, S), "i32")
    lr, c1, c2 = g.arg((), "f32"), g.arg((), "f32"), g.arg((), "f32")

    def row_bcast(v, rows):  # [n] -> [rows, n]
        return g.bcast(v, (rows, v.shape[0]), (1,))

    def col_bcast(v, cols):  # [rows] -> [rows, cols]
        return g.bcast(v, (v.shape[0], cols), (0,))

    def layernorm(x, gam, bet):
        n = x.shape[1]
        inv_n = g.full(1.0 / n, (x.shape[0],))
        mean = g.mul(g.reduce_sum(x, [1]), inv_n)
        xc = g.sub(x, col_bcast(mean, n))
        var = g.mul(g.reduce_sum(g.mul(xc, xc), [1]), inv_n)
        r = g.rsqrt(g.add(var, g.full(cfg.ln_eps, var.shape)))
        y = g.mul(xc, col_bcast(r, n))
        return g.add(g.mul(y, row_bcast(gam, x.shape[0])), row_bcast(bet, x.shape[0]))

    def gelu(x):  # 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
        s = x.shape
        inner = g.add(x, g.mul(g.full(0.044715, s), g.mul(x, g.mul(x, x))))
        t = g.tanh(g.mul(g.full(math.sqrt(2.0 / math.pi), s), inner))
        return g.mul(g.mul(g.full(0.5, s), x), g.add(g.full(1.0, s), t))

    def heads(t):  # [T, d] -> [B, H, S, hd]
        return g.transpose(g.reshape(t, (B, S, H, hd)), (0, 2, 1, 3))

    # embeddings
    ids_flat = g.reshape(ids, (T,))
    pos = P["wpe"] if P["wpe"].shape[0] == S else g.slice(P["wpe"], (0, 0), (S, d))
    x = g.add(g.gather_rows(P["wte"], ids_flat), g.reshape(g.bcast(pos, (B, S, d), (1, 2)), (T, d)))
    # causal mask [B, H, S, S]
    qi, ki = g.iota((S, S), 0), g.iota((S, S), 1)
    causal = g.bcast(g.compare(qi, ki, "GE"), (B, H, S, S), (2, 3))
    scale = g.full(1.0 / math.sqrt(hd), (B, H, S, S))
    neg_inf = g.full(-math.inf, (B, H, S, S))
    for layer in range(L):
        p = lambda n: P[f"h{layer}.{n}"]  # noqa: E731
        h = layernorm(x, p("ln1_g"), p("ln1_b"))
        qkv = g.add(g.mm(h, p("w_qkv")), row_bcast(p("b_qkv"), T))
        q, k, v = (heads(t) for t in g.split(qkv, 1, (d, d, d)))
        s = g.select(causal, g.mul(g.bmm(q, k, 3, 3), scale), neg_inf)
        pr = g.softmax_last(s)
        o = g.bmm(pr, v, 3, 2)  # [B, H, S, hd]
        a = g.reshape(g.transpose(o, (0, 2, 1, 3)), (T, d))
        x = g.add(x, g.add(g.mm(a, p("w_o")), row_bcast(p("b_o"), T)))
        h2 = layernorm(x, p("ln2_g"), p("ln2_b"))
        f = gelu(g.add(g.mm(h2, p("w_fc")), row_bcast(p("b_fc"), T)))
        x = g.add(x, g.add(g.mm(f, p("w_pr")), row_bcast(p("b_pr"), T)))
    hf = layernorm(x, P["lnf_g"], P["lnf_b"])
    logits = g.mm(hf, P["wte"], "nt")  # [T, V]
    # mean softmax cross-entropy: logsumexp(logits) - logits[label]
    mx = g.reduce_max(logits, [1])
    lse = g.add(g.log(g.reduce_sum(g.exp(g.sub(logits, col_bcast(mx, Vv))), [1])), mx)
    onehot = g.compare(g.iota((T, Vv), 1), g.bcast(g.reshape(labels, (T,)), (T, Vv), (0,)), "EQ")
    picked = g.reduce_sum(g.select(onehot, logits, g.full(0.0, (T, Vv))), [1])
    loss = g.mul(g.reduce_sum(g.sub(lse, picked), [0]), g.scalar(1.0 / T))
    names = [n for n, _ in shapes]
    grads = g.grad(loss, [P[n] for n in names])
    # Adam (temp/dp_train.py:71-75), the step's scalars broadcast per tensor
    new_p, new_m, new_v = [], [], []
    for n, gr in zip(names, grads):
        s = P[n].shape
        bc = lambda c: g.bcast(c, s, ())  # noqa: E731
        m1 = g.add(g.mul(g.full(b1, s), M[n]), g.mul(g.full(1 - b1, s), gr))
        v1 = g.add(g.mul(g.full(b2, s), Vs[n]), g.mul(g.full(1 - b2, s), g.mul(gr, gr)))
        step = g.div(g.mul(g.mul(bc(lr), m1), bc(c1)), g.add(g.sqrt(g.mul(v1, bc(c2))), g.full(eps, s)))
        new_p.append(g.sub(g.stop(P[n]), g.stop(step)))
        new_m.append(m1)
        new_v.append(v1)
    outs = [loss] + new_p + new_m + new_v + (list(grads) if return_grads else [])
    return g.module("jit_train_step", outs)
