"""StableHLO text of the benchmark config functions, in the form jax.jit
lowers them (``jax.jit(f).lower(*args).as_text()``): pretty-printed ops,
``func.call`` for nested jits (``@relu``), keepdims via ``broadcast_in_dim``,
the iota/compare causal mask, generic-form gather/scatter.

JAX is not installed in this image, so these texts are written from the jnp
definitions given in each docstring; they are the inputs of the PJRT
end-to-end tests and of the compile-structure tests.
"""

from __future__ import annotations


def _t(shape, dt):
    return "tensor<" + "".join(f"{d}x" for d in shape) + dt + ">"


def mlp(m=256, k=1024, h=4096, n=1024) -> str:
    """C1: relu(x @ w1 + b1) @ w2 + b2, fp32 (jax.nn.relu is a nested jit)."""
    x, w1, b1, w2, b2 = _t((m, k), "f32"), _t((k, h), "f32"), _t((h,), "f32"), _t((h, n), "f32"), _t((n,), "f32")
    mh, mn = _t((m, h), "f32"), _t((m, n), "f32")
    return f"""module @jit_mlp attributes {{mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32}} {{
  func.func public @main(%arg0: {x}, %arg1: {w1}, %arg2: {b1}, %arg3: {w2}, %arg4: {b2}) -> ({mn} {{jax.result_info = ""}}) {{
    %0 = stablehlo.dot_general %arg0, %arg1, contracting_dims = [1] x [0], precision = [DEFAULT, DEFAULT] : ({x}, {w1}) -> {mh}
    %1 = stablehlo.broadcast_in_dim %arg2, dims = [1] : ({b1}) -> {_t((1, h), "f32")}
    %2 = stablehlo.broadcast_in_dim %1, dims = [0, 1] : ({_t((1, h), "f32")}) -> {mh}
    %3 = stablehlo.add %0, %2 : {mh}
    %4 = call @relu(%3) : ({mh}) -> {mh}
    %5 = stablehlo.dot_general %4, %arg3, contracting_dims = [1] x [0], precision = [DEFAULT, DEFAULT] : ({mh}, {w2}) -> {mn}
    %6 = stablehlo.broadcast_in_dim %arg4, dims = [1] : ({b2}) -> {_t((1, n), "f32")}
    %7 = stablehlo.broadcast_in_dim %6, dims = [0, 1] : ({_t((1, n), "f32")}) -> {mn}
    %8 = stablehlo.add %5, %7 : {mn}
    return %8 : {mn}
  }}
  func.func private @relu(%arg0: {mh}) -> {mh} {{
    %cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %0 = stablehlo.broadcast_in_dim %cst, dims = [] : (tensor<f32>) -> {mh}
    %1 = stablehlo.maximum %arg0, %0 : {mh}
    return %1 : {mh}
  }}
}}
"""


def layernorm(rows=8192, cols=4096, eps=1e-5) -> str:
    """C2a: xf = x.astype(f32); mean = xf.mean(-1, keepdims); xc = xf - mean;
    var = (xc * xc).mean(-1, keepdims);
    y = xc * rsqrt(var + eps) * gamma.astype(f32) + beta.astype(f32); y.astype(bf16)."""
    xb, xf = _t((rows, cols), "bf16"), _t((rows, cols), "f32")
    v, c1 = _t((cols,), "bf16"), _t((rows, 1), "f32")
    r1, vf, vc = _t((rows,), "f32"), _t((cols,), "f32"), _t((1, cols), "f32")
    return f"""module @jit_layernorm attributes {{mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32}} {{
  func.func public @main(%arg0: {xb}, %arg1: {v}, %arg2: {v}) -> ({xb} {{jax.result_info = ""}}) {{
    %0 = stablehlo.convert %arg0 : ({xb}) -> {xf}
    %cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %1 = stablehlo.reduce(%0 init: %cst) applies stablehlo.add across dimensions = [1] : ({xf}, tensor<f32>) -> {r1}
    %2 = stablehlo.broadcast_in_dim %1, dims = [0] : ({r1}) -> {c1}
    %cst_0 = stablehlo.constant dense<{float(cols):e}> : tensor<f32>
    %3 = stablehlo.broadcast_in_dim %cst_0, dims = [] : (tensor<f32>) -> {c1}
    %4 = stablehlo.divide %2, %3 : {c1}
    %5 = stablehlo.broadcast_in_dim %4, dims = [0, 1] : ({c1}) -> {xf}
    %6 = stablehlo.subtract %0, %5 : {xf}
    %7 = stablehlo.multiply %6, %6 : {xf}
    %8 = stablehlo.reduce(%7 init: %cst) applies stablehlo.add across dimensions = [1] : ({xf}, tensor<f32>) -> {r1}
    %9 = stablehlo.broadcast_in_dim %8, dims = [0] : ({r1}) -> {c1}
    %10 = stablehlo.divide %9, %3 : {c1}
    %cst_1 = stablehlo.constant dense<{eps:e}> : tensor<f32>
    %11 = stablehlo.broadcast_in_dim %cst_1, dims = [] : (tensor<f32>) -> {c1}
    %12 = stablehlo.add %10, %11 : {c1}
    %13 = stablehlo.rsqrt %12 : {c1}
    %14 = stablehlo.broadcast_in_dim %13, dims = [0, 1] : ({c1}) -> {xf}
    %15 = stablehlo.multiply %6, %14 : {xf}
    %16 = stablehlo.convert %arg1 : ({v}) -> {vf}
    %17 = stablehlo.broadcast_in_dim %16, dims = [1] : ({vf}) -> {vc}
    %18 = stablehlo.broadcast_in_dim %17, dims = [0, 1] : ({vc}) -> {xf}
    %19 = stablehlo.multiply %15, %18 : {xf}
    %20 = stablehlo.convert %arg2 : ({v}) -> {vf}
    %21 = stablehlo.broadcast_in_dim %20, dims = [1] : ({vf}) -> {vc}
    %22 = stablehlo.broadcast_in_dim %21, dims = [0, 1] : ({vc}) -> {xf}
    %23 = stablehlo.add %19, %22 : {xf}
    %24 = stablehlo.convert %23 : ({xf}) -> {xb}
    return %24 : {xb}
  }}
}}
"""


def gelu(rows=8192, cols=16384) -> str:
    """C2b: jax.nn.gelu(x.astype(f32), approximate=True).astype(bf16);
    x ** 3 lowers (integer_pow) to x * (x * x)."""
    xb, xf = _t((rows, cols), "bf16"), _t((rows, cols), "f32")

    def splat(name, val):
        return (f"    %{name} = stablehlo.constant dense<{val}> : tensor<f32>\n"
                f"    %{name}_b = stablehlo.broadcast_in_dim %{name}, dims = [] : (tensor<f32>) -> {xf}\n")
    return f"""module @jit_gelu attributes {{mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32}} {{
  func.func public @main(%arg0: {xb}) -> ({xb} {{jax.result_info = ""}}) {{
    %0 = stablehlo.convert %arg0 : ({xb}) -> {xf}
    %1 = stablehlo.multiply %0, %0 : {xf}
    %2 = stablehlo.multiply %0, %1 : {xf}
{splat("c0", "4.471500e-02")}    %3 = stablehlo.multiply %c0_b, %2 : {xf}
    %4 = stablehlo.add %0, %3 : {xf}
{splat("c1", "0.797884583")}    %5 = stablehlo.multiply %c1_b, %4 : {xf}
    %6 = stablehlo.tanh %5 : {xf}
{splat("c2", "1.000000e+00")}    %7 = stablehlo.add %c2_b, %6 : {xf}
{splat("c3", "5.000000e-01")}    %8 = stablehlo.multiply %c3_b, %7 : {xf}
    %9 = stablehlo.multiply %0, %8 : {xf}
    %10 = stablehlo.convert %9 : ({xf}) -> {xb}
    return %10 : {xb}
  }}
}}
"""


def reduce_sum(rows=65536, cols=1024) -> str:
    """C2c: x.astype(f32).sum(-1)."""
    xb, xf, r = _t((rows, cols), "bf16"), _t((rows, cols), "f32"), _t((rows,), "f32")
    return f"""module @jit_reduce_sum attributes {{mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32}} {{
  func.func public @main(%arg0: {xb}) -> ({r} {{jax.result_info = ""}}) {{
    %0 = stablehlo.convert %arg0 : ({xb}) -> {xf}
    %cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %1 = stablehlo.reduce(%0 init: %cst) applies stablehlo.add across dimensions = [1] : ({xf}, tensor<f32>) -> {r}
    return %1 : {r}
  }}
}}
"""


def argmax(rows=65536, cols=1024, is_min=False) -> str:
    """C2d: jnp.argmax(x, axis=-1) on bf16 -> i32: the variadic reduce over
    (x, iota) with the NaN-aware, lower-index-on-tie comparator JAX emits."""
    xb, ib = _t((rows, cols), "bf16"), _t((rows, cols), "i32")
    rv, ri = _t((rows,), "bf16"), _t((rows,), "i32")
    d = "LT" if is_min else "GT"
    init = "0x7F80" if is_min else "0xFF80"
    return f"""module @jit_argmax attributes {{mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32}} {{
  func.func public @main(%arg0: {xb}) -> ({ri} {{jax.result_info = ""}}) {{
    %0 = stablehlo.iota dim = 1 : {ib}
    %cst = stablehlo.constant dense<{init}> : tensor<bf16>
    %c = stablehlo.constant dense<0> : tensor<i32>
    %1:2 = stablehlo.reduce(%arg0 init: %cst), (%0 init: %c) across dimensions = [1] : ({xb}, {ib}, tensor<bf16>, tensor<i32>) -> ({rv}, {ri})
     reducer(%arg1: tensor<bf16>, %arg3: tensor<bf16>) (%arg2: tensor<i32>, %arg4: tensor<i32>)  {{
      %2 = stablehlo.compare  {d}, %arg1, %arg3,  FLOAT : (tensor<bf16>, tensor<bf16>) -> tensor<i1>
      %3 = stablehlo.compare  NE, %arg1, %arg1,  FLOAT : (tensor<bf16>, tensor<bf16>) -> tensor<i1>
      %4 = stablehlo.or %2, %3 : tensor<i1>
      %5 = stablehlo.compare  EQ, %arg1, %arg3,  FLOAT : (tensor<bf16>, tensor<bf16>) -> tensor<i1>
      %6 = stablehlo.compare  LT, %arg2, %arg4,  SIGNED : (tensor<i32>, tensor<i32>) -> tensor<i1>
      %7 = stablehlo.and %5, %6 : tensor<i1>
      %8 = stablehlo.or %4, %7 : tensor<i1>
      %9 = stablehlo.select %4, %arg1, %arg3 : tensor<i1>, tensor<bf16>
      %10 = stablehlo.select %8, %arg2, %arg4 : tensor<i1>, tensor<i32>
      stablehlo.return %9, %10 : tensor<bf16>, tensor<i32>
    }}
    return %1#1 : {ri}
  }}
}}
"""


def sdpa(b=4, h=16, s=8192, d=128, causal=True, mask_ops=None) -> str:
    """C3: s = einsum('bhqd,bhkd->bhqk', q, k) / sqrt(d) (bf16, the constant
    rounded to bf16); s = where(tril(ones((S, S), bool)), s, -inf);
    p = jax.nn.softmax(s, -1) (max, exp, sum in f32 via convert, divide);
    o = einsum('bhqk,bhkd->bhqd', p, v).

    ``mask_ops``: StableHLO lines that define ``%6``, the [b,h,s,s] i1 mask
    (any form), in place of the iota/compare causal mask."""
    q = _t((b, h, s, d), "bf16")
    sc = _t((b, h, s, s), "bf16")
    sf = _t((b, h, s, s), "f32")
    r3, r4 = _t((b, h, s), "bf16"), _t((b, h, s, 1), "bf16")
    r3f, r4f = _t((b, h, s), "f32"), _t((b, h, s, 1), "f32")
    m2, m4 = _t((s, s), "i1"), _t((b, h, s, s), "i1")
    i2 = _t((s, s), "i32")
    sqrt_d = float(d) ** 0.5
    mask = ""
    use = "%2"
    if mask_ops is not None:
        mask = mask_ops + f"""    %cst_1 = stablehlo.constant dense<0xFF80> : tensor<bf16>
    %7 = stablehlo.broadcast_in_dim %cst_1, dims = [] : (tensor<bf16>) -> {sc}
    %8 = stablehlo.select %6, %2, %7 : {m4}, {sc}
"""
        use = "%8"
    elif causal:
        mask = f"""    %3 = stablehlo.iota dim = 0 : {i2}
    %4 = stablehlo.iota dim = 1 : {i2}
    %5 = stablehlo.compare  GE, %3, %4,  SIGNED : ({i2}, {i2}) -> {m2}
    %6 = stablehlo.broadcast_in_dim %5, dims = [2, 3] : ({m2}) -> {m4}
    %cst_1 = stablehlo.constant dense<0xFF80> : tensor<bf16>
    %7 = stablehlo.broadcast_in_dim %cst_1, dims = [] : (tensor<bf16>) -> {sc}
    %8 = stablehlo.select %6, %2, %7 : {m4}, {sc}
"""
        use = "%8"
    return f"""module @jit_sdpa attributes {{mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32}} {{
  func.func public @main(%arg0: {q}, %arg1: {q}, %arg2: {q}) -> ({q} {{jax.result_info = ""}}) {{
    %0 = stablehlo.dot_general %arg0, %arg1, batching_dims = [0, 1] x [0, 1], contracting_dims = [3] x [3], precision = [DEFAULT, DEFAULT] : ({q}, {q}) -> {sc}
    %cst = stablehlo.constant dense<{sqrt_d:.6e}> : tensor<bf16>
    %1 = stablehlo.broadcast_in_dim %cst, dims = [] : (tensor<bf16>) -> {sc}
    %2 = stablehlo.divide %0, %1 : {sc}
{mask}    %cst_2 = stablehlo.constant dense<0xFF80> : tensor<bf16>
    %9 = stablehlo.reduce({use} init: %cst_2) applies stablehlo.maximum across dimensions = [3] : ({sc}, tensor<bf16>) -> {r3}
    %10 = stablehlo.broadcast_in_dim %cst_2, dims = [] : (tensor<bf16>) -> {r3}
    %11 = stablehlo.maximum %10, %9 : {r3}
    %12 = stablehlo.broadcast_in_dim %11, dims = [0, 1, 2] : ({r3}) -> {r4}
    %13 = stablehlo.broadcast_in_dim %12, dims = [0, 1, 2, 3] : ({r4}) -> {sc}
    %14 = stablehlo.subtract {use}, %13 : {sc}
    %15 = stablehlo.exponential %14 : {sc}
    %16 = stablehlo.convert %15 : ({sc}) -> {sf}
    %cst_3 = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %17 = stablehlo.reduce(%16 init: %cst_3) applies stablehlo.add across dimensions = [3] : ({sf}, tensor<f32>) -> {r3f}
    %18 = stablehlo.broadcast_in_dim %17, dims = [0, 1, 2] : ({r3f}) -> {r4f}
    %19 = stablehlo.convert %18 : ({r4f}) -> {r4}
    %20 = stablehlo.broadcast_in_dim %19, dims = [0, 1, 2, 3] : ({r4}) -> {sc}
    %21 = stablehlo.divide %15, %20 : {sc}
    %22 = stablehlo.dot_general %21, %arg2, batching_dims = [0, 1] x [0, 1], contracting_dims = [3] x [2], precision = [DEFAULT, DEFAULT] : ({sc}, {q}) -> {q}
    return %22 : {q}
  }}
}}
"""


def gather(ids=(32, 2048), vocab=50257, dim=768) -> str:
    """C4a: table[ids] (jnp indexing), bf16 rows; the index vector gets a
    trailing unit dim (index_vector_dim = rank)."""
    it, ie = _t(ids, "i32"), _t(tuple(ids) + (1,), "i32")
    tt, ot = _t((vocab, dim), "bf16"), _t(tuple(ids) + (dim,), "bf16")
    r = len(ids)
    return f"""module @jit_gather attributes {{mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32}} {{
  func.func public @main(%arg0: {tt}, %arg1: {it}) -> ({ot} {{jax.result_info = ""}}) {{
    %0 = stablehlo.broadcast_in_dim %arg1, dims = [{", ".join(str(i) for i in range(r))}] : ({it}) -> {ie}
    %1 = "stablehlo.gather"(%arg0, %0) <{{dimension_numbers = #stablehlo.gather<offset_dims = [{r}], collapsed_slice_dims = [0], start_index_map = [0], index_vector_dim = {r}>, indices_are_sorted = false, slice_sizes = array<i64: 1, {dim}>}}> : ({tt}, {ie}) -> {ot}
    return %1 : {ot}
  }}
}}
"""


def scatter_add(n=65536, vocab=50257, dim=768) -> str:
    """C4b: table.at[ids].add(grads) with FILL_OR_DROP, fp32."""
    tt, it, ie, ut = _t((vocab, dim), "f32"), _t((n,), "i32"), _t((n, 1), "i32"), _t((n, dim), "f32")
    return f"""module @jit_scatter_add attributes {{mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32}} {{
  func.func public @main(%arg0: {tt}, %arg1: {it}, %arg2: {ut}) -> ({tt} {{jax.result_info = ""}}) {{
    %0 = stablehlo.broadcast_in_dim %arg1, dims = [0] : ({it}) -> {ie}
    %1 = "stablehlo.scatter"(%arg0, %0, %arg2) <{{indices_are_sorted = false, scatter_dimension_numbers = #stablehlo.scatter<update_window_dims = [1], inserted_window_dims = [0], scatter_dims_to_operand_dims = [0], index_vector_dim = 1>, unique_indices = false}}> ({{
    ^bb0(%arg3: tensor<f32>, %arg4: tensor<f32>):
      %2 = stablehlo.add %arg3, %arg4 : tensor<f32>
      stablehlo.return %2 : tensor<f32>
    }}) : ({tt}, {ie}, {ut}) -> {tt}
    return %1 : {tt}
  }}
}}
"""


ALL = {"mlp": mlp, "layernorm": layernorm, "gelu": gelu, "reduce_sum": reduce_sum,
       "argmax": argmax, "sdpa": sdpa, "gather": gather, "scatter_add": scatter_add}


def adam_update(n=1 << 20, b1=0.9, b2=0.999, eps=1e-8) -> str:
    """The per-parameter Adam update of temp/dp_train.py:71-75 as its own
    jit with the state donated, ``jax.jit(upd, donate_argnums=(0, 1, 2))``:
    upd(p, m, v, g, bc1, bc2, lr) -> (p - lr (m'/bc1) / (sqrt(v'/bc2) + eps),
    m' = b1 m + (1-b1) g, v' = b2 v + (1-b2) g g).  JAX marks each donated
    argument with the output it aliases (``tf.aliasing_output``); the
    Python-float constants fold to f32."""
    t, s = _t((n,), "f32"), "tensor<f32>"

    def c(x):
        return f"{float(x):.9e}"

    def bc(v):
        return f"stablehlo.broadcast_in_dim {v}, dims = [] : ({s}) -> {t}"
    return f"""module @jit_upd attributes {{mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32}} {{
  func.func public @main(%arg0: {t} {{tf.aliasing_output = 0 : i32}}, %arg1: {t} {{tf.aliasing_output = 1 : i32}}, %arg2: {t} {{tf.aliasing_output = 2 : i32}}, %arg3: {t}, %arg4: {s}, %arg5: {s}, %arg6: {s}) -> ({t} {{jax.result_info = "[0]"}}, {t} {{jax.result_info = "[1]"}}, {t} {{jax.result_info = "[2]"}}) {{
    %cst = stablehlo.constant dense<{c(b1)}> : {s}
    %0 = {bc("%cst")}
    %1 = stablehlo.multiply %0, %arg1 : {t}
    %cst_0 = stablehlo.constant dense<{c(1 - b1)}> : {s}
    %2 = {bc("%cst_0")}
    %3 = stablehlo.multiply %2, %arg3 : {t}
    %4 = stablehlo.add %1, %3 : {t}
    %cst_1 = stablehlo.constant dense<{c(b2)}> : {s}
    %5 = {bc("%cst_1")}
    %6 = stablehlo.multiply %5, %arg2 : {t}
    %cst_2 = stablehlo.constant dense<{c(1 - b2)}> : {s}
    %7 = {bc("%cst_2")}
    %8 = stablehlo.multiply %7, %arg3 : {t}
    %9 = stablehlo.multiply %8, %arg3 : {t}
    %10 = stablehlo.add %6, %9 : {t}
    %11 = {bc("%arg4")}
    %12 = stablehlo.divide %4, %11 : {t}
    %13 = {bc("%arg6")}
    %14 = stablehlo.multiply %13, %12 : {t}
    %15 = {bc("%arg5")}
    %16 = stablehlo.divide %10, %15 : {t}
    %17 = stablehlo.sqrt %16 : {t}
    %cst_3 = stablehlo.constant dense<{c(eps)}> : {s}
    %18 = {bc("%cst_3")}
    %19 = stablehlo.add %17, %18 : {t}
    %20 = stablehlo.divide %14, %19 : {t}
    %21 = stablehlo.subtract %arg0, %20 : {t}
    return %21, %4, %10 : {t}, {t}, {t}
  }}
}}
"""


def donated(kind: str, n=64) -> str:
    """Small donation cases: 'matmul' (x @ w with x donated: the GEMM reads
    x while writing, so no in-place alias), 'transpose_add' (x.T + y with x
    donated: read in another layout), 'donor_add' (x + y with x marked
    ``jax.buffer_donor``: output chosen by type, in place)."""
    t = _t((n, n), "f32")
    if kind == "matmul":
        body = f"%0 = stablehlo.dot_general %arg0, %arg1, contracting_dims = [1] x [0] : ({t}, {t}) -> {t}"
        attr = "{tf.aliasing_output = 0 : i32}"
    elif kind == "transpose_add":
        body = (f"%t = stablehlo.transpose %arg0, dims = [1, 0] : ({t}) -> {t}\n"
                f"    %0 = stablehlo.add %t, %arg1 : {t}")
        attr = "{tf.aliasing_output = 0 : i32}"
    elif kind == "donor_add":
        body = f"%0 = stablehlo.add %arg0, %arg1 : {t}"
        attr = "{jax.buffer_donor = true}"
    else:
        raise ValueError(kind)
    return f"""module @jit_donated attributes {{mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32}} {{
  func.func public @main(%arg0: {t} {attr}, %arg1: {t}) -> ({t} {{jax.result_info = ""}}) {{
    {body}
    return %0 : {t}
  }}
}}
"""
