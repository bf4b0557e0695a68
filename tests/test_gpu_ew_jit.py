"""Generated elementwise kernels (jam's ew steps compiled with hiprtc at the
first run) against the register-program interpreter they replace: the same
module compiled with and without them (env JAM_NO_EW_JIT) must give the same
bits on every output, over every opcode the lowering emits, every element
type, dense / broadcast / transposed operands, inner dims that do and do not
take the 4-lane vector form, and inputs holding NaN, infinities, signed
zeros, subnormals and integer extremes.  The interpreter itself is pinned
against the CPU oracle by the other GPU tests.  JAM_EW_JIT_STRICT makes any
fallback to the interpreter an error, so the generated kernels are what runs."""

import os

import numpy as np
import pytest

from mi355x_pjrt import gpt2, pjrt, train_hlo
from test_gpu_pjrt import client  # noqa: F401  (fixture)

pytestmark = pytest.mark.gpu


def run_both(client, text, args):
    """Outputs of `text` on `args` with generated kernels (strict) and with
    the interpreter; also returns the plan of the first."""
    res, plans = [], []
    for env in ({"JAM_EW_JIT_STRICT": "1"}, {"JAM_NO_EW_JIT": "1"}):
        saved = {k: os.environ.pop(k, None) for k in ("JAM_EW_JIT_STRICT", "JAM_NO_EW_JIT")}
        os.environ.update(env)
        try:
            e = client.compile(text)
        finally:
            for k in env:
                del os.environ[k]
            for k, v in saved.items():
                if v is not None:
                    os.environ[k] = v
        plans.append(e.plan())
        bufs = [client.put(a, code) for a, code in args]
        outs = e.execute(bufs)
        res.append([o.to_numpy() for o in outs])
        for b in bufs + outs:
            b.destroy()
        e.destroy()
    assert "ew_jit" in plans[0] and "ew_jit" not in plans[1]
    return res[0], res[1], plans[0]


def assert_same_bits(a, b, inputs=()):
    """Outputs equal byte for byte; on a mismatch the first few differing
    elements are listed (as bit patterns, with the inputs there)."""
    assert len(a) == len(b)
    for k, (x, y) in enumerate(zip(a, b)):
        x, y = np.asarray(x), np.asarray(y)
        assert x.dtype == y.dtype and x.shape == y.shape, k
        xb, yb = x.reshape(-1).view(np.uint8), y.reshape(-1).view(np.uint8)
        if np.array_equal(xb, yb):
            continue
        w = x.dtype.itemsize
        bad = np.nonzero((xb != yb).reshape(-1, w).any(axis=1))[0]
        lines = []
        for i in bad[:8]:
            ins = " ".join(f"{np.asarray(v).reshape(-1)[i]!r}" for v in inputs if np.asarray(v).size == x.size)
            lines.append(f"  [{i}] jit {x.reshape(-1)[i]!r} ({xb.reshape(-1, w)[i].tobytes()[::-1].hex()}) "
                         f"interp {y.reshape(-1)[i]!r} ({yb.reshape(-1, w)[i].tobytes()[::-1].hex()}) in {ins}")
        raise AssertionError(f"output {k}: {bad.size} of {x.size} elements differ\n" + "\n".join(lines))


def special_f32(rng, shape):
    x = (rng.standard_normal(shape) * 3).astype(np.float32)
    flat = x.reshape(-1)
    sp = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40, -1e-40, 3e38, -3e38, 1.0, -1.0, 0.5, 88.0, -104.0,
                   2.5, -2.5], np.float32)
    idx = rng.choice(flat.size, size=min(flat.size, 4 * sp.size), replace=False)
    flat[idx] = np.resize(sp, idx.size)
    return x


FLOAT_MODULE = """func.func public @main(%x: tensor<64x36xf32>, %y: tensor<64x36xf32>, %b: tensor<36xf32>,
    %r: tensor<64xf32>, %t: tensor<36x64xf32>, %h: tensor<64x36xbf16>, %g: tensor<64x36xf16>)
    -> (tensor<64x36xf32>, tensor<64x36xf32>, tensor<64x36xbf16>, tensor<64x36xf16>, tensor<64x36xi1>,
        tensor<64x36xf32>, tensor<64x36xf32>) {
  %bb = stablehlo.broadcast_in_dim %b, dims = [1] : (tensor<36xf32>) -> tensor<64x36xf32>
  %rb = stablehlo.broadcast_in_dim %r, dims = [0] : (tensor<64xf32>) -> tensor<64x36xf32>
  %tt = stablehlo.transpose %t, dims = [1, 0] : (tensor<36x64xf32>) -> tensor<64x36xf32>
  %hf = stablehlo.convert %h : (tensor<64x36xbf16>) -> tensor<64x36xf32>
  %gf = stablehlo.convert %g : (tensor<64x36xf16>) -> tensor<64x36xf32>
  %a1 = stablehlo.add %x, %bb : tensor<64x36xf32>
  %a2 = stablehlo.multiply %a1, %rb : tensor<64x36xf32>
  %a3 = stablehlo.subtract %a2, %tt : tensor<64x36xf32>
  %a4 = stablehlo.divide %a3, %y : tensor<64x36xf32>
  %ax = stablehlo.abs %x : tensor<64x36xf32>
  %ay = stablehlo.abs %y : tensor<64x36xf32>
  %e = stablehlo.exponential %x : tensor<64x36xf32>
  %l = stablehlo.log %ay : tensor<64x36xf32>
  %th = stablehlo.tanh %a4 : tensor<64x36xf32>
  %sq = stablehlo.sqrt %ax : tensor<64x36xf32>
  %rs = stablehlo.rsqrt %ay : tensor<64x36xf32>
  %lg = stablehlo.logistic %a3 : tensor<64x36xf32>
  %pw = stablehlo.power %ax, %y : tensor<64x36xf32>
  %mx = stablehlo.maximum %a4, %e : tensor<64x36xf32>
  %mn = stablehlo.minimum %mx, %th : tensor<64x36xf32>
  %s1 = stablehlo.add %mn, %l : tensor<64x36xf32>
  %s2 = stablehlo.add %sq, %rs : tensor<64x36xf32>
  %s3 = stablehlo.multiply %lg, %pw : tensor<64x36xf32>
  %o0 = stablehlo.add %s1, %s2 : tensor<64x36xf32>
  %fl = stablehlo.floor %a3 : tensor<64x36xf32>
  %ce = stablehlo.ceil %a4 : tensor<64x36xf32>
  %sg = stablehlo.sign %x : tensor<64x36xf32>
  %ng = stablehlo.negate %hf : tensor<64x36xf32>
  %c = stablehlo.compare GT, %x, %y, FLOAT : (tensor<64x36xf32>, tensor<64x36xf32>) -> tensor<64x36xi1>
  %c2 = stablehlo.compare LE, %hf, %gf, FLOAT : (tensor<64x36xf32>, tensor<64x36xf32>) -> tensor<64x36xi1>
  %c3 = stablehlo.compare EQ, %x, %tt, FLOAT : (tensor<64x36xf32>, tensor<64x36xf32>) -> tensor<64x36xi1>
  %c4 = stablehlo.compare NE, %y, %bb, FLOAT : (tensor<64x36xf32>, tensor<64x36xf32>) -> tensor<64x36xi1>
  %sel = stablehlo.select %c, %fl, %ce : tensor<64x36xi1>, tensor<64x36xf32>
  %cl = stablehlo.clamp %rb, %sel, %bb : (tensor<64x36xf32>, tensor<64x36xf32>, tensor<64x36xf32>) -> tensor<64x36xf32>
  %o1 = stablehlo.add %cl, %sg : tensor<64x36xf32>
  %o2 = stablehlo.convert %o0 : (tensor<64x36xf32>) -> tensor<64x36xbf16>
  %m3 = stablehlo.multiply %ng, %gf : tensor<64x36xf32>
  %o3 = stablehlo.convert %m3 : (tensor<64x36xf32>) -> tensor<64x36xf16>
  %p1 = stablehlo.and %c2, %c3 : tensor<64x36xi1>
  %p2 = stablehlo.or %p1, %c4 : tensor<64x36xi1>
  %p3 = stablehlo.not %c : tensor<64x36xi1>
  %o4 = stablehlo.xor %p2, %p3 : tensor<64x36xi1>
  %o5 = stablehlo.add %s3, %a1 : tensor<64x36xf32>
  %ge = stablehlo.compare GE, %a3, %tt, FLOAT : (tensor<64x36xf32>, tensor<64x36xf32>) -> tensor<64x36xi1>
  %lt = stablehlo.compare LT, %x, %rb, FLOAT : (tensor<64x36xf32>, tensor<64x36xf32>) -> tensor<64x36xi1>
  %q1 = stablehlo.select %ge, %x, %hf : tensor<64x36xi1>, tensor<64x36xf32>
  %q2 = stablehlo.select %lt, %q1, %gf : tensor<64x36xi1>, tensor<64x36xf32>
  %o6 = stablehlo.multiply %q2, %e : tensor<64x36xf32>
  return %o0, %o1, %o2, %o3, %o4, %o5, %o6 : tensor<64x36xf32>, tensor<64x36xf32>, tensor<64x36xbf16>,
      tensor<64x36xf16>, tensor<64x36xi1>, tensor<64x36xf32>, tensor<64x36xf32>
}"""


def test_float_opcodes_and_layouts(client):
    rng = np.random.default_rng(11)
    from oracle import bf16

    x, y = special_f32(rng, (64, 36)), special_f32(rng, (64, 36))
    args = [(x, None), (y, None), (special_f32(rng, (36,)), None), (special_f32(rng, (64,)), None),
            (special_f32(rng, (36, 64)), None),
            (bf16.to_bf16_bits(special_f32(rng, (64, 36))), pjrt.BF16),
            (special_f32(rng, (64, 36)).astype(np.float16), None)]
    print("case: ew jit float opcodes [64,36]", flush=True)
    a, b, plan = run_both(client, FLOAT_MODULE, args)
    assert_same_bits(a, b, [v for v, _ in args])


def _odd(text):
    """The float module on a [5,7] shape (inner dim not a multiple of 4: the
    one-element-per-thread form)."""
    return (text.replace("64x36", "5x7").replace("36x64", "7x5").replace("tensor<36x", "tensor<7x")
            .replace("tensor<36xf32>", "tensor<7xf32>").replace("tensor<64xf32>", "tensor<5xf32>"))


def test_float_opcodes_odd_inner_dim(client):
    rng = np.random.default_rng(12)
    from oracle import bf16

    args = [(special_f32(rng, (5, 7)), None), (special_f32(rng, (5, 7)), None), (special_f32(rng, (7,)), None),
            (special_f32(rng, (5,)), None), (special_f32(rng, (7, 5)), None),
            (bf16.to_bf16_bits(special_f32(rng, (5, 7))), pjrt.BF16),
            (special_f32(rng, (5, 7)).astype(np.float16), None)]
    print("case: ew jit float opcodes [5,7]", flush=True)
    a, b, _ = run_both(client, _odd(FLOAT_MODULE), args)
    assert_same_bits(a, b, [v for v, _ in args])


INT_MODULE = """func.func public @main(%a: tensor<8x12xi32>, %b: tensor<8x12xi32>, %c: tensor<12xi32>,
    %d: tensor<8x12xi8>, %e: tensor<8x12xui8>, %f: tensor<8x12xi16>, %g: tensor<8x12xui16>, %h: tensor<8x12xi64>)
    -> (tensor<8x12xi32>, tensor<8x12xi32>, tensor<8x12xf32>, tensor<8x12xi32>, tensor<8x12xi8>,
        tensor<8x12xi16>, tensor<8x12xi64>, tensor<8x12xui32>, tensor<8x12xf32>, tensor<8x12xi32>) {
  %cb = stablehlo.broadcast_in_dim %c, dims = [1] : (tensor<12xi32>) -> tensor<8x12xi32>
  %s = stablehlo.add %a, %b : tensor<8x12xi32>
  %m = stablehlo.multiply %s, %cb : tensor<8x12xi32>
  %d1 = stablehlo.subtract %m, %a : tensor<8x12xi32>
  %mx = stablehlo.maximum %d1, %b : tensor<8x12xi32>
  %mn = stablehlo.minimum %mx, %cb : tensor<8x12xi32>
  %ng = stablehlo.negate %mn : tensor<8x12xi32>
  %an = stablehlo.and %ng, %a : tensor<8x12xi32>
  %o = stablehlo.or %an, %b : tensor<8x12xi32>
  %o0 = stablehlo.xor %o, %cb : tensor<8x12xi32>
  %lt = stablehlo.compare LT, %a, %b, SIGNED : (tensor<8x12xi32>, tensor<8x12xi32>) -> tensor<8x12xi1>
  %ge = stablehlo.compare GE, %a, %cb, SIGNED : (tensor<8x12xi32>, tensor<8x12xi32>) -> tensor<8x12xi1>
  %eq = stablehlo.compare EQ, %b, %cb, SIGNED : (tensor<8x12xi32>, tensor<8x12xi32>) -> tensor<8x12xi1>
  %ne = stablehlo.compare NE, %a, %s, SIGNED : (tensor<8x12xi32>, tensor<8x12xi32>) -> tensor<8x12xi1>
  %le = stablehlo.compare LE, %m, %a, SIGNED : (tensor<8x12xi32>, tensor<8x12xi32>) -> tensor<8x12xi1>
  %gt = stablehlo.compare GT, %d1, %b, SIGNED : (tensor<8x12xi32>, tensor<8x12xi32>) -> tensor<8x12xi1>
  %p1 = stablehlo.and %lt, %ge : tensor<8x12xi1>
  %p2 = stablehlo.or %p1, %eq : tensor<8x12xi1>
  %p3 = stablehlo.xor %p2, %ne : tensor<8x12xi1>
  %p4 = stablehlo.or %le, %gt : tensor<8x12xi1>
  %p5 = stablehlo.and %p3, %p4 : tensor<8x12xi1>
  %o1 = stablehlo.select %p5, %a, %m : tensor<8x12xi1>, tensor<8x12xi32>
  %o2 = stablehlo.convert %o0 : (tensor<8x12xi32>) -> tensor<8x12xf32>
  %fx = stablehlo.convert %o2 : (tensor<8x12xf32>) -> tensor<8x12xi32>
  %p6 = stablehlo.convert %p5 : (tensor<8x12xi1>) -> tensor<8x12xi32>
  %o3 = stablehlo.add %fx, %p6 : tensor<8x12xi32>
  %dd = stablehlo.convert %d : (tensor<8x12xi8>) -> tensor<8x12xi32>
  %ee = stablehlo.convert %e : (tensor<8x12xui8>) -> tensor<8x12xi32>
  %ff = stablehlo.convert %f : (tensor<8x12xi16>) -> tensor<8x12xi32>
  %gg = stablehlo.convert %g : (tensor<8x12xui16>) -> tensor<8x12xi32>
  %hh = stablehlo.convert %h : (tensor<8x12xi64>) -> tensor<8x12xi32>
  %t1 = stablehlo.add %dd, %ee : tensor<8x12xi32>
  %t2 = stablehlo.add %ff, %gg : tensor<8x12xi32>
  %t3 = stablehlo.add %t1, %t2 : tensor<8x12xi32>
  %t4 = stablehlo.multiply %t3, %hh : tensor<8x12xi32>
  %o4 = stablehlo.convert %t4 : (tensor<8x12xi32>) -> tensor<8x12xi8>
  %o5 = stablehlo.convert %t4 : (tensor<8x12xi32>) -> tensor<8x12xi16>
  %o6 = stablehlo.convert %t4 : (tensor<8x12xi32>) -> tensor<8x12xi64>
  %o7 = stablehlo.convert %t3 : (tensor<8x12xi32>) -> tensor<8x12xui32>
  %u = stablehlo.convert %o7 : (tensor<8x12xui32>) -> tensor<8x12xf32>
  %o8 = stablehlo.multiply %u, %o2 : tensor<8x12xf32>
  %nz = stablehlo.compare NE, %t4, %cb, SIGNED : (tensor<8x12xi32>, tensor<8x12xi32>) -> tensor<8x12xi1>
  %o9 = stablehlo.convert %nz : (tensor<8x12xi1>) -> tensor<8x12xi32>
  return %o0, %o1, %o2, %o3, %o4, %o5, %o6, %o7, %o8, %o9 : tensor<8x12xi32>, tensor<8x12xi32>, tensor<8x12xf32>,
      tensor<8x12xi32>, tensor<8x12xi8>, tensor<8x12xi16>, tensor<8x12xi64>, tensor<8x12xui32>, tensor<8x12xf32>,
      tensor<8x12xi32>
}"""


def test_integer_opcodes_and_types(client):
    rng = np.random.default_rng(13)
    ext = np.array([2 ** 31 - 1, -2 ** 31, 0, -1, 1, 65536, -65537], np.int64)

    def i32(shape):
        v = rng.integers(-2 ** 31, 2 ** 31, shape, dtype=np.int64)
        v.reshape(-1)[: ext.size] = ext[: v.size]
        return v.astype(np.int32)

    args = [(i32((8, 12)), None), (i32((8, 12)), None), (i32((12,)), None),
            (rng.integers(-128, 128, (8, 12)).astype(np.int8), None),
            (rng.integers(0, 256, (8, 12)).astype(np.uint8), None),
            (rng.integers(-2 ** 15, 2 ** 15, (8, 12)).astype(np.int16), None),
            (rng.integers(0, 2 ** 16, (8, 12)).astype(np.uint16), None),
            (rng.integers(-2 ** 40, 2 ** 40, (8, 12)).astype(np.int64), None)]
    print("case: ew jit integer opcodes [8,12]", flush=True)
    a, b, _ = run_both(client, INT_MODULE, args)
    assert_same_bits(a, b)


RANK4_MODULE = """func.func public @main(%x: tensor<3x8x5x4xf32>, %y: tensor<4x5x3x8xbf16>, %s: tensor<f32>)
    -> (tensor<3x8x5x4xf32>, tensor<3x8x5x4xbf16>) {
  %yt = stablehlo.transpose %y, dims = [2, 3, 1, 0] : (tensor<4x5x3x8xbf16>) -> tensor<3x8x5x4xbf16>
  %yf = stablehlo.convert %yt : (tensor<3x8x5x4xbf16>) -> tensor<3x8x5x4xf32>
  %sb = stablehlo.broadcast_in_dim %s, dims = [] : (tensor<f32>) -> tensor<3x8x5x4xf32>
  %m = stablehlo.multiply %x, %yf : tensor<3x8x5x4xf32>
  %o0 = stablehlo.add %m, %sb : tensor<3x8x5x4xf32>
  %t = stablehlo.tanh %o0 : tensor<3x8x5x4xf32>
  %o1 = stablehlo.convert %t : (tensor<3x8x5x4xf32>) -> tensor<3x8x5x4xbf16>
  return %o0, %o1 : tensor<3x8x5x4xf32>, tensor<3x8x5x4xbf16>
}"""


def test_rank4_transposed_bf16_and_scalar(client):
    """A transposed bf16 operand (inner stride not 1: four scalar loads per
    thread) and a rank-0 operand broadcast to every element."""
    rng = np.random.default_rng(14)
    from oracle import bf16

    args = [(special_f32(rng, (3, 8, 5, 4)), None), (bf16.to_bf16_bits(special_f32(rng, (4, 5, 3, 8))), pjrt.BF16),
            (np.float32(0.375), None)]
    print("case: ew jit rank-4 transposed bf16", flush=True)
    a, b, _ = run_both(client, RANK4_MODULE, args)
    assert_same_bits(a, b)


def test_reduced_c5_training_step(client):
    """Forward, backward and Adam of the reduced GPT-2 step against the
    interpreter's run of the same module: the elementwise work is bitwise
    the interpreter's, but reductions of elementwise values run fused in
    generated kernels with their own summation order, so each output is
    compared within 1e-4 of its largest magnitude (loss within 1e-6)."""
    cfg = gpt2.GPT2Config(n_layer=2, d_model=128, n_head=2, seq=128, batch=2, vocab=257)
    print("case: ew jit reduced C5 training step", flush=True)
    params = gpt2.init_params(cfg, 4)
    names = [n for n, _ in cfg.param_shapes()]
    rng = np.random.default_rng(5)
    ids = rng.integers(0, cfg.vocab, (cfg.batch, cfg.seq)).astype(np.int32)
    labels = rng.integers(0, cfg.vocab, (cfg.batch, cfg.seq)).astype(np.int32)
    m0 = [(rng.standard_normal(params[n].shape) * 1e-3).astype(np.float32) for n in names]
    v0 = [(rng.random(params[n].shape) * 1e-6).astype(np.float32) for n in names]
    host = [params[n] for n in names] + m0 + v0 + [ids, labels, np.float32(1e-3), np.float32(1 / (1 - 0.9 ** 3)),
                                                   np.float32(1 / (1 - 0.999 ** 3))]
    a, b, plan = run_both(client, train_hlo.gpt2_train_step(cfg), [(np.asarray(h), None) for h in host])
    assert " ew_jit " in plan and "ew_reduce" in plan
    assert abs(float(a[0]) - float(b[0])) <= 1e-6 * abs(float(b[0]))
    for k, (x, y) in enumerate(zip(a[1:], b[1:])):
        assert np.max(np.abs(x - y)) <= 1e-4 * np.max(np.abs(y)) + 1e-30, k


UNARY = ["exponential", "log", "tanh", "sqrt", "rsqrt", "logistic", "floor", "ceil", "sign", "abs", "negate"]
BINARY = ["add", "subtract", "multiply", "divide", "power", "maximum", "minimum"]


@pytest.mark.parametrize("op", UNARY + BINARY)
def test_each_float_op(client, op):
    """One operation at a time on [64,36] f32 inputs with special values."""
    rng = np.random.default_rng(15)
    x, y = special_f32(rng, (64, 36)), special_f32(rng, (64, 36))
    if op in UNARY:
        body = f"%o = stablehlo.{op} %x : tensor<64x36xf32>"
    else:
        body = f"%o = stablehlo.{op} %x, %y : tensor<64x36xf32>"
    text = f"""func.func public @main(%x: tensor<64x36xf32>, %y: tensor<64x36xf32>) -> tensor<64x36xf32> {{
  {body}
  return %o : tensor<64x36xf32>
}}"""
    print(f"case: ew jit single op {op}", flush=True)
    a, b, _ = run_both(client, text, [(x, None), (y, None)])
    assert_same_bits(a, b, (x, y))


def _reduce_module(shape, rdims, body, vtype="f32", otype="f32", kind="add", init="0.000000e+00"):
    """reduce(body(x, y)) over rdims; x, y f32 of `shape`."""
    keep = [d for d in range(len(shape)) if d not in rdims]
    st = "x".join(str(d) for d in shape)
    ot = "x".join(str(shape[d]) for d in keep)
    ot_t = f"tensor<{ot}x{otype}>" if keep else f"tensor<{otype}>"
    return f"""func.func public @main(%x: tensor<{st}xf32>, %y: tensor<{st}xf32>) -> {ot_t} {{
  {body}
  %v = stablehlo.convert %e : (tensor<{st}xf32>) -> tensor<{st}x{vtype}>
  %z = stablehlo.constant dense<{init}> : tensor<{vtype}>
  %r = stablehlo.reduce(%v init: %z) applies stablehlo.{kind} across dimensions = {rdims} : (tensor<{st}x{vtype}>, tensor<{vtype}>) -> tensor<{ot if keep else ""}{"x" if keep else ""}{vtype}>
  %o = stablehlo.convert %r : (tensor<{ot if keep else ""}{"x" if keep else ""}{vtype}>) -> {ot_t}
  return %o : {ot_t}
}}"""


REDUCE_CASES = {
    # rows of a product (layer-norm statistics): one wave per row, 4-wide
    "row_sum": ((64, 768), [1], "%e = stablehlo.multiply %x, %y : tensor<64x768xf32>", "f32", "add"),
    # odd row length: one element per lane
    "row_sum_odd": ((33, 101), [1], "%e = stablehlo.multiply %x, %y : tensor<33x101xf32>", "f32", "add"),
    # max with NaN inputs propagates NaN
    "row_max": ((40, 256), [1], "%e = stablehlo.subtract %x, %y : tensor<40x256xf32>", "f32", "maximum"),
    # sum over the leading dims (bias / gamma gradients): column partials
    "col_sum": ((6, 512, 768), [0, 1], "%e = stablehlo.multiply %x, %y : tensor<6x512x768xf32>", "f32", "add"),
    "col_sum_odd": ((300, 37), [0], "%e = stablehlo.add %x, %y : tensor<300x37xf32>", "f32", "add"),
    # a middle dim (strided after moving it last)
    "mid_sum": ((8, 96, 20), [1], "%e = stablehlo.multiply %x, %y : tensor<8x96x20xf32>", "f32", "add"),
    # bf16 value: rounded before it is summed
    "row_sum_bf16": ((32, 512), [1], "%e = stablehlo.multiply %x, %y : tensor<32x512xf32>", "bf16", "add"),
}


@pytest.mark.parametrize("case", sorted(REDUCE_CASES))
def test_fused_reduction_of_elementwise_value(client, case):
    """A reduction whose operand is an elementwise value read by nothing
    else runs as one generated kernel (ew_reduce) that evaluates the value
    where it reads it.  Against the float64 reduction of the value (rounded
    to its type first): within 1e-6 of the sum of magnitudes (sums), exact
    (max), NaN where the reference has NaN."""
    shape, rdims, body, vtype, kind = REDUCE_CASES[case]
    rng = np.random.default_rng(31)
    x = rng.standard_normal(shape).astype(np.float32)
    y = rng.standard_normal(shape).astype(np.float32)
    if kind == "maximum":
        x.reshape(-1)[::97] = np.nan
    init = "0xFF800000" if kind == "maximum" else "0.000000e+00"
    text = _reduce_module(shape, rdims, body, vtype, "f32", kind, init)
    print(f"case: ew_reduce {case}", flush=True)
    saved = os.environ.pop("JAM_NO_EW_JIT", None)
    os.environ["JAM_EW_JIT_STRICT"] = "1"
    try:
        e = client.compile(text)
    finally:
        del os.environ["JAM_EW_JIT_STRICT"]
        if saved is not None:
            os.environ["JAM_NO_EW_JIT"] = saved
    assert "ew_reduce" in e.plan()
    bufs = [client.put(x), client.put(y)]
    (out,) = e.execute(bufs)
    got = out.to_numpy()
    for b in bufs + [out]:
        b.destroy()
    e.destroy()
    op = {"multiply": np.multiply, "subtract": np.subtract, "add": np.add}[body.split("stablehlo.")[1].split(" ")[0]]
    v = op(x, y).astype(np.float32)
    if vtype == "bf16":
        from oracle import bf16
        v = bf16.round_bf16(v)
    axes = tuple(rdims)
    if kind == "maximum":
        want = np.max(v.astype(np.float64), axis=axes)
        np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
        ok = ~np.isnan(want)
        np.testing.assert_array_equal(got[ok], want[ok].astype(np.float32))
    else:
        want = np.sum(v.astype(np.float64), axis=axes)
        mag = np.sum(np.abs(v).astype(np.float64), axis=axes)
        # a bf16 reduce result is rounded to bf16 once (half an ulp: at most
        # 2^-8 of its magnitude)
        out_round = 2.0 ** -8 * np.abs(want) if vtype == "bf16" else 0
        bad = np.abs(got - want) > 1e-6 * mag + out_round + 1e-30
        assert not bad.any(), (case, got[bad][:4], want[bad][:4], mag[bad][:4])


@pytest.mark.parametrize("shape,rdims", [((64, 768), [1]), ((33, 101), [1]), ((6, 512, 768), [0, 1]),
                                         ((300, 37), [0])])
def test_fused_reduction_stores_a_shared_value(client, shape, rdims):
    """A reduced elementwise value that other ops also read is stored by the
    reduction's kernel in the same pass (ew_reduce, value stored): the
    stored value exactly the f32 product, the sum within 1e-6 of the sum of
    magnitudes, and its other reader (here a second output) sees it."""
    st = "x".join(str(d) for d in shape)
    keep = [d for d in range(len(shape)) if d not in rdims]
    ot = "x".join(str(shape[d]) for d in keep)
    text = f"""func.func public @main(%x: tensor<{st}xf32>, %y: tensor<{st}xf32>) -> (tensor<{ot}xf32>, tensor<{st}xf32>) {{
  %e = stablehlo.multiply %x, %y : tensor<{st}xf32>
  %z = stablehlo.constant dense<0.000000e+00> : tensor<f32>
  %r = stablehlo.reduce(%e init: %z) applies stablehlo.add across dimensions = {rdims} : (tensor<{st}xf32>, tensor<f32>) -> tensor<{ot}xf32>
  %two = stablehlo.constant dense<2.000000e+00> : tensor<{st}xf32>
  %d = stablehlo.multiply %e, %two : tensor<{st}xf32>
  return %r, %d : tensor<{ot}xf32>, tensor<{st}xf32>
}}"""
    rng = np.random.default_rng(32)
    x = rng.standard_normal(shape).astype(np.float32)
    y = rng.standard_normal(shape).astype(np.float32)
    print(f"case: ew_reduce stored value {shape} over {rdims}", flush=True)
    os.environ["JAM_EW_JIT_STRICT"] = "1"
    try:
        e = client.compile(text)
    finally:
        del os.environ["JAM_EW_JIT_STRICT"]
    assert "value stored" in e.plan()
    bufs = [client.put(x), client.put(y)]
    outs = e.execute(bufs)
    r, d = (o.to_numpy() for o in outs)
    for b in bufs + outs:
        b.destroy()
    e.destroy()
    v = x * y
    np.testing.assert_array_equal(d, v * np.float32(2))
    want = np.sum(v.astype(np.float64), axis=tuple(rdims))
    mag = np.sum(np.abs(v).astype(np.float64), axis=tuple(rdims))
    assert np.all(np.abs(r - want) <= 1e-6 * mag + 1e-30)


def test_sum_of_a_product_also_rounded_to_bf16(client):
    """A bf16 product with an f32 result that is both rounded to bf16 and
    summed: the sum is of the f32 values (within 1e-5 of the float64 sum of
    the products, scaled by magnitudes), the rounded copy RNE of them."""
    from oracle import bf16
    from test_pjrt_cpu import SUM_AND_ROUND

    rng = np.random.default_rng(33)
    a = bf16.round_bf16(rng.standard_normal((256, 128)).astype(np.float32))
    b = bf16.round_bf16(rng.standard_normal((128, 256)).astype(np.float32))
    print("case: product summed and rounded", flush=True)
    e = client.compile(SUM_AND_ROUND)
    bufs = [client.put(bf16.to_bf16_bits(a), pjrt.BF16), client.put(bf16.to_bf16_bits(b), pjrt.BF16)]
    outs = e.execute(bufs)
    z, s = (o.to_numpy() for o in outs)
    for x in bufs + outs:
        x.destroy()
    e.destroy()
    y = a.astype(np.float64) @ b
    mag = np.abs(a).astype(np.float64) @ np.abs(b)
    want = y.sum(axis=0)
    assert np.all(np.abs(s - want) <= 1e-5 * mag.sum(axis=0))
    zf = bf16.from_bf16_bits(z).astype(np.float64)
    assert np.all(np.abs(zf - y) <= 2.0 ** -8 * np.abs(y) + 1e-5 * mag)


@pytest.mark.parametrize("shape,rdims", [((64, 768), [1]), ((6, 512, 768), [0, 1])])
def test_fused_reduction_stores_a_bf16_copy(client, shape, rdims):
    """The value's other readers only convert it to bf16: the reduction's
    kernel stores just that bf16 copy (its f32 form is never written) and
    sums the exact f32 values."""
    from oracle import bf16

    st = "x".join(str(d) for d in shape)
    keep = [d for d in range(len(shape)) if d not in rdims]
    ot = "x".join(str(shape[d]) for d in keep)
    text = f"""func.func public @main(%x: tensor<{st}xf32>, %y: tensor<{st}xf32>) -> (tensor<{ot}xf32>, tensor<{st}xbf16>) {{
  %e = stablehlo.multiply %x, %y : tensor<{st}xf32>
  %z = stablehlo.constant dense<0.000000e+00> : tensor<f32>
  %r = stablehlo.reduce(%e init: %z) applies stablehlo.add across dimensions = {rdims} : (tensor<{st}xf32>, tensor<f32>) -> tensor<{ot}xf32>
  %d = stablehlo.convert %e : (tensor<{st}xf32>) -> tensor<{st}xbf16>
  return %r, %d : tensor<{ot}xf32>, tensor<{st}xbf16>
}}"""
    rng = np.random.default_rng(34)
    x = rng.standard_normal(shape).astype(np.float32)
    y = rng.standard_normal(shape).astype(np.float32)
    print(f"case: ew_reduce bf16 copy {shape} over {rdims}", flush=True)
    os.environ["JAM_EW_JIT_STRICT"] = "1"
    try:
        e = client.compile(text)
    finally:
        del os.environ["JAM_EW_JIT_STRICT"]
    assert "bf16 copy stored" in e.plan()
    bufs = [client.put(x), client.put(y)]
    outs = e.execute(bufs)
    r, d = (o.to_numpy() for o in outs)
    for b in bufs + outs:
        b.destroy()
    e.destroy()
    v = x * y
    np.testing.assert_array_equal(d, bf16.to_bf16_bits(v))
    want = np.sum(v.astype(np.float64), axis=tuple(rdims))
    mag = np.sum(np.abs(v).astype(np.float64), axis=tuple(rdims))
    assert np.all(np.abs(r - want) <= 1e-6 * mag + 1e-30)
