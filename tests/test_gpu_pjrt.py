"""End-to-end parity through the PJRT C API on the MI355X: the StableHLO of
each benchmark config is compiled by the plugin, inputs are uploaded with
PJRT_Client_BufferFromHostBuffer, the executable runs, results come back
with PJRT_Buffer_ToHostBuffer and are compared with the CPU oracle on the
same seeded inputs — the path jaxlib drives (pjrt_c_api.cc:681-829)."""

import math
import os

import numpy as np
import pytest

from mi355x_pjrt import modules, pjrt
from oracle import bf16, inputs, native, ops

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def client():
    p = pjrt.Plugin()
    c = p.client()
    if c.device_kind(c.devices()[0]) != "MI355X":
        pytest.skip("no device")
    yield c
    c.close()


def run(client, text, *args):
    e = client.compile(text)
    bufs = [client.put(a, code) for a, code in args]
    outs = e.execute(bufs)
    res = [o.to_numpy() for o in outs]
    for b in bufs + outs:
        b.destroy()
    e.destroy()
    return res


def test_roundtrip_all_dtypes(client):
    rng = np.random.default_rng(0)
    for dt in (np.float32, np.int32, np.int8, np.uint8, np.int16, np.uint16, np.float16, np.bool_, np.int64):
        a = (rng.standard_normal((3, 5, 7)) * 50).astype(dt)
        b = client.put(a)
        np.testing.assert_array_equal(b.to_numpy(), a)
        b.destroy()
    bits = bf16.to_bf16_bits(rng.standard_normal(1001).astype(np.float32))
    b = client.put(bits, pjrt.BF16)
    assert b.type == pjrt.BF16 and b.shape == (1001,)
    np.testing.assert_array_equal(b.to_numpy(), bits)
    b.destroy()


def test_c1_mlp_fp32(client):
    d = inputs.c1_mlp()
    print("case: pjrt C1 mlp", flush=True)
    (y,) = run(client, modules.mlp(), *[(d[k], None) for k in ("x", "w1", "b1", "w2", "b2")])
    want = ops.mlp_forward(d["x"], d["w1"], d["b1"], d["w2"], d["b2"])
    hh = np.maximum(np.abs(d["x"]).astype(np.float64) @ np.abs(d["w1"]) + np.abs(d["b1"]), 0)
    norm = hh @ np.abs(d["w2"]) + np.abs(d["b2"])
    assert np.max(np.abs(y - want) / norm) < 1e-5


def test_c2_reduce_sum_and_argmax(client):
    x = inputs.c2_reduce()["x"]
    print("case: pjrt C2 reduce_sum / argmax", flush=True)
    (s,) = run(client, modules.reduce_sum(), (x, pjrt.BF16))
    ref = native.row_sum_bf16(x)
    norm = native.row_sum_bf16(bf16.to_bf16_bits(np.abs(bf16.from_bf16_bits(x))))
    assert np.max(np.abs(s - ref) / norm) < 1e-5
    for is_min in (False, True):
        (i,) = run(client, modules.argmax(is_min=is_min), (x, pjrt.BF16))
        np.testing.assert_array_equal(i, native.argmax_rows_bf16(x, is_min)[0])


def test_c2_layernorm(client):
    d = inputs.c2_layernorm()
    print("case: pjrt C2 layernorm", flush=True)
    (y,) = run(client, modules.layernorm(), (d["x"], pjrt.BF16), (d["gamma"], pjrt.BF16), (d["beta"], pjrt.BF16))
    x, g, b = (bf16.from_bf16_bits(d[n]) for n in ("x", "gamma", "beta"))
    for r0 in range(0, 8192, 2048):
        sl = slice(r0, r0 + 2048)
        want = ops.layernorm(x[sl], g, b, 1e-5)
        got = bf16.from_bf16_bits(y[sl]).astype(np.float64)
        xs = np.asarray(x[sl], np.float64)
        xh = np.abs(xs - xs.mean(-1, keepdims=True)) / np.sqrt(xs.var(-1, keepdims=True) + 1e-5)
        scale = (xh + 1) * np.abs(g) + np.abs(b)
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-38))) - 7)
        assert np.all(np.abs(got - want) <= ulp + 1e-5 * scale)


def test_c2_gelu(client):
    x = inputs.c2_gelu()["x"]
    print("case: pjrt C2 gelu (fused)", flush=True)
    (y,) = run(client, modules.gelu(), (x, pjrt.BF16))
    for r0 in range(0, x.shape[0], 1024):
        want = ops.round_to(ops.gelu_tanh(bf16.from_bf16_bits(x[r0:r0 + 1024])), "bf16")
        dist = bf16.bf16_ulp_distance(y[r0:r0 + 1024], want)
        assert dist.max() <= 1 and np.mean(dist == 0) > 0.99


def test_c2_gelu_unfused_generic_path(client):
    """JAM_NO_GELU: the jnp chain in the elementwise interpreter, fp32 per op
    like XLA:CPU.  0.5*x*(1+tanh(u)) cancels for negative x in fp32, so the
    bound is one bf16 ulp plus the fp32 cancellation term 2^-22 * |x|."""
    x = inputs.c2_gelu(1024, 16384)["x"]
    os.environ["JAM_NO_GELU"] = "1"
    try:
        (y,) = run(client, modules.gelu(1024, 16384), (x, pjrt.BF16))
    finally:
        del os.environ["JAM_NO_GELU"]
    xf = bf16.from_bf16_bits(x).astype(np.float64)
    want = ops.gelu_tanh(xf)
    got = bf16.from_bf16_bits(y).astype(np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-38))) - 7)
    assert np.all(np.abs(got - want) <= ulp + 2.0 ** -22 * np.abs(xf))


def test_c2_layernorm_unfused_generic_path(client):
    d = inputs.c2_layernorm(512, 4096)
    os.environ["JAM_NO_LAYERNORM"] = "1"
    try:
        (y,) = run(client, modules.layernorm(512, 4096), (d["x"], pjrt.BF16), (d["gamma"], pjrt.BF16),
                   (d["beta"], pjrt.BF16))
    finally:
        del os.environ["JAM_NO_LAYERNORM"]
    x, g, b = (bf16.from_bf16_bits(d[n]) for n in ("x", "gamma", "beta"))
    want = ops.layernorm(x, g, b, 1e-5)
    got = bf16.from_bf16_bits(y).astype(np.float64)
    xs = np.asarray(x, np.float64)
    xh = np.abs(xs - xs.mean(-1, keepdims=True)) / np.sqrt(xs.var(-1, keepdims=True) + 1e-5)
    scale = (xh + 1) * np.abs(g) + np.abs(b)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-38))) - 7)
    assert np.all(np.abs(got - want) <= ulp + 1e-5 * scale)


def check_sdpa_sampled(d, o, S, scale, causal=True):
    """C3 output `o` [4,16,S,128] (bf16 bits) against the float64 oracle.
    Up to S=4096, three (b,h) pairs in full; above, eight pairs including the
    last on ~70 rows each (a causal row needs only its key prefix), the
    first, middle and last rows among them.  The 2e-2 absolute bar of the
    config, and 2e-2 of the pair's largest |O|."""
    if S <= 4096:
        pairs, rows = [(0, 0), (2, 9), (3, 15)], np.arange(S)
    else:
        pairs = [(0, 0), (0, 15), (1, 3), (1, 7), (2, 9), (2, 12), (3, 0), (3, 15)]
        rng = np.random.default_rng(20 + S)
        rows = np.array(sorted(set([0, 1, 63, 64, 127, 128, 255, 256, S // 2 - 1, S // 2, S - 2, S - 1] +
                                   list(rng.integers(0, S, 58)))))
    for b, h in pairs:
        qf, kf, vf = (bf16.from_bf16_bits(d[k][b, h]).astype(np.float64) for k in ("q", "k", "v"))
        kmax = int(rows.max()) + 1 if causal else S
        sc = (qf[rows] @ kf[:kmax].T) * scale
        if causal:
            sc[np.arange(kmax)[None, :] > rows[:, None]] = -np.inf
        p = np.exp(sc - sc.max(axis=1, keepdims=True))
        want = (p @ vf[:kmax]) / p.sum(axis=1, keepdims=True)
        err = np.abs(bf16.from_bf16_bits(o[b, h, rows]).astype(np.float64) - want)
        assert err.max() < 2e-2 and err.max() < 2e-2 * np.abs(want).max(), (b, h, float(err.max()))


@pytest.mark.parametrize("S,causal", [(512, True), (512, False), (1024, True), (2048, True), (4096, True),
                                      (8192, True), (16384, True)])
def test_c3_sdpa_fused(client, S, causal):
    """The C3 module through PJRT at every length of the sweep (the jam plan
    is one flash launch at each)."""
    d = inputs.c3_sdpa(S)
    print(f"case: pjrt C3 sdpa S={S} causal={causal}", flush=True)
    (o,) = run(client, modules.sdpa(4, 16, S, 128, causal), *[(d[k], pjrt.BF16) for k in ("q", "k", "v")])
    check_sdpa_sampled(d, o, S, 1 / 11.3125, causal)  # the module divides by bf16(sqrt(128))


def test_c3_sdpa_unfused_generic_path(client):
    """JAM_NO_SDPA: the same module through the generic lowering (batched
    bf16 GEMMs, iota/compare mask, bf16 reduce-max, f32 sum, divide)."""
    d = inputs.c3_sdpa(256, batch=2, heads=3)
    os.environ["JAM_NO_SDPA"] = "1"
    try:
        (o,) = run(client, modules.sdpa(2, 3, 256, 128, True), *[(d[k], pjrt.BF16) for k in ("q", "k", "v")])
    finally:
        del os.environ["JAM_NO_SDPA"]
    want = ops.sdpa(*(bf16.from_bf16_bits(d[k]) for k in ("q", "k", "v")), 1 / 11.3125, True)
    err = np.abs(bf16.from_bf16_bits(o) - want)
    assert err.max() < 2e-2


def test_c4_gather_and_scatter_add(client):
    d = inputs.c4_indexing()
    print("case: pjrt C4 gather / scatter-add", flush=True)
    (g,) = run(client, modules.gather(), (d["table_bf16"], pjrt.BF16), (d["ids"], None))
    np.testing.assert_array_equal(g.reshape(-1, 768), native.gather_rows(d["table_bf16"], d["ids"]))
    ids = d["ids"].reshape(-1)
    (t,) = run(client, modules.scatter_add(), (d["table_f32"], None), (ids, None), (d["grads"], None))
    np.testing.assert_array_equal(t, native.scatter_add_f32(d["table_f32"], ids, d["grads"]))


def test_reshape_of_strided_views(client):
    """Reshapes of slices (kept as strided views), of transposes and of
    broadcasts (copied), each feeding an add: x + x is exact, so the result
    must equal numpy's bit for bit."""
    from test_pjrt_cpu import RESHAPE_VIEWS

    for case, (body, at, rt, _) in sorted(RESHAPE_VIEWS.items()):
        print(f"case: reshape view {case}", flush=True)
        text = f"func.func public @main(%arg0: {at}) -> {rt} {{\n{body}\n}}"
        shape = tuple(int(d) for d in at[len("tensor<"):-len("xf32>")].split("x"))
        x = np.arange(np.prod(shape), dtype=np.float32).reshape(shape) * 0.5 - 3
        (got,) = run(client, text, (x, pjrt.F32))
        if case == "slice_split":
            want = x[:, 1:4].reshape(2, 2, 3)
        elif case == "slice_unit_dim":
            want = x[:, 0, 1:4]
        elif case == "slice_merge":
            want = x[:, 1:4].reshape(12)
        elif case == "transpose_merge":
            want = x.T.reshape(24)
        else:
            want = np.broadcast_to(x, (4, 6)).reshape(24)
        np.testing.assert_array_equal(got, want + want)


def test_constants_bf16_f16_rne(client):
    """Dense decimal constants are rounded once from the literal's double
    value to the element type, nearest-even, with subnormals and overflow to
    inf (numpy's float64 -> float16 cast; the pinned oracle's f64 -> bf16).
    Includes a value that rounds differently if it goes through f32 first."""
    vals = [1 / 3, 0.1, 1 + 2 ** -8 + 2 ** -40, 1 + 2 ** -8, 6.0e-08, 65519.0, 65520.0, -2.5e-7,
            1e-40, -3.0e38, 5e-324, 0.0]
    n = len(vals)
    txt = ", ".join(repr(float(v)) for v in vals)
    text = f"""func.func public @main(%x: tensor<{n}xf32>) -> (tensor<{n}xbf16>, tensor<{n}xf16>, tensor<{n}xf32>) {{
  %c = stablehlo.constant dense<[{txt}]> : tensor<{n}xbf16>
  %h = stablehlo.constant dense<[{txt}]> : tensor<{n}xf16>
  %cf = stablehlo.convert %c : (tensor<{n}xbf16>) -> tensor<{n}xf32>
  %s = stablehlo.add %cf, %x : tensor<{n}xf32>
  return %c, %h, %s : tensor<{n}xbf16>, tensor<{n}xf16>, tensor<{n}xf32>
}}"""
    x = np.arange(n, dtype=np.float32)
    c, h, s = run(client, text, (x, None))
    want_bf16 = bf16.to_bf16_bits_f64(np.array(vals, np.float64))
    np.testing.assert_array_equal(c, want_bf16)
    assert c[2] != bf16.to_bf16_bits(np.array([vals[2]], np.float32))[0]  # the double-rounding case
    np.testing.assert_array_equal(h.view(np.uint16), np.array(vals, np.float64).astype(np.float16).view(np.uint16))
    np.testing.assert_array_equal(s, bf16.from_bf16_bits(want_bf16) + x)


def test_buffer_lifecycle_errors(client):
    e = client.compile(modules.reduce_sum(4, 8))
    x = client.put(np.ones((4, 8), np.uint16) * 0x3F80, pjrt.BF16)
    (y,) = e.execute([x])
    np.testing.assert_array_equal(y.to_numpy(), np.full(4, 8.0, np.float32))
    x.delete()
    with pytest.raises(pjrt.PjrtError) as ei:
        e.execute([x])
    assert "was deleted" in ei.value.message
    with pytest.raises(pjrt.PjrtError):
        x.to_numpy()
    y2 = client.put(np.ones((4, 8), np.float32))
    with pytest.raises(pjrt.PjrtError) as ei:
        e.execute([y2])  # wrong byte size for a bf16 [4,8] input
    assert "size mismatch" in ei.value.message
    for b in (x, y, y2):
        b.destroy()
    e.destroy()


def test_donation_reuses_input_memory(client):
    """The Adam update jitted with its state donated: outputs 0-2 are written
    over inputs 0-2 (same device pointers; the donated buffers are deleted),
    unless the caller lists them in non_donatable_input_indices; both runs
    give the same values, equal to the same fp32 arithmetic on the CPU."""
    n = 1 << 20
    rng = np.random.default_rng(7)
    p, m, g = (rng.standard_normal(n).astype(np.float32) for _ in range(3))
    v = np.abs(rng.standard_normal(n)).astype(np.float32) * 1e-2
    bc1, bc2, lr = np.float32(1 - 0.9 ** 3), np.float32(1 - 0.999 ** 3), np.float32(1e-3)
    e = client.compile(modules.adam_update(n))
    print("case: pjrt donated adam update", flush=True)
    results = []
    for keep in (None, [0, 1, 2]):
        bufs = [client.put(a) for a in (p, m, v, g, np.array(bc1), np.array(bc2), np.array(lr))]
        ptrs = [b.device_pointer for b in bufs[:3]]
        outs = e.execute(bufs, non_donatable=keep)
        res = [o.to_numpy() for o in outs]
        if keep is None:
            assert [b.is_deleted for b in bufs[:3]] == [True] * 3
            assert [o.device_pointer for o in outs] == ptrs
        else:
            assert not any(b.is_deleted for b in bufs[:3])
            assert not set(o.device_pointer for o in outs) & set(ptrs)
            np.testing.assert_array_equal(bufs[0].to_numpy(), p)  # the kept input is untouched
        results.append(res)
        for b in bufs + outs:
            b.destroy()
    for a, b in zip(*results):
        np.testing.assert_array_equal(a, b)
    f = np.float32
    m1 = f(0.9) * m + f(1 - 0.9) * g
    v1 = f(0.999) * v + f(1 - 0.999) * g * g
    p1 = p - lr * (m1 / bc1) / (np.sqrt(v1 / bc2) + f(1e-8))
    pr, mr, vr = results[0]
    np.testing.assert_allclose(mr, m1, rtol=2e-7, atol=1e-7)
    np.testing.assert_allclose(vr, v1, rtol=2e-7, atol=1e-12)
    np.testing.assert_allclose(pr, p1, rtol=1e-6, atol=1e-9)
    e.destroy()


def test_concurrent_execute_from_threads(client):
    """Several Python threads run one compiled executable at once (ctypes
    releases the GIL, so the plugin sees concurrent PJRT_LoadedExecutable_Execute
    and buffer transfers): every thread gets its own inputs' result, equal
    to a single-threaded run of the same inputs."""
    import threading

    e = client.compile(modules.sdpa(1, 2, 256, 128, causal=True))
    rng = np.random.default_rng(11)
    cases = [[bf16.to_bf16_bits((rng.standard_normal((1, 2, 256, 128)) / math.sqrt(128)).astype(np.float32))
              for _ in range(3)] for _ in range(4)]

    def run_once(qkv):
        bufs = [client.put(a, pjrt.BF16) for a in qkv]
        (o,) = e.execute(bufs)
        res = o.to_numpy()
        for b in bufs + [o]:
            b.destroy()
        return res

    want = [run_once(c) for c in cases]
    errors, got = [], [[None] * 5 for _ in cases]

    def worker(t):
        try:
            for it in range(5):
                got[t][it] = run_once(cases[t])
        except Exception as ex:  # noqa: BLE001 - reported below
            errors.append(repr(ex))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(len(cases))]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads), "a worker did not finish"
    assert not errors, errors
    for t in range(len(cases)):
        for it in range(5):
            np.testing.assert_array_equal(got[t][it], want[t])
    e.destroy()


def _queue_long_work(client, reps=24):
    """Queue about reps x 1.1 ms of attention on the compute stream; returns
    the executable, its input buffers, the outputs and the last event."""
    d = inputs.c3_sdpa(8192)
    e = client.compile(modules.sdpa(4, 16, 8192, 128, True))
    bufs = [client.put(d[k], pjrt.BF16) for k in ("q", "k", "v")]
    for b in bufs:
        b.ready()
    outs, ev = [], None
    for _ in range(reps):
        if ev is not None:
            client.p.call("Event_Destroy", event=ev)
        o, ev = e.execute(bufs, wait="event")
        outs += o
    return e, bufs, outs, ev


def test_upload_does_not_wait_for_queued_kernels():
    """BufferFromHostBuffer with tens of milliseconds of kernels queued: the
    upload goes to the transfer stream, so its ready event completes while
    the queued work is still running, and a program reading the uploaded
    buffer (queued after it) sees its bytes.  Then an upload into a block
    freed while kernels still read it waits for them (the pool's reuse
    event).  Run in a fresh process holding only the plugin's streams
    (tests/async_upload_check.py says why)."""
    import subprocess
    import sys

    print("case: pjrt async upload behind queued sdpa (subprocess)", flush=True)
    script = os.path.join(os.path.dirname(os.path.abspath(__file__)), "async_upload_check.py")
    r = subprocess.run([sys.executable, script], capture_output=True, text=True, timeout=100)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


def test_download_is_asynchronous_and_callbacks_fire(client):
    """ToHostBuffer queued behind running kernels returns at once; its event
    completes later with the right bytes, and PJRT_Event_OnReady callbacks
    (run by the plugin's watcher thread) fire for both events."""
    import threading

    print("case: pjrt async download + OnReady", flush=True)
    e, bufs, outs, ev = _queue_long_work(client)
    fired = []
    done = threading.Event()

    def note(err):
        fired.append(err)
        if len(fired) == 2:
            done.set()

    keep = [client.p.on_ready(ev, note)]
    arr, dev = outs[-1].to_numpy_async()
    assert not client.p.event_ready(dev), "ToHostBuffer blocked until the kernels finished"
    keep.append(client.p.on_ready(dev, note))
    assert done.wait(30), fired
    assert fired == [None, None]
    client.p.await_event(dev)
    client.p.await_event(ev)
    np.testing.assert_array_equal(arr, outs[0].to_numpy())  # every rep computes the same output
    for b in bufs + outs:
        b.destroy()
    e.destroy()
