"""The benchmark configs through the plugin as jaxlib drives it: each module is
handed to PJRT_Client_Compile as a StableHLO portable artifact (VHLO in MLIR
bytecode v1; tests/golden/vhlo/*.mlirbc, written by tests/vhlo_writer.cc from
the config modules' text, tests/golden/make_vhlo.py), run with
PJRT_LoadedExecutable_Execute on the seeded config inputs, and compared with
the CPU oracle at the configs' bars: integer and index results bit-exact,
attention within 2e-2, fp32 within 1e-5 relative (cf. the reference's
ClientCompile, pjrt_c_api.cc:681-697, and LoadedExecute, 753-829)."""

import os

import numpy as np
import pytest

from mi355x_pjrt import gpt2, pjrt, train_hlo
from oracle import bf16, inputs, native, ops
from test_gpu_pjrt import check_sdpa_sampled, client, run  # noqa: F401  (client is a fixture)

pytestmark = pytest.mark.gpu

VHLO = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "vhlo")


def artifact(name):
    with open(os.path.join(VHLO, name + ".mlirbc"), "rb") as f:
        blob = f.read()
    assert blob[:4] == b"ML\xefR"
    return blob


def test_c1_mlp_artifact(client):
    d = inputs.c1_mlp()
    print("case: vhlo C1 mlp", flush=True)
    (y,) = run(client, artifact("c1_mlp"), *[(d[k], None) for k in ("x", "w1", "b1", "w2", "b2")])
    want = ops.mlp_forward(d["x"], d["w1"], d["b1"], d["w2"], d["b2"])
    hh = np.maximum(np.abs(d["x"]).astype(np.float64) @ np.abs(d["w1"]) + np.abs(d["b1"]), 0)
    norm = hh @ np.abs(d["w2"]) + np.abs(d["b2"])
    assert np.max(np.abs(y - want) / norm) < 1e-5


def test_c2_argmax_and_reduce_sum_artifacts(client):
    x = inputs.c2_reduce()["x"]
    print("case: vhlo C2 argmax / reduce_sum", flush=True)
    (i,) = run(client, artifact("c2_argmax"), (x, pjrt.BF16))
    np.testing.assert_array_equal(i, native.argmax_rows_bf16(x, False)[0])
    (s,) = run(client, artifact("c2_reduce_sum"), (x, pjrt.BF16))
    ref = native.row_sum_bf16(x)
    norm = native.row_sum_bf16(bf16.to_bf16_bits(np.abs(bf16.from_bf16_bits(x))))
    assert np.max(np.abs(s - ref) / norm) < 1e-5


def test_c2_layernorm_artifact(client):
    d = inputs.c2_layernorm()
    print("case: vhlo C2 layernorm", flush=True)
    (y,) = run(client, artifact("c2_layernorm"), (d["x"], pjrt.BF16), (d["gamma"], pjrt.BF16),
               (d["beta"], pjrt.BF16))
    x, g, b = (bf16.from_bf16_bits(d[n]) for n in ("x", "gamma", "beta"))
    sl = slice(0, 2048)
    want = ops.layernorm(x[sl], g, b, 1e-5)
    got = bf16.from_bf16_bits(y[sl]).astype(np.float64)
    xs = np.asarray(x[sl], np.float64)
    xh = np.abs(xs - xs.mean(-1, keepdims=True)) / np.sqrt(xs.var(-1, keepdims=True) + 1e-5)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-38))) - 7)
    assert np.all(np.abs(got - want) <= ulp + 1e-5 * ((xh + 1) * np.abs(g) + np.abs(b)))


@pytest.mark.parametrize("S", [1024, 8192])
def test_c3_sdpa_artifact(client, S):
    d = inputs.c3_sdpa(S)
    print(f"case: vhlo C3 sdpa S={S}", flush=True)
    (o,) = run(client, artifact(f"c3_sdpa_s{S}"), *[(d[k], pjrt.BF16) for k in ("q", "k", "v")])
    np.testing.assert_array_equal(o[:, :, 0, :], d["v"][:, :, 0, :])  # row 0 sees one key
    check_sdpa_sampled(d, o, S, 1 / 11.3125)


def test_c4_gather_and_scatter_add_artifacts(client):
    d = inputs.c4_indexing()
    print("case: vhlo C4 gather / scatter-add", flush=True)
    (g,) = run(client, artifact("c4_gather"), (d["table_bf16"], pjrt.BF16), (d["ids"], None))
    np.testing.assert_array_equal(g.reshape(-1, 768), native.gather_rows(d["table_bf16"], d["ids"]))
    ids = d["ids"].reshape(-1)
    (t,) = run(client, artifact("c4_scatter_add"), (d["table_f32"], None), (ids, None), (d["grads"], None))
    np.testing.assert_array_equal(t, native.scatter_add_f32(d["table_f32"], ids, d["grads"]))


def test_c5_train_step_artifact_matches_text(client):
    """The reduced C5 training step (forward, backward, Adam) from its
    artifact gives bit for bit what the same module as text gives (the two
    compile to one plan), and its loss is the float64 oracle's."""
    from oracle import gpt2_ref

    cfg = gpt2.GPT2Config(n_layer=2, d_model=128, n_head=2, seq=128, batch=2, vocab=257)
    print("case: vhlo C5 reduced training step", flush=True)
    params = gpt2.init_params(cfg, 4)
    names = [n for n, _ in cfg.param_shapes()]
    rng = np.random.default_rng(5)
    ids = rng.integers(0, cfg.vocab, (cfg.batch, cfg.seq)).astype(np.int32)
    labels = rng.integers(0, cfg.vocab, (cfg.batch, cfg.seq)).astype(np.int32)
    zeros = [np.zeros_like(params[n]) for n in names]
    host = ([params[n] for n in names] + zeros + zeros + [ids, labels, np.float32(1e-3),
                                                           np.float32(1 / (1 - 0.9)), np.float32(1 / (1 - 0.999))])
    args = [(np.asarray(a), None) for a in host]
    outs_a = run(client, artifact("c5_train_small"), *args)
    outs_t = run(client, train_hlo.gpt2_train_step(cfg), *args)
    assert len(outs_a) == len(outs_t) == 1 + 3 * len(names)
    for a, t in zip(outs_a, outs_t):
        np.testing.assert_array_equal(a, t)
    loss, _ = gpt2_ref.loss_and_grads(params, ids, labels, cfg.n_layer, cfg.n_head)
    assert abs(float(outs_a[0]) - loss) <= 2e-3 * abs(loss), (float(outs_a[0]), loss)
