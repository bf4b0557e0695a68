"""The PJRT plugin through its C API, without a GPU: the function table,
platform identity, compile structure of every config module (fused patterns,
launch counts) and the named-error surface (cf. the reference's
pjrt_c_api.cc:124-127, 681-697, 753-829 and lower.mm:308-310)."""

import os
import subprocess

import pytest

from mi355x_pjrt import PJRT_LIBRARY, modules, pjrt

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def plugin():
    return pjrt.Plugin()


@pytest.fixture(scope="module")
def client(plugin):
    c = plugin.client()
    yield c
    c.close()


def test_api_table_complete(plugin):
    assert plugin.version == (0, 55)
    assert plugin.struct_size == 840          # sizeof(PJRT_Api) for v0.55
    assert [s for s in pjrt.SLOTS if not plugin.slot(s)] == []


def test_platform_identity(client):
    assert client.platform_name == "mi355x"   # not rocm/cuda: no GPU custom_calls from JAX
    assert "PJRT 0.55" in client.platform_version
    devs = client.devices()
    assert len(devs) >= 1
    assert client.device_kind(devs[0]) == "MI355X"


def _plan(client, text):
    e = client.compile(text)
    try:
        return e.plan(), e.output_types(), e.output_shapes()
    finally:
        e.destroy()


def test_compile_mlp_fuses_bias_relu(client):
    """C1's fp32 products have 64 and 16 output tiles of 128x128: each is cut
    along K into about 256 workgroups (gemm_splitk), and the matched bias /
    bias + ReLU epilogue is applied by the pass that sums the slices: two
    steps in all."""
    plan, types, shapes = _plan(client, modules.mlp())
    assert types == [pjrt.F32] and shapes == [(256, 1024)]
    assert "pattern gemm+bias+relu" in plan and "pattern gemm+bias\n" in plan
    assert "] gemm_splitk (256x4096x1024 in 4 slices, + bias + relu)" in plan
    assert "] gemm_splitk (256x1024x4096 in 16 slices, + bias)" in plan
    assert plan.count("] gemm") == 2 and plan.count("] ew") == 0


def test_compile_sdpa_is_one_flash_launch(client):
    for causal in (True, False):
        plan, types, shapes = _plan(client, modules.sdpa(4, 16, 8192, 128, causal=causal))
        assert shapes == [(4, 16, 8192, 128)] and types == [pjrt.BF16]
        assert f"sdpa({'causal' if causal else 'full'}, scale=0.088398)" in plan  # 1/bf16(sqrt(128))
        assert " 1 steps" in plan and "arena 0 B" in plan       # no [S,S] tensor anywhere


def test_compile_sdpa_unfused_when_disabled(client):
    os.environ["JAM_NO_SDPA"] = "1"
    try:
        plan, _, _ = _plan(client, modules.sdpa(1, 2, 64, 64))
    finally:
        del os.environ["JAM_NO_SDPA"]
    assert "pattern sdpa" not in plan and plan.count("] gemm") == 2


def test_compile_argmax_reduce_gelu(client):
    plan, types, _ = _plan(client, modules.argmax())
    assert "pattern argmax" in plan and " 1 steps" in plan and types == [pjrt.S32]
    plan, _, _ = _plan(client, modules.argmax(is_min=True))
    assert "pattern argmin" in plan
    plan, _, _ = _plan(client, modules.reduce_sum())
    assert " 1 steps" in plan and "row_reduce" in plan       # convert folded into the reduce load
    plan, _, _ = _plan(client, modules.gelu())
    assert "pattern gelu_tanh(bf16)" in plan and " 1 steps" in plan and "] gelu" in plan
    os.environ["JAM_NO_GELU"] = "1"
    try:
        plan, _, _ = _plan(client, modules.gelu())
    finally:
        del os.environ["JAM_NO_GELU"]
    assert " 1 steps" in plan and "] ew" in plan             # generic path: still one pass over HBM


def test_compile_indexing(client):
    plan, _, shapes = _plan(client, modules.gather())
    assert "] gather" in plan and shapes == [(32, 2048, 768)]
    plan, _, shapes = _plan(client, modules.scatter_add())
    assert "] scatter_add" in plan and shapes == [(50257, 768)]


def test_compile_jitted_training_step(client):
    """The C5 step as one module (train_hlo: forward, reverse-mode gradients,
    Adam) compiles: one output per loss / parameter / m / v (/ gradient), the
    embedding gather and its gradient's scatter-add, the weight products on
    the GEMM, each layer's attention forward and backward as one flash
    forward (with lse) and one flash backward step (nothing S x S), the
    cross-entropy with its gradient as one launch, and no layout copies or
    conversions around the attention (bf16 data kept narrow in the layouts
    its readers take)."""
    from mi355x_pjrt import gpt2, train_hlo

    cfg = gpt2.GPT2Config(n_layer=2, d_model=128, n_head=2, seq=128, batch=2, vocab=257)
    k = len(cfg.param_shapes())
    for grads in (False, True):
        plan, types, shapes = _plan(client, train_hlo.gpt2_train_step(cfg, return_grads=grads))
        assert len(types) == 1 + (4 if grads else 3) * k and shapes[0] == () and set(types) == {pjrt.F32}
        assert shapes[1:1 + k] == [s for _, s in cfg.param_shapes()]
    assert plan.count("] gather") == 1 and plan.count("] scatter_add") == 1
    # per layer 4 weight products forward and 8 backward; the tied logits
    # 1 + 2; the attention products are inside the two flash steps
    assert plan.count("] gemm") == 2 * 12 + 3
    assert plan.count("pattern sdpa_train(causal") == 2
    assert plan.count("] sdpa (causal +lse)") == 2 and plan.count("] sdpa_bwd (causal") == 2
    # the attention gradients are written into the fused QKV gradient's layout
    assert plan.count("into the merged QKV gradient") == 2
    # the mean softmax cross-entropy and its gradient: one fused launch, over
    # logits and a gradient whose 257-element rows are padded to 264 so that
    # the three vocabulary products take aligned rows on the hand-written
    # GEMM (none on the library GEMM)
    assert "pattern softmax_xent(256x257, grad_scale=0.003906)" in plan and plan.count("] softmax_xent") == 1
    assert "] softmax_xent (rows padded)" in plan and "gemm_blas" not in plan
    # no layout copies around the attention: O is written in [B,S,H,D] order
    # and read back narrow; only the position-embedding broadcast is copied
    assert plan.count("] copy_strided") <= 1
    # bias gradients: sums over the leading (token) dims read in place
    assert "] col_sum" in plan
    # each LayerNorm (2 per layer and the final one) with its backward: one
    # forward launch on the fp32 residual stream writing the bf16 operand of
    # the next product, and one backward launch writing dx (the residual
    # branch's cotangent added), dgamma, dbeta and, where a projection wrote
    # x, that projection's bias gradient, and dx rounded to bf16 where the
    # products that read it next take it so
    assert plan.count("pattern layernorm_train(f32 -> bf16, eps=0.000010") == 5
    assert plan.count("] layernorm (f32 -> bf16") == 5 and plan.count("] layernorm_bwd (") == 5
    # the residual updates x + proj(...) are added by the LayerNorm that
    # reads them (the embedding sum, a broadcast view, is not)
    assert plan.count("] layernorm (f32 -> bf16, input added)") == 4
    assert plan.count("] layernorm_bwd (residual, bias gradient, bf16 copy)") == 3
    assert plan.count("] layernorm_bwd (no residual, bias gradient, bf16 copy)") == 1  # the final LayerNorm
    assert plan.count("] layernorm_bwd (residual)") == 1  # the first, over the embeddings
    # the QKV projection (+ fp32 bias) is only read in bf16 (the attention's
    # operands): written in bf16 by its epilogue, no conversion pass
    assert plan.count("] gemm (1x256x384x128 -> bf16)") == 2
    assert "convert chain (1 instr, 1 inputs), 3 independent instances" not in plan
    # the MLP's up-projection (+ bias) writes the bf16 GELU of its result as
    # a side output: the forward GELU chain is not a step of its own
    assert plan.count("pattern gemm+bias+gelu(bf16 side output)") == 2
    assert plan.count("] gemm (1x256x512x128 + gelu side output)") == 2


def test_layernorm_train_needs_its_whole_backward(client):
    """The training LayerNorm pattern takes the forward and the backward
    together: when one rule of the backward differs (here the rsqrt
    derivative's -0.5 factor of one LayerNorm made -0.25), that LayerNorm
    keeps the generic path (forward and backward), and the others still
    match."""
    from mi355x_pjrt import gpt2, train_hlo

    cfg = gpt2.GPT2Config(n_layer=1, d_model=128, n_head=2, seq=128, batch=2, vocab=257)
    text = train_hlo.gpt2_train_step(cfg)
    plan, _, _ = _plan(client, text)
    assert plan.count("] layernorm_bwd (") == 3
    cst = "stablehlo.constant dense<-5.000000000e-01> : tensor<f32>"
    assert text.count(cst) == 3
    i = text.index(cst)
    bad = text[:i] + cst.replace("-5.0", "-2.5") + text[i + len(cst):]
    plan, _, _ = _plan(client, bad)
    assert plan.count("] layernorm_bwd (") == 2 and plan.count("pattern layernorm_train") == 2
    assert plan.count("] layernorm (f32 -> bf16") == 2


def test_gemm_gelu_side_output_needs_the_gelu(client):
    """The up-projection's GELU side output is taken only for gelu_tanh
    itself: with the cubic coefficient changed (0.044715 -> 0.05) in one
    layer, that layer's product is written alone and its chain stays an
    elementwise step; the other layer keeps the side output."""
    from mi355x_pjrt import gpt2, train_hlo

    cfg = gpt2.GPT2Config(n_layer=2, d_model=128, n_head=2, seq=128, batch=2, vocab=257)
    text = train_hlo.gpt2_train_step(cfg)
    cst = "dense<4.471500000e-02>"
    assert text.count(cst) == 2
    i = text.index(cst)
    bad = text[:i] + "dense<5.000000000e-02>" + text[i + len(cst):]
    plan, _, _ = _plan(client, bad)
    assert plan.count("+ gelu side output") == 1
    assert plan.count("pattern gemm+bias+gelu(bf16 side output)") == 1


def test_sdpa_backward_needs_the_row_broadcast(client):
    """The attention backward matcher follows the row sums sum(dP * P) back to
    [B,H,Sq,Sk]: only a broadcast of the [B,H,Sq] axes onto dims {0,1,2}
    (along the keys) is the softmax backward.  With Sq == Sk a broadcast onto
    {0,1,3} type-checks but computes something else, so that layer must not
    become the flash backward."""
    from mi355x_pjrt import gpt2, train_hlo

    cfg = gpt2.GPT2Config(n_layer=2, d_model=128, n_head=2, seq=128, batch=2, vocab=257)
    text = train_hlo.gpt2_train_step(cfg)
    sig = "dims = [0, 1, 2] : (tensor<2x2x128xf32>) -> tensor<2x2x128x128xf32>"
    at = [i for i, ln in enumerate(text.split("\n")) if sig in ln]
    assert len(at) == 6  # per layer: the forward's max and sum, the backward's row sum
    lines = text.split("\n")
    lines[at[-1]] = lines[at[-1]].replace("dims = [0, 1, 2]", "dims = [0, 1, 3]")
    plan, _, _ = _plan(client, "\n".join(lines))
    assert plan.count("] sdpa_bwd (causal") == 1
    plan, _, _ = _plan(client, text)
    assert plan.count("] sdpa_bwd (causal") == 2


def _steps(client, body, arg_type, result_type):
    text = (f"func.func public @main(%arg0: {arg_type}) -> {result_type} {{\n{body}\n}}")
    plan, _, _ = _plan(client, text)
    return [ln.split("] ", 1)[1].split(" ")[0] for ln in plan.splitlines() if "] " in ln]


# reshape of a strided view: (module body, argument type, result type, steps)
RESHAPE_VIEWS = {
    # splitting the rows of a column slice keeps a view (no copy before the add)
    "slice_split": ("""  %0 = stablehlo.slice %arg0 [0:4, 1:4] : (tensor<4x6xf32>) -> tensor<4x3xf32>
  %1 = stablehlo.reshape %0 : (tensor<4x3xf32>) -> tensor<2x2x3xf32>
  %2 = stablehlo.add %1, %1 : tensor<2x2x3xf32>
  return %2 : tensor<2x2x3xf32>""", "tensor<4x6xf32>", "tensor<2x2x3xf32>", ["ew"]),
    # a unit dim inside the merged run is linear too
    "slice_unit_dim": ("""  %0 = stablehlo.slice %arg0 [0:4, 0:1, 1:4] : (tensor<4x1x6xf32>) -> tensor<4x1x3xf32>
  %1 = stablehlo.reshape %0 : (tensor<4x1x3xf32>) -> tensor<4x3xf32>
  %2 = stablehlo.add %1, %1 : tensor<4x3xf32>
  return %2 : tensor<4x3xf32>""", "tensor<4x1x6xf32>", "tensor<4x3xf32>", ["ew"]),
    # merging rows of a column slice is not linear in memory: copy
    "slice_merge": ("""  %0 = stablehlo.slice %arg0 [0:4, 1:4] : (tensor<4x6xf32>) -> tensor<4x3xf32>
  %1 = stablehlo.reshape %0 : (tensor<4x3xf32>) -> tensor<12xf32>
  %2 = stablehlo.add %1, %1 : tensor<12xf32>
  return %2 : tensor<12xf32>""", "tensor<4x6xf32>", "tensor<12xf32>", ["copy_strided", "ew"]),
    "transpose_merge": ("""  %0 = stablehlo.transpose %arg0, dims = [1, 0] : (tensor<4x6xf32>) -> tensor<6x4xf32>
  %1 = stablehlo.reshape %0 : (tensor<6x4xf32>) -> tensor<24xf32>
  %2 = stablehlo.add %1, %1 : tensor<24xf32>
  return %2 : tensor<24xf32>""", "tensor<4x6xf32>", "tensor<24xf32>", ["copy_strided", "ew"]),
    "broadcast_merge": ("""  %0 = stablehlo.broadcast_in_dim %arg0, dims = [1] : (tensor<6xf32>) -> tensor<4x6xf32>
  %1 = stablehlo.reshape %0 : (tensor<4x6xf32>) -> tensor<24xf32>
  %2 = stablehlo.add %1, %1 : tensor<24xf32>
  return %2 : tensor<24xf32>""", "tensor<6xf32>", "tensor<24xf32>", ["copy_strided", "ew"]),
}


@pytest.mark.parametrize("case", sorted(RESHAPE_VIEWS))
def test_reshape_of_strided_views(client, case):
    body, at, rt, want = RESHAPE_VIEWS[case]
    assert _steps(client, body, at, rt) == want


def test_col_sum_respects_its_grid_limit(client):
    """Sums over the leading dim lower to col_sum while the kept extent fits
    its grid (65535 blocks of 256 columns); wider ones take the row-reduce
    path (compile only: nothing is allocated)."""
    def body(n):
        return (f"  %c = stablehlo.constant dense<0.0> : tensor<f32>\n"
                f"  %0 = stablehlo.reduce(%arg0 init: %c) applies stablehlo.add across dimensions = [0] : "
                f"(tensor<2x{n}xf32>, tensor<f32>) -> tensor<{n}xf32>\n"
                f"  return %0 : tensor<{n}xf32>")
    ok = 65535 * 256
    assert "col_sum" in _steps(client, body(ok), f"tensor<2x{ok}xf32>", f"tensor<{ok}xf32>")
    wide = ok + 256
    steps = _steps(client, body(wide), f"tensor<2x{wide}xf32>", f"tensor<{wide}xf32>")
    assert "col_sum" not in steps and "row_reduce" in steps


def test_compile_layernorm(client):
    plan, types, shapes = _plan(client, modules.layernorm(64, 256))
    assert types == [pjrt.BF16] and shapes == [(64, 256)]
    assert "pattern layernorm(bf16, eps=0.000010)" in plan and " 1 steps" in plan
    os.environ["JAM_NO_LAYERNORM"] = "1"
    try:
        plan, _, _ = _plan(client, modules.layernorm(64, 256))
    finally:
        del os.environ["JAM_NO_LAYERNORM"]
    # the mean's sum reads x; the variance's sum runs fused with its
    # elementwise operand (ew_reduce)
    assert "pattern layernorm" not in plan and plan.count("row_reduce") + plan.count("] ew_reduce") == 2


BAD = {
    "parse": ("module { func.func public @main( -> }", "parse error"),
    "unhandled": ("""func.func public @main(%a: tensor<4x4xf32>) -> tensor<4x4xf32> {
  %0 = stablehlo.cholesky %a, lower = true : tensor<4x4xf32>
  return %0 : tensor<4x4xf32>
}""", "unhandled op 'stablehlo.cholesky'"),
    "no_main": ("""func.func private @helper(%a: tensor<f32>) -> tensor<f32> {
  return %a : tensor<f32>
}""", "no @main"),
    "bytecode": ("ML\xefR\x00\x01garbage", "bytecode"),
    "bad_type": ("""func.func public @main(%a: tensor<4xc64>) -> tensor<4xc64> {
  return %a : tensor<4xc64>
}""", "unsupported element type"),
    "undefined": ("""func.func public @main(%a: tensor<4xf32>) -> tensor<4xf32> {
  %0 = stablehlo.add %a, %b : tensor<4xf32>
  return %0 : tensor<4xf32>
}""", "undefined value %b"),
}


@pytest.mark.parametrize("case", sorted(BAD))
def test_compile_errors_are_named(client, case):
    text, needle = BAD[case]
    with pytest.raises(pjrt.PjrtError) as ei:
        client.compile(text.encode("latin-1"))
    assert ei.value.code == "INVALID_ARGUMENT"
    assert ei.value.message.startswith("jam compile: ")
    assert needle in ei.value.message


def test_unimplemented_slots_and_multinode(plugin, client):
    with pytest.raises(pjrt.PjrtError) as ei:
        plugin.client({"node_id": 0, "num_nodes": 2})
    assert ei.value.code == "UNIMPLEMENTED"
    # a stub slot answers UNIMPLEMENTED with its name
    import ctypes
    fn = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p)(plugin.slot("CopyToDeviceStream_TotalBytes"))
    err = fn(None)
    e = plugin._error(err)
    assert e.code == "UNIMPLEMENTED" and "PJRT_CopyToDeviceStream_TotalBytes" in e.message
    # exactly the copy-to-device-stream group and topology serialization are stubs
    stubs = [s for s in pjrt.SLOTS
             if s.startswith("CopyToDeviceStream_") or s == "TopologyDescription_Serialize"]
    assert len(stubs) == 6


def test_plugin_attributes_and_device_description(plugin, client):
    """PJRT_Plugin_Attributes carries the StableHLO version window a client
    serializes for; device descriptions carry what HIP reports."""
    attrs = plugin.attributes()
    assert attrs["xla_version"] == 2
    assert attrs["stablehlo_current_version"] == [1, 0, 0]
    assert attrs["stablehlo_minimum_version"] == [1, 0, 0]
    dev = client.devices()[0]
    d = client.device_attributes(dev)
    assert set(d) == {"gfx_arch", "compute_units", "hbm_bytes", "pci_bus_id"}
    assert client.device_string(dev).startswith("MI355X#0 (")


def test_serialize_round_trip(client):
    """Executable_Serialize then DeserializeAndLoad gives the same plan and
    fingerprint; foreign bytes are refused with a named error."""
    e = client.compile(modules.reduce_sum(4, 8))
    blob = e.serialize()
    assert blob.startswith(b"mi355x-jam/1\n") and modules.reduce_sum(4, 8).encode() in blob
    e2 = client.deserialize(blob)
    assert e2.plan() == e.plan() and e2.output_shapes() == [(4,)]
    with pytest.raises(pjrt.PjrtError) as ei:
        client.deserialize(b"not an executable")
    assert ei.value.code == "INVALID_ARGUMENT" and "mi355x-pjrt" in ei.value.message
    e.destroy()
    e2.destroy()


def test_execute_argument_count_checked(client):
    e = client.compile(modules.reduce_sum(4, 8))
    with pytest.raises(pjrt.PjrtError) as ei:
        e.execute([])
    assert ei.value.code == "INVALID_ARGUMENT" and "takes 1 arguments, got 0" in ei.value.message
    e.delete()
    with pytest.raises(pjrt.PjrtError) as ei:
        e.execute([])
    assert "executable was deleted" in ei.value.message
    e.destroy()


def test_cpp_driver_compiles(tmp_path):
    mod = tmp_path / "sdpa.mlir"
    mod.write_text(modules.sdpa(1, 2, 128, 64))
    exe = os.path.join(ROOT, "mccl-jax_amd", "bin", "pjrt_e2e")
    r = subprocess.run([exe, PJRT_LIBRARY, str(mod), "--compile-only"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert "PJRT API 0.55" in r.stdout and "platform mi355x" in r.stdout and "compiled: 1 outputs" in r.stdout


def test_donation_aliases_in_plan(client):
    """tf.aliasing_output / jax.buffer_donor on @main's arguments: the plan
    writes an output over its donated input only where that is safe
    (element-for-element, no later reader), and says why otherwise."""
    plan, _, shapes = _plan(client, modules.adam_update(4096))
    assert shapes == [(4096,)] * 3
    for i in range(3):
        assert f"alias input {i} -> output {i} in place (tf.aliasing_output)" in plan, plan
    plan, _, _ = _plan(client, modules.donated("matmul"))
    assert "alias input 0 -> output 0 not in place (tf.aliasing_output): writer is gemm" in plan
    plan, _, _ = _plan(client, modules.donated("transpose_add"))
    assert "alias input 0 -> output 0 not in place" in plan and "layout" in plan
    plan, _, _ = _plan(client, modules.donated("donor_add"))
    assert "alias input 0 -> output 0 in place (jax.buffer_donor)" in plan


SUM_AND_ROUND = """func.func public @main(%a: tensor<256x128xbf16>, %b: tensor<128x256xbf16>) -> (tensor<256x256xbf16>, tensor<256xf32>) {
  %y = stablehlo.dot_general %a, %b, contracting_dims = [1] x [0] : (tensor<256x128xbf16>, tensor<128x256xbf16>) -> tensor<256x256xf32>
  %z = stablehlo.convert %y : (tensor<256x256xf32>) -> tensor<256x256xbf16>
  %c = stablehlo.constant dense<0.000000e+00> : tensor<f32>
  %s = stablehlo.reduce(%y init: %c) applies stablehlo.add across dimensions = [0] : (tensor<256x256xf32>, tensor<f32>) -> tensor<256xf32>
  return %z, %s : tensor<256x256xbf16>, tensor<256xf32>
}"""


def test_product_read_by_a_sum_stays_f32(client):
    """An f32 product that a sum reads is written in f32 (the sum of its
    bf16 roundings would differ); a product only ever rounded to bf16 is
    written in bf16."""
    plan, _, _ = _plan(client, SUM_AND_ROUND)
    assert "] gemm (1x256x256x128)\n" in plan and "-> bf16" not in plan
    plan, _, _ = _plan(client, SUM_AND_ROUND.replace(", %s : tensor<256x256xbf16>, tensor<256xf32>",
                                                         " : tensor<256x256xbf16>")
                       .replace("-> (tensor<256x256xbf16>, tensor<256xf32>)", "-> tensor<256x256xbf16>"))
    assert "-> bf16" in plan
