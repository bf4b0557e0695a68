"""The portable-artifact path of PJRT_Client_Compile: every benchmark config
module, written as a StableHLO portable artifact (VHLO in MLIR bytecode v1,
what jaxlib sends; the reference reads it with deserializePortableArtifact,
src/jam/parse.cc:53-63, from ClientCompile, pjrt_c_api.cc:681-697), must
compile to exactly the launch plan of the same module as text: same steps,
buffers, integer and float parameters, elementwise programs, strides,
constants (bytes), arena and aliases.  The artifacts come from the test-only
writer tests/vhlo_writer.cc (MLIR's bytecode writer rules; no MLIR or jaxlib
exists here); tests/test_bytecode.py assembles one by hand, byte for byte,
as an independent check of the encodings.  CPU only."""

import importlib.util
import json
import os
import subprocess

import pytest

from mi355x_pjrt import gpt2, modules, pjrt, train_hlo

HERE = os.path.dirname(os.path.abspath(__file__))


def _make_vhlo():
    spec = importlib.util.spec_from_file_location("make_vhlo", os.path.join(HERE, "golden", "make_vhlo.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="module")
def writer(tmp_path_factory):
    return _make_vhlo().build_writer(str(tmp_path_factory.mktemp("vhlo")))


def _constants_module():
    vals = [1 / 3, 0.1, 1 + 2 ** -8 + 2 ** -40, 1 + 2 ** -8, 6.0e-08, 65519.0, 65520.0, -2.5e-7, 1e-40, -3.0e38,
            5e-324, 0.0]
    n = len(vals)
    txt = ", ".join(repr(float(v)) for v in vals)
    return f"""func.func public @main(%x: tensor<{n}xf32>, %i: tensor<3xi32>) -> (tensor<{n}xbf16>, tensor<{n}xf16>, tensor<{n}xf32>, tensor<3xi32>, tensor<4xi1>, tensor<2x3xi64>) {{
  %c = stablehlo.constant dense<[{txt}]> : tensor<{n}xbf16>
  %h = stablehlo.constant dense<[{txt}]> : tensor<{n}xf16>
  %f = stablehlo.constant dense<[{txt}]> : tensor<{n}xf32>
  %s = stablehlo.add %f, %x : tensor<{n}xf32>
  %k = stablehlo.constant dense<[-1, 2147483647, -2147483648]> : tensor<3xi32>
  %a = stablehlo.add %k, %i : tensor<3xi32>
  %b = stablehlo.constant dense<[true, false, true, true]> : tensor<4xi1>
  %l = stablehlo.constant dense<[[1, -2, 3], [-4, 5, -6000000000]]> : tensor<2x3xi64>
  return %c, %h, %s, %a, %b, %l : tensor<{n}xbf16>, tensor<{n}xf16>, tensor<{n}xf32>, tensor<3xi32>, tensor<4xi1>, tensor<2x3xi64>
}}"""


def _modules():
    small = gpt2.GPT2Config(n_layer=2, d_model=128, n_head=2, seq=128, batch=2, vocab=257)
    return {
        "c1_mlp": modules.mlp(),
        "c2_reduce_sum": modules.reduce_sum(),
        "c2_argmax": modules.argmax(),
        "c2_argmin": modules.argmax(is_min=True),
        "c2_layernorm": modules.layernorm(),
        "c2_gelu": modules.gelu(),
        "c3_sdpa_causal": modules.sdpa(),
        "c3_sdpa_full": modules.sdpa(causal=False),
        "c4_gather": modules.gather(),
        "c4_scatter_add": modules.scatter_add(),
        "adam": modules.adam_update(),
        "donated_matmul": modules.donated("matmul"),
        "donated_transpose_add": modules.donated("transpose_add"),
        "donated_donor_add": modules.donated("donor_add"),
        "c5_train_small": train_hlo.gpt2_train_step(small),
        "c5_train_small_grads": train_hlo.gpt2_train_step(small, return_grads=True),
        "c5_train_full": train_hlo.gpt2_train_step(gpt2.GPT2Config()),
        "constants": _constants_module(),
    }


MODULES = _modules()


@pytest.mark.parametrize("name", sorted(MODULES))
def test_artifact_compiles_to_the_text_plan(writer, tmp_path, name):
    src = tmp_path / (name + ".mlir")
    src.write_text(MODULES[name])
    r = subprocess.run([writer, "check", str(src)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("same plan:"), r.stdout


@pytest.fixture(scope="module")
def client():
    c = pjrt.Plugin().client()
    yield c
    c.close()


def _plan(client, program):
    e = client.compile(program)
    try:
        return e.plan(), e.output_types(), e.output_shapes(), e.serialize()
    finally:
        e.destroy()


@pytest.mark.parametrize("name", ["c3_sdpa_causal", "c5_train_small", "donated_donor_add"])
def test_artifact_through_the_c_api(writer, client, tmp_path, name):
    """PJRT_Client_Compile with the artifact bytes (format "mlir") gives the
    text's plan and output types / shapes; its serialized executable keeps
    the artifact and loads back to the same plan."""
    src, art = tmp_path / "m.mlir", tmp_path / "m.mlirbc"
    src.write_text(MODULES[name])
    subprocess.run([writer, "write", str(src), str(art)], check=True, capture_output=True, timeout=120)
    blob = art.read_bytes()
    assert blob[:4] == b"ML\xefR"
    plan_a, types_a, shapes_a, ser = _plan(client, blob)
    plan_t, types_t, shapes_t, _ = _plan(client, MODULES[name])
    assert (plan_a, types_a, shapes_a) == (plan_t, types_t, shapes_t)
    e = client.deserialize(ser)
    try:
        assert e.plan() == plan_t
    finally:
        e.destroy()


def test_gpu_fixtures_are_current():
    """tests/golden/vhlo/*.mlirbc (the GPU artifact tests' inputs) were
    written from today's module texts."""
    mv = _make_vhlo()
    with open(os.path.join(HERE, "golden", "vhlo", "manifest.json")) as f:
        manifest = json.load(f)
    texts = mv.config_modules()
    assert sorted(manifest) == sorted(texts)
    for name, text in texts.items():
        assert manifest[name]["text_sha256_16"] == mv.text_digest(text), f"{name}: rerun tests/golden/make_vhlo.py"
        assert os.path.getsize(os.path.join(HERE, "golden", "vhlo", name + ".mlirbc")) == manifest[name]["bytes"]
