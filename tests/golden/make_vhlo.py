"""StableHLO portable artifacts of the benchmark config modules, for the GPU
parity tests of the plugin's artifact path (tests/test_gpu_vhlo.py).

jaxlib hands PJRT_Client_Compile a portable artifact (MLIR bytecode of VHLO
operations), not text.  Neither jaxlib nor MLIR exists here, so the
artifacts are written by tests/vhlo_writer.cc (a test-only writer following
MLIR's bytecode writer rules) from the same StableHLO text the text-path
tests compile.  `build_writer()` compiles that program against the jam
sources; it is also used by tests/test_vhlo.py.

    python tests/golden/make_vhlo.py     # rewrites tests/golden/vhlo/*.mlirbc
"""

import concurrent.futures
import hashlib
import json
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
PKG = os.path.join(ROOT, "mccl-jax_amd")
OUT = os.path.join(HERE, "vhlo")


def build_writer(outdir):
    """Compile tests/vhlo_writer.cc with the jam compiler sources into
    `outdir`/vhlo_writer; returns its path."""
    src = os.path.join(PKG, "src")
    sources = sorted(os.path.join(src, d, f) for d in ("jam", "execution")
                     for f in os.listdir(os.path.join(src, d)) if f.endswith(".cc"))
    sources.append(os.path.join(ROOT, "tests", "vhlo_writer.cc"))
    flags = ["-std=c++17", "-O1", "-fPIC", "-D__HIP_PLATFORM_AMD__", "-I" + src, "-I" + os.path.join(ROOT, "include"),
             "-I/opt/rocm/include"]
    os.makedirs(outdir, exist_ok=True)

    def cc(path):
        obj = os.path.join(outdir, os.path.basename(path) + ".o")
        subprocess.run(["g++", *flags, "-c", path, "-o", obj], check=True)
        return obj

    with concurrent.futures.ThreadPoolExecutor(8) as ex:
        objs = list(ex.map(cc, sources))
    exe = os.path.join(outdir, "vhlo_writer")
    lib = os.path.join(PKG, "lib")
    subprocess.run(["g++", "-o", exe, *objs, "-L" + lib, "-lmk_kernels", "-L/opt/rocm/lib", "-lamdhip64", "-ldl",
                    "-Wl,-rpath," + lib, "-Wl,-rpath,/opt/rocm/lib"], check=True)
    return exe


def config_modules():
    """name -> StableHLO text of the modules the GPU artifact tests run."""
    sys.path[:0] = [ROOT, PKG]
    from mi355x_pjrt import gpt2, modules, train_hlo

    return {
        "c1_mlp": modules.mlp(),
        "c2_reduce_sum": modules.reduce_sum(),
        "c2_argmax": modules.argmax(),
        "c2_layernorm": modules.layernorm(),
        "c3_sdpa_s1024": modules.sdpa(4, 16, 1024, 128, True),
        "c3_sdpa_s8192": modules.sdpa(4, 16, 8192, 128, True),
        "c4_gather": modules.gather(),
        "c4_scatter_add": modules.scatter_add(),
        "c5_train_small": train_hlo.gpt2_train_step(
            gpt2.GPT2Config(n_layer=2, d_model=128, n_head=2, seq=128, batch=2, vocab=257)),
    }


def text_digest(text):
    return hashlib.sha256(text.encode()).hexdigest()[:16]


def main():
    import tempfile

    with tempfile.TemporaryDirectory() as tmp:
        exe = build_writer(tmp)
        os.makedirs(OUT, exist_ok=True)
        manifest = {}
        for name, text in config_modules().items():
            src = os.path.join(tmp, name + ".mlir")
            with open(src, "w") as f:
                f.write(text)
            subprocess.run([exe, "check", src], check=True)
            dst = os.path.join(OUT, name + ".mlirbc")
            subprocess.run([exe, "write", src, dst], check=True, capture_output=True)
            manifest[name] = {"text_sha256_16": text_digest(text), "bytes": os.path.getsize(dst)}
            print(f"{name}: {manifest[name]['bytes']} bytes")
        with open(os.path.join(OUT, "manifest.json"), "w") as f:
            json.dump(manifest, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
