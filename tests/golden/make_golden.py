"""Writes the small golden fixtures of this directory: fixed seeded inputs and
the oracle's outputs for them (test infrastructure).

    python tests/golden/make_golden.py

Each <case>.npz holds the inputs (bf16 as uint16 bits) and the expected
outputs, computed by the float64 / exact oracle in oracle/.  tests/test_golden.py
checks that the oracle still reproduces every file (CPU) and that the HIP
kernels match them (GPU).  The reference ships no vectors for this path, so
these are the oracle's own, frozen."""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import bf16, gpt2_ref, ops  # noqa: E402


def bits(x):
    return bf16.to_bf16_bits(np.asarray(x, dtype=np.float32))


def vals(b):
    return bf16.from_bf16_bits(b).astype(np.float64)


def cases():
    rng = np.random.default_rng(20261201)
    out = {}
    # C3 causal SDPA, one (b, h) pair per head, S 64, D 64 and 128
    for d in (64, 128):
        q, k, v = (bits(rng.standard_normal((1, 2, 64, d)) / np.sqrt(d)) for _ in range(3))
        scale = 1.0 / np.sqrt(d)
        o = ops.sdpa(vals(q), vals(k), vals(v), scale, causal=True)
        lse = ops.sdpa_lse(vals(q), vals(k), scale, causal=True)
        out[f"sdpa_causal_d{d}"] = dict(q=q, k=k, v=v, scale=np.float64(scale), o=o, lse=lse)
    # C2 LayerNorm (bf16 rows, fp32 stats)
    x = bits(rng.standard_normal((16, 256)) * 2 + 0.3)
    g = bits(1 + 0.1 * rng.standard_normal(256))
    b = bits(0.1 * rng.standard_normal(256))
    out["layernorm"] = dict(x=x, gamma=g, beta=b, eps=np.float64(1e-5),
                            y=ops.layernorm(vals(x), vals(g), vals(b), 1e-5))
    # C2 argmax with forced ties and NaNs (exact)
    xa = bits(rng.standard_normal((32, 300)))
    xa[3, 10] = xa[3, 200] = bits(np.array([9.0]))[0]      # tie: lower index wins
    xa[5, 7] = 0x7FC0                                      # NaN wins
    xa[6, :] = bits(np.ones(300))                          # all equal: index 0
    idx, _ = ops.argmax_rows(bf16.from_bf16_bits(xa))
    out["argmax"] = dict(x=xa, index=idx.astype(np.int32))
    # C4 gather (clamped ids) and sequential scatter-add (duplicates, out of range)
    table = bits(rng.standard_normal((50, 8)))
    ids = rng.integers(-3, 53, size=40).astype(np.int32)
    out["gather"] = dict(table=table, ids=ids, rows=ops.gather_rows(table, ids))
    t32 = rng.standard_normal((40, 12)).astype(np.float32)
    sid = np.concatenate([rng.integers(0, 40, 250), np.full(30, 7), [-1, 40, 99]]).astype(np.int32)
    rng.shuffle(sid)
    upd = (rng.standard_normal((sid.size, 12)) * 10).astype(np.float32)
    out["scatter_add"] = dict(table=t32, ids=sid, updates=upd, out=ops.scatter_add_rows_f32(t32, sid, upd))
    # C5 softmax cross-entropy (bf16 logits)
    lg = bits(rng.standard_normal((8, 300)) * 3)
    lab = rng.integers(0, 300, 8).astype(np.int32)
    lab[-1] = 300
    loss, dl = ops.softmax_xent(vals(lg), lab, 1.0 / 8)
    out["softmax_xent"] = dict(logits=lg, labels=lab, loss=loss, dlogits=dl)
    # C5 training step on a tiny decoder (1 layer, d 64, 1 head of 64, S 32, B 2, V 97)
    L, d, H, S, B, V, F = 1, 64, 1, 32, 2, 97, 256
    p = {"wte": rng.standard_normal((V, d)) * 0.1, "wpe": rng.standard_normal((S, d)) * 0.1}
    q = "h0."
    p.update({q + "ln1_g": 1 + 0.1 * rng.standard_normal(d), q + "ln1_b": 0.05 * rng.standard_normal(d),
              q + "w_qkv": rng.standard_normal((d, 3 * d)) * 0.05, q + "b_qkv": 0.05 * rng.standard_normal(3 * d),
              q + "w_o": rng.standard_normal((d, d)) * 0.05, q + "b_o": 0.05 * rng.standard_normal(d),
              q + "ln2_g": 1 + 0.1 * rng.standard_normal(d), q + "ln2_b": 0.05 * rng.standard_normal(d),
              q + "w_fc": rng.standard_normal((d, F)) * 0.05, q + "b_fc": 0.05 * rng.standard_normal(F),
              q + "w_pr": rng.standard_normal((F, d)) * 0.05, q + "b_pr": 0.05 * rng.standard_normal(d),
              "lnf_g": 1 + 0.1 * rng.standard_normal(d), "lnf_b": 0.05 * rng.standard_normal(d)})
    # parameters as the GPU step holds them: bf16 values
    p = {n: vals(bits(a)).astype(np.float32) for n, a in p.items()}
    ids = rng.integers(0, V, (B, S)).astype(np.int32)
    labels = rng.integers(0, V, (B, S)).astype(np.int32)
    loss, grads = gpt2_ref.loss_and_grads(p, ids, labels, L, H)
    rec = {"ids": ids, "labels": labels, "loss": np.float64(loss)}
    rec.update({"p." + n: a for n, a in p.items()})
    rec.update({"g." + n: a.astype(np.float32) for n, a in grads.items()})
    out["gpt2_tiny_step"] = rec
    return out


def main():
    for name, rec in cases().items():
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **rec)
        print(name, sum(np.asarray(v).nbytes for v in rec.values()), "bytes")


if __name__ == "__main__":
    main()
