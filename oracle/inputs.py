"""Seeded synthetic inputs for the benchmark configs C1-C5 (oracle; test
infrastructure only).

Both sides of every parity check draw from numpy's PCG64
(`np.random.default_rng(seed)`, float32 normals), so the GPU and the CPU see
byte-identical inputs.  Seeds are fixed per config and tensor:
seed = 1000 * config + tensor_index.  bf16 tensors are the RNE rounding of
the float32 draw and travel as uint16 bits.
"""

from __future__ import annotations

import numpy as np

from .bf16 import to_bf16_bits


def rng(config: int, tensor: int) -> np.random.Generator:
    return np.random.default_rng(1000 * config + tensor)


def normal_f32(config: int, tensor: int, shape, std=1.0, mean=0.0) -> np.ndarray:
    x = rng(config, tensor).standard_normal(size=shape, dtype=np.float32)
    if std != 1.0:
        x *= np.float32(std)
    if mean != 0.0:
        x += np.float32(mean)
    return x


def normal_bf16(config: int, tensor: int, shape, std=1.0, mean=0.0) -> np.ndarray:
    return to_bf16_bits(normal_f32(config, tensor, shape, std=std, mean=mean))


def uniform_ids(config: int, tensor: int, shape, high: int) -> np.ndarray:
    return rng(config, tensor).integers(0, high, size=shape, dtype=np.int32)


# ---- the benchmark configs (C1 MLP, C2 fusions, C3 SDPA, C4 indexing)

def c1_mlp():
    """C1: x[256,1024], W1[1024,4096], b1[4096], W2[4096,1024], b2[1024] ~ N(0, 0.02) fp32."""
    return dict(
        x=normal_f32(1, 0, (256, 1024), std=0.02),
        w1=normal_f32(1, 1, (1024, 4096), std=0.02),
        b1=normal_f32(1, 2, (4096,), std=0.02),
        w2=normal_f32(1, 3, (4096, 1024), std=0.02),
        b2=normal_f32(1, 4, (1024,), std=0.02),
    )


def c2_layernorm(rows=8192, cols=4096):
    """C2a: x ~ N(0,1), gamma ~ N(1, 0.1), beta ~ N(0, 0.1), all bf16."""
    return dict(
        x=normal_bf16(2, 0, (rows, cols)),
        gamma=normal_bf16(2, 1, (cols,), std=0.1, mean=1.0),
        beta=normal_bf16(2, 2, (cols,), std=0.1),
    )


def c2_gelu(rows=8192, cols=16384):
    """C2b: x ~ N(0,1) bf16."""
    return dict(x=normal_bf16(2, 3, (rows, cols)))


def c2_reduce(rows=65536, cols=1024):
    """C2c/d: x ~ N(0,1) bf16 for reduce_sum and argmax."""
    return dict(x=normal_bf16(2, 4, (rows, cols)))


def c3_sdpa(seq, batch=4, heads=16, dim=128):
    """C3: Q, K, V ~ N(0,1)/sqrt(128) bf16, [B, H, S, D]."""
    shape = (batch, heads, seq, dim)
    s = 1.0 / np.sqrt(128.0)
    return dict(
        q=normal_bf16(3, 0, shape, std=s),
        k=normal_bf16(3, 1, shape, std=s),
        v=normal_bf16(3, 2, shape, std=s),
    )


def c4_indexing(n_ids=(32, 2048), vocab=50257, dim=768):
    """C4: ids ~ U[0, 50257) int32, table[50257, 768] bf16 ~ N(0,1) for the
    gather; grads[prod(n_ids), 768] fp32 ~ N(0,1) and a random fp32 table
    for the scatter-add."""
    ids = uniform_ids(4, 0, n_ids, vocab)
    return dict(
        ids=ids,
        table_bf16=normal_bf16(4, 1, (vocab, dim)),
        table_f32=normal_f32(4, 2, (vocab, dim)),
        grads=normal_f32(4, 3, (int(np.prod(n_ids)), dim)),
    )
