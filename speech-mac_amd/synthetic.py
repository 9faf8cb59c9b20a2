"""Seeded synthetic inputs of the Flow decode step (no checkpoint is used).

Q8 weights: q ~ U{-127..127}; one scale per row ~ U[1e-3, 1e-2] drawn in fp32,
rounded to fp16 and stored in every 32-column Q8_0 block of the row, so the
matrix is both "per-row fp32 scale" and a valid GGML Q8_0 tensor
(src/phonon_q8.h:7-17). Norm vectors are BF16 (src/phonon_transformer.h:30).
"""
from __future__ import annotations

import numpy as np

from . import FFN, Q8_BLOCK, WIDTH


def bf16_bits(x) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def q8_matrix(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    assert cols % 32 == 0
    q = rng.integers(-127, 128, size=(rows, cols), dtype=np.int8)
    scale = rng.uniform(1e-3, 1e-2, size=rows).astype(np.float32)
    bits = scale.astype(np.float16).view(np.uint16)
    blocks = np.empty(rows * cols // 32, Q8_BLOCK)
    blocks["scale_bits"] = np.repeat(bits, cols // 32)
    blocks["values"] = q.reshape(-1, 32)
    return blocks


def flow_layer(rng: np.random.Generator, dtype: str = "q8") -> dict:
    """One layer: Q8 (or BF16) matrices and BF16 LayerNorm vectors."""
    shapes = {"qkv": (3 * WIDTH, WIDTH), "out": (WIDTH, WIDTH),
              "mlp_in": (FFN, WIDTH), "mlp_out": (WIDTH, FFN)}
    layer = {}
    for name, (r, c) in shapes.items():
        if dtype == "q8":
            layer[name] = q8_matrix(rng, r, c)
        else:
            layer[name] = bf16_bits(rng.standard_normal((r, c)).astype(np.float32) * 0.04)
    layer["norm1_weight"] = bf16_bits(1.0 + 0.1 * rng.standard_normal(WIDTH))
    layer["norm1_bias"] = bf16_bits(0.1 * rng.standard_normal(WIDTH))
    layer["norm2_weight"] = bf16_bits(1.0 + 0.1 * rng.standard_normal(WIDTH))
    layer["norm2_bias"] = bf16_bits(0.1 * rng.standard_normal(WIDTH))
    return layer


def flow_model(seed: int, layers: int, dtype: str = "q8") -> list:
    rng = np.random.default_rng(seed)
    return [flow_layer(rng, dtype) for _ in range(layers)]


def contexts(seed: int, streams: int, low: int, high: int) -> np.ndarray:
    """Per-stream committed lengths ~ U{low..high} (the step attends length+1
    keys after appending at position = length)."""
    rng = np.random.default_rng(seed)
    return rng.integers(low, high + 1, size=streams)


def block_tables(seed: int, lengths, capacity_blocks: int, total_blocks: int):
    """Shuffled block tables (seeded Fisher-Yates over the pool's ids): each
    stream gets capacity_blocks distinct ids."""
    rng = np.random.default_rng(seed)
    streams = len(lengths)
    assert streams * capacity_blocks <= total_blocks
    ids = rng.permutation(total_blocks)[: streams * capacity_blocks].astype(np.int32)
    return ids.reshape(streams, capacity_blocks)
