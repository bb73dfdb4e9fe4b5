"""Seeded inputs of the full-attention decode core (one full-attention layer),
shared by tests/golden/make_attention_golden.py, the oracle pins and the GPU
attention tests.

A case is (context, position, rows): rows consecutive decode rows at
positions position .. position + rows - 1 over a KV cache whose rows
0 .. position - 1 are already filled.  Cache rows are N(0, 1) values stored
as fp16 and widened exactly to fp32 (the reference keeps fp32 caches,
src/qwen38/qwen38_model.c:842-846); each new row is [24 x (256 q | 256
gate) | 1024 key | 1024 value] ~ N(0, 1) in fp32; q_norm / k_norm are
uniform in [0.9, 1.1].
"""
import hashlib

import numpy as np

ROW = 14336          # q+gate 12288 | key 1024 | value 1024
KEY, VALUE = 12288, 13312


def inputs(context, position, rows, seed=5):
    rng = np.random.Generator(np.random.PCG64(seed * 1000003 + position))
    key_cache = np.zeros((context, 1024), dtype=np.float32)
    value_cache = np.zeros((context, 1024), dtype=np.float32)
    key_cache[:position] = rng.normal(size=(position, 1024)).astype(np.float16).astype(np.float32)
    value_cache[:position] = rng.normal(size=(position, 1024)).astype(np.float16).astype(np.float32)
    rows_in = rng.normal(size=(rows, ROW)).astype(np.float32)
    q_norm = rng.uniform(0.9, 1.1, size=256).astype(np.float32)
    k_norm = rng.uniform(0.9, 1.1, size=256).astype(np.float32)
    return rows_in, q_norm, k_norm, key_cache, value_cache


def run_rows(core, rows_in, q_norm, k_norm, key_cache, value_cache, position):
    """core(q_and_gate, key, value, key_cache, value_cache, q_norm, k_norm,
    position) -> attention[6144] for one row (updates the caches); returns
    [rows, 6144]."""
    out = []
    for t, row in enumerate(rows_in):
        out.append(core(row[:KEY], row[KEY:VALUE], row[VALUE:], key_cache, value_cache, q_norm, k_norm,
                        position + t))
    return np.stack(out)


def digest(array):
    return hashlib.sha256(np.ascontiguousarray(array, dtype=np.float32).tobytes()).hexdigest()
