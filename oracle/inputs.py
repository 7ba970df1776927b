"""Seeded synthetic inputs for the tiered-KV workloads (numpy, CPU).

Test infrastructure only.  Values are drawn in float32 with
``numpy.random.default_rng(seed)`` (PCG64, stable across numpy releases) and,
for bf16/fp16 workloads, rounded to that dtype here so the GPU tensors built
from them hold exactly the same numbers.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16, returned as uint16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7F800000) == 0x7F800000
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "float32":
        return x.astype(np.float32)
    if dtype == "bfloat16":
        return round_bf16(x)
    if dtype == "float16":
        return x.astype(np.float16).astype(np.float32)
    raise ValueError(dtype)


@dataclass
class DecodeInputs:
    q: np.ndarray   # (B, H, 1, D) float32 holding dtype-exact values
    k: np.ndarray   # (B, H_kv, T, D)
    v: np.ndarray
    dtype: str
    planted: np.ndarray  # planted key channels (may be empty)


def decode_inputs(seed: int, *, B: int, H: int, H_kv: int, T: int, D: int,
                  dtype: str = "float32", n_planted: int = 0, sigma: float = 1.0,
                  q_scale: float = 1.0) -> DecodeInputs:
    """q, k, v ~ N(0, 1); ``n_planted`` key channels (seeded choice) drawn
    from N(0, sigma^2) instead."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, H, 1, D), dtype=np.float32) * np.float32(q_scale)
    k = rng.standard_normal((B, H_kv, T, D), dtype=np.float32)
    v = rng.standard_normal((B, H_kv, T, D), dtype=np.float32)
    planted = np.sort(rng.choice(D, size=n_planted, replace=False)) if n_planted else np.zeros(0, int)
    if n_planted:
        k[..., planted] *= np.float32(sigma)
    return DecodeInputs(round_to(q, dtype), round_to(k, dtype), round_to(v, dtype), dtype, planted)


# Workload shapes (the five benchmark configurations).
C1 = dict(seed=0, B=1, H=8, H_kv=8, T=4096, D=64, dtype="float32", chunk=256, n_hot=4, top_k=2)
C2 = dict(seed=1, B=1, H=32, H_kv=8, T=32768, D=128, dtype="bfloat16", chunk=1024, n_hot=8, top_k=4,
          n_planted=4, sigma=8.0, layers=32)
C3 = dict(seed=2, B=1, H=32, H_kv=8, T_q=4096, T_prior=28672, D=128, dtype="bfloat16", chunk=1024)
C4 = dict(seed=3, B=16, H=32, H_kv=8, D=128, dtype="bfloat16", chunk=2048, lo=8192, hi=131072,
          hot_ratio=0.25, top_k=8)
C5 = dict(seed=4, B=1, H=28, H_kv=4, T=131072, D=128, dtype="float16", chunk=2048, group=32,
          residual=128, n_planted=2, sigma=10.0, layers=28)


def ragged_lengths(seed: int, n: int, lo: int, hi: int, chunk: int) -> np.ndarray:
    """ctx_i = floor(U[lo, hi] / chunk) * chunk (build-defined rounding), >= chunk."""
    rng = np.random.default_rng(seed)
    u = rng.uniform(lo, hi, size=n)
    return np.maximum((np.floor(u / chunk) * chunk).astype(np.int64), chunk)


def hot_count(n_chunks: int, hot_ratio: float) -> int:
    """Per-sequence hot chunks: the last floor(hot_ratio * n) chunks, min 1."""
    return max(1, int(np.floor(hot_ratio * n_chunks)))
