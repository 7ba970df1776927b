"""Oracle: KIVI-style per-group 2/4-bit quantisation (numpy).

Test infrastructure only (see oracle/__init__.py).

Arithmetic of baselines/kivi_cache.py:44-78, with every operation rounded in
the storage dtype exactly as torch evaluates a chain of fp16/bf16 tensor ops
(compute in fp32, round each result to the storage dtype; for +, -, *, /
that double rounding equals the correctly rounded fp16/bf16 result because
fp32 carries more than 2p+2 bits):

  x_min, x_max   per group of ``group_size`` consecutive elements
  scale = ((x_max - x_min).clamp_min(1e-8)) / qmax        (storage dtype)
  zero  = x_min
  code  = clamp(round_half_even((x - zero) / scale), 0, qmax)
  deq   = dtype( fp32(fp32(code) * fp32(scale)) + fp32(zero) )   -- two fp32
          roundings, no fused multiply-add, one final rounding.

Edge rule of this build: in fp16 the 1e-8 floor rounds to 0, so a constant
group has scale 0 and the reference's code is round(0/0) = NaN cast to int8
(undefined); such codes are defined here as 0 (what bf16/fp32 give).  A
nonzero difference over a zero scale is +inf and clamps to qmax, as in the
reference.

The reference quantises along the last axis only (kivi_cache.py:56).  K
"per-channel" (groups of consecutive tokens within one channel) applies the
same per-element arithmetic along the token axis.
"""
from __future__ import annotations

import numpy as np

from .inputs import round_to


def _r(x: np.ndarray, dtype: str) -> np.ndarray:
    return round_to(np.asarray(x, dtype=np.float32), dtype)


def quantize_last_axis(x: np.ndarray, *, bits: int, group_size: int, dtype: str):
    """_quantize_per_group(axis=-1) (baselines/kivi_cache.py:44-69).
    x holds dtype-exact float32 values.  Returns (codes uint8 (..., g, gs),
    scale (..., g, 1), zero (..., g, 1)) with scale/zero dtype-exact float32."""
    qmax = (1 << bits) - 1
    shape = x.shape
    n = shape[-1]
    assert n % group_size == 0
    xg = x.reshape(*shape[:-1], n // group_size, group_size).astype(np.float32)
    x_min = xg.min(axis=-1, keepdims=True)
    x_max = xg.max(axis=-1, keepdims=True)
    rng = _r(x_max - x_min, dtype)
    eps = np.float32(_r(np.float32(1e-8), dtype))
    rng = _r(np.maximum(rng, eps), dtype)
    scale = _r(rng / np.float32(qmax), dtype)
    zero = x_min
    diff = _r(xg - zero, dtype)
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = _r(diff / scale, dtype)          # x/0 -> inf (clamps to qmax)
    ratio = np.where(np.isnan(ratio), 0.0, ratio).astype(np.float32)  # 0/0 -> code 0
    codes = np.clip(np.rint(ratio), 0, qmax).astype(np.uint8)
    return codes, scale.astype(np.float32), zero.astype(np.float32)


def dequantize(codes: np.ndarray, scale: np.ndarray, zero: np.ndarray, *, dtype: str) -> np.ndarray:
    """_dequantize_per_group (baselines/kivi_cache.py:72-78) without the
    reshape: fp32 multiply, fp32 add, one rounding to ``dtype``."""
    prod = (codes.astype(np.float32) * scale.astype(np.float32)).astype(np.float32)
    s = (prod + zero.astype(np.float32)).astype(np.float32)
    return _r(s, dtype)


def quantize_v_per_token(v: np.ndarray, *, bits: int, group_size: int, dtype: str):
    """V: groups of ``group_size`` consecutive channels of one token
    (the reference's axis=-1 path).  v (..., T, D) -> codes (..., T, D),
    scale/zero (..., T, D/gs)."""
    codes, s, z = quantize_last_axis(v, bits=bits, group_size=group_size, dtype=dtype)
    return codes.reshape(v.shape), s[..., 0], z[..., 0]


def quantize_k_per_channel(k: np.ndarray, *, bits: int, group_size: int, dtype: str):
    """K: groups of ``group_size`` consecutive tokens of one channel.
    k (..., T, D) with T % gs == 0 -> codes (..., T, D), scale/zero
    (..., T/gs, D)."""
    kt = np.swapaxes(k, -1, -2)                           # (..., D, T)
    codes, s, z = quantize_last_axis(kt, bits=bits, group_size=group_size, dtype=dtype)
    codes = np.swapaxes(codes.reshape(kt.shape), -1, -2)  # (..., T, D)
    return codes, np.swapaxes(s[..., 0], -1, -2), np.swapaxes(z[..., 0], -1, -2)


def dequant_v(codes, scale, zero, *, group_size: int, dtype: str) -> np.ndarray:
    s = np.repeat(scale, group_size, axis=-1)
    z = np.repeat(zero, group_size, axis=-1)
    return dequantize(codes, s, z, dtype=dtype)


def dequant_k(codes, scale, zero, *, group_size: int, dtype: str) -> np.ndarray:
    s = np.repeat(scale, group_size, axis=-2)
    z = np.repeat(zero, group_size, axis=-2)
    return dequantize(codes, s, z, dtype=dtype)
