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


# ---------------------------------------------------------------------------
# Packed block layout of this build (the reference stores unpacked int8 codes,
# kivi_cache.py:50-53).  One block = 32 tokens of one (b, h_kv):
#   K codes (32 token rows x D*bits/8), K scale (D), K zero (D),
#   V codes (D channel rows x 32*bits/8), V scale (D/32 groups x 32 tokens),
#   V zero (D/32 x 32); scales/zeros in the storage dtype.  Within a row:
#   4-bit codes, element e at bit 4e; 2-bit codes, each 16-bit word holds 8
#   elements, the even ones (2j) at bits 2j of its low byte and the odd ones
#   (2j+1) at bits 8+2j of its high byte.  The V side's 32 tokens are stored
#   in slot order: slot 8g + j holds token 4g + j (j < 4) or 16 + 4g + j - 4
#   (j >= 4).
# ---------------------------------------------------------------------------
GROUP = 32
V_SLOT_TOKEN = np.array([(16 if s & 4 else 0) + 4 * (s >> 3) + (s & 3) for s in range(GROUP)])  # slot -> token
V_TOKEN_SLOT = np.argsort(V_SLOT_TOKEN)                                                        # token -> slot


def block_bytes(D: int, bits: int) -> int:
    return 2 * GROUP * D * bits // 8 + 8 * D


def _dtype_bits(x: np.ndarray, dtype: str) -> np.ndarray:
    from .inputs import f32_to_bf16_bits
    x = np.asarray(x, np.float32)
    if dtype == "float16":
        return x.astype(np.float16).view(np.uint16)
    return f32_to_bf16_bits(x)


def _bits_to_f32(b: np.ndarray, dtype: str) -> np.ndarray:
    from .inputs import bf16_bits_to_f32
    b = np.asarray(b, np.uint16)
    if dtype == "float16":
        return b.view(np.float16).astype(np.float32)
    return bf16_bits_to_f32(b)


def code_bit(n: int, bits: int) -> np.ndarray:
    """Bit position, within a row, of each of the row's n elements."""
    e = np.arange(n)
    if bits == 2:
        return 16 * (e >> 3) + 2 * ((e & 7) >> 1) + 8 * (e & 1)
    return e * bits


def _pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """codes (..., D) uint8 -> (..., D*bits/8) bytes, element e at code_bit(D, bits)[e]."""
    n = codes.shape[-1]
    pos = code_bit(n, bits)
    out = np.zeros((*codes.shape[:-1], n * bits // 8), np.uint32)
    for e in range(n):
        out[..., pos[e] >> 3] |= codes[..., e].astype(np.uint32) << np.uint32(pos[e] & 7)
    return out.astype(np.uint8)


def _unpack_codes(packed: np.ndarray, bits: int) -> np.ndarray:
    n = packed.shape[-1] * 8 // bits
    pos = code_bit(n, bits)
    p = packed.astype(np.uint32)
    return ((p[..., pos >> 3] >> (pos & 7).astype(np.uint32)) & np.uint32((1 << bits) - 1)).astype(np.uint8)


def pack_blocks(k: np.ndarray, v: np.ndarray, *, bits: int, dtype: str) -> np.ndarray:
    """k, v (B, H_kv, T, D) dtype-exact float32, T % 32 == 0 -> uint8
    (B, H_kv, T/32, block_bytes): K per-channel and V per-token groups of 32."""
    B, H, T, D = k.shape
    nb = T // GROUP
    ck, sk, zk = quantize_k_per_channel(k, bits=bits, group_size=GROUP, dtype=dtype)   # sk (B,H,nb,D)
    cv, sv, zv = quantize_v_per_token(v, bits=bits, group_size=GROUP, dtype=dtype)     # sv (B,H,T,D/32)
    ck = ck.reshape(B, H, nb, GROUP, D)
    cv = cv.reshape(B, H, nb, GROUP, D)
    NG = D // GROUP
    sv = np.swapaxes(sv.reshape(B, H, nb, GROUP, NG), -1, -2)[..., V_SLOT_TOKEN]   # (.., NG, 32 slots)
    zv = np.swapaxes(zv.reshape(B, H, nb, GROUP, NG), -1, -2)[..., V_SLOT_TOKEN]
    parts = [
        _pack_codes(ck, bits).reshape(B, H, nb, -1),
        _dtype_bits(sk, dtype).view(np.uint8).reshape(B, H, nb, -1),
        _dtype_bits(zk, dtype).view(np.uint8).reshape(B, H, nb, -1),
        _pack_codes(np.ascontiguousarray(np.swapaxes(cv, -1, -2)[..., V_SLOT_TOKEN]), bits).reshape(B, H, nb, -1),
        _dtype_bits(np.ascontiguousarray(sv), dtype).view(np.uint8).reshape(B, H, nb, -1),
        _dtype_bits(np.ascontiguousarray(zv), dtype).view(np.uint8).reshape(B, H, nb, -1),
    ]
    out = np.concatenate(parts, axis=-1)
    assert out.shape[-1] == block_bytes(D, bits)
    return np.ascontiguousarray(out)


def unpack_blocks(blocks: np.ndarray, *, D: int, bits: int, dtype: str):
    """Inverse of pack_blocks through the dequant arithmetic: returns the
    dequantised (k, v) (B, H_kv, T, D) as dtype-exact float32."""
    B, H, nb, nbytes = blocks.shape
    C = GROUP * D * bits // 8
    assert nbytes == block_bytes(D, bits)
    o = 0
    ck = _unpack_codes(blocks[..., o:o + C].reshape(B, H, nb, GROUP, D * bits // 8), bits); o += C
    sk = _bits_to_f32(blocks[..., o:o + 2 * D].copy().view(np.uint16), dtype); o += 2 * D
    zk = _bits_to_f32(blocks[..., o:o + 2 * D].copy().view(np.uint16), dtype); o += 2 * D
    cv = np.swapaxes(_unpack_codes(blocks[..., o:o + C].reshape(B, H, nb, D, GROUP * bits // 8), bits)
                     [..., V_TOKEN_SLOT], -1, -2); o += C
    sv = np.swapaxes(_bits_to_f32(blocks[..., o:o + 2 * D].copy().view(np.uint16), dtype)
                     .reshape(B, H, nb, D // GROUP, GROUP)[..., V_TOKEN_SLOT], -1, -2); o += 2 * D
    zv = np.swapaxes(_bits_to_f32(blocks[..., o:o + 2 * D].copy().view(np.uint16), dtype)
                     .reshape(B, H, nb, D // GROUP, GROUP)[..., V_TOKEN_SLOT], -1, -2)
    k = dequantize(ck, sk[:, :, :, None, :], zk[:, :, :, None, :], dtype=dtype)
    v = dequantize(cv, np.repeat(sv, GROUP, axis=-1), np.repeat(zv, GROUP, axis=-1), dtype=dtype)
    return k.reshape(B, H, nb * GROUP, D), v.reshape(B, H, nb * GROUP, D)
