"""GPU parity of the KIVI 2/4/8-bit cold format: packed blocks and dequantised
values bit-exact with the oracle; decode attention over quantised blocks
plus unquantised recent rows within the 16-bit tolerance of the float64
closed form over the dequantised cache."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import kivi as K
from oracle.inputs import decode_inputs

pytestmark = pytest.mark.gpu
TDT = {"bfloat16": torch.bfloat16, "float16": torch.float16}


def _gpu(a, dtype, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(TDT[dtype])


def _edge_cases(k, v, bits=2):
    """Plant the edge groups of the format: a constant K channel group (zero
    range: fp16 scale 0), a constant V token group, +/- extremes, and a K
    and a V group of ties (range qmax, half-integer values: the quotient
    lands exactly on .5)."""
    k = k.copy()
    v = v.copy()
    k[0, 0, 0:32, 5] = 0.75          # constant K group (per channel, 32 tokens)
    v[0, 0, 3, 32:64] = -1.5         # constant V group (per token, 32 channels)
    k[0, -1, 40, 7] = 60.0           # large outlier
    v[0, -1, 70, v.shape[-1] - 5] = -60.0
    qmax = (1 << bits) - 1
    ties = np.minimum(np.array([0.0, float(qmax)] + [0.5 + j for j in range(30)], np.float32), qmax)
    k[0, 0, 64:96, 9] = ties         # K channel group of ties
    v[0, -1, 100, 0:32] = ties       # V token group of ties
    return k, v


@pytest.mark.parametrize("dtype,bits,D", [("float16", 2, 128), ("bfloat16", 2, 128), ("float16", 4, 64),
                                          ("float16", 2, 256), ("float16", 8, 128), ("bfloat16", 8, 64),
                                          ("bfloat16", 8, 256), ("float16", 4, 256)])
def test_quantize_and_dequantize_bitexact(dev, dtype, bits, D):
    from halo_amd import kivi
    x = decode_inputs(4, B=1, H=4, H_kv=2, T=256, D=D, dtype=dtype, n_planted=2, sigma=10.0)
    k, v = _edge_cases(x.k, x.v, bits)
    from oracle.inputs import round_to
    k, v = round_to(k, dtype), round_to(v, dtype)
    blocks = kivi.quantize(_gpu(k, dtype, dev), _gpu(v, dtype, dev), bits=bits)
    want = K.pack_blocks(k, v, bits=bits, dtype=dtype)
    got = blocks.cpu().numpy()
    assert got.shape == want.shape
    assert np.array_equal(got, want), f"{(got != want).sum()} of {got.size} bytes differ"
    kd, vd = kivi.dequantize(blocks, D=D, dtype=TDT[dtype], bits=bits)
    rk, rv = K.unpack_blocks(want, D=D, bits=bits, dtype=dtype)
    assert np.array_equal(kd.float().cpu().numpy(), rk)
    assert np.array_equal(vd.float().cpu().numpy(), rv)


def test_quantize_strided_views(dev):
    """Inputs that are views into a larger cache (non-contiguous rows)."""
    from halo_amd import kivi
    x = decode_inputs(9, B=2, H=4, H_kv=2, T=192, D=128, dtype="float16")
    big_k = torch.zeros((2, 2, 256, 128), device=dev, dtype=torch.float16)
    big_v = torch.zeros_like(big_k)
    big_k[:, :, 32:224] = _gpu(x.k, "float16", dev)
    big_v[:, :, 32:224] = _gpu(x.v, "float16", dev)
    blocks = kivi.quantize(big_k[:, :, 32:224], big_v[:, :, 32:224])
    assert np.array_equal(blocks.cpu().numpy(), K.pack_blocks(x.k, x.v, bits=2, dtype="float16"))


@pytest.mark.parametrize("dtype,H,H_kv", [("float16", 28, 4), ("bfloat16", 32, 8), ("float16", 8, 8)])
def test_kivi_decode_matches_closed_form(dev, dtype, H, H_kv):
    from halo_amd import kivi
    from halo_amd.decode import ChunkRef
    T_cold, T_rec, D = 2048, 128, 128
    T = T_cold + T_rec
    x = decode_inputs(4, B=1, H=H, H_kv=H_kv, T=T, D=D, dtype=dtype, n_planted=2, sigma=10.0)
    q, k, v = (_gpu(a, dtype, dev) for a in (x.q, x.k, x.v))
    blocks = kivi.quantize(k[:, :, :T_cold], v[:, :, :T_cold])
    recent = [ChunkRef(k[:, :, T_cold:], v[:, :, T_cold:], T_cold, True)]
    layer = kivi.KiviDecodeLayer(B=1, H=H, H_kv=H_kv, D=D, dtype=TDT[dtype], cold_blocks=blocks, recent=recent,
                                 device=dev, chunk_tokens=512)
    out = torch.empty((1, H, D), device=dev, dtype=TDT[dtype])
    lse = torch.empty((1, H), device=dev)
    scale = 1 / math.sqrt(D)
    layer.step(q[:, :, 0], scale=scale, out=out, lse=lse,
               q_pos=torch.tensor([T - 1], device=dev, dtype=torch.int64))
    kd, vd = K.unpack_blocks(K.pack_blocks(x.k[:, :, :T_cold], x.v[:, :, :T_cold], bits=2, dtype=dtype),
                             D=D, bits=2, dtype=dtype)
    kk = np.concatenate([kd, x.k[:, :, T_cold:]], axis=2)
    vv = np.concatenate([vd, x.v[:, :, T_cold:]], axis=2)
    ro, rl = A.attention_f64(x.q[:, :, 0], kk, vv, scale=scale)
    assert np.abs(out.float().cpu().numpy() - ro).max() <= 2e-2
    # The kernel folds code*scale + zero into the products, i.e. it attends
    # over the dequantised values before their final rounding to the dtype:
    # against the rounded cache the LSE moves by that rounding (bf16: up to a
    # few 1e-3, inside the 16-bit bound 2e-2), against the unrounded values
    # it agrees to 1e-3 in both dtypes.
    assert np.abs(lse.cpu().numpy() - rl).max() <= (1e-3 if dtype == "float16" else 2e-2)
    ck, sk, zk = K.quantize_k_per_channel(x.k[:, :, :T_cold], bits=2, group_size=32, dtype=dtype)
    cv, sv, zv = K.quantize_v_per_token(x.v[:, :, :T_cold], bits=2, group_size=32, dtype=dtype)
    ku = ck.astype(np.float64) * np.repeat(sk, 32, axis=-2) + np.repeat(zk, 32, axis=-2)
    vu = cv.astype(np.float64) * np.repeat(sv, 32, axis=-1) + np.repeat(zv, 32, axis=-1)
    ro_u, rl_u = A.attention_f64(x.q[:, :, 0], np.concatenate([ku, x.k[:, :, T_cold:]], axis=2),
                                 np.concatenate([vu, x.v[:, :, T_cold:]], axis=2), scale=scale)
    assert np.abs(lse.cpu().numpy() - rl_u).max() <= 1e-3
    assert np.abs(out.float().cpu().numpy() - ro_u).max() <= 2e-2


def test_kivi_decode_causal_and_split(dev):
    """A query position inside the quantised region masks later blocks; a
    split that is not a block multiple is refused."""
    from halo_amd import kivi
    from halo_amd.decode import build_plan, launch
    x = decode_inputs(5, B=2, H=8, H_kv=2, T=1024, D=64, dtype="float16")
    q, k, v = (_gpu(a, "float16", dev) for a in (x.q, x.k, x.v))
    blocks = kivi.quantize(k, v)
    ref = [kivi.KiviChunkRef(blocks, 0, True)]
    with pytest.raises(AssertionError):
        build_plan(B=2, H=8, H_kv=2, D=64, dtype=torch.float16, chunks=ref, device=dev, split=48)
    plan = build_plan(B=2, H=8, H_kv=2, D=64, dtype=torch.float16, chunks=ref, device=dev, split=256)
    qp = np.array([700, 1023])
    out = torch.empty((2, 8, 64), device=dev)
    lse = torch.empty((2, 8), device=dev)
    launch(plan, q[:, :, 0], scale=0.125, q_pos=torch.from_numpy(qp).to(dev), out=out, lse=lse)
    kd, vd = K.unpack_blocks(K.pack_blocks(x.k, x.v, bits=2, dtype="float16"), D=64, bits=2, dtype="float16")
    ro, rl = A.attention_f64(x.q[:, :, 0], kd, vd, scale=0.125, q_pos=qp)
    assert np.abs(out.cpu().numpy() - ro).max() <= 2e-2
    assert np.abs(lse.cpu().numpy() - rl).max() <= 1e-3
