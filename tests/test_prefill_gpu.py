"""GPU parity of the MFMA chunked causal prefill against the float64 closed
form (2e-2 max-abs on the 16-bit output, 1e-3 on the LSE)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle.inputs import decode_inputs, round_to

pytestmark = pytest.mark.gpu
TDT = {"bfloat16": torch.bfloat16, "float16": torch.float16}


def _gpu(a, dtype, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(TDT[dtype])


def _case(seed, *, B, H, H_kv, T_prior, T_q, D, dtype, chunk):
    rng = np.random.default_rng(seed)
    T = T_prior + T_q
    k = round_to(rng.standard_normal((B, H_kv, T, D), dtype=np.float32), dtype)
    v = round_to(rng.standard_normal((B, H_kv, T, D), dtype=np.float32), dtype)
    q = round_to(rng.standard_normal((B, H, T_q, D), dtype=np.float32), dtype)
    return q, k, v


@pytest.mark.parametrize("dtype,H,H_kv,D,T_prior,T_q,chunk", [
    ("bfloat16", 8, 2, 128, 384, 200, 128),     # ragged query block, 3 prior chunks
    ("float16", 4, 4, 64, 256, 128, 64),        # MHA, d64
    ("bfloat16", 32, 8, 128, 1024, 256, 256),   # 8B GQA shape, small
    ("bfloat16", 4, 1, 128, 0, 300, 128),       # self chunk only
    ("bfloat16", 14, 2, 128, 192, 77, 64),      # rep 7: flattened rows straddle positions, ragged last block
    ("float16", 16, 2, 64, 130, 45, 64),        # rep 8, d64, ragged prior chunk
])
def test_prefill_matches_closed_form(dev, dtype, H, H_kv, D, T_prior, T_q, chunk):
    from halo_amd.decode import ChunkRef
    from halo_amd.prefill import prefill_attention
    q, k, v = _case(7, B=1, H=H, H_kv=H_kv, T_prior=T_prior, T_q=T_q, D=D, dtype=dtype, chunk=chunk)
    qg, kg, vg = (_gpu(a, dtype, dev) for a in (q, k, v))
    chunks = [ChunkRef(kg[:, :, s:min(s + chunk, T_prior)], vg[:, :, s:min(s + chunk, T_prior)], s, False)
              for s in range(0, T_prior, chunk)]
    chunks.append(ChunkRef(kg[:, :, T_prior:], vg[:, :, T_prior:], T_prior, True))
    scale = 1 / math.sqrt(D)
    out, lse = prefill_attention(qg, chunks, scale=scale, return_lse=True)
    torch.cuda.synchronize()
    ro, rl = A.prefill_f64(q, k, v, scale=scale, q_start=T_prior)
    assert np.abs(out.float().cpu().numpy() - ro).max() <= 2e-2
    assert np.abs(lse.cpu().numpy() - rl).max() <= 1e-3


def test_prefill_chunk_order_and_partition_invariance(dev):
    """Splitting the prior context differently or listing chunks in another
    order changes nothing beyond rounding (the LSE merge is associative)."""
    from halo_amd.decode import ChunkRef
    from halo_amd.prefill import prefill_attention
    q, k, v = _case(3, B=2, H=8, H_kv=2, T_prior=512, T_q=128, D=128, dtype="bfloat16", chunk=128)
    qg, kg, vg = (_gpu(a, "bfloat16", dev) for a in (q, k, v))
    self_c = ChunkRef(kg[:, :, 512:], vg[:, :, 512:], 512, True)
    a = [ChunkRef(kg[:, :, s:s + 128], vg[:, :, s:s + 128], s, False) for s in range(0, 512, 128)] + [self_c]
    b = [ChunkRef(kg[:, :, s:s + 256], vg[:, :, s:s + 256], s, False) for s in (256, 0)] + [self_c]
    oa, la = prefill_attention(qg, a, return_lse=True, out_dtype=torch.float32)
    ob, lb = prefill_attention(qg, b, return_lse=True, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert (oa - ob).abs().max().item() <= 2e-2
    assert (la - lb).abs().max().item() <= 1e-3


def test_prefill_fp32_runs_on_the_decode_path(dev):
    """fp32 queries are accepted (the reference computes any T_q in fp32,
    halo/kv_cache_chunked.py:241-276) and match the float64 closed form."""
    from halo_amd.decode import ChunkRef
    from halo_amd.prefill import prefill_attention
    rng = np.random.default_rng(21)
    q = rng.standard_normal((1, 4, 16, 64)).astype(np.float32)
    k = rng.standard_normal((1, 2, 80, 64)).astype(np.float32)
    v = rng.standard_normal((1, 2, 80, 64)).astype(np.float32)
    kd, vd = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)
    out = prefill_attention(torch.from_numpy(q).to(dev), [ChunkRef(kd[:, :, :64], vd[:, :, :64], 0, True),
                                                          ChunkRef(kd[:, :, 64:], vd[:, :, 64:], 64, True)])
    want, _ = A.prefill_f64(q, k, v, scale=1 / math.sqrt(64), q_start=80 - 16)
    assert np.abs(out.cpu().numpy() - want).max() <= 1e-5
