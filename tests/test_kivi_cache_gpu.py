"""GPU parity of the KIVI cache (quantise-on-demote, baselines/kivi_cache.py:
80-195): the reference tests' shapes and recent-window invariant
(tests/test_kivi_cache.py), packed blocks and the returned dequantised cache
bit-exact against the oracle over a sequence of updates, and attention over
the cache (decode in registers, T_q > 1 through the prefill) against the
float64 closed form over the dequantised values."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import kivi as K
from oracle.inputs import round_to

pytestmark = pytest.mark.gpu

TDT = {"float16": torch.float16, "bfloat16": torch.bfloat16}


def _rows(rng, shape, dtype):
    return round_to(rng.standard_normal(shape).astype(np.float32), dtype)


def _deq(k, v, n, dtype, bits=2):
    """Oracle view of the cache after n tokens were demoted: dequantised
    blocks for [0, n), the raw rows after."""
    if n == 0:
        return k, v
    kd, vd = K.unpack_blocks(K.pack_blocks(k[:, :, :n], v[:, :, :n], bits=bits, dtype=dtype), D=k.shape[-1],
                             bits=bits, dtype=dtype)
    return np.concatenate([kd, k[:, :, n:]], axis=2), np.concatenate([vd, v[:, :, n:]], axis=2)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_reference_shapes_and_recent_window(dev, dtype):
    """tests/test_kivi_cache.py:36-80: 100 then 10 tokens give 100 and 110
    rows; with residual 64, after 200 tokens 128 are quantised and the last
    64 come back bit-exact."""
    from halo_amd.kivi_cache import KIVICache
    torch.manual_seed(0)
    cache = KIVICache(bits=4, group_size=32, residual_length=32)
    B, H, D = 1, 4, 128
    kk, vv = cache.update(torch.randn(B, H, 100, D, device=dev).to(TDT[dtype]),
                          torch.randn(B, H, 100, D, device=dev).to(TDT[dtype]), layer_idx=0)
    assert kk.shape == vv.shape == (B, H, 100, D)
    kk, vv = cache.update(torch.randn(B, H, 10, D, device=dev).to(TDT[dtype]),
                          torch.randn(B, H, 10, D, device=dev).to(TDT[dtype]), layer_idx=0)
    assert kk.shape == vv.shape == (B, H, 110, D)
    assert cache.get_seq_length(0) == 110
    cache = KIVICache(bits=2, group_size=32, residual_length=64)
    k_full = torch.randn(B, H, 200, D, device=dev).to(TDT[dtype])
    v_full = torch.randn(B, H, 200, D, device=dev).to(TDT[dtype])
    cache.update(k_full[..., :100, :], v_full[..., :100, :], layer_idx=0)
    kk, vv = cache.update(k_full[..., 100:, :], v_full[..., 100:, :], layer_idx=0)
    assert cache._n_seen[0] == 128 and cache.recent(0)[0].shape[-2] == 72
    assert torch.equal(kk[..., -64:, :], k_full[..., -64:, :])
    assert torch.equal(vv[..., -64:, :], v_full[..., -64:, :])
    # storage: 2-bit blocks against 16-bit rows of the same 128 tokens
    nb = cache.blocks(0).numel()
    assert nb * 5.0 < 128 * B * H * D * 2 * 2


@pytest.mark.parametrize("dtype,residual", [("float16", 32), ("bfloat16", 48)])
def test_blocks_and_cache_bit_exact_over_updates(dev, dtype, residual):
    from halo_amd.kivi_cache import KIVICache
    rng = np.random.default_rng(6)
    B, H_kv, D = 2, 4, 128
    sizes = [300, 1, 1, 37, 1, 64, 5, 1, 90]
    T = sum(sizes)
    k = _rows(rng, (B, H_kv, T, D), dtype)
    v = _rows(rng, (B, H_kv, T, D), dtype)
    kg = torch.from_numpy(k).to(dev).to(TDT[dtype])
    vg = torch.from_numpy(v).to(dev).to(TDT[dtype])
    cache = KIVICache(bits=2, residual_length=residual)
    t = 0
    for n in sizes:
        kk, vv = cache.update(kg[:, :, t:t + n], vg[:, :, t:t + n], layer_idx=1)
        t += n
        n_seen = max(0, (t - residual) // 32 * 32)  # closed form of the demotion policy
        assert cache._n_seen[1] == n_seen and cache.get_seq_length(1) == t
        blk = cache.blocks(1)
        if n_seen:
            assert np.array_equal(blk.cpu().numpy(), K.pack_blocks(k[:, :, :n_seen], v[:, :, :n_seen], bits=2,
                                                                   dtype=dtype))
        wk, wv = _deq(k[:, :, :t], v[:, :, :t], n_seen, dtype)
        assert np.array_equal(kk.float().cpu().numpy(), wk)
        assert np.array_equal(vv.float().cpu().numpy(), wv)


@pytest.mark.parametrize("dtype,H,H_kv", [("float16", 28, 4), ("bfloat16", 32, 8)])
def test_attention_over_the_cache(dev, dtype, H, H_kv):
    """Decode through the fused-dequant kernel and T_q > 1 through the
    prefill, against the float64 closed form over the dequantised cache; a
    cache that never materialises (and splits its blocks differently)
    agrees within the merge's rounding, and bit for bit at T_q > 1."""
    from halo_amd.kivi_cache import KIVICache
    rng = np.random.default_rng(7)
    B, D, T0 = 1, 128, 3000
    k = _rows(rng, (B, H_kv, T0 + 8, D), dtype)
    v = _rows(rng, (B, H_kv, T0 + 8, D), dtype)
    kg = torch.from_numpy(k).to(dev).to(TDT[dtype])
    vg = torch.from_numpy(v).to(dev).to(TDT[dtype])
    full = KIVICache(bits=2, residual_length=128)
    lean = KIVICache(bits=2, residual_length=128, materialize=False, chunk_tokens=512)
    full.update(kg[:, :, :T0], vg[:, :, :T0], 0)
    assert lean.update(kg[:, :, :T0], vg[:, :, :T0], 0) is None
    scale = 1 / math.sqrt(D)
    for t in range(T0, T0 + 8):
        full.update(kg[:, :, t:t + 1], vg[:, :, t:t + 1], 0)
        lean.update(kg[:, :, t:t + 1], vg[:, :, t:t + 1], 0)
    T = T0 + 8
    n_seen = full._n_seen[0]
    wk, wv = _deq(k, v, n_seen, dtype)
    q = _rows(rng, (B, H, 1, D), dtype)
    qg = torch.from_numpy(q).to(dev).to(TDT[dtype])
    out, lse = full.compute_attention(qg, layer_idx=0, return_lse=True)
    out2 = lean.compute_attention(qg, layer_idx=0)
    ro, rl = A.attention_f64(q[:, :, 0], wk, wv, scale=scale)
    assert np.abs(out[:, :, 0].float().cpu().numpy() - ro).max() <= 2e-2
    assert np.abs(lse[:, :, 0].cpu().numpy() - rl).max() <= (1e-3 if dtype == "float16" else 2e-2)
    assert out.shape == (B, H, 1, D)
    # another table split of the same blocks: equal within rounding of the merge
    assert np.abs(out2[:, :, 0].float().cpu().numpy() - ro).max() <= 2e-2
    assert (out2.float() - out.float()).abs().max().item() <= 8e-3
    # causal T_q > 1: the last 40 positions as queries
    qp = _rows(rng, (B, H, 40, D), dtype)
    outp = full.compute_attention(torch.from_numpy(qp).to(dev).to(TDT[dtype]), layer_idx=0)
    wp, _ = A.prefill_f64(qp, wk, wv, scale=scale, q_start=T - 40)
    assert np.abs(outp.float().cpu().numpy() - wp).max() <= 2e-2
    outl = lean.compute_attention(torch.from_numpy(qp).to(dev).to(TDT[dtype]), layer_idx=0)
    assert torch.equal(outl, outp)


@pytest.mark.parametrize("dtype,bits", [("float16", 8), ("bfloat16", 4), ("bfloat16", 8)])
def test_wider_codes_blocks_and_attention(dev, dtype, bits):
    """4- and 8-bit caches (from_memory_ratio 4 and 2, as the reference maps
    them): blocks and the returned cache bit-exact over updates; decode (over
    the dequantised blocks: the fused kernel reads 2-bit blocks) and T_q > 1
    against the float64 closed form."""
    from halo_amd.kivi_cache import KIVICache
    rng = np.random.default_rng(11)
    B, H, H_kv, D = 1, 8, 2, 128
    sizes = [200, 1, 63, 1, 40]
    T = sum(sizes)
    k = _rows(rng, (B, H_kv, T, D), dtype)
    v = _rows(rng, (B, H_kv, T, D), dtype)
    kg = torch.from_numpy(k).to(dev).to(TDT[dtype])
    vg = torch.from_numpy(v).to(dev).to(TDT[dtype])
    cache = KIVICache.from_memory_ratio(memory_ratio=16 // bits, residual_length=32)
    assert cache.bits == bits
    t = 0
    for n in sizes:
        kk, vv = cache.update(kg[:, :, t:t + n], vg[:, :, t:t + n], layer_idx=0)
        t += n
        n_seen = max(0, (t - 32) // 32 * 32)
        assert cache._n_seen[0] == n_seen
        if n_seen:
            assert np.array_equal(cache.blocks(0).cpu().numpy(),
                                  K.pack_blocks(k[:, :, :n_seen], v[:, :, :n_seen], bits=bits, dtype=dtype))
        wk, wv = _deq(k[:, :, :t], v[:, :, :t], n_seen, dtype, bits)
        assert np.array_equal(kk.float().cpu().numpy(), wk)
        assert np.array_equal(vv.float().cpu().numpy(), wv)
    scale = 1 / math.sqrt(D)
    q = _rows(rng, (B, H, 1, D), dtype)
    out, lse = cache.compute_attention(torch.from_numpy(q).to(dev).to(TDT[dtype]), layer_idx=0, return_lse=True)
    ro, rl = A.attention_f64(q[:, :, 0], wk, wv, scale=scale)
    assert np.abs(out[:, :, 0].float().cpu().numpy() - ro).max() <= 2e-2
    assert np.abs(lse[:, :, 0].cpu().numpy() - rl).max() <= 2e-2
    qp = _rows(rng, (B, H, 16, D), dtype)
    outp = cache.compute_attention(torch.from_numpy(qp).to(dev).to(TDT[dtype]), layer_idx=0)
    wp, _ = A.prefill_f64(qp, wk, wv, scale=scale, q_start=T - 16)
    assert np.abs(outp.float().cpu().numpy() - wp).max() <= 2e-2


def _tiny_models(dev, dtype):
    from transformers import AutoModelForCausalLM
    from transformers.models.qwen2 import Qwen2Config

    def cfg():
        return Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                           num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096,
                           rope_theta=10000.0, tie_word_embeddings=False, attn_implementation="sdpa")
    torch.manual_seed(0)
    ref = AutoModelForCausalLM.from_config(cfg()).eval()
    torch.manual_seed(0)
    kv = AutoModelForCausalLM.from_config(cfg()).eval()
    kv.load_state_dict(ref.state_dict())
    return ref.to(dev, dtype), kv.to(dev, dtype)


def test_wrap_with_kivi_generate(dev):
    """``wrap_with_kivi`` (baselines/kivi_cache.py:205-226) inside a tiny
    randomly initialised Qwen2 in fp16: with a recent window longer than the
    sequence nothing is quantised and greedy generation equals the plain
    model's token for token; with a 32-token window the blocks form, every
    layer's cache holds the dequantised blocks followed by the recent rows,
    and the sequence length counts every token."""
    pytest.importorskip("transformers")
    from halo_amd import kivi
    from halo_amd.kivi_cache import KIVICache, wrap_with_kivi
    ref, kv = _tiny_models(dev, torch.float16)
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(10, 500, (1, 200), generator=g).to(dev)
    with torch.no_grad():
        want = ref.generate(ids, max_new_tokens=12, do_sample=False)
        wrap_with_kivi(kv, memory_ratio=8, residual_length=4096)
        got = kv.generate(ids, max_new_tokens=12, do_sample=False)
    assert torch.equal(got, want)
    assert kv._kivi_cache.bits == 2
    # quantised: a 32-token recent window
    _, kv2 = _tiny_models(dev, torch.float16)
    wrap_with_kivi(kv2, memory_ratio=8, residual_length=32)
    with torch.no_grad():
        out = kv2.generate(ids, max_new_tokens=8, do_sample=False)
    cache = kv2._kivi_cache
    assert isinstance(cache, KIVICache) and out.shape == (1, 208)
    T = cache.get_seq_length(0)
    assert T == 207                       # the last generated token is not fed back
    for li in range(2):
        blocks = cache.blocks(li)
        n = blocks.shape[2]
        assert n * 32 + cache.recent(li)[0].shape[-2] == T and n >= 5
        kd, vd = kivi.dequantize(blocks, D=64, dtype=torch.float16, bits=2)
        lay = cache.layers[li]
        assert lay.keys.shape[-2] == T
        assert torch.equal(lay.keys[:, :, : n * 32], kd) and torch.equal(lay.values[:, :, : n * 32], vd)
        assert torch.equal(lay.keys[:, :, n * 32:], cache.recent(li)[0])
