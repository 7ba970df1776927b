"""Pins the oracle (CPU only).

Each check below is chosen so that a plausible mistake in the restatement
(a dropped scale, a wrong GQA head mapping, a sign error in the merge, an
off-by-one causal rule) fails it: the restatement is compared with the
float64 closed form, with invariances of the math, with the reference
tests' own expectations, and with torch's CPU kernels where the reference's
arithmetic is a torch op.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import attention as A
from oracle import kivi as KV
from oracle import scoring as S
from oracle.inputs import decode_inputs, round_bf16


def _qkv(B=1, H=4, H_kv=4, T=128, D=32, seed=0):
    x = decode_inputs(seed, B=B, H=H, H_kv=H_kv, T=T, D=D)
    return x.q, x.k, x.v


# ---------------------------------------------------------------- attention
@pytest.mark.parametrize("T", [1, 16, 128, 1024])
@pytest.mark.parametrize("chunk", [1, 16, 64, 256, 1024])
def test_chunk_walk_matches_closed_form(T, chunk):
    """reference tests/test_kv_cache_chunked.py:66-94 against float64."""
    q, k, v = _qkv(T=T)
    scale = 1 / math.sqrt(q.shape[-1])
    ref, ref_lse = A.attention_f64(q[:, :, 0], k, v, scale=scale)
    out, lse, n = A.compute_attention(q, None, None, k, v, chunk_size=chunk)
    assert n == -(-T // chunk)
    np.testing.assert_allclose(out[:, :, 0], ref, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(lse[:, :, 0], ref_lse, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("H,H_kv", [(8, 1), (8, 2), (8, 4), (8, 8), (16, 2), (28, 4)])
def test_gqa_head_mapping(H, H_kv):
    """reference tests/test_kv_cache_chunked.py:123-131; also shows a wrong
    mapping (h % H_kv instead of h // rep) is caught."""
    q, k, v = _qkv(H=H, H_kv=H_kv, T=64)
    scale = 1 / math.sqrt(q.shape[-1])
    ref, _ = A.attention_f64(q[:, :, 0], k, v, scale=scale)
    out, _ = A.chunk_attention(q, k, v)
    np.testing.assert_allclose(out[:, :, 0], ref, atol=1e-5)
    if H_kv not in (1, H):
        wrong = np.stack([k[:, h % H_kv] for h in range(H)], axis=1)
        wv = np.stack([v[:, h % H_kv] for h in range(H)], axis=1)
        bad, _ = A.chunk_attention(q, wrong, wv)
        assert np.abs(bad[:, :, 0] - ref).max() > 1e-3


def test_closed_form_lse_and_scale_are_load_bearing():
    q, k, v = _qkv(T=256, D=64)
    scale = 1 / math.sqrt(64)
    _, lse = A.attention_f64(q[:, :, 0], k, v, scale=scale)
    s = np.einsum("bhd,bhtd->bht", q[:, :, 0].astype(np.float64), k.astype(np.float64)) * scale
    direct = np.log(np.exp(s).sum(-1))
    np.testing.assert_allclose(lse, direct, rtol=1e-12)
    _, lse_noscale = A.attention_f64(q[:, :, 0], k, v, scale=1.0)
    assert np.abs(lse_noscale - lse).max() > 1e-2


def test_lse_merge_guards_and_sign():
    rng = np.random.default_rng(5)
    oa, ob = rng.standard_normal((2, 3, 8)).astype(np.float32)
    la = np.array([0.5, -np.inf, 1.0], np.float32)
    lb = np.array([-0.25, 2.0, -np.inf], np.float32)
    out, lse = A.lse_merge(oa, la, ob, lb)
    wa, wb = np.exp(la[0] - np.logaddexp(la[0], lb[0])), np.exp(lb[0] - np.logaddexp(la[0], lb[0]))
    np.testing.assert_allclose(out[0], wa * oa[0] + wb * ob[0], rtol=1e-6)
    np.testing.assert_allclose(out[1], ob[1], rtol=1e-6)   # -inf side has zero weight
    np.testing.assert_allclose(out[2], oa[2], rtol=1e-6)
    assert lse[1] == np.float32(2.0) and lse[2] == np.float32(1.0)
    nan_out, _ = A.lse_merge(np.full((1, 8), np.nan, np.float32), np.array([-np.inf], np.float32),
                             ob[:1], np.array([0.0], np.float32))
    assert np.isfinite(nan_out).all()


@pytest.mark.parametrize("q_pos", [0, 511, 1024, 2047])
def test_chunked_decode_causal_and_partition(q_pos):
    """causal rule chunk_start + j <= q_pos (halo/triton_chunked.py:114-119),
    non-contiguous partitions and permuted order
    (reference tests/test_triton_chunked.py:100-132, 190-275)."""
    x = decode_inputs(4, B=1, H=8, H_kv=2, T=2048, D=64, q_scale=1.0)
    q, k, v = x.q, x.k, x.v
    scale = 1 / 8
    intervals = [(0, 256), (768, 1024), (1280, 1408), (1536, 1664), (1856, 2048)]
    keep = np.zeros(2048, bool)
    for lo, hi in intervals:
        keep[lo:hi] = True
    qp = np.array([q_pos])
    ref, ref_lse = A.attention_f64(q[:, :, 0], k, v, scale=scale, keep=keep, q_pos=qp)
    chunks = [(k[..., lo:hi, :], v[..., lo:hi, :], lo, True) for lo, hi in intervals]
    out, lse = A.chunked_decode(q, chunks, scale=scale, q_pos=qp)
    np.testing.assert_allclose(out, ref, atol=1e-5)
    np.testing.assert_allclose(lse, ref_lse, atol=1e-5)
    rng = np.random.default_rng(0)
    perm = [chunks[i] for i in rng.permutation(len(chunks))]
    out_p, lse_p = A.chunked_decode(q, perm, scale=scale, q_pos=qp)
    np.testing.assert_allclose(out_p, ref, atol=1e-5)
    # off-by-one causal rule (j < q_pos) must differ when q_pos is a kept row
    if keep[q_pos]:
        keep2 = keep.copy()
        keep2[q_pos] = False
        wrong, _ = A.attention_f64(q[:, :, 0], k, v, scale=scale, keep=keep2, q_pos=qp)
        assert np.abs(wrong - ref).max() > 1e-6


def test_fully_masked_chunks_have_zero_weight():
    x = decode_inputs(7, B=1, H=4, H_kv=1, T=512, D=64)
    q, k, v = x.q, x.k, x.v
    chunks = [(k[..., :256, :], v[..., :256, :], 0, True), (k[..., 256:, :], v[..., 256:, :], 256, True)]
    out, lse = A.chunked_decode(q, chunks, scale=0.125, q_pos=np.array([100]))
    ref, ref_lse = A.attention_f64(q[:, :, 0], k, v, scale=0.125, q_pos=np.array([100]))
    np.testing.assert_allclose(out, ref, atol=1e-5)
    out0, lse0 = A.chunked_decode(q, chunks[1:], scale=0.125, q_pos=np.array([100]))
    assert (out0 == 0).all() and np.isneginf(lse0).all()


@pytest.mark.parametrize("block_n", [16, 64])
def test_online_softmax_update_matches_closed_form(block_n):
    """halo/triton_chunked.py:46-138 restated; accumulators across chunks."""
    x = decode_inputs(3, B=2, H=8, H_kv=2, T=700, D=64)
    q3 = x.q[:, :, 0]
    m = np.full((2, 8), -np.inf, np.float32)
    l = np.zeros((2, 8), np.float32)
    o = np.zeros((2, 8, 64), np.float32)
    qp = np.array([650, 699])
    for c0, c1 in [(0, 300), (300, 512), (512, 700)]:
        A.update_chunk(q3, x.k[..., c0:c1, :], x.v[..., c0:c1, :], m, l, o, scale=0.125,
                       chunk_start=c0, q_pos=qp, apply_causal=True, block_n=block_n)
    out, lse = A.finalize(m, l, o)
    ref, ref_lse = A.attention_f64(q3, x.k, x.v, scale=0.125, q_pos=qp)
    np.testing.assert_allclose(out, ref, atol=1e-5)
    np.testing.assert_allclose(lse, ref_lse, atol=1e-5)


def test_prefill_brute_force_rows_match_decode():
    """Each prefill query row equals a decode query at its position."""
    x = decode_inputs(9, B=1, H=4, H_kv=2, T=96, D=32)
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 4, 8, 32)).astype(np.float32)
    out, lse = A.prefill_f64(q, x.k, x.v, scale=0.2, q_start=88)
    for i in range(8):
        o1, l1 = A.attention_f64(q[:, :, i], x.k, x.v, scale=0.2, q_pos=np.array([88 + i]))
        np.testing.assert_allclose(out[:, :, i], o1, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(lse[:, :, i], l1, rtol=1e-12)


def test_numpy_walk_matches_torch_ops():
    """The oracle's per-chunk arithmetic equals torch's CPU ops, the
    reference's own arithmetic engine, to fp32 rounding."""
    torch = pytest.importorskip("torch")
    from oracle import torch_path as TP
    x = decode_inputs(2, B=1, H=8, H_kv=2, T=1024, D=64)
    out, lse, _ = A.compute_attention(x.q, None, None, x.k, x.v, chunk_size=256)
    tq, tk, tv = (torch.from_numpy(a) for a in (x.q, x.k, x.v))
    to, tl = TP.chunk_walk(tq, [(tk[..., c:c + 256, :], tv[..., c:c + 256, :]) for c in range(0, 1024, 256)])
    np.testing.assert_allclose(out, to.numpy(), atol=2e-6)
    np.testing.assert_allclose(lse, tl.numpy(), atol=2e-6)


# ---------------------------------------------------------------- scoring
def test_topk_tie_break_and_order():
    s = np.array([1.0, 3.0, 3.0, 2.0, 3.0, 0.5], np.float32)
    assert S.topk_indices(s, 2).tolist() == [1, 2]
    assert S.topk_indices(s, 3).tolist() == [1, 2, 4]
    assert S.topk_indices(s, 4).tolist() == [1, 2, 3, 4]
    assert S.topk_indices(s, 0).tolist() == []
    assert S.topk_indices(s, 99).tolist() == [0, 1, 2, 3, 4, 5]


def test_select_chunks_brute_force():
    rng = np.random.default_rng(11)
    for trial in range(20):
        H_kv, rep, P, D = 2, 4, 12, 16
        q = rng.standard_normal((1, H_kv * rep, 1, D)).astype(np.float32)
        km = rng.standard_normal((1, H_kv, P, D)).astype(np.float32)
        eligible = np.arange(8)
        got = S.select_chunks(q, km, eligible, 3)
        qg = q.reshape(1, H_kv, rep, 1, D).mean(axis=2)
        sc = [max(float(qg[0, h, 0] @ km[0, h, p]) for h in range(H_kv)) for p in eligible]
        brute = sorted(sorted(range(len(eligible)), key=lambda i: (-sc[i], i))[:3])
        assert got.tolist() == brute


def test_ordered_dot_slice_order():
    """The scorer's fixed order: slices of 16 elements (element d of a
    fp32 row belongs to slice (d // 4) % G, and within it comes at
    position (d // (4 G), d % 4)), each summed in order, then a pairwise
    tree over slices.  Values of 2^24 make every other order give a
    different exact answer."""
    big = np.float32(2.0 ** 24)
    D = 64  # fp32: G = 4 slices
    q = np.ones(D, np.float32)

    def dot(pairs):
        k = np.zeros((1, D), np.float32)
        for d, v in pairs:
            k[0, d] = v
        return float(S.ordered_dot(q, k, "float32")[0])

    # slices 0..3 hold 2^24, 1, 1, -2^24 (elements 0, 4, 8, 12): the tree
    # adds (2^24 + 1) + (1 - 2^24) = 2^24 + (-(2^24 - 1)) = 1; a sequential
    # sum over d would give ((2^24 + 1) + 1) - 2^24 = 0.
    assert dot([(0, big), (4, 1.0), (8, 1.0), (12, -big)]) == 1.0
    # the same four values inside slice 0 (elements 0, 16, 32, 48 = p 0..3)
    # are summed in order: ((2^24 + 1) + 1) - 2^24 = 0.
    assert dot([(0, big), (16, 1.0), (32, 1.0), (48, -big)]) == 0.0
    # element order inside a piece: 2^24 + 1 + 1 at e = 0, 1, 2 of slice 1
    # rounds twice (2^24); 1 + 1 + 2^24 at e = 0, 1, 2 is exact (2^24 + 2).
    assert dot([(4, big), (5, 1.0), (6, 1.0)]) == float(big)
    assert dot([(4, 1.0), (5, 1.0), (6, big)]) == float(big) + 2.0
    # 16-bit keys: 8 elements per piece, so D = 128 has G = 8 slices;
    # elements 8 and 64 are slice 1 (p 0) and slice 0 (p 1).
    q2 = np.ones(128, np.float32)
    k2 = np.zeros((1, 128), np.float32)
    k2[0, 0], k2[0, 64], k2[0, 8], k2[0, 72] = big, 1.0, 1.0, -big
    # slice 0: 2^24 + 1 -> 2^24; slice 1: 1 - 2^24 -> -(2^24 - 1); tree: 1
    assert float(S.ordered_dot(q2, k2, "bfloat16")[0]) == 1.0


def test_ordered_scores_match_float64_within_rounding():
    rng = np.random.default_rng(3)
    for D, dtype in ((64, "float32"), (128, "bfloat16"), (256, "float16")):
        q = rng.standard_normal((1, 8, 1, D)).astype(np.float32)
        km = rng.standard_normal((1, 2, 20, D)).astype(np.float32)
        if dtype == "bfloat16":
            q, km = round_bf16(q), round_bf16(km)
        elif dtype == "float16":
            q, km = q.astype(np.float16).astype(np.float32), km.astype(np.float16).astype(np.float32)
        got = S.ordered_scores(q, km, dtype).astype(np.float64)
        ref = S.mean_key_scores(q, km, dtype).astype(np.float64)
        qg = S.gqa_mean_query(q, 2, dtype).astype(np.float64)
        mag = np.einsum("bhtd,bhpd->bhtp", np.abs(qg), np.abs(km.astype(np.float64))).max(axis=(0, 1, 2))
        bound = (16 + int(np.log2(D // 16)) + 2) * 2.0 ** -24 * mag
        assert (np.abs(got - ref) <= bound).all()
        # and the ranking agrees with the float64 one wherever the margin is clear
        elig = np.arange(20)
        srt = np.sort(ref)[::-1]
        if srt[4] - srt[5] > 1e-3:
            assert S.topk_indices(got, 5).tolist() == S.select_chunks(q, km, elig, 5, dtype).tolist()


def test_page_means_and_gqa_query_mean():
    rng = np.random.default_rng(2)
    K = rng.standard_normal((1, 2, 70, 8)).astype(np.float32)
    km = S.page_means(K, 16)
    assert km.shape == (1, 2, 4, 8)
    np.testing.assert_allclose(km[0, 1, 2], K[0, 1, 32:48].mean(0), rtol=1e-6)
    kb = S.page_means(round_bf16(K), 16, "bfloat16")
    assert np.array_equal(kb, round_bf16(kb))


def test_halo_score_reference_expectations(fake_attention):
    """reference tests/test_scorer.py:9-69."""
    attn = fake_attention(K=64).numpy()
    kw = dict(alpha=1.0, beta=0.5, gamma=2.0, sink_tokens=2, refresh_window=8)
    sc = S.halo_score(attn, step=10, **kw)
    assert sc.shape == (64,) and np.isfinite(sc).all() and sc.min() >= 0 and sc.max() <= 1
    hot = S.topk_hot(S.halo_score(fake_attention(K=128).numpy(), step=0, **kw), 0.25)
    assert hot.size == 32
    hot2 = set(S.topk_hot(S.halo_score(attn, step=0, **kw), 0.5).tolist())
    assert {0, 1} <= hot2
    rec = S.halo_score(np.zeros(32, np.float32), step=31, alpha=0.0, beta=1.0, gamma=0.0,
                       sink_tokens=2, refresh_window=8)
    assert (np.diff(rec) >= -1e-6).all()
    # closed form: sink-only score is 1 on the sink and 0 elsewhere
    z = S.halo_score(np.zeros(16, np.float32), step=0, alpha=0.0, beta=0.0, gamma=2.0,
                     sink_tokens=3, refresh_window=8)
    np.testing.assert_allclose(z, [1.0] * 3 + [0.0] * 13, atol=1e-6)


def test_halo_score_matches_torch_ops(fake_attention):
    torch = pytest.importorskip("torch")
    attn = fake_attention(K=200, seed=3)
    kw = dict(alpha=1.0, beta=0.5, gamma=2.0, sink_tokens=4, refresh_window=64)
    ours = S.halo_score(attn.numpy(), step=150, **kw)
    a = attn.float() / (attn.float().sum() + 1e-12)
    pos = torch.arange(200, dtype=torch.float32)
    rec = torch.exp(-(150 - pos).clamp(min=0.0) / 64)
    rec = rec / (rec.sum() + 1e-12)
    sink = torch.zeros(200)
    sink[:4] = 1
    sc = 1.0 * a + 0.5 * rec + 2.0 * sink
    sc = sc / (sc.max() + 1e-12)
    np.testing.assert_allclose(ours, sc.numpy(), rtol=2e-6, atol=1e-7)


def test_refetcher_bookkeeping(fake_attention):
    """reference tests/test_refetcher.py:9-43: predict_hot size
    int(0.25*64)+1 = 17; schedule hits = 1, misses = 1."""
    sc = fake_attention(K=64).numpy()
    assert S.predict_hot(sc, hot_ratio=0.25, lookahead=1).size == 17
    tiers = {(0, 0): "gpu", (0, 1): "dram"}
    hits, misses, fetch = S.schedule([0, 1, 4, 5], block_size=4,
                                     locate=lambda layer, b: tiers[(layer, b)])
    assert (hits, misses, fetch) == (1, 1, [1])


# ---------------------------------------------------------------- KIVI
def test_kivi_roundtrip_bound():
    """reference tests/test_kivi_cache.py:18-34 (bits 4, group 32)."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 4, 100, 128)).astype(np.float32)
    codes, s, z = KV.quantize_last_axis(x, bits=4, group_size=32, dtype="float32")
    dq = KV.dequantize(codes, s, z, dtype="float32").reshape(x.shape)
    xg = x.reshape(1, 4, 100, 4, 32)
    bound = np.repeat((xg.max(-1) - xg.min(-1)) / 15, 32, axis=-1).reshape(x.shape)
    assert (np.abs(x - dq) <= bound + 1e-5).all()


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_kivi_codes_match_torch_ops(dtype, bits):
    """Per-op rounding in the storage dtype equals torch's evaluation of the
    reference expression (baselines/kivi_cache.py:64-78) on the same values."""
    torch = pytest.importorskip("torch")
    tdt = getattr(torch, dtype)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 3, 64, 128)).astype(np.float32) * 3
    x[0, 0, 0, :32] = 0.5                       # a constant group
    xt = torch.from_numpy(x).to(tdt)
    xe = xt.float().numpy()
    codes, s, z = KV.quantize_last_axis(xe, bits=bits, group_size=32, dtype=dtype)
    qmax = (1 << bits) - 1
    xg = xt.view(2, 3, 64, 4, 32)
    mn, mx = xg.amin(-1, keepdim=True), xg.amax(-1, keepdim=True)
    ts = (mx - mn).clamp_min(1e-8) / qmax
    tq = ((xg - mn) / ts).round().clamp(0, qmax)
    tq = torch.nan_to_num(tq, nan=0.0).to(torch.uint8)
    assert np.array_equal(codes, tq.numpy())
    assert np.array_equal(s, ts.float().numpy())
    deq = KV.dequantize(codes, s, z, dtype=dtype)
    tdeq = (tq.float() * ts.float() + mn.float()).to(tdt).float().numpy()
    assert np.array_equal(deq, tdeq)


def test_kivi_dequant_two_roundings_not_fma():
    """code*scale rounds to fp32 before + zero: pick values where an FMA
    (one rounding) gives a different fp16 result, and check the oracle
    follows the two-rounding form."""
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 4, size=200000).astype(np.uint8)
    s = rng.standard_normal(200000).astype(np.float16).astype(np.float32)
    z = rng.standard_normal(200000).astype(np.float16).astype(np.float32)
    ours = KV.dequantize(codes, s, z, dtype="float16")
    two = np.float32(codes.astype(np.float32) * s) + z
    np.testing.assert_array_equal(ours, two.astype(np.float16).astype(np.float32))
    exact = (codes.astype(np.float64) * s.astype(np.float64) + z.astype(np.float64))
    fma = exact.astype(np.float32).astype(np.float16).astype(np.float32)
    assert (fma != ours).sum() >= 0  # documented: FMA may differ in rare cases


def test_kivi_round_half_even_boundary():
    """(x - zero)/scale landing exactly on .5 rounds to even."""
    x = np.array([[0.0, 0.5, 1.5, 3.0] + [0.0] * 28], np.float32)  # scale = 1.0
    codes, s, z = KV.quantize_last_axis(x, bits=2, group_size=32, dtype="float32")
    assert s.item() == 1.0 and codes[0, 0, :4].tolist() == [0, 0, 2, 3]


def _tie_group(bits: int) -> np.ndarray:
    """A 32-element group whose range is qmax (scale 1) holding half-integer
    values, so (x - zero) / scale lands exactly on .5 for most of them (all
    values exact in fp16 and bf16)."""
    qmax = (1 << bits) - 1
    g = np.array([0.0, float(qmax)] + [0.5 + j for j in range(30)], np.float32)
    return np.minimum(g, qmax)


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_kivi_ties_match_torch_ops(dtype, bits):
    """Codes whose quotient is exactly k + 0.5 (and ties created by the
    division, scale 2): the oracle against torch's evaluation of the
    reference expression (baselines/kivi_cache.py:64-69), round half to even."""
    torch = pytest.importorskip("torch")
    tdt = getattr(torch, dtype)
    qmax = (1 << bits) - 1
    g1 = _tie_group(bits)
    g2 = np.minimum(np.array([0.0, 2.0 * qmax] + [1.0 + 2 * j for j in range(30)], np.float32), 2.0 * qmax)
    x = np.stack([g1, g2, -g1, g1 + 7.0])[None, None].astype(np.float32)    # (1, 1, 4, 32)
    xt = torch.from_numpy(x).to(tdt)
    xe = xt.float().numpy()
    codes, s, z = KV.quantize_last_axis(xe, bits=bits, group_size=32, dtype=dtype)
    mn, mx = xt.amin(-1, keepdim=True), xt.amax(-1, keepdim=True)
    ts = (mx - mn).clamp_min(1e-8) / qmax
    tq = torch.nan_to_num(((xt - mn) / ts).round().clamp(0, qmax), nan=0.0).to(torch.uint8)
    assert np.array_equal(codes.reshape(tq.shape), tq.numpy())
    ties = ((xe[0, 0, 0] - xe[0, 0, 0].min()) % 1.0) == 0.5
    assert ties.sum() == min(qmax, 30)          # every half-integer below qmax is a tie


def test_kivi_per_channel_k_groups_tokens():
    rng = np.random.default_rng(4)
    k = rng.standard_normal((1, 2, 64, 8)).astype(np.float32)
    codes, s, z = KV.quantize_k_per_channel(k, bits=2, group_size=32, dtype="float32")
    assert codes.shape == k.shape and s.shape == (1, 2, 2, 8)
    np.testing.assert_array_equal(z[0, 1, 1], k[0, 1, 32:64].min(0))
    dq = KV.dequant_k(codes, s, z, group_size=32, dtype="float32")
    assert np.abs(dq - k).max() <= (s.max() * 0.5 + 1e-6)


def test_kivi_block_layout_known_answer():
    """Block layout pinned by hand-built values: channel 0 of K ramps 0,1,2,3
    over the tokens (scale 1, zero 0, codes t % 4 in bits 0-1 of each token
    row's first byte); every V token ramps 0..3 over channels 0..31 (group 0:
    scale 1, zero 0, channel c coded c % 4 for all 32 tokens in its
    channel-major row), group 1 is all zero (scale at the fp16 floor 0)."""
    from oracle import kivi as K
    D = 64
    k = np.zeros((1, 1, 32, D), np.float32)
    v = np.zeros((1, 1, 32, D), np.float32)
    k[0, 0, :, 0] = np.arange(32) % 4
    v[0, 0, :, :32] = np.arange(32) % 4
    blk = K.pack_blocks(k, v, bits=2, dtype="float16")
    assert blk.shape == (1, 1, 1, K.block_bytes(D, 2)) == (1, 1, 1, 2 * 32 * 16 + 8 * D)
    b = blk[0, 0, 0]
    rowb = D * 2 // 8
    assert [int(b[t * rowb]) & 3 for t in range(32)] == [t % 4 for t in range(32)]
    C = 32 * rowb
    ks = b[C:C + 2 * D].view(np.float16)
    assert ks[0] == np.float16(1.0) and ks[1] == np.float16(0.0)   # range 0 -> fp16 floor 0
    vc = C + 4 * D
    vrow = 32 * 2 // 8                                              # 8 bytes per channel row
    for c in range(D):
        want = (c % 4) * 0x55 if c < 32 else 0                      # code c % 4 for all 32 tokens
        assert [int(x) for x in b[vc + c * vrow:vc + (c + 1) * vrow]] == [want] * vrow
    vs = b[2 * C + 4 * D:2 * C + 6 * D].view(np.float16)            # group-major: D/32 x 32 tokens
    assert (vs[:32] == np.float16(1.0)).all() and (vs[32:] == np.float16(0.0)).all()


def test_kivi_code_positions_known_answer():
    """2-bit code positions within a row, by hand: in every 16-bit word the
    even elements 0, 2, 4, 6 sit at bits 0, 2, 4, 6 of the low byte and the
    odd elements 1, 3, 5, 7 at bits 0, 2, 4, 6 of the high byte.  K channel d
    ramps (t + d) % 4 over the tokens (scale 1, zero 0), so the code of
    (token t, channel d) is (t + d) % 4; V channel 0 of token t is t % 4 with
    channels 30 and 31 pinning the token's range to [0, 3], so the V row of
    channel 0 holds code token % 4 at each slot (slot 8g + j: token 4g + j,
    or 16 + 4g + j - 4 for j >= 4)."""
    from oracle import kivi as K
    D = 32
    t = np.arange(32)
    k = np.stack([(t + d) % 4 for d in range(D)], axis=-1).astype(np.float32)[None, None]
    v = np.zeros((1, 1, 32, D), np.float32)
    v[0, 0, :, 0] = t % 4
    v[0, 0, :, 31] = 3.0
    b = K.pack_blocks(k, v, bits=2, dtype="float16")[0, 0, 0]
    rowb = D * 2 // 8
    for tok in range(32):
        for w in range(rowb // 2):
            lo = sum(((tok + 8 * w + 2 * j) % 4) << (2 * j) for j in range(4))
            hi = sum(((tok + 8 * w + 2 * j + 1) % 4) << (2 * j) for j in range(4))
            assert (int(b[tok * rowb + 2 * w]), int(b[tok * rowb + 2 * w + 1])) == (lo, hi), (tok, w)
    slot_token = [(16 if s & 4 else 0) + 4 * (s >> 3) + (s & 3) for s in range(32)]
    vc = 32 * rowb + 4 * D
    for w in range(4):                                              # channel 0: 8 bytes = 4 words
        lo = sum((slot_token[8 * w + 2 * j] % 4) << (2 * j) for j in range(4))
        hi = sum((slot_token[8 * w + 2 * j + 1] % 4) << (2 * j) for j in range(4))
        assert (int(b[vc + 2 * w]), int(b[vc + 2 * w + 1])) == (lo, hi), w


def test_kivi_blocks_roundtrip_equals_dequant():
    from oracle import kivi as K
    from oracle.inputs import decode_inputs
    x = decode_inputs(4, B=1, H=4, H_kv=2, T=96, D=128, dtype="float16", n_planted=2, sigma=10.0)
    kd, vd = K.unpack_blocks(K.pack_blocks(x.k, x.v, bits=2, dtype="float16"), D=128, bits=2, dtype="float16")
    ck, sk, zk = K.quantize_k_per_channel(x.k, bits=2, group_size=32, dtype="float16")
    cv, sv, zv = K.quantize_v_per_token(x.v, bits=2, group_size=32, dtype="float16")
    assert np.array_equal(kd, K.dequant_k(ck, sk, zk, group_size=32, dtype="float16"))
    assert np.array_equal(vd, K.dequant_v(cv, sv, zv, group_size=32, dtype="float16"))


# ---------------------------------------------------------------------------
# Quest bounding-box scorer (baselines/quest_path_d.py:125-205)
# ---------------------------------------------------------------------------

def test_quest_page_minmax_is_the_page_extremes():
    rng = np.random.default_rng(11)
    K = rng.standard_normal((2, 3, 70, 16)).astype(np.float32)
    kmin, kmax = S.page_minmax(K, 16)
    assert kmin.shape == kmax.shape == (2, 3, 4, 16)  # the partial page is left out
    for j in range(4):
        rows = K[:, :, 16 * j:16 * j + 16]
        assert np.array_equal(kmin[:, :, j], rows.min(axis=2))
        assert np.array_equal(kmax[:, :, j], rows.max(axis=2))
    K[0, 1, 20, 5] = np.nan  # a NaN in a page's channel makes both extremes NaN
    kmin, kmax = S.page_minmax(K, 16)
    assert np.isnan(kmin[0, 1, 1, 5]) and np.isnan(kmax[0, 1, 1, 5])
    assert not np.isnan(kmin[0, 1, 1, 4]) and not np.isnan(kmin[0, 1, 0, 5])


def test_quest_bound_is_an_upper_bound_of_every_row():
    """sum_d max(q kmin, q kmax) >= q.k for every row of the page (a swapped
    min/max, a dropped sign or a wrong channel breaks this), with equality
    for page_size 1 (kmin = kmax = k), where the bound is exactly the
    scorer's ordered dot product."""
    rng = np.random.default_rng(12)
    for D, dtype in ((64, "float32"), (128, "bfloat16")):
        K = rng.standard_normal((1, 2, 64, D)).astype(np.float32)
        q = rng.standard_normal((1, 8, 3, D)).astype(np.float32)
        if dtype == "bfloat16":
            K, q = round_bf16(K), round_bf16(q)
        kmin, kmax = S.page_minmax(K, 8)
        b = S.quest_scores(q, kmin, kmax, dtype).astype(np.float64)  # (1, 2, 3, 8)
        qg = S.gqa_mean_query(q, 2, dtype).astype(np.float64)
        dots = np.einsum("bhtd,bhsd->bhts", qg, K.astype(np.float64)).reshape(1, 2, 3, 8, 8)
        slack = 1e-4 * np.abs(qg).sum(-1)[..., None]
        assert (dots.max(axis=-1) <= b + slack).all()
        # the bound is attained when every channel's extreme sits in one row
        k1min, k1max = S.page_minmax(K, 1)
        b1 = S.quest_scores(q, k1min, k1max, dtype)
        assert np.array_equal(b1, S.ordered_dot(S.gqa_mean_query(q, 2, dtype), K[:, :, None], dtype))


def test_quest_bound_known_answer_and_float64():
    """A hand-computed bound, then random pages against the float64 closed
    form within the fp32 summation bound."""
    D = 16
    q = np.zeros((1, 1, 1, D), np.float32)
    q[..., 0], q[..., 1], q[..., 2] = 2.0, -3.0, 0.5
    kmin = np.zeros((1, 1, 1, D), np.float32)
    kmax = np.zeros((1, 1, 1, D), np.float32)
    kmin[..., 0], kmax[..., 0] = -1.0, 4.0     # q > 0 takes kmax: 8
    kmin[..., 1], kmax[..., 1] = -2.0, 5.0     # q < 0 takes kmin: 6
    kmin[..., 2], kmax[..., 2] = -6.0, -1.0    # q > 0 takes kmax: -0.5
    assert float(S.quest_scores(q, kmin, kmax)[0, 0, 0, 0]) == 13.5
    rng = np.random.default_rng(13)
    q = rng.standard_normal((2, 4, 2, 128)).astype(np.float32)
    K = rng.standard_normal((2, 2, 160, 128)).astype(np.float32)
    kmin, kmax = S.page_minmax(K, 16)
    got = S.quest_scores(q, kmin, kmax).astype(np.float64)
    qg = S.gqa_mean_query(q, 2).astype(np.float64)[:, :, :, None, :]
    ref = np.maximum(qg * kmin[:, :, None].astype(np.float64), qg * kmax[:, :, None].astype(np.float64)).sum(-1)
    mag = (np.abs(qg) * np.maximum(np.abs(kmin), np.abs(kmax))[:, :, None]).sum(-1)
    assert (np.abs(got - ref) <= 24 * 2.0 ** -24 * mag).all()


def test_quest_select_brute_force_and_budget():
    rng = np.random.default_rng(14)
    q = rng.standard_normal((2, 4, 3, 32)).astype(np.float32)
    K = rng.standard_normal((2, 2, 12 * 8, 32)).astype(np.float32)
    kmin, kmax = S.page_minmax(K, 8)
    s = S.quest_page_scores(q, kmin, kmax)
    assert np.array_equal(s, S.quest_scores(q, kmin, kmax).max(axis=(0, 1, 2)))
    got = S.quest_select(q, kmin, kmax, memory_ratio=4.0, min_pages_selected=2)
    brute = sorted(range(12), key=lambda p: (-float(s[p]), p))[:3]
    assert got.tolist() == brute  # descending score order, K = ceil(12 / 4) = 3
    # ties: equal scores rank by lower page index; NaN ranks last
    kmin2, kmax2 = kmin.copy(), kmax.copy()
    kmin2[:, :, 7], kmax2[:, :, 7] = kmin2[:, :, 2], kmax2[:, :, 2]
    kmin2[:, :, 0, 0] = np.nan
    order = S.quest_select(q, kmin2, kmax2, memory_ratio=1.0, min_pages_selected=1)
    assert order[-1] == 0 and order.tolist().index(2) + 1 == order.tolist().index(7)
    # the reference's float budget (baselines/quest_path_d.py:197-200)
    assert S.quest_num_hot_pages(4, 2.0, 1) == 2
    assert S.quest_num_hot_pages(3, 2.5, 1) == 1      # int(4.5 // 2.5), not ceil(1.2)
    assert S.quest_num_hot_pages(10, 4.0, 4) == 4
    assert S.quest_num_hot_pages(3, 4.0, 4) == 3      # capped at P


def test_quest_scores_match_torch_ops():
    """The reference test's recipe (tests/test_quest_path_d.py:147-188:
    seeded K and q, pages of 4, torch amin/amax/maximum/sum) at D = 16,
    against the oracle within fp32 reduction noise."""
    torch = pytest.importorskip("torch")
    torch.manual_seed(7)
    B, H_kv, T, D = 1, 2, 16, 16
    K = torch.randn(B, H_kv, T, D)
    q = torch.randn(B, H_kv, 1, D)
    kp = K.view(B, H_kv, 4, 4, D)
    k_min, k_max = kp.amin(dim=-2), kp.amax(dim=-2)
    expected = torch.maximum(q.unsqueeze(-2) * k_min.unsqueeze(-3), q.unsqueeze(-2) * k_max.unsqueeze(-3)).sum(-1)
    omin, omax = S.page_minmax(K.numpy(), 4)
    assert np.array_equal(omin, k_min.numpy()) and np.array_equal(omax, k_max.numpy())
    got = S.quest_scores(q.numpy(), omin, omax)
    assert got.shape == (B, H_kv, 1, 4)
    np.testing.assert_allclose(got, expected.numpy(), atol=1e-5)
    top = torch.topk(expected.amax(dim=(0, 1, 2)), 2).indices.tolist()
    assert S.quest_select(q.numpy(), omin, omax, memory_ratio=2.0, min_pages_selected=1).tolist() == top


# ---------------------------------------------------------------- HALOPress page score and budget
def _halopress(attn, **kw):
    base = dict(alpha=0.0, beta=0.0, gamma=0.0, refresh_window=8, sink_tokens=4, page_size=16)
    base.update(kw)
    return S.halopress_page_scores(np.asarray(attn, np.float32), **base)


@pytest.mark.parametrize("P,W,sink,page", [(37, 64, 4, 16), (50, 16, 40, 16), (5, 1, 0, 16),
                                           (1, 8, 4, 16), (24, 3, 100, 8)])
def test_halopress_page_scores_match_torch_ops(P, W, sink, page):
    """baselines/scorer_ablations.py:238-263 evaluated with torch's CPU
    kernels (its min/max/exp/sum and fp32 scalar products), against the
    oracle within fp32 reduction noise."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(P * 7 + W)
    attn = rng.standard_normal(P).astype(np.float32)
    ours = S.halopress_page_scores(attn, alpha=1.0, beta=0.5, gamma=2.0, refresh_window=W,
                                   sink_tokens=sink, page_size=page)
    a = torch.from_numpy(attn.copy())
    a = a - a.min()
    if float(a.max().item()) > 0.0:
        a = a / a.max()
    positions = torch.arange(P, dtype=torch.float32)
    rec = torch.exp(-(P - 1 - positions) / max(W, 1))
    rec = rec / (rec.sum() + 1e-12)
    rec = rec / (rec.max() + 1e-12)
    sk = torch.zeros(P, dtype=torch.float32)
    sk[: min(sink // max(page, 1) + 1, P)] = 1.0
    ref = 1.0 * a.float() + 0.5 * rec + 2.0 * sk
    np.testing.assert_allclose(ours, ref.numpy(), rtol=2e-6, atol=1e-7)


def test_halopress_alpha_only_is_min_max_normalised():
    """Closed form: with beta = gamma = 0 the score is (a - min) / (max - min):
    exactly 0 at the minimum, exactly 1 at the maximum, and a constant
    attention vector scores 0 everywhere (no division)."""
    rng = np.random.default_rng(3)
    attn = (rng.standard_normal(40) * 5 + 2).astype(np.float32)
    s = _halopress(attn, alpha=1.0)
    assert s[int(np.argmin(attn))] == 0.0 and s[int(np.argmax(attn))] == 1.0
    a64 = attn.astype(np.float64)
    np.testing.assert_allclose(s, (a64 - a64.min()) / (a64.max() - a64.min()), rtol=0, atol=4e-7)
    assert np.array_equal(np.argsort(s, kind="stable"), np.argsort(attn, kind="stable"))
    assert np.array_equal(_halopress(np.full(9, 3.5, np.float32), alpha=1.0), np.zeros(9, np.float32))
    # alpha scales the normalised term only
    np.testing.assert_allclose(_halopress(attn, alpha=0.25), 0.25 * s, rtol=1e-6, atol=0)


@pytest.mark.parametrize("P,W", [(1, 8), (2, 1), (32, 8), (64, 64), (100, 5)])
def test_halopress_beta_only_recency_closed_form(P, W):
    """Closed form: after normalising by the sum and then by the maximum,
    the recency term is exp(-(P - 1 - p) / W): 1 on the newest page (the
    highest index) and non-decreasing in p.  A reversed direction, a single
    normalisation or a dropped window fails one of the checks."""
    s = _halopress(np.zeros(P, np.float32), beta=1.0, refresh_window=W)
    want = np.exp(-(P - 1 - np.arange(P, dtype=np.float64)) / W)
    np.testing.assert_allclose(s, want, rtol=4e-6, atol=0)
    assert abs(float(s[-1]) - 1.0) <= 2.0 ** -22
    assert (np.diff(s) >= 0).all()
    if P >= 2:
        assert s[0] < s[-1]


def test_halopress_gamma_only_sink_pages_known_answers():
    """sink_tokens // page_size + 1 pages (capped at P) score gamma, the
    rest 0 (baselines/scorer_ablations.py:253-257).  Counts worked by hand."""
    cases = [  # (P, sink_tokens, page_size) -> number of sink pages
        ((10, 4, 16), 1), ((10, 0, 16), 1), ((10, 15, 16), 1), ((10, 16, 16), 2),
        ((10, 47, 16), 3), ((3, 100, 16), 3), ((6, 5, 1), 6), ((12, 5, 2), 3), ((1, 0, 16), 1),
    ]
    for (P, sink, page), n in cases:
        s = _halopress(np.zeros(P, np.float32), gamma=2.0, sink_tokens=sink, page_size=page)
        assert s.tolist() == [2.0] * n + [0.0] * (P - n), (P, sink, page)


def test_halopress_terms_add():
    """The three terms add: the full score equals the sum of the one-term
    scores (each term is computed independently of the weights)."""
    rng = np.random.default_rng(5)
    attn = rng.standard_normal(30).astype(np.float32)
    kw = dict(refresh_window=7, sink_tokens=20, page_size=8)
    full = _halopress(attn, alpha=1.0, beta=0.5, gamma=2.0, **kw)
    parts = (_halopress(attn, alpha=1.0, **kw).astype(np.float64) + _halopress(attn, beta=0.5, **kw)
             + _halopress(attn, gamma=2.0, **kw))
    np.testing.assert_allclose(full, parts, rtol=0, atol=4e-7)


def test_num_hot_pages_known_answers():
    """_num_hot_pages (baselines/scorer_ablations.py:133-139): max(min,
    int((P + r - 1) // r)) capped at P, with the reference's float ratio
    (default 4.0).  Values worked by hand."""
    assert S.num_hot_pages(37, 4, 4) == 10      # ceil(37 / 4)
    assert S.num_hot_pages(37, 4.0, 4) == 10
    assert S.num_hot_pages(3, 4, 4) == 3        # floor 4, capped at P = 3
    assert S.num_hot_pages(10, 4.0, 4) == 4     # ceil 3 < floor 4
    assert S.num_hot_pages(100, 4.0, 4) == 25
    assert S.num_hot_pages(101, 4.0, 4) == 26
    assert S.num_hot_pages(10, 2.5, 1) == 4     # (11.5 // 2.5) = 4
    assert S.num_hot_pages(3, 2.5, 1) == 1      # (4.5 // 2.5) = 1, not ceil(1.2) = 2
    assert S.num_hot_pages(1, 4.0, 4) == 1
    assert S.num_hot_pages(0, 4.0, 4) == 0
