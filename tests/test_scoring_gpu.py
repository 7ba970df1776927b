"""GPU parity of the chunk scorer (page means, q.Kbar scores, top-k) and of
the tiered decode layer (scorer -> chunk table -> attention, no host sync)."""
from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import scoring as S
from oracle.inputs import C1, C2, decode_inputs, round_bf16

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TDT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}


def _gpu(a, dtype, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(TDT[dtype])


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_chunk_means(dev, dtype):
    from halo_amd.chunk_scorer import chunk_means
    x = decode_inputs(21, B=2, H=4, H_kv=2, T=1100, D=128, dtype=dtype)
    k = _gpu(x.k, dtype, dev)
    km = chunk_means(k, 256).float().cpu().numpy()
    ref = S.page_means(x.k, 256, dtype)
    assert km.shape == ref.shape == (2, 2, 4, 128)
    if dtype == "float32":
        np.testing.assert_allclose(km, ref, rtol=1e-6, atol=1e-7)
    else:  # at most one rounding step of the storage dtype apart
        ulp = np.abs(ref) * (2.0 ** -7 if dtype == "bfloat16" else 2.0 ** -10) + 1e-6
        assert (np.abs(km - ref) <= ulp).all()
        assert (km == ref).mean() > 0.97


@pytest.mark.parametrize("H,H_kv,dtype", [(8, 8, "float32"), (32, 8, "bfloat16"), (28, 4, "float16")])
def test_scores_and_topk_match_oracle(dev, H, H_kv, dtype):
    from halo_amd.chunk_scorer import score_topk
    rng = np.random.default_rng(5)
    D, P = 128, 40
    for trial in range(5):
        q = rng.standard_normal((1, H, 1, D)).astype(np.float32)
        km = rng.standard_normal((1, H_kv, P, D)).astype(np.float32) * 0.3
        if dtype != "float32":
            q = q.astype(np.float16).astype(np.float32) if dtype == "float16" else round_bf16(q)
            km = km.astype(np.float16).astype(np.float32) if dtype == "float16" else round_bf16(km)
        elig = np.sort(rng.choice(P, size=30, replace=False))
        idx, sc = score_topk(_gpu(q, dtype, dev), _gpu(km, dtype, dev), torch.from_numpy(elig).to(dev), 6)
        ref_sc = S.mean_key_scores(q, km, dtype)[elig]
        np.testing.assert_allclose(sc[0, :30].cpu().numpy(), ref_sc, rtol=1e-5, atol=1e-5)
        # the kernel's fixed summation order, bit for bit
        np.testing.assert_array_equal(sc[0, :30].cpu().numpy(), S.ordered_scores(q, km, dtype)[elig])
        ref_sel = S.select_chunks(q, km, elig, 6, dtype)
        srt = np.sort(ref_sc.astype(np.float64))[::-1]
        if srt[5] - srt[6] > 1e-4:  # margin-checked
            assert idx[0].cpu().numpy().tolist() == ref_sel.tolist()


def test_topk_tie_break_on_device(dev):
    from halo_amd.chunk_scorer import score_topk
    # identical means for chunks 1, 2 and 4: ties resolve to lower index
    km = np.zeros((1, 1, 6, 64), np.float32)
    km[0, 0, [1, 2, 4], 0] = 3.0
    km[0, 0, 3, 0] = 2.0
    km[0, 0, 0, 0] = 1.0
    q = np.zeros((1, 1, 1, 64), np.float32)
    q[..., 0] = 1.0
    for k, want in [(1, [1]), (2, [1, 2]), (3, [1, 2, 4]), (4, [1, 2, 3, 4]), (8, [0, 1, 2, 3, 4, 5, -1, -1])]:
        idx, _ = score_topk(_gpu(q, "float32", dev), _gpu(km, "float32", dev),
                            torch.arange(6, device=dev), k)
        assert idx[0].cpu().tolist() == want


def test_halopress_normalised_score(dev):
    from halo_amd.chunk_scorer import score_topk
    rng = np.random.default_rng(8)
    q = rng.standard_normal((1, 8, 1, 64)).astype(np.float32)
    km = rng.standard_normal((1, 2, 50, 64)).astype(np.float32)
    kw = dict(alpha=1.0, beta=0.5, gamma=2.0, refresh_window=16, sink_tokens=4, page_size=16)
    attn = S.mean_key_scores(q, km)
    ref = S.halopress_page_scores(attn, **kw)
    idx, sc = score_topk(_gpu(q, "float32", dev), _gpu(km, "float32", dev), torch.arange(50, device=dev), 13,
                         normalize=True, alpha=1.0, beta=0.5, gamma=2.0, refresh_window=16,
                         sink_pages=min(4 // 16 + 1, 50), P_total=50)
    np.testing.assert_allclose(sc[0].cpu().numpy(), ref, rtol=1e-5, atol=1e-6)
    assert idx[0].cpu().numpy().tolist() == S.topk_indices(ref, 13).tolist()


def test_per_row_ragged_selection(dev):
    from halo_amd.chunk_scorer import score_topk
    rng = np.random.default_rng(9)
    B, H, H_kv, D, P = 4, 8, 2, 64, 20
    q = rng.standard_normal((B, H, 1, D)).astype(np.float32)
    km = rng.standard_normal((B, H_kv, P, D)).astype(np.float32)
    n_el = np.array([20, 7, 3, 12], np.int32)
    elig = np.tile(np.arange(P, dtype=np.int32), (B, 1))
    idx, sc = score_topk(_gpu(q, "float32", dev), _gpu(km, "float32", dev), torch.from_numpy(elig).to(dev), 5,
                         per_row=True, n_elig_per_sel=torch.from_numpy(n_el).to(dev))
    for b in range(B):
        want = S.select_chunks(q[b:b + 1], km[b:b + 1], np.arange(n_el[b]), 5).tolist()
        want += [-1] * (5 - len(want))
        assert idx[b].cpu().tolist() == want


def _tiered_from_fixture(cfg, dev, fused=True):
    from halo_amd.decode import ChunkRef
    from halo_amd.tiered import TieredDecodeLayer
    x = decode_inputs(cfg["seed"], B=1, H=cfg["H"], H_kv=cfg["H_kv"], T=cfg["T"], D=cfg["D"], dtype=cfg["dtype"],
                      n_planted=cfg.get("n_planted", 0), sigma=cfg.get("sigma", 1.0))
    q, k, v = (_gpu(a, cfg["dtype"], dev) for a in (x.q, x.k, x.v))
    c = cfg["chunk"]
    n = cfg["T"] // c
    n_cold = n - cfg["n_hot"]
    refs = [ChunkRef(k[..., i * c:(i + 1) * c, :], v[..., i * c:(i + 1) * c, :], i * c, True) for i in range(n)]
    layer = TieredDecodeLayer(B=1, H=cfg["H"], H_kv=cfg["H_kv"], D=cfg["D"], dtype=TDT[cfg["dtype"]],
                              hot=refs[n_cold:], cold=refs[:n_cold], top_k=cfg["top_k"], device=dev, fused=fused)
    assert layer.fused == fused
    return layer, q


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "two_kernel"])
@pytest.mark.parametrize("name,cfg", [("c1_decode", C1), ("c2_layer0", C2)])
def test_tiered_layer_matches_golden(dev, name, cfg, fused):
    """Scorer picks the fixture's chunks bit-exactly; attention over hot +
    selected matches the float64 closed form (1e-5 fp32, 2e-2 bf16)."""
    fx = np.load(os.path.join(GOLD, name + ".npz"))
    layer, q = _tiered_from_fixture(cfg, dev, fused)
    out = torch.empty((1, cfg["H"], cfg["D"]), device=dev, dtype=TDT[cfg["dtype"]])
    lse = torch.empty((1, cfg["H"]), device=dev)
    layer.step(q[:, :, 0], scale=1 / math.sqrt(cfg["D"]), out=out, lse=lse)
    assert layer.idx[0].cpu().numpy().tolist() == fx["selected"].tolist()
    tol = 1e-5 if cfg["dtype"] == "float32" else 2e-2
    assert np.abs(out.float().cpu().numpy() - fx["out"]).max() <= tol
    ltol = 1e-5 if cfg["dtype"] == "float32" else 1e-3
    assert np.abs(lse.cpu().numpy() - fx["lse"]).max() <= ltol
    np.testing.assert_allclose(layer.scores[0].cpu().numpy(), fx["scores"], rtol=1e-4, atol=1e-5)


def test_fused_selection_matches_two_kernel_path(dev):
    """In-kernel selection and the standalone scorer produce identical
    indices, scores, outputs and LSEs (same arithmetic, same tie rule)."""
    scale = 1 / math.sqrt(C2["D"])
    res = []
    for fused in (True, False):
        layer, q = _tiered_from_fixture(C2, dev, fused)
        out = torch.empty((1, C2["H"], C2["D"]), device=dev, dtype=torch.bfloat16)
        lse = torch.empty((1, C2["H"]), device=dev)
        layer.step(q[:, :, 0], scale=scale, out=out, lse=lse)
        torch.cuda.synchronize()
        res.append((layer.idx.clone(), layer.scores.clone(), out, lse))
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_fused_selection_lead_items_miscount(dev):
    """lead_items is a scheduling hint: understated (0) or overstated (every
    record, so hot items also stage the selection's page means into LDS
    before attending), the outputs, LSEs, indices and scores are identical
    to the planner's count."""
    scale = 1 / math.sqrt(C2["D"])
    layer, q = _tiered_from_fixture(C2, dev, True)
    cfg = layer.select_cfg
    true_lead = cfg.lead_items
    assert 0 < true_lead < layer.plan.n_work
    res = []
    for lead in (true_lead, 0, layer.plan.n_work):
        cfg.lead_items = lead
        out = torch.empty((1, C2["H"], C2["D"]), device=dev, dtype=torch.bfloat16)
        lse = torch.empty((1, C2["H"]), device=dev)
        layer.step(q[:, :, 0], scale=scale, out=out, lse=lse)
        torch.cuda.synchronize()
        res.append((layer.idx.clone(), layer.scores.clone(), out, lse))
    cfg.lead_items = true_lead
    for other in res[1:]:
        for a, b in zip(res[0], other):
            assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_fused_selection_per_row_ragged(dev, dtype):
    """halo_decode_attn_tiered with one selection per batch row over a
    ragged number of eligible chunks; a slot past the eligible count attends
    nothing and reports -1.  Checked against the oracle's selector and the
    float64 closed form over hot + selected rows."""
    from halo_amd import _native as nat
    from halo_amd.chunk_scorer import chunk_means
    from halo_amd.decode import ChunkRef, build_plan, descs_to_device, launch, pack_descs
    B, H, H_kv, D, T, c, top_k = 2, 8, 2, 64, 1024, 128, 3
    n_el = np.array([5, 2], np.int32)
    x = decode_inputs(44, B=B, H=H, H_kv=H_kv, T=T, D=D, dtype=dtype, n_planted=2, sigma=4.0)
    q, k, v = (_gpu(a, dtype, dev) for a in (x.q, x.k, x.v))
    refs = [ChunkRef(k[..., i * c:(i + 1) * c, :], v[..., i * c:(i + 1) * c, :], i * c, True) for i in range(T // c)]
    cold, hot = refs[:6], refs[6:]
    plan = build_plan(B=B, H=H, H_kv=H_kv, D=D, dtype=TDT[dtype], chunks=[cold[0]] * top_k + hot, device=dev)
    cat_np, keep = pack_descs(cold + cold, B=B, H_kv=H_kv, D=D, dtype=TDT[dtype])
    cat = descs_to_device(cat_np, dev)
    km = chunk_means(k, c, n_pages=6)
    n_el_d = torch.from_numpy(n_el).to(dev)
    idx = torch.full((B, top_k), -7, device=dev, dtype=torch.int32)
    sc = torch.full((B, 6), -7.0, device=dev)
    cfg = nat.SelectCfg(kmean=km.data_ptr(), km_stride_b=km.stride(0), km_stride_h=km.stride(1),
                        km_stride_p=km.stride(2), catalog=cat.data_ptr(), catalog_stride=6,
                        n_cold_per_sel=n_el_d.data_ptr(), n_cold=6, top_k=top_k, slot0=0, per_row=1,
                        idx_out=idx.data_ptr(), score_out=sc.data_ptr())
    out = torch.empty((B, H, D), device=dev)
    lse = torch.empty((B, H), device=dev)
    launch(plan, q[:, :, 0], scale=0.125, out=out, lse=lse, select=cfg)
    torch.cuda.synchronize()
    km_np = km.float().cpu().numpy()
    for b in range(B):
        ref_sc = S.mean_key_scores(x.q[b:b + 1], km_np[b:b + 1], dtype)[: n_el[b]]
        np.testing.assert_allclose(sc[b, : n_el[b]].cpu().numpy(), ref_sc, rtol=1e-5, atol=1e-5)
        np.testing.assert_array_equal(sc[b, : n_el[b]].cpu().numpy(),
                                      S.ordered_scores(x.q[b:b + 1], km_np[b:b + 1], dtype)[: n_el[b]])
        assert (sc[b, n_el[b]:].cpu().numpy() == -7.0).all()
        srt = np.sort(ref_sc.astype(np.float64))[::-1]
        assert len(srt) <= top_k or srt[top_k - 1] - srt[top_k] > 1e-4, "fixture seed lost its margin"
        want = S.select_chunks(x.q[b:b + 1], km_np[b:b + 1], np.arange(n_el[b]), top_k, dtype).tolist()
        assert idx[b].cpu().tolist() == want + [-1] * (top_k - len(want))
        keep_rows = np.zeros(T, bool)
        keep_rows[6 * c:] = True
        for j in want:
            keep_rows[j * c:(j + 1) * c] = True
        ro, rl = A.attention_f64(x.q[b:b + 1, :, 0], x.k[b:b + 1], x.v[b:b + 1], scale=0.125, keep=keep_rows)
        tol = 1e-5 if dtype == "float32" else 2e-2
        assert np.abs(out[b:b + 1].cpu().numpy() - ro).max() <= tol
        assert np.abs(lse[b:b + 1].cpu().numpy() - rl).max() <= (1e-5 if dtype == "float32" else 1e-3)


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "two_kernel"])
def test_tiered_layer_in_hip_graph(dev, fused):
    """The decode step replays from a captured graph; every replay matches
    the eager result (fresh inputs copied in between replays)."""
    layer, q = _tiered_from_fixture(C1, dev, fused)
    q3 = q[:, :, 0].contiguous()
    out = torch.empty((1, 8, 64), device=dev)
    lse = torch.empty((1, 8), device=dev)
    layer.step(q3, scale=0.125, out=out, lse=lse)  # warm the workspace
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        layer.step(q3, scale=0.125, out=out, lse=lse)  # warm the capture stream's workspace
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            layer.step(q3, scale=0.125, out=out, lse=lse)
    torch.cuda.current_stream().wait_stream(s)
    rng = np.random.default_rng(3)
    for rep in range(4):
        newq = torch.from_numpy(rng.standard_normal((1, 8, 64)).astype(np.float32)).to(dev)
        q3.copy_(newq)
        g.replay()
        torch.cuda.synchronize()
        got_o, got_l, got_i = out.clone(), lse.clone(), layer.idx.clone()
        layer.step(q3, scale=0.125, out=out, lse=lse)
        torch.cuda.synchronize()
        assert torch.equal(got_i, layer.idx)
        assert torch.equal(got_o, out) and torch.equal(got_l, lse)


@pytest.mark.parametrize("ctx", [[1024, 2560, 1536], [256, 2560, 512]])
@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_ragged_batched_decode(dev, dtype, ctx):
    """Per-sequence chunk tables of different lengths in one launch: each
    row scores its own cold chunks (bit-exact top-k against the oracle's
    selector, margin-checked), a row with fewer cold chunks than top_k leaves
    -1 slots (a row with no cold chunk at all, row 0 of the second case,
    selects none and attends its hot rows), and every row's output matches
    the float64 closed form over its hot + selected rows."""
    from halo_amd.decode import ChunkRef
    from halo_amd.tiered import RaggedTieredDecodeLayer
    H, H_kv, D, c, top_k = 8, 2, 128, 256, 4
    rng = np.random.default_rng(17)
    rows, host = [], []
    for b, T in enumerate(ctx):
        k = rng.standard_normal((H_kv, T, D), dtype=np.float32)
        k[:, :, [3, 77]] *= 6.0
        v = rng.standard_normal((H_kv, T, D), dtype=np.float32)
        from oracle.inputs import round_to
        k, v = round_to(k, dtype), round_to(v, dtype)
        kg, vg = _gpu(k, dtype, dev), _gpu(v, dtype, dev)
        n = T // c
        n_hot = max(1, n // 4)
        refs = [ChunkRef(kg[:, i * c:(i + 1) * c], vg[:, i * c:(i + 1) * c], i * c, True, batch=b) for i in range(n)]
        rows.append((refs[n - n_hot:], refs[:n - n_hot]))
        host.append((k, v, n, n_hot))
    q = round_to(rng.standard_normal((len(ctx), H, D), dtype=np.float32), dtype)
    layer = RaggedTieredDecodeLayer(H=H, H_kv=H_kv, D=D, dtype=TDT[dtype], rows=rows, top_k=top_k, device=dev)
    out = torch.empty((len(ctx), H, D), device=dev, dtype=TDT[dtype])
    lse = torch.empty((len(ctx), H), device=dev)
    q_pos = torch.tensor([T - 1 for T in ctx], device=dev, dtype=torch.int64)
    layer.step(_gpu(q, dtype, dev), scale=1 / math.sqrt(D), out=out, lse=lse, q_pos=q_pos)
    torch.cuda.synchronize()
    km = layer.kmean.float().cpu().numpy()
    for b, (k, v, n, n_hot) in enumerate(host):
        n_cold = n - n_hot
        ref_sc = S.mean_key_scores(q[b:b + 1, :, None], km[b:b + 1, :, :n_cold], dtype)
        np.testing.assert_array_equal(layer.scores[b, :n_cold].cpu().numpy(),
                                      S.ordered_scores(q[b:b + 1, :, None], km[b:b + 1, :, :n_cold], dtype))
        srt = np.sort(ref_sc.astype(np.float64))[::-1]
        assert len(srt) <= top_k or srt[top_k - 1] - srt[top_k] > 1e-4, "fixture seed lost its margin"
        want = S.select_chunks(q[b:b + 1, :, None], km[b:b + 1, :, :n_cold], np.arange(n_cold), top_k, dtype).tolist()
        assert layer.idx[b].cpu().tolist() == want + [-1] * (top_k - len(want))
        keep = np.zeros(k.shape[1], bool)
        keep[(n - n_hot) * c:] = True
        for j in want:
            keep[j * c:(j + 1) * c] = True
        ro, rl = A.attention_f64(q[b:b + 1], k[None], v[None], scale=1 / math.sqrt(D), keep=keep)
        tol = 1e-5 if dtype == "float32" else 2e-2
        assert np.abs(out[b:b + 1].float().cpu().numpy() - ro).max() <= tol
        assert np.abs(lse[b:b + 1].cpu().numpy() - rl).max() <= (1e-5 if dtype == "float32" else 1e-3)


@pytest.mark.parametrize("case", ["lds_qbar", "many_units", "unaligned_q"])
def test_fused_selection_paths(dev, case):
    """The fused selector's other paths against the standalone scorer path,
    bit for bit (indices, scores, outputs, LSE): 'lds_qbar' (3 batch rows x 2
    KV heads: a lane's head varies across its dot-product units, so the GQA
    query mean is staged in LDS), 'many_units' (64 candidates x 8 KV heads =
    4096 units, past the six per lane held in registers), 'unaligned_q'
    (query rows not 16-byte aligned: the element-wise q-bar)."""
    from halo_amd.decode import ChunkRef
    from halo_amd.tiered import TieredDecodeLayer
    B, H, H_kv, c, n_hot, n_cold, top_k = {
        "lds_qbar": (3, 8, 2, 128, 4, 12, 3),
        "many_units": (1, 16, 8, 64, 4, 64, 5),
        "unaligned_q": (1, 32, 8, 128, 4, 12, 4),
    }[case]
    D, T = 128, (n_hot + n_cold) * c
    x = decode_inputs(61, B=B, H=H, H_kv=H_kv, T=T, D=D, dtype="bfloat16", n_planted=2, sigma=6.0)
    q, k, v = (_gpu(a, "bfloat16", dev) for a in (x.q, x.k, x.v))
    q = q[:, :, 0]
    if case == "unaligned_q":
        wide = torch.zeros((B, H, D + 1), device=dev, dtype=torch.bfloat16)
        wide[..., 1:] = q
        q = wide[..., 1:]
        assert (q.stride(1) * 2) % 16 != 0
    refs = [ChunkRef(k[..., i * c:(i + 1) * c, :], v[..., i * c:(i + 1) * c, :], i * c, True)
            for i in range(n_hot + n_cold)]
    res = []
    for fused in (True, False):
        layer = TieredDecodeLayer(B=B, H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, hot=refs[n_cold:],
                                  cold=refs[:n_cold], top_k=top_k, device=dev, fused=fused)
        assert layer.fused == fused
        out = torch.empty((B, H, D), device=dev, dtype=torch.bfloat16)
        lse = torch.empty((B, H), device=dev)
        layer.step(q, scale=D ** -0.5, out=out, lse=lse)
        torch.cuda.synchronize()
        res.append((layer.idx.clone(), layer.scores.clone(), out, lse))
    for a, b in zip(*res):
        assert torch.equal(a, b)
    # the choice itself: top_k of the oracle's fixed-order scores
    km = S.page_means(x.k[..., :n_cold * c, :], c, "bfloat16")
    qn = q.float().cpu().numpy()[:, :, None, :]
    sc = S.ordered_scores(qn, km, "bfloat16")
    np.testing.assert_array_equal(res[0][1].cpu().numpy()[0, :n_cold], sc[:n_cold])


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "two_kernel"])
def test_cold_chunks_read_in_place_from_pinned_host(dev, fused):
    """Cold chunks kept in pinned host memory (descriptors hold their
    device-visible addresses) are read by the kernels in place: indices,
    scores, outputs and LSE equal the same layer with the chunks in HBM."""
    from halo_amd.decode import ChunkRef
    from halo_amd.tiered import TieredDecodeLayer
    H, H_kv, D, c, n_hot, n_cold, top_k = 32, 8, 128, 256, 4, 12, 4
    x = decode_inputs(71, B=1, H=H, H_kv=H_kv, T=(n_hot + n_cold) * c, D=D, dtype="bfloat16", n_planted=4,
                      sigma=8.0)
    q, k, v = (_gpu(a, "bfloat16", dev) for a in (x.q, x.k, x.v))
    refs = [ChunkRef(k[..., i * c:(i + 1) * c, :], v[..., i * c:(i + 1) * c, :], i * c, True)
            for i in range(n_hot + n_cold)]
    dev_layer = TieredDecodeLayer(B=1, H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, hot=refs[n_cold:],
                                  cold=refs[:n_cold], top_k=top_k, device=dev, fused=fused)
    host_cold = [ChunkRef(r.k.cpu().pin_memory(), r.v.cpu().pin_memory(), r.chunk_start, r.causal)
                 for r in refs[:n_cold]]
    assert all(r.k.is_pinned() and r.k.device.type == "cpu" for r in host_cold)
    host_layer = TieredDecodeLayer(B=1, H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, hot=refs[n_cold:],
                                   cold=host_cold, top_k=top_k, device=dev, cold_kmean=dev_layer.kmean,
                                   fused=fused)
    res = []
    for layer in (dev_layer, host_layer):
        out = torch.empty((1, H, D), device=dev, dtype=torch.bfloat16)
        lse = torch.empty((1, H), device=dev)
        layer.step(q[:, :, 0], scale=D ** -0.5, out=out, lse=lse)
        torch.cuda.synchronize()
        res.append((layer.idx.clone(), layer.scores.clone(), out, lse))
    for a, b in zip(*res):
        assert torch.equal(a, b)


@pytest.mark.parametrize("n_cold,H,H_kv,B,per_row", [
    (96, 32, 8, 1, False),     # 768 (chunk, row, KV head) triples: the 131072-token layer's catalog
    (128, 24, 6, 1, False),    # 128 candidates, 768 triples
    (65, 16, 4, 2, False),     # one candidate past a wave, 520 triples over two rows
    (100, 16, 4, 2, True),     # per-row selection over 100 and 70 eligible chunks
])
def test_fused_selection_wide_catalog(dev, n_cold, H, H_kv, B, per_row):
    """The fused selection over more than 64 cold chunks (two ranking waves)
    and up to 768 triples: chunk scores bit-exact against the oracle's fixed
    summation order, the top-k against the oracle's ranking (margin-checked),
    and the output and LSE against the float64 closed form over the hot and
    the chosen rows."""
    from halo_amd import _native as nat
    from halo_amd.chunk_scorer import chunk_means
    from halo_amd.decode import ChunkRef, build_plan, descs_to_device, launch, pack_descs
    dtype, D, c, n_hot, top_k = "bfloat16", 128, 64, 4, 4
    T = (n_cold + n_hot) * c
    x = decode_inputs(60 + n_cold, B=B, H=H, H_kv=H_kv, T=T, D=D, dtype=dtype, n_planted=4, sigma=8.0)
    q, k, v = (_gpu(a, dtype, dev) for a in (x.q, x.k, x.v))
    refs = [ChunkRef(k[..., i * c:(i + 1) * c, :], v[..., i * c:(i + 1) * c, :], i * c, True)
            for i in range(T // c)]
    cold, hot = refs[:n_cold], refs[n_cold:]
    plan = build_plan(B=B, H=H, H_kv=H_kv, D=D, dtype=TDT[dtype], chunks=[cold[0]] * top_k + hot, device=dev)
    n_sel = B if per_row else 1
    cat_np, keep = pack_descs(cold * n_sel, B=B, H_kv=H_kv, D=D, dtype=TDT[dtype])
    cat = descs_to_device(cat_np, dev)
    km = chunk_means(k, c, n_pages=n_cold)
    n_el = np.array([n_cold, 70][:B] if per_row else [n_cold], np.int32)
    n_el_d = torch.from_numpy(n_el).to(dev)
    idx = torch.full((n_sel, top_k), -7, device=dev, dtype=torch.int32)
    sc = torch.full((n_sel, n_cold), -7.0, device=dev)
    cfg = nat.SelectCfg(kmean=km.data_ptr(), km_stride_b=km.stride(0), km_stride_h=km.stride(1),
                        km_stride_p=km.stride(2), catalog=cat.data_ptr(), catalog_stride=n_cold,
                        n_cold_per_sel=n_el_d.data_ptr() if per_row else None, n_cold=n_cold, top_k=top_k,
                        slot0=0, per_row=int(per_row), idx_out=idx.data_ptr(), score_out=sc.data_ptr())
    out = torch.empty((B, H, D), device=dev, dtype=torch.bfloat16)
    lse = torch.empty((B, H), device=dev)
    launch(plan, q[:, :, 0], scale=D ** -0.5, out=out, lse=lse, select=cfg)
    torch.cuda.synchronize()
    km_np = km.float().cpu().numpy()
    for s in range(n_sel):
        rows = slice(s, s + 1) if per_row else slice(0, B)
        ne = int(n_el[s])
        got = sc[s, :ne].cpu().numpy()
        np.testing.assert_array_equal(got, S.ordered_scores(x.q[rows], km_np[rows], dtype)[:ne])
        ref_sc = S.mean_key_scores(x.q[rows], km_np[rows], dtype)[:ne]
        srt = np.sort(ref_sc.astype(np.float64))[::-1]
        assert srt[top_k - 1] - srt[top_k] > 1e-4, "seed lost its top-k margin"
        want = S.select_chunks(x.q[rows], km_np[rows], np.arange(ne), top_k, dtype).tolist()
        assert idx[s].cpu().tolist() == want
        for b in (range(s, s + 1) if per_row else range(B)):
            keep_rows = np.zeros(T, bool)
            keep_rows[n_cold * c:] = True
            for j in want:
                keep_rows[j * c:(j + 1) * c] = True
            ro, rl = A.attention_f64(x.q[b:b + 1, :, 0], x.k[b:b + 1], x.v[b:b + 1], scale=D ** -0.5,
                                     keep=keep_rows)
            assert np.abs(out[b:b + 1].float().cpu().numpy() - ro).max() <= 2e-2
            assert np.abs(lse[b:b + 1].cpu().numpy() - rl).max() <= 1e-3
