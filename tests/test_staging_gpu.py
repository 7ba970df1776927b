"""The HBM staging cache for cold chunks in pinned host memory
(``ColdStaging``): with the cold tier on the host and a drifting query,
every step's output, LSE and selection equal those of the same layer with
every cold chunk in HBM, bit for bit, whether a chosen chunk is served from
a staging slot or read in place over the host link; fills and evictions
commit only between steps; a constant query ends with every selection a
hit.  Eager steps and HIP-graph replays are both covered."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _setup(dev, *, L=2, n_chunks=16, chunk=256, n_hot=4, top_k=3, slots=6, keep=None, seed=0, fill_mode="dma",
           adjacent=False, fused=True):
    """``adjacent``: each cold chunk's K and V rows adjacent in one pinned
    buffer (filled by one copy), else separate pinned tensors."""
    from halo_amd.decode import ChunkRef
    from halo_amd.staging import ColdStaging
    from halo_amd.tiered import TieredDecodeLayer
    H, H_kv, D = 16, 4, 128
    g = torch.Generator(device=dev).manual_seed(seed)
    hbm, staged = [], []
    for _ in range(L):
        k = torch.randn((1, H_kv, n_chunks * chunk, D), generator=g, device=dev)
        k[..., :3] *= 6
        k = k.to(torch.bfloat16)
        v = torch.randn((1, H_kv, n_chunks * chunk, D), generator=g, device=dev).to(torch.bfloat16)
        refs = [ChunkRef(k[..., i * chunk:(i + 1) * chunk, :], v[..., i * chunk:(i + 1) * chunk, :], i * chunk, True)
                for i in range(n_chunks)]
        n_cold = n_chunks - n_hot
        a = TieredDecodeLayer(B=1, H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, hot=refs[n_cold:], cold=refs[:n_cold],
                              top_k=top_k, device=dev, fused=fused)
        host = []
        buf = torch.empty((n_cold, 2) + tuple(refs[0].k.shape), dtype=torch.bfloat16, pin_memory=True)
        for j, c in enumerate(refs[:n_cold]):
            if adjacent:
                hk, hv = buf[j, 0], buf[j, 1]
            else:
                hk = torch.empty(tuple(c.k.shape), dtype=c.k.dtype, pin_memory=True)
                hv = torch.empty(tuple(c.v.shape), dtype=c.v.dtype, pin_memory=True)
            hk.copy_(c.k)
            hv.copy_(c.v)
            host.append(ChunkRef(hk, hv, c.chunk_start, True))
        b = TieredDecodeLayer(B=1, H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, hot=refs[n_cold:], cold=host,
                              top_k=top_k, device=dev, cold_kmean=a.kmean, fused=fused)
        hbm.append(a)
        staged.append(b)
    st = ColdStaging(staged, n_slots=slots, keep=keep, max_inflight=4, fill_mode=fill_mode)
    return hbm, staged, st, (H, D)


def _queries(dev, steps, L, H, D, rho, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn((L, 1, H, D), generator=g, device=dev)
    out = []
    for _ in range(steps):
        q = rho * q + math.sqrt(1 - rho * rho) * torch.randn((L, 1, H, D), generator=g, device=dev)
        out.append(q.to(torch.bfloat16))
    return out


@pytest.mark.parametrize("fill_mode,adjacent", [("dma", False), ("dma", True), ("kernel", False),
                                               ("kernel", True)])
def test_staged_steps_match_all_hbm_bit_for_bit(dev, fill_mode, adjacent):
    hbm, staged, st, (H, D) = _setup(dev, fill_mode=fill_mode, adjacent=adjacent)
    L = len(hbm)
    scale = 1 / math.sqrt(D)
    served = set()
    for t, q in enumerate(_queries(dev, 30, L, H, D, 0.8, 1)):
        st.before_step()
        outs = []
        for li in range(L):
            o1 = torch.empty((1, H, D), device=dev, dtype=torch.bfloat16)
            l1 = torch.empty((1, H), device=dev)
            o2, l2 = torch.empty_like(o1), torch.empty_like(l1)
            hbm[li].step(q[li], scale=scale, out=o1, lse=l1)
            staged[li].step(q[li], scale=scale, out=o2, lse=l2)
            outs.append((o1, l1, o2, l2))
        st.after_step()
        torch.cuda.synchronize()
        for li, (o1, l1, o2, l2) in enumerate(outs):
            assert torch.equal(o1, o2) and torch.equal(l1, l2), (t, li)
            assert torch.equal(hbm[li].idx[0], st.idx[li]), (t, li)
            res = st.res_out[li].cpu().numpy()
            served |= {int(c) for c, r in zip(st.idx[li].cpu().numpy(), res) if r >= 0}
        st.service()
    assert st.hits > 0 and st.misses > 0 and served
    assert st.fills > 0


def test_constant_query_ends_all_hits_in_a_graph(dev):
    hbm, staged, st, (H, D) = _setup(dev, seed=3)
    L = len(hbm)
    scale = 1 / math.sqrt(D)
    q = _queries(dev, 1, L, H, D, 0.0, 4)[0]
    qbuf = q.clone()
    outs = [torch.empty((1, H, D), device=dev, dtype=torch.bfloat16) for _ in range(L)]
    ref = [torch.empty_like(o) for o in outs]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for li in range(L):
            staged[li].step(qbuf[li], scale=scale, out=outs[li])
            hbm[li].step(q[li], scale=scale, out=ref[li])
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for li in range(L):
                staged[li].step(qbuf[li], scale=scale, out=outs[li])
        for _ in range(8):
            st.before_step()
            g.replay()
            st.after_step()
            st.service()
        torch.cuda.synchronize()
        for li in range(L):
            assert torch.equal(outs[li], ref[li])
            top = set(int(c) for c in st.idx[li].cpu().tolist())
            assert top <= set(st.resident(li))
        st.drain()
        st.reset_counters()
        for _ in range(3):
            st.before_step()
            g.replay()
            st.after_step()
            st.service()
        st.drain()
    assert st.misses == 0 and st.hits == 3 * L * 3
    for li in range(L):
        assert torch.equal(outs[li], ref[li])


def test_feedback_publication_in_unusual_call_orders(dev):
    """after_step only marks a segment's feedback rows; the next before_step
    on the same stream publishes them (one boundary kernel with its
    residency stores).  Every other order still gets every row processed
    exactly once: two after_step calls in a row, after_step on one stream and
    before_step on another, a lagged service that must not wait for a marked
    entry, and clear() with a marked entry (dropped)."""
    hbm, staged, st, (H, D) = _setup(dev, seed=5)
    L = len(hbm)
    k = staged[0].top_k
    scale = 1 / math.sqrt(D)
    q = _queries(dev, 1, L, H, D, 0.0, 6)[0]
    out = torch.empty((1, H, D), device=dev, dtype=torch.bfloat16)

    def run(li):
        staged[li].step(q[li], scale=scale, out=out)

    def counted():
        return st.hits + st.misses

    st.reset_counters()
    # two segments marked back to back (no before_step between them)
    st.before_step(0, 1)
    run(0)
    st.after_step(0, 1)
    run(1)
    st.after_step(1, 2)
    st.service(lag=1)          # must not wait for the newest, unpublished entry
    st.drain()
    assert counted() == L * k
    # marked on a side stream, the next before_step on the default stream
    s2 = torch.cuda.Stream()
    s2.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s2):
        for li in range(L):
            run(li)
        st.after_step()
    torch.cuda.current_stream().wait_stream(s2)
    st.before_step()
    for li in range(L):
        run(li)
    st.after_step()
    st.drain()
    assert counted() == 3 * L * k
    # a marked entry is dropped by clear(); the next steps count normally
    st.before_step()
    for li in range(L):
        run(li)
    st.after_step()
    st.clear()
    assert counted() == 0
    for _ in range(2):
        st.before_step()
        for li in range(L):
            run(li)
        st.after_step()
        st.service()
    st.drain()
    assert counted() == 2 * L * k


def test_staging_validates_its_inputs(dev):
    from halo_amd.staging import ColdStaging
    hbm, staged, st, _ = _setup(dev, L=1, slots=4)
    with pytest.raises(AssertionError):
        ColdStaging(hbm, n_slots=4)              # cold chunks in HBM, not pinned host memory
    with pytest.raises(AssertionError):
        ColdStaging(staged, n_slots=4, keep=2)   # keep below top_k
    with pytest.raises(AssertionError):
        ColdStaging(staged, n_slots=4, copy_streams=3)


@pytest.mark.parametrize("write_allocate", [True, False])
def test_write_allocate_commits_the_rows_read_in_place(dev, write_allocate):
    """A missed chunk's rows, read in place over the host link, are also
    written into the launch's reserved slot and committed as its residency:
    every slot the cache calls resident holds its chunk's K/V bit for bit
    (write-allocated or filled), results stay equal to the all-HBM layer, and
    with write-allocate off nothing is committed that way."""
    from halo_amd.staging import ColdStaging
    hbm, staged, _, (H, D) = _setup(dev, seed=5)
    st = ColdStaging(staged, n_slots=6, max_inflight=4, write_allocate=write_allocate)
    assert st.write_allocate == write_allocate
    L = len(hbm)
    scale = 1 / math.sqrt(D)
    reported = 0
    for t, q in enumerate(_queries(dev, 40, L, H, D, 0.7, 6)):
        st.before_step()
        outs = []
        for li in range(L):
            o1 = torch.empty((1, H, D), device=dev, dtype=torch.bfloat16)
            o2 = torch.empty_like(o1)
            hbm[li].step(q[li], scale=scale, out=o1)
            staged[li].step(q[li], scale=scale, out=o2)
            outs.append((o1, o2))
        st.after_step()
        torch.cuda.synchronize()
        for li, (o1, o2) in enumerate(outs):
            assert torch.equal(o1, o2), (t, li)
            res = st.res_out[li].cpu().numpy()
            reported += int((res <= -2).sum())
            # a reported write names one of the layer's reservations
            for r in res[res <= -2]:
                assert -2 - int(r) in set(int(w) for w in st.wa[li]) | set(range(st.n_slots))
        st.service()
    st.drain()
    torch.cuda.synchronize()
    if write_allocate:
        assert reported > 0 and st.wa_commits > 0
    else:
        assert reported == 0 and st.wa_commits == 0
    for li, lay in enumerate(staged):
        for s in range(st.n_slots):
            if st.state[li, s] != 2:  # READY
                continue
            c = int(st.holds[li, s])
            assert torch.equal(st._slot_k[li][s].cpu(), lay.cold[c].k), (li, s, c)
            assert torch.equal(st._slot_v[li][s].cpu(), lay.cold[c].v), (li, s, c)


@pytest.mark.parametrize("copy_streams", [1, 2])
def test_benchmark_loop_matches_all_hbm_every_step(dev, copy_streams):
    """The timed loop of the benchmark (``bench.refetch_run``: segment
    graphs, commits before each segment, feedback one segment late, fills
    and evictions planned while the next segments run, no synchronisation
    between steps), at a small scale with evictions (rho 0.8, 6 slots for
    12 cold chunks), with the fills on one copy stream or alternating
    between two: every step's output, LSE and picks, copied out in stream
    order, equal those of the all-HBM layers bit for bit; fills, commits and
    evictions were issued while launches were still queued."""
    import bench
    hbm, staged, _, (H, D) = _setup(dev, L=8, n_chunks=16, chunk=1024, n_hot=4, top_k=3, slots=6, keep=4,
                                    seed=11, adjacent=True)
    L, steps, k = len(hbm), 24, 3
    scale = 1 / math.sqrt(D)
    qtraj = bench.query_trajectory(torch, dev, steps=steps, L=L, H=H, D=D, rho=0.8, seed=12)
    out_hist = torch.zeros((steps, L, 1, H, D), device=dev, dtype=torch.bfloat16)
    lse_hist = torch.zeros((steps, L, 1, H), device=dev)
    idx_hist = torch.full((steps, L, k), -7, device=dev, dtype=torch.int32)
    res_hist = torch.full((steps, L, k), -7, device=dev, dtype=torch.int32)
    lses = [torch.zeros((1, H), device=dev) for _ in range(L)]

    def record(t, lo, hi, outs):
        for li in range(lo, hi):
            out_hist[t, li].copy_(outs[li])
            lse_hist[t, li].copy_(lses[li])
        idx_hist[t, lo:hi].copy_(st.idx[lo:hi])
        res_hist[t, lo:hi].copy_(st.res_out[lo:hi])

    # count what the runtime issues while the replay stream still has work queued
    from halo_amd.staging import ColdStaging
    st = ColdStaging(staged, n_slots=6, keep=4, max_inflight=6, track_busy=True, copy_streams=copy_streams)
    bench.refetch_run(torch, staged, st, qtraj, warmup=0, steps=steps, scale=scale, label="test", segments=2,
                      record=record, lses=lses)
    torch.cuda.synchronize()
    assert st.fills_while_busy > 0 and st.commits_while_busy > 0 and st.evictions_while_busy > 0, st.stats
    assert st.hits > 0 and st.misses > 0
    res = res_hist.cpu().numpy()
    assert (res >= 0).any() and ((res == -1).any())   # both slots and host reads served picks
    o_ref = torch.empty((1, H, D), device=dev, dtype=torch.bfloat16)
    l_ref = torch.empty((1, H), device=dev)
    for t in range(steps):
        for li in range(L):
            hbm[li].step(qtraj[t % steps, li], scale=scale, out=o_ref, lse=l_ref)
            assert torch.equal(out_hist[t, li], o_ref), (t, li)
            assert torch.equal(lse_hist[t, li], l_ref), (t, li)
            assert torch.equal(idx_hist[t, li], hbm[li].idx[0].to(torch.int32)), (t, li)


def _ragged_setup(dev, *, L=2, ctx=(1536, 3072, 768, 4096), chunk=256, top_k=2, seed=21):
    """All-HBM and staged ragged layers over the same K/V: per row, the last
    quarter of its chunks hot in HBM and the rest cold (staged: K and V of a
    chunk adjacent in one pinned buffer per row)."""
    from halo_amd.decode import ChunkRef
    from halo_amd.tiered import RaggedTieredDecodeLayer
    H, H_kv, D = 16, 4, 128
    g = torch.Generator(device=dev).manual_seed(seed)
    hbm, staged = [], []
    for _ in range(L):
        rows_h, rows_s = [], []
        for b, T in enumerate(ctx):
            k = torch.randn((H_kv, T, D), generator=g, device=dev)
            k[..., :3] *= 6
            k = k.to(torch.bfloat16)
            v = torch.randn((H_kv, T, D), generator=g, device=dev).to(torch.bfloat16)
            n = T // chunk
            n_hot = max(1, n // 4)
            refs = [ChunkRef(k[:, i * chunk:(i + 1) * chunk], v[:, i * chunk:(i + 1) * chunk], i * chunk, True,
                             batch=b) for i in range(n)]
            buf = torch.empty((n - n_hot, 2, H_kv, chunk, D), dtype=torch.bfloat16, pin_memory=True)
            host = []
            for j, c in enumerate(refs[:n - n_hot]):
                buf[j, 0].copy_(c.k)
                buf[j, 1].copy_(c.v)
                host.append(ChunkRef(buf[j, 0], buf[j, 1], c.chunk_start, True, batch=b))
            rows_h.append((refs[n - n_hot:], refs[:n - n_hot]))
            rows_s.append((refs[n - n_hot:], host))
        a = RaggedTieredDecodeLayer(H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, rows=rows_h, top_k=top_k, device=dev)
        s = RaggedTieredDecodeLayer(H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, rows=rows_s, top_k=top_k, device=dev,
                                    cold_kmean=a.kmean)
        hbm.append(a)
        staged.append(s)
    return hbm, staged, (len(ctx), H, D)


def test_staged_ragged_batch_matches_all_hbm(dev):
    """Per-row staging of a ragged batch (each row its own cold chunks,
    slots and policy; rows with 3 to 12 cold chunks and 4 slots) through the
    benchmark's loop: every step's outputs, LSEs and per-row picks equal the
    all-HBM ragged layers' bit for bit, and rows are served both from their
    slots and in place."""
    import bench
    from halo_amd.staging import ColdStaging
    hbm, staged, (B, H, D) = _ragged_setup(dev)
    L, steps, k = len(hbm), 20, 2
    scale = 1 / math.sqrt(D)
    st = ColdStaging(staged, n_slots=4, keep=3, max_inflight=6)
    assert st.sels == B and st.per_row
    qtraj = bench.query_trajectory(torch, dev, steps=steps, L=L, H=H, D=D, rho=0.8, seed=22, B=B)
    q_pos = torch.tensor([T - 1 for T in (1536, 3072, 768, 4096)], device=dev, dtype=torch.int64)
    out_hist = torch.zeros((steps, L, B, H, D), device=dev, dtype=torch.bfloat16)
    lse_hist = torch.zeros((steps, L, B, H), device=dev)
    idx_hist = torch.full((steps, L, B, k), -7, device=dev, dtype=torch.int32)
    res_hist = torch.full((steps, L, B, k), -7, device=dev, dtype=torch.int32)
    lses = [torch.zeros((B, H), device=dev) for _ in range(L)]

    def record(t, lo, hi, outs):
        for li in range(lo, hi):
            out_hist[t, li].copy_(outs[li])
            lse_hist[t, li].copy_(lses[li])
        idx_hist[t, lo:hi].copy_(st.idx[lo:hi])
        res_hist[t, lo:hi].copy_(st.res_out[lo:hi])

    bench.refetch_run(torch, staged, st, qtraj, warmup=0, steps=steps, scale=scale, label="ragged test",
                      segments=2, record=record, lses=lses, q_pos=q_pos)
    torch.cuda.synchronize()
    assert st.hits > 0 and st.misses > 0 and st.fills > 0
    res = res_hist.cpu().numpy()
    assert (res >= 0).any() and (res == -1).any()
    o_ref = torch.empty((B, H, D), device=dev, dtype=torch.bfloat16)
    l_ref = torch.empty((B, H), device=dev)
    for t in range(steps):
        for li in range(L):
            hbm[li].step(qtraj[t, li], scale=scale, out=o_ref, lse=l_ref, q_pos=q_pos)
            assert torch.equal(out_hist[t, li], o_ref), (t, li)
            assert torch.equal(lse_hist[t, li], l_ref), (t, li)
            assert torch.equal(idx_hist[t, li], hbm[li].idx), (t, li)
    # every ready slot of every row holds its chunk bit for bit
    state, holds = st.state, st.holds
    for li, lay in enumerate(staged):
        for b, (_, cold) in enumerate(lay.rows):
            u = li * B + b
            for s in range(st.n_slots):
                if state[u, s] == 2:
                    c = int(holds[u, s])
                    assert torch.equal(st._slot_k[u][s].cpu(), cold[c].k), (li, b, s, c)
                    assert torch.equal(st._slot_v[u][s].cpu(), cold[c].v), (li, b, s, c)


@pytest.mark.parametrize("fused", [False, True], ids=["two_launch", "fused"])
def test_staged_layers_wide_catalog(dev, fused):
    """Layers with 72 cold chunks, on the two-launch path (the staged scorer
    writes the chosen descriptors, with a staged chunk's slot addresses,
    into the table, then the attention launch; the path of layers beyond the
    fused selection's limits) and on the fused selection (two ranking
    waves past 64 chunks), match the all-HBM layers bit for bit through the
    benchmark's loop, with hits and misses both served."""
    import bench
    from halo_amd.staging import ColdStaging
    hbm, staged, _, (H, D) = _setup(dev, L=4, n_chunks=96, chunk=64, n_hot=24, top_k=4, slots=10, keep=6,
                                    seed=31, adjacent=True, fused=fused)
    assert staged[0].fused == fused and hbm[0].fused == fused
    L, steps, k = len(hbm), 20, 4
    scale = 1 / math.sqrt(D)
    st = ColdStaging(staged, n_slots=10, keep=6, max_inflight=8)
    assert st.all_fused == fused and (staged[0].staging is not None) == (not fused)
    qtraj = bench.query_trajectory(torch, dev, steps=steps, L=L, H=H, D=D, rho=0.8, seed=32)
    out_hist = torch.zeros((steps, L, 1, H, D), device=dev, dtype=torch.bfloat16)
    idx_hist = torch.full((steps, L, k), -7, device=dev, dtype=torch.int32)
    res_hist = torch.full((steps, L, k), -7, device=dev, dtype=torch.int32)

    def record(t, lo, hi, outs):
        for li in range(lo, hi):
            out_hist[t, li].copy_(outs[li])
        idx_hist[t, lo:hi].copy_(st.idx[lo:hi])
        res_hist[t, lo:hi].copy_(st.res_out[lo:hi])

    bench.refetch_run(torch, staged, st, qtraj, warmup=0, steps=steps, scale=scale, label="unfused test",
                      segments=2, record=record)
    torch.cuda.synchronize()
    assert st.hits > 0 and st.misses > 0 and st.fills > 0
    res = res_hist.cpu().numpy()
    assert (res >= 0).any() and (res == -1).any()
    o_ref = torch.empty((1, H, D), device=dev, dtype=torch.bfloat16)
    for t in range(steps):
        for li in range(L):
            hbm[li].step(qtraj[t, li], scale=scale, out=o_ref)
            assert torch.equal(out_hist[t, li], o_ref), (t, li)
            assert torch.equal(idx_hist[t, li], hbm[li].idx[0]), (t, li)
