"""GPU parity of the split-K decode-attention kernel against the oracle.

Mirrors the reference's kernel tests (tests/test_triton_chunked.py:72-312)
at the reference tolerances (rel-L2 1e-4 fp32 / 5e-3 bf16) and the
stricter max-abs ones of this path (1e-5 fp32 outputs and LSE, 2e-2 bf16),
calling the HIP path through the C-ABI.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle.inputs import decode_inputs

pytestmark = pytest.mark.gpu

TDT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}
TOL = {"float32": 1e-5, "bfloat16": 2e-2, "float16": 1e-2}


def _gpu(x, dtype, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev).to(TDT[dtype])


def _check(out, lse, ref, ref_lse, dtype):
    o = out.float().cpu().numpy().reshape(ref.shape)
    err = np.abs(o - ref).max()
    assert err <= TOL[dtype], f"max-abs {err:.3e} > {TOL[dtype]}"
    rel = np.linalg.norm(o - ref) / max(np.linalg.norm(ref), 1e-12)
    assert rel <= (1e-4 if dtype == "float32" else 5e-3), f"rel-L2 {rel:.3e}"
    if lse is not None:
        l = lse.float().cpu().numpy().reshape(ref_lse.shape)
        fin = np.isfinite(ref_lse)
        assert np.array_equal(np.isfinite(l), fin)
        lerr = np.abs(l[fin] - ref_lse[fin]).max() if fin.any() else 0.0
        assert lerr <= (1e-5 if dtype == "float32" else 1e-3 * max(1.0, np.abs(ref_lse[fin]).max())), \
            f"lse max-abs {lerr:.3e}"


def _split(k, v, cs, T):
    return [(k[..., c:min(c + cs, T), :].contiguous(), v[..., c:min(c + cs, T), :].contiguous(), c, True)
            for c in range(0, T, cs)]


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("chunk_size", [128, 512])
def test_matches_reference_small(dev, dtype, chunk_size):
    """reference test_triton_matches_reference_small: B1 H8 Hkv2 D64 T1024, x0.1."""
    from halo_amd.triton_chunked import triton_chunked_attention
    x = decode_inputs(0, B=1, H=8, H_kv=2, T=1024, D=64, dtype=dtype, q_scale=1.0)
    q = _gpu(x.q * 0.1, dtype, dev)
    k = _gpu(x.k * 0.1, dtype, dev)
    v = _gpu(x.v * 0.1, dtype, dev)
    qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
    scale = 1 / 8
    ref, ref_lse = A.attention_f64(qn[:, :, 0], kn, vn, scale=scale)
    out, lse = triton_chunked_attention(q, _split(k, v, chunk_size, 1024), scale=scale,
                                        q_pos=torch.tensor([1023], device=dev), return_lse=True)
    assert out.shape == (1, 8, 1, 64) and out.dtype == TDT[dtype]
    _check(out, lse, ref, ref_lse, dtype)


@pytest.mark.parametrize("chunk_size", [256, 512])
def test_causal_masking_and_truncation(dev, chunk_size):
    from halo_amd.triton_chunked import triton_chunked_attention
    x = decode_inputs(1, B=1, H=4, H_kv=1, T=2048, D=64)
    q, k, v = (_gpu(a * 0.1, "float32", dev) for a in (x.q, x.k, x.v))
    qn, kn, vn = x.q * 0.1, x.k * 0.1, x.v * 0.1
    qp = torch.tensor([1024], device=dev)
    ref, ref_lse = A.attention_f64(qn[:, :, 0], kn, vn, scale=0.125, q_pos=np.array([1024]))
    out, lse = triton_chunked_attention(q, _split(k, v, chunk_size, 2048), scale=0.125, q_pos=qp,
                                        return_lse=True)
    _check(out, lse, ref, ref_lse, "float32")
    half = [(k[..., :1025, :].contiguous(), v[..., :1025, :].contiguous(), 0, True)]
    out_h = triton_chunked_attention(q, half, scale=0.125, q_pos=qp)
    rel = (out - out_h).norm() / out.norm()
    assert rel.item() <= 1e-5


def test_single_launch_cold_hot(dev):
    from halo_amd.triton_chunked import triton_chunked_attention_single_launch as sl
    x = decode_inputs(3, B=1, H=8, H_kv=2, T=1280, D=64)
    q, k, v = (_gpu(a * 0.1, "float32", dev) for a in (x.q, x.k, x.v))
    ref, ref_lse = A.attention_f64(x.q[:, :, 0] * 0.1, x.k * 0.1, x.v * 0.1, scale=0.125)
    qp = torch.tensor([1279], device=dev)
    ck, cv = k[..., :1024, :].cpu().pin_memory(), v[..., :1024, :].cpu().pin_memory()
    out, lse = sl(q, ck, cv, k[..., 1024:, :].contiguous(), v[..., 1024:, :].contiguous(),
                  scale=0.125, q_pos=qp, return_lse=True)
    _check(out, lse, ref, ref_lse, "float32")
    out_c = sl(q, k.cpu().pin_memory(), v.cpu().pin_memory(), None, None, scale=0.125, q_pos=qp)
    _check(out_c, None, ref, ref_lse, "float32")
    out_h = sl(q, None, None, k, v, scale=0.125, q_pos=qp)
    _check(out_h, None, ref, ref_lse, "float32")


def test_non_contiguous_partition_and_permutation(dev):
    from halo_amd.triton_chunked import triton_chunked_attention
    x = decode_inputs(4, B=1, H=8, H_kv=2, T=2048, D=64)
    q, k, v = (_gpu(a * 0.1, "float32", dev) for a in (x.q, x.k, x.v))
    intervals = [(0, 256), (768, 1024), (1280, 1408), (1536, 1664), (1856, 2048)]
    keep = np.zeros(2048, bool)
    for lo, hi in intervals:
        keep[lo:hi] = True
    ref, ref_lse = A.attention_f64(x.q[:, :, 0] * 0.1, x.k * 0.1, x.v * 0.1, scale=0.125,
                                   keep=keep, q_pos=np.array([2047]))
    chunks = [(k[..., lo:hi, :].contiguous(), v[..., lo:hi, :].contiguous(), lo, True) for lo, hi in intervals]
    qp = torch.tensor([2047], device=dev)
    out, lse = triton_chunked_attention(q, chunks, scale=0.125, q_pos=qp, return_lse=True)
    _check(out, lse, ref, ref_lse, "float32")
    rng = np.random.default_rng(0)
    perm = [chunks[i] for i in rng.permutation(len(chunks))]
    out_p, lse_p = triton_chunked_attention(q, perm, scale=0.125, q_pos=qp, return_lse=True)
    _check(out_p, lse_p, ref, ref_lse, "float32")


def test_update_chunk_accumulates_like_one_shot(dev):
    from halo_amd.triton_chunked import finalize, init_acc, update_chunk
    x = decode_inputs(5, B=2, H=8, H_kv=2, T=700, D=64)
    q, k, v = (_gpu(a, "float32", dev) for a in (x.q, x.k, x.v))
    q3 = q[:, :, 0]
    m, l, o = init_acc(B=2, H=8, D_v=64, device=dev)
    qp = torch.tensor([650, 699], device=dev)
    for c0, c1 in [(0, 300), (300, 512), (512, 700)]:
        update_chunk(q=q3, k=k[..., c0:c1, :].contiguous(), v=v[..., c0:c1, :].contiguous(),
                     m=m, l=l, o=o, scale=0.125, chunk_start=c0, q_pos=qp, apply_causal=True)
    out, lse = finalize(m=m, l=l, o=o, out_dtype=torch.float32, return_lse=True)
    ref, ref_lse = A.attention_f64(x.q[:, :, 0], x.k, x.v, scale=0.125, q_pos=np.array([650, 699]))
    _check(out, lse, ref, ref_lse, "float32")
    # accumulators follow the oracle's (m, l, o) convention
    mo = np.full((2, 8), -np.inf, np.float32)
    lo_ = np.zeros((2, 8), np.float32)
    oo = np.zeros((2, 8, 64), np.float32)
    for c0, c1 in [(0, 300), (300, 512), (512, 700)]:
        A.update_chunk(x.q[:, :, 0], x.k[..., c0:c1, :], x.v[..., c0:c1, :], mo, lo_, oo, scale=0.125,
                       chunk_start=c0, q_pos=np.array([650, 699]), apply_causal=True)
    np.testing.assert_allclose(m.cpu().numpy(), mo, atol=1e-5)
    np.testing.assert_allclose(l.cpu().numpy(), lo_, rtol=1e-4)
    np.testing.assert_allclose(o.cpu().numpy(), oo, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("H,H_kv,D,dtype", [
    (8, 1, 64, "float32"), (8, 2, 64, "bfloat16"), (8, 4, 128, "float32"), (8, 8, 64, "float16"),
    (16, 2, 128, "bfloat16"), (28, 4, 128, "float16"), (32, 8, 128, "bfloat16"),
    (6, 2, 256, "bfloat16"), (32, 2, 64, "bfloat16"), (12, 4, 128, "float32"),
])
def test_gqa_shapes_and_dtypes(dev, H, H_kv, D, dtype):
    from halo_amd.triton_chunked import triton_chunked_attention
    x = decode_inputs(6, B=2, H=H, H_kv=H_kv, T=777, D=D, dtype=dtype)
    q, k, v = (_gpu(a, dtype, dev) for a in (x.q, x.k, x.v))
    scale = 1 / math.sqrt(D)
    ref, ref_lse = A.attention_f64(x.q[:, :, 0], x.k, x.v, scale=scale)
    out, lse = triton_chunked_attention(q, _split(k, v, 300, 777), scale=scale, return_lse=True)
    _check(out, lse, ref, ref_lse, dtype)


def test_edge_cases(dev):
    from halo_amd.triton_chunked import triton_chunked_attention
    x = decode_inputs(8, B=1, H=4, H_kv=1, T=512, D=64)
    q, k, v = (_gpu(a, "float32", dev) for a in (x.q, x.k, x.v))
    z = triton_chunked_attention(q, [])
    assert z.shape == (1, 4, 1, 64) and (z == 0).all()
    # the second chunk lies after the query: zero weight, not NaN
    chunks = [(k[..., :256, :].contiguous(), v[..., :256, :].contiguous(), 0, True),
              (k[..., 256:, :].contiguous(), v[..., 256:, :].contiguous(), 256, True)]
    qp = torch.tensor([100], device=dev)
    out, lse = triton_chunked_attention(q, chunks, scale=0.125, q_pos=qp, return_lse=True)
    ref, ref_lse = A.attention_f64(x.q[:, :, 0], x.k, x.v, scale=0.125, q_pos=np.array([100]))
    _check(out, lse, ref, ref_lse, "float32")
    # every row masked: out 0, lse -inf
    out0, lse0 = triton_chunked_attention(q, chunks[1:], scale=0.125, q_pos=qp, return_lse=True)
    assert (out0 == 0).all() and torch.isneginf(lse0).all()
    # ragged chunk lengths (not multiples of 64) and a 1-row chunk
    odd = [(k[..., :1, :].contiguous(), v[..., :1, :].contiguous(), 0, True),
           (k[..., 1:101, :].contiguous(), v[..., 1:101, :].contiguous(), 1, True),
           (k[..., 101:, :].contiguous(), v[..., 101:, :].contiguous(), 101, True)]
    out2, lse2 = triton_chunked_attention(q, odd, scale=0.125, return_lse=True)
    ref2, ref2_lse = A.attention_f64(x.q[:, :, 0], x.k, x.v, scale=0.125)
    _check(out2, lse2, ref2, ref2_lse, "float32")


@pytest.mark.parametrize("D,H,H_kv", [(64, 8, 2), (128, 16, 2), (256, 6, 2)])
@pytest.mark.parametrize("n_items", [12, 70, 130, 200])
def test_merge_shapes_by_partials_per_group(dev, D, H, H_kv, n_items):
    """The split-K merge takes a head's columns in slices (64 partials per
    group or fewer: 32-column slices; up to 80 and up to 144: 16-column
    slices) and one workgroup per head beyond that and whenever it reads and
    writes the caller's m/l: every form against the float64 closed form."""
    from halo_amd.decode import ChunkRef, build_plan, launch
    split = 64
    T = n_items * split - 17            # a short last item
    x = decode_inputs(40 + n_items, B=1, H=H, H_kv=H_kv, T=T, D=D, dtype="bfloat16")
    q, k, v = (_gpu(a, "bfloat16", dev) for a in (x.q, x.k, x.v))
    plan = build_plan(B=1, H=H, H_kv=H_kv, D=D, dtype=torch.bfloat16, chunks=[ChunkRef(k, v, 0, True)],
                      device=dev, split=split)
    assert plan.n_work == plan.n_groups * n_items
    scale = 1 / math.sqrt(D)
    ref, ref_lse = A.attention_f64(x.q[:, :, 0], x.k, x.v, scale=scale)
    out = torch.empty(1, H, D, device=dev, dtype=torch.bfloat16)
    lse = torch.empty(1, H, device=dev)
    launch(plan, q[:, :, 0], scale=scale, out=out, lse=lse)
    _check(out, lse, ref, ref_lse, "bfloat16")
    # read-and-write accumulators (one workgroup per head): from an empty
    # accumulator the result is the attention's (m, l, o)
    m = torch.full((1, H), -math.inf, device=dev)
    l = torch.zeros((1, H), device=dev)
    o = torch.zeros((1, H, D), device=dev)
    launch(plan, q[:, :, 0], scale=scale, m=m, l=l, o=o, acc_mode=3)
    fin = (o / l[..., None]).to(torch.bfloat16)
    _check(fin, m + torch.log(l), ref, ref_lse, "bfloat16")


def test_strided_views_need_no_copy(dev):
    """Chunks may be strided views of a larger cache (rows 16-byte aligned)."""
    from halo_amd.decode import ChunkRef, build_plan, launch
    x = decode_inputs(10, B=2, H=8, H_kv=2, T=1024, D=128, dtype="bfloat16")
    q, k, v = (_gpu(a, "bfloat16", dev) for a in (x.q, x.k, x.v))
    chunks = [ChunkRef(k[..., c:c + 256, :], v[..., c:c + 256, :], c, True) for c in range(0, 1024, 256)]
    plan = build_plan(B=2, H=8, H_kv=2, D=128, dtype=torch.bfloat16, chunks=chunks, device=dev)
    out = torch.empty(2, 8, 128, device=dev, dtype=torch.bfloat16)
    lse = torch.empty(2, 8, device=dev)
    launch(plan, q[:, :, 0], scale=1 / math.sqrt(128), out=out, lse=lse)
    ref, ref_lse = A.attention_f64(x.q[:, :, 0], x.k, x.v, scale=1 / math.sqrt(128))
    _check(out, lse, ref, ref_lse, "bfloat16")
    # a second launch with the same plan reuses the self-cleaning counters
    out_b = torch.empty_like(out)
    launch(plan, q[:, :, 0], scale=1 / math.sqrt(128), out=out_b)
    assert torch.equal(out, out_b)


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_misaligned_output_rows(dev, dtype):
    """An output view that is not 8/16-byte aligned takes the per-element
    store path and gives the same values as an aligned one."""
    from halo_amd.decode import ChunkRef, build_plan, launch
    x = decode_inputs(11, B=1, H=8, H_kv=2, T=512, D=64, dtype=dtype)
    q, k, v = (_gpu(a, dtype, dev) for a in (x.q, x.k, x.v))
    chunks = [ChunkRef(k[..., c:c + 256, :], v[..., c:c + 256, :], c, True) for c in range(0, 512, 256)]
    plan = build_plan(B=1, H=8, H_kv=2, D=64, dtype=TDT[dtype], chunks=chunks, device=dev)
    flat = torch.zeros(8 * 64 + 1, device=dev, dtype=TDT[dtype])
    out_mis = flat[1:].view(1, 8, 64)
    out = torch.empty(1, 8, 64, device=dev, dtype=TDT[dtype])
    launch(plan, q[:, :, 0], scale=0.125, out=out)
    launch(plan, q[:, :, 0], scale=0.125, out=out_mis)
    torch.cuda.synchronize()
    assert torch.equal(out, out_mis) and flat[0].item() == 0
    ref, _ = A.attention_f64(x.q[:, :, 0], x.k, x.v, scale=0.125)
    _check(out_mis, None, ref, None, dtype)


def test_ragged_batch_rows(dev):
    """Per-row chunk tables (varlen): row b attends only its own chunks."""
    from halo_amd.decode import ChunkRef, build_plan, launch
    lens = [300, 1000, 64]
    H, H_kv, D = 8, 2, 64
    rng = np.random.default_rng(12)
    qn = rng.standard_normal((3, H, D)).astype(np.float32)
    chunks, refs = [], []
    for b, T in enumerate(lens):
        kn = rng.standard_normal((H_kv, T, D)).astype(np.float32)
        vn = rng.standard_normal((H_kv, T, D)).astype(np.float32)
        kt, vt = torch.from_numpy(kn).to(dev), torch.from_numpy(vn).to(dev)
        for c in range(0, T, 256):
            chunks.append(ChunkRef(kt[:, c:c + 256], vt[:, c:c + 256], c, True, batch=b))
        refs.append(A.attention_f64(qn[b:b + 1], kn[None], vn[None], scale=0.125))
    plan = build_plan(B=3, H=H, H_kv=H_kv, D=D, dtype=torch.float32, chunks=chunks, device=dev)
    out = torch.empty(3, H, D, device=dev)
    lse = torch.empty(3, H, device=dev)
    launch(plan, torch.from_numpy(qn).to(dev), scale=0.125, out=out, lse=lse,
           q_pos=torch.tensor([T - 1 for T in lens], device=dev))
    for b in range(3):
        _check(out[b:b + 1], lse[b:b + 1], refs[b][0], refs[b][1], "float32")


def test_uniform_group_offsets_optional(dev):
    """A table whose groups own equal, consecutive slot ranges may omit
    group_offsets (NULL): the merge then derives them; results are
    bit-identical to passing the offsets, and the planner marks such tables."""
    import dataclasses

    from halo_amd.decode import ChunkRef, build_plan, launch
    x = decode_inputs(7, B=2, H=8, H_kv=2, T=2048, D=128, dtype="bfloat16")
    q, k, v = (_gpu(a, "bfloat16", dev) for a in (x.q, x.k, x.v))
    refs = [ChunkRef(k[..., c:c + 512, :], v[..., c:c + 512, :], c, True) for c in range(0, 2048, 512)]
    plan = build_plan(B=2, H=8, H_kv=2, D=128, dtype=torch.bfloat16, chunks=refs, device=dev, split=256)
    assert plan.uniform_groups and plan.n_work % plan.n_groups == 0
    outs = []
    for p in (plan, dataclasses.replace(plan, uniform_groups=False)):
        out = torch.empty((2, 8, 128), device=dev, dtype=torch.bfloat16)
        lse = torch.empty((2, 8), device=dev)
        launch(p, q[:, :, 0], scale=128 ** -0.5, out=out, lse=lse)
        torch.cuda.synchronize()
        outs.append((out, lse))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
    ref, ref_lse = A.attention_f64(qn[:, :, 0], kn, vn, scale=128 ** -0.5)
    _check(outs[0][0], outs[0][1], ref, ref_lse, "bfloat16")
    # a table with unequal groups (row 1 attends 3 items per group, row 0
    # attends 8) cannot omit the offsets: the entry point rejects it
    ragged = build_plan(B=2, H=8, H_kv=2, D=128, dtype=torch.bfloat16, chunks=refs, device=dev, split=256,
                        q_pos_host=[2047, 600])
    assert not ragged.uniform_groups and ragged.n_work % ragged.n_groups != 0
    out = torch.empty((2, 8, 128), device=dev, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        launch(dataclasses.replace(ragged, uniform_groups=True), q[:, :, 0], scale=128 ** -0.5, out=out)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_many_partials_per_group(dev, dtype):
    """Groups of more than 64 partials (here 128 and 130) take the merge's
    512-thread form; results match the float64 closed form like the
    256-thread form's."""
    from halo_amd.decode import ChunkRef, build_plan, launch
    x = decode_inputs(11, B=1, H=4, H_kv=1, T=16640, D=128, dtype=dtype)
    q, k, v = (_gpu(a, dtype, dev) for a in (x.q, x.k, x.v))
    qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
    ref, ref_lse = A.attention_f64(qn[:, :, 0], kn, vn, scale=128 ** -0.5)
    for T, split in ((16384, 128), (16640, 128), (16384, 256)):
        refs = [ChunkRef(k[..., c:min(c + 1024, T), :], v[..., c:min(c + 1024, T), :], c, True)
                for c in range(0, T, 1024)]
        plan = build_plan(B=1, H=4, H_kv=1, D=128, dtype=TDT[dtype], chunks=refs, device=dev, split=split)
        assert (plan.n_work > 64 * plan.n_groups) == (split == 128)
        out = torch.empty((1, 4, 128), device=dev, dtype=TDT[dtype])
        lse = torch.empty((1, 4), device=dev)
        launch(plan, q[:, :, 0], scale=128 ** -0.5, out=out, lse=lse)
        torch.cuda.synchronize()
        r, rl = (ref, ref_lse) if T == 16640 else A.attention_f64(qn[:, :, 0], kn[..., :T, :], vn[..., :T, :],
                                                                 scale=128 ** -0.5)
        _check(out, lse, r, rl, dtype)
