"""Oracle: chunk-relevance scoring, top-k and refetch bookkeeping (numpy).

Test infrastructure only (see oracle/__init__.py).

Top-k order.  torch.topk leaves the order of tied scores undefined; this
build defines it as (score descending, index ascending) and returns the
selected indices sorted ascending, as every reference call site does with
``.sort()`` (baselines/scorer_ablations.py:266, halo/scorer.py:88,
halo/refetcher.py:57).
"""
from __future__ import annotations

from typing import Iterable, Optional

import numpy as np

from .inputs import round_to


def topk_indices(score: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest scores, ties broken by lower index, returned
    sorted ascending (int64)."""
    score = np.asarray(score)
    k = int(min(max(k, 0), score.shape[-1]))
    order = np.lexsort((np.arange(score.shape[-1]), -score.astype(np.float64)))
    return np.sort(order[:k]).astype(np.int64)


def page_means(K: np.ndarray, page_size: int, dtype: str = "float32") -> np.ndarray:
    """Per-page mean key (baselines/scorer_ablations.py:209-216):
    K[..., :n_full*p, :].view(B, H_kv, n_full, p, D).mean(-2), kept in K's
    dtype (``.mean`` on bf16/fp16 returns bf16/fp16).  The mean is taken in
    float64 and rounded once to the storage dtype.  Parity unpinned at the
    last fp32 bit for fp32 keys (torch's summation order); ranking is pinned
    instead (margin-checked fixtures)."""
    B, H_kv, T, D = K.shape
    n_full = T // page_size
    v = K[..., : n_full * page_size, :].reshape(B, H_kv, n_full, page_size, D)
    return round_to(v.astype(np.float64).mean(axis=-2).astype(np.float32), dtype)


def gqa_mean_query(query: np.ndarray, H_kv: int, dtype: str = "float32") -> np.ndarray:
    """query (B, H, T_q, D) -> q_g (B, H_kv, T_q, D): mean over the rep query
    heads of each KV head, in the query's dtype
    (baselines/scorer_ablations.py:223-232)."""
    B, H, T_q, D = query.shape
    if H == H_kv:
        return query.astype(np.float32)
    rep = H // H_kv
    g = query.reshape(B, H_kv, rep, T_q, D).astype(np.float32)
    # torch's mean: fp32 accumulation in order, times the fp32 factor 1/rep,
    # one rounding to the query dtype.
    acc = np.zeros((B, H_kv, T_q, D), np.float32)
    for r in range(rep):
        acc = (acc + g[:, :, r]).astype(np.float32)
    acc = (acc * np.float32(1.0 / rep)).astype(np.float32)
    return round_to(acc, dtype)


def mean_key_scores(query: np.ndarray, k_mean: np.ndarray, dtype: str = "float32") -> np.ndarray:
    """attn_p = max over (b, h_kv, t_q) of sum_d q_g . Kbar_p, in fp32
    (baselines/scorer_ablations.py:233-237).  Returns (P,) float32."""
    H_kv = k_mean.shape[1]
    q_g = gqa_mean_query(query, H_kv, dtype)
    attn = np.einsum("bhtd,bhpd->bhtp", q_g.astype(np.float64), k_mean.astype(np.float64))
    return attn.max(axis=(0, 1, 2)).astype(np.float32)


def ordered_dot(q_g: np.ndarray, k_mean: np.ndarray, dtype: str = "float32") -> np.ndarray:
    """sum_d q_g[..., d] * k_mean[..., p, d] in the build's fixed fp32 order:
    q_g (..., D), k_mean (..., P, D) -> (..., P) float32.

    The reference sums in torch's (unspecified) order
    (baselines/scorer_ablations.py:233-236); the build fixes one: D is cut
    into G = D/16 slices, slice c holding elements EP*(c + p*G) + e (EP =
    elements per 16 bytes: 4 for fp32, 8 for 16-bit keys; p < 16/EP,
    e < EP), each slice summed in (p, e) order with products and sums
    rounded to fp32 separately, then the G slice sums added as a balanced
    pairwise tree in slice order."""
    prod = (q_g.astype(np.float32)[..., None, :] * k_mean.astype(np.float32)).astype(np.float32)
    return slice_order_sum(prod, dtype)


def slice_order_sum(terms: np.ndarray, dtype: str = "float32") -> np.ndarray:
    """Sum float32 ``terms`` (..., D) over the last axis in the kernels'
    fixed order (the order ``ordered_dot`` describes), every addition
    rounded to fp32.  Returns (...,) float32."""
    D = terms.shape[-1]
    if D % 16:
        raise ValueError(f"head dim {D} must be a multiple of 16")
    EP = 4 if dtype == "float32" else 8
    G, PPS = D // 16, 16 // EP
    sl = terms.astype(np.float32).reshape(terms.shape[:-1] + (PPS, G, EP))
    sl = np.swapaxes(sl, -3, -2).reshape(terms.shape[:-1] + (G, 16))  # (..., G, 16) in (p, e) order
    part = np.zeros(sl.shape[:-1], np.float32)
    for j in range(16):
        part = (part + sl[..., j]).astype(np.float32)
    w = 1
    while w < G:
        for c in range(0, G - w, 2 * w):
            part[..., c] = (part[..., c] + part[..., c + w]).astype(np.float32)
        w *= 2
    return part[..., 0]


def ordered_scores(query: np.ndarray, k_mean: np.ndarray, dtype: str = "float32") -> np.ndarray:
    """Chunk scores as the kernels compute them: the GQA-mean query
    (rounded to the query dtype), ``ordered_dot`` with every page mean, max
    over (b, h_kv, t_q) ignoring NaN; a score that is NaN everywhere is -inf.
    Returns (P,) float32."""
    H_kv = k_mean.shape[1]
    q_g = gqa_mean_query(query, H_kv, dtype)  # (B, H_kv, T_q, D)
    dots = ordered_dot(q_g, k_mean[:, :, None], dtype)  # (B, H_kv, T_q, P)
    dots = np.where(np.isnan(dots), -np.inf, dots)
    return dots.max(axis=(0, 1, 2)).astype(np.float32)


def select_chunks(query: np.ndarray, k_mean: np.ndarray, eligible: np.ndarray, k: int,
                  dtype: str = "float32") -> np.ndarray:
    """The build's chunk selector: the alpha-only mean-key scorer
    (baselines/scorer_ablations.py:218-268 with halopress_beta =
    halopress_gamma = 0; the min-max normalisation there is monotone and
    does not change the ranking) restricted to ``eligible`` chunks, top-k
    with the (score desc, index asc) tie-break.  Returns chunk indices
    sorted ascending."""
    scores = mean_key_scores(query, k_mean, dtype).astype(np.float64)
    elig = np.asarray(eligible, dtype=np.int64)
    picked = topk_indices(scores[elig], k)
    return np.sort(elig[picked])


def num_hot_pages(P: int, memory_ratio: int, min_pages_selected: int) -> int:
    """_num_hot_pages (baselines/scorer_ablations.py:133-139), with the
    reference's float ratio.  Pinned by hand-worked known answers
    (tests/test_oracle.py::test_num_hot_pages_known_answers)."""
    K = max(min_pages_selected, int((P + memory_ratio - 1) // memory_ratio))
    return min(K, P)


def halopress_page_scores(attn: np.ndarray, *, alpha: float, beta: float, gamma: float,
                          refresh_window: int, sink_tokens: int, page_size: int) -> np.ndarray:
    """Full page score of HALOPressScorerAdapter.select_hot_pages
    (baselines/scorer_ablations.py:238-263), fp32: min-max normalised
    attention + recency + sink.  Pinned by torch's CPU ops on the
    reference's expression, the alpha-only min-max closed form, the
    beta-only closed form exp(-(P-1-p)/W), hand-counted sink pages and the
    additivity of the three terms (tests/test_oracle.py)."""
    a = attn.astype(np.float32) - attn.astype(np.float32).min()
    if float(a.max()) > 0.0:
        a = (a / a.max()).astype(np.float32)
    P = a.shape[0]
    pos = np.arange(P, dtype=np.float32)
    rec = np.exp(-(np.float32(P - 1) - pos) / np.float32(max(refresh_window, 1))).astype(np.float32)
    rec = (rec / (rec.sum() + np.float32(1e-12))).astype(np.float32)
    rec = (rec / (rec.max() + np.float32(1e-12))).astype(np.float32)
    sink = np.zeros(P, np.float32)
    sink[: min(sink_tokens // max(page_size, 1) + 1, P)] = 1.0
    return (np.float32(alpha) * a + np.float32(beta) * rec + np.float32(gamma) * sink).astype(np.float32)


def halo_score(attention: np.ndarray, *, step: int, alpha: float, beta: float, gamma: float,
               sink_tokens: int, refresh_window: int) -> np.ndarray:
    """HALOScorer.score (halo/scorer.py:36-72), fp32:
    attn / (sum + 1e-12); recency exp(-clamp(step - p, 0) / max(refresh, 1))
    normalised the same way; sink[:n] = 1; score / (max + 1e-12).
    Parity unpinned at the last fp32 bit (torch's sum order); the tests pin
    range, ranking and closed-form values."""
    K = attention.shape[-1]
    attn = attention.astype(np.float32)
    attn = (attn / (attn.sum(dtype=np.float32) + np.float32(1e-12))).astype(np.float32)
    pos = np.arange(K, dtype=np.float32)
    decay = np.float32(max(refresh_window, 1))
    rec = np.exp(-np.maximum(np.float32(step) - pos, 0.0) / decay).astype(np.float32)
    rec = (rec / (rec.sum(dtype=np.float32) + np.float32(1e-12))).astype(np.float32)
    sink = np.zeros(K, np.float32)
    if sink_tokens > 0:
        sink[: min(sink_tokens, K)] = 1.0
    score = (np.float32(alpha) * attn + np.float32(beta) * rec + np.float32(gamma) * sink).astype(np.float32)
    return (score / (score.max() + np.float32(1e-12))).astype(np.float32)


def topk_hot(score: np.ndarray, ratio: float) -> np.ndarray:
    """HALOScorer.topk_hot (halo/scorer.py:74-88): k = clamp(int(ratio*K), 1, K);
    ratio >= 1 returns arange(K)."""
    K = score.shape[-1]
    if ratio >= 1.0:
        return np.arange(K, dtype=np.int64)
    k = min(max(int(ratio * K), 1), K)
    return topk_indices(score, k)


def predict_hot(last_score: np.ndarray, *, hot_ratio: float, lookahead: int) -> np.ndarray:
    """HALORefetcher.predict_hot (halo/refetcher.py:38-57):
    top-(clamp(int(hot*K), 1) + lookahead) positions, sorted."""
    K = last_score.shape[-1]
    if hot_ratio >= 1.0:
        return np.arange(K, dtype=np.int64)
    k = min(max(int(hot_ratio * K), 1) + lookahead, K)
    return topk_indices(last_score, k)


def schedule(predicted: Iterable[int], *, block_size: int, locate, inflight: Optional[set] = None,
             layer: int = 0):
    """HALORefetcher.schedule (halo/refetcher.py:59-89) as pure bookkeeping:
    position -> block, dedupe, GPU-resident blocks are hits, others misses
    (unless already in flight).  Returns (hits, misses, blocks_to_fetch)."""
    inflight = set() if inflight is None else inflight
    seen, hits, misses, fetch = set(), 0, 0, []
    for pos in predicted:
        blk = int(pos) // block_size
        if blk in seen:
            continue
        seen.add(blk)
        tier = locate(layer, blk)
        if tier == "gpu":
            hits += 1
            continue
        if (layer, blk) in inflight:
            continue
        misses += 1
        inflight.add((layer, blk))
        fetch.append(blk)
    return hits, misses, fetch


# ---------------------------------------------------------------------------
# Quest bounding-box page scorer (baselines/quest_path_d.py:125-205)
# ---------------------------------------------------------------------------

def page_minmax(K: np.ndarray, page_size: int):
    """Per-page channel-wise K_min / K_max over the full pages of K
    (B, H_kv, T, D) (baselines/quest_path_d.py:125-150: ``amin`` / ``amax``
    over the page's rows, kept in K's dtype, so exact).  A NaN in a
    channel makes that channel's min and max NaN, as torch's amin/amax
    propagate it.  Returns (k_min, k_max) (B, H_kv, n_full, D)."""
    B, H_kv, T, D = K.shape
    n_full = T // page_size
    v = K[..., : n_full * page_size, :].reshape(B, H_kv, n_full, page_size, D)
    return v.min(axis=-2), v.max(axis=-2)


def quest_bound_dot(q_g: np.ndarray, k_min: np.ndarray, k_max: np.ndarray,
                    dtype: str = "float32") -> np.ndarray:
    """Quest's per-page upper bound sum_d max(q_d K_min_d, q_d K_max_d)
    (baselines/quest_path_d.py:175-178) for q_g (..., D) against pages
    (..., P, D): products rounded to fp32, the larger of the two taken
    (NaN if either is NaN, as ``torch.maximum``), summed in the kernels'
    fixed order (``slice_order_sum``; the reference's order is torch's).
    Returns (..., P) float32."""
    q = q_g.astype(np.float32)[..., None, :]
    a = (q * k_min.astype(np.float32)).astype(np.float32)
    b = (q * k_max.astype(np.float32)).astype(np.float32)
    with np.errstate(invalid="ignore"):
        m = np.maximum(a, b)  # np.maximum propagates NaN like torch.maximum
    return slice_order_sum(m, dtype)


def quest_scores(query: np.ndarray, k_min: np.ndarray, k_max: np.ndarray,
                 dtype: str = "float32") -> np.ndarray:
    """``score_pages`` (baselines/quest_path_d.py:152-182): the GQA-mean
    query (rounded to the query dtype, kept as is when H == H_kv) against
    every page's bounding box.  Returns (B, H_kv, T_q, P) float32."""
    H_kv = k_min.shape[1]
    q_g = gqa_mean_query(query, H_kv, dtype)  # (B, H_kv, T_q, D)
    return quest_bound_dot(q_g, k_min[:, :, None], k_max[:, :, None], dtype)


def quest_page_scores(query: np.ndarray, k_min: np.ndarray, k_max: np.ndarray,
                      dtype: str = "float32") -> np.ndarray:
    """Per-page score of ``select_hot_pages`` (baselines/quest_path_d.py:196):
    the max of ``quest_scores`` over (b, h_kv, t_q).  NaN bounds are ranked
    as -inf (the build's rule; torch.topk would rank NaN first).  Returns
    (P,) float32."""
    s = quest_scores(query, k_min, k_max, dtype)
    s = np.where(np.isnan(s), -np.inf, s)
    return s.max(axis=(0, 1, 2)).astype(np.float32)


def quest_num_hot_pages(P: int, memory_ratio: float, min_pages_selected: int) -> int:
    """K = min(P, max(min_pages_selected, int((P + r - 1) // r))) with the
    reference's float ratio (baselines/quest_path_d.py:197-200)."""
    K = max(int(min_pages_selected), int((P + memory_ratio - 1) // memory_ratio))
    return min(K, P)


def quest_select(query: np.ndarray, k_min: np.ndarray, k_max: np.ndarray, *, memory_ratio: float,
                 min_pages_selected: int, dtype: str = "float32") -> np.ndarray:
    """``select_hot_pages`` (baselines/quest_path_d.py:185-205): the top-K
    pages by ``quest_page_scores`` in descending score order (as
    ``torch.topk``), ties by lower page index.  Returns int64 (K,)."""
    s = quest_page_scores(query, k_min, k_max, dtype).astype(np.float64)
    K = quest_num_hot_pages(s.shape[0], memory_ratio, min_pages_selected)
    order = np.lexsort((np.arange(s.shape[0]), -s))
    return order[:K].astype(np.int64)
