/*
 * halo_hip.h -- C-ABI of the MI355X-native tiered-KV attention path.
 *
 * Every entry point is stateless apart from the caller-owned buffers it is
 * handed, takes plain device pointers, element strides and sizes, and
 * enqueues its work on the HIP stream passed as `stream` (a hipStream_t cast
 * to void*; NULL means the null stream).  Nothing here allocates device
 * memory: partial results and merge tickets live in a caller-provided
 * workspace whose size the *_workspace_size() helpers report.  Return value
 * is 0 on success or a negative HALO_E* code; halo_last_error() returns a
 * thread-local description of the last failure.
 *
 * The Python shim in halo_amd/ maps these codes to the exceptions the
 * reference raises (AssertionError for shape errors, RuntimeError otherwise).
 */
#ifndef HALO_HIP_H
#define HALO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define HALO_OK 0
#define HALO_E_INVALID -1     /* bad argument / shape (reference: AssertionError) */
#define HALO_E_UNSUPPORTED -2 /* shape/dtype combination not instantiated        */
#define HALO_E_HIP -3         /* HIP runtime error                               */
#define HALO_E_WORKSPACE -4   /* workspace too small                             */

/* ---- element types ----------------------------------------------------- */
#define HALO_F32 0
#define HALO_BF16 1
#define HALO_F16 2

/* ---- chunk descriptor flags -------------------------------------------- */
#define HALO_CHUNK_CAUSAL 1   /* mask rows with chunk_start + t > q_pos[b] */
#define HALO_CHUNK_KIVI2  2   /* a run of 2-bit KIVI blocks (halo_decode_attn_kivi):
                                 k = first block, k_stride_b/h in bytes, v unused */

/*
 * One KV chunk: rows [0, T_c) of K and V at global key positions
 * [chunk_start, chunk_start + T_c).  `batch` = -1 means the chunk has a
 * batch dimension (row b of the call's batch at k + b*k_stride_b); batch >= 0
 * means the chunk belongs to that batch row only (ragged / varlen tables) and
 * k points at that row's (h=0, t=0, d=0) element.  The head dimension is
 * contiguous (unit stride).  Replaces the (k, v, chunk_start, apply_causal)
 * tuple of halo/triton_chunked.py:212 and the per-launch arguments of
 * halo/triton_chunked.py:180-192.
 */
typedef struct halo_chunk_desc {
  const void* k;
  const void* v;
  int64_t k_stride_b, k_stride_h, k_stride_t; /* elements */
  int64_t v_stride_b, v_stride_h, v_stride_t; /* elements */
  int64_t chunk_start;
  int32_t T_c;
  int32_t flags;
  int32_t batch;
  int32_t reserved;
} halo_chunk_desc; /* 88 bytes */

/*
 * Work decomposition for one decode-attention launch.  Work record i (int32 x8):
 *   { desc index, group, t0, t1, slot, 0, 0, 0 }  -- rows [t0, t1) of chunk
 * `desc` for query-head group `group` = (b * H_kv + h_kv) * n_sub + sub, where
 * sub selects q heads [h_kv*rep + sub*rep_t, ...) of that KV head; the item's
 * partial goes to workspace slot `slot`.  Group g's partials occupy slots
 * group_offsets[g] .. group_offsets[g+1]-1, and every group owns at least one
 * item (an item with t0 == t1 is an empty partial).  Records are in dispatch
 * order, which need not follow the slot order.
 */

/* Bytes of workspace a launch with `n_work` items needs (one partial per item). */
size_t halo_decode_workspace_size(int n_work, int rep_t, int D);

/*
 * Split-K GQA decode attention over a chunk table with a log-sum-exp merge.
 * One query token per batch row.
 *
 *   q        (B, H, D) elements of `dtype`, q[b*q_stride_b + h*q_stride_h + d]
 *   descs    device array of n_desc halo_chunk_desc
 *   work     device int32 array [n_work][8] of {desc, group, t0, t1, slot, 0,
 *            0, 0} in dispatch order: the item attends rows [t0, t1) of
 *            descs[desc] for query-head group `group` = (b*H_kv + h_kv)*n_sub
 *            + sub (n_sub = ceil(rep/rep_t)) and writes partial `slot`;
 *            the slots of group g are group_offsets[g] .. group_offsets[g+1]-1
 *            (device int32 [n_groups+1]), a permutation of 0 .. n_work-1;
 *            NULL when every group owns n_work / n_groups slots, group g
 *            slots g*(n_work/n_groups) .. (g+1)*(n_work/n_groups)-1 (the merge
 *            then reads no offsets)
 *   q_pos    device int64 [B] global query position, or NULL (no causal mask)
 *   scale    softmax scale applied to q.k in fp32
 *   m,l,o    fp32 online-softmax accumulators (B,H), (B,H), (B,H,D) with the
 *            convention m = running max of scale*q.k, l = sum exp(s-m),
 *            o = sum exp(s-m) v (halo/triton_chunked.py:84-87,132-138).
 *            acc_mode bit0: merge the incoming (m,l,o) into the result;
 *            bit1: write the merged (m,l,o) back.  Ignored when m == NULL.
 *   out      (B,H,D) of `out_dtype` = o/l (0 where l == 0), or NULL
 *   lse      (B,H) fp32 = m + log(l) (-inf where l == 0), or NULL
 *   workspace caller-owned device memory of halo_decode_workspace_size()
 *            bytes; calls that overlap on one stream must not share it
 *
 * Enqueues two kernels on `stream`: the split-K attention pass, which writes
 * one partial per work item, and a merge pass that combines each group's
 * partials (in slot order: results are deterministic) with the accumulators.
 * Replaces update_chunk / finalize / triton_chunked_attention
 * (halo/triton_chunked.py:151-267) and the PyTorch chunk walk
 * (halo/kv_cache_chunked.py:194-276, 864-964) for T_q == 1.
 */
int halo_decode_attn(const void* q, int64_t q_stride_b, int64_t q_stride_h, int dtype,
                     int B, int H, int H_kv, int D, int rep_t,
                     const halo_chunk_desc* descs, int n_desc,
                     const int32_t* work, int n_work,
                     const int32_t* group_offsets, int n_groups,
                     const int64_t* q_pos, float scale,
                     float* m, float* l, float* o, int64_t acc_stride_b, int acc_mode,
                     void* out, int out_dtype, float* lse,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * In-kernel chunk selection for halo_decode_attn_tiered.  Work items whose
 * descriptor index d lies in [slot0, slot0 + top_k) are selection slots:
 * their workgroup scores the cold chunks catalog[s*catalog_stride + p],
 * p < n_cold (or n_cold_per_sel[s]), with the alpha-only mean-key score of
 * halo_chunk_score_topk (raw q.Kbar, max over rows and KV heads; selection s
 * is batch row s when per_row != 0, else all rows) and attends the
 * (d - slot0)-th chosen chunk in ascending index order (top-k order: score
 * descending, then index ascending); a slot past the number of eligible
 * chunks attends nothing.  idx_out[s*top_k + j] / score_out[s*n_cold + p]
 * receive the selection when non-NULL.  Limits: n_cold <= 128 and
 * n_cold * rows * H_kv <= 768 for bf16/fp16 (64 and 512 for fp32),
 * rows * H_kv * D <= 2048 per selection and
 * head_dim % 16 == 0 (rows = 1 when per_row).  The dot products use the
 * scorer's fixed summation order (halo_chunk_score_topk).  The work
 * items of a slot must cover as many rows as the largest catalog chunk (rows
 * past a chunk's T_c are skipped).
 */
typedef struct halo_select_cfg {
  const void* kmean; /* (B|1, H_kv, n_cold, D) page means, K dtype, rows 16-byte aligned */
  int64_t km_stride_b, km_stride_h, km_stride_p;
  const halo_chunk_desc* catalog;
  int64_t catalog_stride;
  const int32_t* n_cold_per_sel; /* NULL: n_cold for every selection */
  int32_t n_cold, top_k, slot0, per_row;
  int32_t* idx_out;
  float* score_out;
  /* The first lead_items work records (dispatch order) are selection-slot
   * items (0 = not stated).  Those workgroups start the selection's loads
   * before reading their record; a wrong count costs loads, not results. */
  int32_t lead_items;
  /* HBM staging of the cold chunks (all NULL / 0: every chosen chunk is
   * read through its catalog descriptor).  residency[s*catalog_stride + p]
   * is the staging slot that holds cold chunk p (-1: none); the kernel then
   * reads the chunk's rows through the addresses and strides of
   * slot_catalog[s*n_slots + slot] (its rows, start, flags and batch still
   * come from the chunk's catalog entry, so slot descriptors never change).  Writers
   * store a slot index only after the slot's rows have landed, and -1 only
   * when the slot will not be overwritten before the launches that may have
   * read the old index have finished, so a launch reads either descriptor
   * and the same rows.  res_out[s*top_k + j] receives the residency entry
   * used for the j-th chosen chunk (>= 0: served from HBM staging).
   * n_slots <= 64. */
  int32_t n_slots;
  const halo_chunk_desc* slot_catalog;
  const int32_t* residency;
  int32_t* res_out;
  /* Write-allocate (NULL: off; needs residency, bf16/fp16, per_row == 0).
   * *alloc_slot names a staging slot that no residency entry names (-1:
   * none this launch).  The first chosen chunk (in pick order) that is not
   * staged is read in place as usual and its rows are also written into
   * that slot's storage by the same workgroups; res_out then holds
   * -2 - slot for it.  The slot holds the chunk once the launch has
   * finished, so a later launch may be pointed at it without a copy over
   * the host link. */
  const int32_t* alloc_slot;
} halo_select_cfg;

/*
 * halo_decode_attn with the chunk selection fused in (sel != NULL), so a
 * decode layer over hot + scorer-chosen cold chunks is one attention launch
 * plus its merge, with no host round trip.  Replaces the select_hot_pages ->
 * chunk walk sequence (baselines/scorer_ablations.py:218-268,
 * halo/kv_cache_chunked.py:416-457, 571-763) for T_q == 1.
 */
int halo_decode_attn_tiered(const void* q, int64_t q_stride_b, int64_t q_stride_h, int dtype,
                            int B, int H, int H_kv, int D, int rep_t,
                            const halo_chunk_desc* descs, int n_desc,
                            const int32_t* work, int n_work,
                            const int32_t* group_offsets, int n_groups,
                            const int64_t* q_pos, float scale,
                            float* m, float* l, float* o, int64_t acc_stride_b, int acc_mode,
                            void* out, int out_dtype, float* lse,
                            void* workspace, size_t workspace_bytes,
                            const halo_select_cfg* sel, void* stream);

/*
 * Allocation-free variant of halo_decode_attn_tiered (sel != NULL) and
 * halo_decode_attn (sel == NULL): same arguments and results, but the split-K
 * partials go to a static device array inside the library instead of a
 * caller workspace, so the caller passes only inputs and outputs.  No
 * counterpart in the reference; it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Each GPU holds one copy of the array,
 * halo_decode_static_scratch_bytes() bytes (8 MiB), until the process ends;
 * a table whose partials (halo_decode_workspace_size) exceed it is refused
 * with HALO_E_WORKSPACE before anything is launched.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (two streams) race.
 * Nothing in the array needs clearing between calls (every work item writes
 * its own partial before the merge reads it).
 */
size_t halo_decode_static_scratch_bytes(void);
int halo_decode_attn_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h, int dtype,
                             int B, int H, int H_kv, int D, int rep_t,
                             const halo_chunk_desc* descs, int n_desc,
                             const int32_t* work, int n_work,
                             const int32_t* group_offsets, int n_groups,
                             const int64_t* q_pos, float scale,
                             float* m, float* l, float* o, int64_t acc_stride_b, int acc_mode,
                             void* out, int out_dtype, float* lse,
                             const halo_select_cfg* sel, void* stream);

/*
 * finalize: out = o / (l > 0 ? l : 1) cast to out_dtype, optional
 * lse = m + log(l).  Replaces halo/triton_chunked.py:195-207 (which does not
 * return the LSE).  m,l: (B,H) fp32 contiguous, o: (B,H,D) fp32 contiguous.
 */
int halo_finalize(const float* m, const float* l, const float* o, int B, int H, int D,
                  void* out, int out_dtype, float* lse, void* stream);

/*
 * LSE merge of two partial (out, lse) pairs, fp32, n rows of width D:
 * lse = logaddexp(la, lb); out = wa*oa + wb*ob with zero weight (and zero
 * contribution) for a side whose lse is -inf.  Replaces
 * HALOCacheChunked._lse_merge (halo/kv_cache_chunked.py:194-239).
 */
int halo_lse_merge(const float* out_a, const float* lse_a, const float* out_b,
                   const float* lse_b, int64_t n, int D, float* out, float* lse,
                   void* stream);

/* ---- chunked causal prefill -------------------------------------------- */

/*
 * Prefill attention of T_q query rows per (b, h) over a chunk table, bf16 or
 * fp16 on MFMA: out[b,h,i,:] = softmax over every attended key row of every
 * chunk, where row t of chunk c is attended by query row i iff the chunk is
 * not causal or c.chunk_start + t <= q_start[b] + i; lse[b,h,i] = log of the
 * softmax denominator of scale*q.k (-inf when nothing is attended, out 0).
 * q[b*q_stride_b + h*q_stride_h + i*q_stride_t + d] (16-byte aligned rows);
 * out likewise with its own strides and out_dtype; lse (B,H,T_q) fp32 or
 * NULL; q_start device int64 [B].  One pass over the table gives the same
 * result as the reference's per-chunk partials merged by log-sum-exp:
 * replaces the T_q > 1 route of HALOCacheChunked.compute_attention
 * (halo/kv_cache_chunked.py:864-964 with _chunk_attention/_lse_merge,
 * :194-276).  D in {64, 128}.
 */
int halo_prefill_attn(const void* q, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t,
                      int dtype, int B, int H, int H_kv, int T_q, int D, const int64_t* q_start,
                      const halo_chunk_desc* descs, int n_desc, float scale,
                      void* out, int64_t out_stride_b, int64_t out_stride_h, int64_t out_stride_t,
                      int out_dtype, float* lse, void* stream);

/* ---- chunk-relevance scoring ------------------------------------------- */

/*
 * Page-mean keys for `n_pages` pages of `page` rows starting at row `row0`:
 * kmean[b,h,j,:] = dtype(sum_t K[b,h,row0+j*page+t,:] / page), fp32 sums in
 * row order, one rounding to the key dtype (torch's .mean keeps the dtype).
 * Replaces the per-update recomputation of baselines/scorer_ablations.py:
 * 209-216; called once per page when it fills.
 */
int halo_chunk_means(const void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
                     int dtype, int B, int H_kv, int D, int64_t row0, int page, int n_pages,
                     void* kmean, int64_t km_stride_b, int64_t km_stride_h, int64_t km_stride_p,
                     void* stream);

/*
 * Chunk scoring + top-k, one selection per batch row (per_row != 0) or one
 * over all rows (per_row == 0: the reference's amax over batch).  For
 * selection s, eligible chunk indices are eligible[s*elig_stride + i],
 * i < n_elig_per_sel[s] (or n_elig when that array is NULL; n_elig <= 1024).
 *   attn[i] = max over (rows, h_kv) of sum_d qbar[h_kv,d] * kmean[p_i,d], with
 *   qbar the mean of each KV head's query heads rounded to the q dtype
 *   (baselines/scorer_ablations.py:223-237).  With normalize != 0 the score is
 *   alpha*minmax(attn) + beta*recency + gamma*sink over P_total pages
 *   (:238-263); otherwise the raw attn.
 * Top-k order: score descending, then chunk index ascending; the k chosen
 * indices are written ascending to idx_out[s*k + j] (-1 when fewer than k are
 * eligible); raw/final scores to score_out[s*n_elig + i] when non-NULL.  When
 * `table` is non-NULL, descriptor catalog[s*catalog_stride + p] of each chosen
 * chunk p is copied to table[s*table_stride + table_slot0 + j] (an empty
 * descriptor, T_c = 0, fills unused slots), so a following halo_decode_attn
 * on the same stream attends the selection with no host round trip.
 * Replaces select_hot_pages (baselines/scorer_ablations.py:218-268) and the
 * torch.topk + .cpu() sync at :266.
 */
int halo_chunk_score_topk(const void* q, int64_t q_stride_b, int64_t q_stride_h, int dtype,
                          int B, int H, int H_kv, int D,
                          const void* kmean, int64_t km_stride_b, int64_t km_stride_h,
                          int64_t km_stride_p,
                          const int32_t* eligible, int64_t elig_stride,
                          const int32_t* n_elig_per_sel, int n_elig, int k, int per_row,
                          int32_t* idx_out, float* score_out,
                          const halo_chunk_desc* catalog, int64_t catalog_stride,
                          halo_chunk_desc* table, int64_t table_stride, int table_slot0,
                          int normalize, float alpha, float beta, float gamma,
                          int refresh, int sink_pages, int P_total,
                          void* stream);

/*
 * halo_chunk_score_topk (raw attn scores, normalize = 0) for a layer whose
 * cold chunks are served by an HBM staging cache: a chosen chunk p whose
 * residency[s*catalog_stride + p] names a slot r in [0, n_slots) is written
 * to the table with the addresses and strides of slot_catalog[s*n_slots + r]
 * (its rows, start, flags and batch from its own catalog entry), and
 * res_out[s*k + j] receives the entry used for the j-th chosen chunk (-1:
 * read in place; unfilled slots -1).  The two-launch selection path (this,
 * then halo_decode_attn over the table) of layers beyond the fused
 * selection's limits (more than 128 cold chunks or 768 (chunk, row, KV head)
 * triples); the same residency protocol as halo_select_cfg.  The reference
 * selects on the host and refetches with HALORefetcher
 * (baselines/scorer_ablations.py:218-268, halo/refetcher.py:59-114).
 */
int halo_chunk_score_topk_staged(const void* q, int64_t q_stride_b, int64_t q_stride_h, int dtype,
                                 int B, int H, int H_kv, int D,
                                 const void* kmean, int64_t km_stride_b, int64_t km_stride_h,
                                 int64_t km_stride_p,
                                 const int32_t* eligible, int64_t elig_stride,
                                 const int32_t* n_elig_per_sel, int n_elig, int k, int per_row,
                                 int32_t* idx_out, float* score_out,
                                 const halo_chunk_desc* catalog, int64_t catalog_stride,
                                 halo_chunk_desc* table, int64_t table_stride, int table_slot0,
                                 const int32_t* residency, const halo_chunk_desc* slot_catalog,
                                 int n_slots, int32_t* res_out, void* stream);

/*
 * Quest page metadata: channel-wise minima and maxima of `n_pages` pages of
 * `page` rows starting at row `row0`, kmin[b,h,j,:] / kmax[b,h,j,:] in the
 * key dtype (exact; a NaN in a channel propagates, as torch.amin / amax).
 * Replaces the K_min / K_max build of _QuestScorerAdapter.observe_keys
 * (baselines/quest_path_d.py:125-150); called once per page when it fills.
 */
int halo_page_minmax(const void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
                     int dtype, int B, int H_kv, int D, int64_t row0, int page, int n_pages,
                     void* kmin, void* kmax, int64_t km_stride_b, int64_t km_stride_h,
                     int64_t km_stride_p, void* stream);

/*
 * Quest upper-bound page scores and top-k.  q (B, H, T_q, D) by strides;
 * kmin / kmax (B, H_kv, P, D) share strides, P <= 8192, D % 16 == 0,
 * D <= 256.  For every (b, h_kv, t) row:
 *   bound[p] = sum_d max(qbar[d] * kmin[p,d], qbar[d] * kmax[p,d])
 * with qbar the mean of the KV head's query heads rounded to the q dtype,
 * fp32 products, summed in the fixed order of halo_chunk_score_topk.  The
 * bounds go to dots_out (B, H_kv, T_q, P) fp32 when non-NULL (score_pages,
 * baselines/quest_path_d.py:152-182).  Selection s (batch row s when
 * per_row != 0, else all rows) scores page p as the max bound over its rows
 * (NaN ranks as -inf), written to score_out[s*P + p] when non-NULL, and the
 * top k pages go to idx_out[s*k + j] in descending score order, ties by
 * lower page index (select_hot_pages, :185-205, whose torch.topk leaves
 * ties undefined).  workspace: n_sel * P uint32 (n_sel = B if per_row else 1).
 */
int halo_quest_score_topk(const void* q, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t,
                          int dtype, int B, int H, int H_kv, int T_q, int D,
                          const void* kmin, const void* kmax, int64_t km_stride_b, int64_t km_stride_h,
                          int64_t km_stride_p, int P, int k, int per_row, uint32_t* workspace,
                          float* dots_out, float* score_out, int32_t* idx_out, void* stream);

/* ---- HALOScorer: closed-form hotness and sorted top-k -------------------- */

/*
 * score[p] for p < K from the head-mean attention snapshot attention[p]
 * (fp32): a = attention/(sum + 1e-12), r = exp(-max(step - p, 0) /
 * max(refresh_window, 1)), r /= (sum r + 1e-12), s = 1 for p <
 * sink_tokens, score = (alpha*a + beta*r + gamma*s) / (max + 1e-12).
 * Sums run in index order (deterministic).  Replaces HALOScorer.score
 * (halo/scorer.py:36-72).  K <= 2^24.
 */
int halo_halo_score(const float* attention, int K, int step, float alpha, float beta, float gamma,
                    int sink_tokens, int refresh_window, float* score, void* stream);

/*
 * Indices of the k largest of score[0..K) (fp32), written ascending to
 * idx_out (int64, k entries); ties go to the lower index, NaN ranks as -inf.
 * Replaces torch.topk(score, k).indices.sort() of HALOScorer.topk_hot and
 * HALORefetcher.predict_hot (halo/scorer.py:74-88, halo/refetcher.py:38-57),
 * whose tie order torch leaves undefined.  1 <= k <= K <= 2^24.
 */
int halo_topk_sorted(const float* score, int K, int k, int64_t* idx_out, void* stream);

/* ---- KIVI 2/4/8-bit cold-chunk format ---------------------------------- */

/*
 * Block format: one block = 32 tokens of one (b, h_kv), all in one
 * contiguous record of halo_kivi_block_bytes(D, bits) bytes:
 *   K codes   32 token rows of D*bits/8 bytes, one code per channel (K is
 *             grouped per channel over the block's 32 tokens)
 *   K scale   D elements of the storage dtype, then K zero (D elements)
 *   V codes   D channel rows of 32*bits/8 bytes, one code per token slot
 *             (V is grouped per token over 32 channels); slot 8g + j holds
 *             token 4g + j (j < 4) or 16 + 4g + j - 4 (j >= 4)
 *   V scale   D/32 groups x 32 token slots (group-major), then V zero (same)
 * Code positions within a row: 4- and 8-bit codes, element e at bit
 * e*bits; 2-bit codes, each 16-bit word holds 8 elements, the even ones (2j)
 * at bits 2j of its low byte and the odd ones (2j+1) at bits 8+2j of its
 * high byte.  bits is 2, 4 or 8 (the decode kernel reads 2-bit blocks).
 * D=128, bits=2: 3072 bytes per block (5.33x smaller than fp16 K+V).
 * The reference keeps unpacked int8 codes plus separate scale/zero tensors
 * (baselines/kivi_cache.py:50-69, :121-195); this layout is this library's.
 */
size_t halo_kivi_block_bytes(int D, int bits);

/*
 * Quantise K and V (B, H_kv, T, D) of `dtype` (fp16 or bf16; element strides)
 * into blocks[b*blk_stride_b + h*blk_stride_h + j*block_bytes] (byte
 * strides), T % 32 == 0.  Per group: scale = dtype(dtype(max(dtype(x_max -
 * x_min), dtype(1e-8))) / qmax), zero = x_min, code = clamp(rint(dtype(
 * dtype(x - zero) / scale)), 0, qmax) with NaN -> 0.  Replaces
 * _quantize_per_group (baselines/kivi_cache.py:44-69).
 */
int halo_kivi_quantize(const void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
                       const void* v, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_t,
                       int dtype, int B, int H_kv, int T, int D, int bits,
                       void* blocks, int64_t blk_stride_b, int64_t blk_stride_h, void* stream);

/*
 * Dequantise n_blocks blocks per (b, h_kv) into K and V of `dtype`:
 * x = dtype(fp32(fp32(code) * fp32(scale)) + fp32(zero)), bit-exact with
 * _dequantize_per_group (baselines/kivi_cache.py:72-78).
 */
int halo_kivi_dequantize(const void* blocks, int64_t blk_stride_b, int64_t blk_stride_h,
                         int dtype, int B, int H_kv, int n_blocks, int D, int bits,
                         void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
                         void* v, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_t,
                         void* stream);

/*
 * halo_decode_attn over a table of KIVI chunks (flags HALO_CHUNK_KIVI2, 2-bit
 * blocks of halo_kivi_quantize, scales in `dtype`, which must be fp16 or
 * bf16): every block is dequantised in registers with the arithmetic of
 * halo_kivi_dequantize, so scores and outputs see exactly the dequantised
 * cache.  Same arguments and accumulator contract as halo_decode_attn; a
 * layer whose recent rows are unquantised runs this call with acc_mode 2 and
 * a halo_decode_attn over the recent rows with acc_mode 1.  Work items must
 * start on 32-token block boundaries.  Replaces the dequantise-and-concat of
 * KIVICache.update (baselines/kivi_cache.py:187-195) followed by attention.
 */
int halo_decode_attn_kivi(const void* q, int64_t q_stride_b, int64_t q_stride_h, int dtype,
                          int B, int H, int H_kv, int D, int rep_t,
                          const halo_chunk_desc* descs, int n_desc,
                          const int32_t* work, int n_work,
                          const int32_t* group_offsets, int n_groups,
                          const int64_t* q_pos, float scale,
                          float* m, float* l, float* o, int64_t acc_stride_b, int acc_mode,
                          void* out, int out_dtype, float* lse,
                          void* workspace, size_t workspace_bytes, void* stream);

/* ---- tier block moves -------------------------------------------------- */

/*
 * Copy whole blocks between two tier buffers of the cold-KV store: for each
 * i < n_blocks with b = blocks[i] in [0, max_blocks) (and, when tier_of is
 * non-NULL, tier_of[b] == src_tier), bytes [b*block_bytes, (b+1)*block_bytes)
 * of src_k go to dst_k, and likewise src_v -> dst_v when both are non-NULL.
 * Other entries are skipped, so a device-computed candidate list needs no
 * host-side filtering.  Pointers are device-visible addresses (pinned host
 * memory through halo_host_device_pointer is read or written in place);
 * 16-byte aligned, block_bytes % 16 == 0.  One launch on `stream`.
 * Replaces the per-block TieredStorage.move_block calls of HALORefetcher._issue
 * and HALODemoter.flush (halo/memory_tier.py:150-157, halo/refetcher.py:
 * 102-114, halo/demoter.py:49-77).
 */
int halo_copy_blocks(void* dst_k, const void* src_k, void* dst_v, const void* src_v,
                     int64_t block_bytes, const int32_t* blocks, int n_blocks, int64_t max_blocks,
                     const int8_t* tier_of, int src_tier, void* stream);

/*
 * Directory update after a move: for each i < n_blocks with b = blocks[i] in
 * [0, max_blocks) and (src_tier < 0 or tier_of[b] == src_tier), set
 * tier_of[b] = dst_tier.  Only the listed entries are written (duplicates
 * write the same value), so moves of other blocks of the same layer enqueued
 * on other streams are never undone.  One launch on `stream`; enqueue it
 * after the halo_copy_blocks it records.  Replaces the directory write of
 * TieredStorage.move_block (halo/memory_tier.py:150-157).
 */
int halo_set_tier(int8_t* tier_of, const int32_t* blocks, int n_blocks, int64_t max_blocks, int src_tier,
                  int dst_tier, void* stream);

/* ---- HBM staging of cold chunks ---------------------------------------- */

/* One host-to-device chunk copy of the staging cache: bytes from src_k to
 * dst_k and, when dst_v is non-NULL, from src_v to dst_v. */
typedef struct halo_fill {
  void* dst_k;
  const void* src_k;
  void* dst_v;
  const void* src_v;
  int64_t bytes;
} halo_fill;

/*
 * Enqueue n fills as hipMemcpyAsync host-to-device copies on `stream`
 * (sources pinned host memory), in list order.  Replaces the per-block
 * move_block calls of HALORefetcher._issue (halo/refetcher.py:102-114) for
 * the staging cache of halo_select_cfg.residency.
 */
int halo_stage_fills(const halo_fill* fills, int n, void* stream);

/*
 * The same fills as copy kernels on `stream` (one launch per 16 fills) that
 * read the sources in place over the host link: src_k / src_v must be
 * device-visible addresses of pinned host memory (halo_host_device_pointer);
 * all addresses 16-byte aligned, bytes % 16 == 0.  Kernel reads of pinned
 * memory sustain a higher host-link rate than hipMemcpyAsync of 2-4 MiB
 * pieces.  Replaces move_block's copies in HALORefetcher._issue
 * (halo/refetcher.py:102-114) for the staging cache.
 */
int halo_stage_fills_read(const halo_fill* fills, int n, void* stream);

/*
 * base[idx[i]] = vals[i] for i < n (entries with idx outside [0, n_elems)
 * are skipped), as kernels on `stream` whose pairs travel in the kernel
 * arguments: the host arrays are read during the call only.  For a policy of
 * the caller's own that commits and releases residency entries on the
 * compute stream (the halo_staging runtime does the same inside its
 * segment-boundary kernel).  No counterpart in
 * the reference (whose tier directory is a host dict,
 * halo/memory_tier.py:133).
 */
int halo_store_i32(int32_t* base, int64_t n_elems, const int64_t* idx, const int32_t* vals, int n, void* stream);

/* ---- HBM staging cache: host runtime ------------------------------------ */

/*
 * Description of a staging cache over n_layers decode layers whose fused
 * selections (halo_select_cfg) already point at `residency`, the slot
 * catalogs and `feedback`.  The cache's unit is one selection:
 * sels_per_layer = 1 for a layer with one selection, B for a layer with
 * per-row selection (per_row = 1: each batch row selects among its own cold
 * chunks, with its own n_slots slots); unit u = layer * sels_per_layer + row.
 * All arrays are copied at creation.
 *   residency:   device int32[U * n_cold + n_layers] (U = n_layers *
 *                sels_per_layer): the residency entries of each unit (slot or
 *                -1; n_cold = the selection's catalog_stride) then each
 *                layer's write-allocate slot;
 *   feedback:    device fp32, per layer sels_per_layer * (n_cold + 2 * top_k)
 *                words: scores (sels, n_cold) | picks (sels, top_k) int32 |
 *                residency used (sels, top_k) int32, as the selection writes
 *                them (score_out, idx_out, res_out);
 *   slot_addr:   (U, n_slots, 2) device addresses of each slot's K, V;
 *   chunk_addr:  (U, n_cold, 2) addresses of each cold chunk's K, V:
 *                host pointers of pinned memory (fill_mode 0, hipMemcpyAsync)
 *                or device-visible ones (fill_mode 1, copy kernels); a chunk
 *                whose V follows its K, staged into a slot laid out the same
 *                way, is filled by one copy;
 *   chunk_nbytes:(U, n_cold) bytes of one chunk's K (= its V);
 *   n_cold_per_unit: (U) cold chunks of each unit (NULL: n_cold each);
 *   copy_stream / urgent_stream: where fills run (urgent: fills the next
 *                launch of their layer waits for; NULL = copy_stream);
 *   copy_stream2: NULL, or a second stream for the other fills: copies then
 *                alternate between copy_stream and copy_stream2, so two DMA
 *                engines overlap each copy's start-up (4 MiB host-to-device
 *                pieces with an event after each: 56 GB/s over two streams
 *                against 46 GB/s on one); fills then land sooner but leave
 *                less of the link to chunks read in place.  Fill mode 1
 *                (copy kernels) keeps to copy_stream.
 * keep in [top_k, n_slots] best-scoring chunks per unit are staged; at most
 * max_inflight fills in flight; `spare` slots per unit kept free;
 * `ring` feedback entries in flight (>= segments per step + 1);
 * write_allocate needs sels_per_layer == 1; track_busy counts operations
 * issued while the compute stream still had work queued (a test aid; costs
 * one stream query each).
 */
typedef struct halo_staging_desc {
  int32_t n_layers, n_cold, n_slots, top_k, keep, max_inflight, spare, ring;
  int32_t write_allocate, fill_mode, track_busy, sels_per_layer;
  int32_t* residency;
  const float* feedback;
  const uint64_t* slot_addr;
  const uint64_t* chunk_addr;
  const int64_t* chunk_nbytes;
  const int32_t* n_cold_per_unit;
  void* copy_stream;
  void* urgent_stream;
  void* copy_stream2;
} halo_staging_desc;

/* Counters of a staging cache; ns_* are host nanoseconds spent planning
 * (including fill issue), issuing fills, and waiting for feedback. */
typedef struct halo_staging_stats {
  int64_t hits, misses, misses_predicted, fills, fill_bytes, miss_bytes, wa_commits, wa_dups;
  int64_t fills_while_busy, commits_while_busy, evictions_while_busy;
  int64_t ns_plan, ns_issue, ns_wait;
} halo_staging_stats;

typedef struct halo_staging halo_staging;

/*
 * The cache's host side, one call per segment of layers [lo, hi) run as
 * one graph (or launches) on the compute `stream`:
 *   halo_staging_before  -- commit the landed (and, after a compute-stream
 *                           wait, the urgent) fills of the segment's layers
 *                           and name their write-allocate slots; call before
 *                           the segment's launches;
 *   halo_staging_after   -- mark the segment's feedback rows for the host;
 *                           call after.  One small kernel per segment does
 *                           both: the next halo_staging_before on the same
 *                           stream stores the residency entries and writes
 *                           the marked rows into a pinned ring entry, then
 *                           its sequence word, which the host polls;
 *   halo_staging_service -- process returned feedback (waiting for all but
 *                           the `lag` newest segments, taking those too when
 *                           done): count hits and misses, evict, and issue
 *                           the fills of the best-ranked missing chunks.
 * The reference's HALORefetcher.predict_hot / schedule / _issue / wait
 * (halo/refetcher.py:38-114) with the scores written by the selection.
 * Calls on one cache are not thread-safe.  halo_staging_reset waits for the
 * cache's copies and forgets every slot (the caller clears `residency`);
 * halo_staging_set changes max_inflight and can zero the counters;
 * halo_staging_get copies the counters and the host mirror: slot state
 * (U, n_slots) int8 (0 free, 1 filling, 2 ready, 4 reserved), the chunk
 * each slot holds (int64, -1 none) and the write-allocate slots
 * (n_layers, 2) int64; any output may be NULL.
 */
int halo_staging_create(const halo_staging_desc* desc, halo_staging** out);
int halo_staging_destroy(halo_staging* cache);
int halo_staging_before(halo_staging* cache, int lo, int hi, void* stream);
int halo_staging_after(halo_staging* cache, int lo, int hi, void* stream);
int halo_staging_service(halo_staging* cache, int lag, void* stream);
int halo_staging_reset(halo_staging* cache);
int halo_staging_set(halo_staging* cache, int max_inflight, int reset_counters);
int halo_staging_get(const halo_staging* cache, halo_staging_stats* stats, int8_t* state, int64_t* holds,
                     int64_t* wa_slot);

/* ---- build metadata ---------------------------------------------------- */
/*
 * Device-visible address of pinned host memory (allocated by hipHostMalloc,
 * e.g. a pinned torch tensor), written to *dev.  A chunk descriptor holding
 * that address makes the decode kernels read the chunk in place from host
 * DRAM over the host link: the refetch of selected cold chunks then happens
 * inside the attention launch with no host round trip.  Replaces the
 * DRAM -> GPU block moves of the pinned cold tier (halo/memory_tier.py:
 * 150-157, 197-205; halo/triton_chunked.py:325-350).  HALO_E_INVALID when
 * `host` is not pinned host memory.
 */
int halo_host_device_pointer(const void* host, void** dev);

const char* halo_last_error(void);
const char* halo_build_info(void);

#ifdef __cplusplus
}
#endif

#endif /* HALO_HIP_H */
