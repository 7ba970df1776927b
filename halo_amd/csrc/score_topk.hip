// Chunk-relevance scoring: page-mean keys, q.Kbar scores and a
// deterministic top-k that writes the selected chunks into a device chunk
// table (gfx950, wave64).  All of it is HBM/L2-bound reduction work; none of
// it is shaped into a GEMM.
//
// Reference semantics:
//   page means        baselines/scorer_ablations.py:209-216
//   GQA mean query    baselines/scorer_ablations.py:223-232 (kept in q dtype)
//   score             baselines/scorer_ablations.py:233-237 (max over rows, heads)
//   top-k             baselines/scorer_ablations.py:265-266 with the build's
//                     tie rule (score desc, chunk index asc), indices sorted
//   budget            baselines/scorer_ablations.py:133-139 (host side)

#include "common.hpp"

namespace halo {

// ---------------------------------------------------------------------------
// Page means: kmean[b,h,j,d] = dtype(sum_t K[b,h,row0+j*page+t,d] / page).
// One workgroup per (b, h, page).  Thread t owns the 16-byte piece
// t % SL of rows t/SL, t/SL + RG, ... (RG = 256/SL row groups), so loads are
// whole coalesced rows and independent; the RG fp32 partial sums are then
// added in row-group order through LDS and rounded once to the key dtype.
// ---------------------------------------------------------------------------
template <int DT>
__global__ void __launch_bounds__(256) chunk_means_kernel(const void* k, int64_t ksb, int64_t ksh, int64_t kst,
                                                          int H_kv, int D, int64_t row0, int page, int n_pages,
                                                          void* km, int64_t msb, int64_t msh, int64_t msp) {
  constexpr int ESZ = DT == HALO_F32 ? 4 : 2;
  constexpr int EPC = 16 / ESZ;
  __shared__ float s_part[256 * 8];
  const int j = blockIdx.x % n_pages;
  const int bh = blockIdx.x / n_pages;
  const int h = bh % H_kv, b = bh / H_kv;
  const int SL = D / EPC;
  const int RG = 256 / SL;
  const int tid = threadIdx.x;
  const int col = tid % SL, rg = tid / SL;
  float acc[EPC];
#pragma unroll
  for (int e = 0; e < EPC; ++e) acc[e] = 0.f;
  if (rg < RG) {
    const char* base = reinterpret_cast<const char*>(k) +
                       ((int64_t)b * ksb + (int64_t)h * ksh + (row0 + (int64_t)j * page) * kst) * ESZ + col * 16;
#pragma unroll 8
    for (int t = rg; t < page; t += RG) {
      const uint4 v = *reinterpret_cast<const uint4*>(base + (int64_t)t * kst * ESZ);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
      if constexpr (DT == HALO_F32) {
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] += __uint_as_float(w[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float lo, hi;
          if constexpr (DT == HALO_BF16) {
            lo = bf16_lo(w[e]);
            hi = bf16_hi(w[e]);
          } else {
            lo = f16_bits_to_f32((uint16_t)(w[e] & 0xffffu));
            hi = f16_bits_to_f32((uint16_t)(w[e] >> 16));
          }
          acc[2 * e] += lo;
          acc[2 * e + 1] += hi;
        }
      }
    }
  }
#pragma unroll
  for (int e = 0; e < EPC; ++e) s_part[tid * 8 + e] = acc[e];
  __syncthreads();
  const float inv = 1.0f / (float)page;
  for (int d = tid; d < D; d += 256) {
    const int c = d / EPC, e = d % EPC;
    float sum = 0.f;
    for (int g = 0; g < RG; ++g) sum += s_part[(g * SL + c) * 8 + e];
    store_elem(km, (int64_t)b * msb + (int64_t)h * msh + (int64_t)j * msp + d, DT, sum * inv);
  }
}

// ---------------------------------------------------------------------------
// Score + top-k.  One workgroup per selection.  Selection s covers batch row
// s (per_row) or every row (per_row == 0, the reference's amax over batch).
// ---------------------------------------------------------------------------
struct ScoreParams {
  const void* q;
  int64_t qsb, qsh;
  int dtype;
  int B, H, H_kv, D, rep;
  float inv_rep;  // fp32(1/rep), rounded on the host: torch's mean factor
  const void* km;
  int64_t msb, msh, msp;
  const int32_t* elig;
  int64_t elig_stride;
  const int32_t* n_elig_per_sel;
  int n_elig;
  int k;
  int per_row;
  int32_t* idx_out;
  float* score_out;
  const halo_chunk_desc* catalog;
  int64_t catalog_stride;
  halo_chunk_desc* table;
  int64_t table_stride;
  int table_slot0;
  // page score = alpha*minmax(attn) + beta*recency + gamma*sink when
  // normalize != 0 (baselines/scorer_ablations.py:238-263); raw attn otherwise.
  int normalize;
  float alpha, beta, gamma;
  int refresh, sink_pages, P_total;
  // HBM staging (residency == NULL: off): a chosen chunk whose residency
  // entry names a slot is written to the table with that slot's addresses
  // and strides; res_out[sel * k + j] gets the entry used (-1: in place).
  const int32_t* residency;
  const halo_chunk_desc* slot_catalog;
  int n_slots;
  int32_t* res_out;
};

constexpr int kMaxElig = 1024;
constexpr int kMaxQg = 8192;    // floats of GQA-mean query rows held in LDS
constexpr int kMaxDots = 4096;  // (page, row, head) dot products per batch

// a ranks before b: larger score, then lower chunk index (NaN scores are
// stored as -inf before ranking).
__device__ __forceinline__ bool beats(float sa, int ea, float sb, int eb) {
  return sa > sb || (sa == sb && ea < eb);
}

// DC: the head dim when known at compile time (64, 128, 256: the dot-product
// loops unroll and every load of a triple is issued before the first use),
// 0 for any other multiple of 16 (runtime loops).
template <int DT, int DC>
__global__ void __launch_bounds__(512) score_topk_kernel(ScoreParams P) {
  __shared__ float s_qg[kMaxQg];
  __shared__ __align__(16) float s_score[kMaxElig];
  __shared__ __align__(16) int s_chunk[kMaxElig];
  __shared__ __align__(16) int s_sel[kMaxElig];
  __shared__ float s_dot[kMaxDots];
  const int sel = blockIdx.x;
  const int tid = threadIdx.x;
  const int nthr = blockDim.x;
  const int b0 = P.per_row ? sel : 0;
  const int nrows = P.per_row ? 1 : P.B;
  const int n = P.n_elig_per_sel ? min(P.n_elig_per_sel[sel], P.n_elig) : P.n_elig;
  const int kk = min(P.k, n);
  const int32_t* elig = P.elig + (int64_t)sel * P.elig_stride;

  // GQA mean of the query heads of each KV head, rounded to the q dtype
  // (torch's .mean keeps the dtype); rep == 1 uses q as is.
  const int Dq = DC ? DC : P.D;
  const int QG = nrows * P.H_kv * Dq;
  for (int i = tid; i < QG; i += nthr) {
    const int d = i % Dq;
    const int h = (i / Dq) % P.H_kv;
    const int r = i / (Dq * P.H_kv);
    const int64_t qb = (int64_t)(b0 + r) * P.qsb;
    float v;
    if (P.rep == 1) {
      v = load_elem(P.q, qb + (int64_t)h * P.qsh + d, DT);
    } else {
      // the rep loads are independent: issue them in batches of 4, then add in head order
      float acc = 0.f;
      for (int j0 = 0; j0 < P.rep; j0 += 4) {
        float x[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          x[j] = j0 + j < P.rep ? load_elem(P.q, qb + (int64_t)(h * P.rep + j0 + j) * P.qsh + d, DT) : 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (j0 + j < P.rep) acc += x[j];
      }
      acc = opaque(acc * P.inv_rep);  // fp32 product, then one rounding to the q dtype
      v = DT == HALO_F32 ? acc
          : (DT == HALO_BF16 ? __uint_as_float((uint32_t)f32_to_bf16_rne(acc) << 16)
                             : f16_bits_to_f32(f32_to_f16_rne(acc)));
    }
    s_qg[i] = v;
  }
  for (int i = tid; i < n; i += nthr) s_chunk[i] = elig[i];
  __syncthreads();

  // score[i] = max over (row, h) of sum_d qg * kbar.  One thread per
  // (page, row, head) triple computes the whole dot product from 16-byte
  // loads that are all independent (one memory round trip per batch of
  // triples), products and sums rounded separately (no fused multiply-add),
  // summed in the scorer's slice order (below); the max over (row, h) is
  // folded in order.
  const int nrh = nrows * P.H_kv;
  const int triples = n * nrh;
  constexpr int esz = DT == HALO_F32 ? 4 : 2;
  constexpr int ep = 16 / esz;
  for (int i = tid; i < n; i += nthr) s_score[i] = -INFINITY;
  for (int t0 = 0; t0 < triples; t0 += kMaxDots) {
    const int nt = min(kMaxDots, triples - t0);
    for (int t = tid; t < nt; t += nthr) {
      const int tt = t0 + t;
      const int i = tt / nrh, rh = tt % nrh;
      const int r = rh / P.H_kv, h = rh % P.H_kv;
      const int64_t mb = (int64_t)(b0 + r) * P.msb + (int64_t)h * P.msh + (int64_t)s_chunk[i] * P.msp;
      const char* row = reinterpret_cast<const char*>(P.km) + mb * esz;
      const float* qg = s_qg + (r * P.H_kv + h) * Dq;
      // D is cut into G = D/16 slices; slice c holds elements
      // ep*(c + p*G) + e (p < 16/ep, e < ep), summed in (p, e) order; the G
      // slice sums are added as a balanced pairwise tree in slice order.  This
      // is the order of the fused selection in decode_attn.hip, whose slices
      // sit in G lanes and meet in an xor butterfly.
      constexpr int GC = DC / 16;  // compile-time slice count (0: runtime)
      const int G = DC ? GC : P.D / 16;
      float part[16];
      // compile-time D: every piece of the row is loaded before the first use
      uint4 rowv[DC ? (DC / 16) * (16 / ep) : 1];
      if constexpr (DC != 0) {
#pragma unroll
        for (int x = 0; x < GC * (16 / ep); ++x) rowv[x] = *reinterpret_cast<const uint4*>(row + x * 16);
      }
#pragma unroll
      for (int c = 0; c < (DC ? GC : 16); ++c) {
        if (!DC && c >= G) break;
        float a = 0.f;
#pragma unroll
        for (int p = 0; p < 16 / ep; ++p) {
          const uint4 v = DC ? rowv[(c + p * G) % (DC ? GC * (16 / ep) : 1)]
                             : *reinterpret_cast<const uint4*>(row + (c + p * G) * 16);
          float f[8];
          if constexpr (DT == HALO_F32) {
            f[0] = __uint_as_float(v.x); f[1] = __uint_as_float(v.y);
            f[2] = __uint_as_float(v.z); f[3] = __uint_as_float(v.w);
          } else if constexpr (DT == HALO_BF16) {
            f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x); f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
            f[4] = bf16_lo(v.z); f[5] = bf16_hi(v.z); f[6] = bf16_lo(v.w); f[7] = bf16_hi(v.w);
          } else {
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              f[2 * e] = f16_bits_to_f32((uint16_t)(w[e] & 0xffffu));
              f[2 * e + 1] = f16_bits_to_f32((uint16_t)(w[e] >> 16));
            }
          }
#pragma unroll
          for (int e = 0; e < ep; ++e) a = __fadd_rn(a, __fmul_rn(qg[ep * (c + p * G) + e], f[e]));
        }
        part[c] = a;
      }
      for (int w = 1; w < G; w <<= 1)
        for (int c = 0; c + w < G; c += 2 * w) part[c] = __fadd_rn(part[c], part[c + w]);
      const float acc = part[0];
      s_dot[t] = acc;
    }
    __syncthreads();
    for (int i = tid; i < n; i += nthr) {
      const int lo = max(i * nrh, t0) - t0, hi = min((i + 1) * nrh, t0 + nt) - t0;
      float best = s_score[i];
      for (int t = lo; t < hi; ++t) best = fmaxf(best, s_dot[t]);
      s_score[i] = best;
    }
    __syncthreads();
  }
  for (int i = tid; i < n; i += nthr) s_score[i] = (s_score[i] != s_score[i]) ? -INFINITY : s_score[i];
  __syncthreads();

  if (P.normalize) {
    __shared__ float s_red[512];
    // min over eligible pages, then max of (attn - min)
    float mn = INFINITY;
    for (int i = tid; i < n; i += nthr) mn = fminf(mn, s_score[i]);
    s_red[tid] = mn;
    __syncthreads();
    for (int w = nthr / 2; w > 0; w >>= 1) {
      if (tid < w) s_red[tid] = fminf(s_red[tid], s_red[tid + w]);
      __syncthreads();
    }
    mn = s_red[0];
    __syncthreads();
    float mx = -INFINITY;
    for (int i = tid; i < n; i += nthr) mx = fmaxf(mx, s_score[i] - mn);
    s_red[tid] = mx;
    __syncthreads();
    for (int w = nthr / 2; w > 0; w >>= 1) {
      if (tid < w) s_red[tid] = fmaxf(s_red[tid], s_red[tid + w]);
      __syncthreads();
    }
    mx = s_red[0];
    __syncthreads();
    // recency over all P_total pages: exp(-(P-1-p)/refresh), / (sum + 1e-12), / (max + 1e-12)
    const float dec = (float)max(P.refresh, 1);
    float rs = 0.f;
    for (int j = tid; j < P.P_total; j += nthr) rs += expf(-((float)(P.P_total - 1) - (float)j) / dec);
    s_red[tid] = rs;
    __syncthreads();
    for (int w = nthr / 2; w > 0; w >>= 1) {
      if (tid < w) s_red[tid] += s_red[tid + w];
      __syncthreads();
    }
    const float rsum = s_red[0] + 1e-12f;
    // the largest recency term is the last page's exp(0) = 1
    const float rmax = 1.0f / rsum + 1e-12f;
    for (int i = tid; i < n; i += nthr) {
      float a = s_score[i] - mn;
      if (mx > 0.f) a = a / mx;
      const int pg = s_chunk[i];
      const float rec = (expf(-((float)(P.P_total - 1) - (float)pg) / dec) / rsum) / rmax;
      const float sink = pg < P.sink_pages ? 1.f : 0.f;
      float v = __fadd_rn(__fadd_rn(__fmul_rn(P.alpha, a), __fmul_rn(P.beta, rec)), __fmul_rn(P.gamma, sink));
      s_score[i] = (v != v) ? -INFINITY : v;
    }
    __syncthreads();
  }

  // Rank by (score desc, chunk asc); selected = rank < kk.  Candidates are
  // read four at a time (16-byte LDS reads, several in flight); entries past
  // n are padding that never outranks (-inf, index past every chunk).
  for (int i = n + tid; i < ((n + 15) & ~15); i += nthr) {
    s_score[i] = -INFINITY;
    s_chunk[i] = 0x7fffffff;
    s_sel[i] = 0;
  }
  __syncthreads();
  const int n16 = (n + 15) & ~15;
  for (int i = tid; i < n; i += nthr) {
    const float si = s_score[i];
    const int ei = s_chunk[i];
    int rank = 0;
    for (int j = 0; j < n16; j += 16) {
      float4 sv[4];
      int4 ev[4];
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        sv[x] = *reinterpret_cast<const float4*>(&s_score[j + 4 * x]);
        ev[x] = *reinterpret_cast<const int4*>(&s_chunk[j + 4 * x]);
      }
#pragma unroll
      for (int x = 0; x < 4; ++x)
        rank += (beats(sv[x].x, ev[x].x, si, ei) ? 1 : 0) + (beats(sv[x].y, ev[x].y, si, ei) ? 1 : 0) +
                (beats(sv[x].z, ev[x].z, si, ei) ? 1 : 0) + (beats(sv[x].w, ev[x].w, si, ei) ? 1 : 0);
    }
    s_sel[i] = rank < kk;
  }
  __syncthreads();
  // Output slot = number of selected chunks with a smaller index (ascending).
  for (int i = tid; i < n; i += nthr) {
    if (P.score_out) P.score_out[(int64_t)sel * P.n_elig + i] = s_score[i];
    if (!s_sel[i]) continue;
    const int ei = s_chunk[i];
    int pos = 0;
    for (int j = 0; j < n16; j += 16) {
      int4 sv[4], ev[4];
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        sv[x] = *reinterpret_cast<const int4*>(&s_sel[j + 4 * x]);
        ev[x] = *reinterpret_cast<const int4*>(&s_chunk[j + 4 * x]);
      }
#pragma unroll
      for (int x = 0; x < 4; ++x)
        pos += (sv[x].x && ev[x].x < ei) + (sv[x].y && ev[x].y < ei) + (sv[x].z && ev[x].z < ei) +
               (sv[x].w && ev[x].w < ei);
    }
    if (P.idx_out) P.idx_out[(int64_t)sel * P.k + pos] = ei;
    int rs = -1;
    if (P.residency != nullptr) {
      const int r = P.residency[(int64_t)sel * P.catalog_stride + ei];
      rs = (r >= 0 && r < P.n_slots) ? r : -1;
    }
    if (P.res_out) P.res_out[(int64_t)sel * P.k + pos] = rs;
    if (P.table) {
      halo_chunk_desc d = P.catalog[(int64_t)sel * P.catalog_stride + ei];
      if (rs >= 0) {  // rows, start, flags and batch stay the chunk's own
        const halo_chunk_desc& sd = P.slot_catalog[(int64_t)sel * P.n_slots + rs];
        d.k = sd.k;
        d.v = sd.v;
        d.k_stride_b = sd.k_stride_b;
        d.k_stride_h = sd.k_stride_h;
        d.k_stride_t = sd.k_stride_t;
        d.v_stride_b = sd.v_stride_b;
        d.v_stride_h = sd.v_stride_h;
        d.v_stride_t = sd.v_stride_t;
      }
      P.table[(int64_t)sel * P.table_stride + P.table_slot0 + pos] = d;
    }
  }
  // Unfilled slots: index -1 and an empty descriptor (T_c = 0, never read).
  for (int j = kk + tid; j < P.k; j += nthr) {
    if (P.idx_out) P.idx_out[(int64_t)sel * P.k + j] = -1;
    if (P.res_out) P.res_out[(int64_t)sel * P.k + j] = -1;
    if (P.table) {
      halo_chunk_desc e = {};
      e.k = nullptr;
      e.v = nullptr;
      e.T_c = 0;
      e.batch = P.per_row ? sel : -1;
      P.table[(int64_t)sel * P.table_stride + P.table_slot0 + j] = e;
    }
  }
}

}  // namespace halo

using namespace halo;

extern "C" int halo_chunk_means(const void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
                                int dtype, int B, int H_kv, int D, int64_t row0, int page, int n_pages,
                                void* kmean, int64_t km_stride_b, int64_t km_stride_h, int64_t km_stride_p,
                                void* stream) {
  HALO_CHECK_ARG(k && kmean, "null pointer");
  HALO_CHECK_ARG(dtype == HALO_F32 || dtype == HALO_BF16 || dtype == HALO_F16, "bad dtype");
  HALO_CHECK_ARG(B > 0 && H_kv > 0 && D > 0 && page > 0 && n_pages >= 0 && row0 >= 0, "bad sizes");
  if (n_pages == 0) return HALO_OK;
  HALO_CHECK_ARG(D % (dtype == HALO_F32 ? 4 : 8) == 0 && D <= 256 * (dtype == HALO_F32 ? 4 : 8),
                 "head dim must fill whole 16-byte pieces");
  HALO_CHECK_ARG(reinterpret_cast<uintptr_t>(k) % 16 == 0 && (k_stride_t * elem_size(dtype)) % 16 == 0 &&
                 (k_stride_h * elem_size(dtype)) % 16 == 0 && (k_stride_b * elem_size(dtype)) % 16 == 0,
                 "key rows must be 16-byte aligned");
  const int64_t blocks = (int64_t)B * H_kv * n_pages;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define HALO_MEANS(DTV)                                                                                  \
  hipLaunchKernelGGL(chunk_means_kernel<DTV>, dim3((unsigned)blocks), dim3(256), 0, st, k, k_stride_b,   \
                     k_stride_h, k_stride_t, H_kv, D, row0, page, n_pages, kmean, km_stride_b, km_stride_h, \
                     km_stride_p)
  if (dtype == HALO_F32) HALO_MEANS(HALO_F32);
  else if (dtype == HALO_BF16) HALO_MEANS(HALO_BF16);
  else HALO_MEANS(HALO_F16);
#undef HALO_MEANS
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}

static int score_topk_impl(const void* q, int64_t q_stride_b, int64_t q_stride_h, int dtype,
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
                                     const int32_t* residency, const halo_chunk_desc* slot_catalog, int n_slots,
                                     int32_t* res_out, void* stream) {
  HALO_CHECK_ARG(q && kmean && eligible, "null pointer");
  HALO_CHECK_ARG(residency == nullptr || (slot_catalog != nullptr && n_slots >= 1 && table != nullptr),
                 "staging needs slot_catalog, n_slots >= 1 and a table");
  HALO_CHECK_ARG(dtype == HALO_F32 || dtype == HALO_BF16 || dtype == HALO_F16, "bad dtype");
  HALO_CHECK_ARG(B > 0 && H > 0 && H_kv > 0 && H % H_kv == 0 && D > 0, "bad head sizes");
  HALO_CHECK_ARG(n_elig >= 0 && n_elig <= kMaxElig, "n_elig must be in [0, 1024]");
  HALO_CHECK_ARG(D % 16 == 0 && D <= 256, "head dim must be a multiple of 16, at most 256");
  HALO_CHECK_ARG(reinterpret_cast<uintptr_t>(kmean) % 16 == 0 &&
                 (km_stride_p * (dtype == HALO_F32 ? 4 : 2)) % 16 == 0 &&
                 (km_stride_h * (dtype == HALO_F32 ? 4 : 2)) % 16 == 0 &&
                 (km_stride_b * (dtype == HALO_F32 ? 4 : 2)) % 16 == 0,
                 "kmean rows must be 16-byte aligned");
  HALO_CHECK_ARG(k >= 0, "k must be >= 0");
  HALO_CHECK_ARG(table == nullptr || catalog != nullptr, "table needs a catalog");
  const int nrows = per_row ? 1 : B;
  HALO_CHECK_ARG((int64_t)nrows * H_kv * D <= kMaxQg, "B*H_kv*D too large for one selection");
  ScoreParams p;
  p.q = q;
  p.qsb = q_stride_b;
  p.qsh = q_stride_h;
  p.dtype = dtype;
  p.B = B;
  p.H = H;
  p.H_kv = H_kv;
  p.D = D;
  p.rep = H / H_kv;
  p.inv_rep = (float)(1.0 / (double)p.rep);
  p.km = kmean;
  p.msb = km_stride_b;
  p.msh = km_stride_h;
  p.msp = km_stride_p;
  p.elig = eligible;
  p.elig_stride = elig_stride;
  p.n_elig_per_sel = n_elig_per_sel;
  p.n_elig = n_elig;
  p.k = k;
  p.per_row = per_row;
  p.idx_out = idx_out;
  p.score_out = score_out;
  p.catalog = catalog;
  p.catalog_stride = catalog_stride;
  p.table = table;
  p.table_stride = table_stride;
  p.table_slot0 = table_slot0;
  p.normalize = normalize;
  p.alpha = alpha;
  p.beta = beta;
  p.gamma = gamma;
  p.refresh = refresh;
  p.sink_pages = sink_pages;
  p.P_total = P_total;
  p.residency = residency;
  p.slot_catalog = slot_catalog;
  p.n_slots = n_slots;
  p.res_out = res_out;
  HALO_CHECK_ARG(!normalize || P_total > 0, "P_total must be positive when normalising");
  const int n_sel = per_row ? B : 1;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define HALO_SCORE(DTV)                                                                                    \
  do {                                                                                                     \
    if (D == 64) hipLaunchKernelGGL((score_topk_kernel<DTV, 64>), dim3(n_sel), dim3(512), 0, st, p);       \
    else if (D == 128) hipLaunchKernelGGL((score_topk_kernel<DTV, 128>), dim3(n_sel), dim3(512), 0, st, p); \
    else if (D == 256) hipLaunchKernelGGL((score_topk_kernel<DTV, 256>), dim3(n_sel), dim3(512), 0, st, p); \
    else hipLaunchKernelGGL((score_topk_kernel<DTV, 0>), dim3(n_sel), dim3(512), 0, st, p);                \
  } while (0)
  if (dtype == HALO_F32) HALO_SCORE(HALO_F32);
  else if (dtype == HALO_BF16) HALO_SCORE(HALO_BF16);
  else HALO_SCORE(HALO_F16);
#undef HALO_SCORE
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}

extern "C" int halo_chunk_score_topk(const void* q, int64_t q_stride_b, int64_t q_stride_h, int dtype,
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
                                     void* stream) {
  return score_topk_impl(q, q_stride_b, q_stride_h, dtype, B, H, H_kv, D, kmean, km_stride_b, km_stride_h,
                         km_stride_p, eligible, elig_stride, n_elig_per_sel, n_elig, k, per_row, idx_out, score_out,
                         catalog, catalog_stride, table, table_stride, table_slot0, normalize, alpha, beta, gamma,
                         refresh, sink_pages, P_total, nullptr, nullptr, 0, nullptr, stream);
}

extern "C" int halo_chunk_score_topk_staged(const void* q, int64_t q_stride_b, int64_t q_stride_h, int dtype,
                                            int B, int H, int H_kv, int D,
                                            const void* kmean, int64_t km_stride_b, int64_t km_stride_h,
                                            int64_t km_stride_p,
                                            const int32_t* eligible, int64_t elig_stride,
                                            const int32_t* n_elig_per_sel, int n_elig, int k, int per_row,
                                            int32_t* idx_out, float* score_out,
                                            const halo_chunk_desc* catalog, int64_t catalog_stride,
                                            halo_chunk_desc* table, int64_t table_stride, int table_slot0,
                                            const int32_t* residency, const halo_chunk_desc* slot_catalog,
                                            int n_slots, int32_t* res_out, void* stream) {
  HALO_CHECK_ARG(residency != nullptr, "residency is NULL: use halo_chunk_score_topk");
  return score_topk_impl(q, q_stride_b, q_stride_h, dtype, B, H, H_kv, D, kmean, km_stride_b, km_stride_h,
                         km_stride_p, eligible, elig_stride, n_elig_per_sel, n_elig, k, per_row, idx_out, score_out,
                         catalog, catalog_stride, table, table_stride, table_slot0, 0, 1.f, 0.f, 0.f, 64, 0, 1,
                         residency, slot_catalog, n_slots, res_out, stream);
}
