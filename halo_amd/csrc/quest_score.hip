// Quest bounding-box page scoring (gfx950, wave64): per-page channel-wise
// key minima and maxima, Quest's per-page upper bound
// sum_d max(q_d * kmin_d, q_d * kmax_d) and a deterministic top-k.  All of
// it is HBM/L2-bound reduction work; none of it is shaped into a GEMM.
//
// Reference semantics:
//   page min / max   baselines/quest_path_d.py:125-150 (amin / amax over the
//                    page's rows, kept in the key dtype: exact)
//   GQA mean query   baselines/quest_path_d.py:166-172 (mean over the rep
//                    query heads, kept in the query dtype)
//   bound            baselines/quest_path_d.py:173-178 (fp32 products,
//                    elementwise maximum, sum over the channels)
//   page score       baselines/quest_path_d.py:196 (max over b, h_kv, t_q)
//   top-K            baselines/quest_path_d.py:197-203 (descending score
//                    order; ties by lower page index, NaN bounds rank as -inf)

#include "common.hpp"

namespace halo {

// torch.amin / amax / maximum propagate NaN; fminf / fmaxf would drop it.
__device__ __forceinline__ float nan_min(float a, float x) { return (x < a || x != x) ? x : a; }
__device__ __forceinline__ float nan_max(float a, float x) { return (x > a || x != x) ? x : a; }

// ---------------------------------------------------------------------------
// Page minima / maxima: one workgroup per (b, h, page).  Thread t owns the
// 16-byte piece t % SL of rows t/SL, t/SL + RG, ... (RG = 256/SL row groups),
// so the loads are whole coalesced rows; the RG partial results meet through
// LDS.  min / max are exact in any order, so the stored elements are the
// key elements themselves.
// ---------------------------------------------------------------------------
template <int DT>
__global__ void __launch_bounds__(256) page_minmax_kernel(const void* k, int64_t ksb, int64_t ksh, int64_t kst,
                                                          int H_kv, int D, int64_t row0, int page, int n_pages,
                                                          void* kmin, void* kmax, int64_t msb, int64_t msh,
                                                          int64_t msp) {
  constexpr int ESZ = DT == HALO_F32 ? 4 : 2;
  constexpr int EPC = 16 / ESZ;
  __shared__ float s_mn[256 * 8];
  __shared__ float s_mx[256 * 8];
  const int j = blockIdx.x % n_pages;
  const int bh = blockIdx.x / n_pages;
  const int h = bh % H_kv, b = bh / H_kv;
  const int SL = D / EPC;
  const int RG = 256 / SL;
  const int tid = threadIdx.x;
  const int col = tid % SL, rg = tid / SL;
  float mn[EPC], mx[EPC];
#pragma unroll
  for (int e = 0; e < EPC; ++e) {
    mn[e] = INFINITY;
    mx[e] = -INFINITY;
  }
  if (rg < RG) {
    const char* base = reinterpret_cast<const char*>(k) +
                       ((int64_t)b * ksb + (int64_t)h * ksh + (row0 + (int64_t)j * page) * kst) * ESZ + col * 16;
#pragma unroll 4
    for (int t = rg; t < page; t += RG) {
      const uint4 v = *reinterpret_cast<const uint4*>(base + (int64_t)t * kst * ESZ);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
      float f[EPC];
      if constexpr (DT == HALO_F32) {
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = __uint_as_float(w[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (DT == HALO_BF16) {
            f[2 * e] = bf16_lo(w[e]);
            f[2 * e + 1] = bf16_hi(w[e]);
          } else {
            f[2 * e] = f16_bits_to_f32((uint16_t)(w[e] & 0xffffu));
            f[2 * e + 1] = f16_bits_to_f32((uint16_t)(w[e] >> 16));
          }
        }
      }
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        mn[e] = nan_min(mn[e], f[e]);
        mx[e] = nan_max(mx[e], f[e]);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < EPC; ++e) {
    s_mn[tid * 8 + e] = mn[e];
    s_mx[tid * 8 + e] = mx[e];
  }
  __syncthreads();
  const int64_t o = (int64_t)b * msb + (int64_t)h * msh + (int64_t)j * msp;
  for (int d = tid; d < D; d += 256) {
    const int c = d / EPC, e = d % EPC;
    float a = INFINITY, z = -INFINITY;
    for (int g = 0; g < RG; ++g) {
      a = nan_min(a, s_mn[(g * SL + c) * 8 + e]);
      z = nan_max(z, s_mx[(g * SL + c) * 8 + e]);
    }
    // a stored element of the key dtype converts back exactly
    store_elem(kmin, o + d, DT, a);
    store_elem(kmax, o + d, DT, z);
  }
}

// ---------------------------------------------------------------------------
// Bound scores.  A selection covers batch row `sel` (per_row) or every row
// (the reference's max over the batch).  Its rows are the (b, h_kv, t_q)
// triples; a workgroup takes 4 rows (one per wave) x 64 pages (one per
// lane), computes the 256 bounds, folds the max over its 4 rows and merges
// it into the selection's page scores with an unsigned atomic max on an
// order-preserving encoding of the float (max is exact in any order, so the
// result does not depend on the order the workgroups run in).
// ---------------------------------------------------------------------------
struct QuestParams {
  const void* q;
  int64_t qsb, qsh, qst;
  int B, H, H_kv, T_q, D, rep;
  float inv_rep;  // fp32(1/rep): torch's mean factor
  const void* kmin;
  const void* kmax;
  int64_t msb, msh, msp;
  int P, per_row, rows_sel, row_tiles, page_tiles;
  float* dots;       // optional (B, H_kv, T_q, P) fp32
  uint32_t* keys;    // (n_sel, P) encoded page scores
};

constexpr int kQuestMaxD = 256;
constexpr int kQuestMaxPages = 8192;
constexpr uint32_t kKeyNegInf = 0x007fffffu;  // key(-inf)

// Larger float <=> larger key (NaN is never encoded: it is ranked as -inf).
__device__ __forceinline__ uint32_t float_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__global__ void __launch_bounds__(256) quest_init_kernel(uint32_t* keys, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) keys[i] = kKeyNegInf;
}

template <int DT>
__global__ void __launch_bounds__(256) quest_score_kernel(QuestParams P) {
  __shared__ float s_q[4][kQuestMaxD];
  __shared__ float s_best[4][64];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int pt = blockIdx.x % P.page_tiles;
  const int rt = (blockIdx.x / P.page_tiles) % P.row_tiles;
  const int sel = blockIdx.x / (P.page_tiles * P.row_tiles);
  const int r = rt * 4 + w;
  const bool row_ok = r < P.rows_sel;
  const int t = r % P.T_q;
  const int h = (r / P.T_q) % P.H_kv;
  const int b = P.per_row ? sel : r / (P.T_q * P.H_kv);
  // GQA mean of the row's query heads, rounded to the query dtype.
  if (row_ok) {
    const int64_t qb = (int64_t)b * P.qsb + (int64_t)t * P.qst;
    for (int d = lane; d < P.D; d += 64) {
      float v;
      if (P.rep == 1) {
        v = load_elem(P.q, qb + (int64_t)h * P.qsh + d, DT);
      } else {
        float acc = 0.f;
        for (int j = 0; j < P.rep; ++j) acc += load_elem(P.q, qb + (int64_t)(h * P.rep + j) * P.qsh + d, DT);
        acc = opaque(acc * P.inv_rep);
        v = DT == HALO_F32 ? acc
            : (DT == HALO_BF16 ? __uint_as_float((uint32_t)f32_to_bf16_rne(acc) << 16)
                               : f16_bits_to_f32(f32_to_f16_rne(acc)));
      }
      s_q[w][d] = v;
    }
  }
  wave_lds_fence();
  const int p = pt * 64 + lane;
  float best = -INFINITY;
  if (row_ok && p < P.P) {
    constexpr int esz = DT == HALO_F32 ? 4 : 2;
    constexpr int ep = 16 / esz;
    const int64_t mo = ((int64_t)b * P.msb + (int64_t)h * P.msh + (int64_t)p * P.msp) * esz;
    const char* rmn = reinterpret_cast<const char*>(P.kmin) + mo;
    const char* rmx = reinterpret_cast<const char*>(P.kmax) + mo;
    const float* qg = s_q[w];
    // D is cut into G = D/16 slices; slice c holds elements ep*(c + pp*G) + e
    // (pp < 16/ep, e < ep), summed in (pp, e) order, products and sums rounded
    // separately; the G slice sums are added as a balanced pairwise tree.
    const int G = P.D / 16;
    float part[16];
    for (int c = 0; c < G; ++c) {
      float a = 0.f;
      for (int pp = 0; pp < 16 / ep; ++pp) {
        const int off = (c + pp * G) * 16;
        const uint4 vn = *reinterpret_cast<const uint4*>(rmn + off);
        const uint4 vx = *reinterpret_cast<const uint4*>(rmx + off);
        const uint32_t wn[4] = {vn.x, vn.y, vn.z, vn.w};
        const uint32_t wx[4] = {vx.x, vx.y, vx.z, vx.w};
        float fn[8], fx[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (DT == HALO_F32) {
            fn[e] = __uint_as_float(wn[e]);
            fx[e] = __uint_as_float(wx[e]);
          } else if constexpr (DT == HALO_BF16) {
            fn[2 * e] = bf16_lo(wn[e]);
            fn[2 * e + 1] = bf16_hi(wn[e]);
            fx[2 * e] = bf16_lo(wx[e]);
            fx[2 * e + 1] = bf16_hi(wx[e]);
          } else {
            fn[2 * e] = f16_bits_to_f32((uint16_t)(wn[e] & 0xffffu));
            fn[2 * e + 1] = f16_bits_to_f32((uint16_t)(wn[e] >> 16));
            fx[2 * e] = f16_bits_to_f32((uint16_t)(wx[e] & 0xffffu));
            fx[2 * e + 1] = f16_bits_to_f32((uint16_t)(wx[e] >> 16));
          }
        }
#pragma unroll
        for (int e = 0; e < ep; ++e) {
          const float qd = qg[ep * (c + pp * G) + e];
          const float lo = __fmul_rn(qd, fn[e]), hi = __fmul_rn(qd, fx[e]);
          a = __fadd_rn(a, (lo > hi || lo != lo) ? lo : hi);
        }
      }
      part[c] = a;
    }
    for (int s = 1; s < G; s <<= 1)
      for (int c = 0; c + s < G; c += 2 * s) part[c] = __fadd_rn(part[c], part[c + s]);
    const float dot = part[0];
    if (P.dots) P.dots[(((int64_t)b * P.H_kv + h) * P.T_q + t) * P.P + p] = dot;
    best = dot != dot ? -INFINITY : dot;
  }
  s_best[w][lane] = best;
  __syncthreads();
  if (w == 0 && p < P.P) {
    float m = s_best[0][lane];
#pragma unroll
    for (int i = 1; i < 4; ++i) m = fmaxf(m, s_best[i][lane]);
    atomicMax(P.keys + (int64_t)sel * P.P + p, float_key(m));
  }
}

// Top-k of one selection: page i's rank is the number of pages with a
// larger score or an equal score and a lower index; ranks below k are
// written in rank order (descending score, as torch.topk returns them).
__global__ void __launch_bounds__(1024) quest_rank_kernel(const uint32_t* keys, int P, int k, int32_t* idx_out,
                                                          float* score_out) {
  __shared__ uint32_t s_key[kQuestMaxPages];
  const int sel = blockIdx.x;
  const uint32_t* kk = keys + (int64_t)sel * P;
  for (int i = threadIdx.x; i < P; i += blockDim.x) s_key[i] = kk[i];
  __syncthreads();
  for (int i = threadIdx.x; i < P; i += blockDim.x) {
    const uint32_t ki = s_key[i];
    int rank = 0;
    for (int j = 0; j < P; ++j) {
      const uint32_t kj = s_key[j];
      rank += (kj > ki || (kj == ki && j < i)) ? 1 : 0;
    }
    if (rank < k) idx_out[(int64_t)sel * k + rank] = i;
    if (score_out) score_out[(int64_t)sel * P + i] = key_float(ki);
  }
}

}  // namespace halo

using namespace halo;

extern "C" int halo_page_minmax(const void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
                                int dtype, int B, int H_kv, int D, int64_t row0, int page, int n_pages,
                                void* kmin, void* kmax, int64_t km_stride_b, int64_t km_stride_h,
                                int64_t km_stride_p, void* stream) {
  HALO_CHECK_ARG(k && kmin && kmax, "null pointer");
  HALO_CHECK_ARG(dtype == HALO_F32 || dtype == HALO_BF16 || dtype == HALO_F16, "bad dtype");
  HALO_CHECK_ARG(B > 0 && H_kv > 0 && D > 0 && page > 0 && n_pages >= 0 && row0 >= 0, "bad sizes");
  if (n_pages == 0) return HALO_OK;
  HALO_CHECK_ARG(D % (dtype == HALO_F32 ? 4 : 8) == 0 && D <= 256 * (dtype == HALO_F32 ? 4 : 8),
                 "head dim must fill whole 16-byte pieces");
  HALO_CHECK_ARG(reinterpret_cast<uintptr_t>(k) % 16 == 0 && (k_stride_t * elem_size(dtype)) % 16 == 0 &&
                 (k_stride_h * elem_size(dtype)) % 16 == 0 && (k_stride_b * elem_size(dtype)) % 16 == 0,
                 "key rows must be 16-byte aligned");
  const int64_t blocks = (int64_t)B * H_kv * n_pages;
  HALO_CHECK_ARG(blocks <= 0x7fffffffLL, "too many pages for one launch");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define HALO_MINMAX(DTV)                                                                                  \
  hipLaunchKernelGGL(page_minmax_kernel<DTV>, dim3((unsigned)blocks), dim3(256), 0, st, k, k_stride_b,    \
                     k_stride_h, k_stride_t, H_kv, D, row0, page, n_pages, kmin, kmax, km_stride_b,       \
                     km_stride_h, km_stride_p)
  if (dtype == HALO_F32) HALO_MINMAX(HALO_F32);
  else if (dtype == HALO_BF16) HALO_MINMAX(HALO_BF16);
  else HALO_MINMAX(HALO_F16);
#undef HALO_MINMAX
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}

extern "C" int halo_quest_score_topk(const void* q, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t,
                                     int dtype, int B, int H, int H_kv, int T_q, int D, const void* kmin,
                                     const void* kmax, int64_t km_stride_b, int64_t km_stride_h,
                                     int64_t km_stride_p, int P, int k, int per_row, uint32_t* workspace,
                                     float* dots_out, float* score_out, int32_t* idx_out, void* stream) {
  HALO_CHECK_ARG(q && kmin && kmax && workspace, "null pointer");
  HALO_CHECK_ARG(dtype == HALO_F32 || dtype == HALO_BF16 || dtype == HALO_F16, "bad dtype");
  HALO_CHECK_ARG(B > 0 && H > 0 && H_kv > 0 && H % H_kv == 0 && T_q > 0, "bad head sizes");
  HALO_CHECK_ARG(D % 16 == 0 && D > 0 && D <= kQuestMaxD, "head dim must be a multiple of 16, at most 256");
  HALO_CHECK_ARG(P > 0 && P <= kQuestMaxPages, "page count must be in [1, 8192]");
  HALO_CHECK_ARG(k >= 0 && k <= P, "k must be in [0, P]");
  HALO_CHECK_ARG(k == 0 || idx_out != nullptr, "idx_out is required when k > 0");
  const int es = elem_size(dtype);
  HALO_CHECK_ARG(reinterpret_cast<uintptr_t>(kmin) % 16 == 0 && reinterpret_cast<uintptr_t>(kmax) % 16 == 0 &&
                 (km_stride_p * es) % 16 == 0 && (km_stride_h * es) % 16 == 0 && (km_stride_b * es) % 16 == 0,
                 "kmin/kmax rows must be 16-byte aligned");
  const int n_sel = per_row ? B : 1;
  const int64_t rows_sel = (int64_t)(per_row ? 1 : B) * H_kv * T_q;
  const int64_t row_tiles = (rows_sel + 3) / 4;
  const int64_t page_tiles = (P + 63) / 64;
  const int64_t blocks = (int64_t)n_sel * row_tiles * page_tiles;
  HALO_CHECK_ARG(blocks <= 0x7fffffffLL, "too many (row, page) tiles for one launch");
  QuestParams p;
  p.q = q;
  p.qsb = q_stride_b;
  p.qsh = q_stride_h;
  p.qst = q_stride_t;
  p.B = B;
  p.H = H;
  p.H_kv = H_kv;
  p.T_q = T_q;
  p.D = D;
  p.rep = H / H_kv;
  p.inv_rep = (float)(1.0 / (double)p.rep);
  p.kmin = kmin;
  p.kmax = kmax;
  p.msb = km_stride_b;
  p.msh = km_stride_h;
  p.msp = km_stride_p;
  p.P = P;
  p.per_row = per_row;
  p.rows_sel = (int)rows_sel;
  p.row_tiles = (int)row_tiles;
  p.page_tiles = (int)page_tiles;
  p.dots = dots_out;
  p.keys = workspace;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int n_keys = n_sel * P;
  hipLaunchKernelGGL(quest_init_kernel, dim3((n_keys + 255) / 256), dim3(256), 0, st, workspace, n_keys);
  if (dtype == HALO_F32) hipLaunchKernelGGL(quest_score_kernel<HALO_F32>, dim3((unsigned)blocks), dim3(256), 0, st, p);
  else if (dtype == HALO_BF16)
    hipLaunchKernelGGL(quest_score_kernel<HALO_BF16>, dim3((unsigned)blocks), dim3(256), 0, st, p);
  else hipLaunchKernelGGL(quest_score_kernel<HALO_F16>, dim3((unsigned)blocks), dim3(256), 0, st, p);
  hipLaunchKernelGGL(quest_rank_kernel, dim3(n_sel), dim3(1024), 0, st, workspace, P, k, idx_out, score_out);
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}
