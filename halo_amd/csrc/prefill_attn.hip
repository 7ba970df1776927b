// Chunked causal prefill attention on CDNA4 bf16/fp16 MFMA (gfx950, wave64).
//
// Reference semantics: HALOCacheChunked._chunk_attention + _lse_merge
// (halo/kv_cache_chunked.py:194-276) walked over the chunk list, i.e. for
// every query row the softmax over all attended key rows of all chunks, with
// the causal rule chunk_start + t <= q_start + i (halo/triton_chunked.py:
// 114-119).  The per-chunk partials of the reference merge associatively by
// log-sum-exp, so one online-softmax pass over the whole chunk list gives the
// same (out, lse).
//
// Tiling: one workgroup = 4 waves = 128 query rows of one query head; each
// wave owns 32 rows as two 16-row MFMA column blocks.  Key tiles of 64 rows
// are staged in LDS by the whole workgroup: K row-major (read as MFMA A
// operands), V transposed (V^T[d][key], read as A operands of O^T = V^T P^T).
//   scores  S^T[key][q] = sum_d K[key][d] Q[q][d]    v_mfma_f32_16x16x32
//   output  O^T[d][q]  += sum_key V^T[d][key] P^T[key][q]
// The P^T operand is built in registers from the S^T accumulators with a
// permuted key order inside each 32-key step (keys 4g..4g+3 and 16+4g..
// 16+4g+3 for lane group g); V^T is read with the same permutation, so no
// cross-lane movement is needed.  Workgroups are mapped so that the query
// heads sharing a KV head run on the same XCD (its L2 serves their K/V).

#include "common.hpp"

namespace halo {

namespace {

typedef __attribute__((ext_vector_type(4))) float pf32x4;

template <int DT>
struct PMfma;
template <>
struct PMfma<HALO_BF16> {
  typedef __attribute__((ext_vector_type(8))) __bf16 v8;
  __device__ static __forceinline__ pf32x4 run(const uint4& a, const uint4& b, pf32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack(float a, float b) {
    return (uint32_t)f32_to_bf16_rne(a) | ((uint32_t)f32_to_bf16_rne(b) << 16);
  }
};
template <>
struct PMfma<HALO_F16> {
  typedef __attribute__((ext_vector_type(8))) _Float16 v8;
  __device__ static __forceinline__ pf32x4 run(const uint4& a, const uint4& b, pf32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack(float a, float b) {
    return (uint32_t)f32_to_f16_rne(a) | ((uint32_t)f32_to_f16_rne(b) << 16);
  }
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t prsrc(const char* base, int64_t bytes) {
  const int nrec = bytes <= 0 ? 0 : (bytes > 0x7fffffffLL ? 0x7fffffff : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), 0, nrec, 0x00020000);
}
__device__ __forceinline__ uint4 pld16(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

}  // namespace

struct PrefillParams {
  const void* q;
  int64_t q_stride_b, q_stride_h, q_stride_t;
  int B, H, H_kv, rep, T_q, n_qt, n_units;
  const int64_t* q_start;  // [B] global position of query row 0
  const halo_chunk_desc* descs;
  int n_desc;
  float scale2;
  void* out;
  int64_t o_stride_b, o_stride_h, o_stride_t;
  int out_dtype;
  float* lse;  // (B, H, T_q) contiguous, or null
};

constexpr int kPfNW = 4;    // waves per workgroup
constexpr int kPfQW = 32;   // query rows per wave
constexpr int kPfBQ = kPfNW * kPfQW;
constexpr int kPfBK = 64;   // key rows per LDS tile

template <int DT, int D>
__global__ void __launch_bounds__(256, 2) prefill_attn_kernel(PrefillParams P) {
  constexpr int KS = D / 32;            // d-steps of the score MFMA
  constexpr int DB = D / 16;            // d-blocks of the output MFMA
  constexpr int SL = D / 8;             // 16-byte pieces per row
  constexpr int KROWB = D * 2 + 16;     // padded K row in LDS (bytes)
  constexpr int VTROW = kPfBK * 2 + 16; // padded V^T row in LDS (bytes)
  constexpr int KPT = kPfBK * SL / 256; // K pieces per thread per tile
  constexpr int KQ = kPfBK / 4;         // key quads per tile
  static_assert(KPT >= 1 && KQ * SL <= 256 * 1, "prefill tile shape");
  __shared__ __attribute__((aligned(16))) char s_k[kPfBK * KROWB];
  __shared__ __attribute__((aligned(16))) char s_vt[D * VTROW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ql = lane & 15, g = lane >> 4;

  // XCD-aware unit order: the units of one XCD (blockIdx % 8) are a
  // contiguous run, so the query heads of one KV group share an L2.
  int unit = blockIdx.x;
  if ((P.n_units & 7) == 0) unit = (blockIdx.x & 7) * (P.n_units >> 3) + (blockIdx.x >> 3);
  const int h = unit % P.H;
  const int qt = (unit / P.H) % P.n_qt;
  const int b = unit / (P.H * P.n_qt);
  const int h_kv = h / P.rep;
  const int row0 = qt * kPfBQ + wave * kPfQW;   // this wave's first query row
  const int64_t qs = P.q_start[b];

  // Q as B operands (lane: query ql of each column block, elements 8g.. of each d-step)
  uint4 qb[2][KS];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int r = row0 + c * 16 + ql;
    const char* qrow = reinterpret_cast<const char*>(P.q) +
                       ((int64_t)b * P.q_stride_b + (int64_t)h * P.q_stride_h + (int64_t)min(r, P.T_q - 1) * P.q_stride_t) * 2;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qb[c][s] = r < P.T_q ? *reinterpret_cast<const uint4*>(qrow + (s * 32 + g * 8) * 2) : make_uint4(0, 0, 0, 0);
  }
  pf32x4 o[2][DB];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int db = 0; db < DB; ++db) o[c][db] = pf32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
  const int64_t qpos0 = qs + row0 + ql;             // column block 0 query position
  const int64_t wg_qmax = qs + min(qt * kPfBQ + kPfBQ, P.T_q) - 1;

  for (int ci = 0; ci < P.n_desc; ++ci) {
    const halo_chunk_desc dsc = P.descs[ci];
    if (dsc.batch >= 0 && dsc.batch != b) continue;
    const bool causal = dsc.flags & HALO_CHUNK_CAUSAL;
    int rows = dsc.T_c;
    if (causal) rows = (int)max<int64_t>(0, min<int64_t>(rows, wg_qmax - dsc.chunk_start + 1));
    if (rows <= 0) continue;
    const char* kbase = reinterpret_cast<const char*>(dsc.k) +
                        ((dsc.batch < 0 ? (int64_t)b * dsc.k_stride_b : 0) + (int64_t)h_kv * dsc.k_stride_h) * 2;
    const char* vbase = reinterpret_cast<const char*>(dsc.v) +
                        ((dsc.batch < 0 ? (int64_t)b * dsc.v_stride_b : 0) + (int64_t)h_kv * dsc.v_stride_h) * 2;
    const int64_t kst = dsc.k_stride_t * 2, vst = dsc.v_stride_t * 2;
    for (int kt = 0; kt < rows; kt += kPfBK) {
      const __amdgpu_buffer_rsrc_t rk = prsrc(kbase + (int64_t)kt * kst, (int64_t)(rows - kt) * kst);
      const __amdgpu_buffer_rsrc_t rv = prsrc(vbase + (int64_t)kt * vst, (int64_t)(rows - kt) * vst);
      uint4 kr[KPT], vr[4];
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const int id = tid + 256 * j;
        kr[j] = pld16(rk, (int)((id / SL) * kst) + (id % SL) * 16);
      }
      const int vp = tid % SL, vq = tid / SL;   // V: d-piece, key quad
      const bool vlive = vq < KQ;
#pragma unroll
      for (int j = 0; j < 4; ++j) vr[j] = vlive ? pld16(rv, (int)((vq * 4 + j) * vst) + vp * 16) : make_uint4(0, 0, 0, 0);
      __syncthreads();  // the previous tile's readers are done
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const int id = tid + 256 * j;
        *reinterpret_cast<uint4*>(s_k + (id / SL) * KROWB + (id % SL) * 16) = kr[j];
      }
      if (vlive) {
        // 4 keys x 8 channels -> 8 channels x 4 keys (two 16-bit keys per dword)
        const uint32_t w0[4] = {vr[0].x, vr[0].y, vr[0].z, vr[0].w};
        const uint32_t w1[4] = {vr[1].x, vr[1].y, vr[1].z, vr[1].w};
        const uint32_t w2[4] = {vr[2].x, vr[2].y, vr[2].z, vr[2].w};
        const uint32_t w3[4] = {vr[3].x, vr[3].y, vr[3].z, vr[3].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint2 lo = make_uint2(__builtin_amdgcn_perm(w1[j], w0[j], 0x05040100u),
                                      __builtin_amdgcn_perm(w3[j], w2[j], 0x05040100u));
          const uint2 hi = make_uint2(__builtin_amdgcn_perm(w1[j], w0[j], 0x07060302u),
                                      __builtin_amdgcn_perm(w3[j], w2[j], 0x07060302u));
          *reinterpret_cast<uint2*>(s_vt + (vp * 8 + 2 * j) * VTROW + vq * 8) = lo;
          *reinterpret_cast<uint2*>(s_vt + (vp * 8 + 2 * j + 1) * VTROW + vq * 8) = hi;
        }
      }
      __syncthreads();

      // scores S^T for 4 key blocks x 2 query column blocks
      pf32x4 st[4][2];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        st[kb][0] = pf32x4{0.f, 0.f, 0.f, 0.f};
        st[kb][1] = pf32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const uint4 a = *reinterpret_cast<const uint4*>(s_k + (kb * 16 + ql) * KROWB + (s * 32 + g * 8) * 2);
          st[kb][0] = PMfma<DT>::run(a, qb[0][s], st[kb][0]);
          st[kb][1] = PMfma<DT>::run(a, qb[1][s], st[kb][1]);
        }
      }
      // online softmax per query column (lane's query ql of each block)
      uint4 pb[2][2];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int64_t qp = qpos0 + c * 16;
        float sv[4][4], bm = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int key = kt + kb * 16 + g * 4 + e;
            bool valid = key < rows;
            if (causal) valid = valid && (dsc.chunk_start + key <= qp);
            sv[kb][e] = valid ? st[kb][c][e] * P.scale2 : -INFINITY;
            bm = fmaxf(bm, sv[kb][e]);
          }
        bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
        bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
        const float m_new = fmaxf(m_run[c], bm);
        const float ms = (m_new == -INFINITY) ? 0.f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run[c] - ms);
        m_run[c] = m_new;
        float p[4][4], psum = 0.f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            p[kb][e] = __builtin_amdgcn_exp2f(sv[kb][e] - ms);
            psum += p[kb][e];
          }
        l_run[c] = l_run[c] * alpha + psum;
        if (alpha != 1.f) {
#pragma unroll
          for (int db = 0; db < DB; ++db) o[c][db] *= alpha;
        }
        // P^T operand of key step t: keys 4g..4g+3 of block 2t, then of block 2t+1
#pragma unroll
        for (int t = 0; t < 2; ++t)
          pb[c][t] = make_uint4(PMfma<DT>::pack(p[2 * t][0], p[2 * t][1]), PMfma<DT>::pack(p[2 * t][2], p[2 * t][3]),
                                PMfma<DT>::pack(p[2 * t + 1][0], p[2 * t + 1][1]),
                                PMfma<DT>::pack(p[2 * t + 1][2], p[2 * t + 1][3]));
      }
      // O^T += V^T P^T
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const char* vrow = s_vt + (db * 16 + ql) * VTROW;
          const uint2 a0 = *reinterpret_cast<const uint2*>(vrow + (t * 32 + g * 4) * 2);
          const uint2 a1 = *reinterpret_cast<const uint2*>(vrow + (t * 32 + 16 + g * 4) * 2);
          const uint4 a = make_uint4(a0.x, a0.y, a1.x, a1.y);
          o[0][db] = PMfma<DT>::run(a, pb[0][t], o[0][db]);
          o[1][db] = PMfma<DT>::run(a, pb[1][t], o[1][db]);
        }
    }
  }

  // normalise and store: lane holds O^T[d = 16db + 4g + e][query ql]
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    float lt = l_run[c] + __shfl_xor(l_run[c], 16, 64);
    lt += __shfl_xor(lt, 32, 64);
    const int r = row0 + c * 16 + ql;
    if (r >= P.T_q) continue;
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const int64_t ob = (int64_t)b * P.o_stride_b + (int64_t)h * P.o_stride_h + (int64_t)r * P.o_stride_t;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int e = 0; e < 4; ++e) store_elem(P.out, ob + db * 16 + g * 4 + e, P.out_dtype, o[c][db][e] * inv);
    if (P.lse != nullptr && g == 0)
      P.lse[((int64_t)b * P.H + h) * P.T_q + r] = lt > 0.f ? (m_run[c] + log2f(lt)) * kLn2 : -INFINITY;
  }
}

}  // namespace halo

using namespace halo;

extern "C" int halo_prefill_attn(const void* q, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t,
                                 int dtype, int B, int H, int H_kv, int T_q, int D, const int64_t* q_start,
                                 const halo_chunk_desc* descs, int n_desc, float scale,
                                 void* out, int64_t out_stride_b, int64_t out_stride_h, int64_t out_stride_t,
                                 int out_dtype, float* lse, void* stream) {
  HALO_CHECK_ARG(q && q_start && descs && out, "null pointer argument");
  HALO_CHECK_ARG(dtype == HALO_BF16 || dtype == HALO_F16, "prefill runs on bf16/fp16 MFMA: dtype must be bf16 or f16");
  HALO_CHECK_ARG(out_dtype == HALO_F32 || out_dtype == HALO_BF16 || out_dtype == HALO_F16, "bad out_dtype");
  HALO_CHECK_ARG(B > 0 && H > 0 && H_kv > 0 && H % H_kv == 0 && T_q >= 0, "need H % H_kv == 0 and positive sizes");
  HALO_CHECK_ARG(D == 64 || D == 128, "head_dim must be 64 or 128");
  HALO_CHECK_ARG(n_desc >= 0, "bad chunk count");
  HALO_CHECK_ARG(reinterpret_cast<uintptr_t>(q) % 16 == 0 && (q_stride_t * 2) % 16 == 0 && (q_stride_h * 2) % 16 == 0 &&
                     (q_stride_b * 2) % 16 == 0,
                 "q rows must be 16-byte aligned");
  if (T_q == 0) return HALO_OK;
  PrefillParams p;
  p.q = q;
  p.q_stride_b = q_stride_b;
  p.q_stride_h = q_stride_h;
  p.q_stride_t = q_stride_t;
  p.B = B;
  p.H = H;
  p.H_kv = H_kv;
  p.rep = H / H_kv;
  p.T_q = T_q;
  p.n_qt = (T_q + kPfBQ - 1) / kPfBQ;
  const int64_t units = (int64_t)B * H * p.n_qt;
  HALO_CHECK_ARG(units < (1ll << 31), "too many query tiles");
  p.n_units = (int)units;
  p.q_start = q_start;
  p.descs = descs;
  p.n_desc = n_desc;
  p.scale2 = (float)((double)scale * 1.4426950408889634);
  p.out = out;
  p.o_stride_b = out_stride_b;
  p.o_stride_h = out_stride_h;
  p.o_stride_t = out_stride_t;
  p.out_dtype = out_dtype;
  p.lse = lse;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == HALO_BF16) {
    if (D == 128) hipLaunchKernelGGL((prefill_attn_kernel<HALO_BF16, 128>), dim3(p.n_units), dim3(256), 0, st, p);
    else hipLaunchKernelGGL((prefill_attn_kernel<HALO_BF16, 64>), dim3(p.n_units), dim3(256), 0, st, p);
  } else {
    if (D == 128) hipLaunchKernelGGL((prefill_attn_kernel<HALO_F16, 128>), dim3(p.n_units), dim3(256), 0, st, p);
    else hipLaunchKernelGGL((prefill_attn_kernel<HALO_F16, 64>), dim3(p.n_units), dim3(256), 0, st, p);
  }
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}
