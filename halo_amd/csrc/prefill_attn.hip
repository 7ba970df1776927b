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
// are loaded straight into LDS (LDS-DMA) by the whole workgroup,
// double-buffered (the next tile's loads are in flight while the current one
// is consumed): K row-major with XOR-swizzled pieces (read as MFMA A
// operands), V row-major with swizzled pieces, read with transposed LDS reads
// as the A operands of O^T = V^T P^T.
//   scores  S^T[key][q] = sum_d K[key][d] Q[q][d]    v_mfma_f32_16x16x32
//   output  O^T[d][q]  += sum_key V^T[d][key] P^T[key][q]
// The P^T operand is built in registers from the S^T accumulators with a
// permuted key order inside each 32-key step (keys 4g..4g+3 and 16+4g..
// 16+4g+3 for lane group g); V^T is read with the same permutation, so no
// cross-lane movement is needed.  Masks are applied only on tiles that cross
// a chunk end or the causal diagonal.  Workgroups are mapped so that the query
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
    typedef __attribute__((ext_vector_type(2))) __bf16 b2;
    const b2 v = {(__bf16)a, (__bf16)b};  // round to nearest even
    return __builtin_bit_cast(uint32_t, v);
  }
};
template <>
struct PMfma<HALO_F16> {
  typedef __attribute__((ext_vector_type(8))) _Float16 v8;
  __device__ static __forceinline__ pf32x4 run(const uint4& a, const uint4& b, pf32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack(float a, float b) {
    typedef __attribute__((ext_vector_type(2))) _Float16 h2;
    const h2 v = {(_Float16)a, (_Float16)b};  // round to nearest even
    return __builtin_bit_cast(uint32_t, v);
  }
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t prsrc(const char* base, int64_t bytes) {
  const int nrec = bytes <= 0 ? 0 : (bytes > 0x7fffffffLL ? 0x7fffffff : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), 0, nrec, 0x00020000);
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

// V tile in LDS: row r holds its 16-byte pieces at positions piece ^ swizzle(r)
// (an even XOR: the piece pairs one transposed read covers stay adjacent; 4
// consecutive rows land on distinct 32-byte bank ranges).
template <int SL>
__device__ __forceinline__ int pf_vswz(int r) {
  return (2 * (r & 3) + 8 * ((r >> 3) & 1)) & (SL - 1);
}
// K tile in LDS: row r holds its 16-byte pieces at positions piece ^ (r % SL),
// so the 16 rows one MFMA operand read touches land on distinct bank ranges.
template <int SL>
__device__ __forceinline__ int pf_kswz(int r) {
  return r & (SL - 1);
}
// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i%4
// of the 8-byte reads of lanes 4e + i/4 (e = 0..3).
typedef short pv4i16_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 pf_tr16(const char* p) {
  const pv4i16_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) pv4i16_t*)(__attribute__((address_space(3))) char*)(p));
  return __builtin_bit_cast(uint2, r);
}
// Slack (log2 units) by which a tile's max may exceed the running max before
// the running max moves: probabilities stay below 2^8 and the accumulators are
// rescaled only when the max really moves; out = o / l and lse = m + log2(l)
// use the same m, so the result does not depend on when m moved.
constexpr float kPfLazyMax = 8.0f;

template <int DT, int D>
__global__ void __launch_bounds__(256, 2) prefill_attn_kernel(PrefillParams P) {
  constexpr int KS = D / 32;              // d-steps of the score MFMA
  constexpr int DB = D / 16;              // d-blocks of the output MFMA
  constexpr int SL = D / 8;               // 16-byte pieces per row
  constexpr int RB = D * 2;               // row bytes
  constexpr int KTB = kPfBK * RB;         // K tile bytes in LDS
  constexpr int STAGE = KTB + kPfBK * RB; // K tile + V tile
  constexpr int RPI = 1024 / RB;          // rows per 1 KiB LDS-DMA instruction
  constexpr int KPT = kPfBK * SL / 256;   // K (and V) pieces per thread per tile
  static_assert(KPT >= 1 && kPfBK * SL % 256 == 0, "prefill tile shape");
  __shared__ __attribute__((aligned(16))) char s_buf[2 * STAGE];

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
  const int64_t wave_qmin = qs + row0;              // smallest query position of this wave

  // ---- walk the (chunk, 64-row tile) sequence, one tile ahead
  struct Tile {
    const char* kb;
    const char* vb;
    int64_t kst, vst, cstart;
    int rows, kt, causal;
  };
  // the first tile of the first chunk at or after `from` that has rows for
  // this workgroup; returns false at the end of the table
  auto open_chunk = [&](int from, int& ci, Tile& t) -> bool {
    for (int c = from; c < P.n_desc; ++c) {
      const halo_chunk_desc d = P.descs[c];
      if (d.batch >= 0 && d.batch != b) continue;
      const int causal = d.flags & HALO_CHUNK_CAUSAL;
      int rows = d.T_c;
      if (causal) rows = (int)max<int64_t>(0, min<int64_t>(rows, wg_qmax - d.chunk_start + 1));
      if (rows <= 0) continue;
      t.kb = reinterpret_cast<const char*>(d.k) +
             ((d.batch < 0 ? (int64_t)b * d.k_stride_b : 0) + (int64_t)h_kv * d.k_stride_h) * 2;
      t.vb = reinterpret_cast<const char*>(d.v) +
             ((d.batch < 0 ? (int64_t)b * d.v_stride_b : 0) + (int64_t)h_kv * d.v_stride_h) * 2;
      t.kst = d.k_stride_t * 2;
      t.vst = d.v_stride_t * 2;
      t.cstart = d.chunk_start;
      t.rows = rows;
      t.kt = 0;
      t.causal = causal;
      ci = c;
      return true;
    }
    ci = P.n_desc;
    return false;
  };
  // Tile loads go straight from memory into LDS stage `st` (LDS-DMA: each
  // 1 KiB instruction of a wave fills RPI consecutive rows, lane l the
  // 16-byte position l % SL of row l / SL; the lane picks which global piece
  // lands there, which lays out the swizzles).  Rows past the chunk read as
  // zeros (buffer range check).  No registers hold the tile, so the loads of
  // the next tile can be in flight during the whole current one.
  auto issue_tile = [&](const Tile& t, char* st) {
    const __amdgpu_buffer_rsrc_t rk = prsrc(t.kb + (int64_t)t.kt * t.kst, (int64_t)(t.rows - t.kt) * t.kst);
    const __amdgpu_buffer_rsrc_t rv = prsrc(t.vb + (int64_t)t.kt * t.vst, (int64_t)(t.rows - t.kt) * t.vst);
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const int blk = wave * KPT + j;            // 1 KiB block of the tile
      const int r = blk * RPI + lane / SL, pos = lane % SL;
      // offsets computed before the calls: a __device__ helper call inside
      // the builtin's arguments makes the host pass drop the kernel's stub
      const int koff = (int)(r * t.kst) + ((pos ^ pf_kswz<SL>(r)) << 4);
      const int voff = (int)(r * t.vst) + ((pos ^ pf_vswz<SL>(r)) << 4);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(st + blk * 1024), 16,
                                               koff, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)(st + KTB + blk * 1024),
                                               16, voff, 0, 0, 0);
    }
  };

  int ci;
  Tile cur;
  bool have = open_chunk(0, ci, cur);
  if (have) issue_tile(cur, s_buf);
  __builtin_amdgcn_s_waitcnt(0);  // this wave's tile loads have landed in LDS
  __syncthreads();
  int stage = 0;
  while (have) {
    // the next tile: its loads are issued after this tile's score MFMAs (a
    // wait for them placed before the first MFMA would stall the wave) and
    // are in flight during the softmax and P.V
    Tile nxt = cur;
    int ni = ci;
    bool have_nxt = true;
    nxt.kt += kPfBK;
    if (nxt.kt >= nxt.rows) have_nxt = open_chunk(ci + 1, ni, nxt);
    const char* sk = s_buf + stage * STAGE;
    const char* sv = sk + KTB;
    // scores S^T for 4 key blocks x 2 query column blocks
    pf32x4 st[4][2];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      st[kb][0] = pf32x4{0.f, 0.f, 0.f, 0.f};
      st[kb][1] = pf32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int kr = kb * 16 + ql;
        const uint4 a = *reinterpret_cast<const uint4*>(sk + kr * RB + (((s * 4 + g) ^ pf_kswz<SL>(kr)) << 4));
        st[kb][0] = PMfma<DT>::run(a, qb[0][s], st[kb][0]);
        st[kb][1] = PMfma<DT>::run(a, qb[1][s], st[kb][1]);
      }
    }
    if (have_nxt) issue_tile(nxt, s_buf + (stage ^ 1) * STAGE);
    // masking only where the tile crosses the chunk end or the causal diagonal
    const bool masked = cur.kt + kPfBK > cur.rows || (cur.causal && cur.cstart + cur.kt + kPfBK - 1 > wave_qmin);
    uint4 pb[2][2];
    bool moved = false;
    float alpha[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int64_t qp = qpos0 + c * 16;
      float sv4[4][4];
      float bm = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float x = st[kb][c][e];
          if (masked) {
            const int key = cur.kt + kb * 16 + g * 4 + e;
            const bool valid = key < cur.rows && (!cur.causal || cur.cstart + key <= qp);
            x = valid ? x : -INFINITY;
          }
          sv4[kb][e] = x;
          bm = fmaxf(bm, x);
        }
      bm = rows4_max(bm);
      const float bms = bm * P.scale2;  // scores scale after the max (scale > 0)
      const float m_old = m_run[c];
      const float m_new = (bms > m_old + kPfLazyMax) ? bms : m_old;
      alpha[c] = (m_new == m_old) ? 1.f : __builtin_amdgcn_exp2f(m_old - m_new);
      moved |= m_new != m_old;
      m_run[c] = m_new;
      const float ms = (m_new == -INFINITY) ? 0.f : m_new;
      float p[4][4], psum = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          p[kb][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv4[kb][e], P.scale2, -ms));
          psum += p[kb][e];
        }
      l_run[c] = l_run[c] * alpha[c] + psum;
      // P^T operand of key step t: keys 4g..4g+3 of block 2t, then of block 2t+1
#pragma unroll
      for (int t = 0; t < 2; ++t)
        pb[c][t] = make_uint4(PMfma<DT>::pack(p[2 * t][0], p[2 * t][1]), PMfma<DT>::pack(p[2 * t][2], p[2 * t][3]),
                              PMfma<DT>::pack(p[2 * t + 1][0], p[2 * t + 1][1]),
                              PMfma<DT>::pack(p[2 * t + 1][2], p[2 * t + 1][3]));
    }
    if (__builtin_amdgcn_read_exec() & __ballot(moved)) {
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int db = 0; db < DB; ++db) o[c][db] *= alpha[c];
    }
    // O^T += V^T P^T; V^T operands by transposed reads in the same key order
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const int rlo = t * 32 + g * 4 + (ql >> 2), rhi = rlo + 16;
        const int pc = 2 * db + ((ql & 3) >> 1), bo = (ql & 1) * 8;
        const uint2 a0 = pf_tr16(sv + rlo * RB + ((pc ^ pf_vswz<SL>(rlo)) << 4) + bo);
        const uint2 a1 = pf_tr16(sv + rhi * RB + ((pc ^ pf_vswz<SL>(rhi)) << 4) + bo);
        const uint4 a = make_uint4(a0.x, a0.y, a1.x, a1.y);
        o[0][db] = PMfma<DT>::run(a, pb[0][t], o[0][db]);
        o[1][db] = PMfma<DT>::run(a, pb[1][t], o[1][db]);
      }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of the next tile have landed
    __syncthreads();  // the next tile is in LDS; this one is free for the tile after
    stage ^= 1;
    cur = nxt;
    ci = ni;
    have = have_nxt;
  }

  // normalise and store: lane holds O^T[d = 16db + 4g + e][query ql]
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const float lt = rows4_sum(l_run[c]);
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
