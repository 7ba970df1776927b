// Split-K GQA decode attention over a KV chunk table with a fused
// log-sum-exp merge (gfx950, wave64).
//
// Reference semantics: halo/triton_chunked.py:46-138 (per-chunk online
// softmax update), :195-207 (finalize), halo/kv_cache_chunked.py:194-276
// (per-chunk attention + LSE merge with -inf guards).
//
// Layout of the work:
//   * one workgroup = one work item {chunk, query-head group, rows [t0,t1)};
//     a query-head group is (b, h_kv, sub): all rep_t query heads that share
//     KV head h_kv, so each K/V row is read from HBM exactly once per group
//     (the reference launches one program per *query* head, rereading K/V
//     rep times: halo/triton_chunked.py:69-73,179).
//   * each of the NW waves owns a contiguous slice of the rows and walks it in
//     64-row tiles.  Every 16-byte load instruction of a wave covers 64/SL
//     whole rows (1 KiB contiguous), for K and V alike.
//   * K tiles are transposed through LDS so that lane t owns row t for the
//     q.k dot products (no cross-lane reduction per row); V stays in the
//     load layout, where each lane accumulates an 8-element (bf16/f16) or
//     4-element (fp32) slice of the output for every query head.
//   * online softmax in the log2 domain, fp32 throughout.
//   * the NW wave partials merge in LDS into one partial per work item; the
//     last workgroup of a query-head group (atomic ticket) merges the group's
//     partials in work order -- deterministic run to run -- together with the
//     caller's accumulators, and writes (m,l,o) and/or (out, lse).

#include "common.hpp"

namespace halo {

struct DecodeParams {
  const void* q;
  int64_t q_stride_b, q_stride_h;
  int H, H_kv, rep, n_sub;
  const halo_chunk_desc* descs;
  const int32_t* work;
  const int32_t* group_offsets;
  const int64_t* q_pos;
  float scale2;  // scale * log2(e)
  float* m;
  float* l;
  float* o;
  int64_t acc_stride_b;  // elements between batch rows of m/l (H); o uses *D
  int acc_mode;
  void* out;
  int out_dtype;
  float* lse;
  float* ws_o;   // [n_work][REP][D]
  float* ws_ml;  // [n_work][REP][2]  (m2, l)
  int32_t* counters;
};

template <int DT>
struct Elem;
template <>
struct Elem<HALO_F32> {
  static constexpr int size = 4;
  static constexpr int per16 = 4;
  // 4 floats of a 16-byte piece
  __device__ static __forceinline__ void unpack(const uint4& p, float* f) {
    f[0] = __uint_as_float(p.x);
    f[1] = __uint_as_float(p.y);
    f[2] = __uint_as_float(p.z);
    f[3] = __uint_as_float(p.w);
  }
  __device__ static __forceinline__ float dot(const uint4& a, const uint4& b, float acc) {
    acc = fmaf(__uint_as_float(a.x), __uint_as_float(b.x), acc);
    acc = fmaf(__uint_as_float(a.y), __uint_as_float(b.y), acc);
    acc = fmaf(__uint_as_float(a.z), __uint_as_float(b.z), acc);
    acc = fmaf(__uint_as_float(a.w), __uint_as_float(b.w), acc);
    return acc;
  }
};
template <>
struct Elem<HALO_BF16> {
  static constexpr int size = 2;
  static constexpr int per16 = 8;
  __device__ static __forceinline__ void unpack(const uint4& p, float* f) {
    f[0] = bf16_lo(p.x); f[1] = bf16_hi(p.x);
    f[2] = bf16_lo(p.y); f[3] = bf16_hi(p.y);
    f[4] = bf16_lo(p.z); f[5] = bf16_hi(p.z);
    f[6] = bf16_lo(p.w); f[7] = bf16_hi(p.w);
  }
  typedef __attribute__((ext_vector_type(2))) __bf16 bf2;
  __device__ static __forceinline__ float dot(const uint4& a, const uint4& b, float acc) {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.x), __builtin_bit_cast(bf2, b.x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.y), __builtin_bit_cast(bf2, b.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.z), __builtin_bit_cast(bf2, b.z), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.w), __builtin_bit_cast(bf2, b.w), acc, false);
    return acc;
  }
};
template <>
struct Elem<HALO_F16> {
  static constexpr int size = 2;
  static constexpr int per16 = 8;
  typedef __attribute__((ext_vector_type(2))) _Float16 h2;
  __device__ static __forceinline__ void unpack(const uint4& p, float* f) {
    h2 a = __builtin_bit_cast(h2, p.x), b = __builtin_bit_cast(h2, p.y);
    h2 c = __builtin_bit_cast(h2, p.z), d = __builtin_bit_cast(h2, p.w);
    f[0] = (float)a.x; f[1] = (float)a.y; f[2] = (float)b.x; f[3] = (float)b.y;
    f[4] = (float)c.x; f[5] = (float)c.y; f[6] = (float)d.x; f[7] = (float)d.y;
  }
  __device__ static __forceinline__ float dot(const uint4& a, const uint4& b, float acc) {
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a.x), __builtin_bit_cast(h2, b.x), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a.y), __builtin_bit_cast(h2, b.y), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a.z), __builtin_bit_cast(h2, b.z), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a.w), __builtin_bit_cast(h2, b.w), acc, false);
    return acc;
  }
};

__device__ __forceinline__ uint4 ld16(const char* p) {
  return *reinterpret_cast<const uint4*>(p);
}

template <int DT, int D, int REP, int NW>
__global__ void __launch_bounds__(64 * NW)
decode_attn_kernel(DecodeParams P) {
  using E = Elem<DT>;
  constexpr int EP = E::per16;        // elements per 16-byte piece
  constexpr int SL = D / EP;          // pieces per row
  constexpr int RPI = kWave / SL;     // rows covered by one load instruction
  constexpr int RB = D * E::size;     // bytes per row
  constexpr int KROW = RB + 16;       // padded LDS row stride (bank-conflict free)
  constexpr int TILE = SL <= 16 ? kWave : kWave * 16 / SL;  // rows per wave tile
  constexpr int PPL = TILE / RPI;     // 16-byte pieces per lane per tile (K and V each)
  static_assert(SL * RPI == kWave, "row must split evenly across the wave");
  static_assert(PPL * RPI == TILE, "tile must be whole load instructions");

  // Phase A (tile loop): q rows, per-wave K tiles, per-wave probabilities.
  // Phase B (wave merge): per-wave output partials, aliasing phase A.
  constexpr int SZ_Q = REP * RB;
  constexpr int SZ_K = NW * TILE * KROW;
  constexpr int SZ_P = NW * TILE * REP * 4;
  constexpr int SZ_A = SZ_Q + SZ_K + SZ_P;
  constexpr int SZ_B = NW * REP * D * 4;
  __shared__ __attribute__((aligned(16))) char smem[SZ_A > SZ_B ? SZ_A : SZ_B];
  char* s_q = smem;
  char* s_kall = smem + SZ_Q;
  float* s_pall = reinterpret_cast<float*>(smem + SZ_Q + SZ_K);
  float* s_wo = reinterpret_cast<float*>(smem);
  __shared__ float s_wm[NW][REP], s_wl[NW][REP];
  __shared__ float s_accm[REP], s_accl[REP];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int witem = blockIdx.x;

  const int4 item = reinterpret_cast<const int4*>(P.work)[witem];
  const halo_chunk_desc dsc = P.descs[item.x];
  const int g = item.y;
  const int sub = g % P.n_sub;
  const int bh = g / P.n_sub;
  const int h_kv = bh % P.H_kv;
  const int b = bh / P.H_kv;
  const int hq0 = h_kv * P.rep + sub * REP;
  const int nvalid_h = min(REP, P.rep - sub * REP);

  // Effective row range after the causal cut (rows t with chunk_start+t <= q_pos).
  int t0 = item.z, t1 = item.w;
  if ((dsc.flags & HALO_CHUNK_CAUSAL) && P.q_pos != nullptr) {
    const int64_t lim = P.q_pos[b] - dsc.chunk_start + 1;  // rows [0, lim) allowed
    if (lim < (int64_t)t1) t1 = (int)max<int64_t>(lim, (int64_t)t0);
  }

  // Stage the rep_t query rows of this group in LDS (zeros for padding heads).
  for (int i = tid; i < REP * D; i += 64 * NW) {
    const int r = i / D, d = i % D;
    if (DT == HALO_F32) {
      float v = 0.f;
      if (r < nvalid_h)
        v = reinterpret_cast<const float*>(P.q)[b * P.q_stride_b + (int64_t)(hq0 + r) * P.q_stride_h + d];
      reinterpret_cast<float*>(s_q)[i] = v;
    } else {
      uint16_t v = 0;
      if (r < nvalid_h)
        v = reinterpret_cast<const uint16_t*>(P.q)[b * P.q_stride_b + (int64_t)(hq0 + r) * P.q_stride_h + d];
      reinterpret_cast<uint16_t*>(s_q)[i] = v;
    }
  }
  __syncthreads();

  const char* kbase = reinterpret_cast<const char*>(dsc.k) +
                      ((dsc.batch < 0 ? (int64_t)b * dsc.k_stride_b : 0) + (int64_t)h_kv * dsc.k_stride_h) * E::size;
  const char* vbase = reinterpret_cast<const char*>(dsc.v) +
                      ((dsc.batch < 0 ? (int64_t)b * dsc.v_stride_b : 0) + (int64_t)h_kv * dsc.v_stride_h) * E::size;
  const int64_t kst = dsc.k_stride_t * E::size;
  const int64_t vst = dsc.v_stride_t * E::size;

  // This wave's slice of rows, in whole tiles.
  const int nrows_total = max(t1 - t0, 0);
  const int ntiles_total = (nrows_total + TILE - 1) / TILE;
  const int tiles_per_wave = (ntiles_total + NW - 1) / NW;
  const int ws = t0 + wave * tiles_per_wave * TILE;
  const int we = min(t1, ws + tiles_per_wave * TILE);

  float m_run[REP], l_run[REP], acc_o[REP][EP];
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    m_run[r] = -INFINITY;
    l_run[r] = 0.f;
#pragma unroll
    for (int e = 0; e < EP; ++e) acc_o[r][e] = 0.f;
  }

  char* kl = s_kall + wave * TILE * KROW;
  float* pl = s_pall + wave * TILE * REP;
  const bool in_tile = lane < TILE;
  const int my_col = lane % SL;
  const int my_row0 = lane / SL;

  for (int tb = ws; tb < we; tb += TILE) {
    const int nrows = min(TILE, we - tb);
    uint4 kreg[PPL], vreg[PPL];
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
      const int row = i * RPI + my_row0;
      if (row < nrows) {
        kreg[i] = ld16(kbase + (int64_t)(tb + row) * kst + my_col * 16);
        vreg[i] = ld16(vbase + (int64_t)(tb + row) * vst + my_col * 16);
      } else {
        kreg[i] = make_uint4(0, 0, 0, 0);
        vreg[i] = make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
      const int row = i * RPI + my_row0;
      *reinterpret_cast<uint4*>(kl + row * KROW + my_col * 16) = kreg[i];
    }
    wave_lds_fence();

    // q.k for row `lane`, all heads of the group.
    float s[REP];
#pragma unroll
    for (int r = 0; r < REP; ++r) s[r] = 0.f;
#pragma unroll
    for (int c = 0; c < SL; ++c) {
      const uint4 kp = *reinterpret_cast<const uint4*>(kl + (in_tile ? lane : 0) * KROW + c * 16);
#pragma unroll
      for (int r = 0; r < REP; ++r) {
        const uint4 qp = *reinterpret_cast<const uint4*>(s_q + r * RB + c * 16);
        s[r] = E::dot(kp, qp, s[r]);
      }
    }
    const bool valid = in_tile && lane < nrows;
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      const float s2 = valid ? s[r] * P.scale2 : -INFINITY;
      const float mt = wave_max(s2);
      const float m_new = fmaxf(m_run[r], mt);
      const float ms = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run[r] - ms);
      const float p = __builtin_amdgcn_exp2f(s2 - ms);
      l_run[r] = l_run[r] * alpha + p;
      m_run[r] = m_new;
#pragma unroll
      for (int e = 0; e < EP; ++e) acc_o[r][e] *= alpha;
      if (in_tile) pl[lane * REP + r] = p;
    }
    wave_lds_fence();

    // P.V: lane accumulates its output slice over the rows it loaded.
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
      const int row = j * RPI + my_row0;
      float vf[EP];
      E::unpack(vreg[j], vf);
      float pr[REP];
#pragma unroll
      for (int r = 0; r < REP; ++r) pr[r] = pl[row * REP + r];
#pragma unroll
      for (int r = 0; r < REP; ++r)
#pragma unroll
        for (int e = 0; e < EP; ++e) acc_o[r][e] = fmaf(pr[r], vf[e], acc_o[r][e]);
    }
    wave_lds_fence();
  }

  // Reduce the wave partial: l across lanes, o across the RPI row groups.
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    l_run[r] = wave_sum(l_run[r]);
#pragma unroll
    for (int off = SL; off < kWave; off <<= 1)
#pragma unroll
      for (int e = 0; e < EP; ++e) acc_o[r][e] += __shfl_xor(acc_o[r][e], off, kWave);
  }
  __syncthreads();  // every wave is out of its tile loop: phase B may reuse LDS
  if (lane < SL) {
#pragma unroll
    for (int r = 0; r < REP; ++r)
#pragma unroll
      for (int e = 0; e < EP; ++e) s_wo[(wave * REP + r) * D + lane * EP + e] = acc_o[r][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      s_wm[wave][r] = m_run[r];
      s_wl[wave][r] = l_run[r];
    }
  }
  __syncthreads();

  // Merge the NW wave partials into this work item's partial.
  float* wso = P.ws_o + (int64_t)witem * REP * D;
  for (int i = tid; i < REP * D; i += 64 * NW) {
    const int r = i / D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_wm[w][r]);
    const float Ms = (M == -INFINITY) ? 0.f : M;
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) acc += __builtin_amdgcn_exp2f(s_wm[w][r] - Ms) * s_wo[w * REP * D + i];
    wso[i] = acc;
  }
  if (tid < REP) {
    const int r = tid;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_wm[w][r]);
    const float Ms = (M == -INFINITY) ? 0.f : M;
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) acc += __builtin_amdgcn_exp2f(s_wm[w][r] - Ms) * s_wl[w][r];
    P.ws_ml[((int64_t)witem * REP + r) * 2 + 0] = M;
    P.ws_ml[((int64_t)witem * REP + r) * 2 + 1] = acc;
  }

  // Publish the partial; the last workgroup of the group merges.
  __threadfence();
  __syncthreads();
  const int gbeg = P.group_offsets[g], gend = P.group_offsets[g + 1];
  if (tid == 0) {
    const int ticket = atomicAdd(&P.counters[g], 1);
    s_last = (ticket == gend - gbeg - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  const bool has_acc = P.m != nullptr;
  const bool merge_in = has_acc && (P.acc_mode & 1);
  const bool write_acc = has_acc && (P.acc_mode & 2);
  if (tid < REP) {
    const int r = tid;
    float am = -INFINITY, al = 0.f;
    if (merge_in && r < nvalid_h) {
      const int64_t a = (int64_t)b * P.acc_stride_b + hq0 + r;
      am = P.m[a] * kLog2e;
      al = P.l[a];
    }
    s_accm[r] = am;
    s_accl[r] = al;
  }
  __syncthreads();

  for (int i = tid; i < REP * D; i += 64 * NW) {
    const int r = i / D, d = i % D;
    if (r >= nvalid_h) continue;
    const int hq = hq0 + r;
    float M = s_accm[r];
    for (int it = gbeg; it < gend; ++it) M = fmaxf(M, P.ws_ml[((int64_t)it * REP + r) * 2]);
    const float Ms = (M == -INFINITY) ? 0.f : M;
    float osum = 0.f, lsum = 0.f;
    for (int it = gbeg; it < gend; ++it) {
      const float w = __builtin_amdgcn_exp2f(P.ws_ml[((int64_t)it * REP + r) * 2] - Ms);
      osum += w * P.ws_o[((int64_t)it * REP + r) * D + d];
      lsum += w * P.ws_ml[((int64_t)it * REP + r) * 2 + 1];
    }
    const int64_t oidx = ((int64_t)b * P.acc_stride_b + hq) * D + d;
    if (merge_in) {
      const float w = __builtin_amdgcn_exp2f(s_accm[r] - Ms);
      osum += w * P.o[oidx];
      lsum += w * s_accl[r];
    }
    if (write_acc) {
      P.o[oidx] = osum;
      if (d == 0) {
        const int64_t a = (int64_t)b * P.acc_stride_b + hq;
        P.m[a] = (M == -INFINITY) ? -INFINITY : M * kLn2;
        P.l[a] = lsum;
      }
    }
    if (P.out != nullptr) {
      const float v = lsum > 0.f ? osum / lsum : 0.f;
      store_elem(P.out, ((int64_t)b * P.H + hq) * D + d, P.out_dtype, v);
    }
    if (P.lse != nullptr && d == 0) {
      P.lse[(int64_t)b * P.H + hq] = lsum > 0.f ? (M + log2f(lsum)) * kLn2 : -INFINITY;
    }
  }
  if (tid == 0) P.counters[g] = 0;
}

// ---------------------------------------------------------------------------
// finalize / lse_merge (elementwise)
// ---------------------------------------------------------------------------
__global__ void finalize_kernel(const float* m, const float* l, const float* o, int64_t BH, int D,
                                void* out, int out_dtype, float* lse) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= BH * D) return;
  const int64_t row = i / D;
  const float lv = l[row];
  const float safe = lv > 0.f ? lv : 1.f;
  if (out) store_elem(out, i, out_dtype, o[i] / safe);
  if (lse && (i % D) == 0) lse[row] = lv > 0.f ? m[row] + logf(lv) : -INFINITY;
}

__global__ void lse_merge_kernel(const float* oa, const float* la, const float* ob, const float* lb,
                                 int64_t n, int D, float* out, float* lse) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * D) return;
  const int64_t row = i / D;
  const float a = la[row], bb = lb[row];
  const bool ai = (a == -INFINITY), bi = (bb == -INFINITY);
  const float mx = fmaxf(a, bb);
  float L;
  if (ai && bi) {
    L = -INFINITY;
  } else {
    L = mx + log1pf(expf(fminf(a, bb) - mx));  // logaddexp
  }
  const float wa = ai ? 0.f : expf(a - L);
  const float wb = bi ? 0.f : expf(bb - L);
  const float va = ai ? 0.f : oa[i];
  const float vb = bi ? 0.f : ob[i];
  out[i] = wa * va + wb * vb;
  if (lse && (i % D) == 0) lse[row] = L;
}

}  // namespace halo

// ===========================================================================
// C-ABI
// ===========================================================================
using namespace halo;

extern "C" size_t halo_decode_workspace_size(int n_work, int rep_t, int D) {
  return (size_t)n_work * rep_t * ((size_t)D + 2) * sizeof(float);
}

namespace {

template <int DT, int D, int REP>
int launch_decode(const DecodeParams& p, int n_work, hipStream_t st) {
  constexpr int NW = 4;
  hipLaunchKernelGGL((decode_attn_kernel<DT, D, REP, NW>), dim3(n_work), dim3(64 * NW), 0, st, p);
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}

template <int DT, int D>
int dispatch_rep(const DecodeParams& p, int rep_t, int n_work, hipStream_t st) {
  switch (rep_t) {
    case 1: return launch_decode<DT, D, 1>(p, n_work, st);
    case 2: return launch_decode<DT, D, 2>(p, n_work, st);
    case 4: return launch_decode<DT, D, 4>(p, n_work, st);
    case 8: return launch_decode<DT, D, 8>(p, n_work, st);
  }
  set_error("rep_t must be 1, 2, 4 or 8");
  return HALO_E_UNSUPPORTED;
}

template <int DT>
int dispatch_d(const DecodeParams& p, int D, int rep_t, int n_work, hipStream_t st) {
  if (D == 64) return dispatch_rep<DT, 64>(p, rep_t, n_work, st);
  if (D == 128) return dispatch_rep<DT, 128>(p, rep_t, n_work, st);
  if constexpr (DT != HALO_F32) {
    if (D == 256) return dispatch_rep<DT, 256>(p, rep_t, n_work, st);
  }
  set_error("head_dim must be 64, 128 or 256 (256 for bf16/f16 only)");
  return HALO_E_UNSUPPORTED;
}

}  // namespace

extern "C" int halo_decode_attn(const void* q, int64_t q_stride_b, int64_t q_stride_h, int dtype,
                                int B, int H, int H_kv, int D, int rep_t,
                                const halo_chunk_desc* descs, int n_desc,
                                const int32_t* work, int n_work,
                                const int32_t* group_offsets, int n_groups,
                                const int64_t* q_pos, float scale,
                                float* m, float* l, float* o, int64_t acc_stride_b, int acc_mode,
                                void* out, int out_dtype, float* lse,
                                void* workspace, size_t workspace_bytes, int32_t* counters,
                                void* stream) {
  HALO_CHECK_ARG(q && descs && work && group_offsets && counters, "null pointer argument");
  HALO_CHECK_ARG(B > 0 && H > 0 && H_kv > 0 && H % H_kv == 0, "need H % H_kv == 0 and positive sizes");
  HALO_CHECK_ARG(dtype == HALO_F32 || dtype == HALO_BF16 || dtype == HALO_F16, "bad dtype");
  HALO_CHECK_ARG(out == nullptr || out_dtype == HALO_F32 || out_dtype == HALO_BF16 || out_dtype == HALO_F16,
                 "bad out_dtype");
  HALO_CHECK_ARG(n_desc > 0 && n_work > 0, "empty chunk table");
  const int rep = H / H_kv;
  HALO_CHECK_ARG(rep_t == 1 || rep_t == 2 || rep_t == 4 || rep_t == 8, "rep_t must be 1, 2, 4 or 8");
  const int n_sub = (rep + rep_t - 1) / rep_t;
  HALO_CHECK_ARG(n_groups == B * H_kv * n_sub, "n_groups must equal B*H_kv*ceil(rep/rep_t)");
  HALO_CHECK_ARG(m != nullptr || out != nullptr, "nothing to write: pass accumulators or out");
  HALO_CHECK_ARG(m == nullptr || (l != nullptr && o != nullptr), "m, l, o must be passed together");
  const size_t need = halo_decode_workspace_size(n_work, rep_t, D);
  if (workspace_bytes < need || workspace == nullptr) {
    set_error("workspace too small");
    return HALO_E_WORKSPACE;
  }
  DecodeParams p;
  p.q = q;
  p.q_stride_b = q_stride_b;
  p.q_stride_h = q_stride_h;
  p.H = H;
  p.H_kv = H_kv;
  p.rep = rep;
  p.n_sub = n_sub;
  p.descs = descs;
  p.work = work;
  p.group_offsets = group_offsets;
  p.q_pos = q_pos;
  p.scale2 = (float)((double)scale * 1.4426950408889634);
  p.m = m;
  p.l = l;
  p.o = o;
  p.acc_stride_b = acc_stride_b;
  p.acc_mode = acc_mode;
  p.out = out;
  p.out_dtype = out_dtype;
  p.lse = lse;
  p.ws_o = reinterpret_cast<float*>(workspace);
  p.ws_ml = p.ws_o + (size_t)n_work * rep_t * D;
  p.counters = counters;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (dtype) {
    case HALO_F32: return dispatch_d<HALO_F32>(p, D, rep_t, n_work, st);
    case HALO_BF16: return dispatch_d<HALO_BF16>(p, D, rep_t, n_work, st);
    default: return dispatch_d<HALO_F16>(p, D, rep_t, n_work, st);
  }
}

extern "C" int halo_finalize(const float* m, const float* l, const float* o, int B, int H, int D,
                             void* out, int out_dtype, float* lse, void* stream) {
  HALO_CHECK_ARG(m && l && o, "null accumulator");
  HALO_CHECK_ARG(B >= 0 && H >= 0 && D > 0, "bad sizes");
  const int64_t n = (int64_t)B * H * D;
  if (n == 0) return HALO_OK;
  const int threads = 256;
  const int64_t blocks = (n + threads - 1) / threads;
  hipLaunchKernelGGL(finalize_kernel, dim3((unsigned)blocks), dim3(threads), 0,
                     reinterpret_cast<hipStream_t>(stream), m, l, o, (int64_t)B * H, D, out, out_dtype, lse);
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}

extern "C" int halo_lse_merge(const float* out_a, const float* lse_a, const float* out_b,
                              const float* lse_b, int64_t n, int D, float* out, float* lse,
                              void* stream) {
  HALO_CHECK_ARG(out_a && lse_a && out_b && lse_b && out, "null pointer");
  HALO_CHECK_ARG(n >= 0 && D > 0, "bad sizes");
  if (n == 0) return HALO_OK;
  const int threads = 256;
  const int64_t blocks = (n * D + threads - 1) / threads;
  hipLaunchKernelGGL(lse_merge_kernel, dim3((unsigned)blocks), dim3(threads), 0,
                     reinterpret_cast<hipStream_t>(stream), out_a, lse_a, out_b, lse_b, n, D, out, lse);
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}
