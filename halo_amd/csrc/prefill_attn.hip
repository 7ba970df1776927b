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
// Work split: the query rows of one KV head's group are flattened position-
// major, row r = (position r / rep, head r % rep), and one workgroup (8 waves)
// takes 256 consecutive flattened rows, so every K/V tile staged in LDS serves
// all query heads of the group.  Each wave owns 32 rows = the 32 columns of
// v_mfma_f32_32x32x16; a lane owns one query row, so the running max and sum
// are per-lane scalars.
//   scores  S^T[key][q]  = sum_d K[key][d] Q[q][d]          (A = K tile, B = Q^T)
//   output  O^T[d][q]   += sum_key V^T[d][key] P^T[key][q]   (A = V^T, B = P^T)
// S^T's accumulator gives lane (q, half h) the keys 8i + 4h + j of a 32-key
// block; the PV step over 16 keys takes, per lane half, the keys
// {4h + j, 8 + 4h + j} of a 16-key run, so P^T is packed from the score
// registers without any cross-lane move, and V^T is read with
// ds_read_b64_tr_b16 in the same key order.  The output's MFMA row m of
// d-block db is d = (m / 16) * D/2 + 16 db + m % 16, which spreads one
// transposed read over the whole 256-byte bank window (with the row swizzles
// below, every LDS read of the loop is bank-conflict free).
//
// Pipeline: K tiles are staged two tiles ahead and V tiles one ahead
// (LDS-DMA, each lane choosing the global piece that lands in its slot, which
// lays out the swizzles), so one barrier per 64-key tile suffices, and the
// score MFMAs of tile t+1 are issued in the same basic block as the softmax of
// tile t, which lets the matrix core and the VALU overlap within a wave.
// Workgroups of one KV group run on one XCD (they share its L2), the ones with
// the longest causal extent first.

#include <type_traits>

#include "common.hpp"

namespace halo {

namespace {

typedef __attribute__((ext_vector_type(16))) float pf32x16;

template <int DT>
struct PMfma;
template <>
struct PMfma<HALO_BF16> {
  typedef __attribute__((ext_vector_type(8))) __bf16 v8;
  __device__ static __forceinline__ pf32x16 run(const uint4& a, const uint4& b, pf32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
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
  __device__ static __forceinline__ pf32x16 run(const uint4& a, const uint4& b, pf32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
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

template <typename T>
__device__ __forceinline__ T uni(T v) {
  return __builtin_amdgcn_readfirstlane(v);
}
__device__ __forceinline__ int64_t uni64(int64_t v) {
  const uint64_t u = (uint64_t)v;
  return (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(u >> 32)) << 32) |
                   (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)u));
}
__device__ __forceinline__ const char* uniptr(const void* p) {
  return reinterpret_cast<const char*>((uintptr_t)uni64((int64_t)(uintptr_t)p));
}

// value of lane l ^ 32 next to the own value: {lanes 0-31 of v, lanes 32-63 of v}
__device__ __forceinline__ float half_max(float v) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float half_sum(float v) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i%4
// of the 8-byte reads of lanes 4e + i/4 (e = 0..3).
typedef short pv4i16_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 pf_tr16(const char* p) {
  const pv4i16_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) pv4i16_t*)(__attribute__((address_space(3))) char*)(p));
  return __builtin_bit_cast(uint2, r);
}

}  // namespace

struct PrefillParams {
  const void* q;
  int64_t q_stride_b, q_stride_h, q_stride_t;
  int B, H, H_kv, rep, T_q, n_wg, n_units;
  const int64_t* q_start;  // [B] global position of query row 0
  const halo_chunk_desc* descs;
  int n_desc;
  float scale2;
  void* out;
  int64_t o_stride_b, o_stride_h, o_stride_t;
  int out_dtype, out_vec4;
  float* lse;  // (B, H, T_q) contiguous, or null
};

constexpr int kPfNW = 8;             // waves per workgroup
constexpr int kPfRows = kPfNW * 32;  // flattened query rows per workgroup
constexpr int kPfBK = 64;            // key rows per LDS tile
// Slack (log2 units) by which a tile's max may exceed the running max before
// the running max moves: probabilities stay below 2^8 and the accumulators are
// rescaled only when the max really moves; out = o / l and lse = m + log2(l)
// use the same m, so the result does not depend on when m moved.
constexpr float kPfLazyMax = 8.0f;

// 16-byte piece swizzles of a staged row (RB = row bytes).  K: the 16 rows of
// one b128 read pass land on distinct banks.  V: the 4 rows x 2 d-halves of
// one transposed read pass land on distinct 32-byte bank windows.
template <int RB>
__device__ __forceinline__ int pf_kswz(int r) {
  return RB == 256 ? (r & 15) : ((r >> 1) & 7);
}
template <int RB>
__device__ __forceinline__ int pf_vswz(int r) {
  return RB == 256 ? 2 * (r & 3) : 2 * ((r >> 1) & 1);
}

// One chunk tile of the walk, all fields wave-uniform.
struct PfTile {
  const char* kb;  // K rows of this (batch, KV head), row 0 of the chunk
  const char* vb;
  int64_t kst, vst;  // row strides in bytes
  int64_t cstart;
  int ci, kt, rows, causal;
  bool valid;
};

template <int DT, int D>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) prefill_attn_kernel(PrefillParams P) {
  constexpr int KS = D / 16;               // d-steps of the score MFMA
  constexpr int DB = D / 32;               // d-blocks of the output MFMA
  constexpr int RB = D * 2;                // row bytes
  constexpr int SL = RB / 16;              // 16-byte pieces per row
  constexpr int TB = kPfBK * RB;           // one K or V tile in LDS
  constexpr int RPI = 1024 / RB;           // rows per 1 KiB LDS-DMA instruction
  constexpr int BPW = TB / 1024 / kPfNW;   // 1 KiB DMA blocks per wave per tile
  static_assert(BPW >= 1 && TB % (1024 * kPfNW) == 0, "prefill tile shape");
  // K stages 0/1 and V stages 0/1 as four LDS objects: the stage a step
  // reads is a compile-time constant in each of the two unrolled steps, so
  // the compiler can tell the tiles being filled by LDS-DMA from the ones
  // being read and does not wait for the fills before every read
  __shared__ __attribute__((aligned(16))) char sK0[TB], sK1[TB], sV0[TB], sV1[TB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = uni(tid >> 6);
  const int qc = lane & 31, hh = lane >> 5;

  // XCD-aware unit order: the units of one XCD (blockIdx % 8) are a
  // contiguous run, so the workgroups of one KV group share an L2; within a
  // group the workgroups with the most keys start first.
  int unit = blockIdx.x;
  if ((P.n_units & 7) == 0) unit = (blockIdx.x & 7) * (P.n_units >> 3) + (blockIdx.x >> 3);
  const int grp = unit / P.n_wg;
  const int wg = P.n_wg - 1 - unit % P.n_wg;
  const int b = grp / P.H_kv, h_kv = grp % P.H_kv;
  const int RG = P.T_q * P.rep;  // flattened rows of the group
  const int wrow0 = wg * kPfRows;
  const int64_t qs = P.q_start[b];
  const int64_t wg_qmax = qs + (min(wrow0 + kPfRows, RG) - 1) / P.rep;
  const int64_t wave_qmin = qs + min(wrow0 + wave * 32, RG - 1) / P.rep;

  // this lane's query row
  const int r_lane = wrow0 + wave * 32 + qc;
  const bool row_ok = r_lane < RG;
  const int r_eff = row_ok ? r_lane : RG - 1;
  const int pos = r_eff / P.rep;
  const int h = h_kv * P.rep + (r_eff - pos * P.rep);
  const int64_t qpos = qs + pos;

  // Q^T as B operands: lane (q, half) holds d = 16 s + 8 half .. +8
  uint4 qb[KS];
  {
    const char* qrow = reinterpret_cast<const char*>(P.q) +
                       ((int64_t)b * P.q_stride_b + (int64_t)h * P.q_stride_h + (int64_t)pos * P.q_stride_t) * 2;
#pragma unroll
    for (int s = 0; s < KS; ++s) qb[s] = *reinterpret_cast<const uint4*>(qrow + (s * 16 + hh * 8) * 2);
  }

  // ---- the (chunk, 64-row tile) walk
  auto open_chunk = [&](int from, PfTile& t) {
    t.valid = false;
    for (int c = uni(from); c < P.n_desc; ++c) {
      const halo_chunk_desc* dp = P.descs + c;
      const int batch = uni(dp->batch);
      if (batch >= 0 && batch != b) continue;
      const int causal = uni(dp->flags) & HALO_CHUNK_CAUSAL;
      const int64_t cstart = uni64(dp->chunk_start);
      int rows = uni(dp->T_c);
      if (causal) rows = (int)max<int64_t>(0, min<int64_t>(rows, wg_qmax - cstart + 1));
      if (rows <= 0) continue;
      const int64_t ksb = uni64(dp->k_stride_b), ksh = uni64(dp->k_stride_h);
      const int64_t vsb = uni64(dp->v_stride_b), vsh = uni64(dp->v_stride_h);
      t.kb = uniptr(dp->k) + ((batch < 0 ? (int64_t)b * ksb : 0) + (int64_t)h_kv * ksh) * 2;
      t.vb = uniptr(dp->v) + ((batch < 0 ? (int64_t)b * vsb : 0) + (int64_t)h_kv * vsh) * 2;
      t.kst = uni64(dp->k_stride_t) * 2;
      t.vst = uni64(dp->v_stride_t) * 2;
      t.cstart = cstart;
      t.rows = rows;
      t.kt = 0;
      t.causal = causal;
      t.ci = c;
      t.valid = true;
      return;
    }
  };
  auto next_tile = [&](PfTile& t) {
    if (!t.valid) return;
    t.kt += kPfBK;
    if (t.kt >= t.rows) open_chunk(t.ci + 1, t);
  };
  // LDS-DMA of one tile's K (or V) rows [kt, kt+64) into `st`: each 1 KiB
  // instruction of a wave fills RPI consecutive rows, lane l the 16-byte slot
  // l % SL of row l / SL, reading the global piece that belongs there.  Rows
  // past the chunk read as zeros (buffer range check).
  auto issue = [&](const char* base, int64_t rst, int kt, int rows, char* st, bool is_v) {
    const __amdgpu_buffer_rsrc_t rs = prsrc(base + (int64_t)kt * rst, (int64_t)(rows - kt) * rst);
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
      const int blk = wave * BPW + j;
      const int r = blk * RPI + lane / SL, slot = lane % SL;
      const int piece = slot ^ (is_v ? pf_vswz<RB>(r) : pf_kswz<RB>(r));
      const int off = (int)(r * rst) + (piece << 4);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(st + blk * 1024), 16,
                                               off, 0, 0, 0);
    }
  };

  // LDS operand reads.  K (A of the score MFMA): step i = (d-step i/2, key
  // block i%2).  V^T (A of the PV MFMA): step i = (key step i/DB, d-block
  // i%DB), two transposed reads.
  auto kread = [&](const char* sk, int i) -> uint4 {
    const int kr = (i & 1) * 32 + qc;
    return *reinterpret_cast<const uint4*>(sk + kr * RB + (((2 * (i >> 1) + hh) ^ pf_kswz<RB>(kr)) << 4));
  };
  const int vG = lane >> 4, vei = (lane & 15) >> 2, vai = lane & 3;
  auto vread = [&](const char* sv, int i) -> uint4 {
    const int t = i / DB, db = i % DB;
    const int rlo = 16 * t + 4 * (vG >> 1) + vei, rhi = rlo + 8;
    const int byte = ((vG & 1) * (D / 2) + 16 * db + 4 * vai) * 2;
    const int pc = byte >> 4, wi = byte & 15;
    const uint2 a0 = pf_tr16(sv + rlo * RB + ((pc ^ pf_vswz<RB>(rlo)) << 4) + wi);
    const uint2 a1 = pf_tr16(sv + rhi * RB + ((pc ^ pf_vswz<RB>(rhi)) << 4) + wi);
    return make_uint4(a0.x, a0.y, a1.x, a1.y);
  };
  constexpr int NKS = 2 * KS;  // score MFMAs per tile
  constexpr int NPV = 4 * DB;  // PV MFMAs per tile
  constexpr int RING = 4;      // operand reads in flight ahead of their MFMA
  // scores of one staged K tile (prologue only; the loop interleaves them)
  auto scores = [&](const char* sk, pf32x16* S) {
#pragma unroll
    for (int i = 0; i < NKS; ++i) S[i & 1] = PMfma<DT>::run(kread(sk, i), qb[i >> 1], i < 2 ? pf32x16{} : S[i & 1]);
  };

  pf32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = pf32x16{};
  float m_run = -INFINITY, l_run = 0.f;

  PfTile c0, c1, c2;
  open_chunk(0, c0);
  c1 = c0;
  next_tile(c1);
  c2 = c1;
  next_tile(c2);
  if (c0.valid) {
    issue(c0.kb, c0.kst, c0.kt, c0.rows, sK0, false);
    issue(c0.vb, c0.vst, c0.kt, c0.rows, sV0, true);
  }
  if (c1.valid) issue(c1.kb, c1.kst, c1.kt, c1.rows, sK1, false);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // Masks tile `c`'s scores: keys at or past `lim` (tile-relative) for this
  // lane are the chunk end, and for a causal chunk the lane's own position.
  auto mask_tile = [&](const PfTile& c, pf32x16* S) {
    const bool masked = c.kt + kPfBK > c.rows || (c.causal && c.cstart + c.kt + kPfBK - 1 > wave_qmin);
    if (masked) {
      int lim = min(c.rows - c.kt, kPfBK);
      if (c.causal) {
        const int64_t dq = qpos - (c.cstart + c.kt) + 1;  // keys this lane may see
        lim = dq < (int64_t)lim ? (int)max<int64_t>(dq, -1) : lim;
      }
      lim -= 4 * hh;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          S[kb][e] = (kb * 32 + 8 * (e >> 2) + (e & 3)) < lim ? S[kb][e] : -INFINITY;
    }
  };
  // The running max takes tile S's max into account (it moves only when the
  // tile's max exceeds it by the slack); returns whether it moved.
  float ms = 0.f;  // exponent offset of the current tile: m_run, or 0 while m_run is -inf
  auto tile_max = [](const pf32x16* S) -> float {
    float bm = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) bm = fmaxf(bm, S[kb][e]);
    return bm;
  };
  auto take_max = [&](float bm, float& m_old) -> bool {
    bm = half_max(bm);
    const float bms = bm * P.scale2;  // scores scale after the max (scale > 0)
    m_old = m_run;
    const float m_new = (bms > m_old + kPfLazyMax) ? bms : m_old;
    m_run = m_new;
    ms = (m_new == -INFINITY) ? 0.f : m_new;
    return m_new != m_old;
  };

  pf32x16 S[2];
  if (c0.valid) {
    scores(sK0, S);
    mask_tile(c0, S);
    float m_old;
    take_max(tile_max(S), m_old);  // o and l are still zero: nothing to rescale
  }
  __syncthreads();  // K stage 0 is refilled below

  // One 64-key tile t (its scores S masked, the running max already updated
  // for it): stage K(t+2) and V(t+1); block 1 = score MFMAs of tile t+1 with
  // the exponentials of tile t between them; mask tile t+1 if it crosses a
  // chunk end or the diagonal (rare); block 2 = O += V(t) P(t) with tile
  // t+1's max between the MFMAs; rescale O and l if the max moved (rare).
  // The loop alternates the roles of the two score arrays instead of copying.
  auto step = [&](auto stage_c, pf32x16* S, pf32x16* Sn) {
    constexpr int stage = decltype(stage_c)::value;
    char* const kcur = stage ? sK1 : sK0;  // K(t), scored; receives K(t+2)
    char* const knxt = stage ? sK0 : sK1;  // K(t+1); stale past the last tile, never used then
    char* const vcur = stage ? sV1 : sV0;  // V(t)
    char* const vnxt = stage ? sV0 : sV1;  // receives V(t+1)
    if (c2.valid) issue(c2.kb, c2.kst, c2.kt, c2.rows, kcur, false);
    if (c1.valid) issue(c1.vb, c1.vst, c1.kt, c1.rows, vnxt, true);

    // Both blocks are issued in source order (a scheduling barrier after
    // each MFMA step): every MFMA's operand was read RING steps earlier, and
    // the VALU work is spread evenly between the MFMAs.
    uint4 kr[RING], vr[RING];
#pragma unroll
    for (int i = 0; i < RING; ++i) kr[i] = kread(knxt, i);
    // P^T operands: key step 2 kb + u holds keys 16u + {4h + j, 8 + 4h + j} of block kb
    constexpr int EPM = 32 / NKS;  // exponentials per score MFMA
    uint4 pb[4];
    float p[8];
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < NKS; ++i) {
      Sn[i & 1] = PMfma<DT>::run(kr[i % RING], qb[i >> 1], i < 2 ? pf32x16{} : Sn[i & 1]);
      if (i + RING < NKS) kr[i % RING] = kread(knxt, i + RING);
      const int st = (i * EPM) >> 3, kb = st >> 1, u = st & 1;
#pragma unroll
      for (int x = 0; x < EPM; ++x) {
        const int e = (i * EPM + x) & 7;
        p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(S[kb][8 * u + e], P.scale2, -ms));
        psum += p[e];
      }
      // keeps the row sum's additions next to their exponentials (sunk
      // below the block they form one serial chain with the matrix pipe idle)
      asm volatile("" : "+v"(psum));
      if (((i + 1) * EPM & 7) == 0) {
        pb[st] = make_uint4(PMfma<DT>::pack(p[0], p[1]), PMfma<DT>::pack(p[2], p[3]), PMfma<DT>::pack(p[4], p[5]),
                            PMfma<DT>::pack(p[6], p[7]));
        // keeps the exponentials here (they would otherwise sink to block 2)
        asm volatile("" : "+v"(pb[st].x), "+v"(pb[st].y), "+v"(pb[st].z), "+v"(pb[st].w));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    l_run += psum;
    if (c1.valid) mask_tile(c1, Sn);

    // block 2: O += V(t) P(t), with tile t+1's max between the MFMAs
    constexpr int MPM = 32 / NPV;  // score elements folded into the max per PV MFMA
    float bm = -INFINITY;
#pragma unroll
    for (int i = 0; i < RING; ++i) vr[i] = vread(vcur, i);
#pragma unroll
    for (int i = 0; i < NPV; ++i) {
      o[i % DB] = PMfma<DT>::run(vr[i % RING], pb[i / DB], o[i % DB]);
      if (i + RING < NPV) vr[i % RING] = vread(vcur, i + RING);
#pragma unroll
      for (int x = 0; x < MPM; ++x) {
        const int e = i * MPM + x;
        bm = fmaxf(bm, Sn[e >> 4][e & 15]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // past the last tile the scores came from a stale (or never filled)
    // stage: no max to take from them
    if (!c1.valid) bm = -INFINITY;
    float m_old;
    const bool moved = take_max(bm, m_old);
    if (__builtin_amdgcn_read_exec() & __ballot(moved)) {
      const float alpha = __builtin_amdgcn_exp2f(m_old - m_run);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[db] *= alpha;
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of K(t+2) and V(t+1) have landed
    __syncthreads();                // every wave's have; tile t's stages are free
    c0 = c1;
    c1 = c2;
    next_tile(c2);
  };
  pf32x16 S2[2];
  while (c0.valid) {
    step(std::integral_constant<int, 0>(), S, S2);
    if (!c0.valid) break;
    step(std::integral_constant<int, 1>(), S2, S);
  }

  // normalise and store: lane holds O^T[d][q] for MFMA rows m = 8i + 4h + j
  const float lt = half_sum(l_run);
  if (row_ok) {
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const int64_t ob = (int64_t)b * P.o_stride_b + (int64_t)h * P.o_stride_h + (int64_t)pos * P.o_stride_t;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 8 * i + 4 * hh;
        const int d = (m >> 4) * (D / 2) + 16 * db + (m & 15);
        float v4[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v4[j] = o[db][4 * i + j] * inv;
        if (P.out_vec4) {
          store_elem4(P.out, ob + d, P.out_dtype, v4);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) store_elem(P.out, ob + d + j, P.out_dtype, v4[j]);
        }
      }
    if (P.lse != nullptr && hh == 0)
      P.lse[((int64_t)b * P.H + h) * P.T_q + pos] = lt > 0.f ? (m_run + log2f(lt)) * kLn2 : -INFINITY;
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
  const int64_t rows = (int64_t)T_q * p.rep;
  p.n_wg = (int)((rows + kPfRows - 1) / kPfRows);
  const int64_t units = (int64_t)B * H_kv * p.n_wg;
  HALO_CHECK_ARG(rows < (1ll << 31) && units < (1ll << 31), "too many query rows");
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
  // 4-element stores need every row start aligned to 4 elements' bytes
  const int64_t ea = out_dtype == HALO_F32 ? 16 : 8;
  const int64_t es = elem_size(out_dtype);
  p.out_vec4 = reinterpret_cast<uintptr_t>(out) % ea == 0 && (out_stride_b * es) % ea == 0 &&
               (out_stride_h * es) % ea == 0 && (out_stride_t * es) % ea == 0;
  p.lse = lse;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(p.n_units), block(kPfNW * 64);
  if (dtype == HALO_BF16) {
    if (D == 128) hipLaunchKernelGGL((prefill_attn_kernel<HALO_BF16, 128>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((prefill_attn_kernel<HALO_BF16, 64>), grid, block, 0, st, p);
  } else {
    if (D == 128) hipLaunchKernelGGL((prefill_attn_kernel<HALO_F16, 128>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((prefill_attn_kernel<HALO_F16, 64>), grid, block, 0, st, p);
  }
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}
