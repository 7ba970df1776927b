// Split-K GQA decode attention over a KV chunk table with a log-sum-exp
// merge (gfx950, wave64).
//
// Reference semantics: halo/triton_chunked.py:46-138 (per-chunk online
// softmax update), :195-207 (finalize), halo/kv_cache_chunked.py:194-276
// (per-chunk attention + LSE merge with -inf guards).
//
// Two kernels per call:
//   decode_attn_kernel  one workgroup per work item {chunk, query-head group,
//     rows [t0, t1)}.  A query-head group is (b, h_kv, sub): the rep_t query
//     heads sharing KV head h_kv, so every K/V row is read from HBM once per
//     group (the reference runs one program per query head and rereads K/V
//     rep times, halo/triton_chunked.py:69-73,179).  Each of the 4 waves walks
//     its slice of rows in tiles; K/V come in with raw buffer loads (1 KiB per
//     instruction, rows past the slice read as zero by the hardware range
//     check), K is transposed through LDS so each lane group scores one query
//     head, the online softmax runs in fp32 in the log2 domain with DPP
//     lane-group reductions, and P.V pairs rows into v_dot2 operands.  Each
//     workgroup writes one partial (m, l, o) with plain stores.
//   decode_merge_kernel  one workgroup per query-head group merges the
//     group's partials in work order (deterministic) with the caller's
//     accumulators.  Splitting the merge into its own launch replaces a
//     device-scope release/acquire per workgroup (an L2 write-back on every
//     XCD) with the ordering the kernel boundary already provides.

#include "common.hpp"

namespace halo {

constexpr int kWorkInts = 8;  // work record: desc, group, t0, t1, partial slot, 3 x pad

struct MergeParams {
  const int32_t* group_offsets;  // NULL: group g owns slots [g * per_group, (g + 1) * per_group)
  int per_group;
  int H, H_kv, rep, n_sub;
  float* m;
  float* l;
  float* o;
  int64_t acc_stride_b;  // elements between batch rows of m/l (H); o uses *D
  int acc_mode;
  void* out;
  int out_dtype;
  int out_vec;  // out is aligned for 4-element vector stores
  float* lse;
  const float* ws_o;
  const float* ws_ml;
};

struct DecodeParams {
  const void* q;
  int64_t q_stride_b, q_stride_h;
  int B, H, H_kv, rep, n_sub;
  const halo_chunk_desc* descs;
  const int32_t* work;
  int n_work;
  const int64_t* q_pos;
  float scale2;  // scale * log2(e)
  int q_aligned;  // q rows 16-byte aligned: stage them with 16-byte loads
  float* ws_o;   // [n_work][REP][D]  per-item partial o (unnormalised)
  float* ws_ml;  // [n_work][REP][2]  per-item (m in log2 units, l)
  int sel_on;     // fused chunk selection (halo_decode_attn_tiered)
  int sel_wide;   // the selection needs the wide form (more than 64 candidates or 512 triples)
  float inv_rep;  // fp32(1/rep): the GQA query-mean factor
  halo_select_cfg sel;
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

// ---------------------------------------------------------------------------
// Lane-group reductions over LPH consecutive lanes with DPP (no LDS traffic).
// LPH = 8: quad swaps + half-row mirror; LPH >= 16: full 16-lane row rotations
// (groups of 32 or 64 lanes are finished with readlane by the caller).
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int LPH>
__device__ __forceinline__ float group_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));  // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f<0x4E>(v));  // quad_perm [2,3,0,1]
  if constexpr (LPH == 8) {
    v = fmaxf(v, dpp_f<0x141>(v));  // row_half_mirror
  } else {
    v = fmaxf(v, dpp_f<0x124>(v));  // row_ror:4
    v = fmaxf(v, dpp_f<0x128>(v));  // row_ror:8
  }
  return v;
}
template <int LPH>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  if constexpr (LPH == 8) {
    v += dpp_f<0x141>(v);
  } else {
    v += dpp_f<0x124>(v);
    v += dpp_f<0x128>(v);
  }
  return v;
}
// Value of head h's group after group_max/group_sum: the group's row(s) are
// combined from lanes h*LPH + 16k with readlane (uniform result).
template <int LPH, bool MAX>
__device__ __forceinline__ float head_value(float v, int h) {
  float r = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), h * LPH));
#pragma unroll
  for (int k = 1; k < (LPH > 16 ? LPH / 16 : 1); ++k) {
    const float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), h * LPH + 16 * k));
    r = MAX ? fmaxf(r, x) : r + x;
  }
  return r;
}

// K/V rows are read once per launch: non-temporal loads (cache policy NT)
// keep them from evicting the small, reused data (work list, descriptors,
// page means, q) out of L2 and the last-level cache.
constexpr int kCachePolicyNT = 2;
__device__ __forceinline__ uint4 buf_ld16(__amdgpu_buffer_rsrc_t r, int voff) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, kCachePolicyNT));
}
// Buffer descriptor over [base, base + bytes).  base and bytes are
// wave-uniform at every call site; reading them through readfirstlane puts
// the descriptor in scalar registers, so each load is one instruction (a
// descriptor the compiler cannot prove uniform turns every load into a
// readfirstlane loop and its waits into vmcnt(0)).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const char* base, int64_t bytes) {
  const int nrec = bytes <= 0 ? 0 : (bytes > 0x7fffffffLL ? 0x7fffffff : (int)bytes);
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  char* ub = reinterpret_cast<char*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(ub, 0, __builtin_amdgcn_readfirstlane(nrec), 0x00020000);
}

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;
typedef __attribute__((ext_vector_type(4))) float f32x4;

// o[h][e] += p_a[h] * va[e] + p_b[h] * vb[e] for two rows whose 16-byte
// pieces are va, vb.  bf16/f16: rows are paired into dot2 operands with
// v_perm (p rounded to the K/V dtype); fp32: two fused multiply-adds.
template <int DT, int REP, int EP>
__device__ __forceinline__ void pv_pair(const uint4& va, const uint4& vb, const float* pa, const float* pb,
                                        float (&o)[REP][EP]) {
  if constexpr (DT == HALO_F32) {
    float fa[4], fb[4];
    Elem<HALO_F32>::unpack(va, fa);
    Elem<HALO_F32>::unpack(vb, fb);
#pragma unroll
    for (int r = 0; r < REP; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) o[r][e] = fmaf(pb[r], fb[e], fmaf(pa[r], fa[e], o[r][e]));
  } else {
    const uint32_t wa[4] = {va.x, va.y, va.z, va.w};
    const uint32_t wb[4] = {vb.x, vb.y, vb.z, vb.w};
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      lo[w] = __builtin_amdgcn_perm(wb[w], wa[w], 0x05040100u);  // (a.elem 2w, b.elem 2w)
      hi[w] = __builtin_amdgcn_perm(wb[w], wa[w], 0x07060302u);  // (a.elem 2w+1, b.elem 2w+1)
    }
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      if constexpr (DT == HALO_BF16) {
        const bf16x2_t pp = {(__bf16)pa[r], (__bf16)pb[r]};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          o[r][2 * w] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, lo[w]), pp, o[r][2 * w], false);
          o[r][2 * w + 1] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, hi[w]), pp, o[r][2 * w + 1], false);
        }
      } else {
        const f16x2_t pp = {(_Float16)pa[r], (_Float16)pb[r]};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          o[r][2 * w] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, lo[w]), pp, o[r][2 * w], false);
          o[r][2 * w + 1] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, hi[w]), pp, o[r][2 * w + 1], false);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Fused chunk selection (selection-slot workgroups only): every global load
// is issued before the first wait, so the selection costs one memory round
// trip; workgroups the launch marks as leading slot items issue those loads
// before reading their work record.
// ---------------------------------------------------------------------------
// Candidates and (chunk, row, KV head) triples one fused selection takes:
// the narrow form (64 and 512) serves most layers; the wide form (128 and
// 768: two ranking waves, more descriptor words per thread, 16-bit K/V only)
// is a kernel of its own, so layers within the narrow limits do not carry
// its costs.
constexpr int kSelMaxColdNarrow = 64, kSelMaxTriplesNarrow = 512;
constexpr int kSelMaxColdWide = 128, kSelMaxTriplesWide = 768;
static_assert(sizeof(halo_chunk_desc) % 8 == 0, "descriptors are copied as 8-byte words");
constexpr int kSelMaxQbar = 2048;
constexpr int kSelQbarLds = kSelMaxQbar + 4 * 64;  // padded rows: at most 2048 / 64 rows of +4 floats
constexpr int kSelMaxSlots = 64;  // HBM staging slots per selection
// LDS of the selection: q-bar rows, dot products, scores, picks, then the
// candidate descriptors, the staging-slot descriptors right after them (so
// entry max_cold + r of the combined table is slot r) and the residency.
template <bool WIDE>
struct SelCap {
  static constexpr int max_cold = WIDE ? kSelMaxColdWide : kSelMaxColdNarrow;
  static constexpr int tpt = (WIDE ? kSelMaxTriplesWide : kSelMaxTriplesNarrow) / 256;  // triples per thread
  static constexpr int cat_off = kSelQbarLds * 4 + (tpt + 3) * 256 * 4;
  static constexpr int bytes = cat_off + (max_cold + kSelMaxSlots) * (int)sizeof(halo_chunk_desc) + max_cold * 4;
};
static_assert(sizeof(halo_select_cfg) == 128, "halo_select_cfg layout");

__device__ __forceinline__ halo_chunk_desc uniform_desc(const halo_chunk_desc& d) {
  halo_chunk_desc u;
  auto rf64 = [](int64_t x) {
    const uint64_t ux = (uint64_t)x;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)ux);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(ux >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
  };
  u.k = reinterpret_cast<const void*>(rf64(reinterpret_cast<int64_t>(d.k)));
  u.v = reinterpret_cast<const void*>(rf64(reinterpret_cast<int64_t>(d.v)));
  u.k_stride_b = rf64(d.k_stride_b);
  u.k_stride_h = rf64(d.k_stride_h);
  u.k_stride_t = rf64(d.k_stride_t);
  u.v_stride_b = rf64(d.v_stride_b);
  u.v_stride_h = rf64(d.v_stride_h);
  u.v_stride_t = rf64(d.v_stride_t);
  u.chunk_start = rf64(d.chunk_start);
  u.T_c = __builtin_amdgcn_readfirstlane(d.T_c);
  u.flags = __builtin_amdgcn_readfirstlane(d.flags);
  u.batch = __builtin_amdgcn_readfirstlane(d.batch);
  u.reserved = 0;
  return u;
}

template <int DT, int D, int NT, bool WIDE>
struct Selector {
  using Cap = SelCap<WIDE>;
  using E = Elem<DT>;
  static constexpr int EP = E::per16;
  static constexpr int PIECES = D / EP;                               // 16-byte pieces per row
  static constexpr int G = D / 16;                                    // dot-product slices
  static_assert(D % 16 == 0, "dot-product slices");
  static constexpr int QP = (kSelMaxQbar / EP + NT - 1) / NT;         // q-bar pieces per thread
  static constexpr int DW2 = (int)sizeof(halo_chunk_desc) / 8;        // 8-byte words per descriptor
  static constexpr int CW = (Cap::max_cold * DW2 + NT - 1) / NT;      // descriptor words per thread
  static constexpr int QB = EP == 8 ? 8 : 4;                          // query heads summed per load batch (LDS path)
  static constexpr int QS = D + 4;                                    // q-bar row stride in LDS (floats)
  // Dot products are cut into units: unit u = (triple t = u / G, slice
  // s = u % G), the 16 elements of pieces s, s + G, ... of one page-mean
  // row.  The G lanes of a triple sit side by side in one wave, so a load
  // instruction reads whole 128-byte runs of rows and the pairwise tree over
  // slices is a butterfly inside the lane group.
  static constexpr int PPS = 16 / EP;                                 // pieces per slice
  static constexpr int KU = EP == 8 ? 6 : 3;                          // units per thread loaded up front
  static_assert((G & (G - 1)) == 0 && G <= kWave, "slices per row");
  uint4 kb[KU][PPS];          // page-mean pieces of this thread's first KU units
  uint2 cw[CW];               // this thread's share of the candidate descriptors
  uint2 sw[CW];               // ... and of the staging-slot descriptors
  int rres;                   // residency of candidate tid (tid < n), -1 without staging
  int staged_slot;            // after finish(): staging slot of this slot's chunk, -1 when read in place
  int wa_in;                  // the launch's write-allocate slot (-1: none)
  int wa_slot;                // after finish(): slot this item writes its in-place rows into, -1: none
  // q pieces loaded up front, 8 x 16 bytes: per lane (qlane) the PPS pieces
  // of its own slice for the first QL query heads (qv[j * QL + h]), else the
  // first QB heads of the thread's share of the LDS-staged q-bar pieces
  // (qv[k * QB + j]); later heads are read where they are summed
  static constexpr int QL = 8 / PPS;
  static_assert(QP * QB == 8, "q pieces loaded up front");
  uint4 qv[8];
  int n, kk, rows, b0, sel, nrh, triples;
  // Every unit of a lane has the same (row, KV head, slice) when the lane
  // groups of one unit batch (NT / G triples) cover whole multiples of nrh:
  // the lane then forms its q-bar slice in registers (no LDS stage).
  bool qlane;

  __device__ __forceinline__ const char* km_row(const halo_select_cfg& S, int t, int H_kv) const {
    const int i = t / nrh, rh = t % nrh;
    return reinterpret_cast<const char*>(S.kmean) +
           ((int64_t)(b0 + rh / H_kv) * S.km_stride_b + (int64_t)(rh % H_kv) * S.km_stride_h +
            (int64_t)i * S.km_stride_p) * E::size;
  }

  // Issue every global load of the selection (no waits): page-mean rows,
  // candidate descriptors, the first batch of query pieces.
  __device__ __forceinline__ void issue(const DecodeParams& P, int b) {
    const halo_select_cfg& S = P.sel;
    const int tid = threadIdx.x;
    rows = S.per_row ? 1 : P.B;
    b0 = S.per_row ? b : 0;
    sel = S.per_row ? b : 0;
    n = __builtin_amdgcn_readfirstlane(S.n_cold_per_sel ? min(S.n_cold_per_sel[sel], S.n_cold) : S.n_cold);
    kk = min(S.top_k, n);
    nrh = rows * P.H_kv;
    triples = n * nrh;
#pragma unroll
    for (int k = 0; k < KU; ++k) {
      const int u = tid + k * NT;
      // past the units (or no candidates at all): a valid row, loads unused
      const int t = min(u / G, max(triples - 1, 0)), sl = u % G;
      const char* row = km_row(S, t, P.H_kv);
#pragma unroll
      for (int j = 0; j < PPS; ++j) kb[k][j] = *reinterpret_cast<const uint4*>(row + (sl + j * G) * 16);
    }
    const uint2* cat = reinterpret_cast<const uint2*>(S.catalog + (int64_t)sel * S.catalog_stride);
#pragma unroll
    for (int k = 0; k < CW; ++k) {
      const int w = tid + k * NT;
      if (w < n * DW2) cw[k] = cat[w];
    }
    rres = -1;
    wa_in = -1;
    if (S.residency != nullptr) {
      // write-allocate: 16-bit rows (the MFMA path stores them) and one selection per launch
      if (DT != HALO_F32 && S.alloc_slot != nullptr && !S.per_row) {
        const int w = __builtin_amdgcn_readfirstlane(*S.alloc_slot);
        wa_in = (w >= 0 && w < S.n_slots) ? w : -1;
      }
      if (tid < n) rres = S.residency[(int64_t)sel * S.catalog_stride + tid];
      const uint2* scat = reinterpret_cast<const uint2*>(S.slot_catalog + (int64_t)sel * S.n_slots);
#pragma unroll
      for (int k = 0; k < CW; ++k) {
        const int w = tid + k * NT;
        if (w < S.n_slots * DW2) sw[k] = scat[w];
      }
    }
    qlane = P.q_aligned && (NT / G) % nrh == 0;
    if (qlane) {
      const int rh = (tid / G) % nrh, sl = tid % G;
      const char* qrow = reinterpret_cast<const char*>(P.q) +
                         ((int64_t)(b0 + rh / P.H_kv) * P.q_stride_b + (int64_t)(rh % P.H_kv) * P.rep * P.q_stride_h) *
                             E::size;
#pragma unroll
      for (int j = 0; j < PPS; ++j)
#pragma unroll
        for (int e = 0; e < QL; ++e)
          if (e < P.rep) qv[j * QL + e] = *reinterpret_cast<const uint4*>(qrow + (int64_t)e * P.q_stride_h * E::size +
                                                                          (sl + j * G) * 16);
    } else if (P.q_aligned) {
      const int npieces = rows * P.H_kv * PIECES;
#pragma unroll
      for (int k = 0; k < QP; ++k) {
        const int pc = tid + k * NT;
        if (pc < npieces) {
          const int c = pc % PIECES, h = (pc / PIECES) % P.H_kv, r = pc / (PIECES * P.H_kv);
          const char* qrow = reinterpret_cast<const char*>(P.q) +
                             ((int64_t)(b0 + r) * P.q_stride_b + (int64_t)h * P.rep * P.q_stride_h) * E::size + c * 16;
#pragma unroll
          for (int j = 0; j < QB; ++j)
            if (j < P.rep) qv[k * QB + j] = *reinterpret_cast<const uint4*>(qrow + (int64_t)j * P.q_stride_h * E::size);
        }
      }
    }
  }

  // Same arithmetic as halo_chunk_score_topk: GQA-mean query rounded to the
  // q dtype, fp32 dot products with the page means in the scorer's fixed
  // order (products and sums rounded separately: D cut into G = D/16 slices,
  // slice s holding the 16-byte pieces s, s + G, ..., each slice summed in
  // order, then a balanced pairwise tree over the slices), max over (row, KV
  // head), rank by (score desc, index asc).  Returns the chunk index p for
  // `slot` (-1: slot past the eligible count); the chunk's catalog entry is
  // left in LDS at Cap::cat_off and staged_slot names the staging slot that
  // holds it (-1: none; its descriptor is entry Cap::max_cold + staged_slot).
  __device__ __forceinline__ int finish(const DecodeParams& P, char* smem, int slot, bool writer) {
    const halo_select_cfg& S = P.sel;
    const int tid = threadIdx.x;
    const int H_kv = P.H_kv, rep = P.rep;
    float* s_qbar = reinterpret_cast<float*>(smem);  // rows of QS floats (padded: conflict-free reads)
    float* s_dot = s_qbar + kSelQbarLds;
    float* s_sc = s_dot + Cap::tpt * 256;  // per-candidate scores for the ranking (-inf past n)
    int* s_pick = reinterpret_cast<int*>(s_dot + (Cap::tpt + 2) * 256);
    halo_chunk_desc* s_cat = reinterpret_cast<halo_chunk_desc*>(s_pick + 256);
    halo_chunk_desc* s_slot = s_cat + Cap::max_cold;
    int* s_res = reinterpret_cast<int*>(s_slot + kSelMaxSlots);
    // GQA-mean query rows: fp32 sum over the rep heads in head order, times
    // fp32(1/rep), one rounding to the q dtype (rep == 1: q itself).
    auto qround = [&](float v) __attribute__((always_inline)) {
      if (rep != 1) {
        v = opaque(v * P.inv_rep);
        v = DT == HALO_F32 ? v
            : (DT == HALO_BF16 ? __uint_as_float((uint32_t)f32_to_bf16_rne(v) << 16)
                               : f16_bits_to_f32(f32_to_f16_rne(v)));
      }
      return v;
    };
    float qs[PPS * EP];  // qlane: this lane's q-bar slice (pieces sl, sl + G, ..)
    if (qlane) {
      const int rh = (tid / G) % nrh, sl = tid % G;
      const char* qrow = reinterpret_cast<const char*>(P.q) +
                         ((int64_t)(b0 + rh / H_kv) * P.q_stride_b + (int64_t)(rh % H_kv) * rep * P.q_stride_h) *
                             E::size;
#pragma unroll
      for (int j = 0; j < PPS; ++j) {
        float acc[EP];
#pragma unroll
        for (int e = 0; e < EP; ++e) acc[e] = 0.f;
#pragma unroll
        for (int h = 0; h < QL; ++h) {
          if (h < rep) {
            float f[EP];
            E::unpack(qv[j * QL + h], f);
#pragma unroll
            for (int e = 0; e < EP; ++e) acc[e] = acc[e] + f[e];
          }
        }
        for (int h = QL; h < rep; ++h) {
          float f[EP];
          E::unpack(*reinterpret_cast<const uint4*>(qrow + (int64_t)h * P.q_stride_h * E::size + (sl + j * G) * 16), f);
#pragma unroll
          for (int e = 0; e < EP; ++e) acc[e] = acc[e] + f[e];
        }
#pragma unroll
        for (int e = 0; e < EP; ++e) qs[j * EP + e] = qround(acc[e]);
      }
    } else if (P.q_aligned) {
      const int npieces = rows * H_kv * PIECES;
#pragma unroll
      for (int k = 0; k < QP; ++k) {
        const int pc = tid + k * NT;
        if (pc >= npieces) break;
        const int c = pc % PIECES, h = (pc / PIECES) % H_kv, r = pc / (PIECES * H_kv);
        const char* qrow = reinterpret_cast<const char*>(P.q) +
                           ((int64_t)(b0 + r) * P.q_stride_b + (int64_t)h * rep * P.q_stride_h) * E::size + c * 16;
        float acc[EP];
#pragma unroll
        for (int e = 0; e < EP; ++e) acc[e] = 0.f;
#pragma unroll
        for (int j = 0; j < QB; ++j) {
          if (j < rep) {
            float f[EP];
            E::unpack(qv[k * QB + j], f);
#pragma unroll
            for (int e = 0; e < EP; ++e) acc[e] = acc[e] + f[e];
          }
        }
        for (int j0 = QB; j0 < rep; j0 += QB) {
          uint4 qx[QB];
#pragma unroll
          for (int j = 0; j < QB; ++j)
            if (j0 + j < rep) qx[j] = *reinterpret_cast<const uint4*>(qrow + (int64_t)(j0 + j) * P.q_stride_h * E::size);
#pragma unroll
          for (int j = 0; j < QB; ++j) {
            if (j0 + j < rep) {
              float f[EP];
              E::unpack(qx[j], f);
#pragma unroll
              for (int e = 0; e < EP; ++e) acc[e] = acc[e] + f[e];
            }
          }
        }
        float* dst = s_qbar + (r * H_kv + h) * QS + c * EP;
#pragma unroll
        for (int e = 0; e < EP; ++e) dst[e] = qround(acc[e]);
      }
    } else {
      for (int e = tid; e < rows * H_kv * D; e += NT) {
        const int d = e % D, h = (e / D) % H_kv, r = e / (D * H_kv);
        const int64_t qb = (int64_t)(b0 + r) * P.q_stride_b;
        float acc = 0.f;
        for (int j = 0; j < rep; ++j) acc += load_elem(P.q, qb + (int64_t)(h * rep + j) * P.q_stride_h + d, DT);
        s_qbar[(e / D) * QS + d] = qround(acc);
      }
    }
#pragma unroll
    for (int k = 0; k < CW; ++k) {
      const int w = tid + k * NT;
      if (w < n * DW2) reinterpret_cast<uint2*>(s_cat)[w] = cw[k];
    }
    if (S.residency != nullptr) {
#pragma unroll
      for (int k = 0; k < CW; ++k) {
        const int w = tid + k * NT;
        if (w < S.n_slots * DW2) reinterpret_cast<uint2*>(s_slot)[w] = sw[k];
      }
      // an entry outside [0, n_slots) reads as "not staged"
      if (tid < n) s_res[tid] = (rres >= 0 && rres < S.n_slots) ? rres : -1;
    }
    // the q-bar stage (not used by qlane) is read across waves; the catalog is
    // read after the ranking's barrier
    if (!qlane) __syncthreads();

    // Unit dot products: slice sl of triple t sums its pieces in order, each
    // product and sum rounded on its own; then the pairwise tree over the G
    // slices (part[sl] += part[sl + w], w = 1, 2, .., G/2) as a DPP
    // butterfly in the triple's lane group: after each step every lane of a
    // block holds the same sum (a + b == b + a), so the mirrors read it and
    // the association is the scorer's; lane sl == 0 holds the triple's score.
    // No LDS traffic beyond the one score per triple.
    const int n_units = triples * G;
    auto unit = [&](int u, const uint4 (&pc)[PPS]) __attribute__((always_inline)) {
      const int t = u / G, sl = u % G;
      float qf[PPS * EP];
      if (qlane) {
#pragma unroll
        for (int x = 0; x < PPS * EP; ++x) qf[x] = qs[x];
      } else {
        const float* qg = s_qbar + (t % nrh) * QS;
#pragma unroll
        for (int j = 0; j < PPS; ++j) {
          const float4* qp = reinterpret_cast<const float4*>(qg + (sl + j * G) * EP);
#pragma unroll
          for (int e4 = 0; e4 < EP / 4; ++e4) {
            const float4 v = qp[e4];
            qf[j * EP + 4 * e4] = v.x;
            qf[j * EP + 4 * e4 + 1] = v.y;
            qf[j * EP + 4 * e4 + 2] = v.z;
            qf[j * EP + 4 * e4 + 3] = v.w;
          }
        }
      }
      float a = 0.f;
#pragma unroll
      for (int j = 0; j < PPS; ++j) {
        float f[EP];
        E::unpack(pc[j], f);
#pragma unroll
        for (int e = 0; e < EP; ++e) a = __fadd_rn(a, __fmul_rn(qf[j * EP + e], f[e]));
      }
      if constexpr (G >= 2) a = __fadd_rn(a, dpp_f<0xB1>(a));   // quad_perm [1,0,3,2]: slices 2m, 2m+1
      if constexpr (G >= 4) a = __fadd_rn(a, dpp_f<0x4E>(a));   // quad_perm [2,3,0,1]: pairs of a quad
      if constexpr (G >= 8) a = __fadd_rn(a, dpp_f<0x141>(a));  // row_half_mirror: quads of 8 lanes
      if constexpr (G >= 16) a = __fadd_rn(a, dpp_f<0x140>(a)); // row_mirror: halves of 16 lanes
      if (sl == 0) s_dot[t] = a;
    };
#pragma unroll
    for (int k = 0; k < KU; ++k) {
      const int u0 = k * NT;
      if (u0 < n_units && tid + u0 < n_units) unit(tid + u0, kb[k]);
    }
    // units past the first KU per thread (more than 192 triples at G = 8):
    // one at a time in the narrow form, in the wide form batches of KU units
    // per thread, every load of a batch issued first
    if constexpr (!WIDE) {
      for (int u0 = KU * NT; u0 < n_units; u0 += NT) {
        const int u = tid + u0;
        if (u < n_units) {
          uint4 pc[PPS];
          const char* row = km_row(S, u / G, H_kv);
#pragma unroll
          for (int j = 0; j < PPS; ++j) pc[j] = *reinterpret_cast<const uint4*>(row + (u % G + j * G) * 16);
          unit(u, pc);
        }
      }
    }
    for (int u0 = KU * NT; WIDE && u0 < n_units; u0 += KU * NT) {
      uint4 pcs[KU][PPS];
#pragma unroll
      for (int k = 0; k < KU; ++k) {
        const int u = tid + u0 + k * NT;
        const int t = min(u / G, triples - 1), sl = u % G;
        const char* row = km_row(S, t, H_kv);
#pragma unroll
        for (int j = 0; j < PPS; ++j) pcs[k][j] = *reinterpret_cast<const uint4*>(row + (sl + j * G) * 16);
      }
#pragma unroll
      for (int k = 0; k < KU; ++k) {
        const int u = tid + u0 + k * NT;
        if (u < n_units) unit(u, pcs[k]);
      }
    }
    __syncthreads();
    // One lane per candidate ranks it (lane i = chunk i: one wave, or two in
    // the wide form past 64 candidates): score = max over (row, KV head),
    // NaN -> -inf; each lane counts the candidates ranked before it (score
    // desc, index asc) from broadcast LDS reads of the scores (entries past n
    // hold -inf, which never outranks); the chosen chunks are listed in
    // ascending index order with a ballot prefix count (two waves: wave 1
    // adds wave 0's count).
    auto cand_score = [&](int i) __attribute__((always_inline)) -> float {
      const float* dr = s_dot + i * nrh;
      float b4[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      int rh = 0;
      if ((nrh & 3) == 0) {  // rows 16-byte aligned: 4 scores per read, 4 reads in flight
        for (; rh + 16 <= nrh; rh += 16) {
          float4 v[4];
#pragma unroll
          for (int x = 0; x < 4; ++x) v[x] = *reinterpret_cast<const float4*>(dr + rh + 4 * x);
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            b4[0] = fmaxf(b4[0], v[x].x);
            b4[1] = fmaxf(b4[1], v[x].y);
            b4[2] = fmaxf(b4[2], v[x].z);
            b4[3] = fmaxf(b4[3], v[x].w);
          }
        }
        for (; rh < nrh; rh += 4) {
          const float4 v = *reinterpret_cast<const float4*>(dr + rh);
          b4[0] = fmaxf(b4[0], v.x);
          b4[1] = fmaxf(b4[1], v.y);
          b4[2] = fmaxf(b4[2], v.z);
          b4[3] = fmaxf(b4[3], v.w);
        }
      }
      for (; rh < nrh; ++rh) b4[0] = fmaxf(b4[0], dr[rh]);
      const float best = fmaxf(fmaxf(b4[0], b4[1]), fmaxf(b4[2], b4[3]));
      return (best != best) ? -INFINITY : best;
    };
    auto rank_of = [&](int i, float sc) __attribute__((always_inline)) -> int {
      int rank = 0;
      for (int j0 = 0; j0 < n; j0 += 16) {
        float4 v[4];
#pragma unroll
        for (int x = 0; x < 4; ++x) v[x] = *reinterpret_cast<const float4*>(s_sc + j0 + 4 * x);
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          const float sj[4] = {v[x].x, v[x].y, v[x].z, v[x].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int j = j0 + 4 * x + e;
            rank += (sj[e] > sc || (sj[e] == sc && j < i)) ? 1 : 0;
          }
        }
      }
      return rank;
    };
    auto prefix = [](uint64_t mask) __attribute__((always_inline)) {
      return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
    };
    if constexpr (!WIDE) {
      if (tid < kWave) {
        const int i = tid;
        const float sc = i < n ? cand_score(i) : -INFINITY;
        s_sc[i] = sc;
        wave_lds_fence();
        const bool chosen = i < n && rank_of(i, sc) < kk;
        const uint64_t mask = __ballot(chosen);
        if (chosen) s_pick[prefix(mask)] = i;
        if (writer && S.score_out && i < n) S.score_out[(int64_t)sel * S.n_cold + i] = sc;
      }
    } else {
      const int nw_rank = n > kWave ? 2 : 1;
      const int n_pad = nw_rank * kWave;
      int* s_cnt = s_pick + Cap::max_cold;  // wave 0's chosen count
      float sc = -INFINITY;
      if (tid < n_pad) {
        if (tid < n) sc = cand_score(tid);
        s_sc[tid] = sc;
      }
      if (nw_rank == 1) {
        wave_lds_fence();
      } else {
        __syncthreads();  // both waves' scores are in LDS
      }
      bool chosen = false;
      uint64_t mask = 0;
      if (tid < n_pad) {
        chosen = tid < n && rank_of(tid, sc) < kk;
        mask = __ballot(chosen);
        if (nw_rank == 2 && tid == 0) *s_cnt = __builtin_popcountll(mask);
      }
      if (nw_rank == 2) __syncthreads();  // wave 0's count for wave 1's positions
      if (tid < n_pad) {
        const int base = (nw_rank == 2 && tid >= kWave) ? *s_cnt : 0;
        if (chosen) s_pick[base + prefix(mask)] = tid;
        if (writer && S.score_out && tid < n) S.score_out[(int64_t)sel * S.n_cold + tid] = sc;
      }
    }
    __syncthreads();
    const bool staged = S.residency != nullptr;
    // write-allocate target: the first chosen chunk (pick order) that is not staged
    int jm = -1;
    if (staged && wa_in >= 0) {
      for (int j = 0; j < kk; ++j)
        if (s_res[s_pick[j]] < 0) {
          jm = j;
          break;
        }
    }
    jm = __builtin_amdgcn_readfirstlane(jm);
    if (writer && S.idx_out) {
      for (int j = tid; j < S.top_k; j += NT) S.idx_out[(int64_t)sel * S.top_k + j] = j < kk ? s_pick[j] : -1;
    }
    if (writer && S.res_out) {
      for (int j = tid; j < S.top_k; j += NT)
        S.res_out[(int64_t)sel * S.top_k + j] =
            (j < kk && staged) ? (j == jm ? -2 - wa_in : s_res[s_pick[j]]) : -1;
    }
    const int pick = slot < kk ? s_pick[slot] : -1;
    staged_slot = __builtin_amdgcn_readfirstlane((pick >= 0 && staged) ? s_res[pick] : -1);
    wa_slot = (slot == jm) ? wa_in : -1;
    return __builtin_amdgcn_readfirstlane(pick);
  }
};

// ---------------------------------------------------------------------------
// Work-item epilogue shared by the decode kernels: reduce each wave's o over
// the lanes that share a column slice, merge the NW wave partials (m, l, o)
// through LDS and store this item's partial at workspace slot `wslot` with
// plain stores (the merge kernel that reads them runs after this kernel).
// ---------------------------------------------------------------------------
template <int D, int REP, int NW, int SL, int EP>
__device__ __forceinline__ void write_partial(const DecodeParams& P, int wslot, float (&acc_o)[REP][EP],
                                              const float* m_run, const float* l_head, float* s_wo,
                                              float (*s_wm)[REP], float (*s_wl)[REP]) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int off = SL; off < kWave; off <<= 1)
#pragma unroll
      for (int e = 0; e < EP; ++e) acc_o[r][e] += __shfl_xor(acc_o[r][e], off, kWave);
  __syncthreads();  // every wave is out of its tile loop: LDS may be reused
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
      s_wl[wave][r] = l_head[r];
    }
  }
  __syncthreads();
  float* wso = P.ws_o + (int64_t)wslot * REP * D;
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
    P.ws_ml[((int64_t)wslot * REP + r) * 2 + 0] = M;
    P.ws_ml[((int64_t)wslot * REP + r) * 2 + 1] = acc;
  }
}

// Epilogue of the producer/consumer layout: pair j's K-wave holds (m, l)
// per head, its V-wave the o columns; the NP pair partials are merged
// through LDS into the work item's partial.
template <int D, int REP, int NP, int SL, int EP>
__device__ __forceinline__ void write_partial_pairs(const DecodeParams& P, int wslot, bool kwave, int pair,
                                                    float (&acc_o)[REP][EP], const float* m_run,
                                                    const float* l_head, float* s_wo, float (*s_wm)[REP],
                                                    float (*s_wl)[REP]) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  if (!kwave) {
#pragma unroll
    for (int r = 0; r < REP; ++r)
#pragma unroll
      for (int off = SL; off < kWave; off <<= 1)
#pragma unroll
        for (int e = 0; e < EP; ++e) acc_o[r][e] += __shfl_xor(acc_o[r][e], off, kWave);
    if (lane < SL) {
#pragma unroll
      for (int r = 0; r < REP; ++r)
#pragma unroll
        for (int e = 0; e < EP; ++e) s_wo[(pair * REP + r) * D + lane * EP + e] = acc_o[r][e];
    }
  } else if (lane == 0) {
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      s_wm[pair][r] = m_run[r];
      s_wl[pair][r] = l_head[r];
    }
  }
  __syncthreads();
  float* wso = P.ws_o + (int64_t)wslot * REP * D;
  for (int i = tid; i < REP * D; i += 64 * 2 * NP) {
    const int r = i / D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NP; ++w) M = fmaxf(M, s_wm[w][r]);
    const float Ms = (M == -INFINITY) ? 0.f : M;
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < NP; ++w) acc += __builtin_amdgcn_exp2f(s_wm[w][r] - Ms) * s_wo[w * REP * D + i];
    wso[i] = acc;
  }
  if (tid < REP) {
    const int r = tid;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NP; ++w) M = fmaxf(M, s_wm[w][r]);
    const float Ms = (M == -INFINITY) ? 0.f : M;
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < NP; ++w) acc += __builtin_amdgcn_exp2f(s_wm[w][r] - Ms) * s_wl[w][r];
    P.ws_ml[((int64_t)wslot * REP + r) * 2 + 0] = M;
    P.ws_ml[((int64_t)wslot * REP + r) * 2 + 1] = acc;
  }
}

// Same, with the V-wave's o held as MFMA accumulators: lane l owns heads
// 4*(l/16)..+4 of columns 16*db + l%16, so no cross-lane reduction is needed.
template <int D, int REP, int NP, int DB>
__device__ __forceinline__ void write_partial_pairs_mfma(const DecodeParams& P, int wslot, bool kwave, int pair,
                                                         const f32x4 (&acc)[DB], const float* m_run,
                                                         const float* l_head, float* s_wo, float (*s_wm)[REP],
                                                         float (*s_wl)[REP]) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  if (!kwave) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int h = 4 * (lane >> 4) + e;
      if (h < REP) {
#pragma unroll
        for (int db = 0; db < DB; ++db) s_wo[(pair * REP + h) * D + db * 16 + (lane & 15)] = acc[db][e];
      }
    }
  } else if (lane == 0) {
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      s_wm[pair][r] = m_run[r];
      s_wl[pair][r] = l_head[r];
    }
  }
  __syncthreads();
  float* wso = P.ws_o + (int64_t)wslot * REP * D;
  for (int i = tid; i < REP * D; i += 64 * 2 * NP) {
    const int r = i / D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NP; ++w) M = fmaxf(M, s_wm[w][r]);
    const float Ms = (M == -INFINITY) ? 0.f : M;
    float acc_o = 0.f;
#pragma unroll
    for (int w = 0; w < NP; ++w) acc_o += __builtin_amdgcn_exp2f(s_wm[w][r] - Ms) * s_wo[w * REP * D + i];
    wso[i] = acc_o;
  }
  if (tid < REP) {
    const int r = tid;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NP; ++w) M = fmaxf(M, s_wm[w][r]);
    const float Ms = (M == -INFINITY) ? 0.f : M;
    float acc_l = 0.f;
#pragma unroll
    for (int w = 0; w < NP; ++w) acc_l += __builtin_amdgcn_exp2f(s_wm[w][r] - Ms) * s_wl[w][r];
    P.ws_ml[((int64_t)wslot * REP + r) * 2 + 0] = M;
    P.ws_ml[((int64_t)wslot * REP + r) * 2 + 1] = acc_l;
  }
}

template <int DT>
__device__ __forceinline__ float from_bits16(uint16_t h) {
  if constexpr (DT == HALO_BF16) return __uint_as_float((uint32_t)h << 16);
  return f16_bits_to_f32(h);
}

template <int DT>
struct MfmaOp;
template <>
struct MfmaOp<HALO_BF16> {
  typedef __attribute__((ext_vector_type(8))) __bf16 v8;
  __device__ static __forceinline__ f32x4 run(const uint4& a, const uint4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
};
template <>
struct MfmaOp<HALO_F16> {
  typedef __attribute__((ext_vector_type(8))) _Float16 v8;
  __device__ static __forceinline__ f32x4 run(const uint4& a, const uint4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
};

// Two fp32 values rounded to the K/V dtype and packed (lower index in the
// low half): the probabilities enter the P.V product in that dtype.
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (DT == HALO_BF16) {
    const bf16x2_t v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  } else {
    const f16x2_t v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
}

// V tile in LDS: row r holds its 16-byte pieces at positions piece ^ vswz(r)
// (an even XOR, so the piece pairs the transposed reads use stay adjacent).
// Four consecutive rows (one 16-lane transposed read) then cover distinct
// 32-byte bank ranges, and rows 8 apart (the next lane group) are offset by
// a further 128 bytes.
template <int SL>
__device__ __forceinline__ int vswz(int r) {
  return (2 * (r & 3) + 8 * ((r >> 3) & 1)) & (SL - 1);
}
// K tile in LDS: row r holds piece c at position c ^ kswz(r), so the 16 rows
// one MFMA operand read touches (same piece) land on distinct bank ranges.
template <int SL>
__device__ __forceinline__ int kswz(int r) {
  return r & ((SL < 16 ? SL : 16) - 1);
}

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i%4
// of the 8-byte reads of lanes 4e + i/4 (e = 0..3).  With lane p reading 4
// consecutive columns 4(p%4).. of row p/4 of a 4-row block, lane i gets
// column i of rows 0..3: the K-major operand layout of the MFMA.
typedef short v4i16_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 lds_read_tr16(const char* p) {
  const v4i16_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16_t*)(__attribute__((address_space(3))) char*)(p));
  return __builtin_bit_cast(uint2, r);
}

// LDS bytes of the plain-row MFMA path (bf16/f16 K/V): per pair 2 p tiles
// (K/V dtype, [head][row]) and 2 rescale vectors, the pair partials, then one
// V tile per V-wave and one K tile per K-wave.  TR: rows per wave tile (0:
// 64 rows, fewer for wide rows); a smaller tile shrinks the footprint.
template <int D, int REP, int NW, int TR = 0>
struct PlainMfmaLds {
  static constexpr int RB = D * 2;
  static constexpr int SL = RB / 16;
  static constexpr int TILE = TR ? TR : (SL <= 16 ? kWave : kWave * 16 / SL);
  static constexpr int NP = NW / 2;
  static constexpr int SZ_P = NP * 2 * REP * TILE * 2;
  static constexpr int SZ_AL = (NP * 2 * REP * 4 + 15) / 16 * 16;
  static constexpr int SZ_WO = NP * REP * D * 4;
  static constexpr int SZ_VT = NP * TILE * RB;
  static constexpr int bytes = SZ_P + SZ_AL + SZ_WO + 2 * SZ_VT;
};

// One work item's rows [t0, t1) of a plain bf16/f16 K/V chunk on the matrix
// cores; writes the item's partial at workspace slot wslot.
// LDS regions of the plain-row path (sizes in PlainMfmaLds).
struct PlainLds {
  char* p;   // SZ_P: p tiles
  char* al;  // SZ_AL: rescale factors
  char* wo;  // SZ_WO: pair partials
  char* vt;  // SZ_VT: V tiles
  char* kt;  // SZ_VT: K tiles
};
template <int D, int REP, int NW, int TR = 0>
__device__ __forceinline__ PlainLds plain_lds_at(char* smem) {
  using L = PlainMfmaLds<D, REP, NW, TR>;
  return PlainLds{smem, smem + L::SZ_P, smem + L::SZ_P + L::SZ_AL, smem + L::SZ_P + L::SZ_AL + L::SZ_WO,
                  smem + L::SZ_P + L::SZ_AL + L::SZ_WO + L::SZ_VT};
}

template <int DT, int D, int REP, int NW, int TR = 0>
__device__ __forceinline__ void plain_rows_mfma(const DecodeParams& P, const PlainLds& lds, float (*s_wm)[REP],
                                                float (*s_wl)[REP], const char* kbase, const char* vbase,
                                                int64_t kst, int64_t vst, int t0, int t1, int b, int hq0,
                                                int nvalid_h, int wslot, char* kdst = nullptr,
                                                char* vdst = nullptr, int64_t dkst = 0, int64_t dvst = 0) {
  using E = Elem<DT>;
  using L = PlainMfmaLds<D, REP, NW, TR>;
  constexpr int EP = E::per16;          // elements per 16-byte piece
  constexpr int SL = D / EP;            // pieces per row
  constexpr int RPI = kWave / SL;       // rows covered by one load instruction
  constexpr int RB = D * E::size;       // bytes per row
  constexpr int TILE = L::TILE;         // rows per wave tile
  constexpr int PPL = TILE / RPI;       // 16-byte pieces per lane per tile (K and V each)
  constexpr int NB = TILE / 16;         // 16-row MFMA blocks
  constexpr int KS = D / 32;            // q.k k-steps
  constexpr int VPB = 16 / RPI;
  constexpr int NP = L::NP;             // producer/consumer wave pairs
  constexpr int DB = D / 16;            // 16-column blocks of the P.V product
  constexpr int KS2 = TILE / 32;        // 32-row k-steps of the P.V product
  static_assert(SL * RPI == kWave && PPL * RPI == TILE && REP <= 16 && VPB % 2 == 0 && NB * VPB == PPL,
                "mfma tile shape");
  float* s_pall = reinterpret_cast<float*>(lds.p);
  float* s_alpha = reinterpret_cast<float*>(lds.al);
  float* s_wo = reinterpret_cast<float*>(lds.wo);
  char* s_vt = lds.vt;
  char* s_kt = lds.kt;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int nrows_total = max(t1 - t0, 0);
  const int ntiles_total = (nrows_total + TILE - 1) / TILE;
  float m_run[REP], l_head[REP];
  f32x4 acc_pv[DB];
#pragma unroll
  for (int r = 0; r < REP; ++r) m_run[r] = -INFINITY;
  const int my_col = lane % SL;
  const int my_row0 = lane / SL;
  const int voff0 = my_col * 16;

  // ---- Producer/consumer wave pairs: every wave streams ONE contiguous
  // row range of ONE tensor (on gfx950 a wave that streams two distant
  // regions at once pulls markedly less bandwidth than one that streams a
  // single region), 1 KiB of consecutive rows per load instruction (whole
  // 128-byte lines; the MFMA operand layout read straight from memory
  // would split every line over two instructions).  Each tile is staged
  // in the wave's own LDS slot and read back in operand layout.  Waves
  // [0, NP) read K and compute the scores on v_mfma_f32_16x16x32 (A = 16 K
  // rows x 32 elements: lane l holds row l%16, elements 8*(l/16)..+8 of
  // the k-step; B = q^T: lane l holds head l%16; D: lane l holds head
  // l%16, rows 4*(l/16)..+4) and the online softmax; waves [NP, NW) read V
  // and accumulate P.V with the tile's probabilities and rescale factors
  // their partner leaves in LDS (double-buffered by tile parity, one
  // workgroup barrier per tile).  Each wave keeps two tiles of loads in
  // flight (one at D = 256).
  constexpr int NBUF = NB * KS;
  static_assert(NBUF == PPL, "K and V tiles use the same register budget");
  constexpr int TIF = D > 128 ? 1 : 2;  // tiles in flight per wave (register budget)
  const bool kwave = wave < NP;
  const int pair = kwave ? wave : wave - NP;
  const int tpp = (ntiles_total + NP - 1) / NP;   // tiles per pair, uniform in the workgroup
  const int ps = t0 + pair * tpp * TILE;
  const int pe = min(t1, ps + tpp * TILE);
  uint16_t* pbuf = reinterpret_cast<uint16_t*>(s_pall) + pair * 2 * REP * TILE;
  float* abuf = s_alpha + pair * 2 * REP;
  const int hl = lane & 15;   // score layout: head
  const int kg = lane >> 4;   // score layout: k-group / row quad
  uint4 qb[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) qb[s] = make_uint4(0, 0, 0, 0);
  if (kwave && hl < nvalid_h) {
    const char* qrow = reinterpret_cast<const char*>(P.q) +
                       ((int64_t)b * P.q_stride_b + (int64_t)(hq0 + hl) * P.q_stride_h) * E::size;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if (P.q_aligned) {
        qb[s] = *reinterpret_cast<const uint4*>(qrow + (s * 32 + kg * 8) * 2);
      } else {
        const uint16_t* qh = reinterpret_cast<const uint16_t*>(qrow) + s * 32 + kg * 8;
        qb[s] = make_uint4(qh[0] | ((uint32_t)qh[1] << 16), qh[2] | ((uint32_t)qh[3] << 16),
                           qh[4] | ((uint32_t)qh[5] << 16), qh[6] | ((uint32_t)qh[7] << 16));
      }
    }
  }
  // The two roles run separate loops with the same number of workgroup
  // barriers (tpp), so each role's registers are live only in its own loop.
  if (kwave) {
    float m_lane = -INFINITY;  // running max of head hl (equal on its 4 lanes)
    float l_lane = 0.f;        // this lane's share of head hl's denominator
    char* kt = s_kt + pair * TILE * RB;
    for (int it = 0; it < tpp; it += TIF) {
      uint4 buf[TIF][NBUF];
#pragma unroll
      for (int u = 0; u < TIF; ++u) {
        const int tb = ps + (it + u) * TILE;
        const __amdgpu_buffer_rsrc_t rr = make_rsrc(kbase + (int64_t)tb * kst, (int64_t)(pe - tb) * kst);
#pragma unroll
        for (int i = 0; i < PPL; ++i) buf[u][i] = buf_ld16(rr, (int)((i * RPI + my_row0) * kst) + voff0);
      }
#pragma unroll
      for (int u = 0; u < TIF; ++u) {
        if (it + u >= tpp) break;
        const int tb = ps + (it + u) * TILE;
        const int nrows = min(TILE, pe - tb);  // <= 0: every row masked
        uint16_t* pt = pbuf + ((it + u) & 1) * REP * TILE;
        float* at = abuf + ((it + u) & 1) * REP;
        // stage the tile (rows past the slice arrived as zeros), read it
        // back as MFMA A operands (this wave's own slot: no barrier)
#pragma unroll
        for (int i = 0; i < PPL; ++i) {
          const int r = i * RPI + my_row0;
          *reinterpret_cast<uint4*>(kt + r * RB + ((my_col ^ kswz<SL>(r)) << 4)) = buf[u][i];
        }
        // write-allocate: the rows also go to their staging slot
        if (kdst != nullptr) {
#pragma unroll
          for (int i = 0; i < PPL; ++i) {
            const int r = i * RPI + my_row0;
            if (r < nrows) *reinterpret_cast<uint4*>(kdst + (int64_t)(tb + r) * dkst + voff0) = buf[u][i];
          }
        }
        f32x4 sc[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          sc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
          const int r = nb * 16 + hl;
#pragma unroll
          for (int s = 0; s < KS; ++s) {
            const uint4 a = *reinterpret_cast<const uint4*>(kt + r * RB + (((s * 4 + kg) ^ kswz<SL>(r)) << 4));
            sc[nb] = MfmaOp<DT>::run(a, qb[s], sc[nb]);
          }
        }
        float sv[NB][4], bm = -INFINITY;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int c = 0; c < 4; ++c) sv[nb][c] = sc[nb][c] * P.scale2;
        if (nrows < TILE) {  // a short tile (the slice's last): mask rows past it
          // The empty volatile asm keeps this a real (wave-uniform) branch
          // instead of compares and selects on every tile.
          asm volatile("");
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (nb * 16 + kg * 4 + c >= nrows) sv[nb][c] = -INFINITY;
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int c = 0; c < 4; ++c) bm = fmaxf(bm, sv[nb][c]);
        bm = rows4_max(bm);
        const float m_new = fmaxf(m_lane, bm);
        const float ms = (m_new == -INFINITY) ? 0.f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_lane - ms);
        m_lane = m_new;
        float psum = 0.f;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          float p4[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            p4[c] = __builtin_amdgcn_exp2f(sv[nb][c] - ms);
            psum += p4[c];
          }
          // rows nb*16 + 4kg .. +3 of head hl: one 8-byte store
          if (hl < REP)
            *reinterpret_cast<uint2*>(pt + hl * TILE + nb * 16 + kg * 4) =
                make_uint2(pack2<DT>(p4[0], p4[1]), pack2<DT>(p4[2], p4[3]));
        }
        l_lane = l_lane * alpha + psum;
        if (lane < REP) at[lane] = alpha;
        __syncthreads();  // hand the tile's p and rescale factors to the V-wave
      }
    }
    const float lsum = rows4_sum(l_lane);
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      m_run[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m_lane), r));
      l_head[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lsum), r));
    }
  } else {
    // P.V on v_mfma_f32_16x16x32: A = P^T (lane l: head l%16, rows
    // 8*(l/16)..+8 of the 32-row k-step, read from the K-wave's [head][row]
    // tile), B = V (lane l: column l%16 of the 16-column block, the same 8
    // rows, gathered from the LDS copy of the tile with two transposed
    // reads), D: lane l holds heads 4*(l/16)..+4 of column l%16.
    char* vt = s_vt + pair * TILE * RB;
    const int hA = lane & 15;           // A operand head
    const int gq = lane >> 4;           // lane group: 8-row slab of the k-step
    const int prow = (lane & 15) >> 2;  // transposed read: row within the 4-row block
    const int pcol = lane & 3;          // transposed read: 4-column group
#pragma unroll
    for (int db = 0; db < DB; ++db) acc_pv[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < tpp; it += TIF) {
      uint4 buf[TIF][NBUF];
#pragma unroll
      for (int u = 0; u < TIF; ++u) {
        const int tb = ps + (it + u) * TILE;
        const __amdgpu_buffer_rsrc_t rr = make_rsrc(vbase + (int64_t)tb * vst, (int64_t)(pe - tb) * vst);
#pragma unroll
        for (int i = 0; i < PPL; ++i) buf[u][i] = buf_ld16(rr, (int)((i * RPI + my_row0) * vst) + voff0);
      }
#pragma unroll
      for (int u = 0; u < TIF; ++u) {
        if (it + u >= tpp) break;
        // stage the tile (rows past the slice arrived as zeros)
#pragma unroll
        for (int i = 0; i < PPL; ++i) {
          const int r = i * RPI + my_row0;
          *reinterpret_cast<uint4*>(vt + r * RB + ((my_col ^ vswz<SL>(r)) << 4)) = buf[u][i];
        }
        if (vdst != nullptr) {  // write-allocate
          const int tb = ps + (it + u) * TILE;
#pragma unroll
          for (int i = 0; i < PPL; ++i) {
            const int r = i * RPI + my_row0;
            if (tb + r < pe) *reinterpret_cast<uint4*>(vdst + (int64_t)(tb + r) * dvst + voff0) = buf[u][i];
          }
        }
        const uint16_t* pt = reinterpret_cast<const uint16_t*>(s_pall) + pair * 2 * REP * TILE +
                             ((it + u) & 1) * REP * TILE;
        const float* at = abuf + ((it + u) & 1) * REP;
        __syncthreads();  // the K-wave's p and rescale factors for this tile are in LDS
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a = at[min(4 * gq + e, REP - 1)];
#pragma unroll
          for (int db = 0; db < DB; ++db) acc_pv[db][e] *= a;
        }
#pragma unroll
        for (int s2 = 0; s2 < KS2; ++s2) {
          const uint4 pa = hA < REP ? *reinterpret_cast<const uint4*>(pt + hA * TILE + s2 * 32 + gq * 8)
                                    : make_uint4(0, 0, 0, 0);
          const int r0 = s2 * 32 + gq * 8 + prow;
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const int pc = 2 * db + (pcol >> 1);
            const int bo = (pcol & 1) * 8;
            const uint2 lo = lds_read_tr16(vt + r0 * RB + ((pc ^ vswz<SL>(r0)) << 4) + bo);
            const uint2 hi = lds_read_tr16(vt + (r0 + 4) * RB + ((pc ^ vswz<SL>(r0 + 4)) << 4) + bo);
            acc_pv[db] = MfmaOp<DT>::run(pa, make_uint4(lo.x, lo.y, hi.x, hi.y), acc_pv[db]);
          }
        }
      }
    }
  }
  write_partial_pairs_mfma<D, REP, NP, DB>(P, wslot, kwave, pair, acc_pv, m_run, l_head, s_wo, s_wm, s_wl);
}

template <int DT, int D, int REP, int NW, bool WIDE = false>
__global__ void __launch_bounds__(64 * NW, 2)
decode_attn_kernel(DecodeParams P) {
  using Cap = SelCap<WIDE>;
  using E = Elem<DT>;
  constexpr bool kMfma = DT != HALO_F32;  // q.k on the matrix cores
  constexpr int EP = E::per16;          // elements per 16-byte piece
  constexpr int SL = D / EP;            // pieces per row
  constexpr int RPI = kWave / SL;       // rows covered by one load instruction
  constexpr int RB = D * E::size;       // bytes per row
  constexpr int KROW = RB + 16;         // padded LDS row stride (bank-conflict free)
  constexpr int TILE = SL <= 16 ? kWave : kWave * 16 / SL;  // rows per wave tile
  constexpr int PPL = TILE / RPI;       // 16-byte pieces per lane per tile (K and V each)
  constexpr int LPH0 = kWave / REP;     // lanes per query head in the VALU q.k phase
  constexpr int LPH = LPH0 < TILE ? LPH0 : TILE;
  constexpr int RPL = TILE / LPH;       // rows per lane in the VALU q.k phase
  static_assert(SL * RPI == kWave && PPL * RPI == TILE && PPL % 2 == 0, "tile shape");
  static_assert(LPH == 8 || LPH == 16 || LPH == 32 || LPH == 64, "lane groups");
  // VALU path: per-wave q copy, K tiles, p tiles; the epilogue reuses the front.
  // MFMA path: per pair 2 p tiles (K/V dtype, [head][row]) and 2 rescale
  // vectors, the pair partials, then one V tile per V-wave.
  constexpr int SZ_Q = kMfma ? 0 : NW * REP * RB;
  constexpr int SZ_K = kMfma ? 0 : NW * TILE * KROW;
  constexpr int SZ_P = kMfma ? 0 : NW * TILE * REP * 4;
  constexpr int SZ_A0 = kMfma ? PlainMfmaLds<D, REP, NW>::bytes : SZ_Q + SZ_K + SZ_P;
  constexpr int SZ_A = SZ_A0 > Cap::bytes ? SZ_A0 : Cap::bytes;
  constexpr int SZ_B = kMfma ? 0 : NW * REP * D * 4;
  __shared__ __attribute__((aligned(16))) char smem[SZ_A > SZ_B ? SZ_A : SZ_B];
  char* s_q = smem + (threadIdx.x / kWave) * REP * RB;
  char* s_kall = smem + SZ_Q;
  float* s_pall = reinterpret_cast<float*>(smem + SZ_Q + SZ_K);
  float* s_wo = reinterpret_cast<float*>(smem);
  __shared__ float s_wm[NW][REP], s_wl[NW][REP];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  // Wave index and work item are wave-uniform; saying so keeps every value
  // derived from them (buffer descriptors, row ranges) in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int witem = blockIdx.x;
  // Leading selection-slot items start the selection's loads at once (the
  // selection does not depend on the record unless it is per batch row).
  Selector<DT, D, 64 * NW, WIDE> selr;
  const bool early_sel = P.sel_on && !P.sel.per_row && witem < P.sel.lead_items;
  if (early_sel) selr.issue(P, 0);

  const int32_t* wrec = P.work + (int64_t)witem * kWorkInts;
  int4 item = *reinterpret_cast<const int4*>(wrec);
  item.x = __builtin_amdgcn_readfirstlane(item.x);
  item.y = __builtin_amdgcn_readfirstlane(item.y);
  item.z = __builtin_amdgcn_readfirstlane(item.z);
  item.w = __builtin_amdgcn_readfirstlane(item.w);
  const int wslot = __builtin_amdgcn_readfirstlane(wrec[4]);
  if ((unsigned)wslot >= (unsigned)P.n_work) return;  // malformed record: no partial slot to write
  const int g = item.y;
  const int sub = g % P.n_sub;
  const int bh = g / P.n_sub;
  const int h_kv = bh % P.H_kv;
  const int b = bh / P.H_kv;
  halo_chunk_desc dsc;
  halo_chunk_desc wdst;  // write-allocate destination (selection slots that read a chunk in place)
  bool wa = false;
  if (P.sel_on && item.x >= P.sel.slot0 && item.x < P.sel.slot0 + P.sel.top_k) {
    // selection slot: choose the chunk first (workgroup-uniform branch)
    const bool writer = (P.sel.per_row || b == 0) && h_kv == 0 && sub == 0 && item.x == P.sel.slot0 && item.z == 0;
    if (!early_sel) selr.issue(P, b);
    const int pick = selr.finish(P, smem, item.x - P.sel.slot0, writer);
    if (pick >= 0) {
      // the chunk's own catalog entry (rows, start, flags); a staged chunk is
      // read through its slot's addresses and strides
      const halo_chunk_desc* tbl = reinterpret_cast<const halo_chunk_desc*>(smem + Cap::cat_off);
      halo_chunk_desc d = tbl[pick];
      if (selr.staged_slot >= 0) {
        const halo_chunk_desc& sd = tbl[Cap::max_cold + selr.staged_slot];
        d.k = sd.k;
        d.v = sd.v;
        d.k_stride_b = sd.k_stride_b;
        d.k_stride_h = sd.k_stride_h;
        d.k_stride_t = sd.k_stride_t;
        d.v_stride_b = sd.v_stride_b;
        d.v_stride_h = sd.v_stride_h;
        d.v_stride_t = sd.v_stride_t;
      }
      dsc = uniform_desc(d);
      if (selr.wa_slot >= 0) {
        wdst = uniform_desc(tbl[Cap::max_cold + selr.wa_slot]);
        wa = true;
      }
    } else {
      dsc = P.descs[item.x];
      dsc.T_c = 0;
    }
    __syncthreads();  // LDS is reused below
  } else {
    dsc = P.descs[item.x];
  }
  const int hq0 = h_kv * P.rep + sub * REP;
  const int nvalid_h = min(REP, P.rep - sub * REP);

  // Row range: never past the chunk's own rows (a table slot a scorer filled
  // with a shorter or empty chunk), then the causal cut chunk_start+t <= q_pos.
  // A KIVI chunk holds no plain rows: this kernel reads nothing of it.
  int t0 = item.z, t1 = (dsc.flags & HALO_CHUNK_KIVI2) ? item.z : min(item.w, dsc.T_c);
  if ((dsc.flags & HALO_CHUNK_CAUSAL) && P.q_pos != nullptr) {
    const int64_t lim = P.q_pos[b] - dsc.chunk_start + 1;
    if (lim < (int64_t)t1) t1 = (int)max<int64_t>(lim, (int64_t)t0);
  }

  const char* kbase = reinterpret_cast<const char*>(dsc.k) +
                      ((dsc.batch < 0 ? (int64_t)b * dsc.k_stride_b : 0) + (int64_t)h_kv * dsc.k_stride_h) * E::size;
  const char* vbase = reinterpret_cast<const char*>(dsc.v) +
                      ((dsc.batch < 0 ? (int64_t)b * dsc.v_stride_b : 0) + (int64_t)h_kv * dsc.v_stride_h) * E::size;
  const int64_t kst = dsc.k_stride_t * E::size;
  const int64_t vst = dsc.v_stride_t * E::size;

  const int nrows_total = max(t1 - t0, 0);
  const int ntiles_total = (nrows_total + TILE - 1) / TILE;
  const int tiles_per_wave = (ntiles_total + NW - 1) / NW;
  const int ws = t0 + wave * tiles_per_wave * TILE;
  const int we = min(t1, ws + tiles_per_wave * TILE);

  float m_run[REP], acc_o[REP][EP], l_head[REP];
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    m_run[r] = -INFINITY;
#pragma unroll
    for (int e = 0; e < EP; ++e) acc_o[r][e] = 0.f;
  }

  float* pl = s_pall + wave * TILE * REP;
  const int my_col = lane % SL;
  const int my_row0 = lane / SL;
  const int voff0 = my_col * 16;

  if constexpr (kMfma) {
    char* kdst = nullptr;
    char* vdst = nullptr;
    if (wa) {
      kdst = reinterpret_cast<char*>(const_cast<void*>(wdst.k)) +
             ((dsc.batch < 0 ? (int64_t)b * wdst.k_stride_b : 0) + (int64_t)h_kv * wdst.k_stride_h) * E::size;
      vdst = reinterpret_cast<char*>(const_cast<void*>(wdst.v)) +
             ((dsc.batch < 0 ? (int64_t)b * wdst.v_stride_b : 0) + (int64_t)h_kv * wdst.v_stride_h) * E::size;
    }
    plain_rows_mfma<DT, D, REP, NW>(P, plain_lds_at<D, REP, NW>(smem), s_wm, s_wl, kbase, vbase, kst, vst, t0, t1, b,
                                    hq0, nvalid_h, wslot, kdst, vdst, wa ? wdst.k_stride_t * E::size : 0,
                                    wa ? wdst.v_stride_t * E::size : 0);
    return;
  } else {
    // ---- VALU path (fp32): K transposed through LDS, lane groups per head.
    float l_lane = 0.f;  // this lane's share of its head's softmax denominator
    char* kl = s_kall + wave * TILE * KROW;
    const bool qk_lane = lane < REP * LPH;
    const int hl = qk_lane ? lane / LPH : 0;  // this lane's head in the q.k phase
    const int rb = lane % LPH;                // its first row

    // Tile loads: rows past the slice read as zeros (hardware range check).
    uint4 kreg[PPL], vreg[PPL];
    auto load_k = [&](int tb) {
      const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase + (int64_t)tb * kst, (int64_t)(we - tb) * kst);
#pragma unroll
      for (int i = 0; i < PPL; ++i) kreg[i] = buf_ld16(rk, (int)((i * RPI + my_row0) * kst) + voff0);
    };
    auto load_v = [&](int tb) {
      const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase + (int64_t)tb * vst, (int64_t)(we - tb) * vst);
#pragma unroll
      for (int i = 0; i < PPL; ++i) vreg[i] = buf_ld16(rv, (int)((i * RPI + my_row0) * vst) + voff0);
    };
    for (int tb = ws; tb < we; tb += TILE) {
      const int nrows = min(TILE, we - tb);
      load_k(tb);
      load_v(tb);
      if (tb == ws) {
        // This wave's copy of the group's query rows (zeros for padding
        // heads), fetched while the first tile's K/V loads are in flight.
        if (P.q_aligned) {
          for (int pc = lane; pc < REP * SL; pc += kWave) {
            const int r = pc / SL, c = pc % SL;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (r < nvalid_h)
              v = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(P.q) +
                                                  (b * P.q_stride_b + (int64_t)(hq0 + r) * P.q_stride_h) * E::size +
                                                  c * 16);
            *reinterpret_cast<uint4*>(s_q + pc * 16) = v;
          }
        } else {
          for (int i = lane; i < REP * D; i += kWave) {
            const int r = i / D, d = i % D;
            const int64_t qi = b * P.q_stride_b + (int64_t)(hq0 + r) * P.q_stride_h + d;
            if (DT == HALO_F32) {
              reinterpret_cast<float*>(s_q)[i] = r < nvalid_h ? reinterpret_cast<const float*>(P.q)[qi] : 0.f;
            } else {
              reinterpret_cast<uint16_t*>(s_q)[i] = r < nvalid_h ? reinterpret_cast<const uint16_t*>(P.q)[qi] : 0;
            }
          }
        }
      }
#pragma unroll
      for (int i = 0; i < PPL; ++i)
        *reinterpret_cast<uint4*>(kl + (i * RPI + my_row0) * KROW + my_col * 16) = kreg[i];
      wave_lds_fence();

      // q.k: lane group hl holds head hl's scores for rows rb + LPH*i.
      float s[RPL];
#pragma unroll
      for (int i = 0; i < RPL; ++i) s[i] = 0.f;
#pragma unroll
      for (int c = 0; c < SL; ++c) {
        const uint4 qp = *reinterpret_cast<const uint4*>(s_q + hl * RB + c * 16);
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
          const uint4 kp = *reinterpret_cast<const uint4*>(kl + (rb + LPH * i) * KROW + c * 16);
          s[i] = E::dot(kp, qp, s[i]);
        }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < RPL; ++i) {
        const bool valid = qk_lane && (rb + LPH * i) < nrows;
        s[i] = valid ? s[i] * P.scale2 : -INFINITY;
        mx = fmaxf(mx, s[i]);
      }
      mx = group_max<LPH>(mx);
      float alpha[REP], my_ms = 0.f, my_alpha = 1.f;
      bool rescale = false;
#pragma unroll
      for (int r = 0; r < REP; ++r) {
        const float tmax = head_value<LPH, true>(mx, r);
        const float m_new = fmaxf(m_run[r], tmax);
        const float ms = (m_new == -INFINITY) ? 0.f : m_new;
        alpha[r] = __builtin_amdgcn_exp2f(m_run[r] - ms);
        rescale |= (alpha[r] != 1.f);
        m_run[r] = m_new;
        if (hl == r) {
          my_ms = ms;
          my_alpha = alpha[r];
        }
      }
      float psum = 0.f;
#pragma unroll
      for (int i = 0; i < RPL; ++i) {
        const float p = __builtin_amdgcn_exp2f(s[i] - my_ms);
        psum += p;
        if (qk_lane) pl[(rb + LPH * i) * REP + hl] = p;
      }
      l_lane = l_lane * my_alpha + psum;
      if (rescale) {
#pragma unroll
        for (int r = 0; r < REP; ++r)
#pragma unroll
          for (int e = 0; e < EP; ++e) acc_o[r][e] *= alpha[r];
      }
      wave_lds_fence();

      // P.V over row pairs (rows j and j+1 of this lane's column slice).
#pragma unroll
      for (int j = 0; j < PPL; j += 2) {
        const int ra = j * RPI + my_row0, rbw = (j + 1) * RPI + my_row0;
        float pa[REP], pb[REP];
#pragma unroll
        for (int r = 0; r < REP; ++r) {
          pa[r] = pl[ra * REP + r];
          pb[r] = pl[rbw * REP + r];
        }
        pv_pair<DT, REP, EP>(vreg[j], vreg[j + 1], pa, pb, acc_o);
      }
      wave_lds_fence();
    }
    // l per head: reduce the lane shares of each head's group
    const float lg = group_sum<LPH>(qk_lane ? l_lane : 0.f);
#pragma unroll
    for (int r = 0; r < REP; ++r) l_head[r] = head_value<LPH, false>(lg, r);
  }

  write_partial<D, REP, NW, SL, EP>(P, wslot, acc_o, m_run, l_head, s_wo, s_wm, s_wl);
}

// ---------------------------------------------------------------------------
// Decode attention over KIVI 2-bit blocks (halo_decode_attn_kivi).  Each wave
// streams a contiguous run of blocks (one tile = TB blocks of 3 KiB at D=128,
// two tiles of loads in flight) and stages each tile in its own LDS slot.
// The dequantisation x = code * scale + zero (baselines/kivi_cache.py:72-78)
// is folded into the two products instead of being applied per element:
//   q.k_t   = sum_d code_td (q_d s_d)     + sum_d q_d z_d          (K per channel)
//   (P V)_d = sum_t (p_t s_tg) code_td    + sum_t p_t z_tg         (V per token group g)
// so each MFMA takes the raw codes (exact small integers in the K/V dtype)
// against a scaled q or p, and the zero terms are one more MFMA each with
// the zeros broadcast across the tile.  The products differ from attention
// over the dequantised cache only by the rounding of q*s and p*s (fp16: one
// fp16 rounding; bf16: a head + remainder pair, about 2^-17).
// ---------------------------------------------------------------------------
// One 16-bit word of 2-bit codes (8 elements: the even ones 2p at bits 2p,
// the odd ones 2p+1 at bits 8+2p) -> 8 small integers in bf16, in element
// order
__device__ __forceinline__ uint4 kivi_codes8_bf16(uint32_t c16) {
  uint32_t w[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const bf16x2_t v = {(__bf16)(float)((c16 >> (2 * p)) & 3u), (__bf16)(float)((c16 >> (8 + 2 * p)) & 3u)};
    w[p] = __builtin_bit_cast(uint32_t, v);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}
// bf16 products are split into a bf16 head and the bf16 rounding of the
// remainder (the fp32 product of two bf16 values is exact), so the MFMA
// pair sees the product to about 2^-17 instead of bf16's 2^-9
__device__ __forceinline__ void mul8_bf16_split(const uint4& a, const uint4& b, uint4& hi, uint4& lo) {
  const uint32_t x[4] = {a.x, a.y, a.z, a.w}, y[4] = {b.x, b.y, b.z, b.w};
  uint32_t h[4], l[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float p0 = bf16_lo(x[p]) * bf16_lo(y[p]), p1 = bf16_hi(x[p]) * bf16_hi(y[p]);
    h[p] = pack2<HALO_BF16>(p0, p1);
    l[p] = pack2<HALO_BF16>(p0 - bf16_lo(h[p]), p1 - bf16_hi(h[p]));
  }
  hi = make_uint4(h[0], h[1], h[2], h[3]);
  lo = make_uint4(l[0], l[1], l[2], l[3]);
}
// fp16 only: one 16-bit word of 2-bit codes (8 elements: the even ones 2p
// at bits 2p, the odd ones 2p+1 at bits 8+2p) as fp16 subnormals.  t = w |
// w << 8 holds elements 2p and 2p+1 at bits 2p and 16+2p, so one mask per
// register places a pair, in place: register p holds c * 4^p * 2^-24
// (exact; the matrix cores keep fp16 subnormal inputs).  The other MFMA
// operand's register p is scaled by 4^-p (kivi_prescale, exact powers of
// two), and products carry a common 2^-24 that the caller removes exactly.
__device__ __forceinline__ uint4 kivi_codes8_sub_inplace(uint32_t c16) {
  const uint32_t t = c16 | (c16 << 8);
  return make_uint4(t & 0x00030003u, t & 0x000C000Cu, t & 0x00300030u, t & 0x00C000C0u);
}
// Registers 1, 2 and 3 of an 8-element fp16 operand times 2^-2, 2^-4, 2^-6.
__device__ __forceinline__ uint4 kivi_prescale(uint4 v) {
  typedef __attribute__((ext_vector_type(2))) _Float16 h2;
  const h2 s2 = {(_Float16)0.25f, (_Float16)0.25f}, s4 = {(_Float16)0.0625f, (_Float16)0.0625f},
           s6 = {(_Float16)0.015625f, (_Float16)0.015625f};
  v.y = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v.y) * s2);
  v.z = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v.z) * s4);
  v.w = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v.w) * s6);
  return v;
}
constexpr float kSub16Scale = 16777216.0f;  // 2^24

// elementwise product of two 8-element K/V-dtype pieces, rounded to the dtype
template <int DT>
__device__ __forceinline__ uint4 mul8(const uint4& a, const uint4& b) {
  const uint32_t x[4] = {a.x, a.y, a.z, a.w}, y[4] = {b.x, b.y, b.z, b.w};
  uint32_t w[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    if constexpr (DT == HALO_F16) {
      typedef __attribute__((ext_vector_type(2))) _Float16 h2;
      w[p] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, x[p]) * __builtin_bit_cast(h2, y[p]));
    } else {
      w[p] = pack2<DT>(bf16_lo(x[p]) * bf16_lo(y[p]), bf16_hi(x[p]) * bf16_hi(y[p]));
    }
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Epilogue for o held as MFMA accumulators (lane l: heads 4*(l/16)..+4 of
// columns 16*db + l%16) by NS partial owners: owner j contributes o (has_o)
// and/or its (m, l) per head (has_ml); the NS partials are merged through
// LDS into the work item's partial.  Owner j's o goes to s_wo + j * OSTR
// floats (OSTR >= REP * D).
template <int D, int REP, int NS, int DB, int OSTR = REP * D>
__device__ __forceinline__ void write_partial_owners(const DecodeParams& P, int wslot, int owner, bool has_o,
                                                     bool has_ml, const f32x4 (&acc)[DB], const float* m_run,
                                                     const float* l_head, float* s_wo, float (*s_wm)[REP],
                                                     float (*s_wl)[REP]) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  if (has_o) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int h = 4 * (lane >> 4) + e;
      if (h < REP) {
#pragma unroll
        for (int db = 0; db < DB; ++db) s_wo[owner * OSTR + h * D + db * 16 + (lane & 15)] = acc[db][e];
      }
    }
  }
  if (has_ml && lane == 0) {
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      s_wm[owner][r] = m_run[r];
      s_wl[owner][r] = l_head[r];
    }
  }
  __syncthreads();
  float* wso = P.ws_o + (int64_t)wslot * REP * D;
  for (int i = tid; i < REP * D; i += blockDim.x) {
    const int r = i / D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NS; ++w) M = fmaxf(M, s_wm[w][r]);
    const float Ms = (M == -INFINITY) ? 0.f : M;
    float acc_o = 0.f;
#pragma unroll
    for (int w = 0; w < NS; ++w) acc_o += __builtin_amdgcn_exp2f(s_wm[w][r] - Ms) * s_wo[w * OSTR + i];
    wso[i] = acc_o;
  }
  if (tid < REP) {
    const int r = tid;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NS; ++w) M = fmaxf(M, s_wm[w][r]);
    const float Ms = (M == -INFINITY) ? 0.f : M;
    float acc_l = 0.f;
#pragma unroll
    for (int w = 0; w < NS; ++w) acc_l += __builtin_amdgcn_exp2f(s_wm[w][r] - Ms) * s_wl[w][r];
    P.ws_ml[((int64_t)wslot * REP + r) * 2 + 0] = M;
    P.ws_ml[((int64_t)wslot * REP + r) * 2 + 1] = acc_l;
  }
}


// Slack (log2 units) by which a block pair's max may exceed the running max
// before the running max moves.
constexpr float kKiviLazyMax = 8.0f;

template <int DT, int D, int REP, int NW>
__global__ void __launch_bounds__(64 * NW, 2)
decode_attn_kivi_kernel(DecodeParams P) {
  using E = Elem<DT>;
  constexpr int RB2 = D / 4;                   // K code bytes per token row (2 bits)
  constexpr int CB = 32 * RB2;                 // code bytes of K (or V) per block
  constexpr int BB = 2 * CB + 8 * D;           // block bytes
  constexpr int NG = D / 32;                   // V groups per token
  constexpr int KS = D / 32;                   // q.k k-steps
  constexpr int DB = D / 16;                   // P.V column blocks
  constexpr int TB = D > 128 ? 2 : 4;         // blocks per wave tile (12 KiB at D = 128, 256)
  constexpr int TBYTES = TB * BB;
  constexpr int LPT = TBYTES / (16 * kWave);   // 16-byte loads per lane per tile
  static_assert(TBYTES % (16 * kWave) == 0 && REP <= 16 && TB % 2 == 0, "kivi tile shape");
  // K side of a block at offset 0: codes [0, CB), scale [CB, CB+2D), zero [CB+2D, CB+4D)
  // V side: codes (channel-major, 8 bytes per channel) at CB+4D, scale/zero (group-major)
  constexpr int VC = CB + 4 * D, VS = 2 * CB + 4 * D, VZ = 2 * CB + 6 * D;

  // LDS: one raw tile per wave (each wave reads only its own, in order, so
  // no fence is needed between its stores and loads); a wave's partial goes
  // into its own tile at the end.  The plain-row path (the unquantised
  // recent rows in the same launch, 32-row tiles) lays its regions over the
  // same bytes.
  constexpr int PL_TR = 32;
  using PL = PlainMfmaLds<D, REP, NW, PL_TR>;
  constexpr int SZ_RAW = NW * TBYTES > PL::bytes ? NW * TBYTES : PL::bytes;
  static_assert(TBYTES >= REP * D * 4, "a wave's partial fits in its raw tile");
  __shared__ __attribute__((aligned(16))) char s_raw[SZ_RAW];
  __shared__ float s_wm[NW][REP], s_wl[NW][REP];
  float* s_wo = reinterpret_cast<float*>(s_raw);  // wave w's partial at raw tile w

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int witem = blockIdx.x;
  const int32_t* wrec = P.work + (int64_t)witem * kWorkInts;
  int4 item = *reinterpret_cast<const int4*>(wrec);
  item.x = __builtin_amdgcn_readfirstlane(item.x);
  item.y = __builtin_amdgcn_readfirstlane(item.y);
  item.z = __builtin_amdgcn_readfirstlane(item.z);
  item.w = __builtin_amdgcn_readfirstlane(item.w);
  const int wslot = __builtin_amdgcn_readfirstlane(wrec[4]);
  if ((unsigned)wslot >= (unsigned)P.n_work) return;  // malformed record: no partial slot to write
  const int g = item.y;
  const int sub = g % P.n_sub;
  const int bh = g / P.n_sub;
  const int h_kv = bh % P.H_kv;
  const int b = bh / P.H_kv;
  const halo_chunk_desc dsc = P.descs[item.x];
  const int hq0 = h_kv * P.rep + sub * REP;
  const int nvalid_h = min(REP, P.rep - sub * REP);

  int t0 = item.z, t1 = min(item.w, dsc.T_c);
  if ((dsc.flags & HALO_CHUNK_CAUSAL) && P.q_pos != nullptr) {
    const int64_t lim = P.q_pos[b] - dsc.chunk_start + 1;
    if (lim < (int64_t)t1) t1 = (int)max<int64_t>(lim, (int64_t)t0);
  }
  if (!(dsc.flags & HALO_CHUNK_KIVI2)) {
    // plain K/V rows (the unquantised recent tokens) in the same launch
    const char* kb = reinterpret_cast<const char*>(dsc.k) +
                     ((dsc.batch < 0 ? (int64_t)b * dsc.k_stride_b : 0) + (int64_t)h_kv * dsc.k_stride_h) * E::size;
    const char* vb = reinterpret_cast<const char*>(dsc.v) +
                     ((dsc.batch < 0 ? (int64_t)b * dsc.v_stride_b : 0) + (int64_t)h_kv * dsc.v_stride_h) * E::size;
    plain_rows_mfma<DT, D, REP, NW, PL_TR>(P, plain_lds_at<D, REP, NW, PL_TR>(s_raw), s_wm, s_wl, kb, vb, dsc.k_stride_t * E::size, dsc.v_stride_t * E::size,
                                    t0, t1, b, hq0, nvalid_h, wslot);
    return;
  }
  // block bytes of this (b, h_kv); strides are in bytes for KIVI chunks
  const char* base = reinterpret_cast<const char*>(dsc.k) +
                     (dsc.batch < 0 ? (int64_t)b * dsc.k_stride_b : 0) + (int64_t)h_kv * dsc.k_stride_h;

  // this wave's run of block pairs (token offsets relative to the chunk),
  // walked in tiles of TB blocks; the last tile of a run may be short
  const int nblk = (max(t1 - t0, 0) + 31) / 32;
  const int npairs = (nblk + 1) / 2;
  const int ppw = (npairs + NW - 1) / NW;
  const int wb0 = min(nblk, 2 * wave * ppw);
  const int wb1 = min(nblk, wb0 + 2 * ppw);
  const int wtok1 = min(t1, t0 + wb1 * 32);                    // end of this wave's tokens
  const int ntw = (wb1 - wb0 + TB - 1) / TB;                   // tiles of the run
  const int64_t wbyte0 = (int64_t)(t0 / 32 + wb0) * BB;        // first byte of the run
  const int64_t wbytes = (int64_t)(wb1 - wb0) * BB;            // bytes of the run

  const int hl = lane & 15;   // score layout: head / A-operand head
  const int kg = lane >> 4;   // score layout: row quad / lane group (8-element slab)
  uint4 qb[KS];               // B operand of q.k: q of head hl, channels 32s + 8kg ..
  {
    const bool live = hl < nvalid_h;
    const char* qrow = reinterpret_cast<const char*>(P.q) +
                       ((int64_t)b * P.q_stride_b + (int64_t)(hq0 + (live ? hl : 0)) * P.q_stride_h) * E::size;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      uint4 v = make_uint4(0, 0, 0, 0);
      if (live) {
        if (P.q_aligned) {
          v = *reinterpret_cast<const uint4*>(qrow + (s * 32 + kg * 8) * 2);
        } else {
          const uint16_t* qh = reinterpret_cast<const uint16_t*>(qrow) + s * 32 + kg * 8;
          v.x = qh[0] | ((uint32_t)qh[1] << 16);
          v.y = qh[2] | ((uint32_t)qh[3] << 16);
          v.z = qh[4] | ((uint32_t)qh[5] << 16);
          v.w = qh[6] | ((uint32_t)qh[7] << 16);
        }
      }
      qb[s] = v;
    }
  }
  uint4 qbs[DT == HALO_F16 ? KS : 1];  // fp16: q with registers 1-3 prescaled for the in-place codes
#pragma unroll
  for (int s = 0; s < (DT == HALO_F16 ? KS : 1); ++s) qbs[s] = DT == HALO_F16 ? kivi_prescale(qb[s]) : qb[s];
  f32x4 acc[DB];
  f32x4 accz[DT == HALO_F16 ? NG : 1];  // fp16: zero terms per V group
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int gg = 0; gg < (DT == HALO_F16 ? NG : 1); ++gg) accz[gg] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_lane = -INFINITY;  // running max of head hl (equal on its 4 lanes)
  float l_lane = 0.f;        // this lane's share of head hl's denominator
  // Lanes of heads past the group's live heads score -inf, so their
  // probabilities are exact zeros without a select per P register.
  const float zbias = hl < nvalid_h ? 0.f : -INFINITY;
  // One block pair staged at bkp, first token tokp: the score MFMAs of both
  // blocks are independent and issue together, one online-softmax step
  // covers their 64 tokens (one max, one rescale), and the P.V MFMAs of
  // both follow; a second block past the range is all masked (its bytes
  // read as zeros) and adds nothing.
  auto do_pair = [&](const char* bkp, int tokp) {
    const int nr0 = min(32, t1 - tokp);
    const int nrw[2] = {nr0, min(32, t1 - (tokp + 32))};
    // ---- scores: per block 2 row blocks of 16 tokens, code MFMAs + one zero-term MFMA per k-step
    f32x4 sc[2][2], sz[2];
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      sc[pb][0] = sc[pb][1] = sz[pb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int c0 = 32 * s + 8 * kg;  // first channel of this lane's k-slab
#pragma unroll
      for (int pb = 0; pb < 2; ++pb) {
        const char* bk = bkp + pb * BB;
        const uint4 sk = *reinterpret_cast<const uint4*>(bk + CB + 2 * c0);
        const uint4 zk = *reinterpret_cast<const uint4*>(bk + CB + 2 * D + 2 * c0);
        uint4 qs, qs_lo;
        if constexpr (DT == HALO_BF16) mul8_bf16_split(qb[s], sk, qs, qs_lo);
        else qs = mul8<DT>(qbs[s], sk);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          const uint32_t c16 = *reinterpret_cast<const uint16_t*>(bk + (nb * 16 + hl) * RB2 + c0 / 4);
          const uint4 cd = DT == HALO_F16 ? kivi_codes8_sub_inplace(c16) : kivi_codes8_bf16(c16);
          sc[pb][nb] = MfmaOp<DT>::run(cd, qs, sc[pb][nb]);
          if constexpr (DT == HALO_BF16) sc[pb][nb] = MfmaOp<DT>::run(cd, qs_lo, sc[pb][nb]);
        }
        sz[pb] = MfmaOp<DT>::run(zk, qb[s], sz[pb]);
      }
    }
    // ---- online softmax over the pair (lane: head hl, tokens 32pb + 16nb + 4kg + c)
    // score (log2 units) = (code product + zero term) * scale2, as one fma
    // with the zero term prescaled; fp16 code products carry 2^-24
    float sv[2][2][4], bm = -INFINITY;
    const float cs = DT == HALO_F16 ? kSub16Scale * P.scale2 : P.scale2;
    float zs[2][4];
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int c = 0; c < 4; ++c) zs[pb][c] = __builtin_fmaf(sz[pb][c], P.scale2, zbias);
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int c = 0; c < 4; ++c) sv[pb][nb][c] = __builtin_fmaf(sc[pb][nb][c], cs, zs[pb][c]);
    if (nrw[0] < 32 || nrw[1] < 32) {  // a short block (the run's last): mask rows past it
      // The empty volatile asm keeps this a real (wave-uniform) branch: the
      // compiler would otherwise turn the rare mask into compares and
      // selects that every pair executes.
      asm volatile("");
#pragma unroll
      for (int pb = 0; pb < 2; ++pb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (nb * 16 + kg * 4 + c >= nrw[pb]) sv[pb][nb][c] = -INFINITY;
    }
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int c = 0; c < 4; ++c) bm = fmaxf(bm, sv[pb][nb][c]);
    bm = rows4_max(bm);
    // Lazy running max: it moves only when the pair's max exceeds it by more
    // than kKiviLazyMax (probabilities stay below 2^8), so the accumulators
    // are rescaled only then; out = o / l and lse = m + log2(l) use the same m.
    const float m_old = m_lane;
    const float m_new = (bm > m_old + kKiviLazyMax) ? bm : m_old;
    const float ms = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_old - ms);
    m_lane = m_new;
    // P operand of block pb in registers: the block's V slots 8kg..8kg+7 are
    // tokens {4kg + c, 16 + 4kg + c} (c = 0..3), exactly this lane's scores
    float psum = 0.f;
    uint4 pa[2];
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      float p8[8];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          p8[4 * nb + c] = __builtin_amdgcn_exp2f(sv[pb][nb][c] - ms);
          psum += p8[4 * nb + c];
        }
      pa[pb] = make_uint4(pack2<DT>(p8[0], p8[1]), pack2<DT>(p8[2], p8[3]), pack2<DT>(p8[4], p8[5]),
                          pack2<DT>(p8[6], p8[7]));
    }
    l_lane = l_lane * alpha + psum;
    // ---- P.V: per block and group, codes against p*s and the zeros against p
    // (a head whose max was -inf holds zero accumulators: nothing to rescale)
    if (__builtin_amdgcn_read_exec() & __ballot(m_new != m_old && m_old != -INFINITY)) {  // some head's max moved
      // the output rows of this lane are heads 4kg + e; head r's factor sits on lane r
      float ar[REP];
#pragma unroll
      for (int r = 0; r < REP; ++r) ar[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), r));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float a = ar[min(e, REP - 1)];
#pragma unroll
        for (int q4 = 1; q4 < 4; ++q4)
          if (4 * q4 + e < REP) a = kg == q4 ? ar[4 * q4 + e] : a;
#pragma unroll
        for (int db = 0; db < DB; ++db) acc[db][e] *= a;
        if constexpr (DT == HALO_F16) {
#pragma unroll
          for (int gg = 0; gg < NG; ++gg) accz[gg][e] *= a;
        }
      }
    }
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      const char* bk = bkp + pb * BB;
#pragma unroll
      for (int gg = 0; gg < NG; ++gg) {
        const uint4 sv8 = *reinterpret_cast<const uint4*>(bk + VS + 2 * (gg * 32 + kg * 8));
        const uint4 zv8 = *reinterpret_cast<const uint4*>(bk + VZ + 2 * (gg * 32 + kg * 8));
        uint4 ps, ps_lo;
        if constexpr (DT == HALO_BF16) mul8_bf16_split(pa[pb], sv8, ps, ps_lo);
        else ps = mul8<DT>(kivi_prescale(pa[pb]), sv8);
#pragma unroll
        for (int d2 = 0; d2 < 2; ++d2) {
          const int db = 2 * gg + d2;
          const uint32_t c16 = *reinterpret_cast<const uint16_t*>(bk + VC + (db * 16 + hl) * 8 + kg * 2);
          const uint4 cd = DT == HALO_F16 ? kivi_codes8_sub_inplace(c16) : kivi_codes8_bf16(c16);
          acc[db] = MfmaOp<DT>::run(ps, cd, acc[db]);
          if constexpr (DT == HALO_BF16) {
            acc[db] = MfmaOp<DT>::run(ps_lo, cd, acc[db]);
            acc[db] = MfmaOp<DT>::run(pa[pb], zv8, acc[db]);
          }
        }
        // fp16: the code products carry 2^-24, so the zero term of the
        // group (equal for all its columns) accumulates on its own
        if constexpr (DT == HALO_F16) accz[gg] = MfmaOp<DT>::run(pa[pb], zv8, accz[gg]);
      }
    }
  };
  // Tiles are software-pipelined through registers one block pair at a
  // time: pair j of tile i is staged in the wave's raw LDS tile, the loads
  // of pair j of tile i+1 are issued into the same registers, and pair j is
  // computed while they and the rest of tile i are in flight.  The first
  // pair's compute so waits for a pair's bytes, not a whole tile's.
  constexpr int NSEG = TB / 2;     // block pairs per tile
  constexpr int LPS = LPT / NSEG;  // 16-byte loads per lane per pair
  static_assert(LPT % NSEG == 0 && LPS * 16 * kWave == 2 * BB, "a pair is a whole number of loads");
  char* raw = s_raw + wave * TBYTES;
  uint4 buf[LPT];
  auto load_pair = [&](int it, int sg) {
    const int64_t off = (int64_t)it * TBYTES;
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(base + wbyte0 + off, wbytes - off);
#pragma unroll
    for (int i = sg * LPS; i < (sg + 1) * LPS; ++i) buf[i] = buf_ld16(rr, (i * kWave + lane) * 16);
  };
  // Every wave of the launch starts at once: the prologue asks HBM for the
  // first pair only, so the queues hold one pair per wave and each wave's
  // first pair lands after about half a tile's worth of chip-wide traffic;
  // the rest of the first tile is asked for once that pair has landed.
  if (ntw > 0) load_pair(0, 0);
  for (int it = 0; it < ntw; ++it) {
    const int tok0 = t0 + (wb0 + it * TB) * 32;  // first token of the tile
#pragma unroll
    for (int sg = 0; sg < NSEG; ++sg) {
      // the previous reads of this pair's bytes were issued before these
      // stores (LDS serves one wave's instructions in order)
      asm volatile("" ::: "memory");
#pragma unroll
      for (int i = sg * LPS; i < (sg + 1) * LPS; ++i) *reinterpret_cast<uint4*>(raw + (i * kWave + lane) * 16) = buf[i];
      asm volatile("" ::: "memory");
      if (sg == 0 && it == 0) {
#pragma unroll
        for (int s2 = 1; s2 < NSEG; ++s2) load_pair(0, s2);
      }
      if (it + 1 < ntw) load_pair(it + 1, sg);
      // a pair past this wave's run belongs to the next wave (or to no one)
      if (tok0 + 2 * sg * 32 < wtok1) do_pair(raw + 2 * sg * BB, tok0 + 2 * sg * 32);
    }
  }
  float m_run[REP], l_head[REP];
  const float lsum = rows4_sum(l_lane);
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    m_run[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m_lane), r));
    l_head[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lsum), r));
  }
  if constexpr (DT == HALO_F16) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[db][e] = acc[db][e] * kSub16Scale + accz[db / 2][e];
  }
  write_partial_owners<D, REP, NW, DB, TBYTES / 4>(P, wslot, wave, true, true, acc, m_run, l_head, s_wo, s_wm, s_wl);
}

// ---------------------------------------------------------------------------
// Merge: one workgroup per (query-head group, head) combines that head's
// partials over the group's work items with the caller's accumulators and
// writes (m,l,o) and/or (out, lse).  A head's D columns are split over CS
// workgroups (blockIdx.z); thread t owns float4 column t % C4 of its
// workgroup's share and the partials p = t / C4 + k * TPC; it merges them
// online (its own running max), so every load is independent and the whole
// merge costs one memory round trip; the TPC per-thread results are then
// combined in a fixed order through LDS (deterministic run to run).  With
// CS > 1 every workgroup of a head reads the incoming accumulator and the
// first writes m/l, so a launch that both reads and writes m/l (acc_mode 3)
// runs with CS = 1.
// ---------------------------------------------------------------------------
template <int D, int REP, int NT, int MB, int CS>
__global__ void __launch_bounds__(NT) decode_merge_kernel(MergeParams P) {
  constexpr int C4A = D / 4;          // float4 columns of one head
  constexpr int C4 = C4A / CS;        // float4 columns of this workgroup
  constexpr int TPC = NT / C4;        // threads sharing a column
  static_assert(C4A % CS == 0 && NT % C4 == 0, "merge shape");
  __shared__ float4 s_o[NT];
  __shared__ float s_m[NT], s_l[NT];
  const int tid = threadIdx.x;
  const int g = blockIdx.x;
  const int r = blockIdx.y;
  const int sub = g % P.n_sub;
  const int bh = g / P.n_sub;
  const int h_kv = bh % P.H_kv;
  const int b = bh / P.H_kv;
  const int hq0 = h_kv * P.rep + sub * REP;
  if (r >= min(REP, P.rep - sub * REP)) return;  // padding head
  const int hq = hq0 + r;
  // uniform tables skip the offsets load (one dependent round trip)
  const int gbeg = P.group_offsets ? P.group_offsets[g] : g * P.per_group;
  const int gend = P.group_offsets ? P.group_offsets[g + 1] : gbeg + P.per_group;
  const int np = gend - gbeg;
  const bool has_acc = P.m != nullptr;
  const bool merge_in = has_acc && (P.acc_mode & 1);
  const bool write_acc = has_acc && (P.acc_mode & 2);
  const int64_t aidx = (int64_t)b * P.acc_stride_b + hq;
  const int col = tid % C4, phase = tid / C4;
  const int gcol = blockIdx.z * C4 + col;  // float4 column within the head

  float mt = -INFINITY, lt = 0.f;
  float4 ot = make_float4(0.f, 0.f, 0.f, 0.f);
  const float4* wo4 = reinterpret_cast<const float4*>(P.ws_o) + ((int64_t)gbeg * REP + r) * C4A + gcol;
  const float* wml = P.ws_ml + ((int64_t)gbeg * REP + r) * 2;
  // MB: partials per thread whose loads are issued together (one batch
  // covers TPC * MB partials of the group)
  // Loads are unconditional (the slot index is clamped into the group) so
  // the batch is issued back to back; slots past the group are masked in
  // the merge arithmetic.
  for (int p0 = phase; p0 < np; p0 += MB * TPC) {
    float2 ml[MB];
    float4 op[MB];
#pragma unroll
    for (int k = 0; k < MB; ++k) {
      const int pp = min(p0 + k * TPC, np - 1);
      ml[k] = *reinterpret_cast<const float2*>(wml + (int64_t)pp * REP * 2);
      op[k] = wo4[(int64_t)pp * REP * C4A];
    }
    // the batch's max first, then independent weights (one rescale of the
    // running values per batch instead of a dependent chain per partial)
    float mb = mt;
#pragma unroll
    for (int k = 0; k < MB; ++k)
      if (p0 + k * TPC < np) mb = fmaxf(mb, ml[k].x);
    const float ms = (mb == -INFINITY) ? 0.f : mb;
    const float a = __builtin_amdgcn_exp2f(mt - ms);
    lt *= a;
    ot.x *= a;
    ot.y *= a;
    ot.z *= a;
    ot.w *= a;
#pragma unroll
    for (int k = 0; k < MB; ++k) {
      if (p0 + k * TPC < np) {
        const float c = __builtin_amdgcn_exp2f(ml[k].x - ms);
        lt += ml[k].y * c;
        ot.x += op[k].x * c;
        ot.y += op[k].y * c;
        ot.z += op[k].z * c;
        ot.w += op[k].w * c;
      }
    }
    mt = mb;
  }
  // The incoming accumulator is read by every thread before the barrier:
  // the column-0 thread overwrites m/l after it.
  const float am = merge_in ? P.m[aidx] * kLog2e : -INFINITY;
  const float al = merge_in ? P.l[aidx] : 0.f;
  s_m[tid] = mt;
  s_l[tid] = lt;
  s_o[tid] = ot;
  __syncthreads();
  if (phase != 0) return;
  // combine the TPC partial merges of this column in phase order (every LDS
  // read issued first)
  float pm[TPC], pl[TPC];
  float4 po[TPC];
#pragma unroll
  for (int ph = 0; ph < TPC; ++ph) {
    pm[ph] = s_m[ph * C4 + col];
    pl[ph] = s_l[ph * C4 + col];
    po[ph] = s_o[ph * C4 + col];
  }
  float M = am;
#pragma unroll
  for (int ph = 0; ph < TPC; ++ph) M = fmaxf(M, pm[ph]);
  const float Ms = (M == -INFINITY) ? 0.f : M;
  float lsum = 0.f;
  float o4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ph = 0; ph < TPC; ++ph) {
    const float w = __builtin_amdgcn_exp2f(pm[ph] - Ms);
    lsum += w * pl[ph];
    o4[0] += w * po[ph].x;
    o4[1] += w * po[ph].y;
    o4[2] += w * po[ph].z;
    o4[3] += w * po[ph].w;
  }
  const int d0 = gcol * 4;
  const int64_t obase = aidx * D + d0;
  if (merge_in) {
    const float w = __builtin_amdgcn_exp2f(am - Ms);
#pragma unroll
    for (int e = 0; e < 4; ++e) o4[e] += w * P.o[obase + e];
    lsum += w * al;
  }
  if (write_acc) {
#pragma unroll
    for (int e = 0; e < 4; ++e) P.o[obase + e] = o4[e];
  }
  if (P.out != nullptr) {
    float ov[4];
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;  // one division per thread, then products
#pragma unroll
    for (int e = 0; e < 4; ++e) ov[e] = o4[e] * inv;
    const int64_t oi = ((int64_t)b * P.H + hq) * D + d0;
    if (P.out_vec) {
      store_elem4(P.out, oi, P.out_dtype, ov);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) store_elem(P.out, oi + e, P.out_dtype, ov[e]);
    }
  }
  if (d0 == 0) {
    if (P.lse != nullptr) P.lse[(int64_t)b * P.H + hq] = lsum > 0.f ? (M + log2f(lsum)) * kLn2 : -INFINITY;
    if (write_acc) {
      P.m[aidx] = (M == -INFINITY) ? -INFINITY : M * kLn2;
      P.l[aidx] = lsum;
    }
  }
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

constexpr int kWavesPerItem = 4;

template <int DT, int D, int REP>
int launch_decode(const DecodeParams& p, const MergeParams& mp, int n_work, int n_groups, bool kivi,
                  hipStream_t st) {
  if constexpr (DT != HALO_F32) {
    if (kivi) {
      hipLaunchKernelGGL((decode_attn_kivi_kernel<DT, D, REP, kWavesPerItem>), dim3(n_work),
                         dim3(64 * kWavesPerItem), 0, st, p);
    } else if (p.sel_wide) {
      hipLaunchKernelGGL((decode_attn_kernel<DT, D, REP, kWavesPerItem, true>), dim3(n_work),
                         dim3(64 * kWavesPerItem), 0, st, p);
    } else {
      hipLaunchKernelGGL((decode_attn_kernel<DT, D, REP, kWavesPerItem>), dim3(n_work), dim3(64 * kWavesPerItem),
                         0, st, p);
    }
  } else {
    hipLaunchKernelGGL((decode_attn_kernel<DT, D, REP, kWavesPerItem>), dim3(n_work), dim3(64 * kWavesPerItem), 0,
                       st, p);
  }
  HALO_CHECK_HIP(hipGetLastError());
  // The merge block and its load batch are sized so that one batch of loads
  // covers a group's partials where that is cheap; a second batch is a second
  // dependent round trip, but much larger batches measured slower (512 x 16
  // at 129 partials: +0.7 us).  Up to 144 partials per group, each head's
  // columns are split over small workgroups (one wave each): 32 columns and
  // 8 partials per thread up to 64 partials, 16 columns and 5 or 9 partials
  // per thread up to 80 / 144 (C2's 64: 17.15 -> 16.92 us per layer; the
  // 131072-token KIVI decode's 129: 22.8 -> 22.2 us; against one workgroup
  // of 256-512 threads per head).  Launches that both read and write the
  // caller's m/l keep one workgroup per head.
  const int per_group = (n_work + n_groups - 1) / n_groups;
  constexpr int C4 = D / 4;
  const bool split_ok = !(mp.m != nullptr && (mp.acc_mode & 3) == 3);
  if (split_ok && per_group <= 64) {
    constexpr int CS = D / 32;
    hipLaunchKernelGGL((decode_merge_kernel<D, REP, 64, 8, CS>), dim3(n_groups, REP, CS), dim3(64), 0, st, mp);
  } else if (split_ok && per_group <= 80) {
    constexpr int CS = D / 16;
    hipLaunchKernelGGL((decode_merge_kernel<D, REP, 64, 5, CS>), dim3(n_groups, REP, CS), dim3(64), 0, st, mp);
  } else if (split_ok && per_group <= 144) {
    constexpr int CS = D / 16;
    hipLaunchKernelGGL((decode_merge_kernel<D, REP, 64, 9, CS>), dim3(n_groups, REP, CS), dim3(64), 0, st, mp);
  } else if (per_group <= (256 / C4) * 8) {
    hipLaunchKernelGGL((decode_merge_kernel<D, REP, 256, 8, 1>), dim3(n_groups, REP), dim3(256), 0, st, mp);
  } else if (per_group > (512 / C4) * 8 && per_group <= (512 / C4) * 9) {
    hipLaunchKernelGGL((decode_merge_kernel<D, REP, 512, 9, 1>), dim3(n_groups, REP), dim3(512), 0, st, mp);
  } else {
    hipLaunchKernelGGL((decode_merge_kernel<D, REP, 512, 8, 1>), dim3(n_groups, REP), dim3(512), 0, st, mp);
  }
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}

template <int DT, int D>
int dispatch_rep(const DecodeParams& p, const MergeParams& mp, int rep_t, int n_work, int n_groups, bool kivi,
                 hipStream_t st) {
  switch (rep_t) {
    case 1: return launch_decode<DT, D, 1>(p, mp, n_work, n_groups, kivi, st);
    case 2: return launch_decode<DT, D, 2>(p, mp, n_work, n_groups, kivi, st);
    case 4: return launch_decode<DT, D, 4>(p, mp, n_work, n_groups, kivi, st);
    case 8: return launch_decode<DT, D, 8>(p, mp, n_work, n_groups, kivi, st);
  }
  set_error("rep_t must be 1, 2, 4 or 8");
  return HALO_E_UNSUPPORTED;
}

template <int DT>
int dispatch_d(const DecodeParams& p, const MergeParams& mp, int D, int rep_t, int n_work, int n_groups, bool kivi,
               hipStream_t st) {
  if (D == 64) return dispatch_rep<DT, 64>(p, mp, rep_t, n_work, n_groups, kivi, st);
  if (D == 128) return dispatch_rep<DT, 128>(p, mp, rep_t, n_work, n_groups, kivi, st);
  if constexpr (DT != HALO_F32) {
    if (D == 256) return dispatch_rep<DT, 256>(p, mp, rep_t, n_work, n_groups, kivi, st);
  }
  set_error("head_dim must be 64, 128 or 256 (256 for bf16/f16 only)");
  return HALO_E_UNSUPPORTED;
}

}  // namespace

namespace {

int decode_impl(const void* q, int64_t q_stride_b, int64_t q_stride_h, int dtype, int B, int H, int H_kv, int D,
                int rep_t, const halo_chunk_desc* descs, int n_desc, const int32_t* work, int n_work,
                const int32_t* group_offsets, int n_groups, const int64_t* q_pos, float scale, float* m, float* l,
                float* o, int64_t acc_stride_b, int acc_mode, void* out, int out_dtype, float* lse, void* workspace,
                size_t workspace_bytes, const halo_select_cfg* sel, bool kivi, void* stream) {
  HALO_CHECK_ARG(q && descs && work, "null pointer argument");
  HALO_CHECK_ARG(group_offsets || (n_groups > 0 && n_work % n_groups == 0),
                 "group_offsets may be NULL only when n_work is a multiple of n_groups");
  HALO_CHECK_ARG(!kivi || dtype == HALO_F16 || dtype == HALO_BF16, "KIVI chunks need fp16 or bf16 q and scales");
  HALO_CHECK_ARG(!(kivi && sel), "in-kernel selection is not available for KIVI chunk tables");
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
  p.B = B;
  p.H = H;
  p.H_kv = H_kv;
  p.rep = rep;
  p.n_sub = n_sub;
  p.descs = descs;
  p.work = work;
  p.n_work = n_work;
  p.q_pos = q_pos;
  p.scale2 = (float)((double)scale * 1.4426950408889634);
  {
    const int esz = elem_size(dtype);
    p.q_aligned = reinterpret_cast<uintptr_t>(q) % 16 == 0 && (q_stride_h * esz) % 16 == 0 &&
                  (q_stride_b * esz) % 16 == 0 && (D * esz) % 16 == 0;
  }
  p.ws_o = reinterpret_cast<float*>(workspace);
  p.ws_ml = p.ws_o + (size_t)n_work * rep_t * D;
  p.inv_rep = 1.0f / (float)rep;
  p.sel_on = sel != nullptr;
  p.sel = {};
  p.sel_wide = 0;
  if (sel) {
    const halo_select_cfg& S = *sel;
    const int esz = elem_size(dtype);
    const int rows = S.per_row ? 1 : B;
    HALO_CHECK_ARG(S.kmean && S.catalog, "selection needs kmean and catalog");
    const bool f32 = dtype == HALO_F32;
    HALO_CHECK_ARG(S.n_cold >= 1 && S.n_cold <= (f32 ? kSelMaxColdNarrow : kSelMaxColdWide),
                   "n_cold must be in [1, 128] (bf16/fp16) or [1, 64] (fp32)");
    HALO_CHECK_ARG(S.top_k >= 1 && S.slot0 >= 0 && S.slot0 + S.top_k <= n_desc,
                   "selection slots [slot0, slot0 + top_k) must lie in the chunk table");
    HALO_CHECK_ARG(S.catalog_stride >= S.n_cold, "catalog_stride < n_cold");
    HALO_CHECK_ARG(S.lead_items >= 0, "lead_items must be >= 0");
    HALO_CHECK_ARG(S.residency == nullptr || (S.slot_catalog != nullptr && S.n_slots >= 1 && S.n_slots <= kSelMaxSlots),
                   "staging needs slot_catalog and 1 <= n_slots <= 64");
    HALO_CHECK_ARG(S.n_cold * rows * H_kv <= (f32 ? kSelMaxTriplesNarrow : kSelMaxTriplesWide),
                   "n_cold * rows * H_kv must be <= 768 (bf16/fp16) or 512 (fp32)");
    HALO_CHECK_ARG(rows * H_kv * D <= kSelMaxQbar, "rows * H_kv * D must be <= 2048");
    HALO_CHECK_ARG(D % 16 == 0, "in-kernel selection needs head_dim % 16 == 0");
    HALO_CHECK_ARG(reinterpret_cast<uintptr_t>(S.kmean) % 16 == 0 && (S.km_stride_b * esz) % 16 == 0 &&
                       (S.km_stride_h * esz) % 16 == 0 && (S.km_stride_p * esz) % 16 == 0,
                   "kmean rows must be 16-byte aligned");
    p.sel = S;
    p.sel_wide = S.n_cold > kSelMaxColdNarrow || S.n_cold * rows * H_kv > kSelMaxTriplesNarrow;
  }
  MergeParams mp;
  mp.group_offsets = group_offsets;
  mp.per_group = n_groups > 0 ? n_work / n_groups : 0;
  mp.H = H;
  mp.H_kv = H_kv;
  mp.rep = rep;
  mp.n_sub = n_sub;
  mp.m = m;
  mp.l = l;
  mp.o = o;
  mp.acc_stride_b = acc_stride_b;
  mp.acc_mode = acc_mode;
  mp.out = out;
  mp.out_dtype = out_dtype;
  mp.out_vec = out != nullptr && reinterpret_cast<uintptr_t>(out) % (4 * elem_size(out_dtype)) == 0;
  mp.lse = lse;
  mp.ws_o = p.ws_o;
  mp.ws_ml = p.ws_ml;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (dtype) {
    case HALO_F32: return dispatch_d<HALO_F32>(p, mp, D, rep_t, n_work, n_groups, kivi, st);
    case HALO_BF16: return dispatch_d<HALO_BF16>(p, mp, D, rep_t, n_work, n_groups, kivi, st);
    default: return dispatch_d<HALO_F16>(p, mp, D, rep_t, n_work, n_groups, kivi, st);
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// Allocation-free decode: the split-K partials live in a file-scope device
// array instead of a caller workspace.  Each GPU holds its own copy of the
// array for the life of the process; its device address is looked up once
// per device (with that device current) and kept, and only that address is
// handed to kernels -- the array's name is a host-side stand-in.
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kScratchBytes = (size_t)8 << 20;
constexpr int kScratchDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};

// Device address of `scratch` on the device that runs `stream` (the current
// device for the null stream).
int scratch_address(hipStream_t stream, void** out) {
  int cur = 0;
  HALO_CHECK_HIP(hipGetDevice(&cur));
  int dev = cur;
  if (stream != nullptr) HALO_CHECK_HIP(hipStreamGetDevice(stream, &dev));
  HALO_CHECK_ARG(dev >= 0 && dev < kScratchDevices, "device index out of range for the static scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    if (dev != cur) HALO_CHECK_HIP(hipSetDevice(dev));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) HALO_CHECK_HIP(hipSetDevice(cur));
    if (e != hipSuccess || p == nullptr) {
      set_error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
      return HALO_E_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return HALO_OK;
}
}  // namespace

extern "C" size_t halo_decode_static_scratch_bytes(void) { return kScratchBytes; }

extern "C" int halo_decode_attn_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h, int dtype,
                                        int B, int H, int H_kv, int D, int rep_t,
                                        const halo_chunk_desc* descs, int n_desc,
                                        const int32_t* work, int n_work,
                                        const int32_t* group_offsets, int n_groups,
                                        const int64_t* q_pos, float scale,
                                        float* m, float* l, float* o, int64_t acc_stride_b, int acc_mode,
                                        void* out, int out_dtype, float* lse,
                                        const halo_select_cfg* sel, void* stream) {
  HALO_CHECK_ARG(n_work > 0 && rep_t > 0 && D > 0, "empty chunk table");
  const size_t need = halo_decode_workspace_size(n_work, rep_t, D);
  if (need > kScratchBytes) {
    set_error("halo_decode_attn_noalloc: " + std::to_string(need) + " bytes of partials for " +
              std::to_string(n_work) + " work items exceed the static scratch of " + std::to_string(kScratchBytes) +
              " bytes; use halo_decode_attn / halo_decode_attn_tiered with a workspace");
    return HALO_E_WORKSPACE;
  }
  void* ws = nullptr;
  const int rc = scratch_address(reinterpret_cast<hipStream_t>(stream), &ws);
  if (rc != HALO_OK) return rc;
  return decode_impl(q, q_stride_b, q_stride_h, dtype, B, H, H_kv, D, rep_t, descs, n_desc, work, n_work,
                     group_offsets, n_groups, q_pos, scale, m, l, o, acc_stride_b, acc_mode, out, out_dtype, lse,
                     ws, kScratchBytes, sel, false, stream);
}

extern "C" int halo_decode_attn(const void* q, int64_t q_stride_b, int64_t q_stride_h, int dtype,
                                int B, int H, int H_kv, int D, int rep_t,
                                const halo_chunk_desc* descs, int n_desc,
                                const int32_t* work, int n_work,
                                const int32_t* group_offsets, int n_groups,
                                const int64_t* q_pos, float scale,
                                float* m, float* l, float* o, int64_t acc_stride_b, int acc_mode,
                                void* out, int out_dtype, float* lse,
                                void* workspace, size_t workspace_bytes, void* stream) {
  return decode_impl(q, q_stride_b, q_stride_h, dtype, B, H, H_kv, D, rep_t, descs, n_desc, work, n_work,
                     group_offsets, n_groups, q_pos, scale, m, l, o, acc_stride_b, acc_mode, out, out_dtype, lse,
                     workspace, workspace_bytes, nullptr, false, stream);
}

extern "C" int halo_decode_attn_tiered(const void* q, int64_t q_stride_b, int64_t q_stride_h, int dtype,
                                       int B, int H, int H_kv, int D, int rep_t,
                                       const halo_chunk_desc* descs, int n_desc,
                                       const int32_t* work, int n_work,
                                       const int32_t* group_offsets, int n_groups,
                                       const int64_t* q_pos, float scale,
                                       float* m, float* l, float* o, int64_t acc_stride_b, int acc_mode,
                                       void* out, int out_dtype, float* lse,
                                       void* workspace, size_t workspace_bytes,
                                       const halo_select_cfg* sel, void* stream) {
  HALO_CHECK_ARG(sel != nullptr, "selection config is null");
  return decode_impl(q, q_stride_b, q_stride_h, dtype, B, H, H_kv, D, rep_t, descs, n_desc, work, n_work,
                     group_offsets, n_groups, q_pos, scale, m, l, o, acc_stride_b, acc_mode, out, out_dtype, lse,
                     workspace, workspace_bytes, sel, false, stream);
}

extern "C" int halo_decode_attn_kivi(const void* q, int64_t q_stride_b, int64_t q_stride_h, int dtype,
                                     int B, int H, int H_kv, int D, int rep_t,
                                     const halo_chunk_desc* descs, int n_desc,
                                     const int32_t* work, int n_work,
                                     const int32_t* group_offsets, int n_groups,
                                     const int64_t* q_pos, float scale,
                                     float* m, float* l, float* o, int64_t acc_stride_b, int acc_mode,
                                     void* out, int out_dtype, float* lse,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  return decode_impl(q, q_stride_b, q_stride_h, dtype, B, H, H_kv, D, rep_t, descs, n_desc, work, n_work,
                     group_offsets, n_groups, q_pos, scale, m, l, o, acc_stride_b, acc_mode, out, out_dtype, lse,
                     workspace, workspace_bytes, nullptr, true, stream);
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
