// KIVI-style 2/4/8-bit cold-chunk format: quantize and dequantize kernels
// (gfx950, wave64).  Byte/integer work bound by HBM; nothing here is a GEMM.
//
// Arithmetic: baselines/kivi_cache.py:44-78 with every operation rounded to
// the storage dtype as torch evaluates a chain of fp16/bf16 tensor ops:
//   scale = dtype(dtype(max(dtype(x_max - x_min), dtype(1e-8))) / qmax)
//   zero  = x_min
//   code  = clamp(rint(dtype(dtype(x - zero) / scale)), 0, qmax), NaN -> 0
//   x'    = dtype(fp32(fp32(code) * fp32(scale)) + fp32(zero))
// (built with -ffp-contract=off: no fused multiply-add anywhere).
// K is grouped per channel over 32 consecutive tokens, V per token over 32
// consecutive channels (the reference groups along the last axis only,
// kivi_cache.py:56; K per-channel applies the same per-element arithmetic
// along the token axis).
//
// Block layout (one block = 32 tokens of one (b, h_kv); byte offsets):
//   [0, C)            K codes, token-major rows of D*bits/8 bytes (code
//                     positions within a row below)
//   [C, C+2D)         K scale, D elements of the dtype (per channel)
//   [C+2D, C+4D)      K zero
//   [C+4D, 2C+4D)     V codes, channel-major rows of 32*bits/8 bytes, one
//                     code per token slot
//   [2C+4D, 2C+6D)    V scale, D/32 groups x 32 token slots (group-major)
//   [2C+6D, 2C+8D)    V zero
// with C = 32*D*bits/8.  D=128, bits=2: 3072 bytes per block.  The V side
// is transposed, and its 32 tokens are stored in slot order: slot 8g + j
// holds token 4g + j (j < 4) or 16 + 4g + j - 4 (j >= 4), the tokens one
// lane group g of a 16x16x32 MFMA holds in its score accumulator (rows
// 4g..4g+3 of both 16-token halves).  So the P.V operand of one lane is 8
// slots = 16 contiguous bits of one channel, its scales (or zeros) are 16
// contiguous bytes of one group, and its p values are its own scores.
// Code positions within a row: 4- and 8-bit codes, element e at bit e*bits
// (8-bit: one byte per code); 2-bit
// codes, each 16-bit word holds 8 elements, the even ones (2j) at bits 2j
// of its low byte and the odd ones (2j+1) at bits 8+2j of its high byte, so
// that w | w << 8 holds elements 2j and 2j+1 at bits 2j and 16+2j: one mask
// places a pair in the two fp16 halves of a register.

#include "common.hpp"

namespace halo {

constexpr int kKiviG = 32;

// token held by V slot s of a block, and the slot of token t
__host__ __device__ constexpr int kivi_vtok(int s) { return (s & 4 ? 16 : 0) + 4 * (s >> 3) + (s & 3); }
__host__ __device__ constexpr int kivi_vslot(int t) { return 8 * ((t >> 2) & 3) + 4 * (t >> 4) + (t & 3); }
static_assert(kivi_vslot(kivi_vtok(13)) == 13 && kivi_vtok(kivi_vslot(21)) == 21, "V slot order");

// element (within its row) of the code at bits [c*BITS, (c+1)*BITS) of byte q
// of the row, and the bit position of element e (its inverse)
template <int BITS>
__host__ __device__ constexpr int kivi_elem(int q, int c) {
  return BITS == 2 ? (q & ~1) * 4 + 2 * c + (q & 1) : q * (8 / BITS) + c;
}
template <int BITS>
__host__ __device__ constexpr int kivi_bit(int e) {
  return BITS == 2 ? 16 * (e >> 3) + 2 * ((e & 7) >> 1) + 8 * (e & 1) : e * BITS;
}
static_assert(kivi_bit<2>(kivi_elem<2>(5, 3)) == 5 * 8 + 3 * 2 && kivi_bit<2>(kivi_elem<2>(6, 1)) == 6 * 8 + 2 &&
                  kivi_bit<4>(kivi_elem<4>(3, 1)) == 3 * 8 + 4,
              "code positions");

__host__ __device__ constexpr int kivi_code_bytes(int D, int bits) { return kKiviG * D * bits / 8; }
__host__ __device__ constexpr int kivi_block_bytes(int D, int bits) { return 2 * kivi_code_bytes(D, bits) + 8 * D; }

template <int DT>
__device__ __forceinline__ float round_dt(float x) {
  if constexpr (DT == HALO_BF16) return __uint_as_float((uint32_t)f32_to_bf16_rne(x) << 16);
  return f16_bits_to_f32(f32_to_f16_rne(x));
}
template <int DT>
__device__ __forceinline__ uint16_t bits_dt(float x) {
  if constexpr (DT == HALO_BF16) return f32_to_bf16_rne(x);
  return f32_to_f16_rne(x);
}
template <int DT>
__device__ __forceinline__ float from_bits(uint16_t h) {
  if constexpr (DT == HALO_BF16) return __uint_as_float((uint32_t)h << 16);
  return f16_bits_to_f32(h);
}

// scale/zero of one group from its (dtype-exact) min and max
template <int DT, int BITS>
__device__ __forceinline__ void kivi_params(float mn, float mx, float& scale, float& zero) {
  constexpr float qmax = (float)((1 << BITS) - 1);
  const float eps = round_dt<DT>(1e-8f);
  float rng = round_dt<DT>(opaque(mx - mn));
  rng = round_dt<DT>(fmaxf(rng, eps));
  scale = round_dt<DT>(opaque(rng / qmax));
  zero = mn;
}
template <int DT, int BITS>
__device__ __forceinline__ uint32_t kivi_code(float x, float scale, float zero) {
  constexpr float qmax = (float)((1 << BITS) - 1);
  const float diff = round_dt<DT>(opaque(x - zero));
  float ratio = round_dt<DT>(opaque(diff / scale));
  if (ratio != ratio) ratio = 0.f;
  const float c = fminf(fmaxf(rintf(ratio), 0.f), qmax);
  return (uint32_t)c;
}

struct KiviQuantParams {
  const void* k;
  int64_t ksb, ksh, kst;
  const void* v;
  int64_t vsb, vsh, vst;
  int H_kv, n_blk;
  uint8_t* blocks;
  int64_t bsb, bsh;  // bytes
  int vec16;         // K and V rows 16-byte aligned: tiles loaded with 16-byte loads
};

// Code of x for a group with precomputed inv = 1/scale (correctly rounded):
// clamp(rint(dtype(dtype(x - zero) / scale)), 0, qmax).  The fp32 quotient
// is formed without a division: q = d * inv, r = fma(-q, scale, d),
// q' = fma(r, inv, q) equals the correctly rounded d / scale whenever d
// (a dtype value >= 0) is 0 or in [2^-63, 2^63] and scale is in [2^-63,
// 2^63] -- checked exhaustively for every pair of fp16 and bf16 values.
// Outside that range (a zero scale, extreme bf16 values) the division runs.
__device__ __forceinline__ float kivi_scale_ok(float scale) {
  return scale >= 0x1p-63f && scale <= 0x1p63f ? 1.f : 0.f;
}
// p = (scale, 1/scale, zero, kivi_scale_ok(scale))
template <int DT, int BITS>
__device__ __forceinline__ uint32_t kivi_code_fma(float x, float4 p) {
  constexpr float qmax = (float)((1 << BITS) - 1);
  const float scale = p.x, inv = p.y, zero = p.z;
  const float d = round_dt<DT>(opaque(x - zero));
  const bool s_ok = p.w != 0.f;
  const bool ok = DT == HALO_F16 ? s_ok : (s_ok && (d == 0.f || (d >= 0x1p-63f && d <= 0x1p63f)));
  float q;
  if (ok) {
    const float q0 = opaque(d * inv);
    const float r = __builtin_fmaf(-q0, scale, d);
    q = __builtin_fmaf(r, inv, q0);
  } else {
    q = opaque(d / scale);
  }
  if constexpr (DT == HALO_F16) {
    // ratio in fp16; NaN -> 0 through the IEEE max, codes in [0, qmax]
    const _Float16 r16 = (_Float16)q;
    _Float16 c16 = __builtin_rintf16(r16);
    c16 = __builtin_fminf16(__builtin_fmaxf16(c16, (_Float16)0.f), (_Float16)qmax);
    return (uint32_t)(unsigned short)c16;
  } else {
    const float ratio = round_dt<DT>(q);
    return (uint32_t)fminf(fmaxf(rintf(ratio), 0.f), qmax);
  }
}

// Store a thread's NB packed code bytes (NB in {2, 4, 8, 16, 32}; dst aligned
// to min(NB, 16) bytes) with vector stores.
template <int NB>
__device__ __forceinline__ void store_codes(uint8_t* dst, const uint64_t (&acc)[4]) {
  static_assert(NB == 2 || NB == 4 || NB == 8 || NB == 16 || NB == 32, "packed code bytes per thread");
  if constexpr (NB == 2) {
    *reinterpret_cast<uint16_t*>(dst) = (uint16_t)acc[0];
  } else if constexpr (NB == 4) {
    *reinterpret_cast<uint32_t*>(dst) = (uint32_t)acc[0];
  } else if constexpr (NB == 8) {
    *reinterpret_cast<uint64_t*>(dst) = acc[0];
  } else {
#pragma unroll
    for (int h = 0; h < NB / 16; ++h)
      reinterpret_cast<uint4*>(dst)[h] = make_uint4((uint32_t)acc[2 * h], (uint32_t)(acc[2 * h] >> 32),
                                                    (uint32_t)acc[2 * h + 1], (uint32_t)(acc[2 * h + 1] >> 32));
  }
}

// One workgroup per block, 256 threads.  The 32 x D K and V tiles are staged
// in LDS in their storage dtype (16-byte loads; rows padded by 16 bytes so
// column and row-run reads spread over the banks); pairs of threads reduce
// each K channel and each V (token, 32-channel group) to its min / max;
// then each thread codes a run of consecutive elements of one output row
// and stores its packed bytes in one store (K rows token-major, V rows
// channel-major in slot order), so every global access is a vector access.
template <int DT, int D, int BITS>
__global__ void __launch_bounds__(256) kivi_quantize_kernel(KiviQuantParams P) {
  constexpr int G = kKiviG;
  constexpr int C = kivi_code_bytes(D, BITS);
  constexpr int NG = D / G;                  // V groups per token
  constexpr int RS = D + 8;                  // LDS row stride (elements)
  constexpr int KR = G * D / 256;            // elements per thread per code run: 8, 16 or 32
  constexpr int KP = D + D / KR;             // padded params (one float4 per channel, a pad per run)
  __shared__ __align__(16) uint16_t s_k[G * RS], s_v[G * RS];
  __shared__ float s_kmn[2][D], s_kmx[2][D], s_vmn[2][G * NG], s_vmx[2][G * NG];
  __shared__ __align__(16) float4 s_kp[KP];  // (scale, 1/scale, zero, scale in range) per channel
  __shared__ __align__(16) float4 s_vp[G * NG];
  const int tid = threadIdx.x;
  const int j = blockIdx.x % P.n_blk;
  const int bh = blockIdx.x / P.n_blk;
  const int h = bh % P.H_kv, b = bh / P.H_kv;
  const uint16_t* kb = reinterpret_cast<const uint16_t*>(P.k) + (int64_t)b * P.ksb + (int64_t)h * P.ksh +
                       (int64_t)j * G * P.kst;
  const uint16_t* vb = reinterpret_cast<const uint16_t*>(P.v) + (int64_t)b * P.vsb + (int64_t)h * P.vsh +
                       (int64_t)j * G * P.vst;
  if (P.vec16) {
    constexpr int PR = D / 8;  // 16-byte pieces per row
    uint4 kk[G * PR / 256], vv[G * PR / 256];
#pragma unroll
    for (int i = 0; i < G * PR / 256; ++i) {
      const int e = tid + 256 * i, t = e / PR, c = e % PR;
      kk[i] = *reinterpret_cast<const uint4*>(kb + (int64_t)t * P.kst + 8 * c);
      vv[i] = *reinterpret_cast<const uint4*>(vb + (int64_t)t * P.vst + 8 * c);
    }
#pragma unroll
    for (int i = 0; i < G * PR / 256; ++i) {
      const int e = tid + 256 * i, t = e / PR, c = e % PR;
      *reinterpret_cast<uint4*>(&s_k[t * RS + 8 * c]) = kk[i];
      *reinterpret_cast<uint4*>(&s_v[t * RS + 8 * c]) = vv[i];
    }
  } else {
    for (int e = tid; e < G * D; e += 256) {
      const int t = e / D, d = e % D;
      s_k[t * RS + d] = kb[(int64_t)t * P.kst + d];
      s_v[t * RS + d] = vb[(int64_t)t * P.vst + d];
    }
  }
  __syncthreads();
  // min / max: K per (channel, half of the tokens), V per (token, group, half of the channels)
  for (int i = tid; i < 2 * D; i += 256) {
    const int d = i % D, hf = i / D;
    float mn = from_bits<DT>(s_k[(16 * hf) * RS + d]), mx = mn;
#pragma unroll
    for (int t = 1; t < 16; ++t) {
      const float x = from_bits<DT>(s_k[(16 * hf + t) * RS + d]);
      mn = fminf(mn, x);
      mx = fmaxf(mx, x);
    }
    s_kmn[hf][d] = mn;
    s_kmx[hf][d] = mx;
  }
  for (int i = tid; i < 2 * G * NG; i += 256) {
    const int tg = i >> 1, hf = i & 1;
    const int t = tg / NG, g = tg % NG;
    const uint4* row = reinterpret_cast<const uint4*>(&s_v[t * RS + g * G + 16 * hf]);
    const uint4 r0 = row[0], r1 = row[1];
    const uint32_t w[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
    float mn = from_bits<DT>((uint16_t)w[0]), mx = mn;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const float lo = from_bits<DT>((uint16_t)w[c]), hi = from_bits<DT>((uint16_t)(w[c] >> 16));
      mn = fminf(mn, fminf(lo, hi));
      mx = fmaxf(mx, fmaxf(lo, hi));
    }
    s_vmn[hf][tg] = mn;
    s_vmx[hf][tg] = mx;
  }
  __syncthreads();
  uint8_t* out = P.blocks + (int64_t)b * P.bsb + (int64_t)h * P.bsh + (int64_t)j * kivi_block_bytes(D, BITS);
  uint16_t* meta_k = reinterpret_cast<uint16_t*>(out + C);
  uint16_t* meta_v = reinterpret_cast<uint16_t*>(out + 2 * C + 4 * D);
  for (int d = tid; d < D; d += 256) {
    float sc, z;
    kivi_params<DT, BITS>(fminf(s_kmn[0][d], s_kmn[1][d]), fmaxf(s_kmx[0][d], s_kmx[1][d]), sc, z);
    s_kp[d + d / KR] = make_float4(sc, 1.0f / sc, z, kivi_scale_ok(sc));
    meta_k[d] = bits_dt<DT>(sc);
    meta_k[D + d] = bits_dt<DT>(z);
  }
  for (int tg = tid; tg < G * NG; tg += 256) {
    float sc, z;
    kivi_params<DT, BITS>(fminf(s_vmn[0][tg], s_vmn[1][tg]), fmaxf(s_vmx[0][tg], s_vmx[1][tg]), sc, z);
    s_vp[tg] = make_float4(sc, 1.0f / sc, z, kivi_scale_ok(sc));
    const int t = tg / NG, g = tg % NG;
    meta_v[g * G + kivi_vslot(t)] = bits_dt<DT>(sc);            // group-major, slot order
    meta_v[G * NG + g * G + kivi_vslot(t)] = bits_dt<DT>(z);
  }
  __syncthreads();
  // K codes: 32 rows x D elements; thread = (token, run of KR consecutive
  // channels starting at a multiple of 8), KR * BITS bits stored at once
  constexpr int RKB = D * BITS / 8;          // K code bytes per token row
  {
    const int t = tid / (D / KR), e0 = (tid % (D / KR)) * KR;
    uint64_t acc[4] = {0, 0, 0, 0};          // up to 256 bits (32 elements x 8 bits)
    const uint4* row = reinterpret_cast<const uint4*>(&s_k[t * RS + e0]);
#pragma unroll
    for (int v8 = 0; v8 < KR / 8; ++v8) {
      const uint4 r = row[v8];
      const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int e = e0 + 8 * v8 + i;
        const float4 pk = s_kp[e + e / KR];
        const uint16_t xb = (uint16_t)(i & 1 ? w[i >> 1] >> 16 : w[i >> 1]);
        const uint32_t c = kivi_code_fma<DT, BITS>(from_bits<DT>(xb), pk);
        const int bit = kivi_bit<BITS>(8 * v8 + i);          // e0 is a multiple of 8
        acc[bit >> 6] |= (uint64_t)c << (bit & 63);
      }
    }
    uint8_t* dst = out + t * RKB + kivi_bit<BITS>(e0) / 8;
    store_codes<KR * BITS / 8>(dst, acc);
  }
  // V codes: D rows (channels) x 32 slots; thread = (channel, run of VR
  // consecutive slots starting at a multiple of 8)
  constexpr int VR = G * D / 256;
  constexpr int VRB = G * BITS / 8;          // V code bytes per channel row
  {
    const int d = tid / (G / VR), s0 = (tid % (G / VR)) * VR;
    const int g = d / G;
    uint64_t acc[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < VR; ++i) {
      const int s = s0 + i, t = kivi_vtok(s);
      const float4 pv = s_vp[t * NG + g];
      const uint32_t c = kivi_code_fma<DT, BITS>(from_bits<DT>(s_v[t * RS + d]), pv);
      const int bit = kivi_bit<BITS>(s) - kivi_bit<BITS>(s0);
      acc[bit >> 6] |= (uint64_t)c << (bit & 63);
    }
    uint8_t* dst = out + C + 4 * D + d * VRB + kivi_bit<BITS>(s0) / 8;
    store_codes<VR * BITS / 8>(dst, acc);
  }
}

struct KiviDequantParams {
  const uint8_t* blocks;
  int64_t bsb, bsh;
  int H_kv, n_blk;
  void* k;
  int64_t ksb, ksh, kst;
  void* v;
  int64_t vsb, vsh, vst;
};

// One workgroup per block; one thread per (token, 8-channel piece) of K and V.
template <int DT, int D, int BITS>
__global__ void __launch_bounds__(256) kivi_dequant_kernel(KiviDequantParams P) {
  constexpr int G = kKiviG;
  constexpr int C = kivi_code_bytes(D, BITS);
  constexpr int NG = D / G;
  constexpr uint32_t MASK = (1u << BITS) - 1;
  const int tid = threadIdx.x;
  const int j = blockIdx.x % P.n_blk;
  const int bh = blockIdx.x / P.n_blk;
  const int h = bh % P.H_kv, b = bh / P.H_kv;
  const uint8_t* blk = P.blocks + (int64_t)b * P.bsb + (int64_t)h * P.bsh + (int64_t)j * kivi_block_bytes(D, BITS);
  const uint16_t* meta_k = reinterpret_cast<const uint16_t*>(blk + C);
  const uint16_t* meta_v = reinterpret_cast<const uint16_t*>(blk + 2 * C + 4 * D);
  uint16_t* ko = reinterpret_cast<uint16_t*>(P.k) + (int64_t)b * P.ksb + (int64_t)h * P.ksh + (int64_t)j * G * P.kst;
  uint16_t* vo = reinterpret_cast<uint16_t*>(P.v) + (int64_t)b * P.vsb + (int64_t)h * P.vsh + (int64_t)j * G * P.vst;
  for (int e = tid; e < G * D; e += 256) {
    const int t = e / D, d = e % D;
    const int bit = kivi_bit<BITS>(d);
    const uint32_t ck = (blk[t * (D * BITS / 8) + bit / 8] >> (bit % 8)) & MASK;
    const int ts = kivi_vslot(t);
    const int tbit = kivi_bit<BITS>(ts);
    const uint32_t cv = (blk[C + 4 * D + d * (G * BITS / 8) + tbit / 8] >> (tbit % 8)) & MASK;
    const float sk = from_bits<DT>(meta_k[d]), zk = from_bits<DT>(meta_k[D + d]);
    const float sv = from_bits<DT>(meta_v[(d / G) * G + ts]), zv = from_bits<DT>(meta_v[G * NG + (d / G) * G + ts]);
    // both fp32 results are materialised so the conversion rounds the fp32
    // sum (no mixed-precision fused add-and-convert)
    ko[(int64_t)t * P.kst + d] = bits_dt<DT>(opaque(opaque((float)ck * sk) + zk));
    vo[(int64_t)t * P.vst + d] = bits_dt<DT>(opaque(opaque((float)cv * sv) + zv));
  }
}

}  // namespace halo

using namespace halo;

extern "C" size_t halo_kivi_block_bytes(int D, int bits) {
  if ((bits != 2 && bits != 4 && bits != 8) || D <= 0 || D % kKiviG) return 0;
  return (size_t)kivi_block_bytes(D, bits);
}

namespace {

template <int DT, int D>
int quant_bits(const KiviQuantParams& p, int bits, int n, hipStream_t st) {
  if (bits == 2) hipLaunchKernelGGL((kivi_quantize_kernel<DT, D, 2>), dim3(n), dim3(256), 0, st, p);
  else if (bits == 4) hipLaunchKernelGGL((kivi_quantize_kernel<DT, D, 4>), dim3(n), dim3(256), 0, st, p);
  else hipLaunchKernelGGL((kivi_quantize_kernel<DT, D, 8>), dim3(n), dim3(256), 0, st, p);
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}
template <int DT, int D>
int dequant_bits(const KiviDequantParams& p, int bits, int n, hipStream_t st) {
  if (bits == 2) hipLaunchKernelGGL((kivi_dequant_kernel<DT, D, 2>), dim3(n), dim3(256), 0, st, p);
  else if (bits == 4) hipLaunchKernelGGL((kivi_dequant_kernel<DT, D, 4>), dim3(n), dim3(256), 0, st, p);
  else hipLaunchKernelGGL((kivi_dequant_kernel<DT, D, 8>), dim3(n), dim3(256), 0, st, p);
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}

}  // namespace

extern "C" int halo_kivi_quantize(const void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
                                  const void* v, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_t,
                                  int dtype, int B, int H_kv, int T, int D, int bits,
                                  void* blocks, int64_t blk_stride_b, int64_t blk_stride_h, void* stream) {
  HALO_CHECK_ARG(k && v && blocks, "null pointer");
  HALO_CHECK_ARG(dtype == HALO_F16 || dtype == HALO_BF16, "KIVI storage dtype must be fp16 or bf16");
  HALO_CHECK_ARG(bits == 2 || bits == 4 || bits == 8, "bits must be 2, 4 or 8");
  HALO_CHECK_ARG(D == 64 || D == 128 || D == 256, "head_dim must be 64, 128 or 256");
  HALO_CHECK_ARG(B >= 0 && H_kv > 0 && T >= 0 && T % kKiviG == 0, "T must be a multiple of the group size 32");
  const int n_blk = T / kKiviG;
  const int64_t n = (int64_t)B * H_kv * n_blk;
  if (n == 0) return HALO_OK;
  HALO_CHECK_ARG(n < (1ll << 31), "too many blocks");
  auto a16 = [](const void* p, int64_t stride_elems) {
    return (reinterpret_cast<uintptr_t>(p) & 15) == 0 && (stride_elems * 2) % 16 == 0;
  };
  const int vec16 = a16(k, k_stride_t) && a16(v, v_stride_t) && (k_stride_b * 2) % 16 == 0 &&
                    (k_stride_h * 2) % 16 == 0 && (v_stride_b * 2) % 16 == 0 && (v_stride_h * 2) % 16 == 0;
  HALO_CHECK_ARG((reinterpret_cast<uintptr_t>(blocks) & 15) == 0 && blk_stride_b % 16 == 0 && blk_stride_h % 16 == 0,
                 "block buffer must be 16-byte aligned");
  KiviQuantParams p{k, k_stride_b, k_stride_h, k_stride_t, v, v_stride_b, v_stride_h, v_stride_t,
                    H_kv, n_blk, reinterpret_cast<uint8_t*>(blocks), blk_stride_b, blk_stride_h, vec16};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == HALO_F16) {
    if (D == 64) return quant_bits<HALO_F16, 64>(p, bits, (int)n, st);
    if (D == 128) return quant_bits<HALO_F16, 128>(p, bits, (int)n, st);
    return quant_bits<HALO_F16, 256>(p, bits, (int)n, st);
  }
  if (D == 64) return quant_bits<HALO_BF16, 64>(p, bits, (int)n, st);
  if (D == 128) return quant_bits<HALO_BF16, 128>(p, bits, (int)n, st);
  return quant_bits<HALO_BF16, 256>(p, bits, (int)n, st);
}

extern "C" int halo_kivi_dequantize(const void* blocks, int64_t blk_stride_b, int64_t blk_stride_h,
                                    int dtype, int B, int H_kv, int n_blocks, int D, int bits,
                                    void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
                                    void* v, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_t,
                                    void* stream) {
  HALO_CHECK_ARG(k && v && blocks, "null pointer");
  HALO_CHECK_ARG(dtype == HALO_F16 || dtype == HALO_BF16, "KIVI storage dtype must be fp16 or bf16");
  HALO_CHECK_ARG(bits == 2 || bits == 4 || bits == 8, "bits must be 2, 4 or 8");
  HALO_CHECK_ARG(D == 64 || D == 128 || D == 256, "head_dim must be 64, 128 or 256");
  HALO_CHECK_ARG(B >= 0 && H_kv > 0 && n_blocks >= 0, "bad sizes");
  const int64_t n = (int64_t)B * H_kv * n_blocks;
  if (n == 0) return HALO_OK;
  HALO_CHECK_ARG(n < (1ll << 31), "too many blocks");
  KiviDequantParams p{reinterpret_cast<const uint8_t*>(blocks), blk_stride_b, blk_stride_h, H_kv, n_blocks,
                      k, k_stride_b, k_stride_h, k_stride_t, v, v_stride_b, v_stride_h, v_stride_t};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == HALO_F16) {
    if (D == 64) return dequant_bits<HALO_F16, 64>(p, bits, (int)n, st);
    if (D == 128) return dequant_bits<HALO_F16, 128>(p, bits, (int)n, st);
    return dequant_bits<HALO_F16, 256>(p, bits, (int)n, st);
  }
  if (D == 64) return dequant_bits<HALO_BF16, 64>(p, bits, (int)n, st);
  if (D == 128) return dequant_bits<HALO_BF16, 128>(p, bits, (int)n, st);
  return dequant_bits<HALO_BF16, 256>(p, bits, (int)n, st);
}
