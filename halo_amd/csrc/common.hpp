// Shared device/host helpers for the HALO MI355X kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <mutex>
#include <string>

#include "../../include/halo_hip.h"

namespace halo {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kWave = 64;

// Thread-local error text behind halo_last_error().
void set_error(const std::string& msg);

#define HALO_CHECK_ARG(cond, msg)            \
  do {                                       \
    if (!(cond)) {                           \
      ::halo::set_error(msg);                \
      return HALO_E_INVALID;                 \
    }                                        \
  } while (0)

#define HALO_CHECK_HIP(expr)                                                       \
  do {                                                                             \
    hipError_t e_ = (expr);                                                        \
    if (e_ != hipSuccess) {                                                        \
      ::halo::set_error(std::string(#expr) + ": " + hipGetErrorString(e_));        \
      return HALO_E_HIP;                                                           \
    }                                                                              \
  } while (0)

inline int elem_size(int dtype) { return dtype == HALO_F32 ? 4 : 2; }

// ---------------------------------------------------------------------------
// Element conversions.  bf16 <-> fp32 are bit manipulations; the fp32 -> bf16
// direction rounds to nearest even, as torch's .to(torch.bfloat16) does.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u) {          // inf / nan
    return (uint16_t)((u >> 16) | ((u & 0xffffu) ? 0x40u : 0u));
  }
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return (float)v;
}
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
  _Float16 v = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
  return __builtin_bit_cast(uint16_t, v);
}

// Materialises an fp32 value in a register so the compiler cannot fold the
// operation that produced it into a later conversion (e.g. fptrunc(fmul) into
// one mixed-precision FMA that rounds once instead of twice).
__device__ __forceinline__ float opaque(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Store one fp32 value as element `dtype`.
__device__ __forceinline__ void store_elem(void* base, int64_t idx, int dtype, float v) {
  if (dtype == HALO_F32) {
    reinterpret_cast<float*>(base)[idx] = v;
  } else if (dtype == HALO_BF16) {
    reinterpret_cast<uint16_t*>(base)[idx] = f32_to_bf16_rne(v);
  } else {
    reinterpret_cast<uint16_t*>(base)[idx] = f32_to_f16_rne(v);
  }
}

// Store four consecutive fp32 values as elements `dtype` (idx a multiple of
// 4 and the row base 8-byte aligned for 16-bit types, 16-byte for fp32).
__device__ __forceinline__ void store_elem4(void* base, int64_t idx, int dtype, const float* v) {
  if (dtype == HALO_F32) {
    *reinterpret_cast<float4*>(reinterpret_cast<float*>(base) + idx) = make_float4(v[0], v[1], v[2], v[3]);
  } else if (dtype == HALO_BF16) {
    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(base) + idx) =
        make_uint2((uint32_t)f32_to_bf16_rne(v[0]) | ((uint32_t)f32_to_bf16_rne(v[1]) << 16),
                   (uint32_t)f32_to_bf16_rne(v[2]) | ((uint32_t)f32_to_bf16_rne(v[3]) << 16));
  } else {
    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(base) + idx) =
        make_uint2((uint32_t)f32_to_f16_rne(v[0]) | ((uint32_t)f32_to_f16_rne(v[1]) << 16),
                   (uint32_t)f32_to_f16_rne(v[2]) | ((uint32_t)f32_to_f16_rne(v[3]) << 16));
  }
}

__device__ __forceinline__ float load_elem(const void* base, int64_t idx, int dtype) {
  if (dtype == HALO_F32) return reinterpret_cast<const float*>(base)[idx];
  uint16_t h = reinterpret_cast<const uint16_t*>(base)[idx];
  return dtype == HALO_BF16 ? __uint_as_float((uint32_t)h << 16) : f16_bits_to_f32(h);
}

// ---------------------------------------------------------------------------
// Wave-level reductions (wave64).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Orders this wave's LDS writes before its later LDS reads (waves of a
// workgroup keep private LDS regions, so no s_barrier is needed).
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Max / sum over lanes l, l^16, l^32, l^48 (the four 16-lane rows of a
// wave) with the gfx950 lane-swap instructions: VALU only, no LDS round trip
// (a ds_bpermute shuffle is one).  Each swap returns both registers: for
// every lane one holds its own value and the other its partner's, so
// combining them gives the pair result in every lane.  The sum is
// (x + x^16) + (..)^32, the association of two xor shuffles (a + b == b + a).
__device__ __forceinline__ float rows4_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows4_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

}  // namespace halo
