// HALOScorer on the GPU: the closed-form hotness score and a sorted top-k
// (gfx950, wave64).  Reduction and selection work over one score vector per
// call; nothing here is a GEMM.
//
// Reference semantics:
//   score    halo/scorer.py:36-72   attn/(sum+1e-12), recency
//            exp(-clamp(step-p,0)/max(refresh,1))/(sum+1e-12), sink[:n] = 1,
//            (alpha*attn + beta*rec + gamma*sink)/(max+1e-12), all fp32
//   top-k    halo/scorer.py:74-88, halo/refetcher.py:38-57: indices of the k
//            largest scores, sorted ascending; ties (left undefined by
//            torch.topk) go to the lower index; NaN ranks as -inf.

#include "common.hpp"

namespace halo {

namespace {

constexpr int kScoreNT = 1024;

__device__ __forceinline__ float block_sum(float v, float* s_red) {
  v = wave_sum(v);
  const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  __syncthreads();
  if (lane == 0) s_red[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < kScoreNT / kWave; ++i) t += s_red[i];  // fixed order: deterministic
  return t;
}
__device__ __forceinline__ float block_max(float v, float* s_red) {
  v = wave_max(v);
  const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  __syncthreads();
  if (lane == 0) s_red[w] = v;
  __syncthreads();
  float t = -INFINITY;
  for (int i = 0; i < kScoreNT / kWave; ++i) t = fmaxf(t, s_red[i]);
  return t;
}

__global__ void __launch_bounds__(kScoreNT) halo_score_kernel(const float* attn, int K, float step, float alpha,
                                                               float beta, float gamma, int sink, float decay,
                                                               float* score) {
  __shared__ float s_red[kScoreNT / kWave];
  const int tid = threadIdx.x;
  // Contiguous per-thread ranges, summed in index order.
  const int per = (K + kScoreNT - 1) / kScoreNT;
  const int i0 = min(K, tid * per), i1 = min(K, i0 + per);
  float sa = 0.f, sr = 0.f;
  for (int i = i0; i < i1; ++i) {
    sa += attn[i];
    sr += expf(-fmaxf(step - (float)i, 0.f) / decay);
  }
  const float inv_a = opaque(block_sum(sa, s_red) + 1e-12f);
  const float inv_r = opaque(block_sum(sr, s_red) + 1e-12f);
  float mx = -INFINITY;
  for (int i = i0; i < i1; ++i) {
    const float a = opaque(attn[i] / inv_a);
    const float r = opaque(expf(-fmaxf(step - (float)i, 0.f) / decay) / inv_r);
    const float sk = i < sink ? 1.f : 0.f;
    const float s = opaque(opaque(opaque(alpha * a) + opaque(beta * r)) + opaque(gamma * sk));
    score[i] = s;
    mx = fmaxf(mx, s);
  }
  const float den = opaque(block_max(mx, s_red) + 1e-12f);
  for (int i = i0; i < i1; ++i) score[i] = score[i] / den;
}

// Order-preserving key of a float (NaN ranks as -inf).
__device__ __forceinline__ uint32_t okey(float x) {
  if (x != x) x = -INFINITY;
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exclusive prefix sum over the workgroup's threads (in thread order).
__device__ __forceinline__ int block_exclusive_scan(int v, int* s_wave) {
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  int x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  __syncthreads();
  if (lane == kWave - 1) s_wave[w] = x;  // wave totals
  __syncthreads();
  int base = 0;
  for (int i = 0; i < w; ++i) base += s_wave[i];
  return base + x - v;
}

// One workgroup: 4 radix passes of 8 bits find the k-th largest key T and
// how many keys equal to T are to be taken; a counting pass over contiguous
// index ranges then writes the chosen indices in ascending order (ties
// resolved by lower index).
__global__ void __launch_bounds__(kScoreNT) topk_sorted_kernel(const float* score, int K, int k, int64_t* idx) {
  __shared__ uint32_t s_hist[256];
  __shared__ uint32_t s_prefix, s_need;
  __shared__ int s_wave[kScoreNT / kWave];
  const int tid = threadIdx.x;
  if (tid == 0) {
    s_prefix = 0;
    s_need = (uint32_t)k;
  }
  uint32_t mask = 0;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    if (tid < 256) s_hist[tid] = 0;
    __syncthreads();
    const uint32_t prefix = s_prefix;
    for (int i = tid; i < K; i += kScoreNT) {
      const uint32_t key = okey(score[i]);
      if ((key & mask) == prefix) atomicAdd(&s_hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      // largest digit d with (#keys of digit > d) < need <= (#keys of digit >= d)
      uint32_t above = 0, need = s_need;
      int d = 255;
      for (; d > 0; --d) {
        if (above + s_hist[d] >= need) break;
        above += s_hist[d];
      }
      s_need = need - above;
      s_prefix = prefix | ((uint32_t)d << shift);
    }
    mask |= 255u << shift;
    __syncthreads();
  }
  const uint32_t T = s_prefix;
  const int need_eq = (int)s_need;
  const int per = (K + kScoreNT - 1) / kScoreNT;
  const int i0 = min(K, tid * per), i1 = min(K, i0 + per);
  int n_gt = 0, n_eq = 0;
  for (int i = i0; i < i1; ++i) {
    const uint32_t key = okey(score[i]);
    n_gt += key > T;
    n_eq += key == T;
  }
  const int eq_before = block_exclusive_scan(n_eq, s_wave);
  // equal keys this range contributes: those whose rank among equals < need_eq
  const int eq_take = max(0, min(n_eq, need_eq - eq_before));
  const int pos0 = block_exclusive_scan(n_gt + eq_take, s_wave);
  int pos = pos0, eq_seen = 0;
  for (int i = i0; i < i1; ++i) {
    const uint32_t key = okey(score[i]);
    bool chosen = key > T;
    if (key == T) {
      chosen = eq_seen < eq_take;
      ++eq_seen;
    }
    if (chosen) idx[pos++] = i;
  }
}

}  // namespace

}  // namespace halo

using namespace halo;

extern "C" int halo_halo_score(const float* attention, int K, int step, float alpha, float beta, float gamma,
                               int sink_tokens, int refresh_window, float* score, void* stream) {
  HALO_CHECK_ARG(attention && score, "null pointer");
  HALO_CHECK_ARG(K > 0 && K <= (1 << 24), "K must be in [1, 2^24]");
  const float decay = (float)(refresh_window > 1 ? refresh_window : 1);
  const int sink = sink_tokens > 0 ? (sink_tokens < K ? sink_tokens : K) : 0;
  hipLaunchKernelGGL(halo_score_kernel, dim3(1), dim3(kScoreNT), 0, reinterpret_cast<hipStream_t>(stream),
                     attention, K, (float)step, alpha, beta, gamma, sink, decay, score);
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}

extern "C" int halo_topk_sorted(const float* score, int K, int k, int64_t* idx_out, void* stream) {
  HALO_CHECK_ARG(score && idx_out, "null pointer");
  HALO_CHECK_ARG(K > 0 && K <= (1 << 24), "K must be in [1, 2^24]");
  HALO_CHECK_ARG(k >= 1 && k <= K, "k must be in [1, K]");
  hipLaunchKernelGGL(topk_sorted_kernel, dim3(1), dim3(kScoreNT), 0, reinterpret_cast<hipStream_t>(stream), score,
                     K, k, idx_out);
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}
