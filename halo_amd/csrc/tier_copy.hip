// Batched block moves between the tiers of the cold-KV store (gfx950).
//
// A tier buffer holds fixed-size blocks (one block = one layer's K or V rows
// of `block_size` tokens for every KV head).  A move of many blocks is one
// launch that reads the block list on the device, so the caller's schedule
// (which blocks, from which tier) never goes through the host.  Either side
// may be pinned host memory addressed through its device-visible mapping:
// the DRAM tier is then read or written in place over the host link.
//
// Reference semantics: TieredStorage.move_block (halo/memory_tier.py:150-157)
// moves one block per call through torch copies; HALORefetcher._issue and
// HALODemoter.flush (halo/refetcher.py:102-114, halo/demoter.py:49-77) call it
// once per block from a Python loop.
#include "common.hpp"

namespace halo {
namespace {

constexpr int kCopyThreads = 256;
constexpr int64_t kCopyPiece = 64 * 1024;  // bytes per workgroup
constexpr int kCopyUnroll = 4;             // 16-byte loads in flight per thread

struct CopyPair {
  char* dst;
  const char* src;
};

__global__ void __launch_bounds__(kCopyThreads)
    copy_blocks_kernel(CopyPair p0, CopyPair p1, int64_t block_bytes, const int32_t* blocks, int n_blocks,
                       int64_t max_blocks, const int8_t* tier_of, int src_tier, int pieces) {
  const int item = blockIdx.x / pieces;
  const int piece = blockIdx.x % pieces;
  if (item >= n_blocks) return;
  const int32_t b = blocks[item];
  if (b < 0 || (int64_t)b >= max_blocks) return;
  if (tier_of != nullptr && (int)tier_of[b] != src_tier) return;
  const CopyPair pr = blockIdx.y == 0 ? p0 : p1;
  const int64_t lo = (int64_t)piece * kCopyPiece;
  const int64_t hi = min(lo + kCopyPiece, block_bytes);
  const uint4* s = reinterpret_cast<const uint4*>(pr.src + (int64_t)b * block_bytes + lo);
  uint4* d = reinterpret_cast<uint4*>(pr.dst + (int64_t)b * block_bytes + lo);
  const int n16 = (int)((hi - lo) / 16);
  for (int base = 0; base < n16; base += kCopyThreads * kCopyUnroll) {
    uint4 r[kCopyUnroll];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const int j = base + u * kCopyThreads + (int)threadIdx.x;
      if (j < n16) r[u] = s[j];
    }
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const int j = base + u * kCopyThreads + (int)threadIdx.x;
      if (j < n16) d[j] = r[u];
    }
  }
}

__global__ void __launch_bounds__(kCopyThreads)
    set_tier_kernel(int8_t* tier_of, const int32_t* blocks, int n_blocks, int64_t max_blocks, int src_tier,
                    int dst_tier) {
  const int i = blockIdx.x * kCopyThreads + (int)threadIdx.x;
  if (i >= n_blocks) return;
  const int32_t b = blocks[i];
  if (b < 0 || (int64_t)b >= max_blocks) return;
  // A duplicate entry may already have written dst_tier: the store is the
  // same either way.
  if (src_tier >= 0 && (int)tier_of[b] != src_tier && (int)tier_of[b] != dst_tier) return;
  tier_of[b] = (int8_t)dst_tier;
}

}  // namespace
}  // namespace halo

using namespace halo;

extern "C" int halo_set_tier(int8_t* tier_of, const int32_t* blocks, int n_blocks, int64_t max_blocks,
                             int src_tier, int dst_tier, void* stream) {
  HALO_CHECK_ARG(n_blocks >= 0, "n_blocks < 0");
  if (n_blocks == 0) return HALO_OK;
  HALO_CHECK_ARG(tier_of && blocks, "null pointer argument");
  HALO_CHECK_ARG(max_blocks > 0, "max_blocks must be positive");
  HALO_CHECK_ARG(dst_tier >= 0 && dst_tier < 128 && src_tier < 128, "tier codes must fit int8");
  const unsigned grid = (unsigned)((n_blocks + kCopyThreads - 1) / kCopyThreads);
  hipLaunchKernelGGL(set_tier_kernel, dim3(grid), dim3(kCopyThreads), 0, static_cast<hipStream_t>(stream), tier_of,
                     blocks, n_blocks, max_blocks, src_tier, dst_tier);
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}

extern "C" int halo_copy_blocks(void* dst_k, const void* src_k, void* dst_v, const void* src_v,
                                int64_t block_bytes, const int32_t* blocks, int n_blocks, int64_t max_blocks,
                                const int8_t* tier_of, int src_tier, void* stream) {
  HALO_CHECK_ARG(n_blocks >= 0, "n_blocks < 0");
  if (n_blocks == 0) return HALO_OK;
  HALO_CHECK_ARG(dst_k && src_k && blocks, "null pointer argument");
  HALO_CHECK_ARG((dst_v == nullptr) == (src_v == nullptr), "dst_v and src_v must both be set or both NULL");
  HALO_CHECK_ARG(block_bytes > 0 && block_bytes % 16 == 0, "block_bytes must be a positive multiple of 16");
  HALO_CHECK_ARG(max_blocks > 0, "max_blocks must be positive");
  auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  HALO_CHECK_ARG(aligned(dst_k) && aligned(src_k) && aligned(dst_v) && aligned(src_v),
                 "tier buffers must be 16-byte aligned");
  const int64_t pieces = (block_bytes + kCopyPiece - 1) / kCopyPiece;
  HALO_CHECK_ARG(pieces * n_blocks < (int64_t)1 << 31, "too many blocks for one launch");
  const dim3 grid((unsigned)(pieces * n_blocks), dst_v ? 2u : 1u);
  const CopyPair p0{static_cast<char*>(dst_k), static_cast<const char*>(src_k)};
  const CopyPair p1{static_cast<char*>(dst_v ? dst_v : dst_k), static_cast<const char*>(src_v ? src_v : src_k)};
  hipLaunchKernelGGL(copy_blocks_kernel, grid, dim3(kCopyThreads), 0, static_cast<hipStream_t>(stream), p0, p1,
                     block_bytes, blocks, n_blocks, max_blocks, tier_of, src_tier, (int)pieces);
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}

// ---------------------------------------------------------------------------
// Staging-cache helpers: a batch of host-to-device chunk copies in one call,
// and a batch of int32 stores whose (index, value) pairs travel in the kernel
// arguments (no host buffer has to outlive the call).
// ---------------------------------------------------------------------------
namespace halo {
namespace {
constexpr int kStorePairs = 32;
struct StorePairs {
  int64_t idx[kStorePairs];
  int32_t val[kStorePairs];
  int n;
};

__global__ void store_i32_kernel(int32_t* base, int64_t n_elems, StorePairs p) {
  const int i = threadIdx.x;
  if (i < p.n && p.idx[i] >= 0 && p.idx[i] < n_elems) base[p.idx[i]] = p.val[i];
}

// Fills read by a kernel: up to kFillBatch fills per launch, each split into
// K and V tensors of `pieces` 64 KiB pieces; workgroup w copies piece
// w % pieces of tensor (w / pieces) % 2 of fill w / (2 * pieces).  Pieces of
// one fill are dispatched together, so the batch's fills land in list order.
constexpr int kFillBatch = 16;
struct FillBatch {
  halo_fill f[kFillBatch];
  int n;
  int pieces;  // pieces per tensor (of the largest fill in the batch)
};

__global__ void __launch_bounds__(kCopyThreads) fill_read_kernel(FillBatch b) {
  const int per_fill = 2 * b.pieces;
  const int fi = blockIdx.x / per_fill;
  if (fi >= b.n) return;
  const int r = blockIdx.x % per_fill;
  const halo_fill& f = b.f[fi];
  const bool v = r >= b.pieces;
  const int piece = v ? r - b.pieces : r;
  const char* src = static_cast<const char*>(v ? f.src_v : f.src_k);
  char* dst = static_cast<char*>(v ? f.dst_v : f.dst_k);
  if (src == nullptr || dst == nullptr) return;
  const int64_t lo = (int64_t)piece * kCopyPiece;
  if (lo >= f.bytes) return;
  const int64_t hi = min(lo + kCopyPiece, f.bytes);
  const uint4* s = reinterpret_cast<const uint4*>(src + lo);
  uint4* d = reinterpret_cast<uint4*>(dst + lo);
  const int n16 = (int)((hi - lo) / 16);
  for (int base = 0; base < n16; base += kCopyThreads * kCopyUnroll) {
    uint4 t[kCopyUnroll];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const int j = base + u * kCopyThreads + (int)threadIdx.x;
      if (j < n16) t[u] = s[j];
    }
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const int j = base + u * kCopyThreads + (int)threadIdx.x;
      if (j < n16) d[j] = t[u];
    }
  }
}
}  // namespace
}  // namespace halo

extern "C" int halo_stage_fills(const halo_fill* fills, int n, void* stream) {
  HALO_CHECK_ARG(n >= 0 && (n == 0 || fills != nullptr), "bad fill list");
  hipStream_t st = static_cast<hipStream_t>(stream);
  for (int i = 0; i < n; ++i) {
    const halo_fill& f = fills[i];
    HALO_CHECK_ARG(f.bytes >= 0 && (f.bytes == 0 || (f.dst_k && f.src_k)), "fill: null pointer");
    if (f.bytes == 0) continue;
    HALO_CHECK_HIP(hipMemcpyAsync(f.dst_k, f.src_k, (size_t)f.bytes, hipMemcpyHostToDevice, st));
    if (f.dst_v != nullptr) HALO_CHECK_HIP(hipMemcpyAsync(f.dst_v, f.src_v, (size_t)f.bytes, hipMemcpyHostToDevice, st));
  }
  return HALO_OK;
}

extern "C" int halo_stage_fills_read(const halo_fill* fills, int n, void* stream) {
  HALO_CHECK_ARG(n >= 0 && (n == 0 || fills != nullptr), "bad fill list");
  auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  for (int i0 = 0; i0 < n; i0 += kFillBatch) {
    FillBatch b{};
    b.n = n - i0 < kFillBatch ? n - i0 : kFillBatch;
    int64_t most = 0;
    for (int j = 0; j < b.n; ++j) {
      const halo_fill& f = fills[i0 + j];
      HALO_CHECK_ARG(f.bytes >= 0 && f.bytes % 16 == 0, "fill: bytes must be a non-negative multiple of 16");
      HALO_CHECK_ARG(f.bytes == 0 || (f.dst_k && f.src_k), "fill: null pointer");
      HALO_CHECK_ARG(aligned(f.dst_k) && aligned(f.src_k) && aligned(f.dst_v) && aligned(f.src_v),
                     "fill: addresses must be 16-byte aligned");
      HALO_CHECK_ARG((f.dst_v == nullptr) == (f.src_v == nullptr), "fill: dst_v and src_v must both be set or NULL");
      b.f[j] = f;
      most = f.bytes > most ? f.bytes : most;
    }
    if (most == 0) continue;
    b.pieces = (int)((most + kCopyPiece - 1) / kCopyPiece);
    HALO_CHECK_ARG((int64_t)b.pieces * 2 * b.n < (int64_t)1 << 31, "fill too large");
    hipLaunchKernelGGL(fill_read_kernel, dim3((unsigned)(2 * b.pieces * b.n)), dim3(kCopyThreads), 0,
                       static_cast<hipStream_t>(stream), b);
    HALO_CHECK_HIP(hipGetLastError());
  }
  return HALO_OK;
}

extern "C" int halo_store_i32(int32_t* base, int64_t n_elems, const int64_t* idx, const int32_t* vals, int n,
                              void* stream) {
  HALO_CHECK_ARG(n >= 0 && (n == 0 || (base && idx && vals)), "null pointer argument");
  for (int i0 = 0; i0 < n; i0 += kStorePairs) {
    StorePairs p;
    p.n = n - i0 < kStorePairs ? n - i0 : kStorePairs;
    for (int j = 0; j < kStorePairs; ++j) {
      p.idx[j] = j < p.n ? idx[i0 + j] : -1;
      p.val[j] = j < p.n ? vals[i0 + j] : 0;
    }
    hipLaunchKernelGGL(store_i32_kernel, dim3(1), dim3(kStorePairs), 0, static_cast<hipStream_t>(stream), base,
                       n_elems, p);
    HALO_CHECK_HIP(hipGetLastError());
  }
  return HALO_OK;
}
