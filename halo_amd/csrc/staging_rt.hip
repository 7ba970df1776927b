// Host runtime of the HBM staging cache for cold chunks kept in pinned host
// memory: feedback ring, hit/miss accounting, the fill/evict policy, fill
// issue and residency commits, one C call per segment of layers.
//
// The kernels that consume it are the fused selection of
// halo_decode_attn_tiered (residency entries, slot catalog, feedback row);
// this file enqueues work on HIP streams (fill copies and their events, and
// one small boundary kernel per segment) and keeps the host mirror of the
// cache.
//
// Segment boundary: halo_staging_after only marks the segment's feedback rows
// for publication; the next halo_staging_before on the same stream enqueues
// ONE kernel that stores the batched residency entries and copies the marked
// rows into a pinned host ring entry, then sets that entry's sequence word
// (system-scope release).  The host polls the word instead of waiting on an
// event: a device-to-host copy plus an event record cost ~8 us of stream
// time per segment, a store launch ~5 us more, the one kernel ~5 us.
//
// The unit of the cache is a selection: one per layer, or one per batch row
// of a layer with per-row selection (B selections per layer, each over its
// own row's cold chunks with its own slots).  Unit u = layer * B + row.
//
// Reference policy: HALORefetcher.predict_hot / schedule / _issue / wait
// (halo/refetcher.py:38-114): the next hot set is the top (hot + lookahead)
// by the last score, and what is missing is fetched on a side stream.  Here
// the scores are the ones the selection itself wrote, the predicted set is
// the `keep` best per layer, and the fetch is a chunk copy into an HBM slot.
//
// Ordering (no kernel observes a change while it runs):
//  * a fill copies a chunk into a slot that no residency entry names, on a
//    copy stream, followed by an event (each slot has its own event, and a
//    filling slot is never evicted or refilled, so fills on different copy
//    streams need no order among themselves);
//  * a fill is committed (its residency entry stored on the compute stream)
//    before the next launches of its layer once its event has completed --
//    or at once after a compute-stream wait for the event when it is urgent
//    (the chunk was among the layer's current top-k, so the next launch
//    would otherwise read it over the link);
//  * evictions are decided only for layers whose feedback rows came back:
//    every launch of such a layer has finished (the kernel that published
//    the rows ran behind it) and its next launch is not enqueued yet, so the
//    slot can take a fill at once; the -1 store waits for the layer's next
//    halo_staging_before and goes out in the same batched store as that
//    call's commits, ahead of them, so it precedes every later read.
#include <algorithm>
#include <chrono>
#include <numeric>
#include <thread>
#include <vector>

#include "common.hpp"

namespace halo {
namespace {

enum : int8_t { kFree = 0, kFilling = 1, kReady = 2, kReserved = 4 };

struct Pending {
  int unit, chunk, slot;
  bool urgent;
};

}  // namespace
}  // namespace halo

struct halo_staging {
  int L = 0, B = 1, U = 0, n = 0, S = 0, k = 0, keep = 0, max_inflight = 0, spare = 0, ring_n = 0, W = 0;
  bool wa = false, kernel_fills = false, track_busy = false;
  int32_t* dev_i32 = nullptr;  // residency (U * n) then the write-allocate slot per layer (L)
  const float* feedback = nullptr;
  hipStream_t copy = nullptr, urgent = nullptr, copy2 = nullptr;
  uint32_t fill_seq = 0;  // regular DMA fills issued (alternates the copy streams)
  std::vector<uint64_t> dst, src;       // (U, S, 2) slot K/V, (U, n, 2) chunk K/V addresses
  std::vector<int64_t> nbytes;          // (U, n) bytes per K (or V) tensor
  std::vector<int32_t> ncold;           // (U) cold chunks of each unit (<= n)
  std::vector<float*> ring;             // pinned (L, W) rows per ring entry
  std::vector<float*> ring_dev;         // the same rows' device-visible addresses
  uint64_t* ring_seq = nullptr;         // pinned: entry r's sequence word at [r * 8]
  uint64_t* ring_seq_dev = nullptr;
  std::vector<hipStream_t> ring_stream; // stream of the kernel that publishes entry r
  std::vector<std::pair<int, int>> ring_rows;
  int64_t queued = 0, seen = 0;
  int64_t launched = 0;                 // entries [0, launched) have their publish enqueued
  std::vector<int64_t> slot_of, holds, last_rank, wa_slot, launches, processed;
  std::vector<int8_t> state;
  std::vector<hipEvent_t> fill_ev;      // (U, S): the event of the slot's fill in flight
  std::vector<halo::Pending> pending;
  halo_staging_stats st{};
  // scratch reused across calls
  std::vector<int64_t> idx_buf;
  std::vector<int32_t> val_buf;
  // eviction stores held for the unit's next halo_staging_before
  std::vector<int64_t> def_idx;
  std::vector<int32_t> def_val;
  std::vector<int> def_unit;

  int64_t& slot_of_at(int u, int c) { return slot_of[(size_t)u * n + c]; }
  int8_t& state_at(int u, int s) { return state[(size_t)u * S + s]; }
  int64_t& holds_at(int u, int s) { return holds[(size_t)u * S + s]; }
  int64_t chunk_bytes(int u, int c) const { return 2 * nbytes[(size_t)u * n + c]; }
  // feedback of layer li within a row block: scores (B, n) | picks (B, k) | residency used (B, k)
  const float* fb_scores(const float* layer_row, int r) const { return layer_row + (size_t)r * n; }
  const int32_t* fb_idx(const float* layer_row, int r) const {
    return reinterpret_cast<const int32_t*>(layer_row + (size_t)B * n + (size_t)r * k);
  }
  const int32_t* fb_res(const float* layer_row, int r) const {
    return reinterpret_cast<const int32_t*>(layer_row + (size_t)B * n + (size_t)B * k + (size_t)r * k);
  }
};

namespace halo {
namespace {

int64_t now_ns() {
  return std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

bool stream_busy(hipStream_t s) {
  const hipError_t e = hipStreamQuery(s);
  if (e == hipErrorNotReady) {
    (void)hipGetLastError();
    return true;
  }
  return false;
}

// Move the held eviction stores of units [ulo, uhi) into the store batch
// (ahead of any commit added after them).
void take_deferred(halo_staging* h, int ulo, int uhi) {
  size_t w = 0;
  for (size_t i = 0; i < h->def_idx.size(); ++i) {
    if (ulo <= h->def_unit[i] && h->def_unit[i] < uhi) {
      h->idx_buf.push_back(h->def_idx[i]);
      h->val_buf.push_back(h->def_val[i]);
    } else {
      h->def_idx[w] = h->def_idx[i];
      h->def_val[w] = h->def_val[i];
      h->def_unit[w] = h->def_unit[i];
      ++w;
    }
  }
  h->def_idx.resize(w);
  h->def_val.resize(w);
  h->def_unit.resize(w);
}

// One segment boundary on the compute stream: up to kBoundaryPairs residency
// stores and, when `seq` is set, the publication of feedback rows into a
// pinned ring entry followed by its sequence word.  One workgroup.
constexpr int kBoundaryPairs = 32;
constexpr int kBoundaryThreads = 256;
struct BoundaryArgs {
  const float* src;   // device feedback rows
  float* dst;         // device-visible address of the ring entry's rows
  uint64_t* seq;      // device-visible address of its sequence word; NULL: no publication
  uint64_t seq_val;
  int32_t* base;      // residency entries
  int64_t n_elems;
  int n_floats, n_pairs;
  int64_t idx[kBoundaryPairs];
  int32_t val[kBoundaryPairs];
};

__global__ void __launch_bounds__(kBoundaryThreads) boundary_kernel(BoundaryArgs a) {
  const int t = threadIdx.x;
  if (t < a.n_pairs && a.idx[t] >= 0 && a.idx[t] < a.n_elems) a.base[a.idx[t]] = a.val[t];
  if (a.seq == nullptr) return;  // uniform
  // System-scope stores write through to host memory; the wait for their
  // acknowledgements, then the barrier, order every row before the sequence
  // word without a fence (a release fence would also write back the L2's
  // dirty lines of the preceding launches).
  const uint32_t* src = reinterpret_cast<const uint32_t*>(a.src);
  uint32_t* dst = reinterpret_cast<uint32_t*>(a.dst);
  for (int i = t; i < a.n_floats; i += kBoundaryThreads)
    __hip_atomic_store(dst + i, src[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (t == 0) __hip_atomic_store(a.seq, a.seq_val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Enqueue a boundary kernel on `st`: the residency pairs [i0, i0 + cnt) of
// the store batch and, with `publish`, the oldest unpublished ring entry.
int launch_boundary(halo_staging* h, hipStream_t st, bool publish, size_t i0, int cnt) {
  BoundaryArgs a{};
  a.base = h->dev_i32;
  a.n_elems = (int64_t)h->U * h->n + h->L;
  a.n_pairs = cnt;
  for (int j = 0; j < cnt; ++j) {
    a.idx[j] = h->idx_buf[i0 + j];
    a.val[j] = h->val_buf[i0 + j];
  }
  if (publish) {
    const int64_t e = h->launched;
    const int r = (int)(e % h->ring_n);
    const int lo = h->ring_rows[r].first, hi = h->ring_rows[r].second;
    const size_t off = (size_t)lo * h->W;
    a.src = h->feedback + off;
    a.dst = h->ring_dev[r] + off;
    a.n_floats = (int)((size_t)(hi - lo) * h->W);
    a.seq = h->ring_seq_dev + (size_t)r * 8;
    a.seq_val = (uint64_t)(e + 1);
    h->launched += 1;
  }
  hipLaunchKernelGGL(boundary_kernel, dim3(1), dim3(kBoundaryThreads), 0, st, a);
  HALO_CHECK_HIP(hipGetLastError());
  return HALO_OK;
}

// Publish the marked entries up to the first one on `compute` (all of them
// when `all`), each alone on its own stream, behind the launches it follows.
int publish_marked(halo_staging* h, hipStream_t compute, bool all) {
  while (h->launched < h->queued) {
    const hipStream_t ps = h->ring_stream[(size_t)(h->launched % h->ring_n)];
    if (ps == compute && !all) break;
    const int rc = launch_boundary(h, ps, true, 0, 0);
    if (rc != HALO_OK) return rc;
  }
  return HALO_OK;
}

// The batched residency store and the pending feedback publication on
// `compute`, as few boundary kernels as the batch needs (usually one).
int store(halo_staging* h, hipStream_t compute) {
  int rc = publish_marked(h, compute, false);
  if (rc != HALO_OK) return rc;
  const size_t n = h->idx_buf.size();
  size_t i0 = 0;
  while (rc == HALO_OK && (i0 < n || h->launched < h->queued)) {
    const int cnt = (int)std::min<size_t>(kBoundaryPairs, n - i0);
    rc = launch_boundary(h, compute, h->launched < h->queued, i0, cnt);
    i0 += cnt;
  }
  h->idx_buf.clear();
  h->val_buf.clear();
  return rc;
}

// Wait until ring entry `e` has been published: a spin on its sequence
// word.  After 2 ms the stream that carries the publication is queried once
// per millisecond (a query is not free: it is kept off the normal path), so a
// failed or drained stream ends the wait with an error instead of a hang.
int wait_entry(halo_staging* h, int64_t e) {
  const int r = (int)(e % h->ring_n);
  volatile uint64_t* w = h->ring_seq + (size_t)r * 8;
  const uint64_t want = (uint64_t)(e + 1);
  const int64_t t0 = now_ns();
  int64_t next_query = t0 + 2000000;
  for (int64_t spin = 0;; ++spin) {
    if (__atomic_load_n(w, __ATOMIC_ACQUIRE) >= want) return HALO_OK;
    __builtin_ia32_pause();
    if ((spin & 1023) != 1023) continue;
    const int64_t t = now_ns();
    if (t < next_query) continue;
    next_query = t + 1000000;
    const hipError_t q = hipStreamQuery(h->ring_stream[r]);
    if (q == hipSuccess) {
      if (__atomic_load_n(w, __ATOMIC_ACQUIRE) >= want) return HALO_OK;
      set_error("staging feedback: the publishing stream drained without the entry's sequence word");
      return HALO_E_HIP;
    }
    if (q != hipErrorNotReady) HALO_CHECK_HIP(q);
    (void)hipGetLastError();
    std::this_thread::yield();
  }
}

bool entry_ready(const halo_staging* h, int64_t e) {
  const volatile uint64_t* w = h->ring_seq + (size_t)(e % h->ring_n) * 8;
  return __atomic_load_n(w, __ATOMIC_ACQUIRE) >= (uint64_t)(e + 1);
}

// Give every empty write-allocate reservation a free slot (highest index
// first, away from the fills, which take the lowest).  One selection per
// layer only (B == 1: unit == layer).
void reserve_wa(halo_staging* h) {
  if (!h->wa) return;
  for (int li = 0; li < h->L; ++li) {
    for (int q = 0; q < 2; ++q) {
      if (h->wa_slot[(size_t)li * 2 + q] >= 0) continue;
      for (int s = h->S - 1; s >= 0; --s) {
        if (h->state_at(li, s) == kFree) {
          h->state_at(li, s) = kReserved;
          h->wa_slot[(size_t)li * 2 + q] = s;
          break;
        }
      }
    }
  }
}

// Hit/miss accounting of the feedback rows of layers [lo, hi) (`fb` points
// at layer lo's row) and the commits of slots the kernel wrote
// (write-allocate).
int account(halo_staging* h, const float* fb, int lo, int hi, hipStream_t compute) {
  const int n = h->n, k = h->k;
  for (int li = lo; li < hi; ++li) h->processed[li] += 1;
  bool committed = false;
  for (int li = lo; li < hi; ++li) {
    const float* row = fb + (size_t)(li - lo) * h->W;
    for (int r = 0; r < h->B; ++r) {
      const int u = li * h->B + r;
      const int32_t* idx = h->fb_idx(row, r);
      const int32_t* res = h->fb_res(row, r);
      for (int j = 0; j < k; ++j) {
        const int c = idx[j];
        if (c < 0 || c >= h->ncold[u]) continue;
        const int rr = res[j];
        if (rr >= 0) {
          h->st.hits += 1;
          continue;
        }
        h->st.misses += 1;
        h->st.miss_bytes += h->chunk_bytes(u, c);
        if (h->last_rank[(size_t)u * n + c] < h->keep) h->st.misses_predicted += 1;
        if (h->wa && rr <= -2) {
          const int w = -2 - rr;
          int q = -1;
          for (int t = 0; t < 2; ++t)
            if (h->wa_slot[(size_t)li * 2 + t] == w) q = t;
          if (q < 0) continue;  // not a current reservation: nothing to commit
          if (h->slot_of_at(u, c) >= 0) {
            h->st.wa_dups += 1;  // staged or filling elsewhere meanwhile: keep the reservation
            continue;
          }
          h->state_at(u, w) = kReady;
          h->holds_at(u, w) = c;
          h->slot_of_at(u, c) = w;
          h->idx_buf.push_back((int64_t)u * n + c);
          h->val_buf.push_back(w);
          h->wa_slot[(size_t)li * 2 + q] = -1;
          h->st.wa_commits += 1;
          committed = true;
        }
      }
    }
  }
  if (committed) {
    if (h->track_busy && stream_busy(compute)) h->st.commits_while_busy += 1;
    const int rc = store(h, compute);
    if (rc != HALO_OK) return rc;
    reserve_wa(h);
  }
  return HALO_OK;
}

int issue(halo_staging* h, const Pending& p) {
  hipStream_t s = (p.urgent && h->urgent != nullptr) ? h->urgent : h->copy;
  // DMA fills alternate between the two copy streams (two engines overlap
  // each copy's start-up)
  if (s == h->copy && h->copy2 != nullptr && !h->kernel_fills && (h->fill_seq++ & 1)) s = h->copy2;
  const size_t sk = ((size_t)p.unit * h->S + p.slot) * 2, ck = ((size_t)p.unit * h->n + p.chunk) * 2;
  const int64_t nb = h->nbytes[(size_t)p.unit * h->n + p.chunk];
  halo_fill f;
  f.dst_k = reinterpret_cast<void*>(h->dst[sk]);
  f.dst_v = reinterpret_cast<void*>(h->dst[sk + 1]);
  f.src_k = reinterpret_cast<const void*>(h->src[ck]);
  f.src_v = reinterpret_cast<const void*>(h->src[ck + 1]);
  f.bytes = nb;
  if (h->src[ck + 1] == h->src[ck] + (uint64_t)nb && h->dst[sk + 1] == h->dst[sk] + (uint64_t)nb) {
    f.bytes = 2 * nb;  // K rows then V rows on both sides: one copy
    f.dst_v = nullptr;
    f.src_v = nullptr;
  }
  const int64_t t0 = now_ns();
  const int rc = h->kernel_fills ? halo_stage_fills_read(&f, 1, s) : halo_stage_fills(&f, 1, s);
  h->st.ns_issue += now_ns() - t0;
  if (rc != HALO_OK) return rc;
  HALO_CHECK_HIP(hipEventRecord(h->fill_ev[(size_t)p.unit * h->S + p.slot], s));
  h->pending.push_back(p);
  return HALO_OK;
}

// Plan evictions and fills for the units whose feedback was just processed
// (one score row of n per unit in `sc`, in the order of `units`).
int plan(halo_staging* h, const std::vector<int>& units, const std::vector<float>& sc, hipStream_t compute) {
  const int n = h->n, S = h->S;
  std::vector<int> order(n);
  std::vector<int64_t> rank((size_t)units.size() * n);
  struct Miss {
    int64_t rank;
    int unit, chunk, row;
  };
  std::vector<Miss> missing;
  for (size_t i = 0; i < units.size(); ++i) {
    const int u = units[i], nu = h->ncold[u];
    const float* s = sc.data() + i * n;
    auto key = [&](int c) { return (c >= nu || std::isnan(s[c])) ? -INFINITY : s[c]; };
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
      const float ka = key(a), kb = key(b);
      return ka != kb ? ka > kb : (a < nu) > (b < nu);   // chunks past the unit's count rank last
    });
    int64_t* rk = rank.data() + i * n;
    for (int r = 0; r < n; ++r) rk[order[r]] = r;
    for (int c = nu; c < n; ++c) rk[c] = n;                 // never kept
    std::copy(rk, rk + n, h->last_rank.begin() + (size_t)u * n);
    for (int c = 0; c < nu; ++c)
      if (rk[c] < h->keep && h->slot_of_at(u, c) < 0) missing.push_back({rk[c], u, c, (int)i});
  }
  bool evicted = false;
  auto evict = [&](int u, int s) {
    const int64_t c = h->holds_at(u, s);
    h->def_idx.push_back((int64_t)u * n + c);
    h->def_val.push_back(-1);
    h->def_unit.push_back(u);
    h->slot_of_at(u, (int)c) = -1;
    h->state_at(u, s) = kFree;
    h->holds_at(u, s) = -1;
    evicted = true;
  };
  // keep `spare` slots per unit free, evicting the worst-ranked staged
  // chunks outside the kept set
  if (h->spare > 0) {
    for (size_t i = 0; i < units.size(); ++i) {
      const int u = units[i];
      const int64_t* rk = rank.data() + i * n;
      int free_n = 0;
      std::vector<int> ready;
      for (int s = 0; s < S; ++s) {
        if (h->state_at(u, s) == kFree) ++free_n;
        if (h->state_at(u, s) == kReady) ready.push_back(s);
      }
      int short_n = h->spare - free_n;
      std::stable_sort(ready.begin(), ready.end(),
                       [&](int a, int b) { return rk[h->holds_at(u, a)] > rk[h->holds_at(u, b)]; });
      for (size_t j = 0; j < ready.size() && short_n > 0; ++j, --short_n) {
        if (rk[h->holds_at(u, ready[j])] < h->keep) break;
        evict(u, ready[j]);
      }
    }
  }
  // best ranks first, then unit order
  std::stable_sort(missing.begin(), missing.end(), [](const Miss& a, const Miss& b) {
    return a.rank != b.rank ? a.rank < b.rank : a.unit < b.unit;
  });
  int budget = h->max_inflight - (int)h->pending.size();
  std::vector<Pending> fills;
  for (const Miss& m : missing) {
    if (budget <= 0) break;
    const int u = m.unit;
    const int64_t* rk = rank.data() + (size_t)m.row * n;
    int slot = -1;
    for (int s = 0; s < S && slot < 0; ++s)
      if (h->state_at(u, s) == kFree) slot = s;
    if (slot < 0) {
      // no free slot: take the one of the worst-ranked staged chunk outside
      // the kept set, if there is one
      int worst = -1;
      for (int s = 0; s < S; ++s)
        if (h->state_at(u, s) == kReady && (worst < 0 || rk[h->holds_at(u, s)] > rk[h->holds_at(u, worst)]))
          worst = s;
      if (worst < 0 || rk[h->holds_at(u, worst)] < h->keep) continue;
      evict(u, worst);
      slot = worst;
    }
    h->state_at(u, slot) = kFilling;
    h->holds_at(u, slot) = m.chunk;
    h->slot_of_at(u, m.chunk) = slot;
    h->st.fills += 1;
    h->st.fill_bytes += h->chunk_bytes(u, m.chunk);
    fills.push_back({u, m.chunk, slot, m.rank < h->k});
    --budget;
  }
  if (evicted) {
    if (h->track_busy && stream_busy(compute)) h->st.evictions_while_busy += 1;
    reserve_wa(h);
  }
  if (!fills.empty() && h->track_busy && stream_busy(compute)) h->st.fills_while_busy += 1;
  for (const Pending& p : fills) {
    const int rc = issue(h, p);
    if (rc != HALO_OK) return rc;
  }
  return HALO_OK;
}

}  // namespace
}  // namespace halo

using namespace halo;

extern "C" int halo_staging_create(const halo_staging_desc* d, halo_staging** out) {
  HALO_CHECK_ARG(d != nullptr && out != nullptr, "null pointer argument");
  *out = nullptr;
  HALO_CHECK_ARG(d->n_layers > 0 && d->n_cold > 0 && d->top_k > 0, "empty staging cache");
  HALO_CHECK_ARG(d->sels_per_layer >= 1, "sels_per_layer must be >= 1");
  HALO_CHECK_ARG(d->n_slots >= 1 && d->n_slots <= 64, "n_slots must be in [1, 64]");
  HALO_CHECK_ARG(d->top_k <= d->keep && d->keep <= d->n_slots, "keep must be in [top_k, n_slots]");
  HALO_CHECK_ARG(d->ring >= 2 && d->max_inflight >= 0 && d->spare >= 0, "bad ring / max_inflight / spare");
  HALO_CHECK_ARG(d->residency && d->feedback && d->slot_addr && d->chunk_addr && d->chunk_nbytes && d->copy_stream,
                 "null pointer in the staging description");
  HALO_CHECK_ARG(!(d->write_allocate && d->sels_per_layer > 1), "write-allocate needs one selection per layer");
  auto h = new halo_staging();
  h->L = d->n_layers;
  h->B = d->sels_per_layer;
  h->U = h->L * h->B;
  h->n = d->n_cold;
  h->S = d->n_slots;
  h->k = d->top_k;
  h->keep = d->keep;
  h->max_inflight = d->max_inflight;
  h->spare = d->spare;
  h->ring_n = d->ring;
  h->W = h->B * (d->n_cold + 2 * d->top_k);
  h->wa = d->write_allocate != 0;
  h->kernel_fills = d->fill_mode == 1;
  h->track_busy = d->track_busy != 0;
  h->dev_i32 = d->residency;
  h->feedback = d->feedback;
  h->copy = static_cast<hipStream_t>(d->copy_stream);
  h->urgent = static_cast<hipStream_t>(d->urgent_stream);
  h->copy2 = static_cast<hipStream_t>(d->copy_stream2);
  const size_t L = h->L, U = h->U, n = h->n, S = h->S;
  h->dst.assign(d->slot_addr, d->slot_addr + U * S * 2);
  h->src.assign(d->chunk_addr, d->chunk_addr + U * n * 2);
  h->nbytes.assign(d->chunk_nbytes, d->chunk_nbytes + U * n);
  if (d->n_cold_per_unit != nullptr) {
    h->ncold.assign(d->n_cold_per_unit, d->n_cold_per_unit + U);
    for (auto& c : h->ncold) c = std::max(0, std::min(c, h->n));
  } else {
    h->ncold.assign(U, h->n);
  }
  h->slot_of.assign(U * n, -1);
  h->last_rank.assign(U * n, (int64_t)n);
  h->holds.assign(U * S, -1);
  h->state.assign(U * S, kFree);
  h->wa_slot.assign(L * 2, -1);
  h->launches.assign(L, 0);
  h->processed.assign(L, 0);
  h->fill_ev.assign(U * S, nullptr);
  h->ring.assign(h->ring_n, nullptr);
  h->ring_dev.assign(h->ring_n, nullptr);
  h->ring_stream.assign(h->ring_n, nullptr);
  h->ring_rows.assign(h->ring_n, {0, 0});
  int rc = HALO_OK;
  for (auto& e : h->fill_ev)
    if (rc == HALO_OK && hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) rc = HALO_E_HIP;
  // Coherent pinned memory: the boundary kernel's stores go to host memory
  // rather than into the GPU's caches.
  for (int r = 0; r < h->ring_n && rc == HALO_OK; ++r) {
    if (hipHostMalloc(reinterpret_cast<void**>(&h->ring[r]), L * h->W * sizeof(float), hipHostMallocCoherent) !=
            hipSuccess ||
        hipHostGetDevicePointer(reinterpret_cast<void**>(&h->ring_dev[r]), h->ring[r], 0) != hipSuccess)
      rc = HALO_E_HIP;
  }
  if (rc == HALO_OK &&
      (hipHostMalloc(reinterpret_cast<void**>(&h->ring_seq), (size_t)h->ring_n * 8 * sizeof(uint64_t),
                     hipHostMallocCoherent) != hipSuccess ||
       hipHostGetDevicePointer(reinterpret_cast<void**>(&h->ring_seq_dev), h->ring_seq, 0) != hipSuccess))
    rc = HALO_E_HIP;
  if (rc == HALO_OK) std::fill(h->ring_seq, h->ring_seq + (size_t)h->ring_n * 8, (uint64_t)0);
  if (rc != HALO_OK) {
    (void)hipGetLastError();
    set_error("halo_staging_create: event or pinned ring allocation failed");
    halo_staging_destroy(h);
    return rc;
  }
  reserve_wa(h);
  *out = h;
  return HALO_OK;
}

extern "C" int halo_staging_destroy(halo_staging* h) {
  if (h == nullptr) return HALO_OK;
  // pending copies and feedback publications must end before their events
  // and the ring go away (an entry marked but never enqueued is dropped)
  if (h->ring_seq != nullptr)
    for (int64_t e = h->seen; e < h->launched; ++e) (void)wait_entry(h, e);
  for (auto e : h->fill_ev)
    if (e) (void)hipEventSynchronize(e);
  for (auto e : h->fill_ev)
    if (e) (void)hipEventDestroy(e);
  for (auto p : h->ring)
    if (p) (void)hipHostFree(p);
  if (h->ring_seq) (void)hipHostFree(h->ring_seq);
  (void)hipGetLastError();
  delete h;
  return HALO_OK;
}

extern "C" int halo_staging_before(halo_staging* h, int lo, int hi, void* stream) {
  HALO_CHECK_ARG(h != nullptr && 0 <= lo && lo <= hi && hi <= h->L, "bad staging segment");
  hipStream_t compute = static_cast<hipStream_t>(stream);
  const int ulo = lo * h->B, uhi = hi * h->B;
  take_deferred(h, ulo, uhi);
  std::vector<Pending> rest;
  rest.reserve(h->pending.size());
  bool any = false;
  for (const Pending& p : h->pending) {
    bool take = false;
    if (ulo <= p.unit && p.unit < uhi) {
      hipEvent_t ev = h->fill_ev[(size_t)p.unit * h->S + p.slot];
      const hipError_t e = hipEventQuery(ev);
      if (e == hipSuccess) {
        take = true;  // landed: a plain commit
      } else if (e != hipErrorNotReady) {
        HALO_CHECK_HIP(e);
      } else {
        (void)hipGetLastError();
        if (p.urgent) {  // still in flight: the compute stream waits for it
          HALO_CHECK_HIP(hipStreamWaitEvent(compute, ev, 0));
          take = true;
        }
      }
    }
    if (take) {
      h->state_at(p.unit, p.slot) = kReady;
      h->idx_buf.push_back((int64_t)p.unit * h->n + p.chunk);
      h->val_buf.push_back(p.slot);
      any = true;
    } else {
      rest.push_back(p);
    }
  }
  h->pending.swap(rest);
  if (h->wa) {
    const int64_t base = (int64_t)h->U * h->n;
    for (int li = lo; li < hi; ++li) {
      // a reservation is named again only after the feedback of the launch
      // that last named it (two launches back) was processed
      const int par = (int)(h->launches[li] & 1);
      const bool ok = h->launches[li] - h->processed[li] < 2;
      h->idx_buf.push_back(base + li);
      h->val_buf.push_back(ok ? (int32_t)h->wa_slot[(size_t)li * 2 + par] : -1);
    }
  }
  for (int li = lo; li < hi; ++li) h->launches[li] += 1;
  if (any && h->track_busy && stream_busy(compute)) h->st.commits_while_busy += 1;
  return store(h, compute);
}

extern "C" int halo_staging_after(halo_staging* h, int lo, int hi, void* stream) {
  HALO_CHECK_ARG(h != nullptr && 0 <= lo && lo < hi && hi <= h->L, "bad staging segment");
  if (h->queued - h->seen >= h->ring_n) {
    set_error("feedback ring overrun: call halo_staging_service after every halo_staging_after");
    return HALO_E_INVALID;
  }
  hipStream_t compute = static_cast<hipStream_t>(stream);
  // an entry still marked goes out alone first: one publication per kernel
  const int rc = publish_marked(h, compute, true);
  if (rc != HALO_OK) return rc;
  const int r = (int)(h->queued % h->ring_n);
  h->ring_rows[r] = {lo, hi};
  h->ring_stream[r] = compute;
  h->queued += 1;  // marked: the next boundary kernel on `compute` publishes it
  return HALO_OK;
}

extern "C" int halo_staging_service(halo_staging* h, int lag, void* stream) {
  HALO_CHECK_ARG(h != nullptr && lag >= 0, "bad staging service call");
  hipStream_t compute = static_cast<hipStream_t>(stream);
  const int64_t target = h->queued - lag;
  std::vector<int> units;
  std::vector<float> scores;
  while (h->seen < h->queued) {
    const int r = (int)(h->seen % h->ring_n);
    if (h->seen < target) {
      if (h->seen >= h->launched) {  // marked, not enqueued yet: publish it now
        const int rc = publish_marked(h, compute, true);
        if (rc != HALO_OK) return rc;
      }
      const int64_t t0 = now_ns();
      const int rc = wait_entry(h, h->seen);
      h->st.ns_wait += now_ns() - t0;
      if (rc != HALO_OK) return rc;
    } else if (h->seen >= h->launched || !entry_ready(h, h->seen)) {
      break;
    }
    const int lo = h->ring_rows[r].first, hi = h->ring_rows[r].second;
    const float* fb = h->ring[r] + (size_t)lo * h->W;
    const int rc = account(h, fb, lo, hi, compute);
    if (rc != HALO_OK) return rc;
    for (int li = lo; li < hi; ++li) {
      const float* row = fb + (size_t)(li - lo) * h->W;
      for (int r = 0; r < h->B; ++r) {
        units.push_back(li * h->B + r);
        const float* sr = h->fb_scores(row, r);
        scores.insert(scores.end(), sr, sr + h->n);
      }
    }
    h->seen += 1;
  }
  int rc = HALO_OK;
  if (!units.empty()) {
    const int64_t t0 = now_ns();
    rc = plan(h, units, scores, compute);
    h->st.ns_plan += now_ns() - t0;
  }
  if (rc == HALO_OK && lag == 0) {
    // a full drain leaves the device residency equal to the host's
    take_deferred(h, 0, h->U);
    rc = store(h, compute);
  }
  return rc;
}

extern "C" int halo_staging_reset(halo_staging* h) {
  HALO_CHECK_ARG(h != nullptr, "null staging cache");
  for (int64_t e = h->seen; e < h->launched; ++e) {
    const int rc = wait_entry(h, e);
    if (rc != HALO_OK) return rc;
  }
  h->launched = h->queued;  // entries marked but not enqueued are dropped
  for (auto e : h->fill_ev) HALO_CHECK_HIP(hipEventSynchronize(e));
  h->pending.clear();
  h->def_idx.clear();
  h->def_val.clear();
  h->def_unit.clear();
  h->seen = h->queued;
  std::fill(h->slot_of.begin(), h->slot_of.end(), -1);
  std::fill(h->last_rank.begin(), h->last_rank.end(), (int64_t)h->n);
  std::fill(h->state.begin(), h->state.end(), (int8_t)kFree);
  std::fill(h->holds.begin(), h->holds.end(), -1);
  std::fill(h->wa_slot.begin(), h->wa_slot.end(), -1);
  std::fill(h->launches.begin(), h->launches.end(), 0);
  std::fill(h->processed.begin(), h->processed.end(), 0);
  reserve_wa(h);
  h->st = halo_staging_stats{};
  return HALO_OK;
}

extern "C" int halo_staging_set(halo_staging* h, int max_inflight, int reset_counters) {
  HALO_CHECK_ARG(h != nullptr && max_inflight >= 0, "bad staging setting");
  h->max_inflight = max_inflight;
  if (reset_counters) h->st = halo_staging_stats{};
  return HALO_OK;
}

extern "C" int halo_staging_get(const halo_staging* h, halo_staging_stats* stats, int8_t* state, int64_t* holds,
                                int64_t* wa_slot) {
  HALO_CHECK_ARG(h != nullptr, "null staging cache");
  if (stats) *stats = h->st;
  if (state) std::copy(h->state.begin(), h->state.end(), state);
  if (holds) std::copy(h->holds.begin(), h->holds.end(), holds);
  if (wa_slot) std::copy(h->wa_slot.begin(), h->wa_slot.end(), wa_slot);
  return HALO_OK;
}
