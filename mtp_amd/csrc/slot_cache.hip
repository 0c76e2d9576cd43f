// Offloaded-expert slot cache: pinned host pool of every (layer, expert) blob, an HBM pool of
// `slots_per_layer` slots per layer, prefetch with hipMemcpyAsync on two private copy streams,
// demand fetch of misses on the compute stream.
//
// Accounting follows the reference's ControlledExpertCacheManager
// (src/mtp_expert_prefetch/runtime/cache_manager.py:208-279): LRU per (layer, expert) with
// capacity slots_per_layer; a prefetch of a resident key only refreshes its recency; a demand
// miss inserts the key as used; evicting a prefetched-but-unused entry counts as
// evicted-before-use. Unlike the reference (accounting only), the bytes really move.
//
// Ordering (one compute stream per handle):
//  * a demand makes the compute stream wait for the layer's pending prefetches (on either copy
//    stream), fetches its misses on the compute stream, and uploads the layer's expert->slot
//    table (from a pinned staging ring) on the compute stream before the layer's kernels;
//  * the slots a demand names are pinned: a prefetch never picks them as victims until
//    moe_slot_cache_layer_done_v1 says the layer's kernels are enqueued (or the layer's next
//    demand, whose copies are ordered after those kernels on the compute stream, replaces the
//    pins). A prefetch that finds only pinned slots skips that expert;
//  * a prefetch first makes both copy streams wait for all work enqueued so far on the compute
//    stream, so an unpinned slot is never overwritten while an enqueued kernel may read it;
//  * every prefetch copy into slot s goes to copy stream s % kCopyStreams, so two copies into
//    one slot (a list longer than the unpinned slots, or two prefetch calls with no demand
//    between them) run in issue order and the slot ends with the bytes of the expert its table
//    entry names.
// The table entry of an absent expert is -1: the kernels drop the slots routed to it (they
// contribute zero). Handles are not thread-safe: one handle per host thread.
//
// Ready-time accounting (the reference's ReadyTimeExpertCacheManager, cache_manager.py:298-578,
// on real transfers): every prefetch call records a timing event on each copy stream it used
// after its copies, and every demand records one on the compute stream when it is issued (after the work
// already enqueued there, i.e. when the layer needs its experts). The first demand of a
// prefetched expert is ready-late when its copy completed more than ready_deadline_us after the
// demand's event: the compute stream then waits for the copy. The elapsed time between the two
// events settles it once both have completed (polled at every call, waited for by stats).
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <new>
#include <vector>

#include <hip/hip_runtime.h>

#include "launch.h"
#include "moe_w4a16.h"

namespace {

constexpr uint64_t kMagic = 0x4D4F45534C4F5431ull;  // "MOESLOT1"
constexpr int kStagingRing = 512;
constexpr int kEventRing = 1024;  // timing events of prefetch calls and of demands
constexpr int kSignalWords = 64;  // routed-ids flags: one per token of an offload layer call
// Copy streams of the prefetches: one DMA stream moves about 42 GB/s of expert blobs from
// pinned host memory, two together about 53 GB/s, four no more (MI355X, measured); a slot's
// copies always use the same stream (slot index modulo the count). (Splitting a demand's
// misses over the compute stream and a second stream measured slower: the cross-stream wait
// costs more than the parallel copy saves.)
constexpr int kCopyStreams = 2;

struct Slot {
  int expert = -1;
  bool prefetched = false;
  bool used = false;
  bool pinned = false;  // named by the layer's latest demand; its kernels may not be enqueued yet
  uint64_t last_use = 0;
  uint64_t pf_seq = 0;  // prefetch call whose copy filled the slot (0: none)
  int pf_stream = 0;    // copy stream of that copy
};

// A prefetched expert's first demand, settled when both events have completed.
struct ReadyCheck {
  uint64_t pf_seq;
  int pf_stream;
  uint64_t dm_seq;
};

struct Layer {
  std::vector<Slot> slots;
  std::vector<int> slot_of;   // expert -> slot or -1
  // per copy stream: prefetch copies not yet waited for by the compute stream, and the prefetch
  // call whose timing event follows the layer's latest copies on that stream (its event
  // pf_ev[(seq % kEventRing) * kCopyStreams + stream] is also what a demand waits on; if the
  // ring slot has been re-recorded since, the later record on the same stream completes after
  // these copies, so the wait stays correct)
  bool pending[kCopyStreams] = {};
  uint64_t done_seq[kCopyStreams] = {};
};

struct Cache {
  uint64_t magic = kMagic;
  moe_slot_cache_desc_v1 d{};
  std::vector<Layer> layers;
  uint64_t tick = 0;
  hipStream_t side[kCopyStreams] = {};  // prefetch copies
  hipEvent_t compute_mark = nullptr;
  int32_t* staging = nullptr;  // pinned [kStagingRing][num_experts]
  // pinned [kSignalWords], mapped at the same address on the device (nullptr if HIP maps it
  // elsewhere): the routed-ids flags of moe_offload_layer_v1, one per token; signal_seq is the
  // value the latest call waits for
  int32_t* signal = nullptr;
  uint32_t signal_seq = 0;
  std::vector<hipEvent_t> staging_done;
  int staging_next = 0;
  // timing events: pf_ev[(seq % kEventRing) * kCopyStreams + stream], dm_ev[seq % kEventRing]
  std::vector<hipEvent_t> pf_ev, dm_ev;
  uint64_t pf_seq = 0, dm_seq = 0;       // calls recorded so far (sequence numbers from 1)
  std::vector<ReadyCheck> checks;        // unsettled first demands, oldest first
  moe_slot_cache_counters_v1 st{};
};

int fail(int code, const char* msg) {
  snprintf(moe_error_buffer(), kErrorBufferBytes, "%s", msg);
  return code;
}

// Reported through the return code and the message; the thread's last HIP error is cleared.
int hip_fail(hipError_t e, const char* where) {
  (void)hipGetLastError();
  snprintf(moe_error_buffer(), kErrorBufferBytes, "%s: HIP error %d (%s)", where, (int)e,
           hipGetErrorString(e));
  return MOE_ERR_HIP + ((int)e % 100);
}

#define SC_HIP(expr, where)                         \
  do {                                              \
    hipError_t _e = (expr);                         \
    if (_e != hipSuccess) return hip_fail(_e, where); \
  } while (0)

// The calling thread's current device, restored when the guard leaves scope: the handle's
// calls switch to the cache's device and leave the caller's choice as it was.
struct DeviceGuard {
  int prev = -1;
  DeviceGuard() {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
  }
  ~DeviceGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

int setup_live(Cache* c);
void release_live(Cache* c);

Cache* from_handle(uint64_t h) {
  Cache* c = reinterpret_cast<Cache*>(h);
  if (!c || c->magic != kMagic) return nullptr;
  return c;
}

bool live(const Cache* c) { return c->d.dry_run == 0; }

const char* host_blob(const Cache* c, int layer, int expert) {
  return static_cast<const char*>(c->d.host_pool) +
         ((int64_t)layer * c->d.num_experts + expert) * c->d.expert_bytes;
}

char* device_slot(const Cache* c, int layer, int slot) {
  return static_cast<char*>(c->d.device_pool) +
         ((int64_t)layer * c->d.slots_per_layer + slot) * c->d.expert_bytes;
}

// Free slot, else the least recently used one. Pure LRU as in the reference: a miss may evict an
// expert that a later entry of the same demand list names; that entry then misses and is
// fetched again. With at most slots_per_layer distinct experts per call, every expert of the
// list is resident when the call returns (the last touches of the call are its experts).
// A prefetch passes skip_pinned: it never takes a slot the latest demand named (-1 if every
// slot is pinned).
int pick_slot(const Layer& L, bool skip_pinned) {
  int best = -1;
  for (int s = 0; s < (int)L.slots.size(); ++s) {
    if (skip_pinned && L.slots[s].pinned) continue;
    if (L.slots[s].expert < 0) return s;
    if (best < 0 || L.slots[s].last_use < L.slots[best].last_use) best = s;
  }
  return best;
}

void unpin(Layer& L) {
  for (Slot& sl : L.slots) sl.pinned = false;
}

void evict(Cache* c, Layer& L, int s) {
  Slot& sl = L.slots[s];
  if (sl.expert >= 0) {
    if (sl.prefetched && !sl.used) c->st.evicted_before_use_count++;
    L.slot_of[sl.expert] = -1;
  }
  sl = Slot{};
}

// Settles the ready checks whose events have completed (all of them when wait is set, and
// always those that name an event slot about to be reused by reuse_pf / reuse_dm).
int settle(Cache* c, bool wait, uint64_t reuse_pf = 0, uint64_t reuse_dm = 0) {
  std::vector<ReadyCheck> open;
  for (const ReadyCheck& k : c->checks) {
    hipEvent_t pe = c->pf_ev[(k.pf_seq % kEventRing) * kCopyStreams + k.pf_stream],
               de = c->dm_ev[k.dm_seq % kEventRing];
    const bool must = wait || k.pf_seq + kEventRing <= reuse_pf || k.dm_seq + kEventRing <= reuse_dm;
    if (must) {
      SC_HIP(hipEventSynchronize(pe), "ready check");
      SC_HIP(hipEventSynchronize(de), "ready check");
    } else if (hipEventQuery(pe) != hipSuccess || hipEventQuery(de) != hipSuccess) {
      (void)hipGetLastError();  // "not ready" is an answer, not an error to report later
      open.push_back(k);
      continue;
    }
    float ms = 0.0f;  // copy completion relative to the demand: > 0 means it arrived later
    SC_HIP(hipEventElapsedTime(&ms, de, pe), "ready check time");
    const double late_us = (double)ms * 1e3 - (double)c->d.ready_deadline_us;
    if (late_us > 0.0) {
      c->st.ready_late_miss_count++;
      c->st.ready_late_wait_ns += (int64_t)(late_us * 1e3);
    }
  }
  c->checks.swap(open);
  return MOE_OK;
}

}  // namespace

extern "C" {

int moe_slot_cache_create_v1(const moe_slot_cache_desc_v1* desc, uint64_t* handle) {
  if (!desc || !handle) return fail(MOE_ERR_NULL, "slot cache: NULL argument");
  const moe_slot_cache_desc_v1& d = *desc;
  if (d.num_layers < 1 || d.num_experts < 1 || d.slots_per_layer < 0 || d.expert_bytes <= 0 ||
      d.expert_bytes % 16 != 0)
    return fail(MOE_ERR_SHAPE, "slot cache: bad sizes");
  if (!d.dry_run && (!d.host_pool || !d.device_pool || !d.device_expert_row))
    return fail(MOE_ERR_NULL, "slot cache: pools and table are required unless dry_run");
  Cache* c = new (std::nothrow) Cache();
  if (!c) return fail(MOE_ERR_SHAPE, "slot cache: out of host memory");
  c->d = d;
  c->layers.resize(d.num_layers);
  for (Layer& L : c->layers) {
    L.slots.assign(d.slots_per_layer, Slot{});
    L.slot_of.assign(d.num_experts, -1);
  }
  c->st.capacity = d.slots_per_layer;
  if (live(c)) {
    const int rc = setup_live(c);
    if (rc != MOE_OK) {
      release_live(c);  // the partial set-up
      delete c;
      (void)hipGetLastError();  // release_live's own calls on the failed device
      return rc;
    }
  }
  *handle = reinterpret_cast<uint64_t>(c);
  return MOE_OK;
}

int moe_slot_cache_destroy_v1(uint64_t handle) {
  Cache* c = from_handle(handle);
  if (!c) return fail(MOE_ERR_NULL, "slot cache: bad handle");
  if (live(c)) release_live(c);
  c->magic = 0;
  delete c;
  return MOE_OK;
}

}  // extern "C"

namespace {

// HIP objects of a live cache, created on its device (the caller's current device restored).
int setup_live(Cache* c) {
  const moe_slot_cache_desc_v1& d = c->d;
  DeviceGuard guard;
  SC_HIP(hipSetDevice(d.device), "hipSetDevice");
  {
    for (hipStream_t& st : c->side)
      SC_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "create copy stream");
    SC_HIP(hipEventCreateWithFlags(&c->compute_mark, hipEventDisableTiming), "create event");
    SC_HIP(hipHostMalloc((void**)&c->staging, (size_t)kStagingRing * d.num_experts * 4,
                         hipHostMallocDefault), "pinned staging");
    {
      void* sig = nullptr;
      void* dev = nullptr;
      SC_HIP(hipHostMalloc(&sig, kSignalWords * 4, hipHostMallocDefault), "pinned signal words");
      memset(sig, 0, kSignalWords * 4);
      if (hipHostGetDevicePointer(&dev, sig, 0) == hipSuccess && dev == sig) {
        c->signal = static_cast<int32_t*>(sig);
      } else {
        (void)hipGetLastError();
        hipHostFree(sig);
      }
    }
    c->staging_done.assign(kStagingRing, nullptr);
    for (hipEvent_t& e : c->staging_done)
      SC_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming), "create event");
    c->pf_ev.assign((size_t)kEventRing * kCopyStreams, nullptr);
    c->dm_ev.assign(kEventRing, nullptr);
    for (hipEvent_t& e : c->pf_ev) SC_HIP(hipEventCreate(&e), "create timing event");
    for (hipEvent_t& e : c->dm_ev) SC_HIP(hipEventCreate(&e), "create timing event");
  }
  return MOE_OK;
}

// Frees whatever setup_live created (null members are skipped), on the cache's device.
void release_live(Cache* c) {
  DeviceGuard guard;
  (void)hipSetDevice(c->d.device);
  // Table uploads from the staging ring and the top-k kernel's flag stores into the signal
  // words run on the caller's compute stream: wait for the whole device before freeing them.
  (void)hipDeviceSynchronize();
  for (hipStream_t st : c->side)
    if (st) (void)hipStreamSynchronize(st);
  for (hipEvent_t e : c->staging_done)
    if (e) (void)hipEventDestroy(e);
  for (hipEvent_t e : c->pf_ev)
    if (e) (void)hipEventDestroy(e);
  for (hipEvent_t e : c->dm_ev)
    if (e) (void)hipEventDestroy(e);
  if (c->compute_mark) (void)hipEventDestroy(c->compute_mark);
  for (hipStream_t st : c->side)
    if (st) (void)hipStreamDestroy(st);
  if (c->staging) (void)hipHostFree(c->staging);
  if (c->signal) (void)hipHostFree(c->signal);
}

}  // namespace

namespace {

// The prefetch of moe_slot_cache_prefetch_v1. order_after_compute: make the copy streams wait
// for the work already on the compute stream first (an evicted slot may still be read by an
// enqueued kernel). Without it the caller guarantees that every kernel reading an unpinned slot
// of the layer has completed (see slot_cache_prefetch_synced).
int prefetch_impl(Cache* c, int32_t layer, const int32_t* experts, int32_t n,
                  void* compute_stream, int32_t* issued, bool order_after_compute) {
  if (layer < 0 || layer >= c->d.num_layers || n < 0 || (n > 0 && !experts))
    return fail(MOE_ERR_SHAPE, "slot cache prefetch: bad layer or list");
  for (int i = 0; i < n; ++i)
    if (experts[i] < 0 || experts[i] >= c->d.num_experts)
      return fail(MOE_ERR_SHAPE, "slot cache: expert id out of range");
  Layer& L = c->layers[layer];
  int count = 0;
  bool ordered = !order_after_compute;
  bool used[kCopyStreams] = {};
  for (int i = 0; i < n; ++i) {
    const int e = experts[i];
    if (L.slot_of[e] >= 0) {  // resident: refresh recency only
      L.slots[L.slot_of[e]].last_use = ++c->tick;
      continue;
    }
    if (c->d.slots_per_layer == 0) {  // nothing can be kept: counts as evicted before use
      c->st.issued_fetch_count++;
      c->st.evicted_before_use_count++;
      continue;
    }
    const int s = pick_slot(L, true);
    if (s < 0) {  // every slot holds an expert the layer's enqueued-or-pending kernels read
      c->st.prefetch_skipped_pinned_count++;
      continue;
    }
    c->st.issued_fetch_count++;
    evict(c, L, s);
    const int cs_i = s % kCopyStreams;  // one stream per slot: its copies stay in order
    L.slots[s] = Slot{e, true, false, false, ++c->tick, live(c) ? c->pf_seq + 1 : 0, cs_i};
    L.slot_of[e] = s;
    ++count;
    if (live(c)) {
      if (!ordered) {  // the copy streams run after every kernel enqueued so far
        SC_HIP(hipEventRecord(c->compute_mark, (hipStream_t)compute_stream), "record compute mark");
        for (hipStream_t st : c->side)
          SC_HIP(hipStreamWaitEvent(st, c->compute_mark, 0), "copy stream waits compute");
        ordered = true;
      }
      SC_HIP(hipMemcpyAsync(device_slot(c, layer, s), host_blob(c, layer, e), c->d.expert_bytes,
                            hipMemcpyHostToDevice, c->side[cs_i]), "prefetch copy");
      used[cs_i] = true;
      c->st.prefetch_bytes += c->d.expert_bytes;
    }
  }
  if (count > 0 && live(c)) {
    const uint64_t seq = ++c->pf_seq;  // the slots filled above carry this number
    int rc = settle(c, false, seq, 0);
    if (rc) return rc;
    for (int k = 0; k < kCopyStreams; ++k) {
      if (!used[k]) continue;
      L.pending[k] = true;
      L.done_seq[k] = seq;
      SC_HIP(hipEventRecord(c->pf_ev[(seq % kEventRing) * kCopyStreams + k], c->side[k]),
             "record prefetch done");
    }
  }
  if (issued) *issued = count;
  return MOE_OK;
}

}  // namespace

// The routed-ids flags of the next offload layer call: the mapped words (nullptr when the cache
// has none, or T exceeds them) and the value the call's top-k kernel will write into words
// [0, T) once the ids are out; never 0, so words from earlier calls or from creation differ.
int32_t* slot_cache_signal(uint64_t handle, int32_t T, int32_t* seq) {
  Cache* c = from_handle(handle);
  if (!c || !c->signal || T < 1 || T > kSignalWords) return nullptr;
  if (++c->signal_seq == 0) c->signal_seq = 1;
  *seq = (int32_t)c->signal_seq;
  return c->signal;
}

// Prefetch for a caller that synchronised the compute stream after enqueueing every kernel
// that reads the layer's slots, except the kernels of the layer's latest demand, whose slots
// must still be pinned (moe_offload_layer_v1: the routed ids' wait drains the stream, then the
// demand pins its slots and the layer's kernels are enqueued). No unpinned slot can then be
// read by pending work, so the copies need no ordering wait on the compute stream.
int slot_cache_prefetch_synced(uint64_t handle, int32_t layer, const int32_t* experts, int32_t n,
                               void* compute_stream) {
  Cache* c = from_handle(handle);
  if (!c) return fail(MOE_ERR_NULL, "slot cache: bad handle");
  return prefetch_impl(c, layer, experts, n, compute_stream, nullptr, false);
}

extern "C" {

int moe_slot_cache_prefetch_v1(uint64_t handle, int32_t layer, const int32_t* experts, int32_t n,
                               void* compute_stream, int32_t* issued) {
  Cache* c = from_handle(handle);
  if (!c) return fail(MOE_ERR_NULL, "slot cache: bad handle");
  return prefetch_impl(c, layer, experts, n, compute_stream, issued, true);
}

int moe_slot_cache_demand_v1(uint64_t handle, int32_t layer, const int32_t* experts, int32_t n,
                             void* compute_stream, int32_t* hits) {
  Cache* c = from_handle(handle);
  if (!c) return fail(MOE_ERR_NULL, "slot cache: bad handle");
  if (layer < 0 || layer >= c->d.num_layers || n < 0 || (n > 0 && !experts))
    return fail(MOE_ERR_SHAPE, "slot cache demand: bad layer or list");
  Layer& L = c->layers[layer];
  {  // validate ids and count distinct experts before any state changes
    std::vector<char> seen(c->d.num_experts, 0);
    int distinct = 0;
    for (int i = 0; i < n; ++i) {
      const int e = experts[i];
      if (e < 0 || e >= c->d.num_experts)
        return fail(MOE_ERR_SHAPE, "slot cache: expert id out of range");
      distinct += seen[e] ? 0 : 1;
      seen[e] = 1;
    }
    if (distinct > c->d.slots_per_layer && live(c))
      return fail(MOE_ERR_SHAPE, "slot cache demand: more distinct experts than slots");
  }
  hipStream_t cs = (hipStream_t)compute_stream;
  // The previous demand's kernels were enqueued on the compute stream before this call, so
  // its pins can go: this demand's copies and the prefetches after it are ordered after them.
  unpin(L);
  uint64_t dseq = 0;
  if (live(c)) {  // when the layer needs its experts: after the work already on the stream
    dseq = ++c->dm_seq;
    int rc = settle(c, false, 0, dseq);
    if (rc) return rc;
    SC_HIP(hipEventRecord(c->dm_ev[dseq % kEventRing], cs), "record demand time");
  }
  for (int k = 0; k < kCopyStreams; ++k) {
    if (!L.pending[k] || !live(c)) continue;
    SC_HIP(hipStreamWaitEvent(cs, c->pf_ev[(L.done_seq[k] % kEventRing) * kCopyStreams + k], 0),
           "compute waits prefetch");
    L.pending[k] = false;
  }
  int nh = 0;
  for (int i = 0; i < n; ++i) {
    const int e = experts[i];
    c->st.demand_count++;
    int s = L.slot_of[e];
    if (s >= 0) {
      c->st.demand_hit_count++;
      ++nh;
      Slot& sl = L.slots[s];
      if (sl.prefetched && !sl.used) {
        c->st.used_fetch_count++;
        // The copy's timing event is only still its own while fewer than kEventRing prefetch
        // calls have recorded since; an older copy completed long before this demand (counted
        // on time).
        if (dseq && sl.pf_seq && c->pf_seq - sl.pf_seq < (uint64_t)kEventRing)
          c->checks.push_back(ReadyCheck{sl.pf_seq, sl.pf_stream, dseq});
      }
      sl.used = true;
      sl.pinned = true;
      sl.last_use = ++c->tick;
      continue;
    }
    c->st.demand_miss_count++;
    if (c->d.slots_per_layer == 0) continue;
    // With at most slots_per_layer distinct experts per call, the LRU victim is never an expert
    // this call already touched (those hold the newest ticks).
    s = pick_slot(L, false);
    evict(c, L, s);
    L.slots[s] = Slot{e, false, true, true, ++c->tick, 0};
    L.slot_of[e] = s;
    if (live(c)) {
      SC_HIP(hipMemcpyAsync(device_slot(c, layer, s), host_blob(c, layer, e), c->d.expert_bytes,
                            hipMemcpyHostToDevice, cs), "demand copy");
      c->st.demand_bytes += c->d.expert_bytes;
    }
  }
  if (live(c)) {  // publish the layer's expert -> slot table on the compute stream
    const int r = c->staging_next;
    c->staging_next = (r + 1) % kStagingRing;
    SC_HIP(hipEventSynchronize(c->staging_done[r]), "staging reuse");
    int32_t* stage = c->staging + (size_t)r * c->d.num_experts;
    // -1 for experts that are not resident: the kernels drop their slots (never read row -1)
    for (int e = 0; e < c->d.num_experts; ++e) stage[e] = L.slot_of[e];
    SC_HIP(hipMemcpyAsync(c->d.device_expert_row + (size_t)layer * c->d.num_experts, stage,
                          (size_t)c->d.num_experts * 4, hipMemcpyHostToDevice, cs), "table upload");
    SC_HIP(hipEventRecord(c->staging_done[r], cs), "record staging");
  }
  if (hits) *hits = nh;
  return MOE_OK;
}

int moe_slot_cache_layer_done_v1(uint64_t handle, int32_t layer) {
  Cache* c = from_handle(handle);
  if (!c) return fail(MOE_ERR_NULL, "slot cache: bad handle");
  if (layer < 0 || layer >= c->d.num_layers)
    return fail(MOE_ERR_SHAPE, "slot cache layer_done: bad layer");
  unpin(c->layers[layer]);
  return MOE_OK;
}

int moe_slot_cache_stats_v1(uint64_t handle, moe_slot_cache_counters_v1* out) {
  Cache* c = from_handle(handle);
  if (!c || !out) return fail(MOE_ERR_NULL, "slot cache: bad handle or NULL output");
  if (live(c)) {
    int rc = settle(c, true);
    if (rc) return rc;
  }
  moe_slot_cache_counters_v1 s = c->st;
  int64_t resident = 0, unused = 0;
  for (const Layer& L : c->layers)
    for (const Slot& sl : L.slots)
      if (sl.expert >= 0) {
        ++resident;
        if (sl.prefetched && !sl.used) ++unused;
      }
  s.resident_count = resident;
  s.unused_fetch_count = unused;
  *out = s;
  return MOE_OK;
}

int moe_slot_cache_slot_of_v1(uint64_t handle, int32_t layer, int32_t expert) {
  Cache* c = from_handle(handle);
  if (!c || layer < 0 || layer >= c->d.num_layers || expert < 0 || expert >= c->d.num_experts)
    return -2;
  return c->layers[layer].slot_of[expert];
}

}  // extern "C"
