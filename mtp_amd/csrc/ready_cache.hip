// Expert-payload cache accounting on virtual time (host code only; no HIP calls, no payload
// bytes). It answers the question the reference's cache-lab managers answer, for a trace of
// prefetch issues and demands with their arrival times:
//  * MOE_READY_CACHE_CONTROLLED: ControlledExpertCacheManager
//    (src/mtp_expert_prefetch/runtime/cache_manager.py:208-279): one LRU of `capacity`
//    (layer, expert) keys; a prefetch of a missing key enters it at once as an unused prefetch.
//  * MOE_READY_CACHE_READY_TIME: ReadyTimeExpertCacheManager (cache_manager.py:298-578): a
//    prefetch is a transfer served by one queue; it enters the LRU only when virtual time
//    reaches its completion, and a demand counts as a hit only for keys completed by its
//    arrival + queue_deadline_us. Issues are batched (queue_batch_size), each batch starting at
//    max(server free, ready time) and taking service_us_per_batch + service_us_per_issue per
//    issue; a partial batch is released queue_deadline_us after its first issue (never with a
//    zero deadline) or at finish. A demand of a key still in flight is a miss and a ready-late
//    miss; that transfer's later completion finds the key resident (inserted by the demand) and
//    counts as a late completion left unused.
// The slot cache (slot_cache.hip) moves the bytes and measures readiness with HIP events; this
// handle gives the reference's counters for the same call sequence, so both hit rates can be
// reported side by side.
#include <cmath>
#include <cstdio>
#include <deque>
#include <list>
#include <new>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

#include "launch.h"
#include "moe_w4a16.h"

namespace {

constexpr uint64_t kReadyMagic = 0x4D4F455244594331ull;  // "MOERDYC1"

struct Entry {
  uint64_t key;
  bool prefetched;
  bool used;
};

struct ReadyCache {
  uint64_t magic = kReadyMagic;
  int mode = MOE_READY_CACHE_READY_TIME;
  int64_t capacity = 0;
  double per_issue = 0.0, per_batch = 0.0, deadline = 0.0;
  int64_t batch = 1;
  std::list<Entry> lru;  // least recent first
  std::unordered_map<uint64_t, std::list<Entry>::iterator> where;
  std::unordered_set<uint64_t> inflight;
  std::vector<uint64_t> pending;  // issues not yet handed to the server
  bool has_first = false;
  double first_arrival = 0.0;     // arrival of the first pending issue
  std::deque<std::pair<double, std::vector<uint64_t>>> done;  // batches by completion time
  double server_free = 0.0, last_completion = 0.0, last_arrival = 0.0;
  moe_ready_cache_snapshot_v1 st{};
};

uint64_t make_key(int32_t layer, int32_t expert) {
  return ((uint64_t)(uint32_t)layer << 32) | (uint32_t)expert;
}

int fail(int code, const char* msg) {
  snprintf(moe_error_buffer(), kErrorBufferBytes, "%s", msg);
  return code;
}

ReadyCache* from_handle(uint64_t h) {
  ReadyCache* c = reinterpret_cast<ReadyCache*>(h);
  if (!c || c->magic != kReadyMagic) return nullptr;
  return c;
}

void touch(ReadyCache* c, std::list<Entry>::iterator it) {
  c->lru.splice(c->lru.end(), c->lru, it);
}

// Insert a key (absent) at the most recent end, then evict down to capacity; with capacity 0
// nothing is kept (an unused prefetch counts as evicted before use).
void insert(ReadyCache* c, uint64_t key, bool prefetched, bool used) {
  if (c->capacity <= 0) {
    if (prefetched && !used) c->st.evicted_before_use_count++;
    return;
  }
  c->lru.push_back(Entry{key, prefetched, used});
  c->where[key] = std::prev(c->lru.end());
  while ((int64_t)c->lru.size() > c->capacity) {
    const Entry& old = c->lru.front();
    if (old.prefetched && !old.used) c->st.evicted_before_use_count++;
    c->where.erase(old.key);
    c->lru.pop_front();
  }
}

// Hand `keys` to the server as one batch, ready at `ready` (its first issue at `first`).
void serve(ReadyCache* c, std::vector<uint64_t> keys, double ready, double first) {
  if (keys.empty()) return;
  const double svc = c->per_batch + c->per_issue * (double)keys.size();
  const double start = c->server_free > ready ? c->server_free : ready;
  const double end = start + svc;
  c->st.queue_batch_count++;
  c->st.queue_service_us += svc;
  c->st.queue_wait_us += start - ready > 0.0 ? start - ready : 0.0;
  if (end - first > c->st.queue_max_delay_us) c->st.queue_max_delay_us = end - first;
  c->server_free = end;
  c->last_completion = end;
  c->done.emplace_back(end, std::move(keys));
}

void release_full(ReadyCache* c, double now) {
  while ((int64_t)c->pending.size() >= c->batch) {
    const double first = c->has_first ? c->first_arrival : now;
    std::vector<uint64_t> head(c->pending.begin(), c->pending.begin() + c->batch);
    c->pending.erase(c->pending.begin(), c->pending.begin() + c->batch);
    serve(c, std::move(head), now, first);
    c->has_first = !c->pending.empty();
    c->first_arrival = now;
  }
}

void release_due(ReadyCache* c, double now) {
  if (c->pending.empty() || !c->has_first || !(c->deadline > 0.0) ||
      now < c->first_arrival + c->deadline)
    return;
  const double first = c->first_arrival;
  std::vector<uint64_t> keys;
  keys.swap(c->pending);
  c->has_first = false;
  serve(c, std::move(keys), first + c->deadline, first);
}

// Transfers completed by `now` enter the LRU (a key the demand path already inserted is only
// refreshed; if it was not a prefetch, its transfer completed too late to be used).
void complete(ReadyCache* c, double now) {
  while (!c->done.empty() && c->done.front().first <= now) {
    std::vector<uint64_t> keys = std::move(c->done.front().second);
    c->done.pop_front();
    for (uint64_t key : keys) {
      c->inflight.erase(key);
      auto w = c->where.find(key);
      if (w != c->where.end()) {
        if (!w->second->prefetched) c->st.late_completion_unused_count++;
        touch(c, w->second);
        continue;
      }
      insert(c, key, true, false);
    }
  }
}

void advance(ReadyCache* c, double t) {
  const double now = t > 0.0 ? t : 0.0;
  if (now > c->last_arrival) c->last_arrival = now;
  release_due(c, now);
  complete(c, now);
}

bool issue_one(ReadyCache* c, uint64_t key, double t) {
  if (c->mode == MOE_READY_CACHE_READY_TIME) advance(c, t);
  auto w = c->where.find(key);
  if (w != c->where.end()) {  // resident: refresh recency only
    touch(c, w->second);
    return false;
  }
  if (c->mode == MOE_READY_CACHE_CONTROLLED) {
    c->st.issued_fetch_count++;
    insert(c, key, true, false);
    return true;
  }
  if (c->inflight.count(key)) return false;
  c->st.issued_fetch_count++;
  c->inflight.insert(key);
  if (c->pending.empty()) {
    c->has_first = true;
    c->first_arrival = t;
  }
  c->pending.push_back(key);
  release_full(c, t);
  return true;
}

bool demand_one(ReadyCache* c, uint64_t key, double t) {
  if (c->mode == MOE_READY_CACHE_READY_TIME) {
    const double due = t + c->deadline;
    release_due(c, due);
    complete(c, due);
  }
  c->st.demand_count++;
  auto w = c->where.find(key);
  if (w != c->where.end()) {
    c->st.demand_hit_count++;
    Entry& e = *w->second;
    if (e.prefetched && !e.used) c->st.used_fetch_count++;
    e.used = true;
    touch(c, w->second);
    return true;
  }
  if (c->inflight.count(key)) c->st.ready_late_miss_count++;
  c->st.demand_miss_count++;
  insert(c, key, false, true);
  return false;
}

bool finite_times(double a, double b) { return std::isfinite(a) && std::isfinite(b); }

}  // namespace

extern "C" {

int moe_ready_cache_create_v1(int32_t mode, int64_t capacity, double service_us_per_issue,
                              double service_us_per_batch, int64_t queue_batch_size,
                              double queue_deadline_us, uint64_t* handle) {
  if (!handle) return fail(MOE_ERR_NULL, "ready cache: NULL handle");
  if (mode != MOE_READY_CACHE_CONTROLLED && mode != MOE_READY_CACHE_READY_TIME)
    return fail(MOE_ERR_UNSUPPORTED, "ready cache: unknown mode");
  if (!std::isfinite(service_us_per_issue))
    return fail(MOE_ERR_SHAPE, "service_us_per_issue must be finite");
  if (!std::isfinite(service_us_per_batch))
    return fail(MOE_ERR_SHAPE, "service_us_per_batch must be finite");
  if (!std::isfinite(queue_deadline_us))
    return fail(MOE_ERR_SHAPE, "queue_deadline_us must be finite");
  ReadyCache* c = new (std::nothrow) ReadyCache();
  if (!c) return fail(MOE_ERR_SHAPE, "ready cache: out of host memory");
  c->mode = mode;
  c->capacity = capacity;
  c->per_issue = service_us_per_issue > 0.0 ? service_us_per_issue : 0.0;
  c->per_batch = service_us_per_batch > 0.0 ? service_us_per_batch : 0.0;
  c->batch = queue_batch_size >= 1 ? queue_batch_size : 1;
  c->deadline = queue_deadline_us > 0.0 ? queue_deadline_us : 0.0;
  c->st.capacity = capacity;
  *handle = reinterpret_cast<uint64_t>(c);
  return MOE_OK;
}

int moe_ready_cache_destroy_v1(uint64_t handle) {
  ReadyCache* c = from_handle(handle);
  if (!c) return fail(MOE_ERR_NULL, "ready cache: bad handle");
  c->magic = 0;
  delete c;
  return MOE_OK;
}

int moe_ready_cache_prefetch_v1(uint64_t handle, int32_t layer, const int32_t* experts,
                                int32_t n, double arrival_us, int32_t* issued_flags,
                                int32_t* issued) {
  ReadyCache* c = from_handle(handle);
  if (!c) return fail(MOE_ERR_NULL, "ready cache: bad handle");
  if (n < 0 || (n > 0 && !experts)) return fail(MOE_ERR_SHAPE, "ready cache prefetch: bad list");
  if (!finite_times(arrival_us, 0.0)) return fail(MOE_ERR_SHAPE, "arrival_us must be finite");
  int count = 0;
  for (int i = 0; i < n; ++i) {
    const bool ok = issue_one(c, make_key(layer, experts[i]), arrival_us);
    if (issued_flags) issued_flags[i] = ok ? 1 : 0;
    count += ok ? 1 : 0;
  }
  if (issued) *issued = count;
  return MOE_OK;
}

int moe_ready_cache_demand_v1(uint64_t handle, int32_t layer, const int32_t* experts, int32_t n,
                              double arrival_us, int32_t* hit_flags, int32_t* hits) {
  ReadyCache* c = from_handle(handle);
  if (!c) return fail(MOE_ERR_NULL, "ready cache: bad handle");
  if (n < 0 || (n > 0 && !experts)) return fail(MOE_ERR_SHAPE, "ready cache demand: bad list");
  if (!finite_times(arrival_us, 0.0)) return fail(MOE_ERR_SHAPE, "arrival_us must be finite");
  int count = 0;
  for (int i = 0; i < n; ++i) {
    const bool hit = demand_one(c, make_key(layer, experts[i]), arrival_us);
    if (hit_flags) hit_flags[i] = hit ? 1 : 0;
    count += hit ? 1 : 0;
  }
  if (hits) *hits = count;
  return MOE_OK;
}

int moe_ready_cache_advance_v1(uint64_t handle, double arrival_us) {
  ReadyCache* c = from_handle(handle);
  if (!c) return fail(MOE_ERR_NULL, "ready cache: bad handle");
  if (!finite_times(arrival_us, 0.0)) return fail(MOE_ERR_SHAPE, "arrival_us must be finite");
  if (c->mode == MOE_READY_CACHE_READY_TIME) advance(c, arrival_us);
  return MOE_OK;
}

int moe_ready_cache_finish_v1(uint64_t handle) {
  ReadyCache* c = from_handle(handle);
  if (!c) return fail(MOE_ERR_NULL, "ready cache: bad handle");
  if (c->mode != MOE_READY_CACHE_READY_TIME) return MOE_OK;
  if (!c->pending.empty() && c->has_first) {
    const double first = c->first_arrival;
    const double ready = c->deadline > 0.0 ? first + c->deadline : c->last_arrival;
    std::vector<uint64_t> keys;
    keys.swap(c->pending);
    c->has_first = false;
    serve(c, std::move(keys), ready, first);
  }
  complete(c, INFINITY);
  return MOE_OK;
}

int moe_ready_cache_stats_v1(uint64_t handle, moe_ready_cache_snapshot_v1* out) {
  ReadyCache* c = from_handle(handle);
  if (!c || !out) return fail(MOE_ERR_NULL, "ready cache: bad handle or NULL output");
  moe_ready_cache_snapshot_v1 s = c->st;
  int64_t unused = 0;
  for (const Entry& e : c->lru) unused += (e.prefetched && !e.used) ? 1 : 0;
  s.resident_count = (int64_t)c->lru.size();
  s.unused_fetch_count = unused + s.late_completion_unused_count;
  s.queue_total_span_us = s.issued_fetch_count ? c->last_completion : 0.0;
  s.queue_event_interval_us = 0.0;
  s.queue_deadline_us = c->deadline;
  s.queue_batch_size = c->batch;
  *out = s;
  return MOE_OK;
}

}  // extern "C"
