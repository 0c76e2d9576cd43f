// Token->expert align/sort: a stable counting sort of flat slots by expert, each expert group
// padded to block_m with the sentinel num_slots (vLLM moe_align_block_size format, as used at
// src/mtp_expert_prefetch/tracing/vllm_router_trace.py:19647-19660; the format's known-answer
// test is tests/test_vllm_descriptor_mapping_assertion.py:1012-1085).
//
// One workgroup of 16 waves. Wave w owns a contiguous range of slots. Pass 1 builds per-wave
// expert histograms in LDS; pass 2 turns them into exclusive per-(wave, expert) base
// positions; pass 3 walks each range 64 slots at a time in slot order, ranks equal experts
// inside the wave with a ballot-based match, and scatters. The order is therefore:
// experts ascending, slots ascending within an expert - identical to a stable argsort.
#include "common.h"
#include "launch.h"

namespace {

constexpr int kWaves = 16;
constexpr int kMaxGroups = 513;  // 512 routed experts + the shared expert

MOE_DEV int slot_expert(const int32_t* __restrict__ topk_ids, int routed, int E, int f) {
  if (f < routed) {
    const int e = topk_ids[f];
    return (e >= 0 && e < E) ? e : -1;
  }
  return E;  // shared slot
}

__global__ __launch_bounds__(1024) void align_kernel(const int32_t* __restrict__ topk_ids, int T,
                                                     int top_k, int E, int has_shared, int BM,
                                                     int cap, int32_t* __restrict__ sorted,
                                                     int32_t* __restrict__ eids,
                                                     int32_t* __restrict__ ntpp) {
  __shared__ int cnt[kWaves][kMaxGroups];
  __shared__ int off[kMaxGroups];
  __shared__ int pad[kMaxGroups];
  __shared__ int total_padded;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int routed = T * top_k;
  const int n_slots = routed + (has_shared ? T : 0);
  const int G = E + (has_shared ? 1 : 0);
  for (int i = tid; i < kWaves * kMaxGroups; i += 1024) (&cnt[0][0])[i] = 0;
  __syncthreads();

  const int per_wave = (((n_slots + kWaves - 1) / kWaves) + 63) / 64 * 64;
  const int lo = min(w * per_wave, n_slots), hi = min(lo + per_wave, n_slots);
  for (int f = lo + lane; f < hi; f += 64) {
    const int e = slot_expert(topk_ids, routed, E, f);
    if (e >= 0) atomicAdd(&cnt[w][e], 1);
  }
  __syncthreads();
  for (int g = tid; g < G; g += 1024) {
    int tot = 0;
    for (int v = 0; v < kWaves; ++v) tot += cnt[v][g];
    pad[g] = (tot + BM - 1) / BM * BM;
  }
  __syncthreads();
  if (w == 0) {  // exclusive scan of pad[] by one wave: lane owns a contiguous run
    const int per = (G + 63) / 64;
    const int g0 = min(lane * per, G), g1 = min(g0 + per, G);
    int local = 0;
    for (int g = g0; g < g1; ++g) local += pad[g];
    int incl = local;
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(incl, d, 64);
      if (lane >= d) incl += o;
    }
    int run = incl - local;
    for (int g = g0; g < g1; ++g) {
      off[g] = run;
      run += pad[g];
    }
    if (lane == 63) total_padded = incl;
  }
  __syncthreads();
  const int tp = total_padded;
  for (int g = tid; g < G; g += 1024) {
    int run = off[g];
    for (int v = 0; v < kWaves; ++v) {
      const int c = cnt[v][g];
      cnt[v][g] = run;
      run += c;
    }
    const int end = off[g] + pad[g];
    for (int p = run; p < end; ++p)
      if (p < cap * BM) sorted[p] = n_slots;
    for (int b = off[g] / BM; b < end / BM; ++b)
      if (b < cap) eids[b] = g;
  }
  for (int b = tp / BM + tid; b < cap; b += 1024) eids[b] = -1;
  for (int p = tp + tid; p < cap * BM; p += 1024) sorted[p] = n_slots;
  if (tid == 0) *ntpp = tp;
  __syncthreads();

  // Stable scatter: ranges in wave order, slots in order inside a range.
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int base = lo; base < hi; base += 64) {
    const int f = base + lane;
    const int e = (f < hi) ? slot_expert(topk_ids, routed, E, f) : -1;
    const bool valid = e >= 0;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 10; ++bit) {
      const bool b = valid && ((e >> bit) & 1);
      const uint64_t bal = __ballot(b);
      peers &= b ? bal : ~bal;
    }
    if (valid) {
      const int rank = __popcll(peers & lt_mask);
      const int pos = cnt[w][e] + rank;
      if (pos < cap * BM) sorted[pos] = f;
    }
    // wave-local LDS update after every lane has read the old base
    __builtin_amdgcn_wave_barrier();
    if (valid && (__ffsll((long long)peers) - 1) == lane) cnt[w][e] += __popcll(peers);
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace

int align_capacity_blocks(int T, int top_k, int E, int has_shared, int BM) {
  const int n_slots = T * top_k + (has_shared ? T : 0);
  const int groups = E + (has_shared ? 1 : 0);
  const int bound = (n_slots + BM - 1) / BM + (groups < n_slots ? groups : n_slots);
  return bound;
}

hipError_t launch_align(const int32_t* topk_ids, int T, int top_k, int E, int has_shared, int BM,
                        int cap, int32_t* sorted, int32_t* eids, int32_t* ntpp,
                        hipStream_t stream) {
  hipLaunchKernelGGL(align_kernel, dim3(1), dim3(1024), 0, stream, topk_ids, T, top_k, E,
                     has_shared, BM, cap, sorted, eids, ntpp);
  return hipGetLastError();
}
