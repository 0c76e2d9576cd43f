// Token->expert align/sort kernel: a stable counting sort of flat slots by expert, each expert
// group padded to block_m with the sentinel num_slots (vLLM moe_align_block_size format, as
// used at src/mtp_expert_prefetch/tracing/vllm_router_trace.py:19647-19660; the format's
// known-answer test is tests/test_vllm_descriptor_mapping_assertion.py:1012-1085).
//
// Decode sizes: one workgroup of 16 waves (routing.h:align_block). Wave w owns a contiguous
// range of slots. Pass 1 builds per-wave expert histograms in LDS; pass 2 turns them into
// exclusive per-(wave, expert) base positions; pass 3 walks each range 64 slots at a time in slot
// order, ranks equal experts inside the wave with a ballot-based match, and scatters. The order
// is therefore experts ascending, slots ascending within an expert - a stable argsort.
// Large inputs (prefill): the same ranking per chunk in many single-wave workgroups, then one
// block for the offsets and the scatter (align_chunk_kernel / align_finish_kernel below).
#include "launch.h"
#include "routing.h"

namespace {

// ---- Two-kernel align for large inputs (prefill): chunk ranks in parallel, then one block.
// Kernel 1: workgroup c (one wave) ranks the slots of chunk c = [c CH, (c + 1) CH) by expert in
// slot order (the ballot match of align_block, 64 slots at a time) and writes, into the sorted
// buffer used as scratch, each slot's rank inside its chunk at sorted[f] and the chunk's
// per-group counts at sorted[n_slots + c G + g].
// Kernel 2 (one 1024-thread block): reads all counts into LDS and its slots' ranks into
// registers, and only after a barrier writes the final layout: per-group bases per chunk, group
// offsets (exclusive scan of padded sizes), padding sentinels and block ids, then every slot at
// offset + chunk base + rank. The result is the single-block layout: experts ascending, slots
// ascending inside an expert.
constexpr int kAlign2MaxChunks = 64;
constexpr int kAlign2LdsCounts = 16448;       // chunks x groups held in LDS by kernel 2
constexpr int kAlign2MaxSlotsPerThread = 32;  // kernel 2's registers: slots of one thread

__global__ __launch_bounds__(64) void align_chunk_kernel(const int32_t* __restrict__ topk_ids,
                                                         int T, int top_k, int E, int has_shared,
                                                         int CH, int32_t* __restrict__ scratch) {
  __shared__ int cnt[kMaxGroups];
  const int lane = threadIdx.x, c = blockIdx.x;
  const int routed = T * top_k;
  const int n_slots = routed + (has_shared ? T : 0);
  const int G = E + (has_shared ? 1 : 0);
  for (int g = lane; g < G; g += 64) cnt[g] = 0;
  __builtin_amdgcn_wave_barrier();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // one wave: LDS ops complete in order
  const int lo = min(c * CH, n_slots), hi = min(lo + CH, n_slots);
  const __amdgpu_buffer_rsrc_t ir = buf_rsrc(topk_ids, (uint32_t)routed * 4u);
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int base0 = lo; base0 < hi; base0 += 64 * kAlignIds) {
    int eb[kAlignIds];
    align_ids(ir, routed, E, base0, hi, lane, eb);
#pragma unroll
    for (int u = 0; u < kAlignIds; ++u) {
      const int f = base0 + 64 * u + lane;
      if (base0 + 64 * u >= hi) break;  // uniform
      const int e = eb[u];
      const bool valid = e >= 0;
      uint64_t peers = __ballot(valid);
#pragma unroll
      for (int bit = 0; bit < 10; ++bit) {
        const bool b = valid && ((e >> bit) & 1);
        const uint64_t bal = __ballot(b);
        peers &= b ? bal : ~bal;
      }
      if (valid) scratch[f] = cnt[e] + __popcll(peers & lt_mask);
      __builtin_amdgcn_wave_barrier();
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (valid && (__ffsll((long long)peers) - 1) == lane) cnt[e] += __popcll(peers);
      __builtin_amdgcn_wave_barrier();
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
  }
  for (int g = lane; g < G; g += 64) scratch[n_slots + c * G + g] = cnt[g];
}

// Block order for the grouped GEMMs, heaviest first: border[r] = the r-th align block sorted by
// its number of 16-row subtiles holding slots (class BM/16 first, down to 1), ties in block
// order. Big blocks then start in the first wave of workgroups and the light ones fill the tail.
// A group of n > 0 slots has (n - 1) / BM full blocks (class BM/16) and a last block of class
// last_class(n); within a class the blocks come group by group, so with thread g taking group g
// a block's position is its class's base plus an exclusive scan over the threads. Called by
// every thread of a 1024-thread workgroup (it synchronises); wtot: 8 x 16 ints of LDS.
constexpr int kOrderMaxClasses = 8;  // BM <= 128
// Subtiles holding slots in the last block of a group of n > 0 slots.
MOE_DEV int last_class(int n, const BlockDiv& bd) { return (n - bd.div(n - 1) * bd.bm + 15) / 16; }
MOE_DEV void block_order(const int* s_off, const int* s_cnt, int G, const BlockDiv& bd,
                         int (*wtot)[16], int32_t* __restrict__ border) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int NC = bd.bm / 16;
  const int n = tid < G ? s_cnt[tid] : 0;
  const int nfull = n > 0 ? bd.div(n - 1) : 0;
  const int lc = n > 0 ? last_class(n, bd) : 0;  // 0: no blocks
  const int b0 = tid < G ? bd.div(s_off[tid]) : 0;
  int cnt[kOrderMaxClasses], excl[kOrderMaxClasses];
#pragma unroll
  for (int c = 0; c < kOrderMaxClasses; ++c) {
    cnt[c] = (c == NC - 1 ? nfull : 0) + (c == lc - 1 ? 1 : 0);
    const int incl = wave_incl_sum(cnt[c]);
    excl[c] = incl - cnt[c];
    if (lane == 63) wtot[c][w] = incl;
  }
  __syncthreads();
  // positions: classes heaviest first, then the waves before this one, then the lanes
  int base = 0, pos[kOrderMaxClasses];
#pragma unroll
  for (int c = kOrderMaxClasses - 1; c >= 0; --c) {
    int tot = 0, before = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int v = wtot[c][i];
      tot += v;
      before += i < w ? v : 0;
    }
    pos[c] = base + before + excl[c];
    base += tot;
  }
  if (n > 0) {
    for (int j = 0; j < nfull; ++j) border[pos[NC - 1] + j] = b0 + j;
    int pl = 0;  // the last block's position (after this group's full blocks in class BM/16)
#pragma unroll
    for (int c = 0; c < kOrderMaxClasses; ++c) pl = c == lc - 1 ? pos[c] : pl;
    border[pl + (lc == NC ? nfull : 0)] = b0 + nfull;
  }
}

// The one-workgroup align; with `border` (BM a multiple of 16, at most 128) it also writes the
// heaviest-first block order, from the group offsets and slot counts the sort leaves in LDS.
__global__ __launch_bounds__(1024) void align_kernel(const int32_t* __restrict__ topk_ids, int T,
                                                     int top_k, int E, int has_shared, int BM,
                                                     int cap, int32_t* __restrict__ sorted,
                                                     int32_t* __restrict__ eids,
                                                     int32_t* __restrict__ ntpp,
                                                     int32_t* __restrict__ border) {
  __shared__ AlignSmem sm;
  __shared__ int s_wtot[kOrderMaxClasses][16];
  align_block(topk_ids, T, top_k, E, has_shared, BM, cap, sorted, eids, ntpp, sm);
  if (border) {
    __syncthreads();  // every wave's scatter is done with its counters
    const int G = E + (has_shared ? 1 : 0);
    for (int g = threadIdx.x; g < G; g += 1024) sm.cnt[0][g] = sm.pad[g] - sm.off[g];
    __syncthreads();
    block_order(sm.off, sm.cnt[0], G, BlockDiv(BM), s_wtot, border);
  }
}

__global__ __launch_bounds__(1024) void align_finish_kernel(
    const int32_t* __restrict__ topk_ids, int T, int top_k, int E, int has_shared, int BM,
    int cap, int CH, int nchunks, int32_t* __restrict__ sorted, int32_t* __restrict__ eids,
    int32_t* __restrict__ ntpp, int32_t* __restrict__ border) {
  __shared__ int cl[kAlign2LdsCounts];  // [chunk][group]: counts, then bases inside the group
  __shared__ int s_off[kMaxGroups], s_pad[kMaxGroups];
  __shared__ int s_wtot[kOrderMaxClasses][16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int routed = T * top_k;
  const int n_slots = routed + (has_shared ? T : 0);
  const int G = E + (has_shared ? 1 : 0);
  const BlockDiv bd(BM);
  // 1. everything this block reads from the scratch, before anything is written
  {  // 16 count loads per thread in flight together (buffer loads; past the end: zeros)
    constexpr int NL = (kAlign2LdsCounts + 1023) / 1024;
    const int ncnt = nchunks * G;
    const __amdgpu_buffer_rsrc_t cr = buf_rsrc(sorted + n_slots, (uint32_t)ncnt * 4u);
    int v[NL];
#pragma unroll
    for (int k = 0; k < NL; ++k) {
      const int i = tid + 1024 * k;
      v[k] = (int)buf_ld32(cr, i < ncnt ? (uint32_t)i * 4u : kOutOfRange);
    }
#pragma unroll
    for (int k = 0; k < NL; ++k) {
      const int i = tid + 1024 * k;
      if (i < kAlign2LdsCounts) cl[i] = v[k];
    }
  }
  // ranks and raw ids of this thread's slots, all in flight together; the ids are decoded only
  // in the scatter below (a select on a loaded value here would become a branch with a wait)
  int rk[kAlign2MaxSlotsPerThread], raw[kAlign2MaxSlotsPerThread];
  const __amdgpu_buffer_rsrc_t ir = buf_rsrc(topk_ids, (uint32_t)routed * 4u);
  const __amdgpu_buffer_rsrc_t sr = buf_rsrc(sorted, (uint32_t)n_slots * 4u);
#pragma unroll
  for (int i = 0; i < kAlign2MaxSlotsPerThread; ++i) {
    const int f = tid + 1024 * i;
    rk[i] = (int)buf_ld32(sr, f < n_slots ? (uint32_t)f * 4u : kOutOfRange);
    raw[i] = (int)buf_ld32(ir, f < routed ? (uint32_t)f * 4u : kOutOfRange);
  }
  // every scratch read has returned before any thread of the block overwrites the buffer
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  // 2. per group: bases of the chunks (running counts) and the padded size
  for (int g = tid; g < G; g += 1024) {
    int run = 0;
    for (int c = 0; c < nchunks; ++c) {
      const int n = cl[c * G + g];
      cl[c * G + g] = run;
      run += n;
    }
    s_pad[g] = run;  // the group's slot count for now
  }
  __syncthreads();
  // 3. group offsets: exclusive scan of the padded sizes over the groups (thread g: group g)
  int tp;
  {
    const int off = block_excl_sum(tid < G ? bd.pad(s_pad[tid]) : 0, s_wtot[0], tp);
    if (tid < G) s_off[tid] = off;
  }
  __syncthreads();
  const int limit = cap * BM;
  if (border) block_order(s_off, s_pad, G, bd, s_wtot, border);
  // 4. padding sentinels (four threads per group, 16-byte stores) and block ids
  const bool vec = (reinterpret_cast<uintptr_t>(sorted) & 15u) == 0;
  for (int g = tid >> 2; g < G; g += 256) {
    const int sub = tid & 3;
    const int off = s_off[g], real_end = off + s_pad[g];
    const int end = g + 1 < G ? s_off[g + 1] : tp;
    const int fend = min(end, limit);
    const int a4 = vec ? min((real_end + 3) & ~3, fend) : fend;
    const int v_end = a4 + ((fend - a4) & ~3);
    if (sub == 0) {
      for (int p = real_end; p < a4; ++p) sorted[p] = n_slots;
      for (int p = v_end; p < fend; ++p) sorted[p] = n_slots;
    }
    const i32x4 sent = {n_slots, n_slots, n_slots, n_slots};
    for (int p = a4 + 4 * sub; p < v_end; p += 16) *reinterpret_cast<i32x4*>(&sorted[p]) = sent;
    const int bend = min(bd.div(end), cap);
    for (int b = bd.div(off) + sub; b < bend; b += 4) eids[b] = g;
  }
  for (int b = bd.div(tp) + tid; b < cap; b += 1024) eids[b] = -1;
  for (int p = tp + tid; p < limit; p += 1024) sorted[p] = n_slots;
  if (tid == 0) *ntpp = tp;
  // 5. the slots
#pragma unroll
  for (int i = 0; i < kAlign2MaxSlotsPerThread; ++i) {
    const int f = tid + 1024 * i;
    const int e = f < routed ? ((raw[i] >= 0 && raw[i] < E) ? raw[i] : -1) : (f < n_slots ? E : -1);
    if (e >= 0) {
      const int pos = s_off[e] + cl[(f / CH) * G + e] + rk[i];
      if (pos < limit) sorted[pos] = f;
    }
  }
}

// Kernel 2 of the scratch form (fused layer calls, whose workspace holds the ranks and counts
// outside the output buffers): one 1024-thread workgroup per chunk. Every workgroup reads all
// chunk counts, derives the group sizes, the group offsets (exclusive scan of padded sizes) and
// its own chunk's base inside each group, and writes the slots of its chunk at
// offset + chunk base + rank. The groups' padding sentinels and block ids are dealt to the
// workgroups in turn; one extra workgroup (blockIdx nchunks) writes ntpp and the block order. The layout is the one of
// align_finish_kernel, but the 4-byte slot stores come from nchunks CUs instead of one, and each
// group's chunk counts are summed by four threads with independent reads instead of walked
// serially.
__global__ __launch_bounds__(1024) void align_scatter_kernel(
    const int32_t* __restrict__ topk_ids, int T, int top_k, int E, int has_shared, int BM,
    int cap, int CH, int nchunks, const int32_t* __restrict__ scratch,
    int32_t* __restrict__ sorted, int32_t* __restrict__ eids, int32_t* __restrict__ ntpp,
    int32_t* __restrict__ border) {
  __shared__ int cl[kAlign2LdsCounts];  // [chunk][group] counts
  __shared__ int s_off[kMaxGroups], s_cnt[kMaxGroups], s_pre[kMaxGroups];
  __shared__ int s_wtot[kOrderMaxClasses][16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, c = blockIdx.x;
  const int routed = T * top_k;
  const int n_slots = routed + (has_shared ? T : 0);
  const int G = E + (has_shared ? 1 : 0);
  const BlockDiv bd(BM);
  const int ncnt = nchunks * G;
  // 1. all counts (16 loads per thread in flight together) and this thread's first slot of the
  //    chunk (its rank and raw id)
  {
    constexpr int NL = (kAlign2LdsCounts + 1023) / 1024;
    const __amdgpu_buffer_rsrc_t cr = buf_rsrc(scratch + n_slots, (uint32_t)ncnt * 4u);
    int v[NL];
#pragma unroll
    for (int k = 0; k < NL; ++k) {
      const int i = tid + 1024 * k;
      v[k] = (int)buf_ld32(cr, i < ncnt ? (uint32_t)i * 4u : kOutOfRange);
    }
#pragma unroll
    for (int k = 0; k < NL; ++k) {
      const int i = tid + 1024 * k;
      if (i < kAlign2LdsCounts) cl[i] = v[k];
    }
  }
  const int lo = min(c * CH, n_slots), hi = min(lo + CH, n_slots);
  const __amdgpu_buffer_rsrc_t ir = buf_rsrc(topk_ids, (uint32_t)routed * 4u);
  const __amdgpu_buffer_rsrc_t rr = buf_rsrc(scratch, (uint32_t)n_slots * 4u);
  const int f0 = lo + tid;
  const int rk0 = (int)buf_ld32(rr, f0 < hi ? (uint32_t)f0 * 4u : kOutOfRange);
  const int raw0 = (int)buf_ld32(ir, f0 < hi && f0 < routed ? (uint32_t)f0 * 4u : kOutOfRange);
  __syncthreads();
  // 2. per group: its slot count and the slots of the chunks before this one. Four adjacent
  //    threads per group each sum 16 chunks (independent LDS reads, unrolled), then the quad
  //    combines its partial sums.
  static_assert(kAlign2MaxChunks == 64, "four parts of 16 chunks");
  for (int i = tid; i < G * 4; i += 1024) {
    const int g = i >> 2, part = i & 3;
    int tot = 0, pre = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int q = part * 16 + j;
      const int n = cl[q < nchunks ? q * G + g : 0];
      tot += q < nchunks ? n : 0;
      pre += q < c ? n : 0;
    }
    // quad sums through DPP: quad_perm(1,0,3,2) then quad_perm(2,3,0,1) (a quad is always whole)
    tot += __builtin_amdgcn_update_dpp(0, tot, 0xB1, 0xF, 0xF, false);
    pre += __builtin_amdgcn_update_dpp(0, pre, 0xB1, 0xF, 0xF, false);
    tot += __builtin_amdgcn_update_dpp(0, tot, 0x4E, 0xF, 0xF, false);
    pre += __builtin_amdgcn_update_dpp(0, pre, 0x4E, 0xF, 0xF, false);
    if (part == 0) {
      s_cnt[g] = tot;
      s_pre[g] = pre;
    }
  }
  __syncthreads();
  // 3. group offsets: exclusive scan of the padded sizes over the groups (thread g: group g)
  int tp;
  {
    const int off = block_excl_sum(tid < G ? bd.pad(s_cnt[tid]) : 0, s_wtot[0], tp);
    if (tid < G) s_off[tid] = off;
  }
  __syncthreads();
  const int limit = cap * BM;
  // 4. this workgroup's share of the layout: groups c, c + nchunks, ... (padding sentinels and
  //    block ids), a stride of the tail past the padded total, ntpp and the block order
  if (c == nchunks) {  // the extra workgroup: ntpp and the block order only
    if (tid == 0) *ntpp = tp;
    if (border) block_order(s_off, s_cnt, G, bd, s_wtot, border);
    return;
  }
  for (int g = c; g < G; g += nchunks) {
    const int off = s_off[g], real_end = off + s_cnt[g];
    const int end = min(g + 1 < G ? s_off[g + 1] : tp, limit);
    for (int p = real_end + tid; p < end; p += 1024) sorted[p] = n_slots;
    const int bend = bd.div(end);
    for (int b = bd.div(off) + tid; b < bend; b += 1024) eids[b] = g;
  }
  for (int b = bd.div(tp) + c * 1024 + tid; b < cap; b += nchunks * 1024) eids[b] = -1;
  for (int p = tp + c * 1024 + tid; p < limit; p += nchunks * 1024) sorted[p] = n_slots;
  // 5. the slots of this chunk
  for (int f = f0; f < hi; f += 1024) {
    const int rk = f == f0 ? rk0 : scratch[f];
    const int raw = f == f0 ? raw0 : (f < routed ? topk_ids[f] : 0);
    const int e = f < routed ? ((raw >= 0 && raw < E) ? raw : -1) : E;
    if (e >= 0) {
      const int pos = s_off[e] + s_pre[e] + rk;
      if (pos < limit) sorted[pos] = f;
    }
  }
}

}  // namespace

int align_capacity_blocks(int T, int top_k, int E, int has_shared, int BM) {
  const int n_slots = T * top_k + (has_shared ? T : 0);
  const int groups = E + (has_shared ? 1 : 0);
  const int bound = (n_slots + BM - 1) / BM + (groups < n_slots ? groups : n_slots);
  return bound;
}

namespace {
// Chunks of the two-kernel align, or 0 when the input takes the one-block kernel: large inputs.
// With a scratch buffer of its own (the scatter form) any number of slots; otherwise the ranks and
// counts go into the sorted buffer, which needs room for them, and the finish kernel holds at most
// kAlign2MaxSlotsPerThread slots per thread.
int align_chunks(int T, int top_k, int E, int has_shared, int BM, int cap, bool scratch, int* CH) {
  const int n_slots = T * top_k + (has_shared ? T : 0);
  const int G = E + (has_shared ? 1 : 0);
  int nchunks = kAlign2LdsCounts / G;
  if (nchunks > kAlign2MaxChunks) nchunks = kAlign2MaxChunks;
  if (n_slots < 2048 || BM < 64 || BM > 16 * kOrderMaxClasses || nchunks <= 0 || G > kMaxGroups)
    return 0;
  if (!scratch && (n_slots > 1024 * kAlign2MaxSlotsPerThread ||
                   (int64_t)cap * BM < (int64_t)n_slots + (int64_t)nchunks * G))
    return 0;
  *CH = ((n_slots + nchunks - 1) / nchunks + 63) / 64 * 64;
  return (n_slots + *CH - 1) / *CH;
}
}  // namespace

int64_t align_scratch_bytes(int T, int top_k, int E, int has_shared, int BM, int cap) {
  int CH = 0;
  const int nchunks = align_chunks(T, top_k, E, has_shared, BM, cap, true, &CH);
  if (nchunks <= 0) return 0;
  const int64_t n_slots = (int64_t)T * top_k + (has_shared ? T : 0);
  return (n_slots + (int64_t)nchunks * (E + (has_shared ? 1 : 0))) * 4;
}

hipError_t launch_align(const int32_t* topk_ids, int T, int top_k, int E, int has_shared, int BM,
                        int cap, int32_t* sorted, int32_t* eids, int32_t* ntpp, int32_t* border,
                        int32_t* scratch, hipStream_t stream) {
  int CH = 0;
  const int nchunks = align_chunks(T, top_k, E, has_shared, BM, cap, scratch != nullptr, &CH);
  if (nchunks > 0 && scratch) {
    hipLaunchKernelGGL(align_chunk_kernel, dim3(nchunks), dim3(64), 0, stream, topk_ids, T,
                       top_k, E, has_shared, CH, scratch);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(align_scatter_kernel, dim3(nchunks + 1), dim3(1024), 0, stream, topk_ids, T,
                       top_k, E, has_shared, BM, cap, CH, nchunks, scratch, sorted, eids, ntpp,
                       border);
    return hipGetLastError();
  }
  if (nchunks > 0) {
    hipLaunchKernelGGL(align_chunk_kernel, dim3(nchunks), dim3(64), 0, stream, topk_ids, T,
                       top_k, E, has_shared, CH, sorted);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(align_finish_kernel, dim3(1), dim3(1024), 0, stream, topk_ids, T, top_k, E,
                       has_shared, BM, cap, CH, nchunks, sorted, eids, ntpp, border);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(align_kernel, dim3(1), dim3(1024), 0, stream, topk_ids, T, top_k, E,
                     has_shared, BM, cap, sorted, eids, ntpp,
                     (BM % 16 == 0 && BM <= 16 * kOrderMaxClasses) ? border : nullptr);
  return hipGetLastError();
}
