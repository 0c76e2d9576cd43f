// Token->expert align/sort kernel: a stable counting sort of flat slots by expert, each expert
// group padded to block_m with the sentinel num_slots (vLLM moe_align_block_size format, as
// used at src/mtp_expert_prefetch/tracing/vllm_router_trace.py:19647-19660; the format's
// known-answer test is tests/test_vllm_descriptor_mapping_assertion.py:1012-1085).
//
// One workgroup of 16 waves (routing.h:align_block). Wave w owns a contiguous range of slots.
// Pass 1 builds per-wave expert histograms in LDS; pass 2 turns them into exclusive
// per-(wave, expert) base positions; pass 3 walks each range 64 slots at a time in slot order,
// ranks equal experts inside the wave with a ballot-based match, and scatters. The order is
// therefore experts ascending, slots ascending within an expert - a stable argsort.
#include "launch.h"
#include "routing.h"

namespace {

__global__ __launch_bounds__(1024) void align_kernel(const int32_t* __restrict__ topk_ids, int T,
                                                     int top_k, int E, int has_shared, int BM,
                                                     int cap, int32_t* __restrict__ sorted,
                                                     int32_t* __restrict__ eids,
                                                     int32_t* __restrict__ ntpp) {
  __shared__ AlignSmem sm;
  align_block(topk_ids, T, top_k, E, has_shared, BM, cap, sorted, eids, ntpp, sm);
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
