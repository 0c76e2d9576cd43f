// Router kernels: fp32 logits in the canonical order (routing.h:logits_tile), then top-k with
// renormalised softmax weights (routing.h:topk_token).
//
// Semantics: vLLM topk_softmax(renormalize=True) as restated at
// src/mtp_expert_prefetch/tracing/vllm_router_trace.py:4201-4225. Renormalisation cancels the
// softmax denominator, so w_i = exp(l_i - l_max) / sum_{j in top-k} exp(l_j - l_max).
//
// Kernels:
//  * logits (any T; small tiles at decode for more waves in flight, 8 x 8 tiles at prefill for
//    register reuse) - the tile shape never changes the per-(token, row) summation order;
//  * top-k, one wave per token (any T);
//  * top-k + align in one block for decode-size batches (at most 64 slots):
//    the ids stay in LDS between the two steps, so no cross-block visibility is needed and the
//    align launch disappears.
#include "launch.h"
#include "routing.h"

namespace {

template <int TT, int TE>
__global__ __launch_bounds__(256) void router_logits_kernel(
    const uint16_t* __restrict__ x, int T, int H, const uint16_t* __restrict__ W, int E,
    const uint16_t* __restrict__ shared_w, const float* __restrict__ bias,
    float* __restrict__ logits) {
  const int rows = E + (shared_w ? 1 : 0);
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int tiles_e = (rows + TE - 1) / TE;
  const int t0 = (wave / tiles_e) * TT;
  const int e0 = (wave % tiles_e) * TE;
  if (t0 >= T) return;
  logits_tile<TT, TE>(x, T, H, W, E, shared_w, bias, logits, t0, e0, lane);
}

__global__ __launch_bounds__(256) void router_topk_kernel(const float* __restrict__ logits, int T,
                                                          int E, int top_k, int has_shared,
                                                          int32_t* __restrict__ ids,
                                                          float* __restrict__ weights) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;
  topk_token(logits + (int64_t)t * (E + 1), E, top_k, has_shared, T, t, lane, ids, weights,
             nullptr);
}

// One wave per token for the top-k, then wave 0 aligns the (at most 64) slots.
__global__ __launch_bounds__(64 * kTopkAlignMaxTokens) void topk_align_kernel(
    const float* __restrict__ logits, int T, int E, int top_k, int has_shared, int BM, int cap,
    int32_t* __restrict__ ids, float* __restrict__ weights, int32_t* __restrict__ sorted,
    int32_t* __restrict__ eids, int32_t* __restrict__ ntpp) {
  __shared__ int s_ids[kAlignWaveMaxSlots];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (wave < T)
    topk_token(logits + (int64_t)wave * (E + 1), E, top_k, has_shared, T, wave, lane, ids,
               weights, s_ids);
  __syncthreads();
  if (wave == 0) align_wave(s_ids, T, top_k, E, has_shared, BM, cap, sorted, eids, ntpp, lane);
}

template <int TT, int TE>
hipError_t launch_logits_tiled(const uint16_t* x, int T, int H, const uint16_t* W, int E,
                               const uint16_t* shared_w, const float* bias, float* logits,
                               hipStream_t stream) {
  const int rows = E + (shared_w ? 1 : 0);
  const int tiles = ((T + TT - 1) / TT) * ((rows + TE - 1) / TE);
  const int blocks = (tiles + 3) / 4;
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL((router_logits_kernel<TT, TE>), dim3(blocks), dim3(256), 0, stream, x, T, H,
                     W, E, shared_w, bias, logits);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_router_logits(const uint16_t* x, int T, int H, const uint16_t* W, int E,
                                const uint16_t* shared_w, const float* bias, float* logits,
                                hipStream_t stream) {
  if (T <= 4) return launch_logits_tiled<1, 2>(x, T, H, W, E, shared_w, bias, logits, stream);
  if (T <= 64) return launch_logits_tiled<2, 4>(x, T, H, W, E, shared_w, bias, logits, stream);
  return launch_logits_tiled<8, 8>(x, T, H, W, E, shared_w, bias, logits, stream);
}

hipError_t launch_router_topk(const float* logits, int T, int E, int top_k, int has_shared,
                              int32_t* ids, float* weights, hipStream_t stream) {
  const int blocks = (T + 3) / 4;
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(router_topk_kernel, dim3(blocks), dim3(256), 0, stream, logits, T, E, top_k,
                     has_shared, ids, weights);
  return hipGetLastError();
}

hipError_t launch_topk_align(const float* logits, int T, int E, int top_k, int has_shared, int BM,
                             int cap, int32_t* ids, float* weights, int32_t* sorted, int32_t* eids,
                             int32_t* ntpp, hipStream_t stream) {
  if (!topk_align_fits(T, top_k, has_shared)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(topk_align_kernel, dim3(1), dim3(64 * T), 0, stream, logits, T, E, top_k,
                     has_shared, BM, cap, ids, weights, sorted, eids, ntpp);
  return hipGetLastError();
}

// Shared-gate only (no routed experts): weights[T*top_k + t] = sigmoid(logits[t, 0]).
namespace {
__global__ void shared_gate_sigmoid_kernel(const float* __restrict__ logits, int T, int top_k,
                                           float* __restrict__ weights) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  const float g = logits[(int64_t)t * 1];
  weights[(int64_t)T * top_k + t] = 1.0f / (1.0f + expf(-g));
}
}  // namespace

hipError_t launch_shared_gate(const uint16_t* x, int T, int H, const uint16_t* shared_w,
                              int top_k, float* logits_ws, float* weights, hipStream_t stream) {
  // E = 0 rows of router weight; row 0 is the shared gate. logits stride is E + 1 = 1.
  hipError_t err = launch_router_logits(x, T, H, nullptr, 0, shared_w, nullptr, logits_ws, stream);
  if (err != hipSuccess) return err;
  if (T == 0) return hipSuccess;
  hipLaunchKernelGGL(shared_gate_sigmoid_kernel, dim3((T + 255) / 256), dim3(256), 0, stream,
                     logits_ws, T, top_k, weights);
  return hipGetLastError();
}
