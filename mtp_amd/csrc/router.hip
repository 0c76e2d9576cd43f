// Router: fp32 logits in a canonical order, then top-k + renormalised softmax weights.
//
// Semantics: vLLM topk_softmax(renormalize=True) as restated at
// src/mtp_expert_prefetch/tracing/vllm_router_trace.py:4201-4225. Renormalisation cancels the
// softmax denominator, so w_i = exp(l_i - l_max) / sum_{j in top-k} exp(l_j - l_max).
//
// Canonical logit order (reproduced exactly by the CPU oracle): K is cut into chunks of 8
// bf16; chunk q belongs to lane q % 64; a lane accumulates its chunks in increasing q and the
// 8 elements in increasing k with fma from +0.0f (bf16*bf16 products are exact in fp32, so
// fma == add of the product); the 64 partials are combined by v += shfl_xor(v, m) for
// m = 32, 16, 8, 4, 2, 1. Ties in top-k: larger logit first, then lower expert id.
#include "common.h"
#include "launch.h"

namespace {

constexpr int TT = 4;  // tokens per wave tile
constexpr int TE = 4;  // router rows per wave tile

// logits[t, row] for rows 0..E-1 (router_w) and, if shared_w, row E (shared gate).
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
  const uint16_t* wrow[TE];
#pragma unroll
  for (int j = 0; j < TE; ++j) {
    const int e = e0 + j;
    wrow[j] = e < E ? W + (int64_t)e * H : (e == E && shared_w ? shared_w : nullptr);
  }
  float acc[TT][TE];
#pragma unroll
  for (int i = 0; i < TT; ++i)
#pragma unroll
    for (int j = 0; j < TE; ++j) acc[i][j] = 0.0f;

  const int nq = H / 8;
  for (int q = lane; q < nq; q += 64) {
    u32x4 xv[TT], wv[TE];
#pragma unroll
    for (int i = 0; i < TT; ++i)
      xv[i] = (t0 + i < T) ? ld128(x + (int64_t)(t0 + i) * H + 8 * q) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < TE; ++j) wv[j] = wrow[j] ? ld128(wrow[j] + 8 * q) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int el = 0; el < 8; ++el) {
#pragma unroll
      for (int i = 0; i < TT; ++i) {
        const uint32_t xd = xv[i][el >> 1];
        const float xf = (el & 1) ? bf16hi_to_f32(xd) : bf16lo_to_f32(xd);
#pragma unroll
        for (int j = 0; j < TE; ++j) {
          const uint32_t wd = wv[j][el >> 1];
          const float wf = (el & 1) ? bf16hi_to_f32(wd) : bf16lo_to_f32(wd);
          acc[i][j] = __builtin_fmaf(xf, wf, acc[i][j]);
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < TT; ++i)
#pragma unroll
    for (int j = 0; j < TE; ++j) {
      float v = acc[i][j];
      v = wave_xor_sum(v, 32);
      v = wave_xor_sum(v, 16);
      v = wave_xor_sum(v, 8);
      v = wave_xor_sum(v, 4);
      v = wave_xor_sum(v, 2);
      v = wave_xor_sum(v, 1);
      acc[i][j] = v;
    }
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < TT; ++i)
#pragma unroll
      for (int j = 0; j < TE; ++j) {
        const int t = t0 + i, e = e0 + j;
        if (t < T && e < rows) {
          float v = acc[i][j];
          if (bias && e < E) v = v + bias[e];
          logits[(int64_t)t * (E + 1) + e] = v;
        }
      }
  }
}

// One wave per token: iterative arg-max with (value desc, id asc) ordering.
__global__ __launch_bounds__(256) void router_topk_kernel(const float* __restrict__ logits, int T,
                                                          int E, int top_k, int has_shared,
                                                          int32_t* __restrict__ ids,
                                                          float* __restrict__ weights) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;
  constexpr int MAXC = 8;  // E <= 512
  const float* row = logits + (int64_t)t * (E + 1);
  float v[MAXC];
  bool taken[MAXC];
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int e = lane + 64 * c;
    v[c] = e < E ? row[e] : 0.0f;
    taken[c] = !(e < E);
  }
  float my_v = 0.0f;
  int my_i = 0;
  for (int r = 0; r < top_k; ++r) {
    float bv = -__builtin_huge_valf();
    int bi = 0x7fffffff;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const int e = lane + 64 * c;
      if (!taken[c] && (bi == 0x7fffffff || v[c] > bv || (v[c] == bv && e < bi))) {
        bv = v[c];
        bi = e;
      }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      const float ov = __shfl_xor(bv, m, 64);
      const int oi = __shfl_xor(bi, m, 64);
      const bool other_better =
          (oi != 0x7fffffff) && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi));
      if (other_better) {
        bv = ov;
        bi = oi;
      }
    }
    if (bi != 0x7fffffff && (bi & 63) == lane) {
#pragma unroll
      for (int c = 0; c < MAXC; ++c)
        if (c == (bi >> 6)) taken[c] = true;
    }
    if (lane == r) {
      my_v = bv;
      my_i = bi;
    }
  }
  const float vmax = __shfl(my_v, 0, 64);
  const float ex = (lane < top_k) ? expf(my_v - vmax) : 0.0f;
  float s = 0.0f;
  for (int r = 0; r < top_k; ++r) s = s + __shfl(ex, r, 64);
  if (lane < top_k) {
    ids[(int64_t)t * top_k + lane] = my_i;
    weights[(int64_t)t * top_k + lane] = ex / s;
  }
  if (has_shared && lane == 0) {
    const float g = row[E];
    weights[(int64_t)T * top_k + t] = 1.0f / (1.0f + expf(-g));
  }
}

}  // namespace

hipError_t launch_router_logits(const uint16_t* x, int T, int H, const uint16_t* W, int E,
                                const uint16_t* shared_w, const float* bias, float* logits,
                                hipStream_t stream) {
  const int rows = E + (shared_w ? 1 : 0);
  const int tiles = ((T + TT - 1) / TT) * ((rows + TE - 1) / TE);
  const int blocks = (tiles + 3) / 4;
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(router_logits_kernel, dim3(blocks), dim3(256), 0, stream, x, T, H, W, E,
                     shared_w, bias, logits);
  return hipGetLastError();
}

hipError_t launch_router_topk(const float* logits, int T, int E, int top_k, int has_shared,
                              int32_t* ids, float* weights, hipStream_t stream) {
  const int blocks = (T + 3) / 4;
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(router_topk_kernel, dim3(blocks), dim3(256), 0, stream, logits, T, E, top_k,
                     has_shared, ids, weights);
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
