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
//
// The logits kernel tiles TT tokens x TE router rows per wave (small tiles at decode for more
// waves in flight, 8 x 8 at prefill for register reuse); the tile shape never changes the
// per-(token, row) summation order.
#include "common.h"
#include "launch.h"

namespace {

// logits[t, row] for rows 0..E-1 (router_w) and, if shared_w, row E (shared gate).
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
  const uint16_t* wrow[TE];
#pragma unroll
  for (int j = 0; j < TE; ++j) {
    const int e = e0 + j;
    wrow[j] = e < E ? W + (int64_t)e * H : (e == E && shared_w ? shared_w : nullptr);
  }
  const uint16_t* xrow[TT];
#pragma unroll
  for (int i = 0; i < TT; ++i) xrow[i] = (t0 + i < T) ? x + (int64_t)(t0 + i) * H : nullptr;
  float acc[TT][TE];
#pragma unroll
  for (int i = 0; i < TT; ++i)
#pragma unroll
    for (int j = 0; j < TE; ++j) acc[i][j] = 0.0f;

  const int nq = H / 8;
#pragma unroll 4
  for (int q = lane; q < nq; q += 64) {
    u32x4 xv[TT], wv[TE];
#pragma unroll
    for (int i = 0; i < TT; ++i) xv[i] = xrow[i] ? ld128(xrow[i] + 8 * q) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < TE; ++j) wv[j] = wrow[j] ? ld128(wrow[j] + 8 * q) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int el = 0; el < 8; ++el) {
      float wf[TE];
#pragma unroll
      for (int j = 0; j < TE; ++j)
        wf[j] = (el & 1) ? bf16hi_to_f32(wv[j][el >> 1]) : bf16lo_to_f32(wv[j][el >> 1]);
#pragma unroll
      for (int i = 0; i < TT; ++i) {
        const uint32_t xd = xv[i][el >> 1];
        const float xf = (el & 1) ? bf16hi_to_f32(xd) : bf16lo_to_f32(xd);
#pragma unroll
        for (int j = 0; j < TE; ++j) acc[i][j] = __builtin_fmaf(xf, wf[j], acc[i][j]);
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

// Total order on (logit, expert): larger logit first, then lower id. NaN never outranks.
MOE_DEV uint64_t topk_key(float v, int e) {
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  if ((__float_as_uint(v) & 0x7FFFFFFFu) > 0x7F800000u) u = 0;  // NaN ranks last
  return ((uint64_t)u << 32) | (uint32_t)(~(uint32_t)e);
}

#define MOE_DPP(v, ctrl, rmask) \
  (uint32_t) __builtin_amdgcn_update_dpp((int)(v), (int)(v), ctrl, rmask, 0xF, false)

MOE_DEV uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Wave-wide maximum of a 64-bit key through DPP (quad xor 1, quad xor 2, half-row mirror, row
// mirror, row_bcast15, row_bcast31); the result is read from lane 63 and is wave-uniform.
MOE_DEV uint64_t wave_max_u64(uint64_t v) {
#define MOE_DPP_STEP(ctrl, rmask)                                                     \
  do {                                                                                \
    const uint32_t lo = MOE_DPP((uint32_t)v, ctrl, rmask);                            \
    const uint32_t hi = MOE_DPP((uint32_t)(v >> 32), ctrl, rmask);                    \
    v = max_u64(v, ((uint64_t)hi << 32) | lo);                                        \
  } while (0)
  MOE_DPP_STEP(0xB1, 0xF);   // quad_perm(1,0,3,2)
  MOE_DPP_STEP(0x4E, 0xF);   // quad_perm(2,3,0,1)
  MOE_DPP_STEP(0x141, 0xF);  // row_half_mirror
  MOE_DPP_STEP(0x140, 0xF);  // row_mirror
  MOE_DPP_STEP(0x142, 0xA);  // row_bcast15 into rows 1, 3
  MOE_DPP_STEP(0x143, 0xC);  // row_bcast31 into rows 2, 3
#undef MOE_DPP_STEP
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, 63);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}

// One wave per token: top_k rounds of a wave-wide arg-max over (value desc, id asc).
__global__ __launch_bounds__(256) void router_topk_kernel(const float* __restrict__ logits, int T,
                                                          int E, int top_k, int has_shared,
                                                          int32_t* __restrict__ ids,
                                                          float* __restrict__ weights) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;
  constexpr int MAXC = 8;  // E <= 512
  const float* row = logits + (int64_t)t * (E + 1);
  uint64_t key[MAXC];
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int e = lane + 64 * c;
    key[c] = e < E ? topk_key(row[e], e) : 0ull;
  }
  float my_v = 0.0f;
  int my_i = 0;
  for (int r = 0; r < top_k; ++r) {
    uint64_t head = 0;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) head = max_u64(head, key[c]);
    const uint64_t best = wave_max_u64(head);
    const int e = (int)(~(uint32_t)best);
#pragma unroll
    for (int c = 0; c < MAXC; ++c)
      if (key[c] == best) key[c] = 0ull;  // exactly one lane/slot holds the unique key
    if (lane == r) {
      my_i = e;
      my_v = row[e];
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
