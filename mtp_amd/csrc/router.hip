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
#include "norm_row.h"
#include "routing.h"

namespace {

template <int TT, int TE>
__global__ __launch_bounds__(256) void router_logits_kernel(
    const uint16_t* __restrict__ x, int T, int H, const uint16_t* __restrict__ W, int E,
    const uint16_t* __restrict__ shared_w, const float* __restrict__ bias,
    float* __restrict__ logits) {
  const int rows = E + (shared_w ? 1 : 0);
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tiles_e = (rows + TE - 1) / TE;
  const int t0 = (wave / tiles_e) * TT;
  const int e0 = (wave % tiles_e) * TE;
  if (t0 >= T) return;
  logits_tile<TT, TE>(x, T, H, W, E, shared_w, bias, logits, t0, e0, lane);
}

// Router of a decoder step with the step's residual add + RMSNorm folded in: workgroup = one
// tile of TT tokens x (4 waves x TE) router rows. The waves first issue the loads of their
// router rows, then the workgroup normalises its TT tokens into LDS (norm_row, the bits of the
// norm kernel); the first workgroup of each token tile also writes the updated residual and the
// normalised rows (the layer's input for W1). res_out must not be res_in: the other workgroups
// of the tile still read res_in. H <= 2048.
template <int TT, int TE>
__global__ __launch_bounds__(kNormThreads) void router_logits_norm_kernel(
    const uint16_t* __restrict__ res_in, const uint16_t* __restrict__ add,
    const uint16_t* __restrict__ norm_w, float eps, uint16_t* __restrict__ res_out,
    uint16_t* __restrict__ x_out, int T, int H, const uint16_t* __restrict__ W, int E,
    const uint16_t* __restrict__ shared_w, const float* __restrict__ bias,
    float* __restrict__ logits) {
  __shared__ __attribute__((aligned(16))) uint16_t s_x[TT * kNormChunk];
  __shared__ float s_part[TT * (kNormThreads / 64)];
  const int rows = E + (shared_w ? 1 : 0);
  const int tiles_e = (rows + TE - 1) / TE;
  const int groups = (tiles_e + 3) / 4;  // workgroups per token tile
  const int tt = (int)blockIdx.x / groups, eg = (int)blockIdx.x % groups;
  const int t0 = tt * TT;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int e_tile = eg * 4 + wave;
  LdsLogitsTile<TT, TE> tile;
  if (e_tile < tiles_e) tile.load(H, W, E, shared_w, e_tile * TE, lane);
  const bool writer = eg == 0;
  const uint16_t* rin[TT];
  const uint16_t* ad[TT];
  bool valid[TT];
  uint16_t* rout[TT];
  uint16_t* xo[TT];
#pragma unroll
  for (int i = 0; i < TT; ++i) {
    const int t = t0 + i;
    valid[i] = t < T;
    const int64_t o = (int64_t)(valid[i] ? t : 0) * H;
    rin[i] = res_in + o;
    ad[i] = add ? add + o : nullptr;
    rout[i] = writer && valid[i] ? res_out + o : nullptr;
    xo[i] = writer && valid[i] ? x_out + o : nullptr;
  }
  norm_rows<TT, 1>(rin, ad, valid, H, norm_w, eps, s_part, s_x, rout, xo);
  __syncthreads();  // the s_x rows are complete
  if (e_tile < tiles_e)
    tile.compute_store(s_x, T, H, E, shared_w != nullptr, bias, logits, t0, e_tile * TE, lane);
}

template <int TT, int TE>
hipError_t launch_logits_norm(const uint16_t* res_in, const uint16_t* add, const uint16_t* norm_w,
                              float eps, uint16_t* res_out, uint16_t* x_out, int T, int H,
                              const uint16_t* W, int E, const uint16_t* shared_w,
                              const float* bias, float* logits, hipStream_t stream) {
  const int rows = E + (shared_w ? 1 : 0);
  const int groups = ((rows + TE - 1) / TE + 3) / 4;
  const int blocks = (T + TT - 1) / TT * groups;
  hipLaunchKernelGGL((router_logits_norm_kernel<TT, TE>), dim3(blocks), dim3(kNormThreads), 0,
                     stream, res_in, add, norm_w, eps, res_out, x_out, T, H, W, E, shared_w, bias,
                     logits);
  return hipGetLastError();
}

// Prefill-size logits: one wave per 8 x 8 (token x router-row) tile, H a multiple of 512 (one
// step = the 64 lanes' 16-byte chunks of every row). The summation order is the canonical one of
// logits_tile: lane l owns chunks l, l + 64, ..., fma from +0.0f over chunks then elements. The
// loads of step s + 1 are issued before the arithmetic of step s, and the kernel keeps at most
// 256 VGPRs so two waves share each SIMD.
//
// The 64 per-lane partials are then combined by a transposed butterfly: at the step of lane
// mask m every lane keeps the half of its values whose index bit matches its own lane bit and
// adds the partner's (lane ^ m) copy of the same values. Every addition is the one the
// butterfly v += shfl_xor(v, m) makes at that lane (the same two operands, and fp32 addition is
// commutative), so the result is bit-identical, with 63 exchanges instead of 6 x 64. After the
// last step lane l holds value l = (token i = l >> 3, row j = l & 7).
constexpr int kRowsTileT = 8, kRowsTileE = 8;

template <int N, int HALF>
MOE_DEV void fold_swap32(float (&a)[N]) {
#pragma unroll
  for (int v = 0; v < HALF; ++v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[v]),
                                                    __float_as_uint(a[v + HALF]), false, false);
    a[v] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

template <int N, int HALF>
MOE_DEV void fold_swap16(float (&a)[N]) {
#pragma unroll
  for (int v = 0; v < HALF; ++v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[v]),
                                                    __float_as_uint(a[v + HALF]), false, false);
    a[v] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

// Lane mask M in {8, 4, 2, 1}: rows of 16 lanes, exchanged with DPP.
template <int M, int N>
MOE_DEV void fold_dpp(float (&a)[N], int lane) {
  const bool up = (lane & M) != 0;
#pragma unroll
  for (int v = 0; v < M; ++v) {
    const float keep = up ? a[v + M] : a[v];
    const int send = __float_as_int(up ? a[v] : a[v + M]);
    int recv;
    if constexpr (M == 8) {
      recv = __builtin_amdgcn_update_dpp(0, send, 0x128, 0xF, 0xF, false);  // row_ror:8
    } else if constexpr (M == 4) {
      recv = __shfl_xor(send, 4, 64);  // no single row DPP pattern pairs lane i with i ^ 4
    } else if constexpr (M == 2) {
      recv = __builtin_amdgcn_update_dpp(0, send, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else {
      recv = __builtin_amdgcn_update_dpp(0, send, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    }
    a[v] = keep + __int_as_float(recv);
  }
}

MOE_DEV float bf16_elem(const u32x4& v, int el) {
  return (el & 1) ? bf16hi_to_f32(v[el >> 1]) : bf16lo_to_f32(v[el >> 1]);
}

__global__ __launch_bounds__(256, 2) void router_logits_rows_kernel(
    const uint16_t* __restrict__ x, int T, int H, const uint16_t* __restrict__ W, int E,
    const uint16_t* __restrict__ shared_w, const float* __restrict__ bias,
    float* __restrict__ logits) {
  constexpr int TT = kRowsTileT, TE = kRowsTileE;
  const int rows = E + (shared_w ? 1 : 0);
  const int lane = threadIdx.x & 63;
  // wave index as a uniform (scalar) value: row pointers live in SGPRs, loads use saddr forms
  const int wave = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
  const int tiles_e = (rows + TE - 1) / TE;
  const int t0 = (wave / tiles_e) * TT;
  const int e0 = (wave % tiles_e) * TE;
  if (t0 >= T) return;
  // Buffer loads: token rows past T, router rows past the last one and steps past H read zeros
  // without a memory access (their results are not stored), so every step issues the same
  // loads and the waits stay exact.
  const __amdgpu_buffer_rsrc_t xrs = buf_rsrc(x, (uint32_t)T * (uint32_t)H * 2u);
  const __amdgpu_buffer_rsrc_t wrs = buf_rsrc(W, (uint32_t)E * (uint32_t)H * 2u);
  const __amdgpu_buffer_rsrc_t srs = buf_rsrc(shared_w, shared_w ? (uint32_t)H * 2u : 0u);
  uint32_t xo[TT], wo[TE];
#pragma unroll
  for (int i = 0; i < TT; ++i) xo[i] = t0 + i < T ? (uint32_t)(t0 + i) * (uint32_t)H * 2u : kOutOfRange;
#pragma unroll
  for (int j = 0; j < TE; ++j) {
    const int e = e0 + j;
    wo[j] = e < E ? (uint32_t)e * (uint32_t)H * 2u : (e < rows ? 0u : kOutOfRange);
  }
  float acc[TT * TE];
#pragma unroll
  for (int v = 0; v < TT * TE; ++v) acc[v] = 0.0f;

  const int nsteps = H / 512;
  u32x4 xa[TT], wa[TE], xb[TT], wb[TE];
  auto load = [&](u32x4(&xv)[TT], u32x4(&wv)[TE], int step) {
    const uint32_t so = step < nsteps ? (uint32_t)(step * 512 + lane * 8) * 2u : kOutOfRange;
#pragma unroll
    for (int i = 0; i < TT; ++i) xv[i] = buf_ld128(xrs, (xo[i] + so) | (so & kOutOfRange));
#pragma unroll
    for (int j = 0; j < TE; ++j)
      wv[j] = buf_ld128(e0 + j == E ? srs : wrs, (wo[j] + so) | (so & kOutOfRange));
  };
  auto compute = [&](const u32x4(&xv)[TT], const u32x4(&wv)[TE]) {
#pragma unroll
    for (int el = 0; el < 8; ++el) {
      float wf[TE];
#pragma unroll
      for (int j = 0; j < TE; ++j) wf[j] = bf16_elem(wv[j], el);
#pragma unroll
      for (int i = 0; i < TT; ++i) {
        const float xf = bf16_elem(xv[i], el);
#pragma unroll
        for (int j = 0; j < TE; ++j) acc[i * TE + j] = __builtin_fmaf(xf, wf[j], acc[i * TE + j]);
      }
    }
  };
  // The next step's loads are issued before the current step's arithmetic (scheduling barriers
  // keep them there). Steps go in pairs with both computes unconditional (a load whose only use
  // sits under a condition would be moved into that branch, after the other step's arithmetic);
  // an odd last step is computed after the loop, and a step past H is loaded (zeros) but never
  // computed.
  load(xa, wa, 0);
  for (int s = 0; s + 1 < nsteps; s += 2) {
    load(xb, wb, s + 1);
    __builtin_amdgcn_sched_barrier(0);
    compute(xa, wa);
    load(xa, wa, s + 2);
    __builtin_amdgcn_sched_barrier(0);
    compute(xb, wb);
  }
  if (nsteps & 1) compute(xa, wa);

  fold_swap32<TT * TE, 32>(acc);
  fold_swap16<TT * TE, 16>(acc);
  fold_dpp<8>(acc, lane);
  fold_dpp<4>(acc, lane);
  fold_dpp<2>(acc, lane);
  fold_dpp<1>(acc, lane);

  const int t = t0 + (lane >> 3), e = e0 + (lane & 7);
  if (t < T && e < rows) {
    float v = acc[0];
    if (bias && e < E) v = v + bias[e];
    logits[(int64_t)t * (E + 1) + e] = v;
  }
}

__global__ __launch_bounds__(256) void router_topk_kernel(const float* __restrict__ logits, int T,
                                                          int E, int top_k, int has_shared,
                                                          int32_t* __restrict__ ids,
                                                          float* __restrict__ weights,
                                                          int32_t* __restrict__ ids_mirror,
                                                          int32_t* __restrict__ flags,
                                                          int32_t seq) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (t >= T) return;
  topk_token_any(logits + (int64_t)t * (E + 1), E, top_k, has_shared, T, t, lane, ids, weights,
                 nullptr, ids_mirror);
  if (flags) {  // the token's ids (in host memory) before its flag
    __threadfence_system();
    if (lane == 0) __hip_atomic_store(flags + t, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// One wave per token for the top-k, then wave 0 aligns the (at most 64) slots.
__global__ __launch_bounds__(64 * kTopkAlignMaxTokens) void topk_align_kernel(
    const float* __restrict__ logits, int T, int E, int top_k, int has_shared, int BM, int cap,
    int32_t* __restrict__ ids, float* __restrict__ weights, int32_t* __restrict__ sorted,
    int32_t* __restrict__ eids, int32_t* __restrict__ ntpp) {
  __shared__ int s_ids[kAlignWaveMaxSlots];
  __shared__ int s_pad[kMaxGroups];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (wave < T)
    topk_token_any(logits + (int64_t)wave * (E + 1), E, top_k, has_shared, T, wave, lane, ids,
               weights, s_ids);
  __syncthreads();
  if (wave == 0)
    align_wave(s_ids, T, top_k, E, has_shared, BM, cap, sorted, eids, ntpp, lane, s_pad,
               false);  // internal layout: the decode kernels stop at the padded total
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
  if (H % 512 == 0) {
    const int rows = E + (shared_w ? 1 : 0);
    const int tiles = ((T + kRowsTileT - 1) / kRowsTileT) * ((rows + kRowsTileE - 1) / kRowsTileE);
    if (tiles == 0) return hipSuccess;
    hipLaunchKernelGGL(router_logits_rows_kernel, dim3((tiles + 3) / 4), dim3(256), 0, stream, x,
                       T, H, W, E, shared_w, bias, logits);
    return hipGetLastError();
  }
  return launch_logits_tiled<8, 8>(x, T, H, W, E, shared_w, bias, logits, stream);
}

// The fused form writes the new residual from one workgroup per token tile while the others
// still read res_in: the two row sets must not share any byte (in place included).
bool router_norm_fits(int T, int H, const void* res_in, const void* res_out) {
  const uintptr_t p = (uintptr_t)res_in, q = (uintptr_t)res_out, rows = (uintptr_t)T * H * 2;
  return T >= 1 && T <= 64 && H >= 8 && H <= kNormChunk && H % 8 == 0 &&
         (p + rows <= q || q + rows <= p);
}

hipError_t launch_router_logits_norm(const uint16_t* res_in, const uint16_t* add,
                                     const uint16_t* norm_w, float eps, uint16_t* res_out,
                                     uint16_t* x_out, int T, int H, const uint16_t* W, int E,
                                     const uint16_t* shared_w, const float* bias, float* logits,
                                     hipStream_t stream) {
  if (!router_norm_fits(T, H, res_in, res_out)) return hipErrorInvalidValue;
  if (T <= 4)  // the tiles of launch_router_logits
    return launch_logits_norm<1, 2>(res_in, add, norm_w, eps, res_out, x_out, T, H, W, E,
                                    shared_w, bias, logits, stream);
  return launch_logits_norm<2, 4>(res_in, add, norm_w, eps, res_out, x_out, T, H, W, E, shared_w,
                                  bias, logits, stream);
}

hipError_t launch_router_topk(const float* logits, int T, int E, int top_k, int has_shared,
                              int32_t* ids, float* weights, hipStream_t stream,
                              int32_t* ids_mirror, int32_t* flags, int32_t seq) {
  const int blocks = (T + 3) / 4;
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(router_topk_kernel, dim3(blocks), dim3(256), 0, stream, logits, T, E, top_k,
                     has_shared, ids, weights, ids_mirror, flags, seq);
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
