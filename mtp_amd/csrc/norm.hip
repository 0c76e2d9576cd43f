// Residual add + RMSNorm of a decoder step: the caller of the MoE layer in a layer loop.
//
//   res[t, :] = bf16(res[t, :] + add[t, :])        (when add is given; fp32 add, RNE)
//   out[t, :] = bf16((float(res[t, :]) * rsqrt(mean(float(res[t, :])^2) + eps)) * (1 + float(w)))
//
// Semantics of mtp_rms_norm (src/mtp_expert_prefetch/mtp/extra_tensors.py:40-48: fp32 variance
// of the bf16 input, scaled by (1 + weight), cast back to the input dtype) applied to the residual
// stream of the decoder layer loop around moe_forward_with_trace
// (src/mtp_expert_prefetch/tracing/vllm_router_trace.py:17895-17965).
//
// One 256-thread workgroup per token row; each thread owns 8 consecutive columns per 2048-column
// chunk (16-byte loads). The sum of squares is fp32 in a fixed order: per thread over its columns
// in order, then a xor butterfly inside each wave, then the four wave sums in wave order.
#include "common.h"
#include "launch.h"

namespace {

constexpr int kNormThreads = 256;
constexpr int kNormChunk = kNormThreads * 8;  // columns per pass
constexpr int kNormMaxChunks = 4;             // hidden <= 8192

template <int NC>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(uint16_t* __restrict__ res,
                                                               const uint16_t* __restrict__ add,
                                                               int H, const uint16_t* __restrict__ w,
                                                               float eps,
                                                               uint16_t* __restrict__ out) {
  __shared__ float s_part[kNormThreads / 64];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint16_t* rrow = res + (int64_t)t * H;
  const uint16_t* arow = add ? add + (int64_t)t * H : nullptr;
  float v[NC][8];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int col = c * kNormChunk + 8 * tid;
    if (col < H) {
      const u32x4 r = ld128(rrow + col);
      u32x4 rb = r;
      if (arow) {
        const u32x4 a = ld128(arow + col);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          rb[q] = pack_bf16x2(bf16lo_to_f32(r[q]) + bf16lo_to_f32(a[q]),
                              bf16hi_to_f32(r[q]) + bf16hi_to_f32(a[q]));
        *reinterpret_cast<u32x4*>(rrow + col) = rb;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[c][2 * q] = bf16lo_to_f32(rb[q]);
        v[c][2 * q + 1] = bf16hi_to_f32(rb[q]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[c][e] = 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(v[c][e], v[c][e], ss);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss = wave_xor_sum(ss, m);
  if (lane == 0) s_part[wave] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int q = 0; q < kNormThreads / 64; ++q) tot += s_part[q];
  const float r = 1.0f / __builtin_sqrtf(tot / (float)H + eps);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int col = c * kNormChunk + 8 * tid;
    if (col >= H) continue;
    const u32x4 wv = ld128(w + col);
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      o[q] = pack_bf16x2((v[c][2 * q] * r) * (1.0f + bf16lo_to_f32(wv[q])),
                         (v[c][2 * q + 1] * r) * (1.0f + bf16hi_to_f32(wv[q])));
    *reinterpret_cast<u32x4*>(out + (int64_t)t * H + col) = o;
  }
}

}  // namespace

hipError_t launch_rmsnorm(uint16_t* res, const uint16_t* add, int T, int H, const uint16_t* w,
                          float eps, uint16_t* out, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  if (H <= 0 || H % 8 != 0 || H > kNormMaxChunks * kNormChunk) return hipErrorInvalidValue;
  const int nc = (H + kNormChunk - 1) / kNormChunk;
#define MOE_NORM_CASE(NCV)                                                                     \
  if (nc == NCV) {                                                                             \
    hipLaunchKernelGGL((rmsnorm_kernel<NCV>), dim3(T), dim3(kNormThreads), 0, stream, res, add, \
                       H, w, eps, out);                                                        \
    return hipGetLastError();                                                                  \
  }
  MOE_NORM_CASE(1) MOE_NORM_CASE(2) MOE_NORM_CASE(3) MOE_NORM_CASE(4)
#undef MOE_NORM_CASE
  return hipErrorInvalidValue;
}
