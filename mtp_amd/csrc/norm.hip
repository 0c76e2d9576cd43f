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
#include "norm_row.h"

namespace {

// res_out may be res_in (in place).
template <int NC>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const uint16_t* res_in,
                                                               const uint16_t* __restrict__ add,
                                                               int H, const uint16_t* __restrict__ w,
                                                               float eps, uint16_t* res_out,
                                                               uint16_t* __restrict__ out) {
  __shared__ float s_part[kNormThreads / 64];
  const int64_t o = (int64_t)blockIdx.x * H;
  const uint16_t* const rin[1] = {res_in + o};
  const uint16_t* const ad[1] = {add ? add + o : nullptr};
  const bool valid[1] = {true};
  uint16_t* const rout[1] = {res_out + o};
  uint16_t* const xo[1] = {out + o};
  norm_rows<1, NC>(rin, ad, valid, H, w, eps, s_part, nullptr, rout, xo);
}

}  // namespace

hipError_t launch_rmsnorm(const uint16_t* res_in, const uint16_t* add, int T, int H,
                          const uint16_t* w, float eps, uint16_t* res_out, uint16_t* out,
                          hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  if (H <= 0 || H % 8 != 0 || H > kNormMaxChunks * kNormChunk) return hipErrorInvalidValue;
  const int nc = (H + kNormChunk - 1) / kNormChunk;
#define MOE_NORM_CASE(NCV)                                                                     \
  if (nc == NCV) {                                                                             \
    hipLaunchKernelGGL((rmsnorm_kernel<NCV>), dim3(T), dim3(kNormThreads), 0, stream, res_in,   \
                       add, H, w, eps, res_out, out);                                          \
    return hipGetLastError();                                                                  \
  }
  MOE_NORM_CASE(1) MOE_NORM_CASE(2) MOE_NORM_CASE(3) MOE_NORM_CASE(4)
#undef MOE_NORM_CASE
  return hipErrorInvalidValue;
}
