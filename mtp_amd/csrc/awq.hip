// AWQ int4 checkpoints behind the GPTQ kernels: an exact load-time repack into the reference's
// GPTQ layout (qweight int32 [E, K/8, N] packed along K, qzeros int32 [E, K/G, N/8] packed
// along N, scales fp16 [E, K/G, N]). Only nibbles and scale bits move, so every dequantised
// weight (q - z) * s is unchanged.
//
// Source layouts:
//  * MOE_AWQ_WNA16: vLLM's int4 fused-MoE layout that the reference serves its AWQ checkpoint
//    with (src/mtp_expert_prefetch/tracing/vllm_wna16_group_plan.py:394-470): B uint8
//    [E, N, K/2], q(k, n) in nibble k % 2 of byte (n, k / 2); zero points uint8 [E, N/2, K/G],
//    z(g, n) in nibble n % 2 of byte (n / 2, g), or none (zero 8); scales [E, N, K/G] in fp16 or
//    bf16. The bytes of one (n, 8 k) run are exactly one GPTQ word, so qweight is a transpose of
//    32-bit words.
//  * MOE_AWQ_GEMM: the AutoAWQ GEMM checkpoint layout: qweight int32 [E, K, N/8] and qzeros
//    int32 [E, K/G, N/8] packed along N in the order [0, 2, 4, 6, 1, 3, 5, 7]; scales fp16
//    [E, K/G, N].
// A bf16 scale outside [2^-17, 65504] (not exact in fp16) sets *status to 1; 0 means every
// value moved exactly. One thread per output word; byte and integer work, bound by HBM.
#include <stdio.h>

#include "common.h"
#include "launch.h"

namespace {

// nibble i of an AutoAWQ word holds column 8 c + kAwqOrder[i]; column j sits at nibble kAwqInv[j]
__constant__ int kAwqInv[8] = {0, 4, 1, 5, 2, 6, 3, 7};

__global__ void awq_qweight_kernel(int layout, const void* __restrict__ src, int E, int K, int N,
                                   int32_t* __restrict__ dst) {
  const int64_t K8 = K / 8;
  const int64_t total = (int64_t)E * K8 * N;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e = i / (K8 * N), rem = i % (K8 * N);
    const int64_t r = rem / N, n = rem % N;  // GPTQ word (r, n): q(8 r + j, n) at nibble j
    uint32_t w = 0;
    if (layout == MOE_AWQ_WNA16) {
      w = static_cast<const uint32_t*>(src)[(e * N + n) * K8 + r];
    } else {
      const uint32_t* s = static_cast<const uint32_t*>(src);
      const int sh = 4 * kAwqInv[n & 7];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t v = s[(e * K + 8 * r + j) * (N / 8) + (n >> 3)];
        w |= ((v >> sh) & 0xFu) << (4 * j);
      }
    }
    dst[i] = (int32_t)w;
  }
}

__global__ void awq_qzeros_kernel(int layout, const void* __restrict__ src, int E, int NG, int N,
                                  int32_t* __restrict__ dst) {
  const int64_t C = N / 8;
  const int64_t total = (int64_t)E * NG * C;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e = i / (NG * C), rem = i % (NG * C);
    const int64_t g = rem / C, c = rem % C;  // GPTQ word (g, c): z(g, 8 c + j) at nibble j
    uint32_t w = 0;
    if (!src) {
      w = 0x88888888u;  // symmetric checkpoint: zero point 8
    } else if (layout == MOE_AWQ_WNA16) {
      const uint8_t* s = static_cast<const uint8_t*>(src);
#pragma unroll
      for (int j = 0; j < 8; j += 2) {  // columns 8c + j, 8c + j + 1 share byte (4c + j/2, g)
        const uint32_t v = s[(e * (N / 2) + 4 * c + j / 2) * NG + g];
        w |= (v & 0xFu) << (4 * j);
        w |= ((v >> 4) & 0xFu) << (4 * (j + 1));
      }
    } else {
      const uint32_t v = static_cast<const uint32_t*>(src)[(e * NG + g) * C + c];
#pragma unroll
      for (int j = 0; j < 8; ++j) w |= ((v >> (4 * kAwqInv[j])) & 0xFu) << (4 * j);
    }
    dst[i] = (int32_t)w;
  }
}

// fp16 bits of a bf16 value, exact for magnitudes in [2^-17, 65504] and zero; else *bad = 1
// (a plain store: every writer stores the same value).
MOE_DEV uint16_t bf16_to_f16_exact(uint16_t b, int32_t* bad) {
  const float f = bf16_to_f32(b);
  const _Float16 h = (_Float16)f;
  if (!((float)h == f)) *bad = 1;
  return __builtin_bit_cast(uint16_t, h);
}

__global__ void awq_scales_kernel(int layout, const uint16_t* __restrict__ src, int src_bf16,
                                  int E, int NG, int N, uint16_t* __restrict__ dst,
                                  int32_t* __restrict__ bad) {
  const int64_t total = (int64_t)E * NG * N;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e = i / ((int64_t)NG * N), rem = i % ((int64_t)NG * N);
    const int64_t g = rem / N, n = rem % N;
    const uint16_t v = layout == MOE_AWQ_WNA16 ? src[(e * N + n) * NG + g] : src[i];
    dst[i] = src_bf16 ? bf16_to_f16_exact(v, bad) : v;
  }
}

__global__ void awq_status_clear(int32_t* status) { *status = 0; }

unsigned grid_for(int64_t n) { return (unsigned)((n + 255) / 256 < 8192 ? (n + 255) / 256 : 8192); }

}  // namespace

extern "C" {

int moe_awq_to_gptq_v1(int32_t layout, const void* qweight, const void* qzeros,
                       const uint16_t* scales, int32_t scales_bf16, int32_t num_experts,
                       int32_t in_features, int32_t out_features, int32_t group_size,
                       const moe_gptq_proj_v1* out, int32_t* status, void* stream) {
  auto err = [](int code, const char* msg) {
    snprintf(moe_error_buffer(), kErrorBufferBytes, "awq_to_gptq: %s", msg);
    return code;
  };
  if (layout != MOE_AWQ_WNA16 && layout != MOE_AWQ_GEMM) return err(MOE_ERR_UNSUPPORTED, "layout");
  if (!qweight || !scales || !out || !out->qweight || !out->qzeros || !out->scales || !status)
    return err(MOE_ERR_NULL, "NULL pointer");
  if (layout == MOE_AWQ_GEMM && (!qzeros || scales_bf16))
    return err(MOE_ERR_UNSUPPORTED, "the AutoAWQ GEMM layout has zero points and fp16 scales");
  const int K = in_features, N = out_features, G = group_size, E = num_experts;
  if (E < 1 || K < 8 || N < 8 || K % 8 || N % 8 || G < 8 || K % G)
    return err(MOE_ERR_SHAPE, "need K % 8 == 0, N % 8 == 0, G | K");
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(awq_status_clear, dim3(1), dim3(1), 0, s, status);
  const int64_t nq = (int64_t)E * (K / 8) * N, nz = (int64_t)E * (K / G) * (N / 8),
                ns = (int64_t)E * (K / G) * N;
  // out names the caller's GPTQ tensors (the descriptor is the read-only one the kernels take)
  int32_t* oq = const_cast<int32_t*>(out->qweight);
  int32_t* oz = const_cast<int32_t*>(out->qzeros);
  uint16_t* os = const_cast<uint16_t*>(out->scales);
  hipLaunchKernelGGL(awq_qweight_kernel, dim3(grid_for(nq)), dim3(256), 0, s, layout, qweight, E,
                     K, N, oq);
  hipLaunchKernelGGL(awq_qzeros_kernel, dim3(grid_for(nz)), dim3(256), 0, s, layout, qzeros, E,
                     K / G, N, oz);
  hipLaunchKernelGGL(awq_scales_kernel, dim3(grid_for(ns)), dim3(256), 0, s, layout, scales,
                     scales_bf16 ? 1 : 0, E, K / G, N, os, status);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    snprintf(moe_error_buffer(), kErrorBufferBytes, "awq_to_gptq: HIP error %d (%s)", (int)e,
             hipGetErrorString(e));
    return MOE_ERR_HIP + ((int)e % 100);
  }
  return MOE_OK;
}

}  // extern "C"
