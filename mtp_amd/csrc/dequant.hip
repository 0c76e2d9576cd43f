// GPTQ int4 -> bf16 dequantisation (load-time utility path).
//
// Follows src/mtp_expert_prefetch/repack/gptq_unpack.py:88-131:
//   W[k, n] = bf16_rne( (float(q[k, n]) - float(z[g(k), n])) * float(s[g(k), n]) )
// The fp32 product is exact (|q - z| <= 15 times an fp16), so the only rounding is the
// final cast (RNE to bf16 or fp16, none for fp32), which makes the result bit-identical to the
// reference for every output dtype.
#include "common.h"
#include "launch.h"

namespace {

template <int OUT>  // 0 bf16, 1 fp16, 2 fp32
__global__ __launch_bounds__(256) void dequant_kernel(ProjDev p, const int32_t* __restrict__ g_idx,
                                                      int K, int N, int G, int linear,
                                                      void* __restrict__ out_v) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int r = blockIdx.y;
  const int64_t e = blockIdx.z;
  if (n >= N) return;
  const int ngroups = K / G;
  const uint32_t w = (uint32_t)p.qweight[(e * (K / 8) + r) * N + n];
  const int32_t* zrow = p.qzeros + e * ngroups * (N / 8);
  const uint16_t* srow = p.scales + e * ngroups * N;
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int k = 8 * r + j;
    int g = g_idx ? g_idx[e * K + k] : k / G;
    g = g < 0 ? 0 : (g >= ngroups ? ngroups - 1 : g);
    const uint32_t z = ((uint32_t)zrow[g * (N / 8) + n / 8] >> (4 * (n & 7))) & 0xFu;
    const float s = f16_to_f32(srow[g * N + n]);
    const float q = (float)((w >> (4 * j)) & 0xFu);
    v[j] = (q - (float)z) * s;
  }
  if (OUT == 2) {
    float* out = static_cast<float*>(out_v);
    if (linear) {
      f32x4* o = reinterpret_cast<f32x4*>(out + (e * N + n) * K + 8 * r);
      o[0] = f32x4{v[0], v[1], v[2], v[3]};
      o[1] = f32x4{v[4], v[5], v[6], v[7]};
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) out[(e * K + 8 * r + j) * N + n] = v[j];
    }
    return;
  }
  uint32_t hbits[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    hbits[j] = (OUT == 0) ? f32_to_bf16_rne(v[j])
                          : (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[j]);
  uint16_t* out = static_cast<uint16_t*>(out_v);
  if (linear) {
    u32x4 o;
    o[0] = hbits[0] | (hbits[1] << 16);
    o[1] = hbits[2] | (hbits[3] << 16);
    o[2] = hbits[4] | (hbits[5] << 16);
    o[3] = hbits[6] | (hbits[7] << 16);
    *reinterpret_cast<u32x4*>(out + (e * N + n) * K + 8 * r) = o;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) out[(e * K + 8 * r + j) * N + n] = (uint16_t)hbits[j];
  }
}

}  // namespace

hipError_t launch_dequant(const ProjDev& p, const int32_t* g_idx, int E, int K, int N, int G,
                          int linear, int out_dtype, void* out, hipStream_t stream) {
  dim3 grid((N + 255) / 256, K / 8, E);
  switch (out_dtype) {
    case 0:
      hipLaunchKernelGGL(dequant_kernel<0>, grid, dim3(256), 0, stream, p, g_idx, K, N, G, linear, out);
      break;
    case 1:
      hipLaunchKernelGGL(dequant_kernel<1>, grid, dim3(256), 0, stream, p, g_idx, K, N, G, linear, out);
      break;
    case 2:
      hipLaunchKernelGGL(dequant_kernel<2>, grid, dim3(256), 0, stream, p, g_idx, K, N, G, linear, out);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
