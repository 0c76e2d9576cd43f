// The residual add + RMSNorm of one token row by one 256-thread workgroup, shared by the norm
// kernel and the router kernel that normalises its own tokens, so both give the same bits:
//
//   r = bf16(res_in + add)  (fp32 add, RNE; r = res_in without add)
//   x = bf16((float(r) * rsqrt(mean(float(r)^2) + eps)) * (1 + float(w)))
//
// Semantics of mtp_rms_norm (src/mtp_expert_prefetch/mtp/extra_tensors.py:40-48: fp32 variance
// of the bf16 input, scaled by (1 + weight), cast back to the input dtype). Each thread owns 8
// consecutive columns per 2048-column chunk (16-byte loads); the sum of squares is fp32 in a
// fixed order: per thread over its columns in order, then a xor butterfly inside each wave, then
// the four wave sums in wave order.
#pragma once

#include "common.h"

constexpr int kNormThreads = 256;
constexpr int kNormChunk = kNormThreads * 8;  // columns per pass
constexpr int kNormMaxChunks = 4;             // hidden <= 8192

// All kNormThreads threads of the workgroup call it (one barrier inside), for TT token rows at
// once (all of their loads in flight together; each row's arithmetic is the one-row order).
// Row i: res_in[i], add[i] (nullable array entries), outputs (each nullable): res_out[i] = r,
// x_out[i] = x (global rows), x_lds + i * H = x (LDS). s_part: LDS of 4 * TT floats. res_out
// may be res_in (in place: every thread reads its columns before writing them).
template <int TT, int NC>
MOE_DEV void norm_rows(const uint16_t* const (&res_in)[TT], const uint16_t* const (&add)[TT],
                       const bool (&valid)[TT], int H, const uint16_t* __restrict__ w, float eps,
                       float* s_part, uint16_t* x_lds, uint16_t* const (&res_out)[TT],
                       uint16_t* const (&x_out)[TT]) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float v[TT][NC][8];
  float ss[TT];
#pragma unroll
  for (int i = 0; i < TT; ++i) {
    ss[i] = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int col = c * kNormChunk + 8 * tid;
      if (valid[i] && col < H) {
        const u32x4 r = ld128(res_in[i] + col);
        u32x4 rb = r;
        if (add[i]) {
          const u32x4 a = ld128(add[i] + col);
#pragma unroll
          for (int q = 0; q < 4; ++q)
            rb[q] = pack_bf16x2(bf16lo_to_f32(r[q]) + bf16lo_to_f32(a[q]),
                                bf16hi_to_f32(r[q]) + bf16hi_to_f32(a[q]));
        }
        if (res_out[i] && (add[i] || res_out[i] != res_in[i]))
          *reinterpret_cast<u32x4*>(res_out[i] + col) = rb;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          v[i][c][2 * q] = bf16lo_to_f32(rb[q]);
          v[i][c][2 * q + 1] = bf16hi_to_f32(rb[q]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][c][e] = 0.0f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss[i] = __builtin_fmaf(v[i][c][e], v[i][c][e], ss[i]);
    }
    ss[i] = bfly_sum(ss[i]);
    if (lane == 0) s_part[4 * i + wave] = ss[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < TT; ++i) {
    if (!valid[i]) continue;
    float tot = 0.0f;
#pragma unroll
    for (int q = 0; q < kNormThreads / 64; ++q) tot += s_part[4 * i + q];
    const float r = 1.0f / __builtin_sqrtf(tot / (float)H + eps);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int col = c * kNormChunk + 8 * tid;
      if (col >= H) continue;
      const u32x4 wv = ld128(w + col);
      u32x4 o;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        o[q] = pack_bf16x2((v[i][c][2 * q] * r) * (1.0f + bf16lo_to_f32(wv[q])),
                           (v[i][c][2 * q + 1] * r) * (1.0f + bf16hi_to_f32(wv[q])));
      if (x_out[i]) *reinterpret_cast<u32x4*>(x_out[i] + col) = o;
      if (x_lds) *reinterpret_cast<u32x4*>(x_lds + i * H + col) = o;
    }
  }
}
