// Decode path (token batches up to a few hundred slots): grouped int4 GEMM on MFMA with the
// int4 weights dequantised in registers directly into the MFMA B operand.
//
// Block = one expert block of 16 slots (the M dimension of v_mfma_f32_16x16x32_bf16) x one
// 32-column tile; every wave of the block owns a 256-wide slice of K and the per-wave partial
// tiles are summed once through LDS in wave order (deterministic).
//
// B operand: lane l of a wave holds, for k-step s (32 k), the packed int32 row
// r = s*4 + (l >> 4) at columns c0 + 2*(l & 15) and c0 + 2*(l & 15) + 1 (one 8-byte load; 16
// lanes read 128 contiguous bytes of a row). One packed int32 is exactly the 8 k-values one lane
// contributes to a 16x16x32 MFMA, so each int32 becomes one B fragment: the bf16 "magic" pairs
// (128 + q_j, 128 + q_{j+4}) give the k order [0,4,1,5,2,6,3,7]; the A fragment (activations)
// is loaded as 8 consecutive bf16 and permuted to the same order (v_perm), so the dot products
// are unchanged. The two MFMA N-subtiles of a lane are its two columns.
//
// Zero point and scale are applied per quantisation group g on fp32 partial sums:
//   y[m, n] = sum_g s[g, n] * ( sum_{k in g} x[m, k] (128 + q[k, n]) - (128 + z[g, n]) X[m, g] )
// with X[m, g] = sum_{k in g} x[m, k] produced by one extra MFMA against an all-ones B.
// All weight products are exact; the only difference from the reference's dequantise-then-
// matmul is that the reference rounds each (q - z) * s to bf16 first.
//
// W1 (gate_up): A = x[token(slot)], both gate and up tiles, epilogue h = bf16(silu(g) * u).
// W2 (down):    A = h[slot],       epilogue ys[slot, n] = w[slot] * y (fp32).
// Arithmetic references: src/mtp_expert_prefetch/tracing/vllm_wna16_group_plan.py:367-486,
// src/mtp_expert_prefetch/repack/gptq_unpack.py:88-131, 247-256.
#include "common.h"
#include "launch.h"

namespace {

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));

constexpr int kBM = kDecodeBlockM;  // 16 slots
constexpr int kKW = 256;            // k per wave
constexpr int kSteps = kKW / 32;    // MFMA k-steps per wave
constexpr int kMaxWaves = 8;        // K <= 2048
constexpr uint32_t kOnes = 0x3F803F80u;

enum { DEC_W1 = 1, DEC_W2 = 2 };

MOE_DEV bf16x8_v as_frag(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u32x4 v = {a, b, c, d};
  return __builtin_bit_cast(bf16x8_v, v);
}

// B fragment of one packed int32 (8 k of one column): pairs (q0,q4),(q1,q5),(q2,q6),(q3,q7).
MOE_DEV bf16x8_v weight_frag(uint32_t w) {
  return as_frag(magic_pair(w, 0), magic_pair(w, 1), magic_pair(w, 2), magic_pair(w, 3));
}

// SPG = MFMA k-steps per quantisation group (G / 32); NGW = groups per wave.
template <int MODE, int SPG>
__global__ __launch_bounds__(512) void gemm_decode_kernel(
    const uint16_t* __restrict__ act, ExpertsDev ed, SlotsDev sd,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ eids,
    const int32_t* __restrict__ ntpp, const float* __restrict__ topk_w,
    uint16_t* __restrict__ h_out, float* __restrict__ ys) {
  constexpr int NP = (MODE == DEC_W1) ? 2 : 1;  // projections (gate, up) or (down)
  constexpr int NT = 2 * NP;                     // MFMA N-subtiles per lane
  __shared__ float red[(kMaxWaves - 1) * NT * 4 * 64];
  __shared__ int s_slot[kBM];

  const int b = blockIdx.y;
  if (b * kBM >= *ntpp) return;
  const int e = eids[b];
  if (!expert_ok(ed, e)) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int G = ed.group;
  const int K = (MODE == DEC_W1) ? ed.hidden : ed.inter;
  const int NOUT = (MODE == DEC_W1) ? ed.inter : ed.hidden;
  const int c0 = blockIdx.x * 32;
  const bool is_shared = (e == ed.num_experts);
  const int64_t row = is_shared ? 0 : expert_row(ed, e);
  ProjDev pj[NP];
  if (MODE == DEC_W1) {
    pj[0] = is_shared ? ed.sgate : ed.gate;
    pj[NP - 1] = is_shared ? ed.sup : ed.up;
  } else {
    pj[0] = is_shared ? ed.sdown : ed.down;
  }
  if (tid < kBM) s_slot[tid] = sorted[b * kBM + tid];
  __syncthreads();

  // ---- issue every global load of this wave up front
  const int kw0 = wave * kKW;  // first k of this wave
  const int m = lane & 15, kq = lane >> 4;
  const int f_m = s_slot[m];
  const bool valid_m = (unsigned)f_m < (unsigned)sd.num_slots;
  const int64_t arow = valid_m ? ((MODE == DEC_W1) ? (int64_t)slot_token(sd, f_m) : (int64_t)f_m) : 0;
  const uint16_t* ap = act + arow * K + kw0 + 8 * kq;
  u32x4 av[kSteps];
#pragma unroll
  for (int s = 0; s < kSteps; ++s)
    av[s] = valid_m ? ld128(ap + 32 * s) : u32x4{0u, 0u, 0u, 0u};

  const int K8 = K / 8, NG = K / G;
#pragma unroll
  for (int p = 0; p < NP; ++p) pj[p] = proj_row(pj[p], is_shared ? 0 : ed.row_stride, row, K8, NG, NOUT);
  const int cl = c0 + 2 * (lane & 15);  // this lane's first column
  u32x2 bv[NP][kSteps];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int32_t* q = pj[p].qweight + (int64_t)(kw0 / 8 + kq) * NOUT + cl;
#pragma unroll
    for (int s = 0; s < kSteps; ++s)
      bv[p][s] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(q + (int64_t)(4 * s) * NOUT));
  }
  // scales / zeros of this lane's two columns for the wave's NGW groups
  constexpr int NGW = kSteps / SPG;
  float sc[NP][NGW][2], zb[NP][NGW][2];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int gi = 0; gi < NGW; ++gi) {
      {
        const int g = kw0 / G + gi;
        const uint32_t s2 = *reinterpret_cast<const uint32_t*>(pj[p].scales + (int64_t)g * NOUT + cl);
        const uint32_t zw = (uint32_t)pj[p].qzeros[(int64_t)g * (NOUT / 8) + (cl >> 3)] >> (4 * (cl & 7));
        sc[p][gi][0] = f16_to_f32(s2 & 0xFFFFu);
        sc[p][gi][1] = f16_to_f32(s2 >> 16);
        zb[p][gi][0] = kMagicBias + (float)(zw & 0xFu);
        zb[p][gi][1] = kMagicBias + (float)((zw >> 4) & 0xFu);
      }
    }

  // ---- MFMA over the wave's k-slice, one quantisation group at a time
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const bf16x8_v ones = as_frag(kOnes, kOnes, kOnes, kOnes);
#pragma unroll
  for (int gi = 0; gi < NGW; ++gi) {
    f32x4 tmp[NT], tx = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < NT; ++t) tmp[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ss = gi * SPG; ss < (gi + 1) * SPG; ++ss) {
      uint32_t xp[4];
      xpairs(av[ss], xp);
      const bf16x8_v a = as_frag(xp[0], xp[1], xp[2], xp[3]);
      tx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ones, tx, 0, 0, 0);
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          tmp[2 * p + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, weight_frag(bv[p][ss][j]),
                                                                   tmp[2 * p + j], 0, 0, 0);
    }
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[2 * p + j][i] = __builtin_fmaf(sc[p][gi][j],
                                             __builtin_fmaf(-zb[p][gi][j], tx[i], tmp[2 * p + j][i]),
                                             acc[2 * p + j][i]);
  }

  // ---- cross-wave reduction (waves 1.. write, wave 0 sums in order)
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(((wave - 1) * NT + t) * 4 + i) * 64 + lane] = acc[t][i];
  }
  __syncthreads();
  if (wave != 0) return;
  for (int w = 1; w < nwaves; ++w)
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t][i] += red[(((w - 1) * NT + t) * 4 + i) * 64 + lane];

  // D[i][j] of a 16x16 tile: lane j + 16*(i/4), element i%4 -> row 4*(lane>>4)+el, column of
  // N-subtile t = cl + (t & 1).
#pragma unroll
  for (int el = 0; el < 4; ++el) {
    const int r = 4 * (lane >> 4) + el;
    const int f = s_slot[r];
    if ((unsigned)f >= (unsigned)sd.num_slots) continue;
    if (MODE == DEC_W1) {
      const float h0 = silu_f32(acc[0][el]) * acc[2][el];
      const float h1 = silu_f32(acc[1][el]) * acc[3][el];
      *reinterpret_cast<uint32_t*>(h_out + (int64_t)f * NOUT + cl) = pack_bf16x2(h0, h1);
    } else {
      const float w = topk_w[f];
      const float2 v = {w * acc[0][el], w * acc[1][el]};
      *reinterpret_cast<float2*>(ys + (int64_t)f * NOUT + cl) = v;
    }
  }
}

}  // namespace

namespace {
template <int MODE>
hipError_t launch_decode(const uint16_t* act, const ExpertsDev& ed, const SlotsDev& sd,
                         const int32_t* sorted, const int32_t* eids, const int32_t* ntpp, int cap,
                         const float* topk_w, uint16_t* h, float* ys, hipStream_t stream) {
  const int K = (MODE == DEC_W1) ? ed.hidden : ed.inter;
  const int NOUT = (MODE == DEC_W1) ? ed.inter : ed.hidden;
  if (K % kKW != 0 || K / kKW > kMaxWaves || NOUT % 32 != 0) return hipErrorInvalidValue;
  const dim3 grid(NOUT / 32, cap);
  const dim3 block(64 * (K / kKW));
  switch (ed.group) {
    case 64:
      hipLaunchKernelGGL((gemm_decode_kernel<MODE, 2>), grid, block, 0, stream, act, ed, sd,
                         sorted, eids, ntpp, topk_w, h, ys);
      break;
    case 128:
      hipLaunchKernelGGL((gemm_decode_kernel<MODE, 4>), grid, block, 0, stream, act, ed, sd,
                         sorted, eids, ntpp, topk_w, h, ys);
      break;
    case 256:
      hipLaunchKernelGGL((gemm_decode_kernel<MODE, 8>), grid, block, 0, stream, act, ed, sd,
                         sorted, eids, ntpp, topk_w, h, ys);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
}  // namespace

hipError_t launch_w1_decode_mfma(const uint16_t* x, const ExpertsDev& ed, const SlotsDev& sd,
                                 const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                                 int cap, uint16_t* h, hipStream_t stream) {
  return launch_decode<DEC_W1>(x, ed, sd, sorted, eids, ntpp, cap, nullptr, h, nullptr, stream);
}

hipError_t launch_w2_decode_mfma(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                                 const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                                 int cap, const float* topk_w, float* ys, hipStream_t stream) {
  return launch_decode<DEC_W2>(h, ed, sd, sorted, eids, ntpp, cap, topk_w, nullptr, ys, stream);
}
