// Decode path: grouped int4 GEMV for W1 (gate_up + SiLU*mul) and W2 (down * routed weight),
// and the fixed-order top-k sum. HBM-bound: every packed int32 of an expert's weights is
// read once per block with 128-bit coalesced loads and dequantised in registers.
//
// Arithmetic (src/mtp_expert_prefetch/tracing/vllm_wna16_group_plan.py:367-486 and
// src/mtp_expert_prefetch/repack/gptq_unpack.py:88-131, 247-256):
//   y[n] = sum_k x[k] * (q[k,n] - z[g,n]) * s[g,n]
// is evaluated per lane over a k-range inside one quantisation group g as
//   s[g,n] * ( sum_k x[k]*(128 + q[k,n])  -  (128 + z[g,n]) * sum_k x[k] ),
// where (128 + q) is built as an exact bf16 by OR-ing the nibble into the mantissa of 128.0
// (one v_and_or per two weights) and the sums run on v_dot2_f32_bf16. All products are exact;
// the result differs from the reference's bf16-rounded dequantised weight only by that
// reference rounding (<= 2^-9 relative per weight).
//
// Thread layout of a block (one expert block of BM slots x one 32-column tile):
//   cq = tid & 7       -> columns c .. c+3 (one 128-bit load of 4 packed int32)
//   ks = tid >> 3      -> packed rows ks*RPK .. ks*RPK+RPK-1 (8*RPK consecutive k, inside one group)
// so blockDim = K / RPK. A wave load instruction reads 8 rows x 128 contiguous bytes. Partials
// over ks are reduced with xor-shuffles (lane bits 3..5) and then across waves through LDS,
// always in the same order, so results are deterministic.
#include "common.h"
#include "launch.h"

namespace {

constexpr uint32_t kOnePair = 0x3F803F80u;  // bf16 (1.0, 1.0)
constexpr int kRPK = 4;                     // packed rows (8*kRPK k) per lane
constexpr int kMaxWaves = 8;                // K <= 2048 -> blockDim <= 512

enum { GEMV_W1 = 1, GEMV_W2 = 2 };

MOE_DEV int block_valid_run(const int32_t* __restrict__ sorted, int base, int m, int BM,
                            int num_slots, int maxn) {
  int n = 0;
  for (int j = 0; j < maxn && m + j < BM; ++j) {
    if (sorted[base + m + j] >= num_slots) break;
    ++n;
  }
  return n;
}

// Weights, scales and zeros of one lane: NP projections (W1: gate, up; W2: down).
template <int NP>
struct LaneTile {
  u32x4 w[NP][kRPK];
  float s[NP][4], z[NP][4];
};

template <int MODE, int NT>
MOE_DEV void gemv_tokens(const uint16_t* __restrict__ act, int K, int NOUT, const int (&f)[NT],
                         const int (&arow)[NT], const LaneTile<(MODE == GEMV_W1 ? 2 : 1)>& lt,
                         int tid, int nwaves, int col0, float (*red)[8][8][1],
                         const float* __restrict__ topk_w, uint16_t* __restrict__ h,
                         float* __restrict__ ys) {
  constexpr int NP = (MODE == GEMV_W1) ? 2 : 1;
  const int lane = tid & 63, wave = tid >> 6, cq = tid & 7, ks = tid >> 3;
  float acc[NT][NP][4], xs[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    xs[j] = 0.0f;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[j][p][q] = 0.0f;
  }
#pragma unroll
  for (int r = 0; r < kRPK; ++r) {
    const int k0 = (ks * kRPK + r) * 8;
    uint32_t xp[NT][4];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const u32x4 d = ld128(act + (int64_t)arow[j] * K + k0);
      xpairs(d, xp[j]);
      xs[j] = dot2_bf16(xp[j][0], kOnePair, xs[j]);
      xs[j] = dot2_bf16(xp[j][1], kOnePair, xs[j]);
      xs[j] = dot2_bf16(xp[j][2], kOnePair, xs[j]);
      xs[j] = dot2_bf16(xp[j][3], kOnePair, xs[j]);
    }
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t wq = lt.w[p][r][q];
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {
          const uint32_t mq = magic_pair(wq, pr);
#pragma unroll
          for (int j = 0; j < NT; ++j) acc[j][p][q] = dot2_bf16(mq, xp[j][pr], acc[j][p][q]);
        }
      }
  }
  // lane partial: s * (sum x*(128+q) - (128+z) * sum x), then reduce over ks inside the wave
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float t = lt.s[p][q] * (acc[j][p][q] - lt.z[p][q] * xs[j]);
        t = wave_xor_sum(t, 8);
        t = wave_xor_sum(t, 16);
        t = wave_xor_sum(t, 32);
        acc[j][p][q] = t;
      }
  if ((lane >> 3) == 0) {
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int q = 0; q < 4; ++q) red[wave * 4 + j][cq][p * 4 + q][0] = acc[j][p][q];
  }
  __syncthreads();
  if (tid < NT * 8) {
    const int j = tid >> 3, q8 = tid & 7;
    float v[NP][4];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int q = 0; q < 4; ++q) v[p][q] = 0.0f;
    for (int w = 0; w < nwaves; ++w)
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int q = 0; q < 4; ++q) v[p][q] += red[w * 4 + j][q8][p * 4 + q][0];
    int fj = f[0];
#pragma unroll
    for (int jj = 1; jj < NT; ++jj)
      if (j == jj) fj = f[jj];
    const int c = col0 + q8 * 4;
    if (MODE == GEMV_W1) {
      u32x2 o;
      o[0] = pack_bf16x2(silu_f32(v[0][0]) * v[NP - 1][0], silu_f32(v[0][1]) * v[NP - 1][1]);
      o[1] = pack_bf16x2(silu_f32(v[0][2]) * v[NP - 1][2], silu_f32(v[0][3]) * v[NP - 1][3]);
      *reinterpret_cast<u32x2*>(h + (int64_t)fj * NOUT + c) = o;
    } else {
      const float w = topk_w[fj];
      f32x4 o = {v[0][0] * w, v[0][1] * w, v[0][2] * w, v[0][3] * w};
      *reinterpret_cast<f32x4*>(ys + (int64_t)fj * NOUT + c) = o;
    }
  }
  __syncthreads();
}

// W1 (MODE_W1): act = x [T, H], K = H, NOUT = I, out h bf16 [slots, I] = silu(gate) * up.
// W2 (MODE_W2): act = h [slots, I], K = I, NOUT = H, out ys fp32 [slots, H] = w * down.
template <int MODE>
__global__ __launch_bounds__(512) void gemv_decode_kernel(const uint16_t* __restrict__ act,
                                                          ExpertsDev ed, SlotsDev sd,
                                                          const int32_t* __restrict__ sorted,
                                                          const int32_t* __restrict__ eids,
                                                          const int32_t* __restrict__ ntpp,
                                                          int BM, const float* __restrict__ topk_w,
                                                          uint16_t* __restrict__ h,
                                                          float* __restrict__ ys) {
  constexpr int NP = (MODE == GEMV_W1) ? 2 : 1;
  // red[wave*4 + token][cq][value][0]; the trailing dimension keeps the declared shape simple.
  __shared__ float red[kMaxWaves * 4][8][8][1];
  const int b = blockIdx.y;
  if (b * BM >= *ntpp) return;
  const int e = eids[b];
  if (!expert_ok(ed, e)) return;
  const int G = ed.group;
  const int K = (MODE == GEMV_W1) ? ed.hidden : ed.inter;
  const int NOUT = (MODE == GEMV_W1) ? ed.inter : ed.hidden;
  const int tid = threadIdx.x, ks = tid >> 3, cq = tid & 7;
  const int nwaves = blockDim.x >> 6;
  const int col0 = blockIdx.x * 32;
  const int c = col0 + cq * 4;
  const bool is_shared = (e == ed.num_experts);
  ProjDev pj[NP];
  if (MODE == GEMV_W1) {
    pj[0] = is_shared ? ed.sgate : ed.gate;
    pj[NP - 1] = is_shared ? ed.sup : ed.up;
  } else {
    pj[0] = is_shared ? ed.sdown : ed.down;
  }
  const int64_t row = is_shared ? 0 : expert_row(ed, e);
  const int K8 = K / 8, NG = K / G;
  const int g = (ks * kRPK * 8) / G;

  LaneTile<NP> lt;
#pragma unroll
  for (int p = 0; p < NP; ++p) pj[p] = proj_row(pj[p], is_shared ? 0 : ed.row_stride, row, K8, NG, NOUT);
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int32_t* wq = pj[p].qweight + (int64_t)(ks * kRPK) * NOUT + c;
#pragma unroll
    for (int r = 0; r < kRPK; ++r) lt.w[p][r] = ld128_nt(wq + (int64_t)r * NOUT);
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const u32x2 s2 = *reinterpret_cast<const u32x2*>(pj[p].scales + (int64_t)g * NOUT + c);
    const uint32_t zw = (uint32_t)pj[p].qzeros[(int64_t)g * (NOUT / 8) + (c >> 3)];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      lt.s[p][q] = f16_to_f32((s2[q >> 1] >> (16 * (q & 1))) & 0xFFFFu);
      lt.z[p][q] = kMagicBias + (float)((zw >> (4 * ((c & 7) + q))) & 0xFu);
    }
  }
  const int base = b * BM;
  int m = 0;
  while (m < BM) {
    const int n = block_valid_run(sorted, base, m, BM, sd.num_slots, 2);
    if (n == 0) break;
    if (n == 2) {
      int f[2], ar[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        f[j] = sorted[base + m + j];
        ar[j] = (MODE == GEMV_W1) ? slot_token(sd, f[j]) : f[j];
      }
      gemv_tokens<MODE, 2>(act, K, NOUT, f, ar, lt, tid, nwaves, col0, red, topk_w, h, ys);
      m += 2;
    } else {
      int f[1], ar[1];
      f[0] = sorted[base + m];
      ar[0] = (MODE == GEMV_W1) ? slot_token(sd, f[0]) : f[0];
      gemv_tokens<MODE, 1>(act, K, NOUT, f, ar, lt, tid, nwaves, col0, red, topk_w, h, ys);
      m += 1;
    }
  }
}

// ------------------------------------------------------------------------------- moe_sum
// out[t] = bf16(sum over the token's slots in order of ys[slot]) with fp32 sums; ys rows are
// fp32 (YT = float) or bf16 (YT = uint16_t). With `ids`, routed slots whose expert is dropped
// (routed_ok false: their ys rows were never written) are skipped.
// Each thread sums 16 bytes of columns (4 fp32 or 8 bf16). Slots are taken TK at a time: all
// loads of a chunk are issued together (a skipped slot or one past top_k reads zeros without a
// memory access, and +0 leaves the running sum unchanged), so a chunk waits for three memory
// latencies (ids, expert_row, ys) instead of one per slot. With UNIFORM (a token's columns
// cover whole waves) the token index is wave-uniform and its ids and expert rows are scalar
// loads, leaving the vector memory pipeline to the slot rows.
template <typename YT>
struct SumVec {
  static constexpr int N = 16 / sizeof(YT);  // columns per thread
  float v[N];
};

template <typename YT>
MOE_DEV SumVec<YT> ys_vec(__amdgpu_buffer_rsrc_t r, uint32_t elem_off, bool ok) {
  SumVec<YT> o;
  const u32x4 d = buf_ld128(r, ok ? elem_off * (uint32_t)sizeof(YT) : kOutOfRange);
  if constexpr (sizeof(YT) == 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) o.v[j] = __uint_as_float(d[j]);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      o.v[2 * j] = bf16lo_to_f32(d[j]);
      o.v[2 * j + 1] = bf16hi_to_f32(d[j]);
    }
  }
  return o;
}

template <int TK, typename YT, bool UNIFORM>
__global__ __launch_bounds__(256) void moe_sum_kernel(const YT* __restrict__ ys, int T, int top_k,
                                                      int H, int has_shared,
                                                      const int32_t* __restrict__ ids,
                                                      int num_experts,
                                                      const int32_t* __restrict__ expert_row,
                                                      uint16_t* __restrict__ out) {
  constexpr int N = SumVec<YT>::N;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int per_row = H / N;
  int t = (int)(idx / per_row);
  if constexpr (UNIFORM) t = __builtin_amdgcn_readfirstlane(t);
  if (t >= T) return;
  const int c = (int)(idx % per_row) * N;
  const int routed = T * top_k;
  const __amdgpu_buffer_rsrc_t yr = buf_rsrc(
      ys, (uint32_t)(routed + (has_shared ? T : 0)) * (uint32_t)H * (uint32_t)sizeof(YT));
  const __amdgpu_buffer_rsrc_t ir = buf_rsrc(ids, ids ? (uint32_t)routed * 4u : 0u);
  const __amdgpu_buffer_rsrc_t er = buf_rsrc(expert_row, expert_row ? (uint32_t)num_experts * 4u : 0u);
  float s[N];
#pragma unroll
  for (int j = 0; j < N; ++j) s[j] = 0.f;
  for (int i0 = 0; i0 < top_k; i0 += TK) {
    bool ok[TK];
#pragma unroll
    for (int i = 0; i < TK; ++i) ok[i] = i0 + i < top_k;
    if (ids) {
      int e[TK];
      if constexpr (UNIFORM) {  // wave-uniform: scalar loads
#pragma unroll
        for (int i = 0; i < TK; ++i) e[i] = ok[i] ? ids[t * top_k + i0 + i] : -1;
      } else {
#pragma unroll
        for (int i = 0; i < TK; ++i)
          e[i] = (int)buf_ld32(ir, ok[i] ? (uint32_t)(t * top_k + i0 + i) * 4u : kOutOfRange);
      }
#pragma unroll
      for (int i = 0; i < TK; ++i) ok[i] = ok[i] && e[i] >= 0 && e[i] < num_experts;
      if (expert_row) {
        int r[TK];
        if constexpr (UNIFORM) {
#pragma unroll
          for (int i = 0; i < TK; ++i) r[i] = ok[i] ? expert_row[e[i]] : -1;
        } else {
#pragma unroll
          for (int i = 0; i < TK; ++i)
            r[i] = (int)buf_ld32(er, ok[i] ? (uint32_t)e[i] * 4u : kOutOfRange);
        }
#pragma unroll
        for (int i = 0; i < TK; ++i) ok[i] = ok[i] && r[i] >= 0;
      }
    }
    SumVec<YT> v[TK];
#pragma unroll
    for (int i = 0; i < TK; ++i)
      v[i] = ys_vec<YT>(yr, (uint32_t)(t * top_k + i0 + i) * (uint32_t)H + (uint32_t)c, ok[i]);
#pragma unroll
    for (int i = 0; i < TK; ++i)
#pragma unroll
      for (int j = 0; j < N; ++j) s[j] += v[i].v[j];
  }
  if (has_shared) {
    const SumVec<YT> v = ys_vec<YT>(yr, (uint32_t)(routed + t) * (uint32_t)H + (uint32_t)c, true);
#pragma unroll
    for (int j = 0; j < N; ++j) s[j] += v.v[j];
  }
  if constexpr (N == 4) {
    *reinterpret_cast<u32x2*>(out + (int64_t)t * H + c) =
        u32x2{pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3])};
  } else {
    *reinterpret_cast<u32x4*>(out + (int64_t)t * H + c) =
        u32x4{pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3]), pack_bf16x2(s[4], s[5]),
              pack_bf16x2(s[6], s[7])};
  }
}

template <typename YT, bool UNIFORM>
hipError_t launch_moe_sum_u(const YT* ys, int T, int top_k, int H, int has_shared,
                            const int32_t* ids, int num_experts, const int32_t* expert_row,
                            uint16_t* out, hipStream_t stream) {
  const int64_t n = (int64_t)T * (H / SumVec<YT>::N);
  const dim3 grid((unsigned)((n + 255) / 256));
#define MOE_SUM_CASE(TKV)                                                                      \
  if (top_k <= TKV) {                                                                          \
    hipLaunchKernelGGL((moe_sum_kernel<TKV, YT, UNIFORM>), grid, dim3(256), 0, stream, ys, T,   \
                       top_k, H, has_shared, ids, num_experts, expert_row, out);               \
    return hipGetLastError();                                                                  \
  }
  MOE_SUM_CASE(1) MOE_SUM_CASE(2) MOE_SUM_CASE(4) MOE_SUM_CASE(8)
#undef MOE_SUM_CASE
  hipLaunchKernelGGL((moe_sum_kernel<16, YT, UNIFORM>), grid, dim3(256), 0, stream, ys, T, top_k,
                     H, has_shared, ids, num_experts, expert_row, out);
  return hipGetLastError();
}

template <typename YT>
hipError_t launch_moe_sum_t(const YT* ys, int T, int top_k, int H, int has_shared,
                            const int32_t* ids, int num_experts, const int32_t* expert_row,
                            uint16_t* out, hipStream_t stream) {
  constexpr int N = SumVec<YT>::N;
  if ((int64_t)T * H == 0) return hipSuccess;
  if (H % N != 0) return hipErrorInvalidValue;
  if ((int64_t)(T * top_k + T) * H * (int64_t)sizeof(YT) >= kOutOfRange) return hipErrorInvalidValue;
  if ((H / N) % 64 == 0)  // a token's columns cover whole waves
    return launch_moe_sum_u<YT, true>(ys, T, top_k, H, has_shared, ids, num_experts, expert_row,
                                      out, stream);
  return launch_moe_sum_u<YT, false>(ys, T, top_k, H, has_shared, ids, num_experts, expert_row,
                                     out, stream);
}

}  // namespace

hipError_t launch_w1_decode(const uint16_t* x, const ExpertsDev& ed, const SlotsDev& sd,
                            const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                            int BM, int cap, uint16_t* h, hipStream_t stream) {
  // blockDim = 8 column-quads x H / (8 kRPK) k-subsets; one 32-column tile per block.
  const dim3 grid(ed.inter / 32, cap);
  const dim3 block(ed.hidden / kRPK);
  hipLaunchKernelGGL(gemv_decode_kernel<GEMV_W1>, grid, block, 0, stream, x, ed, sd, sorted, eids,
                     ntpp, BM, (const float*)nullptr, h, (float*)nullptr);
  return hipGetLastError();
}

hipError_t launch_w2_decode(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                            const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                            int BM, int cap, const float* topk_w, float* ys, hipStream_t stream) {
  const dim3 grid(ed.hidden / 32, cap);
  const dim3 block(ed.inter / kRPK);
  hipLaunchKernelGGL(gemv_decode_kernel<GEMV_W2>, grid, block, 0, stream, h, ed, sd, sorted, eids,
                     ntpp, BM, topk_w, (uint16_t*)nullptr, ys);
  return hipGetLastError();
}

hipError_t launch_moe_sum(const float* ys, int T, int top_k, int H, int has_shared,
                          const int32_t* ids, int num_experts, const int32_t* expert_row,
                          uint16_t* out, hipStream_t stream) {
  return launch_moe_sum_t<float>(ys, T, top_k, H, has_shared, ids, num_experts, expert_row, out,
                                 stream);
}

hipError_t launch_moe_sum_bf16(const uint16_t* ys, int T, int top_k, int H, int has_shared,
                               const int32_t* ids, int num_experts, const int32_t* expert_row,
                               uint16_t* out, hipStream_t stream) {
  return launch_moe_sum_t<uint16_t>(ys, T, top_k, H, has_shared, ids, num_experts, expert_row,
                                    out, stream);
}
