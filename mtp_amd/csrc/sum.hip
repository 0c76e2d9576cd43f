// The fixed-order top-k sum of the weighted expert rows of each token (vLLM's moe_sum, which
// the reference's fused-MoE call ends with: src/mtp_expert_prefetch/tracing/vllm_router_trace.py:
// 19761-19804). HBM-bound: every slot row is read once with 16-byte loads.
#include "common.h"
#include "launch.h"

namespace {

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

// Sum of the fused W1+W2 partial rows (gemm_decode_kernel FW2): out[t][n] = bf16 of the fp32
// sum over the token's contributing slots (routed t*top_k .. t*top_k + top_k - 1, then the
// shared slot T*top_k + t) and over the nct column tiles c of part[slot][c][n], in that
// (slot, c) order split into 16 consecutive runs whose sums are added in run order. A block
// covers 64 columns of one token: thread (run = tid >> 4, column quad tid & 15). Every partial
// row is written (zeros for a dropped expert), so no ids are read.
constexpr int kPartialRuns = 16;
constexpr int kPartialMaxPerRun = 16;  // slots x column tiles <= 256
__global__ __launch_bounds__(256) void partial_sum_kernel(
    const float* __restrict__ part, int T, int top_k, int H, int nct, int has_shared,
    uint16_t* __restrict__ out) {
  __shared__ float4 s_run[kPartialRuns][16];
  const int t = blockIdx.y, tid = threadIdx.x, cq = tid & 15, run = tid >> 4;
  const int n = blockIdx.x * 64 + 4 * cq;
  const int S = top_k + has_shared, npair = S * nct;
  const int per = (npair + kPartialRuns - 1) / kPartialRuns;
  const int routed = T * top_k, n_slots = routed + (has_shared ? T : 0);
  const __amdgpu_buffer_rsrc_t pr =
      buf_rsrc(part, (uint32_t)n_slots * (uint32_t)nct * (uint32_t)H * 4u);
  u32x4 v[kPartialMaxPerRun];
#pragma unroll
  for (int q = 0; q < kPartialMaxPerRun; ++q) {
    const int p = run * per + q;
    const bool in = q < per && p < npair;
    const int si = in ? p / nct : 0, c = in ? p - si * nct : 0;
    const int f = si < top_k ? t * top_k + si : routed + t;
    v[q] = buf_ld128(pr, in ? (((uint32_t)f * (uint32_t)nct + (uint32_t)c) * (uint32_t)H +
                               (uint32_t)n) * 4u
                            : kOutOfRange);
  }
  float4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < kPartialMaxPerRun; ++q) {
    acc.x += __uint_as_float(v[q][0]);
    acc.y += __uint_as_float(v[q][1]);
    acc.z += __uint_as_float(v[q][2]);
    acc.w += __uint_as_float(v[q][3]);
  }
  s_run[run][cq] = acc;
  __syncthreads();
  if (run != 0) return;
#pragma unroll
  for (int r = 1; r < kPartialRuns; ++r) {
    const float4 o = s_run[r][cq];
    acc.x += o.x;
    acc.y += o.y;
    acc.z += o.z;
    acc.w += o.w;
  }
  *reinterpret_cast<u32x2*>(out + (int64_t)t * H + n) =
      u32x2{pack_bf16x2(acc.x, acc.y), pack_bf16x2(acc.z, acc.w)};
}

}  // namespace

bool partial_sum_fits(int top_k, int has_shared, int H, int nct) {
  return H % 64 == 0 && (top_k + has_shared) * nct <= kPartialRuns * kPartialMaxPerRun;
}

hipError_t launch_partial_sum(const float* part, int T, int top_k, int H, int nct, int has_shared,
                              uint16_t* out, hipStream_t stream) {
  if (!partial_sum_fits(top_k, has_shared, H, nct)) return hipErrorInvalidValue;
  if (T == 0) return hipSuccess;
  hipLaunchKernelGGL(partial_sum_kernel, dim3(H / 64, T), dim3(256), 0, stream, part, T, top_k, H,
                     nct, has_shared, out);
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
