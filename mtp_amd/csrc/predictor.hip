// Expert-demand predictor: per layer head l, a bf16 MLP  hidden -> D (SiLU) -> E logits, then
// the top-k experts of every (head, token).
//
// The reference's predictor (src/mtp_expert_prefetch/training/hidden_residual.py:44-106,
// Linear -> SiLU -> ... -> Linear(w, E), one prediction per layer) is simplified, as the offload
// workload specifies, to a two-layer bf16 MLP per layer with random weights whose top-16 experts
// drive the prefetch of that layer. All heads run in four launches: the first products of every
// head as one [T, L*D] GEMV (w1 heads are contiguous rows), SiLU into a head-major activation,
// the second products with the head on grid.y, and one wave per (head, token) for the top-k.
// Both products use the canonical fp32 dot order of the router (routing.h:logits_tile); the
// hidden activation is SiLU in fp32 rounded once to bf16 (the bf16 Linear output dtype).
#include "launch.h"
#include "routing.h"

namespace {

// out[head][t][n] (row stride N + 1) = x[head][t][:] . W[head][n][:], head = blockIdx.y.
template <int TT, int TE>
__global__ __launch_bounds__(256) void mlp_logits_kernel(
    const uint16_t* __restrict__ x, int64_t x_head, int T, int K, const uint16_t* __restrict__ W,
    int64_t w_head, int N, float* __restrict__ out, int64_t out_head) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tiles_n = (N + TE - 1) / TE;
  const int t0 = (wave / tiles_n) * TT;
  const int n0 = (wave % tiles_n) * TE;
  if (t0 >= T) return;
  const int64_t head = blockIdx.y;
  logits_tile<TT, TE>(x + head * x_head, T, K, W + head * w_head, N, nullptr, nullptr,
                      out + head * out_head, t0, n0, lane);
}

// a[l][t][j] = bf16(silu(z[t][l * D + j])), z with row stride L * D + 1.
__global__ void silu_bf16_kernel(const float* __restrict__ z, int T, int L, int D,
                                 uint16_t* __restrict__ a) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_head = (int64_t)T * D;
  if (i >= per_head * L) return;
  const int64_t l = i / per_head, r = i % per_head;
  const int64_t t = r / D, j = r % D;
  const float v = z[t * ((int64_t)L * D + 1) + l * D + j];
  a[i] = (uint16_t)f32_to_bf16_rne(v / (1.0f + expf(-v)));
}

// One wave per (head, token): logits row (head * T + t) of z2, ids/scores [head][t][top_k].
__global__ __launch_bounds__(256) void predictor_topk_kernel(const float* __restrict__ logits,
                                                             int T, int L, int E, int top_k,
                                                             int32_t* __restrict__ ids,
                                                             float* __restrict__ scores) {
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (w >= T * L) return;
  const int l = w / T, t = w % T;
  const int64_t head_off = (int64_t)l * T * top_k;
  topk_token_any(logits + (int64_t)w * (E + 1), E, top_k, 0, T, t, lane, ids + head_off,
             scores + head_off, nullptr);
}

template <int TT, int TE>
hipError_t launch_mlp_logits(const uint16_t* x, int64_t x_head, int T, int K, const uint16_t* W,
                             int64_t w_head, int N, float* out, int64_t out_head, int heads,
                             hipStream_t stream) {
  const int64_t tiles = (int64_t)((T + TT - 1) / TT) * ((N + TE - 1) / TE);
  hipLaunchKernelGGL((mlp_logits_kernel<TT, TE>), dim3((unsigned)((tiles + 3) / 4), heads),
                     dim3(256), 0, stream, x, x_head, T, K, W, w_head, N, out, out_head);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_predictor(const uint16_t* h, int T, int H, int L, const uint16_t* w1, int D,
                            const uint16_t* w2, int E, int top_k, float* z1, uint16_t* a,
                            float* z2, int32_t* ids, float* scores, hipStream_t stream) {
  const int LD = L * D;
  hipError_t err = launch_mlp_logits<1, 2>(h, 0, T, H, w1, 0, LD, z1, 0, 1, stream);
  if (err != hipSuccess) return err;
  const int64_t n = (int64_t)T * LD;
  hipLaunchKernelGGL(silu_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, z1,
                     T, L, D, a);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  err = launch_mlp_logits<1, 2>(a, (int64_t)T * D, T, D, w2, (int64_t)E * D, E, z2,
                                (int64_t)T * (E + 1), L, stream);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(predictor_topk_kernel, dim3((T * L + 3) / 4), dim3(256), 0, stream, z2, T, L,
                     E, top_k, ids, scores);
  return hipGetLastError();
}
