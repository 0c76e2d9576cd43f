// Forward of the reference's HiddenResidualExpertPredictor
// (src/mtp_expert_prefetch/training/hidden_residual.py:44-106) in bf16, plus the residual
// combination logits = prior + scale * residual (train_hidden_residual_predictor_smoke.py:446)
// and the top-k experts of every (example, future delta):
//
//   z  = bf16(x . W_enc^T + b_enc)                    encoder Linear (canonical fp32 dot)
//   a  = bf16(silu(z))                                SiLU
//   s  = bf16(LayerNorm(a) * ln_w + ln_b)             LayerNorm over the width (fp32 statistics)
//   c_d = bf16(bf16(s + E_layer[layer]) + E_delta[d]) context per future delta d
//   g_d = bf16(silu(c_d))
//   r_d = g_d . W_cls^T + b_cls                       classifier (canonical fp32 dot), fp32
//   out_d = prior_d + scale * r_d                     (prior optional), top-k by (value, id)
//
// Every Linear input is bf16 (the dtype of a bf16 model's activations), so the dot products
// of the canonical order (routing.h:logits_tile) are exact per product and reproducible on the
// CPU. Launches: the encoder GEMV (router_logits), one workgroup per example for
// SiLU/LayerNorm/context, the classifier GEMV over the N * future_window context rows, and one
// wave per row for the combination and the top-k.
#include <math.h>
#include <stdio.h>

#include "launch.h"
#include "routing.h"

namespace {

constexpr int kCtxThreads = 256;
constexpr int kCtxMaxPerThread = 4;  // width <= 1024

// Fixed-order sum over the workgroup: per-thread value -> wave butterfly -> waves in order.
MOE_DEV float block_sum(float v, float* red) {
  v = bfly_sum(v);
  const int wv = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wv] = v;
  __syncthreads();
  float s = 0.0f;
  for (int w = 0; w < kCtxThreads / 64; ++w) s += red[w];
  return s;
}

MOE_DEV float bf16_round(float v) { return bf16_to_f32(f32_to_bf16_rne(v)); }

// One workgroup per example n: the encoder output row z[n] (fp32 dot, stride W + 1) -> the
// future_window context rows g[n * F + d] (bf16).
__global__ __launch_bounds__(kCtxThreads) void hr_context_kernel(
    const float* __restrict__ z, int N, int W, const float* __restrict__ enc_b,
    const uint16_t* __restrict__ ln_w, const uint16_t* __restrict__ ln_b, float ln_eps,
    const int32_t* __restrict__ layer_ids, int num_layers, const uint16_t* __restrict__ layer_emb,
    const uint16_t* __restrict__ delta_emb, int F, uint16_t* __restrict__ g) {
  __shared__ float red[kCtxThreads / 64];
  const int n = blockIdx.x;
  const int tid = threadIdx.x;
  float a[kCtxMaxPerThread];
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < kCtxMaxPerThread; ++i) {
    const int j = tid + kCtxThreads * i;
    a[i] = 0.0f;
    if (j < W) {
      const float zb = bf16_round(z[(int64_t)n * (W + 1) + j] + enc_b[j]);
      a[i] = bf16_round(zb / (1.0f + expf(-zb)));
      sum += a[i];
    }
  }
  const float mean = block_sum(sum, red) / (float)W;
  float sq = 0.0f;
#pragma unroll
  for (int i = 0; i < kCtxMaxPerThread; ++i) {
    const int j = tid + kCtxThreads * i;
    if (j < W) {
      const float d = a[i] - mean;
      sq = __builtin_fmaf(d, d, sq);
    }
  }
  const float var = block_sum(sq, red) / (float)W;
  const float rstd = 1.0f / sqrtf(var + ln_eps);
  const int layer = layer_ids[n];
  const bool layer_ok = layer >= 0 && layer < num_layers;  // else the embedding reads zeros
#pragma unroll
  for (int i = 0; i < kCtxMaxPerThread; ++i) {
    const int j = tid + kCtxThreads * i;
    if (j >= W) continue;
    const float s = bf16_round((a[i] - mean) * rstd * bf16_to_f32(ln_w[j]) + bf16_to_f32(ln_b[j]));
    const float le = layer_ok ? bf16_to_f32(layer_emb[(int64_t)layer * W + j]) : 0.0f;
    const float sl = bf16_round(s + le);
    for (int d = 0; d < F; ++d) {
      const float c = bf16_round(sl + bf16_to_f32(delta_emb[(int64_t)d * W + j]));
      g[((int64_t)n * F + d) * W + j] = (uint16_t)f32_to_bf16_rne(c / (1.0f + expf(-c)));
    }
  }
}

// One wave per row r = n * F + d: v = (prior ? prior[r] : 0) + scale_n * logits[r], optionally
// written to out, and the top-k of v by (value, lower id).
template <int MAXC>
__global__ __launch_bounds__(256) void hr_select_kernel(
    const float* __restrict__ logits, int rows, int F, int E, const float* __restrict__ prior,
    float scale, const float* __restrict__ scale_per_example, int top_k,
    float* __restrict__ out, int32_t* __restrict__ ids) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (r >= rows) return;
  const float sc = scale_per_example ? scale_per_example[r / F] : scale;
  const __amdgpu_buffer_rsrc_t lr = buf_rsrc(logits + (int64_t)r * (E + 1), (uint32_t)E * 4u);
  const __amdgpu_buffer_rsrc_t pr = buf_rsrc(prior ? prior + (int64_t)r * E : nullptr,
                                             prior ? (uint32_t)E * 4u : 0u);
  uint32_t key[MAXC];
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int e = lane + 64 * c;
    const float l = __uint_as_float(buf_ld32(lr, (uint32_t)e * 4u));
    const float p = __uint_as_float(buf_ld32(pr, (uint32_t)e * 4u));
    const float v = p + sc * l;
    if (out && e < E) out[(int64_t)r * E + e] = v;
    key[c] = topk_ord(v) & (0u - (uint32_t)(e < E));
  }
  int my_i;
  uint32_t my_key;
  topk_select_keys<MAXC>(key, top_k, lane, my_i, my_key);
  if (lane < top_k) ids[(int64_t)r * top_k + lane] = my_i;
}

}  // namespace

// Workspace sections: z [N][W + 1] fp32, g [N * F][W] bf16, logits [N * F][E + 1] fp32.
int64_t hr_predictor_workspace(int N, int W, int F, int E) {
  auto a256 = [](int64_t v) { return (v + 255) & ~int64_t(255); };
  return a256((int64_t)N * (W + 1) * 4) + a256((int64_t)N * F * W * 2) +
         a256((int64_t)N * F * (E + 1) * 4);
}

hipError_t launch_hr_predictor(const uint16_t* x, int N, int H, const int32_t* layer_ids,
                               const moe_hr_predictor_params_v1& p, const float* prior, float scale,
                               const float* scale_per_example, int top_k, void* workspace,
                               float* out, int32_t* ids, hipStream_t stream) {
  const int W = p.width, F = p.future_window, E = p.num_experts;
  auto a256 = [](int64_t v) { return (v + 255) & ~int64_t(255); };
  char* ws = static_cast<char*>(workspace);
  float* z = reinterpret_cast<float*>(ws);
  uint16_t* g = reinterpret_cast<uint16_t*>(ws + a256((int64_t)N * (W + 1) * 4));
  float* lg = reinterpret_cast<float*>(ws + a256((int64_t)N * (W + 1) * 4) +
                                       a256((int64_t)N * F * W * 2));
  // encoder: z[n, j] = x_n . W_enc[j] (canonical order), row stride W + 1
  hipError_t err = launch_router_logits(x, N, H, p.enc_w, W, nullptr, nullptr, z, stream);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(hr_context_kernel, dim3(N), dim3(kCtxThreads), 0, stream, z, N, W, p.enc_b,
                     p.ln_w, p.ln_b, p.ln_eps, layer_ids, p.num_layers, p.layer_emb, p.delta_emb,
                     F, g);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  // classifier over the N * F context rows, bias added, row stride E + 1
  err = launch_router_logits(g, N * F, W, p.cls_w, E, nullptr, p.cls_b, lg, stream);
  if (err != hipSuccess) return err;
  const int rows = N * F;
  if (E <= 256)
    hipLaunchKernelGGL((hr_select_kernel<4>), dim3((rows + 3) / 4), dim3(256), 0, stream, lg, rows,
                       F, E, prior, scale, scale_per_example, top_k, out, ids);
  else
    hipLaunchKernelGGL((hr_select_kernel<8>), dim3((rows + 3) / 4), dim3(256), 0, stream, lg, rows,
                       F, E, prior, scale, scale_per_example, top_k, out, ids);
  return hipGetLastError();
}

namespace {
int hr_fail(int code, const char* msg) {
  snprintf(moe_error_buffer(), kErrorBufferBytes, "hidden-residual predictor: %s", msg);
  return code;
}

int hr_check(int32_t N, const moe_hr_predictor_params_v1* p, int32_t top_k) {
  if (!p) return hr_fail(MOE_ERR_NULL, "params is NULL");
  if (!p->enc_w || !p->enc_b || !p->ln_w || !p->ln_b || !p->layer_emb || !p->delta_emb ||
      !p->cls_w || !p->cls_b)
    return hr_fail(MOE_ERR_NULL, "a parameter pointer is NULL");
  if (N < 0) return hr_fail(MOE_ERR_SHAPE, "N < 0");
  if (p->hidden <= 0 || p->hidden % 8 != 0) return hr_fail(MOE_ERR_SHAPE, "hidden % 8 != 0");
  if (p->width < 64 || p->width > kCtxThreads * kCtxMaxPerThread || p->width % 8 != 0)
    return hr_fail(MOE_ERR_SHAPE, "width must be a multiple of 8 in [64, 1024]");
  if (p->num_layers < 1 || p->future_window < 1 || p->future_window > 64)
    return hr_fail(MOE_ERR_SHAPE, "num_layers >= 1 and future_window in [1, 64]");
  if (p->num_experts < 1 || p->num_experts > 512 || top_k < 1 || top_k > p->num_experts ||
      top_k > 64)
    return hr_fail(MOE_ERR_SHAPE, "num_experts in [1, 512] and top_k in [1, min(E, 64)]");
  if (!(p->ln_eps >= 0.0f)) return hr_fail(MOE_ERR_SHAPE, "ln_eps must be >= 0");
  // 32-bit buffer offsets of the GEMVs
  const int64_t lim = int64_t(1) << 31;
  if ((int64_t)N * p->hidden * 2 >= lim || (int64_t)p->width * p->hidden * 2 >= lim ||
      (int64_t)N * p->future_window * p->width * 2 >= lim ||
      (int64_t)N * p->future_window * (p->num_experts + 1) * 4 >= lim)
    return hr_fail(MOE_ERR_SHAPE, "sizes beyond 2 GiB buffers");
  return MOE_OK;
}
}  // namespace

extern "C" {

int64_t moe_hr_predictor_workspace_bytes_v1(int32_t N, const moe_hr_predictor_params_v1* params) {
  if (!params || N < 0) return -1;
  return hr_predictor_workspace(N, params->width, params->future_window, params->num_experts);
}

int moe_hr_predictor_v1(const uint16_t* hidden, int32_t N, const int32_t* layer_ids,
                        const moe_hr_predictor_params_v1* params, const float* prior,
                        float residual_scale, const float* scale_per_example, int32_t top_k,
                        void* workspace, int64_t workspace_bytes, float* logits_out,
                        int32_t* topk_ids, void* stream) {
  int rc = hr_check(N, params, top_k);
  if (rc) return rc;
  if (N == 0) return MOE_OK;
  if (!hidden || !layer_ids || !workspace || !topk_ids)
    return hr_fail(MOE_ERR_NULL, "NULL hidden, layer_ids, workspace or topk_ids");
  if (workspace_bytes < hr_predictor_workspace(N, params->width, params->future_window,
                                               params->num_experts))
    return hr_fail(MOE_ERR_WORKSPACE, "workspace too small");
  if (!workspace_aligned(workspace)) return hr_fail(MOE_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  const hipError_t e = launch_hr_predictor(hidden, N, params->hidden, layer_ids, *params, prior,
                                           residual_scale, scale_per_example, top_k, workspace,
                                           logits_out, topk_ids, (hipStream_t)stream);
  if (e != hipSuccess) {
    snprintf(moe_error_buffer(), kErrorBufferBytes, "hidden-residual predictor: HIP error %d (%s)",
             (int)e, hipGetErrorString(e));
    return MOE_ERR_HIP + ((int)e % 100);
  }
  return MOE_OK;
}

}  // extern "C"
