// Router for prefill-size batches: approximate logits on MFMA, then a certified exact top-k.
//
// The routing ids must equal those of the canonical-order fp32 logits (routing.h:logits_tile,
// the order the oracle restates), but computing every logit in that order is VALU work of
// T x E x H fma (1.07 G at 2048 tokens). Here:
//  1. router_mfma_kernel: m[t, e] = x_t . w_e + bias[e] with v_mfma_f32_16x16x32_bf16 (any
//     summation order), and the squared router-row norms |w_e|^2.
//  2. router_certify_kernel, one wave per token: the top-k of m; a rigorous bound
//     |m[t, e] - l[t, e]| <= eps[t, e] (l the canonical logit) certifies the selected set when
//     min over the set of (m - eps) exceeds max over the rest of (m + eps); otherwise every
//     expert whose m + eps reaches that minimum is a candidate. The canonical logits of the
//     candidates (the selected k when certified) are then computed in the canonical order and
//     the top-k is taken among them with the tie rule, so ids, their order and the
//     renormalised weights are exactly those of the canonical logits.
//
// The bound: with S = sum_i |x_i w_i| <= |x|_2 |w_e|_2 (Cauchy-Schwarz), every fp32 summation
// of the n = H exact bf16 x bf16 products in any order, each addition rounded with relative
// error at most 2u (u = 2^-24; RNE gives u, the factor 2 covers a truncating accumulator), is
// within gamma(2u, n) S of the exact sum, gamma(v, n) = n v / (1 - n v); the canonical order
// (at most 40 roundings per product) is within gamma(u, 40) S. Adding the fp32 bias rounds each
// side once more (<= 2u |m|), and the norms themselves are fp32 (relative error below 1e-3,
// covered by the factor 1.01). Non-finite values make every expert a candidate.
//
// Semantics followed: vLLM topk_softmax(renormalize=True) as restated at
// src/mtp_expert_prefetch/tracing/vllm_router_trace.py:4201-4225, with the canonical logits of
// the decode router.
#include <math.h>

#include "launch.h"
#include "routing.h"

namespace {

typedef __bf16 bf16x8_r __attribute__((ext_vector_type(8)));

MOE_DEV bf16x8_r as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8_r, v); }

constexpr int kTileT = 32, kTileE = 64;  // tokens x experts per workgroup
constexpr int kKSplit = 4;                // waves per workgroup, each a quarter of K
constexpr int kStepK = 64;                // k per step: one 128-byte line of every row
constexpr int kStageRows = kTileT + kTileE;             // rows of one stage: tokens, then experts
constexpr int kStageLoads = kStageRows / 8;             // 1 KB loads per stage (8 rows each)

// Position of 16-byte chunk c (0..7) of stage row R in LDS (elements). The chunks of a row are
// XOR-swizzled so that the fragment reads of 16 rows at one chunk fall in distinct bank groups.
MOE_DEV int stage_chunk(int R, int c) {
  return R * kStepK + 8 * (c ^ ((R & 7) ^ ((R >> 3) & 1)));
}

// One workgroup: a 32 x 64 (token x expert) tile of approximate logits as 2 x 4 MFMA 16x16x32
// tiles; its four waves take a quarter of K each and their partial sums are added through LDS.
// Operands are staged through LDS, one 64-k step per stage and wave (96 rows x 128 bytes, two
// stages per wave): each load instruction moves 8 whole 128-byte rows straight into LDS
// (buffer_load ... lds), so every L1 -> L2 request is a full line. (Loading the MFMA fragments
// directly, 16 rows x 64 bytes per instruction, made every request a half line, and the kernel
// was bound by the requests a CU keeps in flight.) Lane (r, kq) then reads row r at chunk
// 4 S + kq of k-slice S: both operands in the same k order. Workgroups of the first token tile
// also accumulate |w_e|^2 of their expert rows.
__global__ __launch_bounds__(64 * kKSplit) void router_mfma_kernel(
    const uint16_t* __restrict__ x, int T, int H, const uint16_t* __restrict__ W, int E,
    const float* __restrict__ bias, float* __restrict__ approx, float* __restrict__ nw2) {
  // Two stages as separate objects: the compiler then knows that reads of one do not wait for
  // the loads in flight into the other.
  __shared__ __attribute__((aligned(16))) uint16_t stage0[kKSplit][kStageRows * kStepK];
  __shared__ __attribute__((aligned(16))) uint16_t stage1[kKSplit][kStageRows * kStepK];
  __shared__ float part[kKSplit][2 * 4][4][64];  // [wave][tile][element][lane]
  __shared__ float s_n2[kKSplit][4][64];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  // Workgroup b runs on XCD b % 8 (round-robin dispatch): tile index = (b % 8) * chunk + b / 8,
  // so the expert tiles of a token tile, which read the same token rows, share one XCD's L2.
  const int tiles_e = (E + kTileE - 1) / kTileE;
  const int n_tiles = ((T + kTileT - 1) / kTileT) * tiles_e;
  const int chunk = (n_tiles + 7) / 8;
  const int idx = (int)(blockIdx.x % 8) * chunk + (int)(blockIdx.x / 8);
  if (idx >= n_tiles) return;  // workgroup-uniform
  const int tt = idx / tiles_e, te = idx % tiles_e;
  const int t0 = tt * kTileT, e0 = te * kTileE;
  const __amdgpu_buffer_rsrc_t xr = buf_rsrc(x, (uint32_t)T * (uint32_t)H * 2u);
  const __amdgpu_buffer_rsrc_t wr = buf_rsrc(W, (uint32_t)E * (uint32_t)H * 2u);
  const int r = lane & 15, kq = lane >> 4;
  const int steps = H / kStepK / kKSplit;  // H % 512 == 0: even
  const uint32_t k0 = (uint32_t)(wv * steps * kStepK);

  // Load q of a stage: lane l fetches row R = 8 q + (l >> 3) at chunk (l & 7) ^ swizzle(R) and
  // writes it at stage_chunk(R, chunk). Rows 0..31 are tokens t0.., rows 32..95 experts e0..;
  // a row past T or E gets an out-of-range offset (zeros, no memory access).
  uint32_t off[kStageLoads];
#pragma unroll
  for (int q = 0; q < kStageLoads; ++q) {
    const int R = 8 * q + (lane >> 3);
    const uint32_t c = (uint32_t)((lane & 7) ^ ((R & 7) ^ ((R >> 3) & 1)));
    if (R < kTileT) {
      const int t = t0 + R;
      off[q] = t < T ? ((uint32_t)t * (uint32_t)H + k0 + 8u * c) * 2u : kOutOfRange;
    } else {
      const int e = e0 + R - kTileT;
      off[q] = e < E ? ((uint32_t)e * (uint32_t)H + k0 + 8u * c) * 2u : kOutOfRange;
    }
  }
  auto dma = [&](uint16_t* st, int s) {  // a step past the slice loads nothing (zeros, unused)
    const uint32_t so = s < steps ? (uint32_t)(s * kStepK * 2) : kOutOfRange;
#pragma unroll
    for (int q = 0; q < kStageLoads; ++q)
      buf_ld128_lds(q < kTileT / 8 ? xr : wr, st + q * 8 * kStepK, off[q] + so);
  };

  const bool norms = tt == 0;  // workgroup-uniform
  float n2[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  f32x4 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const uint16_t* st) {
    u32x4 a[2][2], b[4][2];  // [subtile][k-slice]
#pragma unroll
    for (int S = 0; S < 2; ++S) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i][S] = *reinterpret_cast<const u32x4*>(st + stage_chunk(16 * i + r, 4 * S + kq));
#pragma unroll
      for (int j = 0; j < 4; ++j)
        b[j][S] = *reinterpret_cast<const u32x4*>(st + stage_chunk(kTileT + 16 * j + r,
                                                                     4 * S + kq));
    }
#pragma unroll
    for (int S = 0; S < 2; ++S)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[i][S]),
                                                              as_bf16x8(b[j][S]), acc[i][j], 0,
                                                              0, 0);
    if (norms) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int S = 0; S < 2; ++S)
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const float lo = bf16lo_to_f32(b[j][S][d]), hi = bf16hi_to_f32(b[j][S][d]);
            n2[j] = __builtin_fmaf(lo, lo, n2[j]);
            n2[j] = __builtin_fmaf(hi, hi, n2[j]);
          }
    }
  };

  // Two stages per wave (the wave's own LDS, no barrier): the wait at the top of a step is for
  // that step's loads only; the next step's stay in flight. A stage is refilled once its
  // fragments are in registers.
  uint16_t* const s0 = stage0[wv];
  uint16_t* const s1 = stage1[wv];
  dma(s0, 0);
  __builtin_amdgcn_sched_barrier(0);  // issue order = step order
  dma(s1, 1);
  for (int s = 0; s < steps; s += 2) {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(kStageLoads));
    compute(s0);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): stage 0's reads done before it is refilled
    __builtin_amdgcn_sched_barrier(0);
    dma(s0, s + 2);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(kStageLoads));
    compute(s1);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_sched_barrier(0);
    dma(s1, s + 3);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int el = 0; el < 4; ++el) part[wv][i * 4 + j][el][lane] = acc[i][j][el];
  if (norms) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v = n2[j];
      v += xor_partner<16>(v);
      v += xor_partner<32>(v);
      s_n2[wv][j][lane] = v;
    }
  }
  __syncthreads();
  // wave wv adds the four partials of tiles 2 wv, 2 wv + 1 and stores them. D of tile (i, j):
  // lane holds rows 4 kq + el, column r.
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int tile = 2 * wv + h, i = tile >> 2, j = tile & 3;
    const int e = e0 + 16 * j + r;
    const float be = (bias && e < E) ? bias[e] : 0.0f;
#pragma unroll
    for (int el = 0; el < 4; ++el) {
      float v = part[0][tile][el][lane];
#pragma unroll
      for (int w = 1; w < kKSplit; ++w) v += part[w][tile][el][lane];
      const int t = t0 + 16 * i + 4 * kq + el;
      if (t < T && e < E) approx[(int64_t)t * (E + 1) + e] = v + be;
    }
  }
  if (norms && wv == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = e0 + 16 * j + r;
      const float v = s_n2[0][j][lane] + s_n2[1][j][lane] + s_n2[2][j][lane] + s_n2[3][j][lane];
      if (kq == 0 && e < E) nw2[e] = v;
    }
  }
}

constexpr int kCertWaves = 4;
constexpr int kCertBatch = 8;  // canonical dots whose loads are in flight together

// Canonical logits (routing.h:logits_tile order, bias added) of up to kCertBatch rows of W
// (row E = the shared gate row sw) against the token chunks xc held by this lane (chunk
// lane + 64 j); ids past n are skipped. Lane 0 writes them to out[id].
template <int NJ>
MOE_DEV void canonical_batch(const u32x4 (&xc)[NJ], int nq, const int* ids, int n,
                             __amdgpu_buffer_rsrc_t wr, __amdgpu_buffer_rsrc_t sr, int H, int E,
                             const float* __restrict__ bias, float* out, int lane) {
  u32x4 wc[kCertBatch][NJ];
#pragma unroll
  for (int b = 0; b < kCertBatch; ++b) {
    const int e = b < n ? ids[b] : -1;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int q = lane + 64 * j;
      const bool ok = e >= 0 && q < nq;
      const uint32_t off = ok ? ((e == E ? 0u : (uint32_t)e * (uint32_t)H) + 8u * (uint32_t)q) * 2u
                              : kOutOfRange;
      wc[b][j] = buf_ld128(e == E ? sr : wr, off);
    }
  }
#pragma unroll
  for (int b = 0; b < kCertBatch; ++b) {
    if (b >= n) break;  // wave-uniform
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (lane + 64 * j >= nq) continue;  // no arithmetic past H (the fma chain stays exact)
#pragma unroll
      for (int el = 0; el < 8; ++el) {
        const uint32_t xd = xc[j][el >> 1], wd = wc[b][j][el >> 1];
        const float xf = (el & 1) ? bf16hi_to_f32(xd) : bf16lo_to_f32(xd);
        const float wf = (el & 1) ? bf16hi_to_f32(wd) : bf16lo_to_f32(wd);
        acc = __builtin_fmaf(xf, wf, acc);
      }
    }
    acc = bfly_sum(acc);
    const int e = ids[b];
    if (bias && e < E) acc = acc + bias[e];
    if (lane == 0) out[e] = acc;
  }
}

// One wave per token. MAXC: E <= 64 MAXC; NJ: H <= 512 NJ.
template <int MAXC, int NJ>
__global__ __launch_bounds__(64 * kCertWaves) void router_certify_kernel(
    const uint16_t* __restrict__ x, int T, int H, const uint16_t* __restrict__ W, int E,
    const uint16_t* __restrict__ shared_w, const float* __restrict__ bias,
    const float* __restrict__ approx, const float* __restrict__ nw2, float rel_bound, int top_k,
    int32_t* __restrict__ ids, float* __restrict__ weights) {
  __shared__ float s_exact[kCertWaves][64 * MAXC + 1];  // canonical logits; [E] = shared gate
  __shared__ int s_list[kCertWaves][64 * MAXC + 1];     // candidate ids, ascending
  const int lane = threadIdx.x & 63;
  const int wb = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int t = blockIdx.x * kCertWaves + wb;
  if (t >= T) return;
  float* exact = s_exact[wb];
  int* list = s_list[wb];
  const int nq = H / 8;

  // this token's chunks (lane + 64 j), the approximate logits and the row norms
  const __amdgpu_buffer_rsrc_t xr = buf_rsrc(x, (uint32_t)T * (uint32_t)H * 2u);
  u32x4 xc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int q = lane + 64 * j;
    xc[j] = buf_ld128(xr, q < nq ? ((uint32_t)t * (uint32_t)H + 8u * (uint32_t)q) * 2u : kOutOfRange);
  }
  const __amdgpu_buffer_rsrc_t ar = buf_rsrc(approx + (int64_t)t * (E + 1), (uint32_t)E * 4u);
  const __amdgpu_buffer_rsrc_t nr = buf_rsrc(nw2, (uint32_t)E * 4u);
  float m[MAXC], w2[MAXC];
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    m[c] = __uint_as_float(buf_ld32(ar, (uint32_t)(lane + 64 * c) * 4u));
    w2[c] = __uint_as_float(buf_ld32(nr, (uint32_t)(lane + 64 * c) * 4u));
  }
  float xs = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float lo = bf16lo_to_f32(xc[j][d]), hi = bf16hi_to_f32(xc[j][d]);
      xs = __builtin_fmaf(lo, lo, xs);
      xs = __builtin_fmaf(hi, hi, xs);
    }
  const float nx = sqrtf(bfly_sum(xs));

  // approximate top-k and its certificate
  uint32_t key[MAXC], key0[MAXC];
  float eps[MAXC];
  bool finite = isfinite(nx);
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const bool in = lane + 64 * c < E;
    key0[c] = key[c] = topk_ord(m[c]) & (0u - (uint32_t)in);
    eps[c] = rel_bound * nx * sqrtf(w2[c]) + 2.384185791e-7f * fabsf(m[c]) + 1e-30f;
    finite = finite && (!in || (isfinite(m[c]) && isfinite(eps[c])));
  }
  int sel_i;
  uint32_t sel_key;
  topk_select_keys<MAXC>(key, top_k, lane, sel_i, sel_key);
  float lower_sel = INFINITY, upper_rest = -INFINITY;
  bool in_sel[MAXC];
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    in_sel[c] = key0[c] != 0u && key[c] == 0u;
    if (in_sel[c]) lower_sel = fminf(lower_sel, m[c] - eps[c]);
    else if (key0[c] != 0u) upper_rest = fmaxf(upper_rest, m[c] + eps[c]);
  }
  const bool all_finite = __ballot(!finite) == 0;
  lower_sel = bfly_min(lower_sel);
  upper_rest = bfly_max(upper_rest);
  const bool certain = all_finite && lower_sel > upper_rest;

  // candidates in ascending id order (the shared gate row E last)
  int n = 0;
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const bool in = key0[c] != 0u;
    const bool cand = in && (in_sel[c] || !all_finite || (!certain && m[c] + eps[c] >= lower_sel));
    const uint64_t bm = __ballot(cand);
    const int pos = n + __popcll(bm & ((1ull << lane) - 1));
    if (cand) list[pos] = lane + 64 * c;
    n += __popcll(bm);
  }
  const bool has_shared = shared_w != nullptr;
  if (has_shared && lane == 0) list[n] = E;
  const int n_dots = n + (has_shared ? 1 : 0);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  const __amdgpu_buffer_rsrc_t wr = buf_rsrc(W, (uint32_t)E * (uint32_t)H * 2u);
  const __amdgpu_buffer_rsrc_t sr = buf_rsrc(shared_w, has_shared ? (uint32_t)H * 2u : 0u);
  for (int b0 = 0; b0 < n_dots; b0 += kCertBatch)
    canonical_batch<NJ>(xc, nq, list + b0, min(kCertBatch, n_dots - b0), wr, sr, H, E, bias,
                        exact, lane);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // exact top-k among the candidates, larger canonical logit first, equal logits by lower id
  int my_rank = 64;
  uint32_t my_key = 0u;
  int my_id = 0;
  if (n <= 64) {  // candidate i in lane i: its rank is the number of candidates ahead of it
    my_id = lane < n ? list[lane] : 0;
    my_key = lane < n ? topk_ord(exact[my_id]) : 0u;
    my_rank = 0;
    for (int j = 0; j < n; ++j) {
      const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)my_key, j);
      const int ij = __builtin_amdgcn_readlane(my_id, j);
      my_rank += (kj > my_key || (kj == my_key && ij < my_id)) ? 1 : 0;
    }
    if (lane >= n) my_rank = 64;
  } else {  // many candidates (near-ties or non-finite logits): round-based selection
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const int e = lane + 64 * c;
      const bool in = key0[c] != 0u;
      const bool cand = in && (in_sel[c] || !all_finite || (!certain && m[c] + eps[c] >= lower_sel));
      key[c] = cand ? topk_ord(exact[e < E ? e : 0]) : 0u;
    }
    topk_select_keys<MAXC>(key, top_k, lane, sel_i, sel_key);
    my_rank = lane < top_k ? lane : 64;
    my_id = sel_i;
    my_key = sel_key;
  }
  // renormalised weights exp(l_r - l_0) / sum_{r < k} exp(l_r - l_0), summed in rank order
  const float my_v = topk_ord_value(my_key);
  const int lane0 = __ffsll((long long)__ballot(my_rank == 0)) - 1;
  const float vmax = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_v), lane0));
  const float ex = my_rank < top_k ? expf(my_v - vmax) : 0.0f;
  float ssum = 0.0f;
  for (int r = 0; r < top_k; ++r) {
    const int lr = __ffsll((long long)__ballot(my_rank == r)) - 1;
    ssum = ssum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), lr));
  }
  if (my_rank < top_k) {
    ids[(int64_t)t * top_k + my_rank] = my_id;
    weights[(int64_t)t * top_k + my_rank] = ex / ssum;
  }
  if (has_shared && lane == 0) weights[(int64_t)T * top_k + t] = 1.0f / (1.0f + expf(-exact[E]));
}

template <int MAXC, int NJ>
hipError_t launch_certify(const uint16_t* x, int T, int H, const uint16_t* W, int E,
                          const uint16_t* shared_w, const float* bias, const float* approx,
                          const float* nw2, float rel, int top_k, int32_t* ids, float* weights,
                          hipStream_t stream) {
  hipLaunchKernelGGL((router_certify_kernel<MAXC, NJ>), dim3((T + kCertWaves - 1) / kCertWaves),
                     dim3(64 * kCertWaves), 0, stream, x, T, H, W, E, shared_w, bias, approx, nw2,
                     rel, top_k, ids, weights);
  return hipGetLastError();
}

}  // namespace

bool router_prefill_fits(int T, int H, int E, int top_k) {
  return T >= 1 && H >= 512 && H <= 2048 && H % 512 == 0 && E >= 1 && E <= 512 && top_k >= 1 &&
         top_k <= 64 && top_k <= E && (int64_t)T * H * 2 < kOutOfRange &&
         (int64_t)E * H * 2 < kOutOfRange;
}

// Relative bound factor: gamma(2u, H) + gamma(u, 40), times 1.01 for the fp32 norms.
float router_prefill_rel_bound(int H) {
  const double u = 1.0 / 16777216.0;
  const double g_any = (2.0 * u * H) / (1.0 - 2.0 * u * H);
  const double g_can = (u * 40.0) / (1.0 - u * 40.0);
  return (float)((g_any + g_can) * 1.01);
}

hipError_t launch_router_prefill(const uint16_t* x, int T, int H, const uint16_t* W, int E,
                                 const uint16_t* shared_w, const float* bias, int top_k,
                                 float* approx, float* nw2, int32_t* ids, float* weights,
                                 hipStream_t stream) {
  if (!router_prefill_fits(T, H, E, top_k)) return hipErrorInvalidValue;
  const int tiles = ((T + kTileT - 1) / kTileT) * ((E + kTileE - 1) / kTileE);
  hipLaunchKernelGGL(router_mfma_kernel, dim3((tiles + 7) / 8 * 8), dim3(64 * kKSplit), 0, stream,
                     x, T, H, W, E, bias, approx, nw2);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const float rel = router_prefill_rel_bound(H);
  const int nj = H / 512;
  if (E <= 256) {
    switch (nj) {
      case 1: return launch_certify<4, 1>(x, T, H, W, E, shared_w, bias, approx, nw2, rel, top_k, ids, weights, stream);
      case 2: return launch_certify<4, 2>(x, T, H, W, E, shared_w, bias, approx, nw2, rel, top_k, ids, weights, stream);
      case 3: return launch_certify<4, 3>(x, T, H, W, E, shared_w, bias, approx, nw2, rel, top_k, ids, weights, stream);
      default: return launch_certify<4, 4>(x, T, H, W, E, shared_w, bias, approx, nw2, rel, top_k, ids, weights, stream);
    }
  }
  switch (nj) {
    case 1: return launch_certify<8, 1>(x, T, H, W, E, shared_w, bias, approx, nw2, rel, top_k, ids, weights, stream);
    case 2: return launch_certify<8, 2>(x, T, H, W, E, shared_w, bias, approx, nw2, rel, top_k, ids, weights, stream);
    case 3: return launch_certify<8, 3>(x, T, H, W, E, shared_w, bias, approx, nw2, rel, top_k, ids, weights, stream);
    default: return launch_certify<8, 4>(x, T, H, W, E, shared_w, bias, approx, nw2, rel, top_k, ids, weights, stream);
  }
}
