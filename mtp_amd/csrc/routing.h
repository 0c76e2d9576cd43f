// Device building blocks of the routing stage, shared by the standalone kernels (router.hip,
// align.hip) and the fused decode routing kernel.
//
// logits_tile: fp32 logits of a TT x TE (token x router-row) tile by one wave in the canonical
//   order (chunk q of 8 bf16 -> lane q % 64; per lane increasing q then k with fma from +0.0f;
//   lanes combined by v += shfl_xor(v, m), m = 32 .. 1). The CPU oracle reproduces this order.
// topk_token: one wave selects the top-k of one token's logits (larger logit first, equal logits
//   -> lower id; vLLM topk_softmax(renormalize=True) semantics,
//   src/mtp_expert_prefetch/tracing/vllm_router_trace.py:4201-4225).
// align_block: one 1024-thread block turns top-k ids into the block-padded expert-grouped slot
//   layout (vLLM moe_align_block_size format, vllm_router_trace.py:19647-19660): experts
//   ascending, slots ascending inside an expert, each group padded to BM with the sentinel
//   num_slots, unused blocks tagged -1.
#pragma once

#include "common.h"

// ---------------------------------------------------------------------------- logits
template <int TT, int TE>
MOE_DEV void logits_tile(const uint16_t* __restrict__ x, int T, int H, const uint16_t* __restrict__ W,
                         int E, const uint16_t* __restrict__ shared_w, const float* __restrict__ bias,
                         float* __restrict__ logits, int t0, int e0, int lane) {
  const int rows = E + (shared_w ? 1 : 0);
  // Buffer loads: a token or router row outside the tile's range, and chunks past H, read zeros
  // without a memory access, so every iteration issues the same loads (exact wait counts).
  // t0 and e0 are wave-uniform: the resources and row offsets live in scalar registers.
  const __amdgpu_buffer_rsrc_t xr = buf_rsrc(x, (uint32_t)T * (uint32_t)H * 2u);
  const __amdgpu_buffer_rsrc_t wr = buf_rsrc(W, (uint32_t)E * (uint32_t)H * 2u);
  const __amdgpu_buffer_rsrc_t sr = buf_rsrc(shared_w, shared_w ? (uint32_t)H * 2u : 0u);
  uint32_t xo[TT], wo[TE];
#pragma unroll
  for (int i = 0; i < TT; ++i) xo[i] = (t0 + i < T) ? (uint32_t)(t0 + i) * (uint32_t)H * 2u : kOutOfRange;
#pragma unroll
  for (int j = 0; j < TE; ++j) {
    const int e = e0 + j;
    wo[j] = e < E ? (uint32_t)e * (uint32_t)H * 2u : (e == E && shared_w ? 0u : kOutOfRange);
  }
  float acc[TT][TE];
#pragma unroll
  for (int i = 0; i < TT; ++i)
#pragma unroll
    for (int j = 0; j < TE; ++j) acc[i][j] = 0.0f;

  // Lane l owns chunks q = l, l + 64, ... (8 bf16 each) and accumulates them in increasing q;
  // NI iterations of loads are in flight before their arithmetic.
  constexpr int NI = 4;
  const int nq = H / 8;
  for (int q0 = 0; q0 < nq; q0 += 64 * NI) {
    u32x4 xv[NI][TT], wv[NI][TE];
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const int q = q0 + 64 * it + lane;
      const uint32_t qo = q < nq ? (uint32_t)q * 16u : kOutOfRange;
#pragma unroll
      for (int i = 0; i < TT; ++i) xv[it][i] = buf_ld128(xr, (xo[i] + qo) | (qo & kOutOfRange));
#pragma unroll
      for (int j = 0; j < TE; ++j)
        wv[it][j] = buf_ld128(e0 + j == E ? sr : wr, (wo[j] + qo) | (qo & kOutOfRange));
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the NI iterations before the first wait
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      if (q0 + 64 * it + lane >= nq) continue;  // no arithmetic past H (keeps the fma chain exact)
#pragma unroll
      for (int el = 0; el < 8; ++el) {
        float wf[TE];
#pragma unroll
        for (int j = 0; j < TE; ++j)
          wf[j] = (el & 1) ? bf16hi_to_f32(wv[it][j][el >> 1]) : bf16lo_to_f32(wv[it][j][el >> 1]);
#pragma unroll
        for (int i = 0; i < TT; ++i) {
          const uint32_t xd = xv[it][i][el >> 1];
          const float xf = (el & 1) ? bf16hi_to_f32(xd) : bf16lo_to_f32(xd);
#pragma unroll
          for (int j = 0; j < TE; ++j) acc[i][j] = __builtin_fmaf(xf, wf[j], acc[i][j]);
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < TT; ++i)
#pragma unroll
    for (int j = 0; j < TE; ++j) {
      float v = acc[i][j];
      v = bfly_sum(v);
      acc[i][j] = v;
    }
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < TT; ++i)
#pragma unroll
      for (int j = 0; j < TE; ++j) {
        const int t = t0 + i, e = e0 + j;
        if (t < T && e < rows) {
          float v = acc[i][j];
          if (bias && e < E) v = v + bias[e];
          logits[(int64_t)t * (E + 1) + e] = v;
        }
      }
  }
}

// logits_tile for H <= 2048 with the TT token rows in LDS (x_lds [TT][H] bf16, rows t0 ..
// t0 + TT - 1 of the batch), in two phases: load() issues every chunk of the wave's TE router
// rows (no dependence on x), compute_store() runs the same chunks per lane, fma order and
// butterfly as logits_tile, so the logits are bit-identical to logits_tile on the same rows.
template <int TT, int TE>
struct LdsLogitsTile {
  static constexpr int NI = 4;  // 64 * NI chunks of 8 = 2048 columns
  u32x4 wv[NI][TE];

  MOE_DEV void load(int H, const uint16_t* __restrict__ W, int E,
                    const uint16_t* __restrict__ shared_w, int e0, int lane) {
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(W, (uint32_t)E * (uint32_t)H * 2u);
    const __amdgpu_buffer_rsrc_t sr = buf_rsrc(shared_w, shared_w ? (uint32_t)H * 2u : 0u);
    const int nq = H / 8;
#pragma unroll
    for (int j = 0; j < TE; ++j) {
      const int e = e0 + j;
      const uint32_t wo =
          e < E ? (uint32_t)e * (uint32_t)H * 2u : (e == E && shared_w ? 0u : kOutOfRange);
#pragma unroll
      for (int it = 0; it < NI; ++it) {
        const int q = 64 * it + lane;
        const uint32_t qo = q < nq ? (uint32_t)q * 16u : kOutOfRange;
        wv[it][j] = buf_ld128(e == E ? sr : wr, (wo + qo) | (qo & kOutOfRange));
      }
    }
  }

  MOE_DEV void compute_store(const uint16_t* x_lds, int T, int H, int E, bool has_shared,
                             const float* __restrict__ bias, float* __restrict__ logits, int t0,
                             int e0, int lane) const {
    const int rows = E + (has_shared ? 1 : 0), nq = H / 8;
    float acc[TT][TE];
#pragma unroll
    for (int i = 0; i < TT; ++i)
#pragma unroll
      for (int j = 0; j < TE; ++j) acc[i][j] = 0.0f;
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const int q = 64 * it + lane;
      if (q >= nq) continue;
      u32x4 xv[TT];
#pragma unroll
      for (int i = 0; i < TT; ++i) xv[i] = ld128(x_lds + i * H + 8 * q);
#pragma unroll
      for (int el = 0; el < 8; ++el) {
        float wf[TE];
#pragma unroll
        for (int j = 0; j < TE; ++j)
          wf[j] = (el & 1) ? bf16hi_to_f32(wv[it][j][el >> 1]) : bf16lo_to_f32(wv[it][j][el >> 1]);
#pragma unroll
        for (int i = 0; i < TT; ++i) {
          const uint32_t xd = xv[i][el >> 1];
          const float xf = (el & 1) ? bf16hi_to_f32(xd) : bf16lo_to_f32(xd);
#pragma unroll
          for (int j = 0; j < TE; ++j) acc[i][j] = __builtin_fmaf(xf, wf[j], acc[i][j]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < TT; ++i)
#pragma unroll
      for (int j = 0; j < TE; ++j) {
        float v = acc[i][j];
        v = bfly_sum(v);
        acc[i][j] = v;
      }
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < TT; ++i)
#pragma unroll
        for (int j = 0; j < TE; ++j) {
          const int t = t0 + i, e = e0 + j;
          if (t < T && e < rows) {
            float v = acc[i][j];
            if (bias && e < E) v = v + bias[e];
            logits[(int64_t)t * (E + 1) + e] = v;
          }
        }
    }
  }
};

// ---------------------------------------------------------------------------- top-k
// 32-bit order key of a logit: unsigned order = logit order, with -0 equal to +0 and NaN (key 1)
// below every number; key 0 marks "not a candidate" (already selected, or past E).
MOE_DEV uint32_t topk_ord(float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7FFFFFFFu) == 0u) u = 0u;  // -0 -> +0
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((__float_as_uint(v) & 0x7FFFFFFFu) > 0x7F800000u) ? 1u : u;
}

// The logit of a key (a NaN for key 1; +0 for either zero).
MOE_DEV float topk_ord_value(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

// DPP move with 0 in the lanes a row mask leaves out (0 is the identity of unsigned max, so the
// move and the max fuse into one v_max_u32_dpp).
#define MOE_DPP(v, ctrl, rmask) \
  (uint32_t) __builtin_amdgcn_update_dpp(0, (int)(v), ctrl, rmask, 0xF, false)

// Wave-wide maximum through DPP (quad xor 1, quad xor 2, half-row mirror, row mirror,
// row_bcast15, row_bcast31); the result is read from lane 63 and is wave-uniform.
MOE_DEV uint32_t wave_max_u32(uint32_t v) {
  v = max(v, MOE_DPP(v, 0xB1, 0xF));   // quad_perm(1,0,3,2)
  v = max(v, MOE_DPP(v, 0x4E, 0xF));   // quad_perm(2,3,0,1)
  v = max(v, MOE_DPP(v, 0x141, 0xF));  // row_half_mirror
  v = max(v, MOE_DPP(v, 0x140, 0xF));  // row_mirror
  v = max(v, MOE_DPP(v, 0x142, 0xA));  // row_bcast15 into rows 1, 3
  v = max(v, MOE_DPP(v, 0x143, 0xC));  // row_bcast31 into rows 2, 3
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// One wave: the top_k (<= 64) largest keys, larger key first and equal keys by lower id (the
// reference's tie rule made explicit). key[c] of lane l belongs to id l + 64 c; key 0 marks
// "not a candidate" (there must be at least top_k candidates). A round is a 32-bit wave
// maximum plus one ballot per column to find the lowest id holding it; the selected keys are
// cleared to 0. Lane r < top_k receives the r-th selection (id, key).
template <int MAXC>
MOE_DEV void topk_select_keys(uint32_t (&key)[MAXC], int top_k, int lane, int& my_i,
                              uint32_t& my_key) {
  my_key = 0u;
  my_i = 0;
  for (int r = 0; r < top_k; ++r) {
    uint32_t m = key[0];
#pragma unroll
    for (int c = 1; c < MAXC; ++c) m = max(m, key[c]);
    m = wave_max_u32(m);
    int sel = -1;  // lowest id whose key is the maximum (wave-uniform)
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const uint64_t b = __ballot(key[c] == m);
      if (sel < 0 && b != 0) sel = 64 * c + __ffsll((long long)b) - 1;
    }
#pragma unroll
    for (int c = 0; c < MAXC; ++c)
      if (lane + 64 * c == sel) key[c] = 0u;
    if (lane == r) {
      my_i = sel;
      my_key = m;
    }
  }
}

// One wave: the top_k (<= 64) largest of row[0..E) (E <= 64 * MAXC), larger logit first and
// equal logits by lower id. Lane r < top_k receives the r-th selection (id, logit). Every logit
// is loaded at once (lanes past E read zeros without a memory access and are masked out).
template <int MAXC>
MOE_DEV void topk_select(const float* __restrict__ row, int E, int top_k, int lane, int& my_i,
                         float& my_v) {
  const __amdgpu_buffer_rsrc_t rr = buf_rsrc(row, (uint32_t)E * 4u);
  float v[MAXC];
#pragma unroll
  for (int c = 0; c < MAXC; ++c) v[c] = __uint_as_float(buf_ld32(rr, (uint32_t)(lane + 64 * c) * 4u));
  uint32_t key[MAXC];
#pragma unroll
  for (int c = 0; c < MAXC; ++c)  // masked with an AND: a select of a loaded value would become
                                  // a branch around the load with a wait inside it
    key[c] = topk_ord(v[c]) & (0u - (uint32_t)(lane + 64 * c < E));
  uint32_t my_key;
  topk_select_keys<MAXC>(key, top_k, lane, my_i, my_key);
  my_v = (lane < top_k) ? topk_ord_value(my_key) : 0.0f;
}

// Renormalised weight of lane r's selection: exp(l_r - l_0) / sum_{j < k} exp(l_j - l_0), the sum
// in selection order. Called by a whole wave (the lane reads are v_readlane, not LDS permutes).
MOE_DEV float topk_weight(float my_v, int top_k, int lane) {
  const float vmax = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_v), 0));
  const float ex = (lane < top_k) ? expf(my_v - vmax) : 0.0f;
  float s = 0.0f;
  for (int r = 0; r < top_k; ++r)
    s = s + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), r));
  return ex / s;
}

// One wave: top-k of row[0..E) (E <= 64 * MAXC). Writes ids[t*k + r], weights[t*k + r]
// (r < k) and, when has_shared, weights[T*k + t] = sigmoid(row[E]). Optionally mirrors the ids
// to ids_lds.
template <int MAXC>
MOE_DEV void topk_token(const float* __restrict__ row, int E, int top_k, int has_shared, int T,
                        int t, int lane, int32_t* __restrict__ ids, float* __restrict__ weights,
                        int* ids_lds, int32_t* ids_mirror = nullptr) {
  // row[E] when has_shared, else zero; issued with the selection's loads
  const float g = __uint_as_float(
      buf_ld32(buf_rsrc(row, (uint32_t)(E + (has_shared ? 1 : 0)) * 4u), (uint32_t)E * 4u));
  int my_i;
  float my_v;
  topk_select<MAXC>(row, E, top_k, lane, my_i, my_v);
  const float w = topk_weight(my_v, top_k, lane);
  if (lane < top_k) {
    ids[(int64_t)t * top_k + lane] = my_i;
    weights[(int64_t)t * top_k + lane] = w;
    if (ids_lds) ids_lds[t * top_k + lane] = my_i;
    if (ids_mirror) ids_mirror[(int64_t)t * top_k + lane] = my_i;
  }
  if (has_shared && lane == 0) weights[(int64_t)T * top_k + t] = 1.0f / (1.0f + expf(-g));
}

// One wave: top-k of row[0..E) into LDS only (ids_lds[r], w_lds[r] for r < top_k), the same
// selection and weights as topk_token.
template <int MAXC>
MOE_DEV void topk_token_lds(const float* __restrict__ row, int E, int top_k, int lane, int* ids_lds,
                            float* w_lds) {
  int my_i;
  float my_v;
  topk_select<MAXC>(row, E, top_k, lane, my_i, my_v);
  const float w = topk_weight(my_v, top_k, lane);
  if (lane < top_k) {
    ids_lds[lane] = my_i;
    w_lds[lane] = w;
  }
}

// topk_token / topk_token_lds for any E <= 512 (a uniform branch on E).
MOE_DEV void topk_token_any(const float* __restrict__ row, int E, int top_k, int has_shared, int T,
                            int t, int lane, int32_t* __restrict__ ids,
                            float* __restrict__ weights, int* ids_lds,
                            int32_t* ids_mirror = nullptr) {
  if (E <= 256)
    topk_token<4>(row, E, top_k, has_shared, T, t, lane, ids, weights, ids_lds, ids_mirror);
  else
    topk_token<8>(row, E, top_k, has_shared, T, t, lane, ids, weights, ids_lds, ids_mirror);
}
MOE_DEV void topk_token_lds_any(const float* __restrict__ row, int E, int top_k, int lane,
                                int* ids_lds, float* w_lds) {
  if (E <= 256)
    topk_token_lds<4>(row, E, top_k, lane, ids_lds, w_lds);
  else
    topk_token_lds<8>(row, E, top_k, lane, ids_lds, w_lds);
}

// ---------------------------------------------------------------------------- align
constexpr int kAlignWaves = 16;   // align_block needs blockDim.x == 1024
constexpr int kMaxGroups = 513;   // 512 routed experts + the shared expert

struct AlignSmem {
  int cnt[kAlignWaves][kMaxGroups];
  int off[kMaxGroups];
  int pad[kMaxGroups];
  int wtot[16];
};

// Inclusive prefix sum over the 64 lanes of a wave through DPP: row shifts by 1, 2, 4 and 8
// (a lane whose source lies before its row keeps 0), then row_bcast15 into rows 1 and 3 and
// row_bcast31 into rows 2 and 3. Six dependent VALU operations instead of six LDS permutes.
MOE_DEV int wave_incl_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast31
  return v;
}

// Exclusive prefix sum of v over the threads of a workgroup of at most 16 waves, in thread order,
// and the total. wtot: 16 ints of LDS. Every thread of the workgroup calls it (it synchronises);
// wtot may be reused only after a further barrier.
MOE_DEV int block_excl_sum(int v, int* wtot, int& total) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, nw = (blockDim.x + 63) >> 6;
  const int incl = wave_incl_sum(v);
  if (lane == 63) wtot[w] = incl;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int t = i < nw ? wtot[i] : 0;
    tot += t;
    before += i < w ? t : 0;
  }
  total = tot;
  return before + incl - v;
}

// Division by the (wave-uniform) align block size for n >= 0: a shift when it is a power of two,
// as the kernels' block sizes are, else an integer division (a uniform branch).
struct BlockDiv {
  int bm, sh;
  MOE_DEV explicit BlockDiv(int b) : bm(b), sh((b & (b - 1)) == 0 ? __builtin_ctz(b) : -1) {}
  MOE_DEV int div(int n) const { return sh >= 0 ? (n >> sh) : n / bm; }
  MOE_DEV int pad(int n) const { return div(n + bm - 1) * bm; }  // n rounded up to blocks
};

MOE_DEV int slot_expert(const int32_t* topk_ids, int routed, int E, int f) {
  if (f < routed) {
    const int e = topk_ids[f];
    return (e >= 0 && e < E) ? e : -1;
  }
  return E;  // shared slot
}

// Experts of kAlignIds consecutive chunks of a wave's slot range (slot f = base + 64 u + lane,
// u < kAlignIds), -1 past hi or for an id outside [0, E). The id loads are buffer loads issued
// together (slots past the routed ones read zeros without a memory access), so a batch costs one
// memory latency instead of one per slot.
constexpr int kAlignIds = 8;

MOE_DEV void align_ids(__amdgpu_buffer_rsrc_t ir, int routed, int E, int base, int hi, int lane,
                       int (&e)[kAlignIds]) {
  int raw[kAlignIds];
#pragma unroll
  for (int u = 0; u < kAlignIds; ++u) {
    const int f = base + 64 * u + lane;
    raw[u] = (int)buf_ld32(ir, (f < routed && f < hi) ? (uint32_t)f * 4u : kOutOfRange);
  }
#pragma unroll
  for (int u = 0; u < kAlignIds; ++u) {
    const int f = base + 64 * u + lane;
    const bool routed_ok = f < routed && f < hi && raw[u] >= 0 && raw[u] < E;
    const bool shared = f >= routed && f < hi;  // the shared slots follow the routed ones
    e[u] = routed_ok ? raw[u] : (shared ? E : -1);
  }
}

// topk_ids in global memory.
MOE_DEV void align_block(const int32_t* topk_ids, int T, int top_k, int E, int has_shared, int BM,
                         int cap, int32_t* __restrict__ sorted, int32_t* __restrict__ eids,
                         int32_t* __restrict__ ntpp, AlignSmem& sm) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int routed = T * top_k;
  const int n_slots = routed + (has_shared ? T : 0);
  const int G = E + (has_shared ? 1 : 0);
  const BlockDiv bd(BM);
  for (int i = tid; i < kAlignWaves * kMaxGroups; i += 1024) (&sm.cnt[0][0])[i] = 0;
  __syncthreads();

  const int per_wave = (((n_slots + kAlignWaves - 1) / kAlignWaves) + 63) / 64 * 64;
  const int lo = min(w * per_wave, n_slots), hi = min(lo + per_wave, n_slots);
  const __amdgpu_buffer_rsrc_t ir = buf_rsrc(topk_ids, (uint32_t)routed * 4u);
  for (int base = lo; base < hi; base += 64 * kAlignIds) {
    int e[kAlignIds];
    align_ids(ir, routed, E, base, hi, lane, e);
#pragma unroll
    for (int u = 0; u < kAlignIds; ++u) {
      if (base + 64 * u >= hi) break;  // uniform
      if (e[u] >= 0) atomicAdd(&sm.cnt[w][e[u]], 1);
    }
  }
  __syncthreads();
  int tp;
  {  // padded group sizes and their exclusive scan over the groups (thread g: group g)
    int tot = 0;
    if (tid < G)
      for (int v = 0; v < kAlignWaves; ++v) tot += sm.cnt[v][tid];
    const int pad = bd.pad(tot);
    if (tid < G) sm.pad[tid] = pad;
    const int off = block_excl_sum(pad, sm.wtot, tp);
    if (tid < G) sm.off[tid] = off;
  }
  __syncthreads();
  // Bases: one thread per group turns the 16 waves' counts into running offsets (all groups in
  // parallel) and leaves the end of the group's real slots in pad[]. Then four threads per group
  // write its padding sentinels with 16-byte stores (scalar stores for an unaligned head or tail)
  // and its block ids; a group's padded end is the next group's offset.
  const int limit = cap * BM;
  for (int g = tid; g < G; g += 1024) {
    int run = sm.off[g];
    for (int v = 0; v < kAlignWaves; ++v) {
      const int c = sm.cnt[v][g];
      sm.cnt[v][g] = run;
      run += c;
    }
    sm.pad[g] = run;
  }
  __syncthreads();
  const bool vec = (reinterpret_cast<uintptr_t>(sorted) & 15u) == 0;
  for (int g = tid >> 2; g < G; g += 256) {
    const int sub = tid & 3;
    const int off = sm.off[g], real_end = sm.pad[g];
    const int end = g + 1 < G ? sm.off[g + 1] : tp;
    const int fend = min(end, limit);
    const int a4 = vec ? min((real_end + 3) & ~3, fend) : fend;  // vector part [a4, v_end)
    const int v_end = a4 + ((fend - a4) & ~3);
    if (sub == 0) {
      for (int p = real_end; p < a4; ++p) sorted[p] = n_slots;
      for (int p = v_end; p < fend; ++p) sorted[p] = n_slots;
    }
    const i32x4 sent = {n_slots, n_slots, n_slots, n_slots};
    for (int p = a4 + 4 * sub; p < v_end; p += 16) *reinterpret_cast<i32x4*>(&sorted[p]) = sent;
    const int bend = min(bd.div(end), cap);
    for (int b = bd.div(off) + sub; b < bend; b += 4) eids[b] = g;
  }
  for (int b = bd.div(tp) + tid; b < cap; b += 1024) eids[b] = -1;
  for (int p = tp + tid; p < cap * BM; p += 1024) sorted[p] = n_slots;
  if (tid == 0) *ntpp = tp;
  __syncthreads();

  // Stable scatter: ranges in wave order, slots in order inside a range.
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int base0 = lo; base0 < hi; base0 += 64 * kAlignIds) {
    int eb[kAlignIds];
    align_ids(ir, routed, E, base0, hi, lane, eb);
#pragma unroll
    for (int u = 0; u < kAlignIds; ++u) {
      const int base = base0 + 64 * u;
      if (base >= hi) break;  // uniform: the rest of the batch lies past the wave's range
      const int f = base + lane;
      const int e = eb[u];
      const bool valid = e >= 0;
      uint64_t peers = __ballot(valid);
#pragma unroll
      for (int bit = 0; bit < 10; ++bit) {
        const bool b = valid && ((e >> bit) & 1);
        const uint64_t bal = __ballot(b);
        peers &= b ? bal : ~bal;
      }
      if (valid) {
        const int rank = __popcll(peers & lt_mask);
        const int pos = sm.cnt[w][e] + rank;
        if (pos < cap * BM) sorted[pos] = f;
      }
      // wave-local LDS update after every lane has read the old base
      __builtin_amdgcn_wave_barrier();
      if (valid && (__ffsll((long long)peers) - 1) == lane) sm.cnt[w][e] += __popcll(peers);
      __builtin_amdgcn_wave_barrier();
    }
  }
}

// Single-wave align for at most 64 slots (decode step sizes); same output as align_block.
// Lane f holds slot f: the slots of one expert are found with a ballot match over the expert
// id bits and the lowest lane of each group is its leader. Each leader writes its group's padded
// size into an LDS table indexed by group id (pad_lds, at least E + 1 ints); one exclusive scan
// of the table by the wave gives every group's offset (groups in ascending id order), so the
// cost does not grow with the number of distinct experts. With fill_tail false the entries past
// the padded total (sentinels up to cap * BM, -1 block ids up to cap) are left as they are: the
// decode kernels never read them (every block checks the padded total first).
constexpr int kAlignWaveMaxSlots = 64;

MOE_DEV void align_wave(const int32_t* topk_ids, int T, int top_k, int E, int has_shared, int BM,
                        int cap, int32_t* __restrict__ sorted, int32_t* __restrict__ eids,
                        int32_t* __restrict__ ntpp, int lane, int* pad_lds, bool fill_tail) {
  const int routed = T * top_k;
  const int n_slots = routed + (has_shared ? T : 0);
  const int G = E + (has_shared ? 1 : 0);
  const int e = (lane < n_slots) ? slot_expert(topk_ids, routed, E, lane) : -1;
  const bool valid = e >= 0;
  uint64_t peers = __ballot(valid);
#pragma unroll
  for (int bit = 0; bit < 10; ++bit) {
    const bool b = valid && ((e >> bit) & 1);
    const uint64_t bal = __ballot(b);
    peers &= b ? bal : ~bal;
  }
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int rank = __popcll(peers & lt_mask);
  const int cnt = __popcll(peers);
  const bool leader = valid && rank == 0;
  const BlockDiv bd(BM);
  const int padded = bd.pad(cnt);

  // padded sizes by group id, then an exclusive scan in place (lane owns a contiguous run)
  for (int g = lane; g < G; g += 64) pad_lds[g] = 0;
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // one wave: LDS ops complete in order
  if (leader) pad_lds[e] = padded;
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const int per = (G + 63) / 64;
  const int g0 = min(lane * per, G), g1 = min(g0 + per, G);
  int local = 0;
  for (int g = g0; g < g1; ++g) local += pad_lds[g];
  const int incl = wave_incl_sum(local);
  const int total = __builtin_amdgcn_readlane(incl, 63);
  int run = incl - local;
  for (int g = g0; g < g1; ++g) {
    const int pg = pad_lds[g];
    pad_lds[g] = run;
    run += pg;
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const int off = valid ? pad_lds[e] : 0;

  const int limit = cap * BM;
  if (valid && off + rank < limit) sorted[off + rank] = lane;
  if (leader) {
    for (int p = off + cnt; p < off + padded && p < limit; ++p) sorted[p] = n_slots;
    const int b1 = min(bd.div(off + padded), cap);
    for (int b = bd.div(off); b < b1; ++b) eids[b] = e;
  }
  if (fill_tail) {
    for (int b = bd.div(total) + lane; b < cap; b += 64) eids[b] = -1;
    for (int p = total + lane; p < limit; p += 64) sorted[p] = n_slots;
  }
  if (lane == 0) *ntpp = total;
}
