// Decode path (token batches up to a few hundred slots): grouped int4 GEMM on MFMA with the
// int4 weights dequantised in registers directly into the MFMA B operand.
//
// Tile = 16 slots (the M dimension of v_mfma_f32_16x16x32_bf16) x 16*CT columns x a K range,
// computed by one wave.
//
// B operand: lane l of a wave holds, for k-step s (32 k), the packed int32 row
// r = s*4 + (l >> 4) at columns cl .. cl + CT - 1 with cl = c0 + CT*(l & 15) (one 8- or 16-byte
// nontemporal load; 16 lanes read 16*CT*4 contiguous bytes of a row). One packed int32 is
// exactly the 8 k-values one lane contributes to a 16x16x32 MFMA, so each int32 becomes one B
// fragment: the bf16 "magic" pairs (128 + q_j, 128 + q_{j+4}) give the k order
// [0,4,1,5,2,6,3,7]; the A fragment (activations) is loaded as 8 consecutive bf16 and permuted
// to the same order (v_perm), so the dot products are unchanged. N-subtile j of a lane holds
// column cl + j.
//
// Zero point and scale are applied per quantisation group g on fp32 partial sums:
//   y[m, n] = sum_g s[g, n] * ( sum_{k in g} x[m, k] (128 + q[k, n]) - (128 + z[g, n]) X[m, g] )
// with X[m, g] = sum_{k in g} x[m, k] produced by one extra MFMA against an all-ones B.
// All weight products are exact; the only difference from the reference's dequantise-then-
// matmul is that the reference rounds each (q - z) * s to bf16 first.
//
// Kernels:
//  * gemm_decode_kernel: block = one 16-slot expert block x one column tile; KS waves split K
//    and are summed through LDS in wave order (deterministic).
//    W1 (gate_up): A = x[token(slot)], gate and up tiles, epilogue h = bf16(silu(g) * u).
//    W2 (down):    A = h[slot], epilogue ys[slot, n] = w[slot] * y (fp32).
//  * w2_token_sum_kernel (one or two tokens): block = one token x one column tile, wave i =
//    the token's routed slot i (or its shared slot); the weighted rows are summed in slot order
//    inside the block, so no separate sum kernel runs.
// Arithmetic references: src/mtp_expert_prefetch/tracing/vllm_wna16_group_plan.py:367-486,
// src/mtp_expert_prefetch/repack/gptq_unpack.py:88-131, 247-256, and the moe_sum order of
// src/mtp_expert_prefetch/tracing/vllm_router_trace.py:19801-19804.
#include <type_traits>

#include "common.h"
#include "launch.h"
#include "routing.h"

namespace {

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));

constexpr int kBM = kDecodeBlockM;  // 16 slots
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

// CT consecutive packed int32 of one qweight row (streamed once: nontemporal).
template <int CT>
MOE_DEV void load_packed(const int32_t* p, uint32_t (&w)[CT]) {
  if constexpr (CT == 2) {
    const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    w[0] = v[0];
    w[1] = v[1];
  } else {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    w[0] = v[0];
    w[1] = v[1];
    w[2] = v[2];
    w[3] = v[3];
  }
}

// Everything one lane needs for one quantisation group (SPG MFMA k-steps of 32).
template <int NP, int SPG, int CT>
struct GroupBuf {
  u32x4 a[SPG];                 // 8 consecutive bf16 activations per k-step
  uint32_t w[NP][SPG][CT];      // packed int4 rows, CT columns
  uint32_t s[NP][CT / 2];       // fp16 scale pairs of the CT columns
  uint32_t z[NP];               // packed zeros word holding the CT columns
};

// One wave: acc[p*CT + j] += A[16 rows, k0 : k0+klen] . W_p[k0 : k0+klen, cl + j] for the NP
// projections, klen a multiple of G. ap points at element (row of this lane, k0 + 8*kq);
// valid_m = false makes this lane's A row zero. A ring of NB group buffers keeps groups
// g + 1 .. g + NB - 1 in flight while group g is multiplied.
template <int NP, int SPG, int CT, int NB>
MOE_DEV void decode_tile(const ProjDev (&pj)[NP], const uint16_t* ap, bool valid_m, int NOUT,
                         int G, int k0, int klen, int cl, int kq, f32x4 (&acc)[NP * CT]) {
  constexpr int NT = NP * CT;
  const int ngw = klen / G;
  const int32_t* qp[NP];
  const uint16_t* sp[NP];
  const int32_t* zp[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    qp[p] = pj[p].qweight + (int64_t)(k0 / 8 + kq) * NOUT + cl;
    sp[p] = pj[p].scales + (int64_t)(k0 / G) * NOUT + cl;
    zp[p] = pj[p].qzeros + (int64_t)(k0 / G) * (NOUT / 8) + (cl >> 3);
  }
  const int zshift = 4 * (cl & 7);

  auto load_group = [&](GroupBuf<NP, SPG, CT>& B, int gi) {
    const int kg = gi * G;
#pragma unroll
    for (int s = 0; s < SPG; ++s)
      B.a[s] = valid_m ? ld128(ap + kg + 32 * s) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int p = 0; p < NP; ++p) {
#pragma unroll
      for (int s = 0; s < SPG; ++s) load_packed<CT>(qp[p] + (int64_t)(kg / 8 + 4 * s) * NOUT, B.w[p][s]);
      const uint32_t* s32 = reinterpret_cast<const uint32_t*>(sp[p] + (int64_t)gi * NOUT);
#pragma unroll
      for (int j = 0; j < CT / 2; ++j) B.s[p][j] = s32[j];
      B.z[p] = (uint32_t)zp[p][(int64_t)gi * (NOUT / 8)];  // shifted at use: no wait here
    }
  };

  const bf16x8_v ones = as_frag(kOnes, kOnes, kOnes, kOnes);
  auto compute_group = [&](const GroupBuf<NP, SPG, CT>& B) {
    f32x4 tmp[NT], tx = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < NT; ++t) tmp[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < SPG; ++s) {
      uint32_t xp[4];
      xpairs(B.a[s], xp);
      const bf16x8_v a = as_frag(xp[0], xp[1], xp[2], xp[3]);
      tx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ones, tx, 0, 0, 0);
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int j = 0; j < CT; ++j)
          tmp[p * CT + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, weight_frag(B.w[p][s][j]),
                                                                    tmp[p * CT + j], 0, 0, 0);
    }
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int j = 0; j < CT; ++j) {
        const uint32_t s2 = B.s[p][j >> 1];
        const float sc = f16_to_f32((j & 1) ? (s2 >> 16) : (s2 & 0xFFFFu));
        const float zb = kMagicBias + (float)((B.z[p] >> (zshift + 4 * j)) & 0xFu);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[p * CT + j][i] =
              __builtin_fmaf(sc, __builtin_fmaf(-zb, tx[i], tmp[p * CT + j][i]), acc[p * CT + j][i]);
      }
  };

  GroupBuf<NP, SPG, CT> ring[NB];
#pragma unroll
  for (int j = 0; j < NB - 1; ++j)
    if (j < ngw) load_group(ring[j], j);
  for (int g0 = 0; g0 < ngw; g0 += NB) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int g = g0 + j;
      if (g < ngw) {
        if (g + NB - 1 < ngw) load_group(ring[(j + NB - 1) % NB], g + NB - 1);
        compute_group(ring[j]);
      }
    }
  }
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, typename F>
MOE_DEV void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// decode_tile for a K range of exactly NGW groups with every load issued up front (straight-line
// code: the compiler's per-register waits let group g be multiplied as soon as it has landed
// while the later groups are still in flight).
template <int NP, int SPG, int CT, int NGW>
MOE_DEV void decode_tile_fixed(const ProjDev (&pj)[NP], const uint16_t* ap, bool valid_m,
                               int NOUT, int G, int k0, int cl, int kq, f32x4 (&acc)[NP * CT]) {
  constexpr int NT = NP * CT;
  // uniform bases + one 32-bit per-lane offset per stream (scalar-base loads)
  const uint32_t qoff = (uint32_t)(((int64_t)kq * NOUT + cl) * 4);
  const uint32_t soff = (uint32_t)(cl * 2);
  const uint32_t zoff = (uint32_t)((cl >> 3) * 4);
  const int zshift = 4 * (cl & 7);
  GroupBuf<NP, SPG, CT> ring[NGW];
  static_for<0, NGW>([&](auto gc) {
    constexpr int gi = gc.value;
    GroupBuf<NP, SPG, CT>& B = ring[gi];
    const int kg = gi * G;
#pragma unroll
    for (int s = 0; s < SPG; ++s)
      B.a[s] = valid_m ? ld128(ap + kg + 32 * s) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const char* qg = reinterpret_cast<const char*>(pj[p].qweight) +
                       (int64_t)((k0 + kg) / 8) * NOUT * 4;
#pragma unroll
      for (int s = 0; s < SPG; ++s)
        load_packed<CT>(reinterpret_cast<const int32_t*>(qg + (int64_t)(4 * s) * NOUT * 4 + qoff),
                        B.w[p][s]);
      const int g = (k0 + kg) / G;
      const char* sg = reinterpret_cast<const char*>(pj[p].scales) + (int64_t)g * NOUT * 2 + soff;
#pragma unroll
      for (int j = 0; j < CT / 2; ++j) B.s[p][j] = reinterpret_cast<const uint32_t*>(sg)[j];
      B.z[p] = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(pj[p].qzeros) +
                                                  (int64_t)g * (NOUT / 8) * 4 + zoff);
    }
  });
  const bf16x8_v ones = as_frag(kOnes, kOnes, kOnes, kOnes);
  static_for<0, NGW>([&](auto gc) {
    const GroupBuf<NP, SPG, CT>& B = ring[gc.value];
    f32x4 tmp[NT], tx = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < NT; ++t) tmp[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < SPG; ++s) {
      uint32_t xp[4];
      xpairs(B.a[s], xp);
      const bf16x8_v a = as_frag(xp[0], xp[1], xp[2], xp[3]);
      tx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ones, tx, 0, 0, 0);
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int j = 0; j < CT; ++j)
          tmp[p * CT + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, weight_frag(B.w[p][s][j]),
                                                                    tmp[p * CT + j], 0, 0, 0);
    }
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int j = 0; j < CT; ++j) {
        const uint32_t s2 = B.s[p][j >> 1];
        const float sc = f16_to_f32((j & 1) ? (s2 >> 16) : (s2 & 0xFFFFu));
        const float zb = kMagicBias + (float)((B.z[p] >> (zshift + 4 * j)) & 0xFu);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[p * CT + j][i] =
              __builtin_fmaf(sc, __builtin_fmaf(-zb, tx[i], tmp[p * CT + j][i]), acc[p * CT + j][i]);
      }
  });
}

MOE_DEV void projections(const ExpertsDev& ed, int mode, bool is_shared, ProjDev* pj) {
  if (mode == DEC_W1) {
    pj[0] = is_shared ? ed.sgate : ed.gate;
    pj[1] = is_shared ? ed.sup : ed.up;
  } else {
    pj[0] = is_shared ? ed.sdown : ed.down;
  }
}

// Block = one 16-slot expert block x (16 * CT) columns; KS waves split K evenly (each slice a
// whole number of quantisation groups) and are summed through LDS in wave order.
template <int MODE, int SPG, int KS, int CT, int NB>
__global__ __launch_bounds__(64 * KS) void gemm_decode_kernel(
    const uint16_t* __restrict__ act, ExpertsDev ed, SlotsDev sd,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ eids,
    const int32_t* __restrict__ ntpp, const float* __restrict__ topk_w,
    uint16_t* __restrict__ h_out, float* __restrict__ ys, SlotGrid sg) {
  constexpr int NP = (MODE == DEC_W1) ? 2 : 1;  // projections (gate, up) or (down)
  constexpr int NT = NP * CT;                    // MFMA N-subtiles per lane
  constexpr int TW = 16 * CT;                    // columns per block
  __shared__ float red[(KS > 1 ? KS - 1 : 1) * NT * 4 * 64];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int e, f_m, f_out[4];  // expert; A row of this lane; D rows of this lane
  if (sg.active) {
    // Slot grid (SlotGrid in launch.h): slots from the routed ids, no align pass.
    __shared__ int s_ids[kSlotGridMaxSlots];
    __shared__ float s_w[kSlotGridMaxSlots + kTopkAlignMaxTokens];
    __shared__ int s_rows[kBM];
    const int E = ed.num_experts, routed = sd.T * sd.top_k, n_slots = sd.num_slots;
    if (sg.logits) {  // every workgroup computes the same top-k of the (at most 8) tokens
      for (int t = wave; t < sd.T; t += KS) {
        const float* row = sg.logits + (int64_t)t * (E + 1);
        topk_token_lds(row, E, sd.top_k, lane, s_ids + t * sd.top_k, s_w + t * sd.top_k);
        if (n_slots > routed && lane == 0) s_w[routed + t] = 1.0f / (1.0f + expf(-row[E]));
      }
    } else if (tid < routed) {
      s_ids[tid] = sg.ids[tid];
    }
    __syncthreads();
    if (sg.logits && blockIdx.x == 0 && blockIdx.y == 0) {  // publish for W2 and the caller
      if (tid < routed) sg.ids[tid] = s_ids[tid];
      if (tid < n_slots) sg.weights[tid] = s_w[tid];
    }
    const int b = blockIdx.y;  // slot index
    auto expert_of = [&](int f) { return f < routed ? s_ids[f] : E; };
    e = expert_of(b);
    const uint64_t mask = __ballot(lane < n_slots && expert_of(lane) == e);
    const int rank_b = __popcll(mask & ((1ull << b) - 1));  // occurrences of e before slot b
    if (rank_b % kBM != 0 || !expert_ok(ed, e)) return;   // uniform over the workgroup
    const int rank = __popcll(mask & ((1ull << lane) - 1));
    if (wave == 0 && ((mask >> lane) & 1) && rank >= rank_b && rank < rank_b + kBM)
      s_rows[rank - rank_b] = lane;
    const int cnt = min(__popcll(mask) - rank_b, kBM);
    __syncthreads();
    f_m = (lane & 15) < cnt ? s_rows[lane & 15] : n_slots;
#pragma unroll
    for (int el = 0; el < 4; ++el) {
      const int r = 4 * (lane >> 4) + el;
      f_out[el] = r < cnt ? s_rows[r] : n_slots;
    }
  } else {
    // Block metadata: every load below is in bounds for any b < gridDim.y, so all of them are
    // issued together (one memory latency before the first weight load, not a chain).
    const int b = blockIdx.y;
    const int n_padded = *ntpp;
    e = eids[b];
    f_m = sorted[b * kBM + (lane & 15)];
#pragma unroll
    for (int el = 0; el < 4; ++el) f_out[el] = sorted[b * kBM + 4 * (lane >> 4) + el];
    if (b * kBM >= n_padded || !expert_ok(ed, e)) return;
  }

  const int G = ed.group;
  const int K = (MODE == DEC_W1) ? ed.hidden : ed.inter;
  const int NOUT = (MODE == DEC_W1) ? ed.inter : ed.hidden;
  const bool is_shared = (e == ed.num_experts);
  const int64_t row = is_shared ? 0 : expert_row(ed, e);
  ProjDev pj[NP];
  projections(ed, MODE, is_shared, pj);
#pragma unroll
  for (int p = 0; p < NP; ++p)
    pj[p] = proj_row(pj[p], is_shared ? 0 : ed.row_stride, row, K / 8, K / G, NOUT);

  const int kslice = K / KS;
  const int kw0 = wave * kslice;
  const int m = lane & 15, kq = lane >> 4;
  const bool valid_m = (unsigned)f_m < (unsigned)sd.num_slots;
  const int64_t arow = valid_m ? ((MODE == DEC_W1) ? (int64_t)slot_token(sd, f_m) : (int64_t)f_m) : 0;
  const int cl = blockIdx.x * TW + CT * m;  // this lane's first column

  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  if constexpr (NB < 0) {  // fixed: the wave's slice is exactly -NB groups, all loads up front
    decode_tile_fixed<NP, SPG, CT, -NB>(pj, act + arow * K + kw0 + 8 * kq, valid_m, NOUT, G, kw0,
                                        cl, kq, acc);
  } else {
    decode_tile<NP, SPG, CT, NB>(pj, act + arow * K + kw0 + 8 * kq, valid_m, NOUT, G, kw0, kslice,
                                 cl, kq, acc);
  }

  if constexpr (KS > 1) {  // cross-wave reduction: waves 1.. write, wave 0 sums in wave order
    if (wave > 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[(((wave - 1) * NT + t) * 4 + i) * 64 + lane] = acc[t][i];
    }
    __syncthreads();
    if (wave != 0) return;
    for (int w = 1; w < KS; ++w)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] += red[(((w - 1) * NT + t) * 4 + i) * 64 + lane];
  }

  // D[i][j] of a 16x16 tile: lane j + 16*(i/4), element i%4 -> row 4*(lane>>4)+el; N-subtile t
  // of projection p holds column cl + t.
#pragma unroll
  for (int el = 0; el < 4; ++el) {
    const int f = f_out[el];
    if ((unsigned)f >= (unsigned)sd.num_slots) continue;
    if constexpr (MODE == DEC_W1) {
      uint32_t hp[CT / 2];
#pragma unroll
      for (int j = 0; j < CT; j += 2)
        hp[j / 2] = pack_bf16x2(silu_f32(acc[j][el]) * acc[CT + j][el],
                                silu_f32(acc[j + 1][el]) * acc[CT + j + 1][el]);
      uint16_t* dst = h_out + (int64_t)f * NOUT + cl;
      if constexpr (CT == 2) {
        *reinterpret_cast<uint32_t*>(dst) = hp[0];
      } else {
        *reinterpret_cast<u32x2*>(dst) = u32x2{hp[0], hp[1]};
      }
    } else {
      const float w = topk_w[f];
      float* dst = ys + (int64_t)f * NOUT + cl;
      if constexpr (CT == 2) {
        *reinterpret_cast<float2*>(dst) = float2{w * acc[0][el], w * acc[1][el]};
      } else {
        *reinterpret_cast<float4*>(dst) =
            float4{w * acc[0][el], w * acc[1][el], w * acc[2][el], w * acc[3][el]};
      }
    }
  }
}

// Token-major W2 + weighted sum: block (column tile, token t); wave i < top_k handles routed slot
// t*top_k + i, wave top_k (when present) the shared slot T*top_k + t. A = h[slot] in MFMA row 0
// (the other 15 rows are zero); the block adds the waves' w[slot] * y rows in slot order.
template <int SPG, int CT, int NB>
__global__ __launch_bounds__(64 * kTokenSumMaxWaves) void w2_token_sum_kernel(
    const uint16_t* __restrict__ h, ExpertsDev ed, SlotsDev sd, const int32_t* __restrict__ ids,
    const float* __restrict__ topk_w, uint16_t* __restrict__ out) {
  constexpr int TW = 16 * CT;
  __shared__ float part[kTokenSumMaxWaves][TW];
  const int t = blockIdx.y;
  const int lane = threadIdx.x & 63, i = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const bool is_shared = i >= sd.top_k;
  const int f = is_shared ? sd.T * sd.top_k + t : t * sd.top_k + i;
  const int e = is_shared ? ed.num_experts : ids[f];
  const bool ok = is_shared || routed_ok(ed.expert_row, ed.num_experts, e);
  const int G = ed.group, K = ed.inter, NOUT = ed.hidden;
  const int m = lane & 15, kq = lane >> 4;
  const int cl = blockIdx.x * TW + CT * m;

  f32x4 acc[CT];
#pragma unroll
  for (int j = 0; j < CT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (ok) {  // wave-uniform: a dropped slot contributes nothing
    const int64_t row = is_shared ? 0 : expert_row(ed, e);
    ProjDev pj[1];
    projections(ed, DEC_W2, is_shared, pj);
    pj[0] = proj_row(pj[0], is_shared ? 0 : ed.row_stride, row, K / 8, K / G, NOUT);
    decode_tile<1, SPG, CT, NB>(pj, h + (int64_t)f * K + 8 * kq, m == 0, NOUT, G, 0, K, cl, kq,
                                acc);
  }
  const float w = ok ? topk_w[f] : 0.0f;
  if (lane < 16) {  // row 0 of the tile: lanes 0..15, element 0
#pragma unroll
    for (int j = 0; j < CT; ++j) part[i][CT * lane + j] = w * acc[j][0];
  }
  __syncthreads();
  if (i == 0 && lane < TW) {
    float s = 0.0f;
    for (int v = 0; v < nwaves; ++v) s += part[v][lane];
    const int c = blockIdx.x * TW + lane;
    out[(int64_t)t * NOUT + c] = (uint16_t)f32_to_bf16_rne(s);
  }
}

template <int MODE, int SPG, int KS, int CT, int NB>
hipError_t launch_cfg(const uint16_t* act, const ExpertsDev& ed, const SlotsDev& sd,
                      const int32_t* sorted, const int32_t* eids, const int32_t* ntpp, int cap,
                      const float* topk_w, uint16_t* h, float* ys, const SlotGrid& sg,
                      hipStream_t stream) {
  const int NOUT = (MODE == DEC_W1) ? ed.inter : ed.hidden;
  const dim3 grid(NOUT / (16 * CT), sg.active ? sd.num_slots : cap);
  hipLaunchKernelGGL((gemm_decode_kernel<MODE, SPG, KS, CT, NB>), grid, dim3(64 * KS), 0, stream,
                     act, ed, sd, sorted, eids, ntpp, topk_w, h, ys, sg);
  return hipGetLastError();
}

template <int MODE, int KS, int CT, int NB>
hipError_t launch_group(const uint16_t* act, const ExpertsDev& ed, const SlotsDev& sd,
                        const int32_t* sorted, const int32_t* eids, const int32_t* ntpp, int cap,
                        const float* topk_w, uint16_t* h, float* ys, const SlotGrid& sg,
                        hipStream_t stream) {
  switch (ed.group) {
    case 64: return launch_cfg<MODE, 2, KS, CT, NB>(act, ed, sd, sorted, eids, ntpp, cap, topk_w, h, ys, sg, stream);
    case 128: return launch_cfg<MODE, 4, KS, CT, NB>(act, ed, sd, sorted, eids, ntpp, cap, topk_w, h, ys, sg, stream);
    case 256: return launch_cfg<MODE, 8, KS, CT, NB>(act, ed, sd, sorted, eids, ntpp, cap, topk_w, h, ys, sg, stream);
    default: return hipErrorInvalidValue;
  }
}

// Any valid (waves per block, columns per lane, ring depth) configuration.
template <int MODE>
hipError_t launch_decode_cfg(const uint16_t* act, const ExpertsDev& ed, const SlotsDev& sd,
                             const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                             int cap, const float* topk_w, uint16_t* h, float* ys, int ks, int ct,
                             int nb, const SlotGrid& sg, hipStream_t stream) {
  const int K = (MODE == DEC_W1) ? ed.hidden : ed.inter;
  const int NOUT = (MODE == DEC_W1) ? ed.inter : ed.hidden;
  if ((ct != 2 && ct != 4) || NOUT % (16 * ct) != 0 || K % (ks * ed.group) != 0)
    return hipErrorInvalidValue;
  if (nb < 0 && K / (ks * ed.group) != -nb) return hipErrorInvalidValue;
#define MOE_DEC_CASE(KSV, CTV, NBV)                                                             \
  if (ks == KSV && ct == CTV && nb == NBV)                                                      \
    return launch_group<MODE, KSV, CTV, NBV>(act, ed, sd, sorted, eids, ntpp, cap, topk_w, h,  \
                                             ys, sg, stream);
  MOE_DEC_CASE(1, 2, 2) MOE_DEC_CASE(2, 2, 2) MOE_DEC_CASE(4, 2, 2) MOE_DEC_CASE(8, 2, 2)
  MOE_DEC_CASE(1, 4, 2) MOE_DEC_CASE(2, 4, 2) MOE_DEC_CASE(4, 4, 2)
  MOE_DEC_CASE(1, 2, 3) MOE_DEC_CASE(2, 2, 3) MOE_DEC_CASE(4, 2, 3)
  MOE_DEC_CASE(1, 4, 3) MOE_DEC_CASE(2, 4, 3)
  // fixed slices (nb = -groups per wave), all loads in flight at once
  MOE_DEC_CASE(1, 2, -4) MOE_DEC_CASE(2, 2, -4) MOE_DEC_CASE(4, 2, -4) MOE_DEC_CASE(8, 2, -2)
  MOE_DEC_CASE(1, 4, -4) MOE_DEC_CASE(2, 4, -4) MOE_DEC_CASE(4, 4, -4) MOE_DEC_CASE(8, 4, -2)
  MOE_DEC_CASE(2, 2, -2) MOE_DEC_CASE(4, 2, -2) MOE_DEC_CASE(2, 4, -2) MOE_DEC_CASE(4, 4, -2)
  MOE_DEC_CASE(1, 2, -2) MOE_DEC_CASE(1, 4, -2)
#undef MOE_DEC_CASE
  return hipErrorInvalidValue;
}

// Configuration by problem size (measured on MI355X, 40 Zipf-skewed layers of H 2048, I 512,
// E 256, top-8): few active expert blocks -> split K over more waves with every load of a wave
// issued up front; many -> two waves per block with a double-buffered ring. W2 (K = 512) uses
// four columns per lane: its 16-slot activation fragment is then shared by more columns.
template <int MODE>
void pick_decode_cfg(const ExpertsDev& ed, const SlotsDev& sd, int* ks, int* ct, int* nb) {
  const int K = (MODE == DEC_W1) ? ed.hidden : ed.inter;
  const int groups = K / ed.group;
  const int blocks_est = sd.num_slots < ed.num_experts ? sd.num_slots : ed.num_experts;
  auto fixed = [&](int k) {  // k waves over K, all of a wave's groups in flight
    if (groups % k == 0 && (groups / k == 4 || groups / k == 2)) {
      *ks = k;
      *nb = -(groups / k);
      return true;
    }
    return false;
  };
  if (MODE == DEC_W1) {
    *ct = 2;
    if (blocks_est < 96 && fixed(groups / 4)) return;
    *ks = 2;
    *nb = 2;
    while (*ks > 1 && K % (*ks * ed.group) != 0) *ks /= 2;
    return;
  }
  *ct = ed.hidden % 64 == 0 ? 4 : 2;
  if (blocks_est < 96 && fixed(groups / 2)) return;
  *ks = 1;
  *nb = 2;
}

template <int SPG, int CT, int NB>
hipError_t launch_token_sum(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                            const int32_t* ids, const float* topk_w, uint16_t* out,
                            hipStream_t stream) {
  const int has_shared = sd.num_slots > sd.T * sd.top_k ? 1 : 0;
  const dim3 grid(ed.hidden / (16 * CT), sd.T);
  hipLaunchKernelGGL((w2_token_sum_kernel<SPG, CT, NB>), grid, dim3(64 * (sd.top_k + has_shared)),
                     0, stream, h, ed, sd, ids, topk_w, out);
  return hipGetLastError();
}

}  // namespace

namespace {
template <int MODE>
hipError_t launch_decode_picked(const uint16_t* act, const ExpertsDev& ed, const SlotsDev& sd,
                                const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                                int cap, const float* topk_w, uint16_t* h, float* ys,
                                const SlotGrid& sg, hipStream_t stream) {
  int ks, ct, nb;
  pick_decode_cfg<MODE>(ed, sd, &ks, &ct, &nb);
  hipError_t e = launch_decode_cfg<MODE>(act, ed, sd, sorted, eids, ntpp, cap, topk_w, h, ys, ks,
                                         ct, nb, sg, stream);
  if (e == hipErrorInvalidValue)  // shape outside the tuned set: one wave, double-buffered
    e = launch_decode_cfg<MODE>(act, ed, sd, sorted, eids, ntpp, cap, topk_w, h, ys, 1, 2, 2, sg,
                                stream);
  return e;
}
}  // namespace

hipError_t launch_w1_decode_mfma(const uint16_t* x, const ExpertsDev& ed, const SlotsDev& sd,
                                 const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                                 int cap, uint16_t* h, hipStream_t stream) {
  return launch_decode_picked<DEC_W1>(x, ed, sd, sorted, eids, ntpp, cap, nullptr, h, nullptr,
                                      SlotGrid{0, nullptr, nullptr, nullptr}, stream);
}

hipError_t launch_w2_decode_mfma(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                                 const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                                 int cap, const float* topk_w, float* ys, hipStream_t stream) {
  return launch_decode_picked<DEC_W2>(h, ed, sd, sorted, eids, ntpp, cap, topk_w, nullptr, ys,
                                      SlotGrid{0, nullptr, nullptr, nullptr}, stream);
}

hipError_t launch_w1_decode_slotgrid(const uint16_t* x, const ExpertsDev& ed, const SlotsDev& sd,
                                     const SlotGrid& sg, uint16_t* h, hipStream_t stream) {
  if (!sg.active || !slot_grid_fits(sd.T, sd.top_k, sd.num_slots > sd.T * sd.top_k ? 1 : 0))
    return hipErrorInvalidValue;
  return launch_decode_picked<DEC_W1>(x, ed, sd, nullptr, nullptr, nullptr, 0, nullptr, h,
                                      nullptr, sg, stream);
}

hipError_t launch_w2_decode_slotgrid(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                                     const SlotGrid& sg, float* ys, hipStream_t stream) {
  if (!sg.active || sg.logits ||
      !slot_grid_fits(sd.T, sd.top_k, sd.num_slots > sd.T * sd.top_k ? 1 : 0))
    return hipErrorInvalidValue;
  return launch_decode_picked<DEC_W2>(h, ed, sd, nullptr, nullptr, nullptr, 0, sg.weights, nullptr,
                                      ys, sg, stream);
}

bool w2_token_sum_fits(const ExpertsDev& ed, const SlotsDev& sd) {
  const int has_shared = sd.num_slots > sd.T * sd.top_k ? 1 : 0;
  return sd.T >= 1 && sd.T <= kTokenSumMaxTokens && sd.top_k + has_shared <= kTokenSumMaxWaves &&
         ed.hidden % 32 == 0 && ed.inter % ed.group == 0;
}

hipError_t launch_w2_token_sum(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                               const int32_t* ids, const float* topk_w, uint16_t* out,
                               hipStream_t stream) {
  if (!w2_token_sum_fits(ed, sd)) return hipErrorInvalidValue;
  switch (ed.group) {  // ring depth: all groups of K = 512 in flight at once
    case 64: return launch_token_sum<2, 2, 8>(h, ed, sd, ids, topk_w, out, stream);
    case 128: return launch_token_sum<4, 2, 4>(h, ed, sd, ids, topk_w, out, stream);
    case 256: return launch_token_sum<8, 2, 2>(h, ed, sd, ids, topk_w, out, stream);
    default: return hipErrorInvalidValue;
  }
}
