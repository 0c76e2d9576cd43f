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
// fragment: bf16 "magic" pairs 128 + q built from two byte planes of the word (weight_frag)
// give the k order [0,2,4,6,1,3,5,7]; the A fragment (activations) is loaded as 8 consecutive
// bf16 and permuted to the same order (v_perm), so the dot products are unchanged. N-subtile j
// of a lane holds column cl + j.
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
//  * w2_token_sum_kernel (up to 8 tokens): block = one token x one column tile, wave i =
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
constexpr int kW2Groups = 4;        // fused W2: 64-column groups of the output per wave
constexpr uint32_t kOnes = 0x3F803F80u;

enum { DEC_W1 = 1, DEC_W2 = 2 };

MOE_DEV bf16x8_v as_frag(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u32x4 v = {a, b, c, d};
  return __builtin_bit_cast(bf16x8_v, v);
}

// B fragment of one packed int32 (8 k of one column) in the k order [0,2,4,6,1,3,5,7]: the
// nibbles are split into two byte planes (even nibbles q0 q2 q4 q6, odd nibbles q1 q3 q5 q7),
// and each bf16 pair (128 + q_a, 128 + q_b) is one byte permute of a plane with the magic
// exponent byte 0x43: 7 VALU operations per word.
constexpr uint32_t kMagicBytes = 0x43434343u;
MOE_DEV bf16x8_v weight_frag(uint32_t w) {
  const uint32_t ev = w & 0x0F0F0F0Fu;         // bytes q0, q2, q4, q6
  const uint32_t od = (w >> 4) & 0x0F0F0F0Fu;  // bytes q1, q3, q5, q7
  return as_frag(__builtin_amdgcn_perm(ev, kMagicBytes, 0x00050004u),   // (q0, q2)
                 __builtin_amdgcn_perm(ev, kMagicBytes, 0x00070006u),   // (q4, q6)
                 __builtin_amdgcn_perm(od, kMagicBytes, 0x00050004u),   // (q1, q3)
                 __builtin_amdgcn_perm(od, kMagicBytes, 0x00070006u));  // (q5, q7)
}

// A fragment of 8 consecutive bf16 activations (d0 = x0|x1<<16, ..., d3 = x6|x7<<16) in the
// k order of weight_frag: (x0,x2), (x4,x6), (x1,x3), (x5,x7).
MOE_DEV bf16x8_v act_frag(const u32x4 d) {
  return as_frag(__builtin_amdgcn_perm(d[1], d[0], 0x05040100u),
                 __builtin_amdgcn_perm(d[3], d[2], 0x05040100u),
                 __builtin_amdgcn_perm(d[1], d[0], 0x07060302u),
                 __builtin_amdgcn_perm(d[3], d[2], 0x07060302u));
}

// Everything one lane needs for one quantisation group (SPG MFMA k-steps of 32): activations
// and packed weights, and the group's scales and zeros.
template <int NP, int SPG, int CT>
struct GroupAW {
  u32x4 a[SPG];                 // 8 consecutive bf16 activations per k-step
  uint32_t w[NP][SPG][CT];      // packed int4 rows, CT columns
};
template <int NP, int CT>
struct GroupSZ {
  uint32_t s[NP][CT / 2];       // fp16 scale pairs of the CT columns
  uint32_t z[NP];               // packed zeros word holding the CT columns
};
template <int NP, int SPG, int CT>
struct GroupBuf {
  GroupAW<NP, SPG, CT> aw;
  GroupSZ<NP, CT> sz;
};

// A operand of one lane: resource over the activation rows and the byte offset of
// (this lane's row, first k of the wave's slice + 8 * kq), kOutOfRange for a padding row.
struct AView {
  __amdgpu_buffer_rsrc_t r;
  uint32_t off;
};

// One wave's view of a K slice [k0, k0 + NGW*G) of the NP projections at columns
// cl .. cl + CT - 1. Every load is a buffer load from a uniform resource with a 32-bit lane
// offset; group gi >= ngw (a ring stage past the slice) and padding rows load zeros with no
// memory access, so the same instructions run on every path.
template <int NP, int SPG, int CT>
struct DecodeTile {
  __amdgpu_buffer_rsrc_t qr[NP], sr[NP], zr[NP];
  AView a;
  uint32_t qoff, soff, zoff;        // lane offsets of group 0
  uint32_t qgrp, sgrp, zgrp, qrow;  // bytes per group (qweight, scales, zeros), per packed row
  int G, ngw, zshift;

  MOE_DEV DecodeTile(const ProjDev (&pj)[NP], AView av, int NOUT, int G_, int k0, int klen,
                     int cl, int kq)
      : a(av), G(G_), ngw(klen / G_), zshift(4 * (cl & 7)) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      qr[p] = buf_rsrc(pj[p].qweight);
      sr[p] = buf_rsrc(pj[p].scales);
      zr[p] = buf_rsrc(pj[p].qzeros);
    }
    qrow = (uint32_t)NOUT * 4u;
    qoff = (uint32_t)(k0 / 8 + kq) * qrow + (uint32_t)cl * 4u;
    soff = (uint32_t)((k0 / G) * NOUT + cl) * 2u;
    zoff = (uint32_t)((k0 / G) * (NOUT / 8) + (cl >> 3)) * 4u;
    qgrp = (uint32_t)(G / 8) * qrow;
    sgrp = (uint32_t)NOUT * 2u;
    zgrp = (uint32_t)(NOUT / 8) * 4u;
  }

  MOE_DEV void load_aw(GroupAW<NP, SPG, CT>& B, int gi) const {
    const uint32_t oob = gi < ngw ? 0u : kOutOfRange;
    const uint32_t ug = (uint32_t)gi;
#pragma unroll
    for (int s = 0; s < SPG; ++s) B.a[s] = buf_ld128(a.r, (a.off + (ug * G + 32 * s) * 2u) | oob);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
#pragma unroll
      for (int s = 0; s < SPG; ++s) {  // weights are streamed once: nontemporal
        const uint32_t o = (qoff + ug * qgrp + (uint32_t)(4 * s) * qrow) | oob;
        if constexpr (CT == 2) {
          const u32x2 v = buf_ld64<kBufNontemporal>(qr[p], o);
          B.w[p][s][0] = v[0];
          B.w[p][s][1] = v[1];
        } else {
          const u32x4 v = buf_ld128<kBufNontemporal>(qr[p], o);
#pragma unroll
          for (int j = 0; j < 4; ++j) B.w[p][s][j] = v[j];
        }
      }
    }
  }

  MOE_DEV void load_sz(GroupSZ<NP, CT>& B, int gi) const {
    const uint32_t oob = gi < ngw ? 0u : kOutOfRange;
    const uint32_t ug = (uint32_t)gi;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      if constexpr (CT == 2) {
        B.s[p][0] = buf_ld32(sr[p], (soff + ug * sgrp) | oob);
      } else {
        const u32x2 v = buf_ld64(sr[p], (soff + ug * sgrp) | oob);
        B.s[p][0] = v[0];
        B.s[p][1] = v[1];
      }
      B.z[p] = buf_ld32(zr[p], (zoff + ug * zgrp) | oob);  // shifted at use: no wait here
    }
  }

  MOE_DEV void load(GroupBuf<NP, SPG, CT>& B, int gi) const {
    load_aw(B.aw, gi);
    load_sz(B.sz, gi);
  }

  // acc[p*CT + j] += s * (sum_k x (128 + q) - (128 + z) * sum_k x) over one group. A group
  // past the slice loaded zeros (scale 0) and adds +0.
  MOE_DEV void compute(const GroupBuf<NP, SPG, CT>& B, f32x4 (&acc)[NP * CT]) const {
    compute(B.aw, B.sz, acc);
  }
  MOE_DEV void compute(const GroupAW<NP, SPG, CT>& B, const GroupSZ<NP, CT>& Z,
                       f32x4 (&acc)[NP * CT]) const {
    constexpr int NT = NP * CT;
    const bf16x8_v ones = as_frag(kOnes, kOnes, kOnes, kOnes);
    f32x4 tmp[NT], tx = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < NT; ++t) tmp[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < SPG; ++s) {
      const bf16x8_v av = act_frag(B.a[s]);
      tx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, ones, tx, 0, 0, 0);
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int j = 0; j < CT; ++j)
          tmp[p * CT + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, weight_frag(B.w[p][s][j]),
                                                                    tmp[p * CT + j], 0, 0, 0);
    }
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int j = 0; j < CT; ++j) {
        const uint32_t s2 = Z.s[p][j >> 1];
        const float sc = f16_to_f32((j & 1) ? (s2 >> 16) : (s2 & 0xFFFFu));
        const float zb = kMagicBias + (float)((Z.z[p] >> (zshift + 4 * j)) & 0xFu);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[p * CT + j][i] =
              __builtin_fmaf(sc, __builtin_fmaf(-zb, tx[i], tmp[p * CT + j][i]), acc[p * CT + j][i]);
      }
  }
};

// One wave: acc[p*CT + j] += A[16 rows, k0 : k0+klen] . W_p[k0 : k0+klen, cl + j] for the NP
// projections, klen a multiple of G. A ring of NB group buffers keeps groups g + 1 .. g + NB - 1
// in flight while group g is multiplied; the loop body issues the same loads on every pass
// (stages past the slice read zeros), so each wait is for exactly the group about to be used.
template <int NP, int SPG, int CT, int NB>
MOE_DEV void decode_tile(const DecodeTile<NP, SPG, CT>& tile, f32x4 (&acc)[NP * CT]) {
  GroupBuf<NP, SPG, CT> ring[NB];
#pragma unroll
  for (int j = 0; j < NB - 1; ++j) tile.load(ring[j], j);
  for (int g0 = 0; g0 < tile.ngw; g0 += NB) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      tile.load(ring[(j + NB - 1) % NB], g0 + j + NB - 1);
      // keep the stage's loads ahead of the wait for group g0 + j (the scheduler would sink
      // them below it, leaving one group in flight)
      __builtin_amdgcn_sched_barrier(0);
      tile.compute(ring[j], acc);
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

// decode_tile for a K slice of exactly NGW groups as straight-line code: every group's scales
// and zeros are loaded first, then a ring of DEPTH activation/weight buffers (DEPTH == NGW: all
// loads up front). Without a loop back-edge each wait is for exactly the group about to be
// multiplied, whatever the ring depth.
template <int NP, int SPG, int CT, int NGW, int DEPTH>
MOE_DEV void decode_tile_static(const DecodeTile<NP, SPG, CT>& tile, f32x4 (&acc)[NP * CT]) {
  static_assert(DEPTH >= 1 && DEPTH <= NGW, "ring depth within the slice");
  GroupSZ<NP, CT> sz[NGW];
  static_for<0, NGW>([&](auto gc) { tile.load_sz(sz[gc.value], gc.value); });
  GroupAW<NP, SPG, CT> ring[DEPTH];
  static_for<0, DEPTH - 1>([&](auto gc) { tile.load_aw(ring[gc.value], gc.value); });
  static_for<0, NGW>([&](auto gc) {
    constexpr int g = gc.value;
    if constexpr (g + DEPTH - 1 < NGW) {
      __builtin_amdgcn_s_setprio(2);  // issue the stage's loads ahead of the other waves' math
      tile.load_aw(ring[(g + DEPTH - 1) % DEPTH], g + DEPTH - 1);
      __builtin_amdgcn_s_setprio(0);
    }
    __builtin_amdgcn_sched_barrier(0);  // this stage's loads before the wait for group g
    tile.compute(ring[g % DEPTH], sz[g], acc);
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
// NB > 0 and NGW == 0: runtime loop over the wave's groups with an NB-deep ring; NB < 0: a
// slice of exactly -NB groups, all loaded up front; NGW > 0: a slice of exactly NGW groups with
// an NB-deep ring, unrolled.
// FW2 (W1 on the slot grid, CT == 2): W2 fused in. The block's 32 h columns are the K rows
// [32 x, 32 x + 32) of the down projection (inside one quantisation group); after the W1
// epilogue every wave multiplies the block's h rows (from LDS) by its kW2Groups x 64 output
// columns and writes the weighted fp32 partial rows ys[slot][x][n] (partial_sum adds them).
// The workgroup of a dropped expert writes zero rows, so every partial row is written.
template <int MODE, int SPG, int KS, int CT, int NB, int NGW = 0, bool FW2 = false>
__global__ __launch_bounds__(64 * KS) void gemm_decode_kernel(
    const uint16_t* __restrict__ act, ExpertsDev ed, SlotsDev sd,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ eids,
    const int32_t* __restrict__ ntpp, const float* __restrict__ topk_w,
    uint16_t* __restrict__ h_out, float* __restrict__ ys, SlotGrid sg) {
  constexpr int NP = (MODE == DEC_W1) ? 2 : 1;  // projections (gate, up) or (down)
  constexpr int NT = NP * CT;                    // MFMA N-subtiles per lane
  constexpr int TW = 16 * CT;                    // columns per block
  static_assert(!FW2 || (MODE == DEC_W1 && CT == 2), "fused W2: W1 blocks of 32 columns");
  __shared__ float red[(KS > 1 ? KS - 1 : 1) * NT * 4 * 64];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar K-slice offsets
  int e, f_m, f_out[4];  // expert; A row of this lane; D rows of this lane
  __shared__ float s_w[kSlotGridMaxSlots + kTopkAlignMaxTokens];  // slot grid: routed weights
  if (sg.active) {
    // Slot grid (SlotGrid in launch.h): slots from the routed ids, no align pass.
    __shared__ int s_ids[kSlotGridMaxSlots];
    __shared__ int s_rows[kBM];
    const int E = ed.num_experts, routed = sd.T * sd.top_k, n_slots = sd.num_slots;
    if (sg.logits) {  // every workgroup computes the same top-k of the (at most 8) tokens
      for (int t = wave; t < sd.T; t += KS) {
        const float* row = sg.logits + (int64_t)t * (E + 1);
        const bool shared = n_slots > routed;  // row[E] is the shared gate's logit
        const float g = __uint_as_float(
            buf_ld32(buf_rsrc(row, (uint32_t)(E + (shared ? 1 : 0)) * 4u), (uint32_t)E * 4u));
        topk_token_lds_any(row, E, sd.top_k, lane, s_ids + t * sd.top_k, s_w + t * sd.top_k);
        if (shared && lane == 0) s_w[routed + t] = 1.0f / (1.0f + expf(-g));
      }
    } else {
      if (tid < routed) s_ids[tid] = sg.ids[tid];
      if (FW2 && tid < n_slots) s_w[tid] = sg.weights[tid];
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
    if constexpr (!FW2) {
      if (rank_b % kBM != 0 || !expert_ok(ed, e)) return;  // uniform over the workgroup
    } else {
      if (rank_b % kBM != 0) return;  // a dropped expert still writes its (zero) partial rows
    }
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
    if constexpr (FW2) {
      if (!expert_ok(ed, e)) {  // dropped slots: zero partial rows for this column block
        const int H = ed.hidden, q4 = H / 4;
        for (int i = tid; i < cnt * q4; i += blockDim.x)
          *reinterpret_cast<float4*>(ys + ((int64_t)s_rows[i / q4] * gridDim.x + blockIdx.x) * H +
                                     4 * (i % q4)) = float4{0.f, 0.f, 0.f, 0.f};
        return;
      }
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
  const uint32_t arow = valid_m ? ((MODE == DEC_W1) ? (uint32_t)slot_token(sd, f_m) : (uint32_t)f_m) : 0u;
  const uint32_t a_rows = (MODE == DEC_W1) ? (uint32_t)sd.T : (uint32_t)sd.num_slots;
  const AView av{buf_rsrc(act, a_rows * (uint32_t)K * 2u),
                 valid_m ? (arow * (uint32_t)K + (uint32_t)(kw0 + 8 * kq)) * 2u : kOutOfRange};
  const int cl = blockIdx.x * TW + CT * m;  // this lane's first column
  const DecodeTile<NP, SPG, CT> tile(pj, av, NOUT, G, kw0, kslice, cl, kq);

  // FW2: the down projection's words, scales and zeros for this wave's output columns, loaded
  // with the W1 stream. Lane (c = lane & 15, kq) takes packed row x * 4 + kq (TW == 32) and the
  // 4 columns n0 + 4 c .. + 3 of each 64-column group: word t is the B fragment of MFMA tile t.
  [[maybe_unused]] u32x4 w2q[FW2 ? kW2Groups : 1];
  [[maybe_unused]] u32x2 w2s[FW2 ? kW2Groups : 1];
  [[maybe_unused]] uint32_t w2z[FW2 ? kW2Groups : 1];
  [[maybe_unused]] int w2n0 = 0;
  if constexpr (FW2) {
    const int I = ed.inter, H = ed.hidden;
    ProjDev pd[1];
    projections(ed, DEC_W2, is_shared, pd);
    pd[0] = proj_row(pd[0], is_shared ? 0 : ed.row_stride, row, I / 8, I / G, H);
    const int k0 = blockIdx.x * TW, g2 = k0 / G;
    w2n0 = wave * (kW2Groups * 64) + 4 * m;
    const __amdgpu_buffer_rsrc_t q2 = buf_rsrc(pd[0].qweight), s2 = buf_rsrc(pd[0].scales),
                                 z2 = buf_rsrc(pd[0].qzeros);
#pragma unroll
    for (int gi = 0; gi < kW2Groups; ++gi) {
      const uint32_t n = (uint32_t)(w2n0 + 64 * gi);
      w2q[gi] = buf_ld128<kBufNontemporal>(q2, ((uint32_t)(k0 / 8 + kq) * (uint32_t)H + n) * 4u);
      w2s[gi] = buf_ld64(s2, ((uint32_t)g2 * (uint32_t)H + n) * 2u);
      w2z[gi] = buf_ld32(z2, ((uint32_t)g2 * (uint32_t)(H / 8) + (n >> 3)) * 4u);
    }
    __builtin_amdgcn_sched_barrier(0);  // issued here, with the W1 stream, not at their use
  }

  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  if constexpr (NB < 0) {  // fixed: the wave's slice is exactly -NB groups, all loads up front
    decode_tile_static<NP, SPG, CT, -NB, -NB>(tile, acc);
  } else if constexpr (NGW > 0) {
    decode_tile_static<NP, SPG, CT, NGW, NB>(tile, acc);
  } else {
    decode_tile<NP, SPG, CT, NB>(tile, acc);
  }

  if constexpr (KS > 1) {  // cross-wave reduction: waves 1.. write, wave 0 sums in wave order
    if (wave > 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[(((wave - 1) * NT + t) * 4 + i) * 64 + lane] = acc[t][i];
    }
    __syncthreads();
    if constexpr (!FW2) {
      if (wave != 0) return;
      for (int w = 1; w < KS; ++w)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[t][i] += red[(((w - 1) * NT + t) * 4 + i) * 64 + lane];
    } else if (wave == 0) {
      for (int w = 1; w < KS; ++w)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[t][i] += red[(((w - 1) * NT + t) * 4 + i) * 64 + lane];
    }
  }

  if constexpr (FW2) {
    // h rows of the block (bf16, as W1 writes them) into LDS as [16 rows][16 column pairs]
    __shared__ uint32_t s_h[kBM * 16];
    if (wave == 0) {
#pragma unroll
      for (int el = 0; el < 4; ++el) {
        const bool real = (unsigned)f_out[el] < (unsigned)sd.num_slots;
        s_h[(4 * kq + el) * 16 + m] =
            real ? pack_bf16x2(silu_f32(acc[0][el]) * acc[CT][el],
                               silu_f32(acc[1][el]) * acc[CT + 1][el])
                 : 0u;
      }
    }
    __syncthreads();
    // A: row m, k 8 kq .. 8 kq + 7 of the block's 32 h columns; X[row] = sum of the row's h
    const u32x4 hv = {s_h[m * 16 + 4 * kq], s_h[m * 16 + 4 * kq + 1], s_h[m * 16 + 4 * kq + 2],
                      s_h[m * 16 + 4 * kq + 3]};
    const bf16x8_v av2 = act_frag(hv);
    const f32x4 tx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        av2, as_frag(kOnes, kOnes, kOnes, kOnes), f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    const int H = ed.hidden, nct = gridDim.x;
    float wrow[4];
#pragma unroll
    for (int el = 0; el < 4; ++el)
      wrow[el] = (unsigned)f_out[el] < (unsigned)sd.num_slots ? s_w[f_out[el]] : 0.0f;
#pragma unroll
    for (int gi = 0; gi < kW2Groups; ++gi) {
      f32x4 d[4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        d[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av2, weight_frag(w2q[gi][t]),
                                                       f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
      const int n = w2n0 + 64 * gi;
      float sc[4], zb[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        sc[t] = f16_to_f32(t & 2 ? ((t & 1) ? (w2s[gi][1] >> 16) : (w2s[gi][1] & 0xFFFFu))
                                 : ((t & 1) ? (w2s[gi][0] >> 16) : (w2s[gi][0] & 0xFFFFu)));
        zb[t] = kMagicBias + (float)((w2z[gi] >> (4 * ((n & 7) + t))) & 0xFu);
      }
#pragma unroll
      for (int el = 0; el < 4; ++el) {
        const int f = f_out[el];
        if ((unsigned)f >= (unsigned)sd.num_slots) continue;
        float4 v;
        v.x = wrow[el] * (sc[0] * __builtin_fmaf(-zb[0], tx[el], d[0][el]));
        v.y = wrow[el] * (sc[1] * __builtin_fmaf(-zb[1], tx[el], d[1][el]));
        v.z = wrow[el] * (sc[2] * __builtin_fmaf(-zb[2], tx[el], d[2][el]));
        v.w = wrow[el] * (sc[3] * __builtin_fmaf(-zb[3], tx[el], d[3][el]));
        *reinterpret_cast<float4*>(ys + ((int64_t)f * nct + blockIdx.x) * H + n) = v;
      }
    }
    return;
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
  const int lane = threadIdx.x & 63;
  const int i = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // uniform: the slot's
                                                                         // resources in SGPRs
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
    const AView av{buf_rsrc(h, (uint32_t)sd.num_slots * (uint32_t)K * 2u),
                   m == 0 ? ((uint32_t)f * (uint32_t)K + (uint32_t)(8 * kq)) * 2u : kOutOfRange};
    const DecodeTile<1, SPG, CT> tile(pj, av, NOUT, G, 0, K, cl, kq);
    if constexpr (NB < 0) {  // K is exactly -NB groups: every load up front
      decode_tile_static<1, SPG, CT, -NB, -NB>(tile, acc);
    } else {
      decode_tile<1, SPG, CT, NB>(tile, acc);
    }
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

// Every buffer offset the decode kernels form (activation rows, one expert's qweight, scales
// and zeros) stays below kOutOfRange.
bool decode_offsets_fit(const ExpertsDev& ed, const SlotsDev& sd) {
  const int64_t lim = kOutOfRange;
  return (int64_t)sd.T * ed.hidden * 2 < lim && (int64_t)sd.num_slots * ed.inter * 2 < lim &&
         (int64_t)ed.hidden * ed.inter / 2 < lim;
}

template <int MODE, int SPG, int KS, int CT, int NB, int NGW = 0>
hipError_t launch_cfg(const uint16_t* act, const ExpertsDev& ed, const SlotsDev& sd,
                      const int32_t* sorted, const int32_t* eids, const int32_t* ntpp, int cap,
                      const float* topk_w, uint16_t* h, float* ys, const SlotGrid& sg,
                      hipStream_t stream) {
  const int NOUT = (MODE == DEC_W1) ? ed.inter : ed.hidden;
  if (!decode_offsets_fit(ed, sd)) return hipErrorInvalidValue;
  const dim3 grid(NOUT / (16 * CT), sg.active ? sd.num_slots : cap);
  hipLaunchKernelGGL((gemm_decode_kernel<MODE, SPG, KS, CT, NB, NGW>), grid, dim3(64 * KS), 0,
                     stream, act, ed, sd, sorted, eids, ntpp, topk_w, h, ys, sg);
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

// Any valid (waves per block, columns per lane, ring depth[, groups per wave]) configuration.
// ngw > 0 selects the unrolled ring over exactly ngw groups per wave (group size 128 only).
template <int MODE>
hipError_t launch_decode_cfg(const uint16_t* act, const ExpertsDev& ed, const SlotsDev& sd,
                             const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                             int cap, const float* topk_w, uint16_t* h, float* ys, int ks, int ct,
                             int nb, int ngw, const SlotGrid& sg, hipStream_t stream) {
  const int K = (MODE == DEC_W1) ? ed.hidden : ed.inter;
  const int NOUT = (MODE == DEC_W1) ? ed.inter : ed.hidden;
  if ((ct != 2 && ct != 4) || NOUT % (16 * ct) != 0 || K % (ks * ed.group) != 0)
    return hipErrorInvalidValue;
  if (nb < 0 && K / (ks * ed.group) != -nb) return hipErrorInvalidValue;
  if (ngw > 0) {
    if (ed.group != 128 || K / (ks * ed.group) != ngw || nb < 1 || nb > ngw)
      return hipErrorInvalidValue;
#define MOE_DEC_STATIC(KSV, CTV, NBV, NGWV)                                                     \
    if (ks == KSV && ct == CTV && nb == NBV && ngw == NGWV)                                     \
      return launch_cfg<MODE, 4, KSV, CTV, NBV, NGWV>(act, ed, sd, sorted, eids, ntpp, cap,     \
                                                      topk_w, h, ys, sg, stream);
    MOE_DEC_STATIC(4, 4, 2, 4) MOE_DEC_STATIC(4, 4, 3, 4) MOE_DEC_STATIC(4, 2, 2, 4)
    MOE_DEC_STATIC(4, 2, 3, 4) MOE_DEC_STATIC(2, 2, 2, 8) MOE_DEC_STATIC(2, 2, 3, 8)
    MOE_DEC_STATIC(2, 4, 2, 8) MOE_DEC_STATIC(2, 4, 3, 8) MOE_DEC_STATIC(1, 4, 2, 4)
    MOE_DEC_STATIC(1, 4, 3, 4) MOE_DEC_STATIC(1, 2, 2, 4) MOE_DEC_STATIC(1, 2, 3, 4)
#undef MOE_DEC_STATIC
    return hipErrorInvalidValue;
  }
#define MOE_DEC_CASE(KSV, CTV, NBV)                                                             \
  if (ks == KSV && ct == CTV && nb == NBV)                                                      \
    return launch_group<MODE, KSV, CTV, NBV>(act, ed, sd, sorted, eids, ntpp, cap, topk_w, h,  \
                                             ys, sg, stream);
  MOE_DEC_CASE(1, 2, 2) MOE_DEC_CASE(2, 2, 2) MOE_DEC_CASE(4, 2, 2) MOE_DEC_CASE(8, 2, 2)
  MOE_DEC_CASE(1, 4, 2) MOE_DEC_CASE(2, 4, 2) MOE_DEC_CASE(4, 4, 2)
  // fixed slices (nb = -groups per wave), all loads in flight at once
  MOE_DEC_CASE(1, 2, -4) MOE_DEC_CASE(2, 2, -4) MOE_DEC_CASE(4, 2, -4) MOE_DEC_CASE(8, 2, -2)
  MOE_DEC_CASE(1, 4, -4) MOE_DEC_CASE(2, 4, -4) MOE_DEC_CASE(4, 4, -4) MOE_DEC_CASE(8, 4, -2)
  MOE_DEC_CASE(2, 2, -2) MOE_DEC_CASE(4, 2, -2) MOE_DEC_CASE(2, 4, -2) MOE_DEC_CASE(4, 4, -2)
  MOE_DEC_CASE(1, 2, -2) MOE_DEC_CASE(1, 4, -2)
#undef MOE_DEC_CASE
  return hipErrorInvalidValue;
}

// Configuration by problem size (measured on MI355X, 40 Zipf-skewed layers of H 2048, I 512,
// E 256, top-8, group 128; num_slots 8 / 64 / 256 / 512 at batch 1 / 8 / 32 / 64):
//   W1: up to 16 slots, 8 waves over K with both of a wave's groups loaded up front (7.2 us);
//       up to 384 slots, four waves over K, two columns per lane, unrolled 2-deep ring over the
//       wave's 4 groups (13.6 us at 64 slots, 23.0 us at 256); beyond, the same with four
//       columns per lane (31.3 us at 512).
//   W2 (K = 512, four columns per lane): two waves over K with both groups up front (7.9 us at
//       64 slots, 17.1 us at 512), except between 128 and 384 slots where one wave with an
//       unrolled 2-deep ring over its 4 groups is faster (12.6 vs 13.1 us).
// The unrolled rings exist for group size 128 and the slices above; other shapes use the
// runtime ring with the same waves and columns.
template <int MODE>
void pick_decode_cfg(const ExpertsDev& ed, const SlotsDev& sd, int* ks, int* ct, int* nb,
                     int* ngw) {
  *ngw = 0;
  const int K = (MODE == DEC_W1) ? ed.hidden : ed.inter;
  const int groups = K / ed.group;
  const int slots = sd.num_slots;
  auto fixed = [&](int k) {  // k waves over K, all of a wave's groups in flight
    if (k >= 1 && groups % k == 0 && (groups / k == 4 || groups / k == 2)) {
      *ks = k;
      *nb = -(groups / k);
      return true;
    }
    return false;
  };
  auto ring = [&](int k, int unrolled_groups) {  // k waves over K, 2-deep ring
    *ks = k;
    *nb = 2;
    while (*ks > 1 && K % (*ks * ed.group) != 0) *ks /= 2;
    if (ed.group == 128 && *ks == k && K == k * 128 * unrolled_groups) *ngw = unrolled_groups;
  };
  if (MODE == DEC_W1) {
    *ct = 2;
    if (slots <= 16 && fixed(groups / 2)) return;
    if (slots > 384 && ed.inter % 64 == 0) *ct = 4;
    return ring(4, 4);
  }
  *ct = ed.hidden % 64 == 0 ? 4 : 2;
  if ((slots <= 128 || slots > 384) && fixed(groups / 2)) return;
  ring(1, 4);
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
  int ks, ct, nb, ngw;
  pick_decode_cfg<MODE>(ed, sd, &ks, &ct, &nb, &ngw);
  hipError_t e = launch_decode_cfg<MODE>(act, ed, sd, sorted, eids, ntpp, cap, topk_w, h, ys, ks,
                                         ct, nb, ngw, sg, stream);
  if (e == hipErrorInvalidValue)  // shape outside the tuned set: one wave, double-buffered
    e = launch_decode_cfg<MODE>(act, ed, sd, sorted, eids, ntpp, cap, topk_w, h, ys, 1, 2, 2, 0,
                                sg, stream);
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

// W1 + fused W2 partials on the slot grid: group 128, one wave per two groups of K = hidden
// (all loads up front), and hidden = 4 x 64 output columns per wave.
bool w1w2_fused_fits(const ExpertsDev& ed, const SlotsDev& sd) {
  const int H = ed.hidden, ks = H / 256;
  return ed.group == 128 && H % 256 == 0 && (ks == 2 || ks == 4 || ks == 8) &&
         ed.inter % 32 == 0 && decode_offsets_fit(ed, sd) &&
         slot_grid_fits(sd.T, sd.top_k, sd.num_slots > sd.T * sd.top_k ? 1 : 0) &&
         (int64_t)sd.num_slots * (ed.inter / 32) * H * 4 < kOutOfRange;
}

hipError_t launch_w1w2_slotgrid(const uint16_t* x, const ExpertsDev& ed, const SlotsDev& sd,
                                const SlotGrid& sg, float* part, hipStream_t stream) {
  if (!sg.active || !w1w2_fused_fits(ed, sd)) return hipErrorInvalidValue;
  const dim3 grid(ed.inter / 32, sd.num_slots);
  switch (ed.hidden / 256) {
#define MOE_W1W2(KSV)                                                                          \
  case KSV:                                                                                    \
    hipLaunchKernelGGL((gemm_decode_kernel<DEC_W1, 4, KSV, 2, -2, 0, true>), grid,             \
                       dim3(64 * KSV), 0, stream, x, ed, sd, nullptr, nullptr, nullptr,        \
                       nullptr, nullptr, part, sg);                                            \
    return hipGetLastError();
    MOE_W1W2(2) MOE_W1W2(4) MOE_W1W2(8)
#undef MOE_W1W2
    default: return hipErrorInvalidValue;
  }
}

bool w2_token_sum_fits(const ExpertsDev& ed, const SlotsDev& sd) {
  const int has_shared = sd.num_slots > sd.T * sd.top_k ? 1 : 0;
  return sd.T >= 1 && sd.T <= kTokenSumMaxTokens && sd.top_k + has_shared <= kTokenSumMaxWaves &&
         ed.hidden % 32 == 0 && ed.inter % ed.group == 0;
}

hipError_t launch_w2_token_sum(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                               const int32_t* ids, const float* topk_w, uint16_t* out,
                               hipStream_t stream) {
  if (!w2_token_sum_fits(ed, sd) || !decode_offsets_fit(ed, sd)) return hipErrorInvalidValue;
  const int groups = ed.inter / ed.group;
  switch (ed.group) {  // K = 512: all of a slot's groups in flight at once; else a 2-deep ring
    case 64:
      return groups == 8 ? launch_token_sum<2, 2, -8>(h, ed, sd, ids, topk_w, out, stream)
                         : launch_token_sum<2, 2, 2>(h, ed, sd, ids, topk_w, out, stream);
    case 128:
      return groups == 4 ? launch_token_sum<4, 2, -4>(h, ed, sd, ids, topk_w, out, stream)
                         : launch_token_sum<4, 2, 2>(h, ed, sd, ids, topk_w, out, stream);
    case 256:
      return groups == 2 ? launch_token_sum<8, 2, -2>(h, ed, sd, ids, topk_w, out, stream)
                         : launch_token_sum<8, 2, 2>(h, ed, sd, ids, topk_w, out, stream);
    default: return hipErrorInvalidValue;
  }
}
