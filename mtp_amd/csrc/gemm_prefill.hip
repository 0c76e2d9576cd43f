// Prefill path: grouped bf16 MFMA GEMMs over block-padded expert groups, with the int4 weights
// dequantised in registers, fused SiLU*mul (W1) and routed-weight (W2) epilogues. Blocks of more
// than two 16-row subtiles dequantise exactly (reference dequant semantics, bit-exact bf16
// weights); lighter blocks fold the zero point and scale into the per-group MFMA sums (the decode
// kernels' arithmetic: weights unrounded, layer outputs within the same tolerance).
//
// Arithmetic follows src/mtp_expert_prefetch/tracing/vllm_wna16_group_plan.py:367-486
// (A row = slot // top_k, b = ((q - z) * s).to(bf16), fp32 accumulation) and the expert MLP of
// src/mtp_expert_prefetch/repack/gptq_unpack.py:247-256.
//
// Block: BM = 128 slots of one expert x 4 waves split along N; every wave covers all 128 rows
// (8 MFMA 16x16x32 row subtiles) and 64 GEMM columns (4 column tiles), so each weight element
// is dequantised once per block and there is no LDS traffic for B.
//   B operand straight from the GPTQ layout: for each 32-k slice, lane (j = lane & 15,
//   kq = lane >> 4) loads 16 bytes = the packed words of 4 consecutive columns c_j .. c_j + 3
//   at packed row kq; word ni is exactly the MFMA B fragment (8 consecutive k of one column)
//   of column tile ni, so tile ni holds the columns {c_j + ni}. A two-step register ring keeps
//   the next two 128-k steps of B in flight.
//   A operand (gathered bf16 rows) is loaded straight into LDS (buffer_load ... lds, no VGPR
//   staging), 128 k per step, double-buffered: the next step's tile is in flight during a step,
//   and one wait + barrier per step orders both its arrival and the reuse of a buffer.
//   W1: a wave's 64 columns are 32 gate columns (lanes j < 8) and the same 32 up columns
//       (lanes j >= 8); the epilogue pairs them with a row rotation by 8 and writes bf16 h.
//   W2: 64 output columns of the hidden dimension; epilogue writes w[slot] * acc (fp32 or bf16).
// 16-row subtiles that hold only padding are neither loaded nor multiplied. Blocks with at most
// two subtiles of slots (experts with few tokens) take a streaming path instead: B in a register
// ring several k-steps deep, A in a ring of LDS stages of the same depth, folded dequant (see
// stream_block). There the exact
// dequant's ~19 VALU operations per packed word cost more than the multiplications they feed;
// the fold needs 7 per word plus two per output element and group (measured: prefill-2048
// 259 -> 248 us per layer).
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace {

constexpr int BM = kPrefillBlockM;  // 128
constexpr int BK = 128;             // k per step: 4 MFMA slices of 32
constexpr int kMTiles = BM / 16;    // 8 row subtiles
// Loads per step of the LDS path's B ring (scales + zeros of two half-steps, 4 weight words),
// the count the wait for a step's A tile leaves in flight.
constexpr int kLoadsPerStepB = 8;


// Streaming path: blocks of at most kStreamMaxTiles row subtiles; ring depth (k-steps in
// flight per wave) for one and for two subtiles (with the group sums of the fold, a 3-deep ring
// for two subtiles spills). K is a multiple of 256, so the step count is even (the
// runtime-count ring is 2 deep).
constexpr int kStreamMaxTiles = 2;
constexpr int kStreamDepth1 = 4;
constexpr int kStreamDepth2 = 2;


typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

enum { MODE_W1 = 1, MODE_W2 = 2 };

// bf16 pair of two fp32 values (v_cvt_pk_bf16_f32, round to nearest even).
MOE_DEV uint32_t pk_bf16(float lo, float hi) {
  bf16x2_t p = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, p);
}

// Folded dequant (light blocks): B fragments hold the exact bf16 values 128 + q, in the k order
// [0,2,4,6,1,3,5,7] (two nibble byte planes, one byte permute per bf16 pair with the exponent
// byte 0x43), and the A fragments are permuted to the same order; per quantisation group the
// MFMA sums S = sum_k x (128 + q) and X = sum_k x (an all-ones B) are folded into the result as
// s (S - (128 + z) X).
constexpr uint32_t kFoldMagic = 0x43434343u;
constexpr uint32_t kFoldOnes = 0x3F803F80u;  // bf16 pair (1, 1)
MOE_DEV bf16x8_v fold_weight_frag(uint32_t w) {
  const uint32_t ev = w & 0x0F0F0F0Fu, od = (w >> 4) & 0x0F0F0F0Fu;
  const u32x4 o = {__builtin_amdgcn_perm(ev, kFoldMagic, 0x00050004u),
                   __builtin_amdgcn_perm(ev, kFoldMagic, 0x00070006u),
                   __builtin_amdgcn_perm(od, kFoldMagic, 0x00050004u),
                   __builtin_amdgcn_perm(od, kFoldMagic, 0x00070006u)};
  return __builtin_bit_cast(bf16x8_v, o);
}
MOE_DEV bf16x8_v fold_act_frag(const u32x4 d) {
  const u32x4 o = {__builtin_amdgcn_perm(d[1], d[0], 0x05040100u),
                   __builtin_amdgcn_perm(d[3], d[2], 0x05040100u),
                   __builtin_amdgcn_perm(d[1], d[0], 0x07060302u),
                   __builtin_amdgcn_perm(d[3], d[2], 0x07060302u)};
  return __builtin_bit_cast(bf16x8_v, o);
}

// Exact bf16((q - z) * s) of the 8 nibbles of w (nibble j = k0 + j) as an MFMA B fragment.
// The fp16 value 1024 + q (bits 0x6400 | q) is assembled by byte permutes from the masked
// nibble bytes; v_fma_mix_f32 widens it and the fp16 scale and adds c = -(1024 + z) * s, which is
// exact in fp32 (11-bit x 11-bit significands). (1024 + q) * s + c = (q - z) * s is then exact,
// so the only rounding is the bf16 conversion, as in the reference's fp32 dequant + cast.
MOE_DEV bf16x8_v dequant8_exact(uint32_t w, _Float16 s, float c) {
  const uint32_t lo = w & 0x0F0F0F0Fu;         // bytes: nibbles 0, 2, 4, 6
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // bytes: nibbles 1, 3, 5, 7
  constexpr uint32_t kHalfExp = 0x64646464u;   // high byte of fp16 1024
  const f16x2_t m02 = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(lo, kHalfExp, 0x00050004u));
  const f16x2_t m46 = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(lo, kHalfExp, 0x00070006u));
  const f16x2_t m13 = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(hi, kHalfExp, 0x00050004u));
  const f16x2_t m57 = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(hi, kHalfExp, 0x00070006u));
  const float sf = (float)s;
  const float f0 = __builtin_fmaf((float)m02[0], sf, c), f2 = __builtin_fmaf((float)m02[1], sf, c);
  const float f4 = __builtin_fmaf((float)m46[0], sf, c), f6 = __builtin_fmaf((float)m46[1], sf, c);
  const float f1 = __builtin_fmaf((float)m13[0], sf, c), f3 = __builtin_fmaf((float)m13[1], sf, c);
  const float f5 = __builtin_fmaf((float)m57[0], sf, c), f7 = __builtin_fmaf((float)m57[1], sf, c);
  const u32x4 o = {pk_bf16(f0, f1), pk_bf16(f2, f3), pk_bf16(f4, f5), pk_bf16(f6, f7)};
  return __builtin_bit_cast(bf16x8_v, o);
}

// Scales (4 fp16 of consecutive columns) and the packed zeros word of one group.
struct GroupSZ {
  u32x2 s;
  uint32_t z;
};

// fp16 scales and c = -(1024 + z) * s of the lane's 4 columns (zero nibbles from bit zsh).
MOE_DEV void group_coeffs(const GroupSZ& q, int zsh, _Float16 (&sc)[4], float (&cc)[4]) {
  const uint32_t zw = q.z >> zsh;
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    sc[n] = __builtin_bit_cast(_Float16, (uint16_t)(q.s[n >> 1] >> (16 * (n & 1))));
    cc[n] = -(1024.0f + (float)((zw >> (4 * n)) & 0xFu)) * (float)sc[n];
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

// ---- Streaming path for blocks whose slots fit in MT row subtiles (an expert with few tokens).
// Such a block reads its 128 KB-per-wave weight slice for very little arithmetic, so its time is
// memory latency: with the LDS-staged path's one-step lookahead every 128-k step waits for a
// full round trip. Here each wave keeps D k-steps of its packed weight words and scales and zeros
// in flight in registers. The block's A rows (MT*16 x 128 k per step) go through a D-stage LDS
// ring filled by buffer_load ... lds, each wave loading MT of the stage's 1 KB runs: whole
// 128-byte lines, once per workgroup (fragments loaded by every wave straight from memory were 16
// half-line requests per instruction, repeated by the four waves). Steps past K read zeros
// without a memory access. The dequant is the folded one (compute_fold).
template <int MT>
struct StreamStage {
  u32x4 bw[4];     // packed words of the lane's 4 columns, k-slice kk
  GroupSZ gz[2];   // groups of k-slices 0-1 and 2-3
};

struct StreamView {
  __amdgpu_buffer_rsrc_t ar;  // A rows (uniform)
  // A ring: stage i of MT*16 rows x BK in LDS object lds[i] (separate objects, so that the
  // compiler's waits for the loads into one stage do not cover reads of another); rows swizzled
  // as in the LDS path.
  uint16_t* lds[4];
  uint32_t a_dma[2];          // this wave's DMA lane offsets at step 0, kOutOfRange for padding rows
  int wave, j, kq;
  // The lane's weights: in W1 lanes j < 8 read gate and lanes j >= 8 up, so these are per-lane
  // global addresses rather than buffer resources.
  const int32_t* bq;          // packed row kq of step 0 at the lane's first column
  const uint16_t* bs;         // scales of group 0 at the lane's first column
  const int32_t* bz;          // zeros word of group 0 holding the lane's columns
  int NOUT, gsh, nsteps, zsh;  // gsh: log2 of the group size

  // A rows of step s into LDS stage `slot`: load u of this wave is run q = wave * MT + u (rows
  // 4q .. 4q + 3). A step past K writes zeros (never read).
  template <int MT>
  MOE_DEV void dma(int s, int slot) const {
    const uint32_t ks = (uint32_t)s * BK * 2u, oob = s < nsteps ? 0u : kOutOfRange;
#pragma unroll
    for (int u = 0; u < MT; ++u)
      buf_ld128_lds(ar, lds[slot] + 4 * (wave * MT + u) * BK, (a_dma[u] + ks) | oob);
  }

  // Weights, scales and zeros of step s; a prefetch past the last step re-reads the last step
  // (in bounds; it is never multiplied), so every pass issues the same loads.
  template <int MT>
  MOE_DEV void load(StreamStage<MT>& st, int s) const {
    const int sc = min(s, nsteps - 1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int g = (sc * BK + 64 * h) >> gsh;
      st.gz[h].s = *reinterpret_cast<const u32x2*>(bs + (int64_t)g * NOUT);
      st.gz[h].z = (uint32_t)bz[(int64_t)g * (NOUT / 8)];
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)  // weights are streamed once: nontemporal
      st.bw[kk] = ld128_nt(bq + (int64_t)(sc * (BK / 8) + kk * 4) * NOUT);
  }

  // Folded form of compute for step `step`: group sums in gs / gx, folded into acc at the end of
  // each quantisation group (group sizes >= 64, so a group ends at a half-step boundary).
  template <int MT>
  MOE_DEV void compute_fold(const StreamStage<MT>& st, int step, int slot, f32x4 (&acc)[MT][4],
                            f32x4 (&gs)[MT][4], f32x4 (&gx)[MT]) const {
    const bf16x8_v ones =
        __builtin_bit_cast(bf16x8_v, u32x4{kFoldOnes, kFoldOnes, kFoldOnes, kFoldOnes});
    // A fragment of row mi*16 + j at chunk 4 kk + kq (stored at chunk position (4 kk + kq) ^ j)
    const uint16_t* la = lds[slot] + j * BK;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      bf16x8_v af[MT];
#pragma unroll
      for (int mi = 0; mi < MT; ++mi) {
        af[mi] = fold_act_frag(
            *reinterpret_cast<const u32x4*>(la + mi * 16 * BK + 8 * ((4 * kk + kq) ^ j)));
        gx[mi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mi], ones, gx[mi], 0, 0, 0);
      }
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const bf16x8_v wf = fold_weight_frag(st.bw[kk][n]);
#pragma unroll
        for (int mi = 0; mi < MT; ++mi)
          gs[mi][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mi], wf, gs[mi][n], 0, 0, 0);
      }
      if ((kk & 1) && (((step * BK + 32 * (kk + 1)) & ((1 << gsh) - 1)) == 0)) {  // group end
        const GroupSZ& q = st.gz[kk >> 1];
        const uint32_t zw = q.z >> zsh;
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          const float s =
              (float)__builtin_bit_cast(_Float16, (uint16_t)(q.s[n >> 1] >> (16 * (n & 1))));
          const float zb = 128.0f + (float)((zw >> (4 * n)) & 0xFu);
#pragma unroll
          for (int mi = 0; mi < MT; ++mi)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              acc[mi][n][i] =
                  __builtin_fmaf(s, __builtin_fmaf(-zb, gx[mi][i], gs[mi][n][i]), acc[mi][n][i]);
        }
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) {
          gx[mi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int n = 0; n < 4; ++n) gs[mi][n] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
  }
};

// acc += A[MT*16 rows, :K] . B[:K, lane columns] over all steps with a D-deep ring (registers for
// B, LDS for A). Step st: the B loads of step st + D - 1; the wait for this wave's loads of step
// st (A and B; the later steps' stay in flight); a barrier (every wave's A of step st landed, and
// every wave is done with the stage that step st + D - 1 refills); the A loads of step st + D - 1;
// the multiplications of step st. NS > 0: exactly NS steps as straight-line code. NS == 0: a
// runtime loop (D divides the step count) whose body issues the same loads on every pass.
template <int MT, int D, int NS>
MOE_DEV void stream_block(const StreamView& v, f32x4 (&acc)[MT][4]) {
  static_assert(D <= 4 && (D <= 2 || MT == 1), "A stages 2 and 3 hold 16 rows");
  // loads issued after step st's A loads when step st is waited for: B of steps st+1 .. st+D-1
  // and A of steps st+1 .. st+D-2
  constexpr int kLater = 8 * (D - 1) + MT * (D - 2);
  StreamStage<MT> ring[D];
  f32x4 gs[MT][4], gx[MT];
#pragma unroll
  for (int mi = 0; mi < MT; ++mi) {
    gx[mi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n = 0; n < 4; ++n) gs[mi][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  static_for<0, D - 1>([&](auto jc) {
    v.load(ring[jc.value], jc.value);
    v.template dma<MT>(jc.value, jc.value);
    __builtin_amdgcn_sched_barrier(0);  // issue order = step order
  });
  // LATER: loads issued after step st's A loads when step st is waited for (kLater while the
  // ring is refilled; in the straight-line tail, the (8 + MT) loads of each step still to come)
  auto step = [&](auto slot_c, auto later_c, int st, bool more) {
    constexpr int slot = decltype(slot_c)::value;
    constexpr int refill = (slot + D - 1) % D;  // the stage of step st + D - 1
    if (more) v.load(ring[refill], st + D - 1);
    __builtin_amdgcn_sched_barrier(0);  // this step's B loads ahead of the wait for step st
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(decltype(later_c)::value));
    // The barrier without __syncthreads' release fence, which would also wait for the A loads
    // of the later stages still in flight. Each wave has waited for its own loads of step st,
    // which are then in LDS for every wave; the signal fences keep the compiler from moving
    // LDS accesses across the barrier.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (more) v.template dma<MT>(st + D - 1, refill);
    __builtin_amdgcn_sched_barrier(0);
    v.compute_fold(ring[slot], st, slot, acc, gs, gx);
  };
  if constexpr (NS > 0) {
    static_for<0, NS>([&](auto sc) {
      constexpr int st = sc.value;
      constexpr bool more = st + D - 1 < NS;
      step(std::integral_constant<int, st % D>{},
           std::integral_constant<int, more ? kLater : (NS - 1 - st) * (8 + MT)>{}, st, more);
    });
  } else {
    for (int s0 = 0; s0 < v.nsteps; s0 += D) {
      static_for<0, D>([&](auto jc) {
        step(jc, std::integral_constant<int, kLater>{}, s0 + jc.value, true);
      });
    }
  }
}

// Epilogue of the first `mtiles` row subtiles. D[i][jj] of a 16x16 tile sits in lane
// jj + 16*(i/4), element i%4; column jj of tile n is projection column col(jj) + n.
template <int MODE, bool YS16, int M>
MOE_DEV void block_epilogue(const f32x4 (&acc)[M][4], int mtiles, const int* s_slot, int j,
                            int kq, int col, int num_slots, int I, int H,
                            const float* s_w, uint16_t* __restrict__ h_out,
                            void* __restrict__ ys) {
#pragma unroll
  for (int mi = 0; mi < M; ++mi) {
    if (mi >= mtiles) break;
    if constexpr (MODE == MODE_W1) {
      // Lanes jj < 8 hold gate and lane jj + 8 the up value of the same column; a row rotation
      // by 8 (row_ror:8) brings each its partner's. Rows are taken in pairs (el, el + 1): lanes
      // jj < 8 form h of row el, lanes jj >= 8 h of row el + 1 from the gate value of lane
      // jj - 8, so every lane computes one SiLU per pair of rows.
      const bool lo = j < 8;
#pragma unroll
      for (int el = 0; el < 4; el += 2) {
        const int f = s_slot[mi * 16 + 4 * kq + el + (lo ? 0 : 1)];
        float hv[4];
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          const float ga = acc[mi][n][el], gb = acc[mi][n][el + 1];
          const float ra = __int_as_float(
              __builtin_amdgcn_update_dpp(0, __float_as_int(ga), 0x128, 0xF, 0xF, false));
          const float rb = __int_as_float(
              __builtin_amdgcn_update_dpp(0, __float_as_int(gb), 0x128, 0xF, 0xF, false));
          hv[n] = silu_f32(lo ? ga : rb) * (lo ? ra : gb);
        }
        if ((unsigned)f < (unsigned)num_slots) {
          const u32x2 o = {pk_bf16(hv[0], hv[1]), pk_bf16(hv[2], hv[3])};
          *reinterpret_cast<u32x2*>(&h_out[(int64_t)f * I + col]) = o;
        }
      }
      continue;
    }
#pragma unroll
    for (int el = 0; el < 4; ++el) {  // W2: the routed weight times the row
      const int r = mi * 16 + 4 * kq + el;
      const int f = s_slot[r];
      if ((unsigned)f < (unsigned)num_slots) {
        const float w = s_w[r];
        const f32x4 o = {w * acc[mi][0][el], w * acc[mi][1][el], w * acc[mi][2][el],
                         w * acc[mi][3][el]};
        if constexpr (YS16) {
          const u32x2 ob = {pk_bf16(o[0], o[1]), pk_bf16(o[2], o[3])};
          *reinterpret_cast<u32x2*>(&static_cast<uint16_t*>(ys)[(int64_t)f * H + col]) = ob;
        } else {
          *reinterpret_cast<f32x4*>(&static_cast<float*>(ys)[(int64_t)f * H + col]) = o;
        }
      }
    }
  }
}

// YS16 (W2): the weighted slot rows are written as bf16 (round to nearest even) instead of fp32.
// NW waves per workgroup, each covering all BM rows x 64 GEMM columns; the block's A tile in
// LDS is shared by the NW waves (8 waves: the tile is loaded once for twice the columns).
template <int MODE, bool YS16 = false, int NW = 4>
__global__ __launch_bounds__(64 * NW, 8 / NW) void grouped_gemm_kernel(
    const uint16_t* __restrict__ A,  // W1: x [T, H]; W2: h [num_slots, I]
    ExpertsDev ed, SlotsDev sd, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ eids, const int32_t* __restrict__ ntpp,
    const int32_t* __restrict__ border, const float* __restrict__ topk_w,
    uint16_t* __restrict__ h_out, void* __restrict__ ys, int a_bytes, int ncolblk) {
  // Two A buffers as separate objects: the compiler then knows that reads of one do not wait
  // for the LDS loads in flight into the other.
  __shared__ __attribute__((aligned(16))) uint16_t lds_a0[BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t lds_a1[BM * BK];
  // Two more stages of the streaming path's A ring (16 rows each; stages 0 and 1 are lds_a0, lds_a1)
  __shared__ __attribute__((aligned(16))) uint16_t lds_s2[16 * BK];
  __shared__ __attribute__((aligned(16))) uint16_t lds_s3[16 * BK];
  __shared__ int s_slot[BM];
  __shared__ float s_w[MODE == MODE_W2 ? BM : 1];  // routed weight of each row (W2)

  // XCD-aware order: workgroup p runs on XCD p % 8 and each XCD runs the column blocks of one
  // align block back to back, so they share the block's A rows in that XCD's L2.
  //  - With a block order (border, heaviest first), the ordered blocks are dealt to the XCDs in
  //    turn: every XCD starts on its share of the big blocks and ends on light ones.
  //  - Without one, XCD c takes the contiguous range [c S, c S + S) of the (block, column block)
  //    items, numbered expert-major.
  const int nblk = *ntpp / BM;
  int b, cblk;
  if (border) {
    const int q = (int)(blockIdx.x >> 3);
    const int r = (q / ncolblk) * 8 + (int)(blockIdx.x & 7);
    if (r >= nblk) return;
    b = border[r];
    cblk = q % ncolblk;
  } else {
    const int used = nblk * ncolblk;
    const int per_xcd = (used + 7) / 8;
    const int logical = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
    if ((int)(blockIdx.x >> 3) >= per_xcd || logical >= used) return;
    b = logical / ncolblk;
    cblk = logical % ncolblk;
  }
  const int e = eids[b];
  if (!expert_ok(ed, e)) return;

  constexpr int kARowsPerWave = BM / NW;       // A rows each wave loads into LDS per step
  constexpr int kADmaLoads = kARowsPerWave / 4;  // 1 KB (4-row) LDS loads per wave and step
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = ed.hidden, I = ed.inter, G = ed.group;
  const int K = (MODE == MODE_W1) ? H : I;     // reduction length
  const int NOUT = (MODE == MODE_W1) ? I : H;  // columns of one projection
  const bool is_shared = (e == ed.num_experts);
  const int64_t row = is_shared ? 0 : expert_row(ed, e);
  const int K8 = K / 8, NG = K / G;
  const int gsh = __builtin_ctz(G);  // group sizes are powers of two (64, 128, 256)

  if (tid < BM) {
    const int f = sorted[b * BM + tid];
    s_slot[tid] = f;
    if constexpr (MODE == MODE_W2) s_w[tid] = (unsigned)f < (unsigned)sd.num_slots ? topk_w[f] : 0.0f;
  }
  __syncthreads();
  // Valid rows come first in a block (an expert's slots, then its padding).
  int nvalid = 0;
#pragma unroll
  for (int r = 0; r < BM; r += 16) nvalid += (unsigned)s_slot[r] < (unsigned)sd.num_slots ? 16 : 0;
  const int mtiles = nvalid / 16;  // row subtiles holding at least one slot

  // ---- B columns of this lane
  const int j = lane & 15, kq = lane >> 4;
  int col;  // first of the lane's 4 projection columns
  ProjDev p;
  if (MODE == MODE_W1) {
    col = cblk * (32 * NW) + wave * 32 + 4 * (j & 7);
    p = (j < 8) ? (is_shared ? ed.sgate : ed.gate) : (is_shared ? ed.sup : ed.up);
  } else {
    col = cblk * (64 * NW) + wave * 64 + 4 * j;
    p = is_shared ? ed.sdown : ed.down;
  }
  const ProjDev pr = proj_row(p, is_shared ? 0 : ed.row_stride, row, K8, NG, NOUT);
  const int32_t* bq = pr.qweight + (int64_t)kq * NOUT + col;
  const uint16_t* bs = pr.scales + col;
  const int32_t* bz = pr.qzeros + (col >> 3);
  const int zsh = 4 * (col & 7);

  // Few slots: the streaming path (B in a register ring several k-steps deep, A in LDS stages).
  const int mt_u = __builtin_amdgcn_readfirstlane(mtiles);
  if (mt_u <= kStreamMaxTiles) {
    const __amdgpu_buffer_rsrc_t ar =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(A), 0, a_bytes, kBufferDword3);
    StreamView v;
    v.ar = ar;
    v.lds[0] = lds_a0;
    v.lds[1] = lds_a1;
    v.lds[2] = lds_s2;  // 16 rows: stages 2 and 3 serve one-subtile blocks only
    v.lds[3] = lds_s3;
    v.wave = wave;
    v.j = j;
    v.kq = kq;
    // DMA run q = wave * MT + u: lane i fetches row 4q + (i >> 4) at chunk (i & 15) ^ (row & 15)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int r = 4 * (wave * mt_u + u) + (lane >> 4);
      const int f = s_slot[r];
      const uint32_t arow = (MODE == MODE_W1) ? slot_token(sd, f) : f;
      const uint32_t c = (uint32_t)((lane & 15) ^ (r & 15));
      v.a_dma[u] = ((unsigned)f < (unsigned)sd.num_slots) ? (arow * (uint32_t)K + 8u * c) * 2u
                                                           : kOutOfRange;
    }
    v.bq = bq;
    v.bs = bs;
    v.bz = bz;
    v.NOUT = NOUT;
    v.gsh = gsh;
    v.nsteps = K / BK;
    v.zsh = zsh;
    // step count of the usual shapes (hidden 2048, intermediate 512): a straight-line ring
    constexpr int kNS = (MODE == MODE_W1) ? 16 : 4;
    if (mt_u == 1) {
      f32x4 acc1[1][4];
#pragma unroll
      for (int n = 0; n < 4; ++n) acc1[0][n] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (v.nsteps == kNS) {
        stream_block<1, kStreamDepth1, kNS>(v, acc1);
      } else {
        stream_block<1, 2, 0>(v, acc1);
      }
      block_epilogue<MODE, YS16>(acc1, 1, s_slot, j, kq, col, sd.num_slots, I, H, s_w, h_out,
                                 ys);
    } else {
      f32x4 acc2[2][4];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int n = 0; n < 4; ++n) acc2[mi][n] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (v.nsteps == kNS) {
        stream_block<2, kStreamDepth2, kNS>(v, acc2);
      } else {
        stream_block<2, 2, 0>(v, acc2);
      }
      block_epilogue<MODE, YS16>(acc2, 2, s_slot, j, kq, col, sd.num_slots, I, H, s_w, h_out,
                                 ys);
    }
    return;
  }

  // ---- A tile in LDS: BM rows x BK k per step, rows of BK bf16 (256 B) without padding; the
  // 16-byte chunk c of row r sits at chunk position c ^ (r & 15), so the 16 rows one MFMA A read
  // spans fall in 16 different bank groups. The tile is loaded straight into LDS
  // (buffer_load ... lds): lane i of one load writes bytes [16 i, 16 i + 16) of a 1 KB run of 4
  // rows, so it fetches row 4q + (i >> 4) of the run at k-chunk (i & 15) ^ row. Wave w fills rows
  // [w BM/NW, (w + 1) BM/NW); a padding row gets an out-of-range offset (zeros, no memory access).
  const __amdgpu_buffer_rsrc_t a_rsrc = buf_rsrc(A, (uint32_t)a_bytes);
  uint32_t a_off[kADmaLoads];  // byte offset of this lane's chunk of load i, step 0
#pragma unroll
  for (int i = 0; i < kADmaLoads; ++i) {
    const int r = wave * kARowsPerWave + 4 * i + (lane >> 4);
    const int f = s_slot[r];
    const uint32_t ar = (MODE == MODE_W1) ? slot_token(sd, f) : f;
    const uint32_t c = (uint32_t)((lane & 15) ^ (r & 15));
    a_off[i] = ((unsigned)f < (unsigned)sd.num_slots) ? (ar * (uint32_t)K + 8u * c) * 2u
                                                       : kOutOfRange;
  }
  const int nsteps = K / BK;
  auto dma_a = [&](uint16_t* buf, int step) {  // a step past K writes zeros (never read)
    const uint32_t ko = (uint32_t)step * BK * 2u | (step < nsteps ? 0u : kOutOfRange);
#pragma unroll
    for (int i = 0; i < kADmaLoads; ++i)
      buf_ld128_lds(a_rsrc, buf + (wave * kARowsPerWave + 4 * i) * BK, a_off[i] + ko);
  };

  f32x4 acc[kMTiles][4];
#pragma unroll
  for (int i = 0; i < kMTiles; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};

  // ---- B ring: slot s & 1 holds the packed weight words and the scales/zeros of step s; each
  // register is reloaded with step s + 2 right after its last read in step s (a step past K
  // re-reads the last one: in bounds, never used). kLoadsPerStepB loads per step.
  u32x4 bw[2][4];
  GroupSZ gz[2][2];
  auto load_gz = [&](int slot, int step, int h) {
    const int g = (min(step, nsteps - 1) * BK + 64 * h) >> gsh;
    gz[slot][h].s = *reinterpret_cast<const u32x2*>(bs + (int64_t)g * NOUT);
    gz[slot][h].z = (uint32_t)bz[(int64_t)g * (NOUT / 8)];
  };
  auto load_bw = [&](int slot, int step, int kk) {
    bw[slot][kk] = ld128(bq + (int64_t)(min(step, nsteps - 1) * 16 + kk * 4) * NOUT);
  };
  auto load_b = [&](int slot, int step) {
    load_gz(slot, step, 0);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) load_bw(slot, step, kk);
    load_gz(slot, step, 1);
  };

  // Pipeline: A of step s + 1 is loaded into LDS during step s, B of step s + 2 into registers.
  // The wait at the top of a step is for this wave's A loads of that step only: the
  // kLoadsPerStepB B loads issued after them stay in flight.
  dma_a(lds_a0, 0);
  __builtin_amdgcn_sched_barrier(0);
  load_b(0, 0);
  __builtin_amdgcn_sched_barrier(0);  // issue order = step order
  load_b(1, 1);
  const int mtu = __builtin_amdgcn_readfirstlane(mtiles);
  auto run_step = [&](auto xc, int step) {
    constexpr int X = decltype(xc)::value;  // step & 1: LDS buffer and B slot
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(kLoadsPerStepB));
    __syncthreads();  // every wave's A of this step landed; the other buffer is free
    dma_a(X ? lds_a0 : lds_a1, step + 1);
    __builtin_amdgcn_sched_barrier(0);
    const uint16_t* la = X ? lds_a1 : lds_a0;
    _Float16 sc[4];
    float cc[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if ((kk & 1) == 0) {
        group_coeffs(gz[X][kk >> 1], zsh, sc, cc);
        load_gz(X, step + 2, kk >> 1);
      }
      bf16x8_v bfr[4];
#pragma unroll
      for (int n = 0; n < 4; ++n) bfr[n] = dequant8_exact(bw[X][kk][n], sc[n], cc[n]);
      load_bw(X, step + 2, kk);
      // A fragment of row mi*16 + j at logical chunk 4 kk + kq, one subtile ahead (a read past
      // mtiles stays inside the buffer, unused)
      const uint16_t* lrow = la + j * BK + 8 * ((4 * kk + kq) ^ j);
      bf16x8_v af_next = *reinterpret_cast<const bf16x8_v*>(lrow);
#pragma unroll
      for (int mi = 0; mi < kMTiles; ++mi) {
        if (mi >= mtu) break;
        const bf16x8_v af = af_next;
        if (mi + 1 < kMTiles)
          af_next = *reinterpret_cast<const bf16x8_v*>(lrow + (mi + 1) * 16 * BK);
#pragma unroll
        for (int n = 0; n < 4; ++n)
          acc[mi][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr[n], acc[mi][n], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // the next subtile's DS read ...
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // ... before these 4 MFMAs
      }
    }
  };
  for (int step = 0; step < nsteps; step += 2) {  // nsteps is even
    run_step(std::integral_constant<int, 0>{}, step);
    run_step(std::integral_constant<int, 1>{}, step + 1);
  }

  block_epilogue<MODE, YS16>(acc, mtiles, s_slot, j, kq, col, sd.num_slots, I, H, s_w, h_out,
                             ys);
}

// Workgroups for up to `cap` align blocks x ncb column blocks in either order: eight XCD shares
// of ceil(cap / 8) blocks (at least ceil(cap ncb / 8) items each).
int xcd_grid(int cap, int ncb) { return ((cap + 7) / 8) * 8 * ncb; }

}  // namespace

// Shapes (checked by the entry points): hidden % 512 == 0, intermediate in {256, 512, 1024},
// group in {64, 128, 256}; so K % 128 == 0, W1 columns % 128 == 0 and W2 columns % 256 == 0.
// Four waves per workgroup (two workgroups per CU): measured faster than eight waves sharing one
// A tile over twice the columns (W1 160 vs 179 us at T = 2048), which leaves one workgroup per CU.
hipError_t launch_w1_prefill(const uint16_t* x, const ExpertsDev& ed, const SlotsDev& sd,
                             const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                             const int32_t* border, int BMr, int cap, uint16_t* h,
                             hipStream_t stream) {
  const int64_t a_bytes = (int64_t)sd.T * ed.hidden * 2;  // x [T, H] bf16
  if (BMr != BM || ed.hidden % BK != 0 || ed.inter % 128 != 0 || ed.group < 64 ||
      a_bytes >= kOutOfRange)
    return hipErrorInvalidValue;
  const int ncb = ed.inter / 128;
  hipLaunchKernelGGL((grouped_gemm_kernel<MODE_W1, false, 4>), dim3(xcd_grid(cap, ncb)),
                     dim3(256), 0, stream, x, ed, sd, sorted, eids, ntpp, border,
                     (const float*)nullptr, h, (void*)nullptr, (int)a_bytes, ncb);
  return hipGetLastError();
}

namespace {
template <bool YS16>
hipError_t launch_w2_prefill_t(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                               const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                               const int32_t* border, int BMr, int cap, const float* topk_w,
                               void* ys, hipStream_t stream) {
  const int64_t a_bytes = (int64_t)sd.num_slots * ed.inter * 2;  // h [num_slots, I] bf16
  if (BMr != BM || ed.inter % BK != 0 || ed.hidden % 256 != 0 || ed.group < 64 ||
      a_bytes >= kOutOfRange)
    return hipErrorInvalidValue;
  const int ncb = ed.hidden / 256;
  hipLaunchKernelGGL((grouped_gemm_kernel<MODE_W2, YS16, 4>), dim3(xcd_grid(cap, ncb)),
                     dim3(256), 0, stream, h, ed, sd, sorted, eids, ntpp, border, topk_w,
                     (uint16_t*)nullptr, ys, (int)a_bytes, ncb);
  return hipGetLastError();
}
}  // namespace

hipError_t launch_w2_prefill(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                             const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                             const int32_t* border, int BMr, int cap, const float* topk_w,
                             float* ys, hipStream_t stream) {
  return launch_w2_prefill_t<false>(h, ed, sd, sorted, eids, ntpp, border, BMr, cap, topk_w, ys,
                                    stream);
}

hipError_t launch_w2_prefill_bf16(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                                  const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                                  const int32_t* border, int BMr, int cap, const float* topk_w,
                                  uint16_t* ys, hipStream_t stream) {
  return launch_w2_prefill_t<true>(h, ed, sd, sorted, eids, ntpp, border, BMr, cap, topk_w, ys,
                                   stream);
}
