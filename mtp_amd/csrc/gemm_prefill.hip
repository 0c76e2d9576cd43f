// Prefill path: grouped bf16 MFMA GEMMs over block-padded expert groups, with the int4 weights
// dequantised exactly in registers (reference dequant semantics, bit-exact bf16), fused
// SiLU*mul (W1) and routed-weight (W2) epilogues.
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
//   of column tile ni, so tile ni holds the columns {c_j + ni}.
//   A operand (gathered bf16 rows) is staged in LDS, 128 k per step, double-buffered so one
//   barrier per step orders both the writes and the reuse of a buffer.
//   W1: a wave's 64 columns are 32 gate columns (lanes j < 8) and the same 32 up columns
//       (lanes j >= 8); the epilogue pairs them with a row rotation by 8 and writes bf16 h.
//   W2: 64 output columns of the hidden dimension; epilogue writes w[slot] * acc (fp32).
// 16-row subtiles that hold only padding are neither loaded nor multiplied.
#include "common.h"
#include "launch.h"

namespace {

constexpr int BM = kPrefillBlockM;  // 128
constexpr int BK = 128;             // k per step: 4 MFMA slices of 32
constexpr int LDS_STRIDE = BK + 8;  // bf16 per LDS row (16 B padding against bank conflicts)
constexpr int kMTiles = BM / 16;    // 8 row subtiles


typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

enum { MODE_W1 = 1, MODE_W2 = 2 };

// bf16 pair of two fp32 values (v_cvt_pk_bf16_f32, round to nearest even).
MOE_DEV uint32_t pk_bf16(float lo, float hi) {
  bf16x2_t p = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, p);
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

// YS16 (W2): the weighted slot rows are written as bf16 (round to nearest even) instead of fp32.
// NW waves per workgroup, each covering all BM rows x 64 GEMM columns; the block's A tile in
// LDS is shared by the NW waves (8 waves: the tile is loaded once for twice the columns).
template <int MODE, bool YS16 = false, int NW = 4>
__global__ __launch_bounds__(64 * NW, 8 / NW) void grouped_gemm_kernel(
    const uint16_t* __restrict__ A,  // W1: x [T, H]; W2: h [num_slots, I]
    ExpertsDev ed, SlotsDev sd, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ eids, const int32_t* __restrict__ ntpp,
    const float* __restrict__ topk_w, uint16_t* __restrict__ h_out, void* __restrict__ ys,
    int a_bytes, int ncolblk) {
  __shared__ __attribute__((aligned(16))) uint16_t lds_a[2][BM * LDS_STRIDE];
  __shared__ int s_slot[BM];

  // XCD-aware order: workgroup p runs on XCD p % 8, and XCD c takes the contiguous range
  // [c S, c S + S) of the used (align block, column block) items, numbered expert-major, so the
  // column blocks of one align block (same A rows) and the align blocks of one expert (same
  // weights) run close together on one XCD and share its L2.
  const int used = (*ntpp / BM) * ncolblk;
  const int per_xcd = (used + 7) / 8;
  const int logical = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
  if ((int)(blockIdx.x >> 3) >= per_xcd || logical >= used) return;
  const int b = logical / ncolblk;  // align block
  const int cblk = logical % ncolblk;
  const int e = eids[b];
  if (!expert_ok(ed, e)) return;

  constexpr int NTH = 64 * NW;                  // threads
  constexpr int AChunks = BM * BK / 8 / NTH;    // 16-byte A chunks per thread and step
  constexpr int ARowStep = NTH / 16;            // rows between a thread's chunks
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = ed.hidden, I = ed.inter, G = ed.group;
  const int K = (MODE == MODE_W1) ? H : I;     // reduction length
  const int NOUT = (MODE == MODE_W1) ? I : H;  // columns of one projection
  const bool is_shared = (e == ed.num_experts);
  const int64_t row = is_shared ? 0 : expert_row(ed, e);
  const int K8 = K / 8, NG = K / G;

  if (tid < BM) s_slot[tid] = sorted[b * BM + tid];
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

  // ---- A staging: chunk i of this thread = row (tid >> 4) + ARowStep i, 16-byte k-chunk tid & 15.
  // Buffer loads: a padding row gets an out-of-range offset, which reads zeros without a memory
  // access, while every thread still issues the same loads on every step (static wait counts).
  const int a_kc = tid & 15;
  const __amdgpu_buffer_rsrc_t a_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(A), 0, a_bytes, kBufferDword3);
  uint32_t a_off[AChunks];  // byte offset of the chunk in A
#pragma unroll
  for (int i = 0; i < AChunks; ++i) {
    const int f = s_slot[(tid >> 4) + ARowStep * i];
    const uint32_t ar = (MODE == MODE_W1) ? slot_token(sd, f) : f;
    a_off[i] = ((unsigned)f < (unsigned)sd.num_slots) ? (ar * (uint32_t)K + a_kc * 8) * 2
                                                       : kOutOfRange;
  }

  f32x4 acc[kMTiles][4];
#pragma unroll
  for (int i = 0; i < kMTiles; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nsteps = K / BK;
  u32x4 ra[AChunks / 2];   // one half of a step's A chunks in flight
  u32x4 bw[4];             // packed weight words of the 4 k-slices of a step
  GroupSZ gz[2];           // groups of k-slices 0-1 and 2-3 (the same group when G >= 128)
  auto load_a = [&](int step, int half) {
#pragma unroll
    for (int i = 0; i < AChunks / 2; ++i)
      ra[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            a_rsrc, a_off[half * (AChunks / 2) + i] + step * BK * 2,
                                            0, 0));
  };
  auto store_a = [&](uint16_t* la, int half) {
#pragma unroll
    for (int i = 0; i < AChunks / 2; ++i) {
      const int r = (tid >> 4) + ARowStep * (half * (AChunks / 2) + i);
      *reinterpret_cast<u32x4*>(&la[r * LDS_STRIDE + a_kc * 8]) = ra[i];
    }
  };
  auto load_gz = [&](int step, int h) {
    const int g = (step * BK + 64 * h) / G;
    gz[h].s = *reinterpret_cast<const u32x2*>(bs + (int64_t)g * NOUT);
    gz[h].z = (uint32_t)bz[(int64_t)g * (NOUT / 8)];
  };
  auto load_bw = [&](int step, int kk) {
    bw[kk] = ld128(bq + (int64_t)(step * 16 + kk * 4) * NOUT);
  };
  load_gz(0, 0);
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) load_bw(0, kk);
  load_gz(0, 1);
  load_a(0, 0);
  store_a(lds_a[0], 0);
  load_a(0, 1);
  store_a(lds_a[0], 1);

  for (int step = 0; step < nsteps; ++step) {
    // Loads for the next step reuse each register right after its last read; on the last step
    // they re-read the last step (in bounds, never used). The next step's A tile goes to the
    // other buffer, whose readers (the previous step) all passed this step's barrier.
    const int nxt = min(step + 1, nsteps - 1);
    const uint16_t* la = lds_a[step & 1];
    uint16_t* la_next = lds_a[(step + 1) & 1];
    __syncthreads();

    _Float16 sc[4];
    float cc[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if ((kk & 1) == 0) {
        // fp16 scales and c = -(1024 + z) * s of the lane's 4 columns for this half-step
        const GroupSZ q = gz[kk >> 1];
        const uint32_t zw = q.z >> zsh;
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          sc[n] = __builtin_bit_cast(_Float16, (uint16_t)(q.s[n >> 1] >> (16 * (n & 1))));
          cc[n] = -(1024.0f + (float)((zw >> (4 * n)) & 0xFu)) * (float)sc[n];
        }
        load_gz(nxt, kk >> 1);
        if (kk == 2) store_a(la_next, 0);
        load_a(nxt, kk >> 1);
      }
      bf16x8_v bfr[4];
#pragma unroll
      for (int n = 0; n < 4; ++n) bfr[n] = dequant8_exact(bw[kk][n], sc[n], cc[n]);
      load_bw(nxt, kk);
      // A fragments one subtile ahead (a read past mtiles stays inside the buffer, unused)
      const uint16_t* lrow = &la[j * LDS_STRIDE + kk * 32 + 8 * kq];
      bf16x8_v af_next = *reinterpret_cast<const bf16x8_v*>(lrow);
#pragma unroll
      for (int mi = 0; mi < kMTiles; ++mi) {
        if (mi >= mtiles) break;
        const bf16x8_v af = af_next;
        if (mi + 1 < kMTiles)
          af_next = *reinterpret_cast<const bf16x8_v*>(lrow + (mi + 1) * 16 * LDS_STRIDE);
#pragma unroll
        for (int n = 0; n < 4; ++n)
          acc[mi][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr[n], acc[mi][n], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // the next subtile's DS read ...
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // ... before these 4 MFMAs
      }
    }
    store_a(la_next, 1);
  }

  // ---- epilogue. D[i][jj] of a 16x16 tile sits in lane jj + 16*(i/4), element i%4; column jj
  // of tile n is projection column col(jj) + n.
#pragma unroll
  for (int mi = 0; mi < kMTiles; ++mi) {
    if (mi >= mtiles) break;
#pragma unroll
    for (int el = 0; el < 4; ++el) {
      const int r = mi * 16 + 4 * kq + el;
      const int f = s_slot[r];
      if (MODE == MODE_W1) {
        float hv[4];
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          const float g = acc[mi][n][el];
          // lanes jj < 8 hold gate, lane jj + 8 the up value of the same column (row_ror:8)
          const float u = __int_as_float(
              __builtin_amdgcn_update_dpp(0, __float_as_int(g), 0x128, 0xF, 0xF, false));
          hv[n] = silu_f32(g) * u;
        }
        if (j < 8 && (unsigned)f < (unsigned)sd.num_slots) {
          const u32x2 o = {pk_bf16(hv[0], hv[1]), pk_bf16(hv[2], hv[3])};
          *reinterpret_cast<u32x2*>(&h_out[(int64_t)f * I + col]) = o;
        }
      } else {
        if ((unsigned)f < (unsigned)sd.num_slots) {
          const float w = topk_w[f];
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
}

// Workgroups for up to `items` items, a multiple of 8 (each XCD gets the same number).
int xcd_grid(int items) { return ((items + 7) / 8) * 8; }

}  // namespace

// Shapes (checked by the entry points): hidden % 512 == 0, intermediate in {256, 512, 1024},
// group in {64, 128, 256}; so K % 128 == 0, W1 columns % 128 == 0 and W2 columns % 256 == 0.
// Four waves per workgroup (two workgroups per CU): measured faster than eight waves sharing one
// A tile over twice the columns (W1 160 vs 179 us at T = 2048), which leaves one workgroup per CU.
hipError_t launch_w1_prefill(const uint16_t* x, const ExpertsDev& ed, const SlotsDev& sd,
                             const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                             int BMr, int cap, uint16_t* h, hipStream_t stream) {
  const int64_t a_bytes = (int64_t)sd.T * ed.hidden * 2;  // x [T, H] bf16
  if (BMr != BM || ed.hidden % BK != 0 || ed.inter % 128 != 0 || ed.group < 64 ||
      a_bytes >= kOutOfRange)
    return hipErrorInvalidValue;
  const int ncb = ed.inter / 128;
  hipLaunchKernelGGL((grouped_gemm_kernel<MODE_W1, false, 4>), dim3(xcd_grid(cap * ncb)),
                     dim3(256), 0, stream, x, ed, sd, sorted, eids, ntpp, (const float*)nullptr, h,
                     (void*)nullptr, (int)a_bytes, ncb);
  return hipGetLastError();
}

namespace {
template <bool YS16>
hipError_t launch_w2_prefill_t(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                               const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                               int BMr, int cap, const float* topk_w, void* ys,
                               hipStream_t stream) {
  const int64_t a_bytes = (int64_t)sd.num_slots * ed.inter * 2;  // h [num_slots, I] bf16
  if (BMr != BM || ed.inter % BK != 0 || ed.hidden % 256 != 0 || ed.group < 64 ||
      a_bytes >= kOutOfRange)
    return hipErrorInvalidValue;
  const int ncb = ed.hidden / 256;
  hipLaunchKernelGGL((grouped_gemm_kernel<MODE_W2, YS16, 4>), dim3(xcd_grid(cap * ncb)),
                     dim3(256), 0, stream, h, ed, sd, sorted, eids, ntpp, topk_w,
                     (uint16_t*)nullptr, ys, (int)a_bytes, ncb);
  return hipGetLastError();
}
}  // namespace

hipError_t launch_w2_prefill(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                             const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                             int BMr, int cap, const float* topk_w, float* ys,
                             hipStream_t stream) {
  return launch_w2_prefill_t<false>(h, ed, sd, sorted, eids, ntpp, BMr, cap, topk_w, ys, stream);
}

hipError_t launch_w2_prefill_bf16(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                                  const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                                  int BMr, int cap, const float* topk_w, uint16_t* ys,
                                  hipStream_t stream) {
  return launch_w2_prefill_t<true>(h, ed, sd, sorted, eids, ntpp, BMr, cap, topk_w, ys, stream);
}
