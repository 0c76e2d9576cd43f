// Prefill path: grouped bf16 MFMA GEMMs over block-padded expert groups, with int4 weights
// dequantised once per tile into LDS (reference dequant semantics, bit-exact bf16), fused
// SiLU*mul (W1) and routed-weight (W2) epilogues.
//
// Arithmetic follows src/mtp_expert_prefetch/tracing/vllm_wna16_group_plan.py:367-486
// (A row = slot // top_k, b = ((q - z) * s).to(bf16), fp32 accumulation) and the expert MLP of
// src/mtp_expert_prefetch/repack/gptq_unpack.py:247-256.
//
// Tile: BM = 128 slots x 128 GEMM columns x BK = 64 (half a quantisation group) per step,
// 4 waves in a 2 x 2 arrangement, each wave 64 x 64 = 4 x 4 MFMA 16x16x32 bf16 tiles.
//   W1: the 128 GEMM columns are 64 gate + the same 64 up columns, so the epilogue computes
//       silu(gate) * up in registers and writes bf16 h.
//   W2: 128 output columns of the hidden dimension; epilogue writes w[slot] * acc (fp32).
// A rows are gathered through the sorted slot list (sentinel rows are zero and not stored).
// Global loads of step k+1 are issued before the MFMAs of step k (register double buffer).
#include "common.h"
#include "launch.h"

namespace {

constexpr int BM = kPrefillBlockM;  // 128
constexpr int BN = 128;
constexpr int BK = 64;
constexpr int LDS_STRIDE = BK + 8;  // bf16 elements per LDS row (padding against bank conflicts)

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));

enum { MODE_W1 = 1, MODE_W2 = 2 };

MOE_DEV uint32_t dq_pair(float qa, float qb, float s, float zs) {
  const float a = __builtin_fmaf(qa, s, -zs);  // == (qa - z) * s exactly
  const float b = __builtin_fmaf(qb, s, -zs);
  bf16x2_t p = {(__bf16)a, (__bf16)b};  // v_cvt_pk_bf16_f32, RNE
  return __builtin_bit_cast(uint32_t, p);
}

// 8 consecutive k of one column: nibble j of w is k0 + j.
MOE_DEV u32x4 dequant8(uint32_t w, float s, float zs) {
  const uint32_t lo = w & 0x0F0F0F0Fu;         // nibbles 0,2,4,6 in bytes 0..3
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // nibbles 1,3,5,7
  u32x4 o;
  o[0] = dq_pair((float)(lo & 0xFFu), (float)(hi & 0xFFu), s, zs);
  o[1] = dq_pair((float)((lo >> 8) & 0xFFu), (float)((hi >> 8) & 0xFFu), s, zs);
  o[2] = dq_pair((float)((lo >> 16) & 0xFFu), (float)((hi >> 16) & 0xFFu), s, zs);
  o[3] = dq_pair((float)(lo >> 24), (float)(hi >> 24), s, zs);
  return o;
}

template <int MODE>
__global__ __launch_bounds__(256) void grouped_gemm_kernel(
    const uint16_t* __restrict__ A,  // W1: x [T, H]; W2: h [num_slots, I]
    ExpertsDev ed, SlotsDev sd, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ eids, const int32_t* __restrict__ ntpp,
    const float* __restrict__ topk_w, uint16_t* __restrict__ h_out, float* __restrict__ ys) {
  __shared__ __attribute__((aligned(16))) uint16_t lds_a[BM * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) uint16_t lds_b[BN * LDS_STRIDE];
  __shared__ int s_slot[BM];

  const int b = blockIdx.y;
  if (b * BM >= *ntpp) return;
  const int e = eids[b];
  if (!expert_ok(ed, e)) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int H = ed.hidden, I = ed.inter, G = ed.group;
  const int K = (MODE == MODE_W1) ? H : I;       // reduction length
  const int NOUT = (MODE == MODE_W1) ? I : H;    // columns of one projection
  const int n0 = blockIdx.x * ((MODE == MODE_W1) ? BN / 2 : BN);  // first projection column
  const bool is_shared = (e == ed.num_experts);
  const int64_t row = is_shared ? 0 : expert_row(ed, e);
  ProjDev p0, p1;
  if (MODE == MODE_W1) {
    p0 = is_shared ? ed.sgate : ed.gate;
    p1 = is_shared ? ed.sup : ed.up;
  } else {
    p0 = is_shared ? ed.sdown : ed.down;
    p1 = p0;
  }
  const int K8 = K / 8, NG = K / G;

  if (tid < BM) s_slot[tid] = sorted[b * BM + tid];
  __syncthreads();
  // Valid rows come first in a block (an expert's slots, then its padding): the 16-row MFMA
  // subtiles past them are all padding and are skipped (the tile is still dequantised once).
  int nvalid = 0;
#pragma unroll
  for (int r = 0; r < BM; r += 16) nvalid += (unsigned)s_slot[r] < (unsigned)sd.num_slots ? 16 : 0;
  const int mtiles = (nvalid - wm * 64 + 15) / 16;  // row subtiles of this wave with data

  // ---- A load mapping: 4 chunks of 16 B per thread; chunk = tid + 256 i -> row, k-chunk
  const uint16_t* a_row[4];
  int a_kc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int chunk = tid + 256 * i;
    const int r = chunk >> 3;
    a_kc[i] = chunk & 7;
    const int f = s_slot[r];
    if ((unsigned)f < (unsigned)sd.num_slots) {
      const int64_t arow = (MODE == MODE_W1) ? (int64_t)slot_token(sd, f) : (int64_t)f;
      a_row[i] = A + arow * K;
    } else {
      a_row[i] = nullptr;
    }
  }
  // ---- B load mapping: one 16 B load (4 columns x 8 k) per thread.
  // W1: threads 0..127 gate, 128..255 up; 8 packed rows x 16 column-quads each.
  // W2: 8 packed rows x 32 column-quads of the 128-column tile.
  int b_prow, b_col;  // packed row within the k-step, first column within the tile
  int b_lds_col;
  bool second = false;  // W1 threads 128..255 load the up projection
  if (MODE == MODE_W1) {
    const int t = tid & 127;
    b_prow = t >> 4;
    b_col = (t & 15) * 4;
    second = tid >= 128;
    b_lds_col = (second ? 64 : 0) + b_col;
  } else {
    b_prow = tid >> 5;
    b_col = (tid & 31) * 4;
    b_lds_col = b_col;
  }
  const ProjDev pr = proj_row(second ? p1 : p0, is_shared ? 0 : ed.row_stride, row, K8, NG, NOUT);
  const int gcol = n0 + b_col;  // projection column of this thread's first column
  const int32_t* bq = pr.qweight + gcol;
  const uint16_t* bs = pr.scales + gcol;
  const int32_t* bz = pr.qzeros + (gcol >> 3);
  const int zshift = 4 * (gcol & 7);

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nsteps = K / BK;
  u32x4 ra[4], rb;
  auto gload = [&](int step) {
    const int kbase = step * BK;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ra[i] = a_row[i] ? ld128(a_row[i] + kbase + a_kc[i] * 8) : u32x4{0, 0, 0, 0};
    rb = ld128_nt(bq + (int64_t)(kbase / 8 + b_prow) * NOUT);
  };
  gload(0);

  for (int step = 0; step < nsteps; ++step) {
    // scales / zeros of this thread's 4 columns for the group of this step
    const int g = (step * BK) / G;
    const u32x2 s2 = *reinterpret_cast<const u32x2*>(bs + (int64_t)g * NOUT);
    const uint32_t zw = (uint32_t)bz[(int64_t)g * (NOUT / 8)] >> zshift;
    __syncthreads();  // previous step's MFMA reads are complete
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = (tid + 256 * i) >> 3;
      *reinterpret_cast<u32x4*>(&lds_a[r * LDS_STRIDE + a_kc[i] * 8]) = ra[i];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float s = f16_to_f32((s2[q >> 1] >> (16 * (q & 1))) & 0xFFFFu);
      const float z = (float)((zw >> (4 * q)) & 0xFu);
      const u32x4 o = dequant8(rb[q], s, z * s);
      *reinterpret_cast<u32x4*>(&lds_b[(b_lds_col + q) * LDS_STRIDE + b_prow * 8]) = o;
    }
    __syncthreads();
    if (step + 1 < nsteps) gload(step + 1);

#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
      const int kofs = kk * 32 + 8 * (lane >> 4);
      bf16x8_v af[4], bfr[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        if (mi >= mtiles) break;
        const int r = wm * 64 + mi * 16 + (lane & 15);
        af[mi] = *reinterpret_cast<const bf16x8_v*>(&lds_a[r * LDS_STRIDE + kofs]);
      }
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) {
        int c;
        if (MODE == MODE_W1)
          c = (ni < 2 ? 0 : 64) + wn * 32 + (ni & 1) * 16 + (lane & 15);
        else
          c = wn * 64 + ni * 16 + (lane & 15);
        bfr[ni] = *reinterpret_cast<const bf16x8_v*>(&lds_b[c * LDS_STRIDE + kofs]);
      }
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        if (mi >= mtiles) break;
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mi], bfr[ni], acc[mi][ni], 0, 0, 0);
      }
    }
  }

  // ---- epilogue. D[i][j] of a 16x16 tile sits in lane j + 16*(i/4), element i%4.
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
    for (int el = 0; el < 4; ++el) {
      const int r = wm * 64 + mi * 16 + 4 * (lane >> 4) + el;
      const int f = s_slot[r];
      if ((unsigned)f >= (unsigned)sd.num_slots) continue;
      if (MODE == MODE_W1) {
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
          const float gte = acc[mi][ni][el], up = acc[mi][ni + 2][el];
          const int col = n0 + wn * 32 + ni * 16 + (lane & 15);
          h_out[(int64_t)f * I + col] = (uint16_t)f32_to_bf16_rne(silu_f32(gte) * up);
        }
      } else {
        const float w = topk_w[f];
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
          const int col = n0 + wn * 64 + ni * 16 + (lane & 15);
          ys[(int64_t)f * H + col] = w * acc[mi][ni][el];
        }
      }
    }
  }
}

}  // namespace

hipError_t launch_w1_prefill(const uint16_t* x, const ExpertsDev& ed, const SlotsDev& sd,
                             const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                             int BMr, int cap, uint16_t* h, hipStream_t stream) {
  if (BMr != BM) return hipErrorInvalidValue;
  const dim3 grid(ed.inter / (BN / 2), cap);
  hipLaunchKernelGGL(grouped_gemm_kernel<MODE_W1>, grid, dim3(256), 0, stream, x, ed, sd, sorted,
                     eids, ntpp, (const float*)nullptr, h, (float*)nullptr);
  return hipGetLastError();
}

hipError_t launch_w2_prefill(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                             const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                             int BMr, int cap, const float* topk_w, float* ys,
                             hipStream_t stream) {
  if (BMr != BM) return hipErrorInvalidValue;
  const dim3 grid(ed.hidden / BN, cap);
  hipLaunchKernelGGL(grouped_gemm_kernel<MODE_W2>, grid, dim3(256), 0, stream, h, ed, sd, sorted,
                     eids, ntpp, topk_w, (uint16_t*)nullptr, ys);
  return hipGetLastError();
}
