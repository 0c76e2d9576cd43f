// Shared device helpers for the gfx950 W4A16 MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_w4a16.h"

#define MOE_DEV __device__ __forceinline__

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// bf16 "magic" exponent: a bf16 with bit pattern 0x4300 | q (q < 16) has value 128 + q.
constexpr uint32_t kMagicPair = 0x43004300u;
constexpr float kMagicBias = 128.0f;

MOE_DEV float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
MOE_DEV float bf16lo_to_f32(uint32_t pair) { return __uint_as_float(pair << 16); }
MOE_DEV float bf16hi_to_f32(uint32_t pair) { return __uint_as_float(pair & 0xFFFF0000u); }

// fp32 -> bf16, IEEE round-to-nearest-even (NaN kept quiet).
MOE_DEV uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
MOE_DEV uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_rne(lo) | (f32_to_bf16_rne(hi) << 16);
}

MOE_DEV float f16_to_f32(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// D = a.lo*b.lo + a.hi*b.hi + c  (v_dot2_f32_bf16)
MOE_DEV float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Pairs (x[j], x[j+4]) of the 8 bf16 held in d0..d3 (d0 = x0|x1<<16, ...), matching the
// nibble pairs (j, j+4) produced by magic_pair().
MOE_DEV void xpairs(const u32x4 d, uint32_t p[4]) {
  p[0] = __builtin_amdgcn_perm(d[2], d[0], 0x05040100u);  // (x0, x4)
  p[1] = __builtin_amdgcn_perm(d[2], d[0], 0x07060302u);  // (x1, x5)
  p[2] = __builtin_amdgcn_perm(d[3], d[1], 0x05040100u);  // (x2, x6)
  p[3] = __builtin_amdgcn_perm(d[3], d[1], 0x07060302u);  // (x3, x7)
}

// bf16 pair (128 + nibble j, 128 + nibble j+4) of a packed int32 of 8 nibbles.
MOE_DEV uint32_t magic_pair(uint32_t w, int j) {
  return ((w >> (4 * j)) & 0x000F000Fu) | kMagicPair;
}

// Raw buffer loads (stride 0, unformatted). A byte offset at or past the resource's
// num_records reads zeros without a memory access, so a lane whose data does not exist (a
// padding row, a ring stage past the end of a slice) still issues the same instruction as the
// others: every thread runs the same loads on every path and the compiler's wait counts stay
// exact. Offsets in use stay below kOutOfRange; ORing kOutOfRange into one moves it out.
constexpr int kBufferDword3 = 0x00020000;
constexpr uint32_t kOutOfRange = 0x80000000u;
// Cache policy of a streamed-once load (nt).
constexpr int kBufNontemporal = 2;

// Resource over [base, base + num_bytes).
MOE_DEV __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t num_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)num_bytes,
                                           kBufferDword3);
}
// Resource over [base, base + 2 GiB) for data addressed by offsets below kOutOfRange.
MOE_DEV __amdgpu_buffer_rsrc_t buf_rsrc(const void* base) { return buf_rsrc(base, kOutOfRange); }

template <int AUX = 0>
MOE_DEV u32x4 buf_ld128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX));
}
template <int AUX = 0>
MOE_DEV u32x2 buf_ld64(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, AUX));
}
template <int AUX = 0>
MOE_DEV uint32_t buf_ld32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX);
}

// s_waitcnt immediate waiting for vmcnt <= n only (expcnt and lgkmcnt at their maximum).
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Buffer load of 16 bytes per lane straight into LDS: lane i writes lds[16 i, 16 i + 16) (bytes;
// lds wave-uniform). An out-of-range offset writes zeros. The load counts in vmcnt until the
// bytes are in LDS. (A device function: the builtin inside a lambda of a kernel makes the host
// pass drop the kernel's launch stub.)
MOE_DEV void buf_ld128_lds(__amdgpu_buffer_rsrc_t r, uint16_t* lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, off, 0, 0, 0);
}

MOE_DEV u32x4 ld128(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
MOE_DEV u32x4 ld128_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// SiLU of the GEMM epilogues: g * (1 / (1 + e^-g)) with the hardware reciprocal (v_rcp_f32, 1 ulp)
// instead of the IEEE division sequence: about 5 VALU operations instead of 15, and the product is
// rounded to bf16 right after. (The predictors, whose activations feed a top-k, keep a division.)
MOE_DEV float silu_f32(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// Device view of one projection of an expert set.
struct ProjDev {
  const int32_t* qweight;
  const int32_t* qzeros;
  const uint16_t* scales;
};

// Everything a GEMM kernel needs to locate expert e's weights.
struct ExpertsDev {
  ProjDev gate, up, down;
  ProjDev sgate, sup, sdown;     // shared expert (expert id == num_experts), may be null
  const int32_t* expert_row;     // nullable
  int64_t row_stride;            // bytes between the rows of the routed experts; 0 = dense
  int32_t num_experts;
  int32_t hidden, inter, group;
};

// Pointers to row `row` of a projection with reduction length K (K8 = K/8 packed rows, NG = K/G
// groups) and NOUT output columns: densely stacked tensors [rows, ...], or per-expert blobs
// `stride_bytes` apart (an expert slot pool).
MOE_DEV ProjDev proj_row(const ProjDev& p, int64_t stride_bytes, int64_t row, int K8, int NG,
                         int NOUT) {
  if (stride_bytes) {
    const int64_t o = row * stride_bytes;
    return ProjDev{reinterpret_cast<const int32_t*>(reinterpret_cast<const char*>(p.qweight) + o),
                   reinterpret_cast<const int32_t*>(reinterpret_cast<const char*>(p.qzeros) + o),
                   reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(p.scales) + o)};
  }
  return ProjDev{p.qweight + row * K8 * NOUT, p.qzeros + row * NG * (NOUT / 8),
                 p.scales + row * NG * NOUT};
}

// A routed slot's expert contributes: its id is in [0, num_experts) and, with an expert_row map
// (a slot pool), it is resident (row >= 0). Other slots are dropped and contribute zero, as the
// reference drops ids outside [0, E) and unmapped experts
// (src/mtp_expert_prefetch/tracing/vllm_router_trace.py:14138-14153).
MOE_DEV bool routed_ok(const int32_t* expert_row, int num_experts, int e) {
  return e >= 0 && e < num_experts && (expert_row == nullptr || expert_row[e] >= 0);
}

// A block's expert id is usable: a contributing routed expert, or the shared expert when one is
// present.
MOE_DEV bool expert_ok(const ExpertsDev& ed, int e) {
  return routed_ok(ed.expert_row, ed.num_experts, e) ||
         (e == ed.num_experts && ed.sgate.qweight != nullptr);
}

MOE_DEV int64_t expert_row(const ExpertsDev& ed, int e) {
  return ed.expert_row ? (int64_t)ed.expert_row[e] : (int64_t)e;
}

// Per-call sizes shared by the kernels.
struct SlotsDev {
  int32_t T;          // tokens
  int32_t top_k;
  int32_t num_slots;  // T*top_k (+T with a shared expert)
};

MOE_DEV int slot_token(const SlotsDev& s, int f) {
  return f < s.T * s.top_k ? f / s.top_k : f - s.T * s.top_k;
}

// Lane i receives lane (i ^ M)'s value, through DPP and cross-row permutes rather than LDS
// (ds_bpermute). A butterfly v = v + xor_partner<M>(v) over M = 32 .. 1 adds the same two
// operands at every lane as v += shfl_xor(v, M) (fp32 addition is commutative), so sums are
// bit-identical to that butterfly. Called by a whole wave.
template <int M>
MOE_DEV float xor_partner(float v) {
  const int iv = __float_as_int(v);
  if constexpr (M == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)iv, (uint32_t)iv, false, false);
    return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
  } else if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)iv, (uint32_t)iv, false, false);
    return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
  } else if constexpr (M == 8) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, iv, 0x128, 0xF, 0xF, false));  // row_ror:8
  } else if constexpr (M == 4) {  // half-row mirror (i -> 7 - i), then quad reverse: i -> i ^ 4
    const int m = __builtin_amdgcn_update_dpp(0, iv, 0x141, 0xF, 0xF, false);
    return __int_as_float(__builtin_amdgcn_update_dpp(0, m, 0x1B, 0xF, 0xF, false));
  } else if constexpr (M == 2) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, iv, 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
  } else {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, iv, 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
  }
}

MOE_DEV float bfly_sum(float v) {
  v = v + xor_partner<32>(v);
  v = v + xor_partner<16>(v);
  v = v + xor_partner<8>(v);
  v = v + xor_partner<4>(v);
  v = v + xor_partner<2>(v);
  v = v + xor_partner<1>(v);
  return v;
}
MOE_DEV float bfly_min(float v) {
  v = fminf(v, xor_partner<32>(v));
  v = fminf(v, xor_partner<16>(v));
  v = fminf(v, xor_partner<8>(v));
  v = fminf(v, xor_partner<4>(v));
  v = fminf(v, xor_partner<2>(v));
  return fminf(v, xor_partner<1>(v));
}
MOE_DEV float bfly_max(float v) {
  v = fmaxf(v, xor_partner<32>(v));
  v = fmaxf(v, xor_partner<16>(v));
  v = fmaxf(v, xor_partner<8>(v));
  v = fmaxf(v, xor_partner<4>(v));
  v = fmaxf(v, xor_partner<2>(v));
  return fmaxf(v, xor_partner<1>(v));
}

