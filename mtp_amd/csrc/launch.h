// Host-side launchers of the kernels (one translation unit per kernel family).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_w4a16.h"

// Thread-local message of the last failed entry point (moe_w4a16_last_error).
constexpr int kErrorBufferBytes = 512;
char* moe_error_buffer();

// Workspaces start on a 256-byte boundary (hipMalloc's and torch's allocations do): their
// sections are laid out at 256-byte offsets and read with 16-byte vector and LDS-direct loads.
inline bool workspace_aligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 255u) == 0; }

// Slot-cache prefetch for moe_offload_layer_v1 (slot_cache.hip): no ordering wait on the compute
// stream; the caller has synchronised that stream after every kernel reading an unpinned slot of
// the layer was enqueued, and the latest demand's slots are still pinned.
int slot_cache_prefetch_synced(uint64_t handle, int32_t layer, const int32_t* experts, int32_t n,
                               void* compute_stream);
// The slot cache's routed-ids flags for an offload layer call of T tokens (slot_cache.hip):
// pinned host words mapped at the same device address, and the value this call waits for;
// nullptr when unavailable (then the call waits on its stream).
int32_t* slot_cache_signal(uint64_t handle, int32_t T, int32_t* seq);

// Argument checks of a routed layer call that involve no workspace (api.hip): 0 or the error
// code moe_layer_v1 returns for the same input (message in moe_error_buffer).
int check_layer_args(const uint16_t* x, int32_t T, const uint16_t* router_w, int32_t top_k,
                     const moe_expert_set_v1* experts, const moe_expert_set_v1* shared,
                     const uint16_t* shared_gate_w, const uint16_t* out, int32_t path);

struct ProjDev;
struct ExpertsDev;
struct SlotsDev;

hipError_t launch_dequant(const ProjDev& p, const int32_t* g_idx, int E, int K, int N, int G,
                          int linear, int out_dtype, void* out, hipStream_t stream);

hipError_t launch_router_logits(const uint16_t* x, int T, int H, const uint16_t* W, int E,
                                const uint16_t* shared_w, const float* bias, float* logits,
                                hipStream_t stream);
// ids_mirror: optional second destination of the ids (e.g. pinned host memory mapped into the
// device's address space), written by the same lanes as ids.
// flags (with ids_mirror): after token t's ids are out, word t is set to seq with a
// system-scope release, so a host that reads flags[t] == seq then reads the token's ids.
hipError_t launch_router_topk(const float* logits, int T, int E, int top_k, int has_shared,
                              int32_t* ids, float* weights, hipStream_t stream,
                              int32_t* ids_mirror = nullptr, int32_t* flags = nullptr,
                              int32_t seq = 0);
// Prefill-size router (router_mfma.hip): approximate logits on MFMA into approx [T][E+1] and
// squared router-row norms into nw2 [E], then per token a certified top-k whose ids, order and
// weights equal those of the canonical logits (weights[T*top_k + t] = shared gate when
// shared_w is given). H % 512 == 0, H <= 2048, E <= 512.
bool router_prefill_fits(int T, int H, int E, int top_k);
float router_prefill_rel_bound(int H);
hipError_t launch_router_prefill(const uint16_t* x, int T, int H, const uint16_t* W, int E,
                                 const uint16_t* shared_w, const float* bias, int top_k,
                                 float* approx, float* nw2, int32_t* ids, float* weights,
                                 hipStream_t stream);
// Top-k of every token (one wave each) and the align/sort of the at most 64 slots by one wave,
// in one launch: the decode-size routing tail. sorted/eids are written up to the padded total
// only (the decode kernels read nothing past it); ntpp holds the total.
constexpr int kTopkAlignMaxTokens = 8;
inline bool topk_align_fits(int T, int top_k, int has_shared) {
  return T >= 1 && T <= kTopkAlignMaxTokens && top_k <= 8 &&
         T * top_k + (has_shared ? T : 0) <= 64;
}
hipError_t launch_topk_align(const float* logits, int T, int E, int top_k, int has_shared, int BM,
                             int cap, int32_t* ids, float* weights, int32_t* sorted, int32_t* eids,
                             int32_t* ntpp, hipStream_t stream);
hipError_t launch_shared_gate(const uint16_t* x, int T, int H, const uint16_t* shared_w,
                              int top_k, float* logits_ws, float* weights, hipStream_t stream);

int align_capacity_blocks(int T, int top_k, int E, int has_shared, int BM);
// Bytes of scratch (outside the output buffers) that lets launch_align spread the large-input
// scatter over many workgroups, for any number of slots; 0 when these sizes take the one-block
// kernel. Every form writes `border` (when non-null and BM is a multiple of 16, at most 128):
// the align blocks sorted by the number of 16-row subtiles holding slots, heaviest first (one
// entry per block up to the padded total).
int64_t align_scratch_bytes(int T, int top_k, int E, int has_shared, int BM, int cap);
// scratch (nullable): align_scratch_bytes bytes the call may overwrite. Without it, inputs of up to
// 32 768 slots still take a two-kernel form (ranks and counts in the sorted buffer), larger ones the
// one-block kernel.
hipError_t launch_align(const int32_t* topk_ids, int T, int top_k, int E, int has_shared, int BM,
                        int cap, int32_t* sorted, int32_t* eids, int32_t* ntpp, int32_t* border,
                        int32_t* scratch, hipStream_t stream);

// Slot-grid routing for decode-size batches (slot_grid_fits): the MFMA decode kernels take their
// expert and rows from the routed ids themselves instead of an align pass. Workgroup y = slot
// index; the workgroup at every 16th occurrence of an expert takes the next (up to) 16 slots of
// that expert, the others leave. With `logits` (W1 of a layer call) every workgroup computes the
// top-k of the (at most 8) tokens itself and workgroup (0, 0) publishes ids and weights; otherwise
// they are read from `ids` / `weights`.
struct SlotGrid {
  int active;
  const float* logits;  // [T][E+1] or nullptr
  int32_t* ids;         // routed ids [T*top_k]
  float* weights;       // routed weights [T*top_k] (+ T shared gates)
};
constexpr int kSlotGridMaxSlots = 64;  // all slots are the lanes of one wave
inline bool slot_grid_fits(int T, int top_k, int has_shared) {
  return topk_align_fits(T, top_k, has_shared);  // T <= 8, slots <= 64
}

// Decode path on MFMA with in-register dequantisation (blocks of kDecodeBlockM slots).
hipError_t launch_w1_decode_mfma(const uint16_t* x, const ExpertsDev& ed, const SlotsDev& sd,
                                 const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                                 int cap, uint16_t* h, hipStream_t stream);
hipError_t launch_w2_decode_mfma(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                                 const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                                 int cap, const float* topk_w, float* ys, hipStream_t stream);
hipError_t launch_w1_decode_slotgrid(const uint16_t* x, const ExpertsDev& ed, const SlotsDev& sd,
                                     const SlotGrid& sg, uint16_t* h, hipStream_t stream);
hipError_t launch_w2_decode_slotgrid(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                                     const SlotGrid& sg, float* ys, hipStream_t stream);

// ids == nullptr: every slot is summed; otherwise routed slots with a dropped expert are skipped.
hipError_t launch_moe_sum(const float* ys, int T, int top_k, int H, int has_shared,
                          const int32_t* ids, int num_experts, const int32_t* expert_row,
                          uint16_t* out, hipStream_t stream);
// moe_sum over bf16 slot rows (summed in fp32 in slot order).
hipError_t launch_moe_sum_bf16(const uint16_t* ys, int T, int top_k, int H, int has_shared,
                               const int32_t* ids, int num_experts, const int32_t* expert_row,
                               uint16_t* out, hipStream_t stream);

// W2 and the weighted sum in one kernel for up to 8 tokens (decode path): block = token x
// column tile, one wave per slot of the token, out written directly (no ys, no sum kernel).
// An expert routed by several tokens is read once per token (from L2 after the first); up to 8
// tokens that costs less than the sum launch and the fp32 rows it saves (measured: 4 tokens
// 27.9 -> 25.6 us per layer, 8 tokens 34.1 -> 33.4 us).
constexpr int kTokenSumMaxTokens = 8;
// Batches whose W1 computes the top-k itself in every workgroup (slot grid from the logits).
constexpr int kGridTopkMaxTokens = 2;
constexpr int kTokenSumMaxWaves = 9;  // top_k <= 8 plus the shared expert
bool w2_token_sum_fits(const ExpertsDev& ed, const SlotsDev& sd);
// W1 with W2 fused in, on the slot grid (T <= kGridTopkMaxTokens): part = fp32 partial rows
// [num_slots][inter / 32][hidden] (weighted), summed per token by launch_partial_sum.
bool w1w2_fused_fits(const ExpertsDev& ed, const SlotsDev& sd);
hipError_t launch_w1w2_slotgrid(const uint16_t* x, const ExpertsDev& ed, const SlotsDev& sd,
                                const SlotGrid& sg, float* part, hipStream_t stream);
bool partial_sum_fits(int top_k, int has_shared, int H, int nct);
hipError_t launch_partial_sum(const float* part, int T, int top_k, int H, int nct, int has_shared,
                              uint16_t* out, hipStream_t stream);
hipError_t launch_w2_token_sum(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                               const int32_t* ids, const float* topk_w, uint16_t* out,
                               hipStream_t stream);

// Prefill (bf16 MFMA) path. border (nullable): the block order written by the large-input align.
hipError_t launch_w1_prefill(const uint16_t* x, const ExpertsDev& ed, const SlotsDev& sd,
                             const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                             const int32_t* border, int BM, int cap, uint16_t* h,
                             hipStream_t stream);
hipError_t launch_w2_prefill(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                             const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                             const int32_t* border, int BM, int cap, const float* topk_w,
                             float* ys, hipStream_t stream);
// The same with bf16 slot rows (the fused layer's workspace; halves the rows' HBM traffic).
hipError_t launch_w2_prefill_bf16(const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                                  const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                                  const int32_t* border, int BM, int cap, const float* topk_w,
                                  uint16_t* ys, hipStream_t stream);

// Predictor MLP with L heads: z1 = h . w1^T over all L*D rows (fp32 [T][L*D+1]),
// a = bf16(silu(z1)) head-major [L][T][D], z2[l] = a[l] . w2[l]^T (fp32 [L][T][E+1]),
// ids/scores [L][T][top_k] = top-k of z2 (scores: renormalised softmax of the top-k).
hipError_t launch_predictor(const uint16_t* h, int T, int H, int L, const uint16_t* w1, int D,
                            const uint16_t* w2, int E, int top_k, float* z1, uint16_t* a,
                            float* z2, int32_t* ids, float* scores, hipStream_t stream);

// Residual add (add nullable) and (1 + w) RMSNorm per token row, hidden % 8 == 0, <= 8192:
// res_out = res_in + add, out = norm(res_out); res_out may be res_in.
hipError_t launch_rmsnorm(const uint16_t* res_in, const uint16_t* add, int T, int H,
                          const uint16_t* w, float eps, uint16_t* res_out, uint16_t* out,
                          hipStream_t stream);
// Decode router with the residual add + RMSNorm of its tokens folded in (router.hip): writes
// res_out, x_out (the launch_rmsnorm bits) and the logits (the launch_router_logits bits of
// x_out). T <= 64, H <= 2048, res_out != res_in.
bool router_norm_fits(int T, int H, const void* res_in, const void* res_out);
hipError_t launch_router_logits_norm(const uint16_t* res_in, const uint16_t* add,
                                     const uint16_t* norm_w, float eps, uint16_t* res_out,
                                     uint16_t* x_out, int T, int H, const uint16_t* W, int E,
                                     const uint16_t* shared_w, const float* bias, float* logits,
                                     hipStream_t stream);

// Block sizes (slots per block) of the two paths.
constexpr int kDecodeBlockM = 16;
constexpr int kPrefillBlockM = 128;
// AUTO takes the prefill path from this many routed slots (T * top_k) on: below it the decode
// kernels were faster at hidden 2048, 256 experts, intermediate 512, top-8 with Zipf skew (per
// layer 112.8 vs 118.1 us at 256 tokens, 126.5 vs 124.8 us at 320 tokens).
constexpr int kAutoPrefillSlots = 2560;

// HiddenResidualExpertPredictor forward (hr_predictor.hip).
int64_t hr_predictor_workspace(int N, int W, int F, int E);
hipError_t launch_hr_predictor(const uint16_t* x, int N, int H, const int32_t* layer_ids,
                               const moe_hr_predictor_params_v1& p, const float* prior, float scale,
                               const float* scale_per_example, int top_k, void* workspace,
                               float* out, int32_t* ids, hipStream_t stream);
