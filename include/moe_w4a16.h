/*
 * moe_w4a16.h - C ABI of the MI355X (gfx950) GPTQ-int4 W4A16 fused-MoE library
 * (libmoe_w4a16.so, built from mtp_amd/csrc/).
 *
 * Conventions (mirroring the reference's native ABI style,
 * microbench/premap_kernel_consumer/premap_payload_cache_inprocess_native_producer_stub.hip:505-595
 * and its ctypes binding in src/mtp_expert_prefetch/tracing/vllm_router_trace.py:8383-8445):
 *   - every entry point is `extern "C" int name_v1(...)`, returning 0 on success,
 *     1xx for argument/shape errors and 2xx for HIP runtime errors; the message of
 *     the last failure on the calling thread is returned by moe_w4a16_last_error();
 *   - every tensor pointer is a DEVICE pointer owned by the caller;
 *   - `stream` is a hipStream_t (NULL = the null stream); calls are stream-ordered,
 *     never synchronise the host and never allocate device memory;
 *   - bf16 and fp16 values travel as uint16_t bit patterns;
 *   - versioning: the _v1 suffix names the interface family, not its layout. Signatures and
 *     structs may change between releases under the same name (moe_sum_v1 gained topk_ids,
 *     num_experts and expert_row in ABI version 2, and moe_slot_cache_counters_v1 its two
 *     ready-time fields); MOE_W4A16_ABI_VERSION is bumped whenever any of them does. A caller
 *     must check moe_w4a16_abi_version() == MOE_W4A16_ABI_VERSION of the header it was built
 *     against before any other call (the Python binding refuses to load on a mismatch).
 *
 * Tensor layouts are the reference's repacked GPTQ layout
 * (src/mtp_expert_prefetch/repack/qwen3_moe_gptq.py:142-198, store.py:126-137),
 * stacked over experts:
 *   qweight int32 [E, K/8, N]   nibble j of qweight[e, r, n] is W[e, 8r + j, n]
 *   qzeros  int32 [E, K/G, N/8] nibble j of qzeros[e, g, c]  is Z[e, g, 8c + j]
 *   scales  fp16  [E, K/G, N]
 *   dequantised W[k, n] = (W_int - Z[g(k), n]) * S[g(k), n],  g(k) = k / G
 *   (src/mtp_expert_prefetch/repack/gptq_unpack.py:54-131).
 */
#ifndef MOE_W4A16_H
#define MOE_W4A16_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_W4A16_ABI_VERSION 2

enum {
  MOE_OK = 0,
  MOE_ERR_NULL = 101,        /* a required pointer is NULL */
  MOE_ERR_SHAPE = 102,       /* a size is out of the supported range or inconsistent */
  MOE_ERR_UNSUPPORTED = 103, /* a valid but unsupported configuration */
  MOE_ERR_WORKSPACE = 104,   /* workspace too small */
  MOE_ERR_HIP = 200          /* 200 + (hipError_t % 100): HIP runtime error */
};

/* One GPTQ projection stacked over experts (or over the slots of a pool). */
typedef struct moe_gptq_proj_v1 {
  const int32_t* qweight;
  const int32_t* qzeros;
  const uint16_t* scales;
} moe_gptq_proj_v1;

/* A set of int4 experts of one layer: gate/up [E, H/8, I], down [E, I/8, H].
 * expert_row: NULL, or a device int32 [num_experts] map from expert id to the row that holds
 *   it (an HBM slot pool).
 * expert_stride_bytes: 0 when each of the nine tensors is densely stacked over rows; otherwise
 *   the byte distance between consecutive rows of every tensor (per-expert blobs of a slot
 *   pool, with the nine base pointers at the tensors' offsets inside row 0). Multiple of 16. */
typedef struct moe_expert_set_v1 {
  moe_gptq_proj_v1 gate;
  moe_gptq_proj_v1 up;
  moe_gptq_proj_v1 down;
  const int32_t* expert_row;
  int32_t num_experts;
  int32_t hidden;
  int32_t intermediate;
  int32_t group_size;
  int64_t expert_stride_bytes;
} moe_expert_set_v1;

/* Kernel path selection for the expert GEMMs (block_m: 16 for DECODE, 128 for PREFILL).
 *   DECODE : MFMA 16x16x32 bf16 on 16-slot blocks, int4 dequantised in registers into the
 *            MFMA operand, K split across waves (token batches up to a few hundred slots);
 *   PREFILL: MFMA on 128-slot blocks, activation tiles staged in LDS, int4 dequantised in
 *            registers into the MFMA operand;
 *   AUTO   : PREFILL when T * top_k >= 2560, else DECODE.
 * Any other value is refused with MOE_ERR_UNSUPPORTED (the workspace query returns -1). */
enum { MOE_PATH_AUTO = 0, MOE_PATH_DECODE = 1, MOE_PATH_PREFILL = 2 };

int moe_w4a16_abi_version(void);
const char* moe_w4a16_last_error(void);

/* Dequantise num_experts stacked projections to bf16.
 * Replaces dequantize_gptq_projection (src/mtp_expert_prefetch/repack/gptq_unpack.py:88-131).
 * g_idx: NULL (g = k / group_size) or device int32 [num_experts, in_features]; out-of-range
 * entries are clamped (the host wrapper rejects them first, as the reference does at :119-124).
 * out_dtype: 0 bf16, 1 fp16, 2 fp32. out: [E, out, in] when linear_weight != 0, else [E, in, out].
 * Bit-exact with the reference for every output dtype (the fp32 product is exact). */
int moe_dequant_v1(const moe_gptq_proj_v1* proj, const int32_t* g_idx, int32_t num_experts,
                   int32_t in_features, int32_t out_features, int32_t group_size,
                   int32_t linear_weight, int32_t out_dtype, void* out, void* stream);

/* Router: logits = x . router_w^T (+ logit_bias) in fp32, softmax, top-k, renormalise.
 * Replaces the gate GEMV (src/mtp_expert_prefetch/mtp/extra_tensors.py:353) and vLLM
 * topk_softmax(renormalize=True) as restated at
 * src/mtp_expert_prefetch/tracing/vllm_router_trace.py:4201-4225.
 * Ties: larger logit first, equal logits (-0 equals +0) -> lower expert id; NaN ranks last.
 * x bf16 [T, H]; router_w bf16 [E, H]; logit_bias NULL or fp32 [E]; shared_gate_w NULL or
 * bf16 [H]. logits: fp32 workspace [T, E + 1]. topk_ids int32 [T, top_k];
 * topk_weights fp32 [T * top_k (+ T when shared_gate_w != NULL)]: entry T*top_k + t holds
 * sigmoid(x[t] . shared_gate_w) (extra_tensors.py:596). */
int moe_router_topk_v1(const uint16_t* x, int32_t T, int32_t hidden, const uint16_t* router_w,
                       int32_t num_experts, const float* logit_bias, int32_t top_k,
                       const uint16_t* shared_gate_w, float* logits, int32_t* topk_ids,
                       float* topk_weights, void* stream);

/* Number of block_m blocks the aligned layout may need (grid size of the GEMMs). */
int moe_capacity_blocks_v1(int32_t T, int32_t top_k, int32_t num_experts, int32_t has_shared,
                           int32_t block_m);

/* Token->expert align/sort: flat slots f = t*top_k + i (plus T shared slots T*top_k + t
 * routed to expert id num_experts when has_shared) grouped by expert (ascending), slots
 * ascending inside a group, each group padded to block_m with the sentinel
 * num_slots = T*top_k (+T). Replaces vLLM moe_align_block_size
 * (src/mtp_expert_prefetch/tracing/vllm_router_trace.py:19647-19660; format pinned by
 * tests/test_vllm_descriptor_mapping_assertion.py:1012-1085).
 * sorted_ids int32 [capacity_blocks*block_m]; expert_ids int32 [capacity_blocks] (-1 for
 * unused blocks); ntpp int32 [1]. Slots whose id is outside [0, E) are dropped. With T = 0
 * and capacity_blocks = 0 only ntpp (0) is written, and sorted_ids/expert_ids may be NULL. */
int moe_align_v1(const int32_t* topk_ids, int32_t T, int32_t top_k, int32_t num_experts,
                 int32_t has_shared, int32_t block_m, int32_t capacity_blocks,
                 int32_t* sorted_ids, int32_t* expert_ids, int32_t* ntpp, void* stream);

/* W1: h[f, :] = silu(x[tok(f)] . Wgate[e]^T) * (x[tok(f)] . Wup[e]^T) for every slot f of
 * every block (bf16 h [num_slots, I]). Replaces invoke_fused_moe_wna16_triton_kernel for
 * W1 + silu_and_mul (src/mtp_expert_prefetch/tracing/vllm_router_trace.py:19674-19718,
 * arithmetic at src/mtp_expert_prefetch/tracing/vllm_wna16_group_plan.py:367-486).
 * shared: NULL or the shared expert (expert id num_experts). sorted_ids, expert_ids and ntpp
 * are moe_align_v1's outputs for the same block_m and capacity_blocks (the kernels read
 * capacity_blocks * block_m sorted ids; the library cannot check the buffers' sizes). */
int moe_w1_gateup_silu_v1(const uint16_t* x, int32_t T, int32_t top_k,
                          const moe_expert_set_v1* experts, const moe_expert_set_v1* shared,
                          const int32_t* sorted_ids, const int32_t* expert_ids,
                          const int32_t* ntpp, int32_t block_m, int32_t capacity_blocks,
                          uint16_t* h, int32_t path, void* stream);

/* W2: ys[f, :] = topk_weights[f] * (h[f] . Wdown[e]^T), fp32 [num_slots, H].
 * Replaces the W2 dispatch with mul_routed_weight=True, top_k=1
 * (src/mtp_expert_prefetch/tracing/vllm_router_trace.py:19761-19783). Routing tables as for
 * moe_w1_gateup_silu_v1; topk_weights fp32 [num_slots]. */
int moe_w2_down_v1(const uint16_t* h, int32_t T, int32_t top_k,
                   const moe_expert_set_v1* experts, const moe_expert_set_v1* shared,
                   const int32_t* sorted_ids, const int32_t* expert_ids, const int32_t* ntpp,
                   int32_t block_m, int32_t capacity_blocks, const float* topk_weights,
                   float* ys, int32_t path, void* stream);

/* out[t, :] = bf16(sum_{i<top_k} ys[t*top_k + i, :] (+ ys[T*top_k + t, :])), fixed order.
 * Replaces ops.moe_sum (src/mtp_expert_prefetch/tracing/vllm_router_trace.py:19801-19804).
 * topk_ids (device int32 [T, top_k], required) are the routed ids the W2 rows were computed
 * for: a slot whose id is outside [0, num_experts), or whose expert has row -1 in expert_row
 * (device int32 [num_experts], NULL = identity), is dropped and its ys row is never read
 * (moe_w2_down_v1 does not write the rows of dropped slots). */
int moe_sum_v1(const float* ys, int32_t T, int32_t top_k, int32_t hidden, int32_t has_shared,
               const int32_t* topk_ids, int32_t num_experts, const int32_t* expert_row,
               uint16_t* out, void* stream);

/* Decoder-step norm around the MoE layer in a layer loop: when add != NULL,
 *   res[t, :] = bf16(res[t, :] + add[t, :])   (in place, fp32 add, round to nearest even);
 * then out[t, :] = bf16((float(res[t, :]) * rsqrt(mean(float(res[t, :])^2) + eps)) * (1 + w)).
 * Replaces mtp_rms_norm (src/mtp_expert_prefetch/mtp/extra_tensors.py:40-48) on the residual
 * stream of the decoder loop around moe_forward_with_trace
 * (src/mtp_expert_prefetch/tracing/vllm_router_trace.py:17895-17965). res, add, out: bf16
 * [T, hidden]; weight bf16 [hidden]; hidden % 8 == 0 and <= 8192; out must not alias res.
 * The mean is an fp32 sum in a fixed order. */
int moe_rmsnorm_v1(uint16_t* res, const uint16_t* add, int32_t T, int32_t hidden,
                   const uint16_t* weight, float eps, uint16_t* out, void* stream);

/* Workspace bytes for moe_layer_v1 / moe_fused_experts_v1 (no state survives between calls;
 * calls that share one workspace must be ordered on one stream). Every workspace argument of
 * this library must start on a 256-byte boundary (hipMalloc and torch allocations do); a
 * misaligned one is refused with MOE_ERR_WORKSPACE. */
int64_t moe_layer_workspace_bytes_v1(int32_t T, int32_t top_k, const moe_expert_set_v1* experts,
                                     int32_t has_shared, int32_t path);

/* Full routed layer: router -> align -> W1 -> W2 -> sum (+ sigmoid-gated shared expert).
 * Replaces fused_experts_impl (src/mtp_expert_prefetch/tracing/vllm_router_trace.py:19330-19817)
 * with its router (:17934, :21719) and MtpExtraRunner.moe_tokens
 * (src/mtp_expert_prefetch/mtp/extra_tensors.py:544-598). out bf16 [T, H].
 * topk_ids_out / topk_weights_out: NULL or int32 [T, top_k] / fp32 [T, top_k] copies. */
int moe_layer_v1(const uint16_t* x, int32_t T, const uint16_t* router_w, const float* logit_bias,
                 int32_t top_k, const moe_expert_set_v1* experts, const moe_expert_set_v1* shared,
                 const uint16_t* shared_gate_w, void* workspace, int64_t workspace_bytes,
                 uint16_t* out, int32_t* topk_ids_out, float* topk_weights_out, int32_t path,
                 void* stream);

/* A decoder step's residual add + RMSNorm in front of the routed layer, as the decoder loop runs
 * them (mtp_rms_norm, src/mtp_expert_prefetch/mtp/extra_tensors.py:40-48, before
 * moe_forward_with_trace in the layer loop of
 * src/mtp_expert_prefetch/tracing/vllm_router_trace.py:17895-17965):
 *   res_out = bf16(res_in + add)   (add NULL: res_out = res_in)
 *   x_out   = the moe_rmsnorm_v1 output of res_out with norm_w, eps
 *   out     = moe_layer_v1(x_out, ...)
 * The bits equal moe_rmsnorm_v1 followed by moe_layer_v1. On the decode path with T <= 64,
 * hidden <= 2048 and res_out != res_in the router normalises its own tokens (no separate norm
 * launch); otherwise the norm runs first. res_out may equal res_in. x_out, out and add must not
 * alias each other or the residual rows. Workspace as moe_layer_v1. */
int moe_norm_layer_v1(const uint16_t* res_in, const uint16_t* add, const uint16_t* norm_w,
                      float eps, uint16_t* res_out, uint16_t* x_out, int32_t T,
                      const uint16_t* router_w, const float* logit_bias, int32_t top_k,
                      const moe_expert_set_v1* experts, const moe_expert_set_v1* shared,
                      const uint16_t* shared_gate_w, void* workspace, int64_t workspace_bytes,
                      uint16_t* out, int32_t* topk_ids_out, float* topk_weights_out, int32_t path,
                      void* stream);

/* moe_layer_v1 without a workspace argument and without any allocation: the workspace is a
 * file-scope device array of moe_layer_noalloc_max_bytes_v1() bytes (64 MiB) per GPU, held until
 * the process ends. No counterpart in the reference: for callers that cannot call hipMalloc
 * (code under HIP graph capture, tight serving loops, harnesses that forbid allocation).
 * Returns MOE_ERR_WORKSPACE when the call needs more than that (moe_layer_workspace_bytes_v1;
 * at hidden 2048, 256 experts, intermediate 512, top-8: above about 890 tokens). Calls
 * on one GPU share its array: calls that overlap on one GPU (several streams or host threads)
 * race; calls ordered on one stream do not. */
int64_t moe_layer_noalloc_max_bytes_v1(void);
int moe_layer_noalloc_v1(const uint16_t* x, int32_t T, const uint16_t* router_w,
                         const float* logit_bias, int32_t top_k, const moe_expert_set_v1* experts,
                         const moe_expert_set_v1* shared, const uint16_t* shared_gate_w,
                         uint16_t* out, int32_t* topk_ids_out, float* topk_weights_out,
                         int32_t path, void* stream);

/* Experts with caller-given routing: topk_ids int32 [T, top_k], topk_weights fp32 [T, top_k].
 * Replaces TopKExpertMlp.forward (src/mtp_expert_prefetch/repack/gptq_unpack.py:293-327)
 * and moe_tokens with given ids (src/mtp_expert_prefetch/mtp/extra_tensors.py:544-598).
 * A slot is dropped (contributes zero) when its id is outside [0, num_experts) or, with an
 * expert_row map, names an expert whose row is negative (not resident), as the reference drops
 * ids outside [0, E) and unmapped experts (vllm_router_trace.py:14138-14153). */
int moe_fused_experts_v1(const uint16_t* x, int32_t T, const int32_t* topk_ids,
                         const float* topk_weights, int32_t top_k,
                         const moe_expert_set_v1* experts, const moe_expert_set_v1* shared,
                         const uint16_t* shared_gate_w, void* workspace, int64_t workspace_bytes,
                         uint16_t* out, int32_t path, void* stream);

/* ---------------------------------------------------------------- AWQ checkpoints */
#define MOE_AWQ_WNA16 1 /* vLLM int4 fused-MoE layout: uint8 [E, N, K/2], zeros uint8 [E, N/2, K/G] */
#define MOE_AWQ_GEMM 2  /* AutoAWQ GEMM: int32 [E, K, N/8] and [E, K/G, N/8], order 0,2,4,6,1,3,5,7 */

/* Exact repack of AWQ int4 experts into the GPTQ layout the kernels read (out: caller-allocated
 * device qweight int32 [E, K/8, N], qzeros int32 [E, K/G, N/8], scales fp16 [E, K/G, N]).
 * Replaces the AWQ weight path of the reference's production run (vLLM wna16,
 * src/mtp_expert_prefetch/tracing/vllm_wna16_group_plan.py:394-470;
 * configs/model/qwen3_6_35b_a3b_awq_4bit.yaml): every (q - z) * s is unchanged. layout
 * MOE_AWQ_WNA16: qzeros NULL = symmetric (zero 8); scales [E, N, K/G] fp16 or bf16
 * (scales_bf16 = 1). MOE_AWQ_GEMM: qweight int32 [E, K, N/8], qzeros int32 [E, K/G, N/8],
 * scales fp16 [E, K/G, N]. *status (device int32) is 0 when every value moved exactly, 1 when
 * a bf16 scale has no exact fp16 value (outside [2^-17, 65504]). Stream-ordered. */
int moe_awq_to_gptq_v1(int32_t layout, const void* qweight, const void* qzeros,
                       const uint16_t* scales, int32_t scales_bf16, int32_t num_experts,
                       int32_t in_features, int32_t out_features, int32_t group_size,
                       const moe_gptq_proj_v1* out, int32_t* status, void* stream);

/* ---------------------------------------------------------------- expert-demand predictor */

/* Parameters of the reference's HiddenResidualExpertPredictor
 * (src/mtp_expert_prefetch/training/hidden_residual.py:44-106) in bf16 (biases as fp32 holding
 * bf16 values): encoder = Linear(hidden, width) -> SiLU -> LayerNorm(width) (key names
 * encoder.0.*, encoder.2.*), layer_embedding [num_layers, width], delta_embedding
 * [future_window, width], classifier = Linear(width, num_experts). */
typedef struct moe_hr_predictor_params_v1 {
  const uint16_t* enc_w;      /* bf16 [width, hidden] */
  const float* enc_b;         /* fp32 [width] */
  const uint16_t* ln_w;       /* bf16 [width] */
  const uint16_t* ln_b;       /* bf16 [width] */
  const uint16_t* layer_emb;  /* bf16 [num_layers, width] */
  const uint16_t* delta_emb;  /* bf16 [future_window, width] */
  const uint16_t* cls_w;      /* bf16 [num_experts, width] */
  const float* cls_b;         /* fp32 [num_experts] */
  int32_t hidden, width, num_layers, future_window, num_experts;
  float ln_eps;
} moe_hr_predictor_params_v1;

/* Workspace bytes of moe_hr_predictor_v1 for N examples (-1 on bad arguments). */
int64_t moe_hr_predictor_workspace_bytes_v1(int32_t N, const moe_hr_predictor_params_v1* params);

/* HiddenResidualExpertPredictor.forward(hidden [N, hidden] bf16, layer_ids [N] int32) ->
 * residual [N, future_window, num_experts], combined as out = prior + scale * residual
 * (train_hidden_residual_predictor_smoke.py:446; prior NULL = 0; scale = scale_per_example[n]
 * when given, else residual_scale, as apply_residual_scale :108-121 with a fixed or learnt
 * gamma), and the top_k experts of every (example, delta) row by (value, lower id).
 * Activations between the Linear layers are bf16; the dot products use the router's canonical
 * fp32 order. A layer id outside [0, num_layers) reads a zero embedding. logits_out: NULL or
 * fp32 [N, future_window, num_experts]; topk_ids int32 [N, future_window, top_k]. */
int moe_hr_predictor_v1(const uint16_t* hidden, int32_t N, const int32_t* layer_ids,
                        const moe_hr_predictor_params_v1* params, const float* prior,
                        float residual_scale, const float* scale_per_example, int32_t top_k,
                        void* workspace, int64_t workspace_bytes, float* logits_out,
                        int32_t* topk_ids, void* stream);

/* Workspace bytes of moe_predictor_v1. */
int64_t moe_predictor_workspace_bytes_v1(int32_t T, int32_t num_heads, int32_t inner,
                                         int32_t num_experts, int32_t top_k);

/* Top-k experts per layer head predicted from one hidden state by a bf16 MLP per head:
 * logits[l] = bf16(silu(h . w1[l]^T)) . w2[l]^T in fp32, top-k by (logit desc, id asc).
 * Replaces the forward of the reference's per-layer predictor
 * (src/mtp_expert_prefetch/training/hidden_residual.py:44-106), simplified to
 * hidden -> inner (SiLU) -> num_experts with one weight set per layer. h bf16 [T, hidden];
 * w1 bf16 [num_heads, inner, hidden]; w2 bf16 [num_heads, num_experts, inner];
 * topk_ids int32 [num_heads, T, top_k]. */
int moe_predictor_v1(const uint16_t* h, int32_t T, int32_t hidden, int32_t num_heads,
                     const uint16_t* w1, int32_t inner, const uint16_t* w2, int32_t num_experts,
                     int32_t top_k, void* workspace, int64_t workspace_bytes, int32_t* topk_ids,
                     void* stream);

/* ------------------------------------------------------------------ offloaded slot cache */

/* Expert blobs (expert_bytes each, the nine GPTQ tensors of one expert back to back) for every
 * (layer, expert) in pinned host memory, and slots_per_layer slots per layer in HBM. The kernels
 * read a layer's slots through moe_expert_set_v1 with expert_row = device_expert_row + layer *
 * num_experts and expert_stride_bytes = expert_bytes. dry_run = 1 keeps only the accounting
 * (no HIP calls; pools may be NULL). */
typedef struct moe_slot_cache_desc_v1 {
  int32_t num_layers;
  int32_t num_experts;
  int32_t slots_per_layer;
  int32_t device;
  int64_t expert_bytes;
  const void* host_pool;      /* pinned host [num_layers][num_experts][expert_bytes] */
  void* device_pool;          /* device [num_layers][slots_per_layer][expert_bytes] */
  int32_t* device_expert_row; /* device [num_layers][num_experts]: expert -> slot, -1 when not
                               resident (its slots are dropped); the caller initialises it */
  int32_t dry_run;
  float ready_deadline_us;    /* a prefetched expert is ready-late when its copy completes more
                               than this after the demand that first uses it */
} moe_slot_cache_desc_v1;

/* Counters with the semantics of ControlledExpertCacheManager
 * (src/mtp_expert_prefetch/runtime/cache_manager.py:208-279), plus bytes moved. */
typedef struct moe_slot_cache_counters_v1 {
  int64_t capacity;
  int64_t resident_count;
  int64_t issued_fetch_count;
  int64_t used_fetch_count;
  int64_t unused_fetch_count;
  int64_t demand_count;
  int64_t demand_hit_count;
  int64_t demand_miss_count;
  int64_t evicted_before_use_count;
  int64_t prefetch_bytes;
  int64_t demand_bytes;
  int64_t prefetch_skipped_pinned_count; /* prefetches not issued: every slot was pinned */
  /* ReadyTimeExpertCacheManager (cache_manager.py:298-578) on real transfers: first demands of a
   * prefetched expert whose copy completed after the demand (+ ready_deadline_us), measured
   * with HIP event timestamps, and their total lateness. The reference counts such a demand as
   * a miss (ready_late_miss_count); here the layer waits for the copy, so the data counters
   * above still count it as a hit. */
  int64_t ready_late_miss_count;
  int64_t ready_late_wait_ns;
} moe_slot_cache_counters_v1;

/* Opaque handle (a magic field is checked on every call). Not thread-safe. */
int moe_slot_cache_create_v1(const moe_slot_cache_desc_v1* desc, uint64_t* handle);
int moe_slot_cache_destroy_v1(uint64_t handle);

/* Prefetch experts (host int32 list) of one layer on the cache's side stream (hipMemcpyAsync),
 * ordered after every kernel already enqueued on compute_stream. Replaces
 * ControlledExpertCacheManager.issue_prefetch (cache_manager.py:222-231) with real transfers.
 * A prefetch never evicts a slot named by the layer's latest demand until
 * moe_slot_cache_layer_done_v1(layer) (those slots may be read by kernels not yet enqueued);
 * an expert for which only such slots remain is skipped. issued: NULL or the number of copies
 * started.
 * Call order per layer on one compute stream: demand -> enqueue the layer's kernels ->
 * layer_done -> prefetch (for later steps). Prefetching between demand and layer_done is safe
 * too, with the pinned slots kept out of the LRU choice. */
int moe_slot_cache_prefetch_v1(uint64_t handle, int32_t layer, const int32_t* experts, int32_t n,
                               void* compute_stream, int32_t* issued);

/* Make experts of one layer resident before the layer runs on compute_stream: waits for the
 * layer's prefetches, fetches misses on compute_stream, uploads the expert -> slot table.
 * Replaces ControlledExpertCacheManager.demand (cache_manager.py:233-247). hits: NULL or the
 * number of hits. */
int moe_slot_cache_demand_v1(uint64_t handle, int32_t layer, const int32_t* experts, int32_t n,
                             void* compute_stream, int32_t* hits);

/* The kernels that read layer's slots (after its latest demand) are enqueued: its slots may be
 * evicted by prefetches again. Host bookkeeping only; no HIP call. No reference counterpart
 * (the reference's cache moves no bytes, so it has no read-after-demand hazard). */
int moe_slot_cache_layer_done_v1(uint64_t handle, int32_t layer);

int moe_slot_cache_stats_v1(uint64_t handle, moe_slot_cache_counters_v1* out);

/* Slot of (layer, expert), -1 if absent, -2 for a bad handle or index. */
int moe_slot_cache_slot_of_v1(uint64_t handle, int32_t layer, int32_t expert);

/* One offloaded MoE layer of a decode step in one call: router logits and top-k into the
 * workspace, the routed ids to ids_host (host, T * top_k int32; the call waits for them on
 * stream: memory from hipHostMalloc receives them from the top-k kernel itself, other host
 * memory through a copy), moe_slot_cache_demand_v1, the routed experts from the layer's slots (experts = the
 * layer's slot view, as for moe_fused_experts_v1), when n_prefetch > 0 the prefetch of the host
 * list prefetch (as moe_slot_cache_prefetch_v1, with the demand's slots still pinned and without
 * the copy streams' wait for the compute stream, which the ids' wait has already drained), then
 * moe_slot_cache_layer_done_v1. Replaces the per-layer
 * sequence of the reference's offloaded decode (router top-k, then
 * ControlledExpertCacheManager.demand, cache_manager.py:233-247, then the expert MLPs, then
 * issue_prefetch, :222-231) with one host call. Workspace as moe_layer_v1 (no shared expert).
 * hits: NULL or the demand's hits. */
int moe_offload_layer_v1(uint64_t cache, int32_t layer, const uint16_t* x, int32_t T,
                         const uint16_t* router_w, const float* logit_bias, int32_t top_k,
                         const moe_expert_set_v1* experts, void* workspace,
                         int64_t workspace_bytes, uint16_t* out, int32_t* ids_host,
                         const int32_t* prefetch, int32_t n_prefetch, int32_t path, void* stream,
                         int32_t* hits);

/* ---- Cache accounting on virtual time (host only: no HIP call, no payload bytes).
 * The reference's cache-lab managers for a trace of prefetch issues and demands with arrival
 * times (microseconds, nondecreasing for meaningful queue timing). Keys are (layer, expert);
 * one LRU of `capacity` keys over all layers, as in the reference.
 *   MOE_READY_CACHE_CONTROLLED: ControlledExpertCacheManager (cache_manager.py:208-279): a
 *     prefetch of a missing key enters the LRU at once; arrival times are ignored.
 *   MOE_READY_CACHE_READY_TIME: ReadyTimeExpertCacheManager (cache_manager.py:298-578): issues
 *     are served in batches of queue_batch_size by one server (service_us_per_batch +
 *     service_us_per_issue per issue, a partial batch released queue_deadline_us after its first
 *     issue or at finish); a transfer's key enters the LRU at its completion time; a demand hits
 *     only keys completed by arrival + queue_deadline_us; a demand of an in-flight key is a miss
 *     and a ready-late miss, and that transfer's completion counts as a late completion left
 *     unused.
 * Non-finite service times or deadline are refused (MOE_ERR_SHAPE, the reference's ValueError);
 * negative ones are clamped to 0 and a batch size below 1 to 1. Not thread-safe. */
enum { MOE_READY_CACHE_CONTROLLED = 0, MOE_READY_CACHE_READY_TIME = 1 };

/* Counters of CacheManagerSnapshot / ReadyTimeCacheManagerSnapshot (cache_manager.py:192-205,
 * 282-295), same names and meaning. */
typedef struct moe_ready_cache_snapshot_v1 {
  int64_t capacity;
  int64_t resident_count;
  int64_t issued_fetch_count;
  int64_t used_fetch_count;
  int64_t unused_fetch_count; /* resident unused prefetches + late completions left unused */
  int64_t demand_count;
  int64_t demand_hit_count;
  int64_t demand_miss_count;
  int64_t evicted_before_use_count;
  int64_t ready_late_miss_count;
  int64_t late_completion_unused_count;
  int64_t queue_batch_count;
  double queue_service_us;
  double queue_total_span_us;
  double queue_wait_us;
  double queue_max_delay_us;
  double queue_event_interval_us;
  double queue_deadline_us;
  int64_t queue_batch_size;
} moe_ready_cache_snapshot_v1;

/* Replaces the managers' constructors (cache_manager.py:211-219, 309-354). */
int moe_ready_cache_create_v1(int32_t mode, int64_t capacity, double service_us_per_issue,
                              double service_us_per_batch, int64_t queue_batch_size,
                              double queue_deadline_us, uint64_t* handle);
int moe_ready_cache_destroy_v1(uint64_t handle);

/* issue_prefetch of each expert of `experts` (host int32 [n]) in order at one arrival time
 * (cache_manager.py:221-230, 356-378; issue_prefetches :380-397). issued_flags: NULL or host
 * int32 [n] (1 = a new transfer); issued: NULL or the count. */
int moe_ready_cache_prefetch_v1(uint64_t handle, int32_t layer, const int32_t* experts,
                                int32_t n, double arrival_us, int32_t* issued_flags,
                                int32_t* issued);

/* demand of each expert in order at one arrival time (cache_manager.py:232-247, 399-425).
 * hit_flags: NULL or host int32 [n]; hits: NULL or the count. */
int moe_ready_cache_demand_v1(uint64_t handle, int32_t layer, const int32_t* experts, int32_t n,
                              double arrival_us, int32_t* hit_flags, int32_t* hits);

/* advance_to (cache_manager.py:427-433) and finish (:435-453); no-ops for CONTROLLED. */
int moe_ready_cache_advance_v1(uint64_t handle, double arrival_us);
int moe_ready_cache_finish_v1(uint64_t handle);

/* snapshot (cache_manager.py:249-262, 455-485). */
int moe_ready_cache_stats_v1(uint64_t handle, moe_ready_cache_snapshot_v1* out);

#ifdef __cplusplus
}
#endif

#endif /* MOE_W4A16_H */
