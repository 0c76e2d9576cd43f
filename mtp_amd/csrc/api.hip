// extern "C" entry points of libmoe_w4a16.so: argument validation, workspace carving and
// stream-ordered orchestration of the kernels. No entry point allocates device memory; none
// synchronises the host except the offload layer call, which waits for its routed ids.
#include <atomic>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>

#include "common.h"
#include "launch.h"

char* moe_error_buffer() {
  thread_local char buf[kErrorBufferBytes] = "";
  return buf;
}

namespace {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(moe_error_buffer(), kErrorBufferBytes, fmt, ap);
  va_end(ap);
  return code;
}

// The error is reported through the return code and the message; the thread's last HIP error
// is cleared so that it does not surface again at the caller's next, unrelated HIP call.
int hip_fail(hipError_t e, const char* where) {
  (void)hipGetLastError();
  return fail(MOE_ERR_HIP + ((int)e % 100), "%s: HIP error %d (%s)", where, (int)e,
              hipGetErrorString(e));
}

#define MOE_CHECK_HIP(expr, where)                 \
  do {                                             \
    hipError_t _e = (expr);                        \
    if (_e != hipSuccess) return hip_fail(_e, where); \
  } while (0)

bool proj_ok(const moe_gptq_proj_v1& p) { return p.qweight && p.qzeros && p.scales; }

ProjDev to_dev(const moe_gptq_proj_v1& p) { return ProjDev{p.qweight, p.qzeros, p.scales}; }

// Shapes every GEMM kernel supports (checked once per call).
int check_experts(const moe_expert_set_v1* ex, const moe_expert_set_v1* sh) {
  if (!ex) return fail(MOE_ERR_NULL, "experts is NULL");
  if (!proj_ok(ex->gate) || !proj_ok(ex->up) || !proj_ok(ex->down))
    return fail(MOE_ERR_NULL, "an expert projection pointer is NULL");
  const int H = ex->hidden, I = ex->intermediate, G = ex->group_size;
  if (ex->num_experts < 1 || ex->num_experts > 512)
    return fail(MOE_ERR_SHAPE, "num_experts=%d outside [1, 512]", ex->num_experts);
  if (H < 512 || H > 2048 || H % 512 != 0)
    return fail(MOE_ERR_SHAPE, "hidden=%d must be a multiple of 512 in [512, 2048]", H);
  if (!(I == 256 || I == 512 || I == 1024))
    return fail(MOE_ERR_SHAPE, "intermediate=%d must be one of 256, 512, 1024", I);
  if (!(G == 64 || G == 128 || G == 256) || H % G != 0 || I % G != 0)
    return fail(MOE_ERR_SHAPE, "group_size=%d unsupported for hidden=%d intermediate=%d", G, H,
                I);
  if (ex->expert_stride_bytes < 0 || ex->expert_stride_bytes % 16 != 0)
    return fail(MOE_ERR_SHAPE, "expert_stride_bytes=%lld must be a non-negative multiple of 16",
                (long long)ex->expert_stride_bytes);
  if (ex->expert_stride_bytes != 0 && !ex->expert_row)
    return fail(MOE_ERR_NULL, "a strided expert pool needs the expert_row map");
  if (sh) {
    if (!proj_ok(sh->gate) || !proj_ok(sh->up) || !proj_ok(sh->down))
      return fail(MOE_ERR_NULL, "a shared-expert projection pointer is NULL");
    if (sh->num_experts != 1 || sh->hidden != H || sh->intermediate != I || sh->group_size != G)
      return fail(MOE_ERR_SHAPE, "shared expert must be one expert of the routed experts' shape");
  }
  return MOE_OK;
}

ExpertsDev make_experts_dev(const moe_expert_set_v1* ex, const moe_expert_set_v1* sh) {
  ExpertsDev d{};
  d.gate = to_dev(ex->gate);
  d.up = to_dev(ex->up);
  d.down = to_dev(ex->down);
  if (sh) {
    d.sgate = to_dev(sh->gate);
    d.sup = to_dev(sh->up);
    d.sdown = to_dev(sh->down);
  }
  d.expert_row = ex->expert_row;
  d.row_stride = ex->expert_stride_bytes;
  d.num_experts = ex->num_experts;
  d.hidden = ex->hidden;
  d.inter = ex->intermediate;
  d.group = ex->group_size;
  return d;
}

// The path the kernels run (AUTO resolved from the slot count); -1 for an unknown value.
int resolve_path(int path, int T, int top_k) {
  if (path == MOE_PATH_DECODE || path == MOE_PATH_PREFILL) return path;
  if (path != MOE_PATH_AUTO) return -1;
  return ((int64_t)T * top_k >= kAutoPrefillSlots) ? MOE_PATH_PREFILL : MOE_PATH_DECODE;
}

int block_m_of(int path) { return path == MOE_PATH_PREFILL ? kPrefillBlockM : kDecodeBlockM; }

hipError_t dispatch_w1(int path, const uint16_t* x, const ExpertsDev& ed, const SlotsDev& sd,
                       const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                       const int32_t* border, int bm, int cap, uint16_t* h, hipStream_t s) {
  if (path == MOE_PATH_PREFILL)
    return launch_w1_prefill(x, ed, sd, sorted, eids, ntpp, border, bm, cap, h, s);
  return launch_w1_decode_mfma(x, ed, sd, sorted, eids, ntpp, cap, h, s);
}

hipError_t dispatch_w2(int path, const uint16_t* h, const ExpertsDev& ed, const SlotsDev& sd,
                       const int32_t* sorted, const int32_t* eids, const int32_t* ntpp,
                       const int32_t* border, int bm, int cap, const float* w, float* ys,
                       hipStream_t s) {
  if (path == MOE_PATH_PREFILL)
    return launch_w2_prefill(h, ed, sd, sorted, eids, ntpp, border, bm, cap, w, ys, s);
  return launch_w2_decode_mfma(h, ed, sd, sorted, eids, ntpp, cap, w, ys, s);
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// Workspace of moe_layer_v1 / moe_fused_experts_v1 (no state survives between calls).
struct Workspace {
  size_t logits, norms, ids, w, sorted, eids, ntpp, border, h, ys, total;
  int cap, bm;
};

Workspace layout(int T, int top_k, const moe_expert_set_v1* ex, int has_shared, int path) {
  Workspace L{};
  const int E = ex->num_experts, H = ex->hidden, I = ex->intermediate;
  const size_t slots = (size_t)T * top_k + (has_shared ? T : 0);
  L.bm = block_m_of(path);
  L.cap = align_capacity_blocks(T, top_k, E, has_shared, L.bm);
  size_t o = 0;
  L.logits = o; o += align256((size_t)T * (E + 1) * 4);
  L.norms = o;  o += align256((size_t)(E + 1) * 4);  // router-row norms of the prefill router
  L.ids = o;    o += align256((size_t)T * top_k * 4);
  L.w = o;      o += align256(slots * 4);
  L.sorted = o; o += align256((size_t)L.cap * L.bm * 4);
  L.eids = o;   o += align256((size_t)L.cap * 4);
  L.ntpp = o;   o += 256;
  L.border = o; o += align256((size_t)L.cap * 4);  // block order of the large-input align
  L.h = o;      o += align256(slots * I * 2);
  // ys: fp32 slot rows, or at one or two decode tokens the fused W1+W2 partial rows
  size_t ys_bytes = slots * H * 4;
  if (path == MOE_PATH_DECODE && T <= kGridTopkMaxTokens)
    ys_bytes = std::max(ys_bytes, slots * (size_t)(I / 32) * H * 4);
  L.ys = o;     o += align256(ys_bytes);
  L.total = o;
  return L;
}

template <typename T>
T* at(void* base, size_t off) { return reinterpret_cast<T*>(static_cast<char*>(base) + off); }

// How run_experts finds each slot's expert.
enum Routing {
  ROUTE_ALIGN,          // ids/weights in place: align, then the blocked kernels
  ROUTE_ALIGNED,        // the sorted slot layout is in place too
  ROUTE_GRID_LOGITS,    // slot grid: W1 computes the top-k from the logits and publishes it
  ROUTE_GRID_IDS        // slot grid over the ids/weights in place
};

// [align ->] W1 -> W2 -> top-k sum over a routed workspace.
int run_experts(const uint16_t* x, int T, int top_k, const moe_expert_set_v1* ex,
                const moe_expert_set_v1* sh, const Workspace& L, void* ws, uint16_t* out,
                int path, Routing routing, hipStream_t stream) {
  const int has_shared = sh ? 1 : 0;
  const ExpertsDev ed = make_experts_dev(ex, sh);
  SlotsDev sd{T, top_k, T * top_k + (has_shared ? T : 0)};
  int32_t* ids = at<int32_t>(ws, L.ids);
  float* w = at<float>(ws, L.w);
  int32_t* sorted = at<int32_t>(ws, L.sorted);
  int32_t* eids = at<int32_t>(ws, L.eids);
  int32_t* ntpp = at<int32_t>(ws, L.ntpp);
  uint16_t* h = at<uint16_t>(ws, L.h);
  float* ys = at<float>(ws, L.ys);
  // The large-input align keeps its ranks and chunk counts in the ys section (not in use until
  // W2). Every align form also orders the blocks heaviest first for the prefill GEMMs.
  int32_t* scratch = nullptr;
  if (routing == ROUTE_ALIGN) {
    const int64_t scratch_bytes =
        align_scratch_bytes(T, top_k, ex->num_experts, has_shared, L.bm, L.cap);
    if (scratch_bytes > 0 && (size_t)scratch_bytes <= L.total - L.ys) scratch = at<int32_t>(ws, L.ys);
  }
  int32_t* border =
      routing == ROUTE_ALIGN && path == MOE_PATH_PREFILL ? at<int32_t>(ws, L.border) : nullptr;
  const bool grid = routing == ROUTE_GRID_LOGITS || routing == ROUTE_GRID_IDS;
  if (grid) {
    const SlotGrid sg{1, routing == ROUTE_GRID_LOGITS ? at<float>(ws, L.logits) : nullptr, ids, w};
    const int nct = ex->intermediate / 32;
    if (T <= kGridTopkMaxTokens && w1w2_fused_fits(ed, sd) &&
        partial_sum_fits(top_k, has_shared, ex->hidden, nct)) {
      // one or two tokens: W2 runs inside the W1 workgroups (weighted partial rows per W1
      // column block), then one fixed-order sum per token
      MOE_CHECK_HIP(launch_w1w2_slotgrid(x, ed, sd, sg, ys, stream), "w1 + w2 (slot grid)");
      MOE_CHECK_HIP(launch_partial_sum(ys, T, top_k, ex->hidden, nct, has_shared, out, stream),
                    "partial sum");
      return MOE_OK;
    }
    MOE_CHECK_HIP(launch_w1_decode_slotgrid(x, ed, sd, sg, h, stream), "w1 (slot grid)");
  } else {
    if (routing == ROUTE_ALIGN) {
      MOE_CHECK_HIP(launch_align(ids, T, top_k, ex->num_experts, has_shared, L.bm, L.cap, sorted,
                                 eids, ntpp, border, scratch, stream), "align");
    }
    MOE_CHECK_HIP(dispatch_w1(path, x, ed, sd, sorted, eids, ntpp, border, L.bm, L.cap, h, stream),
                  "w1");
  }
  if (path == MOE_PATH_DECODE && w2_token_sum_fits(ed, sd)) {
    MOE_CHECK_HIP(launch_w2_token_sum(h, ed, sd, ids, w, out, stream), "w2 + sum");
    return MOE_OK;
  }
  if (path == MOE_PATH_PREFILL) {  // bf16 slot rows: half the rows' HBM traffic
    uint16_t* ys16 = at<uint16_t>(ws, L.ys);
    MOE_CHECK_HIP(launch_w2_prefill_bf16(h, ed, sd, sorted, eids, ntpp, border, L.bm, L.cap, w, ys16,
                                         stream), "w2");
    MOE_CHECK_HIP(launch_moe_sum_bf16(ys16, T, top_k, ex->hidden, has_shared, ids,
                                      ex->num_experts, ex->expert_row, out, stream),
                  "moe_sum");
    return MOE_OK;
  }
  if (grid)
    MOE_CHECK_HIP(launch_w2_decode_slotgrid(h, ed, sd, SlotGrid{1, nullptr, ids, w}, ys, stream),
                  "w2 (slot grid)");
  else
    MOE_CHECK_HIP(dispatch_w2(path, h, ed, sd, sorted, eids, ntpp, nullptr, L.bm, L.cap, w, ys,
                              stream),
                  "w2");
  MOE_CHECK_HIP(launch_moe_sum(ys, T, top_k, ex->hidden, has_shared, ids, ex->num_experts,
                               ex->expert_row, out, stream),
                "moe_sum");
  return MOE_OK;
}

// The layer's routing for a caller that asked for it (ids_out / weights_out nullable).
int copy_routing(const int32_t* ids, const float* w, int T, int top_k, int32_t* ids_out,
                 float* weights_out, hipStream_t s) {
  if (ids_out)
    MOE_CHECK_HIP(hipMemcpyAsync(ids_out, ids, (size_t)T * top_k * 4, hipMemcpyDeviceToDevice, s),
                  "copy ids");
  if (weights_out)
    MOE_CHECK_HIP(hipMemcpyAsync(weights_out, w, (size_t)T * top_k * 4, hipMemcpyDeviceToDevice,
                                 s),
                  "copy weights");
  return MOE_OK;
}

}  // namespace

extern "C" {

int moe_w4a16_abi_version(void) { return MOE_W4A16_ABI_VERSION; }

const char* moe_w4a16_last_error(void) { return moe_error_buffer(); }

int64_t moe_predictor_workspace_bytes_v1(int32_t T, int32_t num_heads, int32_t inner,
                                         int32_t num_experts, int32_t top_k) {
  if (T < 0 || num_heads < 1 || inner < 1 || num_experts < 1 || top_k < 1) return -1;
  const size_t L = num_heads;
  return (int64_t)(align256((size_t)T * (L * inner + 1) * 4) + align256(L * T * inner * 2) +
                   align256(L * T * (num_experts + 1) * 4) + align256(L * T * top_k * 4));
}

int moe_predictor_v1(const uint16_t* h, int32_t T, int32_t hidden, int32_t num_heads,
                     const uint16_t* w1, int32_t inner, const uint16_t* w2, int32_t num_experts,
                     int32_t top_k, void* workspace, int64_t workspace_bytes, int32_t* topk_ids,
                     void* stream) {
  if (T < 0) return fail(MOE_ERR_SHAPE, "predictor: T=%d", T);
  if (T == 0) return MOE_OK;
  if (!h || !w1 || !w2 || !workspace || !topk_ids) return fail(MOE_ERR_NULL, "predictor: NULL pointer");
  if (hidden <= 0 || hidden % 8 != 0 || inner <= 0 || inner % 8 != 0)
    return fail(MOE_ERR_SHAPE, "predictor: hidden=%d inner=%d must be multiples of 8", hidden, inner);
  if (num_heads < 1 || num_heads > 1024 || (int64_t)num_heads * inner > (1 << 24))
    return fail(MOE_ERR_SHAPE, "predictor: num_heads=%d", num_heads);
  if ((int64_t)T * num_heads > (1 << 24)) return fail(MOE_ERR_SHAPE, "predictor: T * num_heads too large");
  // The GEMV kernels address w1 ([L*D, H] bf16), w2 ([L*E, D] bf16) and h through 32-bit
  // buffer offsets: every byte offset must stay below 2^31.
  if ((int64_t)num_heads * inner * hidden * 2 >= (int64_t(1) << 31) ||
      (int64_t)num_heads * num_experts * inner * 2 >= (int64_t(1) << 31) ||
      (int64_t)T * hidden * 2 >= (int64_t(1) << 31))
    return fail(MOE_ERR_SHAPE, "predictor: weights of %d heads (inner %d, hidden %d) exceed 2 GiB",
                num_heads, inner, hidden);
  if (num_experts < 1 || num_experts > 512 || top_k < 1 || top_k > num_experts || top_k > 64)
    return fail(MOE_ERR_SHAPE, "predictor: num_experts=%d top_k=%d", num_experts, top_k);
  if (workspace_bytes < moe_predictor_workspace_bytes_v1(T, num_heads, inner, num_experts, top_k))
    return fail(MOE_ERR_WORKSPACE, "predictor: workspace too small");
  if (!workspace_aligned(workspace))
    return fail(MOE_ERR_WORKSPACE, "predictor: workspace must be 256-byte aligned");
  const size_t L = num_heads;
  char* ws = static_cast<char*>(workspace);
  float* z1 = reinterpret_cast<float*>(ws);
  ws += align256((size_t)T * (L * inner + 1) * 4);
  uint16_t* a = reinterpret_cast<uint16_t*>(ws);
  ws += align256(L * T * inner * 2);
  float* z2 = reinterpret_cast<float*>(ws);
  ws += align256(L * T * (num_experts + 1) * 4);
  float* scores = reinterpret_cast<float*>(ws);
  MOE_CHECK_HIP(launch_predictor(h, T, hidden, num_heads, w1, inner, w2, num_experts, top_k, z1,
                                 a, z2, topk_ids, scores, (hipStream_t)stream), "predictor");
  return MOE_OK;
}

int moe_dequant_v1(const moe_gptq_proj_v1* proj, const int32_t* g_idx, int32_t num_experts,
                   int32_t in_features, int32_t out_features, int32_t group_size,
                   int32_t linear_weight, int32_t out_dtype, void* out, void* stream) {
  if (!proj || !proj_ok(*proj) || !out) return fail(MOE_ERR_NULL, "dequant: NULL pointer");
  if (out_dtype < 0 || out_dtype > 2)
    return fail(MOE_ERR_UNSUPPORTED, "dequant: out_dtype=%d (0 bf16, 1 fp16, 2 fp32)", out_dtype);
  if (num_experts < 1 || num_experts > 65535)
    return fail(MOE_ERR_SHAPE, "dequant: num_experts=%d", num_experts);
  if (in_features <= 0 || in_features % 8 != 0 || out_features <= 0 || out_features % 8 != 0)
    return fail(MOE_ERR_SHAPE, "dequant: in=%d out=%d must be positive multiples of 8",
                in_features, out_features);
  if (in_features / 8 > 65535) return fail(MOE_ERR_SHAPE, "dequant: in_features too large");
  if (group_size <= 0 || in_features % group_size != 0)
    return fail(MOE_ERR_SHAPE, "dequant: group_size=%d does not divide in_features=%d",
                group_size, in_features);
  MOE_CHECK_HIP(launch_dequant(to_dev(*proj), g_idx, num_experts, in_features, out_features,
                               group_size, linear_weight, out_dtype, out, (hipStream_t)stream),
                "dequant");
  return MOE_OK;
}

int moe_router_topk_v1(const uint16_t* x, int32_t T, int32_t hidden, const uint16_t* router_w,
                       int32_t num_experts, const float* logit_bias, int32_t top_k,
                       const uint16_t* shared_gate_w, float* logits, int32_t* topk_ids,
                       float* topk_weights, void* stream) {
  if (T < 0) return fail(MOE_ERR_SHAPE, "router: T=%d", T);
  if (T == 0) return MOE_OK;
  if (!x || !router_w || !logits || !topk_ids || !topk_weights)
    return fail(MOE_ERR_NULL, "router: NULL pointer");
  if (hidden <= 0 || hidden % 8 != 0) return fail(MOE_ERR_SHAPE, "router: hidden=%d", hidden);
  if (num_experts < 1 || num_experts > 512)
    return fail(MOE_ERR_SHAPE, "router: num_experts=%d outside [1, 512]", num_experts);
  if (top_k < 1 || top_k > num_experts || top_k > 64)
    return fail(MOE_ERR_SHAPE, "router: top_k=%d outside [1, min(num_experts, 64)]", top_k);
  hipStream_t s = (hipStream_t)stream;
  MOE_CHECK_HIP(launch_router_logits(x, T, hidden, router_w, num_experts, shared_gate_w,
                                     logit_bias, logits, s), "router logits");
  MOE_CHECK_HIP(launch_router_topk(logits, T, num_experts, top_k, shared_gate_w ? 1 : 0, topk_ids,
                                   topk_weights, s), "router topk");
  return MOE_OK;
}

int moe_capacity_blocks_v1(int32_t T, int32_t top_k, int32_t num_experts, int32_t has_shared,
                           int32_t block_m) {
  if (T < 0 || top_k < 1 || num_experts < 1 || block_m < 1) return 0;
  return align_capacity_blocks(T, top_k, num_experts, has_shared ? 1 : 0, block_m);
}

int moe_align_v1(const int32_t* topk_ids, int32_t T, int32_t top_k, int32_t num_experts,
                 int32_t has_shared, int32_t block_m, int32_t capacity_blocks,
                 int32_t* sorted_ids, int32_t* expert_ids, int32_t* ntpp, void* stream) {
  // No tokens and no capacity: only ntpp (0) is written, and the empty tables may be NULL.
  if (!ntpp || (capacity_blocks > 0 && (!sorted_ids || !expert_ids)) || (T > 0 && !topk_ids))
    return fail(MOE_ERR_NULL, "align: NULL pointer");
  if (T < 0 || top_k < 1 || top_k > 64) return fail(MOE_ERR_SHAPE, "align: T=%d top_k=%d", T, top_k);
  if (capacity_blocks < 0) return fail(MOE_ERR_SHAPE, "align: capacity_blocks=%d", capacity_blocks);
  if (num_experts < 1 || num_experts > 512)
    return fail(MOE_ERR_SHAPE, "align: num_experts=%d outside [1, 512]", num_experts);
  if (block_m < 1 || block_m > 1024) return fail(MOE_ERR_SHAPE, "align: block_m=%d", block_m);
  if ((int64_t)T * (top_k + 1) > (1 << 22)) return fail(MOE_ERR_SHAPE, "align: too many slots");
  const int need = align_capacity_blocks(T, top_k, num_experts, has_shared ? 1 : 0, block_m);
  if (capacity_blocks < need)
    return fail(MOE_ERR_WORKSPACE, "align: capacity_blocks=%d < required %d", capacity_blocks,
                need);
  MOE_CHECK_HIP(launch_align(topk_ids, T, top_k, num_experts, has_shared ? 1 : 0, block_m,
                             capacity_blocks, sorted_ids, expert_ids, ntpp, nullptr, nullptr,
                             (hipStream_t)stream),
                "align");
  return MOE_OK;
}

int moe_w1_gateup_silu_v1(const uint16_t* x, int32_t T, int32_t top_k,
                          const moe_expert_set_v1* experts, const moe_expert_set_v1* shared,
                          const int32_t* sorted_ids, const int32_t* expert_ids,
                          const int32_t* ntpp, int32_t block_m, int32_t capacity_blocks,
                          uint16_t* h, int32_t path, void* stream) {
  int rc = check_experts(experts, shared);
  if (rc) return rc;
  if (T < 0 || top_k < 1) return fail(MOE_ERR_SHAPE, "w1: T=%d top_k=%d", T, top_k);
  if (T == 0) return MOE_OK;
  if (!x || !sorted_ids || !expert_ids || !ntpp || !h) return fail(MOE_ERR_NULL, "w1: NULL pointer");
  const int path_in = path;
  path = resolve_path(path, T, top_k);
  if (path < 0) return fail(MOE_ERR_UNSUPPORTED, "w1: unknown path %d", path_in);
  if (block_m != block_m_of(path))
    return fail(MOE_ERR_UNSUPPORTED, "w1: block_m=%d, path %d needs %d", block_m, path,
                block_m_of(path));
  const ExpertsDev ed = make_experts_dev(experts, shared);
  const SlotsDev sd{T, top_k, T * top_k + (shared ? T : 0)};
  MOE_CHECK_HIP(dispatch_w1(path, x, ed, sd, sorted_ids, expert_ids, ntpp, nullptr, block_m,
                            capacity_blocks, h, (hipStream_t)stream), "w1");
  return MOE_OK;
}

int moe_w2_down_v1(const uint16_t* h, int32_t T, int32_t top_k,
                   const moe_expert_set_v1* experts, const moe_expert_set_v1* shared,
                   const int32_t* sorted_ids, const int32_t* expert_ids, const int32_t* ntpp,
                   int32_t block_m, int32_t capacity_blocks, const float* topk_weights,
                   float* ys, int32_t path, void* stream) {
  int rc = check_experts(experts, shared);
  if (rc) return rc;
  if (T < 0 || top_k < 1) return fail(MOE_ERR_SHAPE, "w2: T=%d top_k=%d", T, top_k);
  if (T == 0) return MOE_OK;
  if (!h || !sorted_ids || !expert_ids || !ntpp || !topk_weights || !ys)
    return fail(MOE_ERR_NULL, "w2: NULL pointer");
  const int path_in = path;
  path = resolve_path(path, T, top_k);
  if (path < 0) return fail(MOE_ERR_UNSUPPORTED, "w2: unknown path %d", path_in);
  if (block_m != block_m_of(path))
    return fail(MOE_ERR_UNSUPPORTED, "w2: block_m=%d, path %d needs %d", block_m, path,
                block_m_of(path));
  const ExpertsDev ed = make_experts_dev(experts, shared);
  const SlotsDev sd{T, top_k, T * top_k + (shared ? T : 0)};
  MOE_CHECK_HIP(dispatch_w2(path, h, ed, sd, sorted_ids, expert_ids, ntpp, nullptr, block_m,
                            capacity_blocks, topk_weights, ys,
                            (hipStream_t)stream), "w2");
  return MOE_OK;
}

int moe_sum_v1(const float* ys, int32_t T, int32_t top_k, int32_t hidden, int32_t has_shared,
               const int32_t* topk_ids, int32_t num_experts, const int32_t* expert_row,
               uint16_t* out, void* stream) {
  if (T < 0 || top_k < 1 || hidden <= 0 || hidden % 4 != 0 || num_experts < 1)
    return fail(MOE_ERR_SHAPE, "moe_sum: T=%d top_k=%d hidden=%d num_experts=%d", T, top_k,
                hidden, num_experts);
  if (T == 0) return MOE_OK;
  if (!ys || !out || !topk_ids) return fail(MOE_ERR_NULL, "moe_sum: NULL pointer");
  MOE_CHECK_HIP(launch_moe_sum(ys, T, top_k, hidden, has_shared ? 1 : 0, topk_ids, num_experts,
                               expert_row, out, (hipStream_t)stream),
                "moe_sum");
  return MOE_OK;
}

int moe_rmsnorm_v1(uint16_t* res, const uint16_t* add, int32_t T, int32_t hidden,
                   const uint16_t* weight, float eps, uint16_t* out, void* stream) {
  if (T < 0 || hidden <= 0 || hidden % 8 != 0 || hidden > 8192)
    return fail(MOE_ERR_SHAPE, "rmsnorm: T=%d hidden=%d (hidden %% 8 == 0, <= 8192)", T, hidden);
  if (!(eps >= 0.0f)) return fail(MOE_ERR_SHAPE, "rmsnorm: eps must be >= 0");
  if (T == 0) return MOE_OK;
  if (!res || !weight || !out) return fail(MOE_ERR_NULL, "rmsnorm: NULL pointer");
  {  // the [T, hidden] bf16 row sets res (updated in place), add and out share no byte
    const uintptr_t rows = (uintptr_t)T * hidden * 2;
    auto overlap = [rows](const void* a, const void* b) {
      const uintptr_t p = (uintptr_t)a, q = (uintptr_t)b;
      return a && b && p < q + rows && q < p + rows;
    };
    if (overlap(out, res) || overlap(out, add) || overlap(add, res))
      return fail(MOE_ERR_SHAPE, "rmsnorm: out, res and add must not overlap");
  }
  MOE_CHECK_HIP(launch_rmsnorm(res, add, T, hidden, weight, eps, res, out, (hipStream_t)stream),
                "rmsnorm");
  return MOE_OK;
}

int64_t moe_layer_workspace_bytes_v1(int32_t T, int32_t top_k, const moe_expert_set_v1* experts,
                                     int32_t has_shared, int32_t path) {
  if (!experts || T < 0 || top_k < 1) return -1;
  path = resolve_path(path, T, top_k);
  if (path < 0) return -1;
  return (int64_t)layout(T, top_k, experts, has_shared ? 1 : 0, path).total;
}

}  // extern "C"

// The argument checks of a routed layer call before any workspace is involved, shared by
// moe_layer_v1, moe_norm_layer_v1 and moe_layer_noalloc_v1 so that one bad input gets one error
// code from all of them. T == 0 passes (the call is then a no-op).
int check_layer_args(const uint16_t* x, int32_t T, const uint16_t* router_w, int32_t top_k,
                     const moe_expert_set_v1* experts, const moe_expert_set_v1* shared,
                     const uint16_t* shared_gate_w, const uint16_t* out, int32_t path) {
  int rc = check_experts(experts, shared);
  if (rc) return rc;
  if (T < 0) return fail(MOE_ERR_SHAPE, "layer: T=%d", T);
  if (T == 0) return MOE_OK;
  if (!x || !router_w || !out) return fail(MOE_ERR_NULL, "layer: NULL pointer");
  if (shared && !shared_gate_w) return fail(MOE_ERR_NULL, "layer: shared expert needs shared_gate_w");
  const int E = experts->num_experts;
  if (top_k < 1 || top_k > E || top_k > 64)
    return fail(MOE_ERR_SHAPE, "layer: top_k=%d outside [1, min(num_experts, 64)]", top_k);
  if (resolve_path(path, T, top_k) < 0)
    return fail(MOE_ERR_UNSUPPORTED, "layer: unknown path %d", path);
  return MOE_OK;
}

namespace {

// The decoder step's residual add + RMSNorm in front of a layer call (moe_norm_layer_v1).
struct PreNorm {
  const uint16_t* res_in;
  const uint16_t* add;
  const uint16_t* weight;
  float eps;
  uint16_t* res_out;
  uint16_t* x_out;  // the layer's input
};

int layer_impl(const uint16_t* x, int32_t T, const uint16_t* router_w, const float* logit_bias,
               int32_t top_k, const moe_expert_set_v1* experts, const moe_expert_set_v1* shared,
               const uint16_t* shared_gate_w, void* workspace, int64_t workspace_bytes,
               uint16_t* out, int32_t* topk_ids_out, float* topk_weights_out, int32_t path,
               void* stream, const PreNorm* pn) {
  if (pn) x = pn->x_out;
  int rc = check_layer_args(x, T, router_w, top_k, experts, shared, shared_gate_w, out, path);
  if (rc) return rc;
  if (T == 0) return MOE_OK;
  if (!workspace) return fail(MOE_ERR_NULL, "layer: NULL pointer");
  const int E = experts->num_experts;
  path = resolve_path(path, T, top_k);
  const Workspace L = layout(T, top_k, experts, shared ? 1 : 0, path);
  if (workspace_bytes < (int64_t)L.total)
    return fail(MOE_ERR_WORKSPACE, "layer: workspace %lld < required %lld",
                (long long)workspace_bytes, (long long)L.total);
  if (!workspace_aligned(workspace))
    return fail(MOE_ERR_WORKSPACE, "layer: workspace must be 256-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  float* logits = at<float>(workspace, L.logits);
  int32_t* ids = at<int32_t>(workspace, L.ids);
  float* w = at<float>(workspace, L.w);
  // decode batches: the router normalises its own tokens; otherwise the norm runs first
  const bool norm_in_router = pn && path == MOE_PATH_DECODE &&
                              router_norm_fits(T, experts->hidden, pn->res_in, pn->res_out);
  if (pn && !norm_in_router)
    MOE_CHECK_HIP(launch_rmsnorm(pn->res_in, pn->add, T, experts->hidden, pn->weight, pn->eps,
                                 pn->res_out, pn->x_out, s), "rmsnorm");
  if (path == MOE_PATH_PREFILL && router_prefill_fits(T, experts->hidden, E, top_k)) {
    // approximate MFMA logits, certified top-k with canonical logits for the selection
    MOE_CHECK_HIP(launch_router_prefill(x, T, experts->hidden, router_w, E,
                                        shared ? shared_gate_w : nullptr, logit_bias, top_k,
                                        logits, at<float>(workspace, L.norms), ids, w, s),
                  "router (prefill)");
    rc = run_experts(x, T, top_k, experts, shared, L, workspace, out, path, ROUTE_ALIGN, s);
    if (rc) return rc;
    return copy_routing(ids, w, T, top_k, topk_ids_out, topk_weights_out, s);
  }
  if (norm_in_router)
    MOE_CHECK_HIP(launch_router_logits_norm(pn->res_in, pn->add, pn->weight, pn->eps, pn->res_out,
                                            pn->x_out, T, experts->hidden, router_w, E,
                                            shared ? shared_gate_w : nullptr, logit_bias, logits,
                                            s),
                  "rmsnorm + router logits");
  else
    MOE_CHECK_HIP(launch_router_logits(x, T, experts->hidden, router_w, E,
                                       shared ? shared_gate_w : nullptr, logit_bias, logits, s),
                  "router logits");
  // decode-size batches: with one or two tokens the MFMA decode kernels compute the top-k
  // themselves (slot grid; every W1 workgroup repeats it, which costs more than the launch it
  // saves beyond two tokens); up to 8 tokens top-k and align come from one block (no align
  // launch). Beyond that the selections are spread over many workgroups: one block would
  // serialise them on one CU. Up to 8 tokens W2 also sums the weighted rows itself
  // (w2_token_sum_fits).
  const bool small = topk_align_fits(T, top_k, shared ? 1 : 0);
  Routing routing = ROUTE_ALIGN;
  if (path == MOE_PATH_DECODE && small && T <= kGridTopkMaxTokens) {
    routing = ROUTE_GRID_LOGITS;
  } else if (path != MOE_PATH_PREFILL && small) {
    MOE_CHECK_HIP(launch_topk_align(logits, T, E, top_k, shared ? 1 : 0, L.bm, L.cap, ids, w,
                                    at<int32_t>(workspace, L.sorted),
                                    at<int32_t>(workspace, L.eids),
                                    at<int32_t>(workspace, L.ntpp), s), "router topk+align");
    routing = ROUTE_ALIGNED;
  } else {
    MOE_CHECK_HIP(launch_router_topk(logits, T, E, top_k, shared ? 1 : 0, ids, w, s),
                  "router topk");
  }
  rc = run_experts(x, T, top_k, experts, shared, L, workspace, out, path, routing, s);
  if (rc) return rc;
  return copy_routing(ids, w, T, top_k, topk_ids_out, topk_weights_out, s);
}

}  // namespace

extern "C" {

int moe_layer_v1(const uint16_t* x, int32_t T, const uint16_t* router_w, const float* logit_bias,
                 int32_t top_k, const moe_expert_set_v1* experts, const moe_expert_set_v1* shared,
                 const uint16_t* shared_gate_w, void* workspace, int64_t workspace_bytes,
                 uint16_t* out, int32_t* topk_ids_out, float* topk_weights_out, int32_t path,
                 void* stream) {
  return layer_impl(x, T, router_w, logit_bias, top_k, experts, shared, shared_gate_w, workspace,
                    workspace_bytes, out, topk_ids_out, topk_weights_out, path, stream, nullptr);
}

int moe_norm_layer_v1(const uint16_t* res_in, const uint16_t* add, const uint16_t* norm_w,
                      float eps, uint16_t* res_out, uint16_t* x_out, int32_t T,
                      const uint16_t* router_w, const float* logit_bias, int32_t top_k,
                      const moe_expert_set_v1* experts, const moe_expert_set_v1* shared,
                      const uint16_t* shared_gate_w, void* workspace, int64_t workspace_bytes,
                      uint16_t* out, int32_t* topk_ids_out, float* topk_weights_out, int32_t path,
                      void* stream) {
  if (T < 0) return fail(MOE_ERR_SHAPE, "norm layer: T=%d", T);
  if (T == 0) return MOE_OK;
  if (!res_in || !norm_w || !res_out || !x_out) return fail(MOE_ERR_NULL, "norm layer: NULL pointer");
  if (!experts) return fail(MOE_ERR_NULL, "experts is NULL");
  const int H = experts->hidden;
  if (H <= 0 || H % 8 != 0 || H > 8192)
    return fail(MOE_ERR_SHAPE, "norm layer: hidden=%d (hidden %% 8 == 0, <= 8192)", H);
  if (!(eps >= 0.0f)) return fail(MOE_ERR_SHAPE, "norm layer: eps must be >= 0");
  // Byte ranges of the [T, H] bf16 row sets: the residual may be updated in place (res_out ==
  // res_in: every row is read and written by one workgroup), but no other pair may share bytes
  // (a row-offset overlap would let one workgroup overwrite rows another still reads).
  const size_t rows = (size_t)T * H * 2;
  auto overlap = [rows](const void* a, const void* b) {
    const uintptr_t p = (uintptr_t)a, q = (uintptr_t)b;
    return a && b && p < q + rows && q < p + rows;
  };
  if (res_out != res_in && overlap(res_out, res_in))
    return fail(MOE_ERR_SHAPE, "norm layer: res_out must equal res_in or not overlap it");
  if (overlap(x_out, res_in) || overlap(x_out, res_out) || overlap(x_out, add) ||
      overlap(res_out, add) || overlap(res_in, add))
    return fail(MOE_ERR_SHAPE, "norm layer: x_out and add must not overlap the residual rows");
  if (overlap(out, x_out) || overlap(out, res_in) || overlap(out, res_out))
    return fail(MOE_ERR_SHAPE, "norm layer: out must not overlap x_out or the residual rows");
  const PreNorm pn{res_in, add, norm_w, eps, res_out, x_out};
  return layer_impl(nullptr, T, router_w, logit_bias, top_k, experts, shared, shared_gate_w,
                    workspace, workspace_bytes, out, topk_ids_out, topk_weights_out, path, stream,
                    &pn);
}

int moe_fused_experts_v1(const uint16_t* x, int32_t T, const int32_t* topk_ids,
                         const float* topk_weights, int32_t top_k,
                         const moe_expert_set_v1* experts, const moe_expert_set_v1* shared,
                         const uint16_t* shared_gate_w, void* workspace, int64_t workspace_bytes,
                         uint16_t* out, int32_t path, void* stream) {
  int rc = check_experts(experts, shared);
  if (rc) return rc;
  if (T < 0 || top_k < 1 || top_k > 64) return fail(MOE_ERR_SHAPE, "experts: T=%d top_k=%d", T, top_k);
  if (T == 0) return MOE_OK;
  if (!x || !topk_ids || !topk_weights || !out || !workspace)
    return fail(MOE_ERR_NULL, "experts: NULL pointer");
  if (shared && !shared_gate_w) return fail(MOE_ERR_NULL, "experts: shared expert needs shared_gate_w");
  const int path_in = path;
  path = resolve_path(path, T, top_k);
  if (path < 0) return fail(MOE_ERR_UNSUPPORTED, "experts: unknown path %d", path_in);
  const Workspace L = layout(T, top_k, experts, shared ? 1 : 0, path);
  if (workspace_bytes < (int64_t)L.total)
    return fail(MOE_ERR_WORKSPACE, "experts: workspace %lld < required %lld",
                (long long)workspace_bytes, (long long)L.total);
  if (!workspace_aligned(workspace))
    return fail(MOE_ERR_WORKSPACE, "experts: workspace must be 256-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  int32_t* ids = at<int32_t>(workspace, L.ids);
  float* w = at<float>(workspace, L.w);
  MOE_CHECK_HIP(hipMemcpyAsync(ids, topk_ids, (size_t)T * top_k * 4, hipMemcpyDeviceToDevice, s),
                "copy ids");
  MOE_CHECK_HIP(hipMemcpyAsync(w, topk_weights, (size_t)T * top_k * 4, hipMemcpyDeviceToDevice, s),
                "copy weights");
  if (shared)
    MOE_CHECK_HIP(launch_shared_gate(x, T, experts->hidden, shared_gate_w, top_k,
                                     at<float>(workspace, L.logits), w, s), "shared gate");
  const Routing routing = (path == MOE_PATH_DECODE && slot_grid_fits(T, top_k, shared ? 1 : 0))
                              ? ROUTE_GRID_IDS
                              : ROUTE_ALIGN;
  return run_experts(x, T, top_k, experts, shared, L, workspace, out, path, routing, s);
}

}  // extern "C"

namespace {

// Spins until flags[t] == seq for every t < T (the top-k kernel's system-scope releases after
// the ids), for at most kFlagSpinUs; false on time-out (the caller then waits on the stream,
// which also reports a failed kernel).
constexpr double kFlagSpinUs = 200000.0;
bool wait_flags(const int32_t* flags, int T, int32_t seq) {
  const volatile int32_t* f = flags;
  const auto t0 = std::chrono::steady_clock::now();
  for (uint64_t it = 0;; ++it) {
    int t = 0;
    while (t < T && f[t] == seq) ++t;
    if (t == T) {
      std::atomic_thread_fence(std::memory_order_acquire);  // the ids after their flags
      return true;
    }
    if ((it & 1023) == 1023 &&
        std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count() >
            kFlagSpinUs)
      return false;
  }
}

}  // namespace

extern "C" {

int moe_offload_layer_v1(uint64_t cache, int32_t layer, const uint16_t* x, int32_t T,
                         const uint16_t* router_w, const float* logit_bias, int32_t top_k,
                         const moe_expert_set_v1* experts, void* workspace,
                         int64_t workspace_bytes, uint16_t* out, int32_t* ids_host,
                         const int32_t* prefetch, int32_t n_prefetch, int32_t path, void* stream,
                         int32_t* hits) {
  int rc = check_experts(experts, nullptr);
  if (rc) return rc;
  if (T < 1) return fail(MOE_ERR_SHAPE, "offload layer: T=%d", T);
  if (!x || !router_w || !out || !workspace || !ids_host || (n_prefetch > 0 && !prefetch))
    return fail(MOE_ERR_NULL, "offload layer: NULL pointer");
  const int E = experts->num_experts;
  if (top_k < 1 || top_k > E || top_k > 64)
    return fail(MOE_ERR_SHAPE, "offload layer: top_k=%d outside [1, min(num_experts, 64)]", top_k);
  if (n_prefetch < 0) return fail(MOE_ERR_SHAPE, "offload layer: n_prefetch=%d", n_prefetch);
  const int path_in = path;
  path = resolve_path(path, T, top_k);
  if (path < 0) return fail(MOE_ERR_UNSUPPORTED, "offload layer: unknown path %d", path_in);
  const Workspace L = layout(T, top_k, experts, 0, path);
  if (workspace_bytes < (int64_t)L.total)
    return fail(MOE_ERR_WORKSPACE, "offload layer: workspace %lld < required %lld",
                (long long)workspace_bytes, (long long)L.total);
  if (!workspace_aligned(workspace))
    return fail(MOE_ERR_WORKSPACE, "offload layer: workspace must be 256-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  float* logits = at<float>(workspace, L.logits);
  int32_t* ids = at<int32_t>(workspace, L.ids);
  float* w = at<float>(workspace, L.w);
  const int n = T * top_k;
  MOE_CHECK_HIP(launch_router_logits(x, T, experts->hidden, router_w, E, nullptr, logit_bias,
                                     logits, s), "offload layer: router logits");
  // The host-managed cache needs the routed ids: the one wait of the layer. Pinned host memory
  // that HIP maps at the same address on the device (hipHostMalloc's) takes them straight from
  // the top-k kernel's lanes, with no copy on the stream; both ends of the range must map, at
  // their own addresses. Other host memory gets a copy.
  int32_t* mirror = nullptr;
  {
    void* d0 = nullptr;
    void* d1 = nullptr;
    const bool mapped =
        hipHostGetDevicePointer(&d0, ids_host, 0) == hipSuccess && d0 == (void*)ids_host &&
        hipHostGetDevicePointer(&d1, ids_host + (n - 1), 0) == hipSuccess &&
        d1 == (void*)(ids_host + (n - 1));
    if (mapped)
      mirror = ids_host;
    else
      (void)hipGetLastError();  // a failed lookup must not surface at the next launch check
  }
  // With mapped ids, the top-k kernel also raises one flag per token in the cache's mapped
  // signal words after the token's ids: the host spins on them instead of waiting for the
  // stream (whose completion signal arrives about 5 us later). The kernels enqueued before the
  // top-k have completed when it runs, so the layer's slots are as free as after a stream wait.
  int32_t seq = 0;
  int32_t* flags = mirror ? slot_cache_signal(cache, T, &seq) : nullptr;
  MOE_CHECK_HIP(launch_router_topk(logits, T, E, top_k, 0, ids, w, s, mirror, flags, seq),
                "offload layer: router topk");
  if (!mirror)
    MOE_CHECK_HIP(hipMemcpyAsync(ids_host, ids, (size_t)n * 4, hipMemcpyDeviceToHost, s),
                  "offload layer: ids to the host");
  if (!flags || !wait_flags(flags, T, seq)) {
    MOE_CHECK_HIP(hipStreamSynchronize(s), "offload layer: wait for the ids");
    if (flags && !wait_flags(flags, T, seq))
      return fail(MOE_ERR_UNSUPPORTED, "offload layer: the routed ids' flags were not raised");
  }
  rc = moe_slot_cache_demand_v1(cache, layer, ids_host, n, stream, hits);
  if (rc) return rc;
  const Routing routing =
      (path == MOE_PATH_DECODE && slot_grid_fits(T, top_k, 0)) ? ROUTE_GRID_IDS : ROUTE_ALIGN;
  rc = run_experts(x, T, top_k, experts, nullptr, L, workspace, out, path, routing, s);
  if (rc) return rc;
  // The wait for the ids drained the compute stream, and the demand's slots (the only ones the
  // kernels just enqueued read) stay pinned until layer_done: the prefetch needs no ordering
  // wait on the compute stream (one event record and two stream waits fewer per layer).
  if (n_prefetch > 0) {
    rc = slot_cache_prefetch_synced(cache, layer, prefetch, n_prefetch, stream);
    if (rc) return rc;
  }
  return moe_slot_cache_layer_done_v1(cache, layer);
}

}  // extern "C"
