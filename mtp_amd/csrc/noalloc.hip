// moe_layer_noalloc_v1: the routed layer of moe_layer_v1 for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// Its workspace (routing logits, ids, the sorted slot layout, the intermediate h rows and the
// weighted W2 rows) is a file-scope device array of kNoallocScratchBytes per GPU, held from the
// library's load until the process ends. Host code never passes the array's name to a kernel
// (on the host it is only a stand-in for the symbol): the device address comes from
// hipGetSymbolAddress, called once per device with that device current, and is kept per device.
// Every call on one GPU shares that GPU's array; the layer writes every workspace byte it reads
// before reading it, so nothing has to start at zero, and calls that overlap on one GPU (two
// streams, or two host threads) race.
#include <cstdio>
#include <mutex>

#include "common.h"
#include "launch.h"

constexpr int64_t kNoallocScratchBytes = int64_t(64) << 20;  // 64 MiB per GPU

static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's scratch array (resolved once per device).
int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // reported here, not at the caller's next HIP call
    snprintf(moe_error_buffer(), kErrorBufferBytes, "noalloc: hipGetDevice: HIP error %d (%s)",
             (int)e, hipGetErrorString(e));
    return MOE_ERR_HIP + ((int)e % 100);
  }
  if (dev < 0 || dev >= kMaxDevices) {
    snprintf(moe_error_buffer(), kErrorBufferBytes, "noalloc: device %d outside [0, %d)", dev,
             kMaxDevices);
    return MOE_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      snprintf(moe_error_buffer(), kErrorBufferBytes,
               "noalloc: hipGetSymbolAddress(scratch) on device %d: HIP error %d (%s)", dev,
               (int)e, hipGetErrorString(e));
      return MOE_ERR_HIP + ((int)e % 100);
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MOE_OK;
}

}  // namespace

extern "C" {

int64_t moe_layer_noalloc_max_bytes_v1(void) { return kNoallocScratchBytes; }

int moe_layer_noalloc_v1(const uint16_t* x, int32_t T, const uint16_t* router_w,
                         const float* logit_bias, int32_t top_k, const moe_expert_set_v1* experts,
                         const moe_expert_set_v1* shared, const uint16_t* shared_gate_w,
                         uint16_t* out, int32_t* topk_ids_out, float* topk_weights_out,
                         int32_t path, void* stream) {
  // moe_layer_v1's own argument checks first: the same bad input gets the same error code
  const int rc0 = check_layer_args(x, T, router_w, top_k, experts, shared, shared_gate_w, out,
                                   path);
  if (rc0 || T == 0) return rc0;
  const int64_t need = moe_layer_workspace_bytes_v1(T, top_k, experts, shared ? 1 : 0, path);
  if (need < 0) {
    snprintf(moe_error_buffer(), kErrorBufferBytes, "noalloc: invalid sizes T=%d top_k=%d", T,
             top_k);
    return MOE_ERR_SHAPE;
  }
  if (need > kNoallocScratchBytes) {
    snprintf(moe_error_buffer(), kErrorBufferBytes,
             "noalloc: T=%d needs %lld workspace bytes, above the %lld-byte scratch of this "
             "entry point; use moe_layer_v1 with a caller workspace",
             T, (long long)need, (long long)kNoallocScratchBytes);
    return MOE_ERR_WORKSPACE;
  }
  void* ws = nullptr;
  const int rc = scratch_for_current_device(&ws);
  if (rc) return rc;
  return moe_layer_v1(x, T, router_w, logit_bias, top_k, experts, shared, shared_gate_w, ws,
                      kNoallocScratchBytes, out, topk_ids_out, topk_weights_out, path, stream);
}

}  // extern "C"
