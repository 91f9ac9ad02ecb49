// Matching forward that allocates nothing: ml_mask_matching_forward with its
// workspace taken from a static device array instead of the caller, for
// callers that cannot call hipMalloc (code under HIP graph capture, tight
// serving loops, harnesses that forbid allocation).  No counterpart in the
// reference.
//
// The array lives in this file.  Its host-side name is only a stand-in for
// registration: the device address is resolved once per device, with that
// device current, through hipGetSymbolAddress, and only that address is ever
// handed to kernels.  Each device holds its own copy until the process ends.
// Every call on a device shares that device's copy, so calls that overlap on
// one device race; nothing in it needs to start at zero (every word a call
// reads is written earlier in the same call: presence records, schedule,
// partial sums, cost planes; the assignment's counters are cleared by the
// finalize kernel of the same call).
#include <atomic>
#include <mutex>

#include "ml_internal.h"

namespace ml {

constexpr size_t kScratchBytes = ML_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];  // device address of `scratch` per device
std::mutex g_scratch_mu;

// The current device's address of `scratch`, resolved on the first call on
// that device.
int scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(ML_ELAUNCH, "no-allocation forward: no current HIP device (or more than 64)");
  void* ptr = g_scratch[dev].load(std::memory_order_acquire);
  if (!ptr) {
    std::lock_guard<std::mutex> g(g_scratch_mu);
    ptr = g_scratch[dev].load(std::memory_order_relaxed);
    if (!ptr) {
      const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !ptr)
        return fail(ML_ELAUNCH, std::string("no-allocation forward: cannot resolve the scratch "
                                            "array: ") + hipGetErrorString(e));
      g_scratch[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return ML_OK;
}
}  // namespace

}  // namespace ml

using namespace ml;

extern "C" size_t ml_mask_matching_forward_noalloc_bytes(const ml_shape* s, const ml_params* p,
                                                         int mask_dtype) {
  if (check_matching_params(p, s->C)) return 0;
  size_t need = 0;
  if (forward_packed_bytes(s, p, mask_dtype, kScratchBytes, need)) return 0;
  return need;
}

extern "C" int ml_mask_matching_forward_noalloc(
    const ml_shape* s, const ml_params* p, int mask_dtype, const void* mask_logits,
    const int64_t* mask_targets, int cls_dtype, const void* cls_logits, const int64_t* cls_targets,
    int64_t* pred_to_gt, int64_t* pred_round, float* layer_means, float* separate_costs,
    void* saved, void* grad_mask_prefill, int32_t* void_found, ml_event_t void_ready,
    ml_stream_t stream) {
  int rc = check_matching_params(p, s->C);
  if (rc) return rc;
  size_t need = 0;
  if ((rc = forward_packed_bytes(s, p, mask_dtype, kScratchBytes, need))) return rc;
  if (need > kScratchBytes)
    return fail(ML_EUNSUPPORTED, "no-allocation forward: this shape needs " + std::to_string(need) +
                                     " bytes of scratch, more than the " +
                                     std::to_string(kScratchBytes) + " of the static array");
  void* ws = nullptr;
  if ((rc = scratch_address(&ws))) return rc;
  return forward_impl(s, p, mask_dtype, mask_logits, mask_targets, cls_dtype, cls_logits,
                      cls_targets, pred_to_gt, pred_round, layer_means, separate_costs, saved,
                      grad_mask_prefill, void_found, (hipEvent_t)void_ready, ws, kScratchBytes,
                      (hipStream_t)stream, false, nullptr, nullptr, nullptr, 0, 0, true);
}
