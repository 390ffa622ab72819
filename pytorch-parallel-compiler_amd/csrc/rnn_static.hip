// wc_rnn_forward_noalloc: wc_rnn_forward with its workspace in a file-scope device array
// instead of a caller-provided buffer, for callers that cannot allocate device memory
// (code under graph capture, serving loops, harnesses that forbid allocation).
//
// Each device holds its own copy of `scratch` from the first call on it until the process
// ends.  In host code the array's name is only a stand-in: its device address, which
// differs per device, comes from hipGetSymbolAddress (taken once per device, with that
// device current) and is the only handle the kernels are given.  Every call on a device
// shares that device's array; the kernels initialise what must start at zero (the
// partitioned LSTM's counters and exchange tags) in the call itself, and calls that
// overlap in time on one device race.
#include <mutex>

#include "wc_common.h"

namespace wc {
namespace {

constexpr int64_t kScratchBytes = int64_t(64) << 20;   // 64 MiB per device
constexpr int kMaxDevices = 64;

static __device__ __align__(256) char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of this device's `scratch` (looked up on the first call on a device).
int32_t scratch_on_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error(static_cast<int32_t>(e), "wc_rnn_forward_noalloc: no current device: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(WC_ERR_LIMIT, "wc_rnn_forward_noalloc: device %d beyond the %d supported", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return set_error(e != hipSuccess ? static_cast<int32_t>(e) : WC_ERR_NULL,
                       "wc_rnn_forward_noalloc: scratch address on device %d unavailable: %s", dev,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return WC_OK;
}

}  // namespace
}  // namespace wc

using namespace wc;

extern "C" int64_t wc_rnn_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" int32_t wc_rnn_forward_noalloc(const wc_rnn_args* a, void* stream) {
  clear_error();
  WC_REQUIRE(a != nullptr, WC_ERR_NULL, "wc_rnn_forward_noalloc: null args");
  const int64_t need = wc_rnn_workspace_bytes(a);
  WC_REQUIRE(need >= 0, WC_ERR_SHAPE, "wc_rnn_forward_noalloc: bad sizes");
  WC_REQUIRE(need <= kScratchBytes, WC_ERR_LIMIT,
             "wc_rnn_forward_noalloc: these sizes need %lld bytes of workspace; the static scratch holds %lld "
             "(use wc_rnn_forward with a caller-provided workspace)",
             static_cast<long long>(need), static_cast<long long>(kScratchBytes));
  wc_rnn_args b = *a;
  void* ptr = nullptr;
  const int32_t rc = scratch_on_current_device(&ptr);
  if (rc) return rc;
  b.workspace = ptr;
  b.workspace_bytes = kScratchBytes;
  return wc_rnn_forward(&b, stream);
}
