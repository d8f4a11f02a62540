// No-allocation prefill entry point (gdn_prefill_fwd_noalloc): the same launches
// as gdn_prefill_fwd with the workspace in a file-scope device array.
//
// The array lives in this translation unit, apart from the prefill kernels, so
// its code object (and the 128 MiB it reserves on a GPU) is loaded only by a
// process that calls this entry point: gdn_prefill_fwd's callers never pay for
// it.  Host code never passes the array's name to a kernel (on the host it is
// only a stand-in for the symbol); the device address comes from
// hipGetSymbolAddress, once per device with that device current.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <mutex>

#include "../../include/gdn_mi355x.h"

namespace gdn {

// The prefill launches for a caller-provided workspace (gdn_prefill.hip).
int prefill_launch(const void* q, const void* k, const void* v, const float* state,
                   const float* A_log, const void* a, const float* dt_bias,
                   const void* b, const void* cu_seqlens, int cu_seqlens_is_int64,
                   int num_seqs, long long total_tokens, float scale, void* output,
                   float* new_state, void* workspace, size_t workspace_bytes, void* stream);

static_assert(GDN_PREFILL_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size");
static __device__ __align__(256) unsigned char scratch[GDN_PREFILL_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static std::atomic<void*> g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// Device address of the current device's scratch array (its first call on a
// device resolves the symbol).  Returns GDN_OK or an error code.
static int current_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return GDN_ERR_INVALID_ARGUMENT;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return static_cast<int>(e);
      if (p == nullptr) return GDN_ERR_INVALID_ARGUMENT;
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return GDN_OK;
}

}  // namespace gdn

extern "C" int gdn_prefill_fwd_noalloc(const void* q, const void* k, const void* v, const float* state,
                                       const float* A_log, const void* a, const float* dt_bias,
                                       const void* b, const void* cu_seqlens, int cu_seqlens_is_int64,
                                       int num_seqs, long long total_tokens, float scale, void* output,
                                       float* new_state, void* stream) {
  using namespace gdn;
  if (num_seqs < 0 || total_tokens < 0) return GDN_ERR_INVALID_ARGUMENT;
  if (num_seqs == 0) return GDN_OK;
  if (gdn_prefill_workspace_min_bytes(num_seqs, total_tokens) > GDN_PREFILL_NOALLOC_SCRATCH_BYTES)
    return GDN_ERR_TOO_LARGE;
  void* ws = nullptr;
  const int st = current_scratch(&ws);
  if (st != GDN_OK) return st;
  // the default workspace's slot count when it fits, so results equal
  // gdn_prefill_fwd's with a default workspace
  const size_t bytes = std::min<size_t>(GDN_PREFILL_NOALLOC_SCRATCH_BYTES,
                                        gdn_prefill_workspace_bytes(num_seqs, total_tokens));
  return prefill_launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_seqlens_is_int64, num_seqs,
                        total_tokens, scale, output, new_state, ws, bytes, stream);
}
