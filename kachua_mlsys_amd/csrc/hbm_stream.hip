// Achievable-bandwidth probe for the MI355X HBM roofline (measurement only;
// not part of the GDN entry points).
//
// stream_copy_kernel moves `n16` 16-byte words from src to dst with the access
// pattern of the decode kernel's state traffic: every byte read once and
// written once, 16-byte non-temporal loads and stores, U loads in flight per
// lane before the first store.  Work-group g copies contiguous tiles of
// 256 * U words (tile g, g + grid, ...), so each wave streams through a few
// DRAM pages at a time.  Its GB/s (read + write bytes / time) is the ceiling
// the decode and prefill rooflines are compared against beside the published
// 8 TB/s.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __attribute__((ext_vector_type(4))) unsigned u32x4;

constexpr int kThreads = 256;

template <int U>
__global__ __launch_bounds__(kThreads) void stream_copy_kernel(const u32x4* __restrict__ src,
                                                               u32x4* __restrict__ dst, long long n16) {
  constexpr long long kTile = static_cast<long long>(kThreads) * U;
  const long long ntiles = n16 / kTile;
  for (long long t = blockIdx.x; t < ntiles; t += gridDim.x) {
    const long long base = t * kTile + threadIdx.x;
    u32x4 r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) r[u] = __builtin_nontemporal_load(src + base + u * kThreads);
#pragma unroll
    for (int u = 0; u < U; ++u) __builtin_nontemporal_store(r[u], dst + base + u * kThreads);
  }
  // the tail (fewer words than one tile)
  for (long long i = ntiles * kTile + static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < n16;
       i += static_cast<long long>(gridDim.x) * kThreads)
    __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

}  // namespace

// Copies n16 16-byte words (src, dst 16-byte aligned, not overlapping) with
// `groups` work-groups of 256 threads and `unroll` (4, 8 or 16) loads in
// flight per lane, on `stream`.  Returns 0, -1 for a bad argument, or a
// hipError_t.
extern "C" int hbm_stream_copy(const void* src, void* dst, long long n16, int groups, int unroll,
                               void* stream) {
  if (!src || !dst || n16 < 0 || groups <= 0) return -1;
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u) return -1;
  if (n16 == 0) return 0;
  const auto* s = static_cast<const u32x4*>(src);
  auto* d = static_cast<u32x4*>(dst);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(groups)), block(kThreads);
  switch (unroll) {
    case 4: stream_copy_kernel<4><<<grid, block, 0, st>>>(s, d, n16); break;
    case 8: stream_copy_kernel<8><<<grid, block, 0, st>>>(s, d, n16); break;
    case 16: stream_copy_kernel<16><<<grid, block, 0, st>>>(s, d, n16); break;
    default: return -1;
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : static_cast<int>(e);
}
