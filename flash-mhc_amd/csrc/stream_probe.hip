// HBM ceiling probe (see include/flash_mhc_probe.h): each thread moves four
// 16-byte vectors, one pass over the buffer, nontemporal reads.  This shape
// measured the highest read / write / copy rates on MI355X among grid-stride
// and one-pass variants.
#include "fmhc_common.h"
#include "../../include/flash_mhc_probe.h"

namespace fmhc {
namespace {

constexpr int kPerThread = 4;

__global__ __launch_bounds__(256) void probe_read(const u32x4* __restrict__ a, int64_t n,
                                                  unsigned* __restrict__ sink) {
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * 256 * kPerThread + threadIdx.x;
  unsigned acc = 0;
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int64_t i = i0 + u * 256;
    if (i < n) {
      const u32x4 v = __builtin_nontemporal_load(a + i);
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;  // keeps the loads; practically never taken
}

__global__ __launch_bounds__(256) void probe_write(u32x4* __restrict__ b, int64_t n) {
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * 256 * kPerThread + threadIdx.x;
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int64_t i = i0 + u * 256;
    if (i < n) b[i] = u32x4{static_cast<unsigned>(i), 1u, 2u, 3u};
  }
}

__global__ __launch_bounds__(256) void probe_copy(const u32x4* __restrict__ a, u32x4* __restrict__ b,
                                                  int64_t n) {
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * 256 * kPerThread + threadIdx.x;
  u32x4 v[kPerThread];
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int64_t i = i0 + u * 256;
    if (i < n) v[u] = __builtin_nontemporal_load(a + i);
  }
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int64_t i = i0 + u * 256;
    if (i < n) __builtin_nontemporal_store(v[u], b + i);
  }
}

}  // namespace
}  // namespace fmhc

extern "C" int fmhc_stream_probe(int kind, const void* src, void* dst, int64_t nbytes, void* stream) {
  using namespace fmhc;
  if (nbytes <= 0 || nbytes % 16 != 0 || !dst) return FMHC_ERR_INVALID_ARGUMENT;
  if (kind != FMHC_PROBE_WRITE && !src) return FMHC_ERR_INVALID_ARGUMENT;
  if (!aligned16(dst) || (src && !aligned16(src))) return FMHC_ERR_INVALID_ARGUMENT;
  const int64_t n = nbytes / 16;
  const dim3 grid(blocks_for(n, 256 * kPerThread));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const u32x4* a = static_cast<const u32x4*>(src);
  u32x4* b = static_cast<u32x4*>(dst);
  switch (kind) {
    case FMHC_PROBE_READ: probe_read<<<grid, 256, 0, s>>>(a, n, static_cast<unsigned*>(dst)); break;
    case FMHC_PROBE_WRITE: probe_write<<<grid, 256, 0, s>>>(b, n); break;
    case FMHC_PROBE_COPY: probe_copy<<<grid, 256, 0, s>>>(a, b, n); break;
    default: return FMHC_ERR_INVALID_ARGUMENT;
  }
  return launch_status();
}
