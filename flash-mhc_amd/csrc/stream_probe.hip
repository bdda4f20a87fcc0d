// HBM ceiling probe and cache flush for bench.py (see include/flash_mhc_probe.h).
// Built into its own library, libflash_mhc_probe.so: it is measurement
// infrastructure and not part of the K1/K3/K4 path.
//
// Each thread moves four 16-byte vectors, one pass over the buffer.  This shape
// measured the highest read / write / copy rates on MI355X among grid-stride
// and one-pass variants.  The ceiling probes use the nontemporal hint on loads
// and stores, as the kernels they are compared with do; the "cached" kinds use
// ordinary loads / stores, which allocate in L2 and the memory-side cache (the
// flush before a cold-cache kernel timing, and a labelled extra ceiling).
#include "fmhc_common.h"
#include "../../include/flash_mhc_probe.h"

namespace fmhc {
namespace {

constexpr int kPerThread = 4;

template <bool NT>
__global__ __launch_bounds__(256) void probe_read(const u32x4* __restrict__ a, int64_t n,
                                                  unsigned* __restrict__ sink) {
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * 256 * kPerThread + threadIdx.x;
  unsigned acc = 0;
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int64_t i = i0 + u * 256;
    if (i < n) {
      const u32x4 v = NT ? __builtin_nontemporal_load(a + i) : a[i];
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;  // keeps the loads; practically never taken
}

template <bool NT>
__global__ __launch_bounds__(256) void probe_write(u32x4* __restrict__ b, int64_t n) {
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * 256 * kPerThread + threadIdx.x;
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int64_t i = i0 + u * 256;
    if (i < n) {
      const u32x4 v = {static_cast<unsigned>(i), 1u, 2u, 3u};
      if constexpr (NT)
        __builtin_nontemporal_store(v, b + i);
      else
        b[i] = v;
    }
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
  const bool reads = kind == FMHC_PROBE_READ || kind == FMHC_PROBE_READ_CACHED || kind == FMHC_PROBE_COPY;
  if (reads && !src) return FMHC_ERR_INVALID_ARGUMENT;
  if (!aligned16(dst) || (src && !aligned16(src))) return FMHC_ERR_INVALID_ARGUMENT;
  const int64_t n = nbytes / 16;
  const dim3 grid(blocks_for(n, 256 * kPerThread));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const u32x4* a = static_cast<const u32x4*>(src);
  u32x4* b = static_cast<u32x4*>(dst);
  unsigned* sink = static_cast<unsigned*>(dst);
  switch (kind) {
    case FMHC_PROBE_READ: probe_read<true><<<grid, 256, 0, s>>>(a, n, sink); break;
    case FMHC_PROBE_WRITE: probe_write<true><<<grid, 256, 0, s>>>(b, n); break;
    case FMHC_PROBE_COPY: probe_copy<<<grid, 256, 0, s>>>(a, b, n); break;
    case FMHC_PROBE_READ_CACHED: probe_read<false><<<grid, 256, 0, s>>>(a, n, sink); break;
    case FMHC_PROBE_WRITE_CACHED: probe_write<false><<<grid, 256, 0, s>>>(b, n); break;
    default: return FMHC_ERR_INVALID_ARGUMENT;
  }
  return launch_status();
}

extern "C" int fmhc_probe_abi_version(void) { return FMHC_PROBE_ABI_VERSION; }
