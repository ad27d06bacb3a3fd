// HBM stream ceilings, for bench.py only (libtq_probe.so; not part of libtq_amd.so's C ABI).
//
// The decode kernels stream packed planes once per step with non-temporal 16-byte loads
// and write f32 scores with non-temporal stores.  This kernel moves bytes the same way and
// nothing else, so its rate is the ceiling those kernels are measured against on the same
// box in the same session: read-only, write-only, and a read/write mix in the scores
// kernel's proportion (13 KiB read per 4 KiB written: 218 MB of key planes per 67 MB of
// scores at the headline shape).
//
// Work is split into units: a wave reads RU KiB (RU loads of 16 B per lane) and writes WU
// KiB of the next unit of each stream; waves take units round-robin over the grid.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int RU, int WU>
__global__ void __launch_bounds__(256) stream_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                     int64_t units) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * 4;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); u < units; u += nwaves) {
    if constexpr (RU > 0) {
      const u32x4* s = src + u * RU * 64 + lane;
      u32x4 v[RU];
#pragma unroll
      for (int r = 0; r < RU; ++r) v[r] = __builtin_nontemporal_load(s + r * 64);
#pragma unroll
      for (int r = 0; r < RU; ++r) acc ^= v[r];
    }
    if constexpr (WU > 0) {
      u32x4* d = dst + u * WU * 64 + lane;
#pragma unroll
      for (int w = 0; w < WU; ++w) __builtin_nontemporal_store(acc + static_cast<unsigned>(w), d + w * 64);
    }
  }
  if constexpr (WU == 0) {
    // keeps the loads live; the data never holds this pattern
    if (acc[0] == 0x9e3779b9u && acc[1] == 0x7f4a7c15u && acc[2] == 0x85ebca6bu && acc[3] == 0xc2b2ae35u)
      dst[threadIdx.x] = acc;
  }
}

}  // namespace

extern "C" {

// bytes read and written per unit for `mode` (0 read-only, 1 write-only, 2 the 13:4 mix)
int64_t tq_probe_unit_bytes(int32_t mode, int32_t write) {
  const int64_t ru = mode == 0 ? 16 : (mode == 2 ? 13 : 0), wu = mode == 1 ? 16 : (mode == 2 ? 4 : 0);
  return (write ? wu : ru) * 1024;
}

// One launch over `units` units.  src must hold units * tq_probe_unit_bytes(mode, 0) bytes,
// dst units * tq_probe_unit_bytes(mode, 1) bytes (at least 4 KiB for read-only).
// Returns 0, or -1 for a bad mode and -3 for a launch error.
int tq_probe_stream(const void* src, void* dst, int64_t units, int32_t mode, int32_t blocks, void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  const u32x4* in = static_cast<const u32x4*>(src);
  u32x4* out = static_cast<u32x4*>(dst);
  if (blocks <= 0 || units < 0) return -1;
  if (mode == 0) stream_kernel<16, 0><<<blocks, 256, 0, s>>>(in, out, units);
  else if (mode == 1) stream_kernel<0, 16><<<blocks, 256, 0, s>>>(in, out, units);
  else if (mode == 2) stream_kernel<13, 4><<<blocks, 256, 0, s>>>(in, out, units);
  else return -1;
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // extern "C"
