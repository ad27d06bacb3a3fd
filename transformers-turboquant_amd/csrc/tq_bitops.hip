// Bit packing, Lloyd-Max quantize/dequantize and the library's error plumbing.
//
// Layout follows src/turboquant_pytorch/kernels/bit_ops.py:243-326: code i of a
// row occupies bits [i*b, i*b+b), LSB first.  Each thread owns one output byte
// (pack / quantize) or one output code (unpack / dequantize), so no atomics are
// needed (the reference's Triton kernels OR into shared bytes,
// bit_ops.py:94-109, quantize.py:124-143).
#include <cstdarg>
#include <cstdio>

#include "tq_common.h"

namespace tq {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: HIP launch failed: %s", what, hipGetErrorString(e));
    return TQ_EHIP;
  }
  return TQ_OK;
}

// One thread per output byte p of row r: OR the (masked) codes whose bits
// overlap [8p, 8p+8).
__global__ void pack_bits_kernel(const int32_t* __restrict__ idx, int64_t n, int d, int64_t ld_idx,
                                 int b, uint8_t* __restrict__ out, int64_t ld_out, int oc) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n * oc) return;
  const int64_t r = t / oc;
  const int p = static_cast<int>(t - r * oc);
  const uint32_t mask = (1u << b) - 1u;
  const int lo_bit = 8 * p;
  const int c0 = lo_bit / b;
  int c1 = (lo_bit + 7) / b;
  if (c1 > d - 1) c1 = d - 1;
  const int32_t* row = idx + r * ld_idx;
  uint32_t acc = 0;
  for (int c = c0; c <= c1; ++c) {
    const uint32_t v = static_cast<uint32_t>(row[c]) & mask;
    const int sh = c * b - lo_bit;
    acc |= (sh >= 0) ? (v << sh) : (v >> (-sh));
  }
  out[r * ld_out + p] = static_cast<uint8_t>(acc & 0xffu);
}

__global__ void unpack_bits_kernel(const uint8_t* __restrict__ packed, int64_t n, int d,
                                   int64_t ld_in, int b, int32_t* __restrict__ out,
                                   int64_t ld_out) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n * d) return;
  const int64_t r = t / d;
  const int i = static_cast<int>(t - r * d);
  out[r * ld_out + i] = static_cast<int32_t>(read_code(packed + r * ld_in, i, b));
}

// searchsorted-left codes of y, packed; the boundary table sits in LDS.
__global__ void quantize_pack_kernel(const float* __restrict__ y, int64_t n, int d, int64_t ld_y,
                                     const float* __restrict__ bounds, int b,
                                     uint8_t* __restrict__ out, int64_t ld_out, int oc) {
  __shared__ float sb[255];
  const int nb = (1 << b) - 1;
  for (int j = threadIdx.x; j < nb; j += blockDim.x) sb[j] = bounds[j];
  __syncthreads();
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n * oc) return;
  const int64_t r = t / oc;
  const int p = static_cast<int>(t - r * oc);
  const int lo_bit = 8 * p;
  const int c0 = lo_bit / b;
  int c1 = (lo_bit + 7) / b;
  if (c1 > d - 1) c1 = d - 1;
  const float* row = y + r * ld_y;
  uint32_t acc = 0;
  for (int c = c0; c <= c1; ++c) {
    const uint32_t v = searchsorted_left(row[c], sb, nb);
    const int sh = c * b - lo_bit;
    acc |= (sh >= 0) ? (v << sh) : (v >> (-sh));
  }
  out[r * ld_out + p] = static_cast<uint8_t>(acc & 0xffu);
}

__global__ void dequantize_kernel(const uint8_t* __restrict__ packed, int64_t n, int d,
                                  int64_t ld_in, const uint16_t* __restrict__ cent, int b,
                                  uint16_t* __restrict__ out, int64_t ld_out) {
  __shared__ uint16_t sc[256];
  for (int j = threadIdx.x; j < (1 << b); j += blockDim.x) sc[j] = cent[j];
  __syncthreads();
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n * d) return;
  const int64_t r = t / d;
  const int i = static_cast<int>(t - r * d);
  out[r * ld_out + i] = sc[read_code(packed + r * ld_in, i, b)];
}

static inline unsigned grid_for(int64_t work, int threads) {
  return static_cast<unsigned>((work + threads - 1) / threads);
}

}  // namespace tq

using namespace tq;

extern "C" {

int tq_version(void) { return 100; }

const char* tq_last_error(void) { return g_err; }

int64_t tq_out_cols(int64_t d, int32_t b) { return out_cols(d, b); }

int tq_pack_bits(const int32_t* idx, int64_t n, int32_t d, int64_t ld_idx, int32_t b,
                 uint8_t* out, int64_t ld_out, void* stream) {
  TQ_REQUIRE(b >= 1 && b <= 8, "tq_pack_bits: b must be between 1 and 8, got %d", b);
  TQ_REQUIRE(n >= 0 && d >= 1, "tq_pack_bits: bad shape n=%lld d=%d", (long long)n, d);
  const int oc = static_cast<int>(out_cols(d, b));
  TQ_REQUIRE(ld_idx >= d && ld_out >= oc, "tq_pack_bits: row strides too small");
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(idx && out, "tq_pack_bits: null pointer");
  const int64_t work = n * oc;
  pack_bits_kernel<<<grid_for(work, 256), 256, 0, as_stream(stream)>>>(idx, n, d, ld_idx, b, out,
                                                                        ld_out, oc);
  return launch_status("tq_pack_bits");
}

int tq_unpack_bits(const uint8_t* packed, int64_t n, int32_t d, int64_t ld_in, int32_t b,
                   int32_t* out, int64_t ld_out, void* stream) {
  TQ_REQUIRE(b >= 1 && b <= 8, "tq_unpack_bits: b must be between 1 and 8, got %d", b);
  TQ_REQUIRE(n >= 0 && d >= 1, "tq_unpack_bits: bad shape");
  TQ_REQUIRE(ld_in >= out_cols(d, b) && ld_out >= d, "tq_unpack_bits: row strides too small");
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(packed && out, "tq_unpack_bits: null pointer");
  unpack_bits_kernel<<<grid_for(n * d, 256), 256, 0, as_stream(stream)>>>(packed, n, d, ld_in, b,
                                                                         out, ld_out);
  return launch_status("tq_unpack_bits");
}

int tq_quantize_pack(const float* y, int64_t n, int32_t d, int64_t ld_y, const float* bounds,
                     int32_t b_eff, uint8_t* out, int64_t ld_out, void* stream) {
  TQ_REQUIRE(b_eff >= 1 && b_eff <= 8, "tq_quantize_pack: b_eff must be between 1 and 8, got %d",
             b_eff);
  TQ_REQUIRE(n >= 0 && d >= 1, "tq_quantize_pack: bad shape");
  const int oc = static_cast<int>(out_cols(d, b_eff));
  TQ_REQUIRE(ld_y >= d && ld_out >= oc, "tq_quantize_pack: row strides too small");
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(y && bounds && out, "tq_quantize_pack: null pointer");
  quantize_pack_kernel<<<grid_for(n * oc, 256), 256, 0, as_stream(stream)>>>(
      y, n, d, ld_y, bounds, b_eff, out, ld_out, oc);
  return launch_status("tq_quantize_pack");
}

int tq_dequantize(const uint8_t* packed, int64_t n, int32_t d, int64_t ld_in,
                  const uint16_t* centroids_f16, int32_t b, uint16_t* out_f16, int64_t ld_out,
                  void* stream) {
  TQ_REQUIRE(b >= 1 && b <= 8, "tq_dequantize: b must be between 1 and 8, got %d", b);
  TQ_REQUIRE(n >= 0 && d >= 1, "tq_dequantize: bad shape");
  TQ_REQUIRE(ld_in >= out_cols(d, b) && ld_out >= d, "tq_dequantize: row strides too small");
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(packed && centroids_f16 && out_f16, "tq_dequantize: null pointer");
  dequantize_kernel<<<grid_for(n * d, 256), 256, 0, as_stream(stream)>>>(
      packed, n, d, ld_in, centroids_f16, b, out_f16, ld_out);
  return launch_status("tq_dequantize");
}

}  // extern "C"
