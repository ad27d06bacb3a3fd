// Shared device/host helpers for the gfx950 TurboQuant kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tq_api.h"

namespace tq {

// ---------------------------------------------------------------- errors
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int launch_status(const char* what);  // TQ_OK or TQ_EHIP after a launch

#define TQ_REQUIRE(cond, ...)           \
  do {                                  \
    if (!(cond)) {                      \
      ::tq::set_error(__VA_ARGS__);     \
      return TQ_EINVAL;                 \
    }                                   \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t out_cols(int64_t d, int b) { return (d * b + 7) / 8; }

// Head dims with byte-aligned packed rows (d * b / 8 whole bytes for every bit width) up to 256;
// the tile kernels run them at d rounded up to a multiple of 32 (pad_dim) with zero padding.
inline bool supported_dim(int d) { return d >= 8 && d <= 256 && d % 8 == 0; }
inline int pad_dim(int d) { return (d + 31) / 32 * 32; }

// Blocks of `kernel` (launched with `threads` threads) resident on the whole current
// device at once: occupancy per CU x CU count, cached per device in `cache[16]`.
inline int resident_blocks(const void* kernel, int threads, int* cache) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) dev = 0;
  if (cache[dev] > 0) return cache[dev];
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess || per_cu < 1) per_cu = 1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 1;
  cache[dev] = per_cu * cus;
  return cache[dev];
}

// ---------------------------------------------------------------- vector types
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}
// round-to-nearest-even f32 -> bf16 (NaN kept quiet)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ float h2f(uint16_t v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, v));
}
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <int DT>
__device__ __forceinline__ float load_act(const void* p, int64_t i) {
  if constexpr (DT == TQ_F32) return static_cast<const float*>(p)[i];
  else if constexpr (DT == TQ_F16) return h2f(static_cast<const uint16_t*>(p)[i]);
  else return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}
template <int DT>
__device__ __forceinline__ void store_act(void* p, int64_t i, float v) {
  if constexpr (DT == TQ_F32) static_cast<float*>(p)[i] = v;
  else if constexpr (DT == TQ_F16) static_cast<uint16_t*>(p)[i] = f2h(v);
  else static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
}

// ---------------------------------------------------------------- MFMA
// v_mfma_f32_16x16x32_f16 (gfx950).  Lane l holds A[m = l%16][k = 8*(l/16) + 0..7],
// B[k = 8*(l/16) + 0..7][n = l%16]; the accumulator holds D[m = 4*(l/16) + 0..3][n = l%16].
__device__ __forceinline__ float4v mfma16x16x32(half8 a, half8 b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// f32 operands of f16 MFMA products are split into hi + lo f16 parts after a
// power-of-two scale (kSplit) that keeps both parts in the normal f16 range for
// entries down to ~1e-4 of the row scale; split matrices are stored pre-scaled
// by kSplit, so a product carries kSplit^2, removed exactly by kUnsplit2.
constexpr float kSplit = 1024.f;
constexpr float kUnsplit2 = 1.f / (1024.f * 1024.f);

// Many values divided by one divisor den: r = 1/den once (IEEE division), then per
// value q = x*r and one Markstein correction q + (x - den*q)*r, the remainder exact
// in an fma (P. Markstein, IBM J. Res. Dev. 34(1), 1990: with r correctly rounded and
// q within one ulp of x/den the corrected value is the correctly rounded quotient).
// Three VALU operations per value instead of a full division's ten.
struct DivBy {
  float den, r;
  __device__ __forceinline__ explicit DivBy(float d) : den(d), r(1.f / d) {}
  __device__ __forceinline__ float operator()(float x) const {
    const float q = x * r;
    return fmaf(fmaf(-q, den, x), r, q);
  }
};

// Eight f32 values as f16 hi + lo parts (hi = f16(x), lo = f16(x - hi)): against an
// exact f16 operand (+-1 signs) two MFMAs reproduce an f32 operand to ~2^-22.
__device__ __forceinline__ void split8(const float* p, half8& hi, half8& lo) {
  const float4v a = *reinterpret_cast<const float4v*>(p);
  const float4v b = *reinterpret_cast<const float4v*>(p + 4);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float x = j < 4 ? a[j] : b[j - 4];
    hi[j] = static_cast<_Float16>(x);
    lo[j] = static_cast<_Float16>(x - static_cast<float>(hi[j]));
  }
}
// split8 of the eight values p[j] * qs
__device__ __forceinline__ void split8s(const float* p, float qs, half8& hi, half8& lo) {
  const float4v a = *reinterpret_cast<const float4v*>(p);
  const float4v b = *reinterpret_cast<const float4v*>(p + 4);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float x = (j < 4 ? a[j] : b[j - 4]) * qs;
    hi[j] = static_cast<_Float16>(x);
    lo[j] = static_cast<_Float16>(x - static_cast<float>(hi[j]));
  }
}
// largest |p[j]| of eight values.  Non-temporal loads: the compiler does not merge them with
// the loads of the split that follows, which would hold every value of a lane in registers
// until the maximum is known
__device__ __forceinline__ float absmax8(const float* p) {
  const float4v a = __builtin_nontemporal_load(reinterpret_cast<const float4v*>(p));
  const float4v b = __builtin_nontemporal_load(reinterpret_cast<const float4v*>(p + 4));
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) m = fmaxf(m, fmaxf(fabsf(a[j]), fabsf(b[j])));
  return m;
}
// Power-of-two scale for q_proj's f16 (hi, lo) split: with m the largest |q_proj| the operands
// hold, m * qs lies in [2^13, 2^14), so hi stays finite (f16 ends at 65504, the reference keeps
// q_proj in f32) and lo stays a normal f16 for every value down to ~2^-17 of m.  The QJL
// term's factor takes 1 / qs; both products are exact.  m = 0 (or not finite) gives 1.
__device__ __forceinline__ float qproj_split_scale(float m) {
  int e;
  frexpf(m, &e);  // m < 2^e
  const float qs = (!(m > 0.f) || m > 3.0e38f) ? 1.f : ldexpf(1.f, 14 - e);
  // wave-uniform: kept in a scalar register (the loops around it sit at their VGPR caps)
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, qs)));
}
// maximum over the wave, as a wave-uniform (scalar) value
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int sh = 32; sh >= 1; sh >>= 1) v = fmaxf(v, __shfl_xor(v, sh, 64));
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

__device__ __forceinline__ half8 round8(const float* p) {
  half8 hi, lo;
  split8(p, hi, lo);
  return hi;
}

// The value of lane l ^ 8 (a rotation by 8 within each row of 16 lanes), through DPP.
__device__ __forceinline__ float dpp_row_ror8(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xF, 0xF, false));
}

// Split a value (already scaled by kSplit) into f16 hi + lo parts.
__device__ __forceinline__ void split_f16(float v, _Float16& hi, _Float16& lo) {
  hi = static_cast<_Float16>(v);
  lo = static_cast<_Float16>(v - static_cast<float>(hi));
}
// Packed f16 pairs through v_fma_mixlo_f16 / v_fma_mixhi_f16, each of which rounds an f32
// fma to f16 into one half of its destination and keeps the other half.  For a power-of-two s:
//   f16x2_scaled:       (f16(v0 s), f16(v1 s))                 2 VALU per pair
//   split_f16x2_scaled: hi = that pair, lo = (f16(v0 s - hi0), f16(v1 s - hi1)), the same values
//                       as split_f16(v s) (v s and v s - hi are exact in f32)  4 VALU per pair
// (the compiler's own form of split_f16 on pairs computes hi twice: 7 VALU per pair; measured
// on the key residual at 1M rows: 199.4 vs 205.6 us; for the bf16 -> f16 row conversion, whose
// compiler form is 2 multiplies and one v_cvt_pk_f16_f32 per pair, the mix form was slower).  A
// zero product can come out as +0 where the conversion of v s gives -0; as an MFMA operand either
// zero leaves every sum unchanged.
__device__ __forceinline__ uint32_t f16x2_scaled(float v0, float v1, float s) {
  uint32_t r;
  asm("v_fma_mixlo_f16 %0, %1, %2, 0" : "=&v"(r) : "v"(v0), "v"(s));
  asm("v_fma_mixhi_f16 %0, %1, %2, 0" : "+v"(r) : "v"(v1), "v"(s));
  return r;
}
__device__ __forceinline__ void split_f16x2_scaled(float v0, float v1, float s, uint32_t& hi, uint32_t& lo) {
  const uint32_t h = f16x2_scaled(v0, v1, s);
  uint32_t l;
  asm("v_fma_mixlo_f16 %0, %1, %2, -%3 op_sel_hi:[0,0,1]" : "=&v"(l) : "v"(v0), "v"(s), "v"(h));
  asm("v_fma_mixhi_f16 %0, %1, %2, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "+v"(l) : "v"(v1), "v"(s), "v"(h));
  hi = h;
  lo = l;
}

// Maximum of values that are never NaN (attention scores, finite or -inf; norms) as
// v_max3_f32 / v_max_f32 on the raw operands.  fmaxf on values that reach it through a select or a phi (the masked and
// unmasked paths of a tile) makes the compiler quiet each operand first, one
// `v_max_f32 x, x` per operand: 12 of the ~150 VALU per tile per wave of the prefill loop.
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float max_raw(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// maximum of 8 scores: 3 VALU
__device__ __forceinline__ float max8_raw(float s0, float s1, float s2, float s3, float s4, float s5, float s6,
                                          float s7) {
  return max3_raw(max3_raw(s0, s1, s2), max3_raw(s3, s4, s5), max_raw(s6, s7));
}

// ---------------------------------------------------------------- bits
// Code i of a packed row: bits [i*b, i*b + b), LSB first.
__device__ __forceinline__ uint32_t read_code(const uint8_t* row, int i, int b) {
  const int bit = i * b;
  const int byte = bit >> 3, off = bit & 7;
  uint32_t v = row[byte] >> off;
  if (off + b > 8) v |= static_cast<uint32_t>(row[byte + 1]) << (8 - off);
  return v & ((1u << b) - 1u);
}

// Number of boundaries strictly below y (torch.searchsorted, side='left').
__device__ __forceinline__ uint32_t searchsorted_left(float y, const float* bounds, int nb) {
  uint32_t c = 0;
  for (int j = 0; j < nb; ++j) c += (bounds[j] < y) ? 1u : 0u;
  return c;
}

}  // namespace tq
