// Fused key/value compression, value decompression and query preparation.
//
// Every d x d product here runs on the gfx950 matrix cores as an f16 MFMA
// (v_mfma_f32_16x16x32_f16) with f32 accumulation.  To keep f32 accuracy the
// f32 operands are split into f16 hi + lo parts (x = hi + lo, |lo| <= 2^-11 |x|)
// and three products hi*hi + lo*hi + hi*lo are accumulated; the dropped lo*lo
// term is below 2^-22 relative.  Operands are scaled by kSplit = 2^10 before
// splitting so that the lo parts stay in the normal f16 range; the 2^20 factor
// is removed exactly afterwards.  Operands that are already f16 values (f16 centroids,
// q_rot, S_eff) skip the lo part and give exactly the f32 accumulation of f16
// products that the reference performs.
//
// A block of 256 threads (4 wave64) owns a tile of R rows held in LDS as f32.
// Each GEMM stage computes Z^T = W X^T so the weight matrix W (row-major,
// pre-split in global memory, L2 resident) is the MFMA A operand and the LDS
// row tile is the B operand; the accumulator layout (4 consecutive output
// columns of one row per lane) is written straight back into the row tile.
#include "tq_common.h"

namespace tq {

template <int D>
struct CTile {
  static constexpr int R = (D == 256) ? 16 : (D == 128 ? 32 : 64);  // rows per block tile
  static constexpr int LDA = D + 8;                                  // padded f32 row stride
  static constexpr int MB = D / 16, NB = R / 16, TPW = MB * NB / 4, KS = D / 32;
  static constexpr int NT = 256;
  static constexpr int TPR = NT / R;  // threads per row for row reductions
  static_assert(MB * NB % 4 == 0, "tile count must split over 4 waves");
};

// Z[row][j] = sum_i X[row][i] * W[j][i] for the R x D tile X (LDS, f32).
// wsplit: f16 bits, [2][D][D] = (hi, lo) of kSplit*W.  xscale[row] multiplies
// the row before it is split (it includes the factor kSplit).  Result left in
// acc (times kSplit * xscale); tile t of this wave covers columns
// j = mb*16 + 4*(lane/16) + 0..3 of row nb*16 + lane%16.
template <int D, bool X_SPLIT, bool W_SPLIT>
__device__ __forceinline__ void stage_gemm(const float* __restrict__ X, const float* __restrict__ xscale,
                                           const uint16_t* __restrict__ wsplit,
                                           float4v (&acc)[CTile<D>::TPW]) {
  using T = CTile<D>;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const half8* Wh = reinterpret_cast<const half8*>(wsplit);
  const half8* Wl = reinterpret_cast<const half8*>(wsplit + D * D);
#pragma unroll
  for (int t = 0; t < T::TPW; ++t) acc[t] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < T::KS; ++ks) {
    const int k0 = ks * 32 + g * 8;
#pragma unroll
    for (int t = 0; t < T::TPW; ++t) {
      const int tile = wave * T::TPW + t;
      const int mb = tile / T::NB, nb = tile % T::NB;
      const int j = mb * 16 + l16;
      const half8 ahi = Wh[(j * D + k0) / 8];
      const int row = nb * 16 + l16;
      const float s = xscale[row];
      const float4v* xr = reinterpret_cast<const float4v*>(X + row * T::LDA + k0);
      const float4v x0 = xr[0], x1 = xr[1];
      half8 bhi, blo;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        _Float16 h, l;
        split_f16(x0[e] * s, h, l);
        bhi[e] = h;
        blo[e] = l;
        split_f16(x1[e] * s, h, l);
        bhi[4 + e] = h;
        blo[4 + e] = l;
      }
      acc[t] = mfma16x16x32(ahi, bhi, acc[t]);
      if constexpr (W_SPLIT) {
        const half8 alo = Wl[(j * D + k0) / 8];
        acc[t] = mfma16x16x32(alo, bhi, acc[t]);
      }
      if constexpr (X_SPLIT) acc[t] = mfma16x16x32(ahi, blo, acc[t]);
    }
  }
}

// Strided [B, H, S, D] activation rows, enumerated in (b, h, s) order.
struct Rows4 {
  int64_t H, S, sb, sh, ss;
  __device__ __forceinline__ int64_t offset(int64_t gr) const {
    const int64_t s = gr % S, bh = gr / S;
    return (bh / H) * sb + (bh % H) * sh + s * ss;
  }
};

// Load R rows of activations into the f32 tile (zero rows past n).
template <int D, int DT>
__device__ __forceinline__ void load_rows(float* __restrict__ A, const void* __restrict__ x,
                                          int64_t row0, int64_t n, const Rows4& rows) {
  using T = CTile<D>;
  for (int e = threadIdx.x; e < T::R * D; e += T::NT) {
    const int r = e / D, i = e % D;
    const int64_t gr = row0 + r;
    A[r * T::LDA + i] = (gr < n) ? load_act<DT>(x, rows.offset(gr) + i) : 0.f;
  }
}

// Row reduction: every thread of the TPR-thread group of row r returns the
// sum over the row of f(value).
template <int D, typename F>
__device__ __forceinline__ float row_sum(const float* __restrict__ A, F f) {
  using T = CTile<D>;
  const int r = threadIdx.x / T::TPR, part = threadIdx.x % T::TPR;
  constexpr int PER = D / T::TPR;
  float s = 0.f;
  for (int i = 0; i < PER; ++i) s += f(A[r * T::LDA + part * PER + i]);
#pragma unroll
  for (int off = T::TPR / 2; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
  return s;
}

// Build packed word w (bits [32w, 32w+32)) of a row from its byte codes.
__device__ __forceinline__ uint32_t pack_word(const uint8_t* __restrict__ codes, int d, int b, int w) {
  const int lo_bit = 32 * w;
  const int c0 = lo_bit / b;
  int c1 = (lo_bit + 31) / b;
  if (c1 > d - 1) c1 = d - 1;
  uint32_t acc = 0;
  for (int c = c0; c <= c1; ++c) {
    const uint32_t v = codes[c];
    const int sh = c * b - lo_bit;
    acc |= (sh >= 0) ? (v << sh) : (v >> (-sh));
  }
  return acc;
}

struct KeyArgs {
  const void* x;
  int64_t n;
  Rows4 rows;
  const uint16_t *pi, *pit, *s;
  const float *cent, *bounds;
  int b;
  uint8_t *codes, *signs;
  uint16_t *rn, *vn;
  float *y_out, *proj_out;
};

template <int D, int DT>
__global__ void __launch_bounds__(256) compress_keys_kernel(KeyArgs a) {
  using T = CTile<D>;
  __shared__ float A[T::R * T::LDA];   // x
  __shared__ float Bm[T::R * T::LDA];  // stage data
  __shared__ uint8_t idx[T::R * D];
  __shared__ float s_vn[T::R], s_sc[T::R], s_rsc[T::R], s_cent16[256], s_bnd[255];

  const int nb = (1 << a.b) - 1;
  for (int j = threadIdx.x; j <= nb; j += T::NT) {
    // reconstruction uses the f16-rounded centroids (compressors.py:120-122)
    s_cent16[j] = static_cast<float>(static_cast<_Float16>(a.cent[j]));
    if (j < nb) s_bnd[j] = a.bounds[j];
  }
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * T::R;
  load_rows<D, DT>(A, a.x, row0, a.n, a.rows);
  if (threadIdx.x < T::R) s_sc[threadIdx.x] = kSplit;
  __syncthreads();

  // vn = ||x||; xn = x / (vn + 1e-8)   (compressors.py:108-109)
  {
    const float ss = row_sum<D>(A, [](float v) { return v * v; });
    const int r = threadIdx.x / T::TPR;
    const float vn = sqrtf(ss);
    if (threadIdx.x % T::TPR == 0) s_vn[r] = vn;
    const float den = vn + 1e-8f;
    constexpr int PER = D / T::TPR;
    const int part = threadIdx.x % T::TPR;
    for (int i = 0; i < PER; ++i) {
      const int c = part * PER + i;
      Bm[r * T::LDA + c] = A[r * T::LDA + c] / den;
    }
  }
  __syncthreads();

  float4v acc[T::TPW];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g = lane >> 4;

  // stage 1: y = xn Pi^T (compressors.py:112)
  stage_gemm<D, true, true>(Bm, s_sc, a.pi, acc);
  __syncthreads();
#pragma unroll
  for (int t = 0; t < T::TPW; ++t) {
    const int tile = wave * T::TPW + t;
    const int row = (tile % T::NB) * 16 + l16, col = (tile / T::NB) * 16 + 4 * g;
#pragma unroll
    for (int e = 0; e < 4; ++e) Bm[row * T::LDA + col + e] = acc[t][e] * kUnsplit2;
  }
  __syncthreads();

  // quantize (searchsorted-left on f32 boundaries), reconstruct with f16 centroids
  for (int e = threadIdx.x; e < T::R * D; e += T::NT) {
    const int r = e / D, i = e % D;
    const float y = Bm[r * T::LDA + i];
    const uint32_t c = searchsorted_left(y, s_bnd, nb);
    idx[r * D + i] = static_cast<uint8_t>(c);
    Bm[r * T::LDA + i] = s_cent16[c];
    const int64_t gr = row0 + r;
    if (a.y_out && gr < a.n) a.y_out[gr * D + i] = y;
  }
  __syncthreads();

  // stage 2: k_mse = (yhat Pi) * vn; r = x - k_mse   (compressors.py:120-126)
  stage_gemm<D, false, true>(Bm, s_sc, a.pit, acc);
  __syncthreads();
#pragma unroll
  for (int t = 0; t < T::TPW; ++t) {
    const int tile = wave * T::TPW + t;
    const int row = (tile % T::NB) * 16 + l16, col = (tile / T::NB) * 16 + 4 * g;
    const float vn = s_vn[row];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float kmse = (acc[t][e] * kUnsplit2) * vn;
      Bm[row * T::LDA + col + e] = A[row * T::LDA + col + e] - kmse;
    }
  }
  __syncthreads();
  {
    const float ss = row_sum<D>(Bm, [](float v) { return v * v; });
    const int r = threadIdx.x / T::TPR;
    if (threadIdx.x % T::TPR == 0) {
      const float rn = sqrtf(ss);
      int e2;
      frexpf(rn, &e2);  // rn = m * 2^e2, m in [0.5, 1)
      s_rsc[r] = ldexpf(1.f, e2);
      s_sc[r] = ldexpf(kSplit, -e2);  // residual scaled to norm in [0.5, 1)
      const int64_t gr = row0 + r;
      if (gr < a.n) {
        a.rn[gr] = f2h(rn);
        a.vn[gr] = f2h(s_vn[r]);
      }
    }
  }
  __syncthreads();

  // stage 3: proj = r S^T; sign bit = proj >= 0   (compressors.py:128-130)
  stage_gemm<D, true, true>(Bm, s_sc, a.s, acc);
  __syncthreads();
#pragma unroll
  for (int t = 0; t < T::TPW; ++t) {
    const int tile = wave * T::TPW + t;
    const int row = (tile % T::NB) * 16 + l16, col = (tile / T::NB) * 16 + 4 * g;
    const float rs = s_rsc[row];
#pragma unroll
    for (int e = 0; e < 4; ++e) Bm[row * T::LDA + col + e] = (acc[t][e] * kUnsplit2) * rs;
  }
  __syncthreads();

  // pack codes (b bits) and signs (1 bit) a 32-bit word per thread
  const int kw = D * a.b / 32, sw = D / 32;
  for (int e = threadIdx.x; e < T::R * (kw + sw); e += T::NT) {
    const int r = e / (kw + sw), w = e % (kw + sw);
    const int64_t gr = row0 + r;
    if (gr >= a.n) continue;
    if (w < kw) {
      reinterpret_cast<uint32_t*>(a.codes + gr * (D * a.b / 8))[w] = pack_word(idx + r * D, D, a.b, w);
    } else {
      const int ws = w - kw;
      uint32_t bits = 0;
      for (int k = 0; k < 32; ++k) bits |= (Bm[r * T::LDA + ws * 32 + k] >= 0.f ? 1u : 0u) << k;
      reinterpret_cast<uint32_t*>(a.signs + gr * (D / 8))[ws] = bits;
    }
  }
  if (a.proj_out) {
    for (int e = threadIdx.x; e < T::R * D; e += T::NT) {
      const int r = e / D, i = e % D;
      const int64_t gr = row0 + r;
      if (gr < a.n) a.proj_out[gr * D + i] = Bm[r * T::LDA + i];
    }
  }
}

struct ValArgs {
  const void* x;
  int64_t n;
  Rows4 rows;
  const uint16_t* pi;
  const float* bounds;
  int b;
  uint8_t* codes;
  uint16_t* vn;
  float* y_out;
};

template <int D, int DT>
__global__ void __launch_bounds__(256) compress_values_kernel(ValArgs a) {
  using T = CTile<D>;
  __shared__ float A[T::R * T::LDA];
  __shared__ uint8_t idx[T::R * D];
  __shared__ float s_sc[T::R], s_bnd[255];
  const int nb = (1 << a.b) - 1;
  for (int j = threadIdx.x; j < nb; j += T::NT) s_bnd[j] = a.bounds[j];
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * T::R;
  load_rows<D, DT>(A, a.x, row0, a.n, a.rows);
  if (threadIdx.x < T::R) s_sc[threadIdx.x] = kSplit;
  __syncthreads();
  {
    const float ss = row_sum<D>(A, [](float v) { return v * v; });
    const int r = threadIdx.x / T::TPR;
    const float vn = sqrtf(ss);
    const int64_t gr = row0 + r;
    if (threadIdx.x % T::TPR == 0 && gr < a.n) a.vn[gr] = f2h(vn);
    const float den = vn + 1e-8f;
    constexpr int PER = D / T::TPR;
    const int part = threadIdx.x % T::TPR;
    __syncthreads();
    for (int i = 0; i < PER; ++i) A[r * T::LDA + part * PER + i] /= den;
  }
  __syncthreads();
  float4v acc[T::TPW];
  stage_gemm<D, true, true>(A, s_sc, a.pi, acc);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int t = 0; t < T::TPW; ++t) {
    const int tile = wave * T::TPW + t;
    const int row = (tile % T::NB) * 16 + l16, col = (tile / T::NB) * 16 + 4 * g;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float y = acc[t][e] * kUnsplit2;
      idx[row * D + col + e] = static_cast<uint8_t>(searchsorted_left(y, s_bnd, nb));
      const int64_t gr = row0 + row;
      if (a.y_out && gr < a.n) a.y_out[gr * D + col + e] = y;
    }
  }
  __syncthreads();
  const int kw = D * a.b / 32;
  for (int e = threadIdx.x; e < T::R * kw; e += T::NT) {
    const int r = e / kw, w = e % kw;
    const int64_t gr = row0 + r;
    if (gr < a.n)
      reinterpret_cast<uint32_t*>(a.codes + gr * (D * a.b / 8))[w] = pack_word(idx + r * D, D, a.b, w);
  }
}

struct DecArgs {
  const uint8_t* codes;
  const uint16_t* vn;
  int64_t n;
  const uint16_t* pit;
  const float* cent;
  int b;
  void* out;
  int64_t ld_out;
};

template <int D, int DT>
__global__ void __launch_bounds__(256) decompress_values_kernel(DecArgs a) {
  using T = CTile<D>;
  __shared__ float A[T::R * T::LDA];
  __shared__ float s_sc[T::R], s_cent[256];
  for (int j = threadIdx.x; j < (1 << a.b); j += T::NT) s_cent[j] = a.cent[j];
  if (threadIdx.x < T::R) s_sc[threadIdx.x] = kSplit;
  __syncthreads();
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * T::R;
  const int kc = D * a.b / 8;
  for (int e = threadIdx.x; e < T::R * D; e += T::NT) {
    const int r = e / D, i = e % D;
    const int64_t gr = row0 + r;
    A[r * T::LDA + i] = (gr < a.n) ? s_cent[read_code(a.codes + gr * kc, i, a.b)] : 0.f;
  }
  __syncthreads();
  float4v acc[T::TPW];
  stage_gemm<D, true, true>(A, s_sc, a.pit, acc);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int t = 0; t < T::TPW; ++t) {
    const int tile = wave * T::TPW + t;
    const int row = (tile % T::NB) * 16 + l16, col = (tile / T::NB) * 16 + 4 * g;
    const int64_t gr = row0 + row;
    if (gr >= a.n) continue;
    const float vn = h2f(a.vn[gr]);
#pragma unroll
    for (int e = 0; e < 4; ++e) store_act<DT>(a.out, gr * a.ld_out + col + e, (acc[t][e] * kUnsplit2) * vn);
  }
}

struct PrepArgs {
  const void* q;
  int B, Hq, Sq;
  int64_t sqb, sqh, sqs;
  const uint16_t *pi, *seff;
  uint16_t *q_rot, *q_proj;
};

template <int D, int DT>
__global__ void __launch_bounds__(256) query_prep_kernel(PrepArgs a) {
  using T = CTile<D>;
  __shared__ float A[T::R * T::LDA];
  __shared__ float s_sc[T::R], s_inv[T::R];
  const int64_t n = static_cast<int64_t>(a.B) * a.Hq * a.Sq;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * T::R;
  for (int e = threadIdx.x; e < T::R * D; e += T::NT) {
    const int r = e / D, i = e % D;
    const int64_t gr = row0 + r;
    float v = 0.f;
    if (gr < n) {
      const int64_t s = gr % a.Sq, bh = gr / a.Sq;
      const int64_t h = bh % a.Hq, b = bh / a.Hq;
      v = load_act<DT>(a.q, b * a.sqb + h * a.sqh + s * a.sqs + i);
    }
    A[r * T::LDA + i] = v;
  }
  __syncthreads();
  // per-row power-of-two scale so |64 * q * scale| <= 64
  {
    const int r = threadIdx.x / T::TPR, part = threadIdx.x % T::TPR;
    constexpr int PER = D / T::TPR;
    float m = 0.f;
    for (int i = 0; i < PER; ++i) m = fmaxf(m, fabsf(A[r * T::LDA + part * PER + i]));
#pragma unroll
    for (int off = T::TPR / 2; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if (part == 0) {
      int e2;
      frexpf(m, &e2);
      s_sc[r] = ldexpf(kSplit, -e2);
      s_inv[r] = ldexpf(kUnsplit2, e2);
    }
  }
  __syncthreads();
  float4v acc[T::TPW];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  // q_rot = f16(q Pi^T)   (compressors.py:186)
  stage_gemm<D, true, true>(A, s_sc, a.pi, acc);
  __syncthreads();
#pragma unroll
  for (int t = 0; t < T::TPW; ++t) {
    const int tile = wave * T::TPW + t;
    const int row = (tile % T::NB) * 16 + l16, col = (tile / T::NB) * 16 + 4 * g;
    const int64_t gr = row0 + row;
    const float inv = s_inv[row];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const _Float16 h = static_cast<_Float16>(acc[t][e] * inv);
      A[row * T::LDA + col + e] = static_cast<float>(h);
      if (gr < n) a.q_rot[gr * D + col + e] = __builtin_bit_cast(uint16_t, h);
    }
  }
  __syncthreads();
  {
    const int r = threadIdx.x / T::TPR, part = threadIdx.x % T::TPR;
    constexpr int PER = D / T::TPR;
    float m = 0.f;
    for (int i = 0; i < PER; ++i) m = fmaxf(m, fabsf(A[r * T::LDA + part * PER + i]));
#pragma unroll
    for (int off = T::TPR / 2; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    __syncthreads();
    if (part == 0) {
      // q_rot holds f16 values: scaling by 2^(12-e) keeps them exact in f16
      int e2;
      frexpf(m, &e2);
      s_sc[r] = ldexpf(4096.f, -e2);
      s_inv[r] = ldexpf(1.f / 4096.f, e2);
    }
  }
  __syncthreads();
  // q_proj = f16(q_rot S_eff^T), f32 accumulation of exact f16 products
  // (kernels/attention.py:158-167); S_eff is used unscaled, hi part only
  stage_gemm<D, false, false>(A, s_sc, a.seff, acc);
#pragma unroll
  for (int t = 0; t < T::TPW; ++t) {
    const int tile = wave * T::TPW + t;
    const int row = (tile % T::NB) * 16 + l16, col = (tile / T::NB) * 16 + 4 * g;
    const int64_t gr = row0 + row;
    if (gr >= n) continue;
    const float inv = s_inv[row];
#pragma unroll
    for (int e = 0; e < 4; ++e) a.q_proj[gr * D + col + e] = f2h(acc[t][e] * inv);
  }
}

// ---------------------------------------------------------------- dispatch
#define TQ_DEFINE_LAUNCH(NAME, KERNEL, ARGS)                                                     \
  template <int D, int DT>                                                                      \
  static void NAME(const ARGS& a, int64_t rows, hipStream_t s) {                               \
    const unsigned grid = static_cast<unsigned>((rows + CTile<D>::R - 1) / CTile<D>::R);        \
    KERNEL<D, DT><<<grid, 256, 0, s>>>(a);                                                      \
  }
TQ_DEFINE_LAUNCH(launch_keys, compress_keys_kernel, KeyArgs)
TQ_DEFINE_LAUNCH(launch_values, compress_values_kernel, ValArgs)
TQ_DEFINE_LAUNCH(launch_decomp, decompress_values_kernel, DecArgs)
TQ_DEFINE_LAUNCH(launch_prep, query_prep_kernel, PrepArgs)

#define TQ_SWITCH_DD(FN, d, dt, ...)                                    \
  switch ((d) * 4 + (dt)) {                                              \
    case 32 * 4 + TQ_F32: FN<32, TQ_F32>(__VA_ARGS__); break;            \
    case 32 * 4 + TQ_F16: FN<32, TQ_F16>(__VA_ARGS__); break;            \
    case 32 * 4 + TQ_BF16: FN<32, TQ_BF16>(__VA_ARGS__); break;          \
    case 64 * 4 + TQ_F32: FN<64, TQ_F32>(__VA_ARGS__); break;            \
    case 64 * 4 + TQ_F16: FN<64, TQ_F16>(__VA_ARGS__); break;            \
    case 64 * 4 + TQ_BF16: FN<64, TQ_BF16>(__VA_ARGS__); break;          \
    case 128 * 4 + TQ_F32: FN<128, TQ_F32>(__VA_ARGS__); break;          \
    case 128 * 4 + TQ_F16: FN<128, TQ_F16>(__VA_ARGS__); break;          \
    case 128 * 4 + TQ_BF16: FN<128, TQ_BF16>(__VA_ARGS__); break;        \
    case 256 * 4 + TQ_F32: FN<256, TQ_F32>(__VA_ARGS__); break;          \
    case 256 * 4 + TQ_F16: FN<256, TQ_F16>(__VA_ARGS__); break;          \
    case 256 * 4 + TQ_BF16: FN<256, TQ_BF16>(__VA_ARGS__); break;        \
    default: break;                                                      \
  }

}  // namespace tq

using namespace tq;

#define TQ_CHECK_DD(what, d, dtype)                                                              \
  do {                                                                                           \
    if (!supported_dim(d)) {                                                                     \
      set_error("%s: head_dim %d not built (supported: 32, 64, 128, 256)", what, (int)(d));     \
      return TQ_EUNSUPPORTED;                                                                    \
    }                                                                                            \
    TQ_REQUIRE((dtype) == TQ_F32 || (dtype) == TQ_F16 || (dtype) == TQ_BF16,                     \
               "%s: unknown dtype %d", what, (int)(dtype));                                     \
  } while (0)

extern "C" {

int tq_compress_keys(const void* x, int32_t dtype, int32_t B, int32_t H, int32_t S, int32_t d,
                     int64_t sxb, int64_t sxh, int64_t sxs, const uint16_t* pi_split, const uint16_t* pit_split, const uint16_t* s_split,
                     const float* centroids, const float* bounds, int32_t b_eff, uint8_t* codes,
                     uint8_t* signs, uint16_t* rn, uint16_t* vn, float* y_out, float* proj_out,
                     void* stream) {
  TQ_CHECK_DD("tq_compress_keys", d, dtype);
  TQ_REQUIRE(b_eff >= 1 && b_eff <= 8, "tq_compress_keys: b_eff must be in [1, 8], got %d", b_eff);
  TQ_REQUIRE(B >= 0 && H >= 0 && S >= 0, "tq_compress_keys: bad shape");
  const int64_t n = static_cast<int64_t>(B) * H * S;
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(x && pi_split && pit_split && s_split && centroids && bounds && codes && signs && rn && vn,
             "tq_compress_keys: null pointer");
  KeyArgs a{x, n, Rows4{H, S, sxb, sxh, sxs}, pi_split, pit_split, s_split, centroids, bounds, b_eff, codes, signs, rn, vn,
            y_out, proj_out};
  TQ_SWITCH_DD(launch_keys, d, dtype, a, n, as_stream(stream));
  return launch_status("tq_compress_keys");
}

int tq_compress_values(const void* x, int32_t dtype, int32_t B, int32_t H, int32_t S, int32_t d,
                       int64_t sxb, int64_t sxh, int64_t sxs, const uint16_t* pi_split, const float* bounds, int32_t b, uint8_t* codes,
                       uint16_t* vn, float* y_out, void* stream) {
  TQ_CHECK_DD("tq_compress_values", d, dtype);
  TQ_REQUIRE(b >= 1 && b <= 8, "tq_compress_values: bits must be in [1, 8], got %d", b);
  TQ_REQUIRE(B >= 0 && H >= 0 && S >= 0, "tq_compress_values: bad shape");
  const int64_t n = static_cast<int64_t>(B) * H * S;
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(x && pi_split && bounds && codes && vn, "tq_compress_values: null pointer");
  ValArgs a{x, n, Rows4{H, S, sxb, sxh, sxs}, pi_split, bounds, b, codes, vn, y_out};
  TQ_SWITCH_DD(launch_values, d, dtype, a, n, as_stream(stream));
  return launch_status("tq_compress_values");
}

int tq_decompress_values(const uint8_t* codes, const uint16_t* vn, int64_t n, int32_t d,
                         const uint16_t* pit_split, const float* centroids, int32_t b, void* out,
                         int32_t out_dtype, int64_t ld_out, void* stream) {
  TQ_CHECK_DD("tq_decompress_values", d, out_dtype);
  TQ_REQUIRE(b >= 1 && b <= 8, "tq_decompress_values: bits must be in [1, 8], got %d", b);
  TQ_REQUIRE(n >= 0 && ld_out >= d, "tq_decompress_values: bad shape");
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(codes && vn && pit_split && centroids && out, "tq_decompress_values: null pointer");
  DecArgs a{codes, vn, n, pit_split, centroids, b, out, ld_out};
  TQ_SWITCH_DD(launch_decomp, d, out_dtype, a, n, as_stream(stream));
  return launch_status("tq_decompress_values");
}

int tq_query_prep(const void* q, int32_t dtype, int32_t B, int32_t Hq, int32_t Sq, int32_t d,
                  int64_t sqb, int64_t sqh, int64_t sqs, const uint16_t* pi_split,
                  const uint16_t* s_eff_f16, uint16_t* q_rot, uint16_t* q_proj, void* stream) {
  TQ_CHECK_DD("tq_query_prep", d, dtype);
  TQ_REQUIRE(B >= 0 && Hq >= 0 && Sq >= 0, "tq_query_prep: bad shape");
  const int64_t n = static_cast<int64_t>(B) * Hq * Sq;
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(q && pi_split && s_eff_f16 && q_rot && q_proj, "tq_query_prep: null pointer");
  PrepArgs a{q, B, Hq, Sq, sqb, sqh, sqs, pi_split, s_eff_f16, q_rot, q_proj};
  TQ_SWITCH_DD(launch_prep, d, dtype, a, n, as_stream(stream));
  return launch_status("tq_query_prep");
}

}  // extern "C"
