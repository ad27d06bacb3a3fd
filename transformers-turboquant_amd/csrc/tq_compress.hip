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
// Two kernel families:
// * row-owned kernels (head_dim 64 / 128, 1-4 code bits): each wave owns 16
//   rows end to end with the weights in LDS; see the section comment below.
// * tile kernels (every head_dim, any bit width; also decompression): a block
//   of 256 threads owns a tile of R rows held in LDS as f32.  Each GEMM stage
//   computes Z^T = W X^T so the weight matrix W (row-major, pre-split in global
//   memory, L2 resident) is the MFMA A operand and the LDS row tile is the B
//   operand; the accumulator layout (4 consecutive output columns of one row per
//   lane) is written straight back into the row tile.
#include <algorithm>
#include <type_traits>

#include "tq_common.h"
#include "tq_stream.h"

typedef float float2v __attribute__((ext_vector_type(2)));

namespace tq {

// D is the head dim padded to a multiple of 32 (the MFMA k-step); a row's d <= D real
// coordinates are followed by zeros in every LDS tile, and weight rows and columns past d
// read as zero, so padded coordinates add nothing to any product.
template <int D>
struct CTile {
  static constexpr int R = (D <= 64) ? 64 : (D <= 224 ? 32 : 16);  // rows per block tile
  static constexpr int LDA = D + 8;                                  // padded f32 row stride
  static constexpr int MB = D / 16, NB = R / 16, TPW = MB * NB / 4, KS = D / 32;
  static constexpr int NT = 256;
  static constexpr int TPR = NT / R;  // threads per row for row reductions
  static_assert(MB * NB % 4 == 0, "tile count must split over 4 waves");
};

// Z[row][j] = sum_i X[row][i] * W[j][i] for the R x D tile X (LDS, f32).
// wsplit: f16 bits, [2][d][d] = (hi, lo) of kSplit*W (rows and columns past d read as 0).  xscale[row] multiplies
// the row before it is split (it includes the factor kSplit).  Result left in
// acc (times kSplit * xscale); tile t of this wave covers columns
// j = mb*16 + 4*(lane/16) + 0..3 of row nb*16 + lane%16.
template <int D, bool X_SPLIT, bool W_SPLIT>
__device__ __forceinline__ void stage_gemm(const float* __restrict__ X, const float* __restrict__ xscale,
                                           const uint16_t* __restrict__ wsplit, int d,
                                           float4v (&acc)[CTile<D>::TPW]) {
  using T = CTile<D>;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const half8* Wh = reinterpret_cast<const half8*>(wsplit);
  const half8* Wl = reinterpret_cast<const half8*>(wsplit + static_cast<int64_t>(d) * d);
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
      const bool win = j < d && k0 < d;  // d % 8 == 0: the 8 columns from k0 are all real or all padding
      const half8 ahi = win ? Wh[(j * d + k0) / 8] : half8{};
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
        const half8 alo = win ? Wl[(j * d + k0) / 8] : half8{};
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

// Load R rows of d activations into the f32 tile (zero rows past n, zero columns past d).
template <int D, int DT>
__device__ __forceinline__ void load_rows(float* __restrict__ A, const void* __restrict__ x,
                                          int64_t row0, int64_t n, int d, const Rows4& rows) {
  using T = CTile<D>;
  for (int e = threadIdx.x; e < T::R * D; e += T::NT) {
    const int r = e / D, i = e % D;
    const int64_t gr = row0 + r;
    A[r * T::LDA + i] = (gr < n && i < d) ? load_act<DT>(x, rows.offset(gr) + i) : 0.f;
  }
}

// Bytes [0, nbytes) of a packed row from its 32-bit words, byte by byte (rows of d * b / 8
// bytes need not be dword aligned).
__device__ __forceinline__ void store_word_bytes(uint8_t* row, int w, int nbytes, uint32_t word) {
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (4 * w + k < nbytes) row[4 * w + k] = static_cast<uint8_t>(word >> (8 * k));
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
  const uint16_t *pi, *seff;
  const float *cent, *bounds;
  int b;
  uint8_t *codes, *signs;
  uint16_t *rn, *vn;
  float *y_out, *proj_out;
  int d;  // head dim, d <= D, d % 8 == 0
  // output rows: input row (b, h, s) of S_in positions goes to (b * H + h) * ldo + off + s;
  // ldo = 0 writes it to row (b, h, s)
  int64_t S_in, ldo, off;
};

__device__ __forceinline__ int64_t map_row(int64_t gr, int64_t S_in, int64_t ldo, int64_t off) {
  return ldo == 0 ? gr : (gr / S_in) * ldo + off + gr % S_in;
}

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
  const int d = a.d;
  load_rows<D, DT>(A, a.x, row0, a.n, d, a.rows);
  if (threadIdx.x < T::R) s_sc[threadIdx.x] = kSplit;
  __syncthreads();

  // vn = ||x||; xn = x / (vn + 1e-8)   (compressors.py:108-109)
  {
    const float ss = row_sum<D>(A, [](float v) { return v * v; });
    const int r = threadIdx.x / T::TPR;
    const float vn = sqrtf(ss);
    if (threadIdx.x % T::TPR == 0) s_vn[r] = vn;
    const DivBy div(vn + 1e-8f);
    constexpr int PER = D / T::TPR;
    const int part = threadIdx.x % T::TPR;
    for (int i = 0; i < PER; ++i) {
      const int c = part * PER + i;
      Bm[r * T::LDA + c] = div(A[r * T::LDA + c]);
    }
  }
  __syncthreads();

  float4v acc[T::TPW];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g = lane >> 4;

  // stage 1: y = xn Pi^T (compressors.py:112)
  stage_gemm<D, true, true>(Bm, s_sc, a.pi, d, acc);
  __syncthreads();
#pragma unroll
  for (int t = 0; t < T::TPW; ++t) {
    const int tile = wave * T::TPW + t;
    const int row = (tile % T::NB) * 16 + l16, col = (tile / T::NB) * 16 + 4 * g;
#pragma unroll
    for (int e = 0; e < 4; ++e) Bm[row * T::LDA + col + e] = acc[t][e] * kUnsplit2;
  }
  __syncthreads();

  // quantize (searchsorted-left on f32 boundaries); the residual in the rotated domain,
  // u = r Pi^T = (vn + 1e-8) y - vn f16(C)[c]  (compressors.py:120-126: r = x - (yhat Pi) vn)
  for (int e = threadIdx.x; e < T::R * D; e += T::NT) {
    const int r = e / D, i = e % D;
    if (i >= d) {  // padding: no code, zero residual
      Bm[r * T::LDA + i] = 0.f;
      continue;
    }
    const float y = Bm[r * T::LDA + i];
    const uint32_t c = searchsorted_left(y, s_bnd, nb);
    idx[r * D + i] = static_cast<uint8_t>(c);
    const float vn = s_vn[r];
    Bm[r * T::LDA + i] = fmaf(vn + 1e-8f, y, -vn * s_cent16[c]);
    const int64_t gr = row0 + r;
    if (a.y_out && gr < a.n) a.y_out[gr * d + i] = y;
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
        const int64_t orow = map_row(gr, a.S_in, a.ldo, a.off);
        a.rn[orow] = f2h(rn);
        a.vn[orow] = f2h(s_vn[r]);
      }
    }
  }
  __syncthreads();

  // stage 2: proj = r S^T = u S_eff^T with S_eff = S Pi^T; sign bit = proj >= 0   (compressors.py:128-130)
  stage_gemm<D, true, true>(Bm, s_sc, a.seff, d, acc);
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

  // pack codes (b bits) and signs (1 bit) a 32-bit word per thread; rows of d * b / 8 and d / 8
  // bytes, stored bytewise when they are not whole words
  const int kbytes = d * a.b / 8, sbytes = d / 8;
  const int kw = (kbytes + 3) / 4, sw = (sbytes + 3) / 4;
  const bool whole = (kbytes % 4 == 0) && (sbytes % 4 == 0);
  for (int e = threadIdx.x; e < T::R * (kw + sw); e += T::NT) {
    const int r = e / (kw + sw), w = e % (kw + sw);
    const int64_t gr = row0 + r;
    if (gr >= a.n) continue;
    const int64_t orow = map_row(gr, a.S_in, a.ldo, a.off);
    if (w < kw) {
      const uint32_t word = pack_word(idx + r * D, d, a.b, w);
      if (whole) reinterpret_cast<uint32_t*>(a.codes + orow * kbytes)[w] = word;
      else store_word_bytes(a.codes + orow * kbytes, w, kbytes, word);
    } else {
      const int ws = w - kw;
      uint32_t bits = 0;
      for (int k = 0; k < 32; ++k) bits |= (Bm[r * T::LDA + ws * 32 + k] >= 0.f ? 1u : 0u) << k;
      if (whole) reinterpret_cast<uint32_t*>(a.signs + orow * sbytes)[ws] = bits;
      else store_word_bytes(a.signs + orow * sbytes, ws, sbytes, bits);
    }
  }
  if (a.proj_out) {
    for (int e = threadIdx.x; e < T::R * D; e += T::NT) {
      const int r = e / D, i = e % D;
      const int64_t gr = row0 + r;
      if (gr < a.n && i < d) a.proj_out[gr * d + i] = Bm[r * T::LDA + i];
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
  int d;  // head dim, d <= D, d % 8 == 0
  int64_t S_in, ldo, off;  // output rows as in KeyArgs
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
  const int d = a.d;
  load_rows<D, DT>(A, a.x, row0, a.n, d, a.rows);
  if (threadIdx.x < T::R) s_sc[threadIdx.x] = kSplit;
  __syncthreads();
  {
    const float ss = row_sum<D>(A, [](float v) { return v * v; });
    const int r = threadIdx.x / T::TPR;
    const float vn = sqrtf(ss);
    const int64_t gr = row0 + r;
    if (threadIdx.x % T::TPR == 0 && gr < a.n) a.vn[map_row(gr, a.S_in, a.ldo, a.off)] = f2h(vn);
    const DivBy div(vn + 1e-8f);
    constexpr int PER = D / T::TPR;
    const int part = threadIdx.x % T::TPR;
    __syncthreads();
    for (int i = 0; i < PER; ++i) A[r * T::LDA + part * PER + i] = div(A[r * T::LDA + part * PER + i]);
  }
  __syncthreads();
  float4v acc[T::TPW];
  stage_gemm<D, true, true>(A, s_sc, a.pi, d, acc);
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
      if (a.y_out && gr < a.n && col + e < d) a.y_out[gr * d + col + e] = y;
    }
  }
  __syncthreads();
  const int kbytes = d * a.b / 8, kw = (kbytes + 3) / 4;
  for (int e = threadIdx.x; e < T::R * kw; e += T::NT) {
    const int r = e / kw, w = e % kw;
    const int64_t gr = row0 + r;
    if (gr >= a.n) continue;
    const int64_t orow = map_row(gr, a.S_in, a.ldo, a.off);
    const uint32_t word = pack_word(idx + r * D, d, a.b, w);
    if (kbytes % 4 == 0) reinterpret_cast<uint32_t*>(a.codes + orow * kbytes)[w] = word;
    else store_word_bytes(a.codes + orow * kbytes, w, kbytes, word);
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
  int d;  // head dim, d <= D, d % 8 == 0
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
  const int d = a.d;
  const int kc = d * a.b / 8;
  for (int e = threadIdx.x; e < T::R * D; e += T::NT) {
    const int r = e / D, i = e % D;
    const int64_t gr = row0 + r;
    A[r * T::LDA + i] = (gr < a.n && i < d) ? s_cent[read_code(a.codes + gr * kc, i, a.b)] : 0.f;
  }
  __syncthreads();
  float4v acc[T::TPW];
  stage_gemm<D, true, true>(A, s_sc, a.pit, d, acc);
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
    for (int e = 0; e < 4; ++e)
      if (col + e < d) store_act<DT>(a.out, gr * a.ld_out + col + e, (acc[t][e] * kUnsplit2) * vn);
  }
}

struct PrepArgs {
  const void* q;
  int B, Hq, Sq;
  int64_t sqb, sqh, sqs;
  const uint16_t *pi, *seff;
  uint16_t* q_rot;
  float* q_proj;
  int d;  // head dim, d <= D, d % 8 == 0
};

template <int D, int DT>
__global__ void __launch_bounds__(256) query_prep_kernel(PrepArgs a) {
  using T = CTile<D>;
  __shared__ float A[T::R * T::LDA];
  __shared__ float s_sc[T::R], s_inv[T::R];
  const int64_t n = static_cast<int64_t>(a.B) * a.Hq * a.Sq;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * T::R;
  const int d = a.d;
  for (int e = threadIdx.x; e < T::R * D; e += T::NT) {
    const int r = e / D, i = e % D;
    const int64_t gr = row0 + r;
    float v = 0.f;
    if (gr < n && i < d) {
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
  stage_gemm<D, true, true>(A, s_sc, a.pi, d, acc);
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
      if (gr < n && col + e < d) a.q_rot[gr * d + col + e] = __builtin_bit_cast(uint16_t, h);
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
  // q_proj = q_rot S_eff^T in f32: f32 accumulation of exact f16 products, as the reference's
  // fp32 q_rot.float() @ S_eff.float().T (kernels/attention.py:158-167, :453); S_eff is used
  // unscaled, hi part only
  stage_gemm<D, false, false>(A, s_sc, a.seff, d, acc);
#pragma unroll
  for (int t = 0; t < T::TPW; ++t) {
    const int tile = wave * T::TPW + t;
    const int row = (tile % T::NB) * 16 + l16, col = (tile / T::NB) * 16 + 4 * g;
    const int64_t gr = row0 + row;
    if (gr >= n) continue;
    const float inv = s_inv[row];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (col + e < d) a.q_proj[gr * d + col + e] = acc[t][e] * inv;
  }
}

// ---------------------------------------------------------------- row-owned kernels (head_dim 64 / 128)
// The same products, organised for throughput.  A block of 16 wave64 walks
// rounds of 256 rows (persistent: the grid is what the device holds at once);
// wave w owns rows 16w .. 16w+15 of a round and computes every output column of
// them, so nothing is exchanged between waves inside a product and row norms
// and maxima are shuffle reductions.  The weights live in LDS for the whole
// block.  A wave's rows are the MFMA B operand, split into f16 (hi, lo) in
// registers: lane (row l16, group g) supplies k = 32*ks + 8g + 0..7.  The weight
// rows (output columns) are stored permuted, so that the accumulator of output
// block mb = 2*ks + h holds columns 32*ks + 8g + 4h + e in lane (row, g): one
// product's output is already the next product's B operand, and each lane's
// outputs are 8 consecutive columns per k-step.
enum { TM_KEYS = 0, TM_VALUES = 1, TM_QUERY = 2 };

// n / d for n < 2^31 as (n * m) >> sh with m = ceil(2^sh / d), sh = 31 + ceil(log2 d):
// the rounding error of m adds less than 1/d to n/d, which never crosses an integer.
struct DivU31 {
  uint32_t d, m, sh;
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    return static_cast<uint32_t>((static_cast<uint64_t>(n) * m) >> sh);
  }
};
static DivU31 make_div(uint32_t d) {
  uint32_t l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  const uint64_t p = uint64_t(1) << (31 + l);
  return DivU31{d, static_cast<uint32_t>((p + d - 1) / d), 31 + l};
}

struct TileArgs {
  const void* x;
  int64_t n;
  DivU31 H, S;          // rows enumerate (batch, head, position)
  int64_t sb, sh, ss;   // element strides; unit stride along d
  int vec;              // row starts 16-byte aligned: vector loads
  const uint16_t *w1, *w2, *w3;  // keys: Pi, -, S_eff split; values: Pi split; queries: Pi split, S_eff f16
  const float *cent, *bounds;
  uint8_t *codes, *signs;
  uint16_t *rn, *vn;
  float *y_out, *proj_out;
  uint16_t* q_rot;
  float* q_proj;
  // output rows: row (b, h, s) of the input goes to (b * H + h) * ldo + off + s of the packed and
  // norm planes (a cache of ldo positions per (batch, head), filled from position off); ldo = 0
  // writes row (b, h, s) to (b * H + h) * S + s
  int64_t ldo, off;
};

// packed / norm plane row of input row gr (< 2^31); MAP = false: the kernel ignores ldo / off
template <bool MAP>
__device__ __forceinline__ int64_t out_row(const TileArgs& a, int64_t gr) {
  if (!MAP || a.ldo == 0) return gr;
  const uint32_t r32 = static_cast<uint32_t>(gr);
  const uint32_t bh = a.S.div(r32);
  return static_cast<int64_t>(bh) * a.ldo + a.off + (r32 - bh * a.S.d);
}

template <int D, int NW_ = 8>
struct RT {
  static constexpr int NW = NW_, NT = 64 * NW, R = 16 * NW;  // waves, threads, rows per round
  static constexpr int KS = D / 32, MB = D / 16, CH = D / 8;  // k-steps, output blocks, 16-byte chunks per row
};

// Weight plane in LDS: row p holds weight row perm_row(p); its 16-byte chunk c sits
// at chunk swz(p, c), so the 16 rows of an A fragment read fall in distinct banks.
__device__ __forceinline__ int perm_row(int p) {
  const int mb = p >> 4, i = p & 15;
  return 32 * (mb >> 1) + 8 * (i >> 2) + 4 * (mb & 1) + (i & 3);
}
template <int D>
__device__ __forceinline__ int swz(int p, int c) {
  return D == 128 ? (c ^ (p & 15)) : (c ^ ((p >> 1) & 7));
}
// Copy NP weight planes src[0 .. NP*D*D) (split (hi, lo) pairs: NP = 2) into dst0 (and
// dst1) in the permuted, swizzled layout with direct-to-LDS buffer loads: LDS chunk L of a
// plane (row p = L / (D/8), swizzled chunk L % (D/8)) receives source chunk swz(p, .) of
// weight row perm_row(p) (swz is an involution).  Every copy is in flight at once and
// holds no registers; the caller waits with wait_vm<0>() and a block barrier.
template <int D, int NT, int NP = 2>
__device__ __forceinline__ void load_planes(_Float16* dst0, _Float16* dst1, const uint16_t* src) {
  constexpr int CH = D * D / 8;  // 16-byte chunks per plane
  static_assert(CH % 64 == 0 && NT % 64 == 0, "whole 64-chunk rounds per wave");
  const uint64_t base = reinterpret_cast<uint64_t>(src);
  const i32x4 desc{static_cast<int>(static_cast<uint32_t>(base)), static_cast<int>(static_cast<uint32_t>(base >> 32) & 0xffffu),
                   NP * D * D * 2, 0x00020000};
  int t = static_cast<int>(threadIdx.x);
  asm volatile("" : "+v"(t));  // recomputed per call: hoisted offsets would hold VGPRs across the tile loop
  const int w0 = __builtin_amdgcn_readfirstlane(t & ~63);
#pragma unroll
  for (int pl = 0; pl < NP; ++pl)
#pragma unroll
    for (int i = 0; i < (CH + NT - 1) / NT; ++i) {
      if (CH % NT != 0 && i * NT + w0 >= CH) break;  // wave-uniform: the last round is partial
      const int L = i * NT + t, p = L / (D / 8);
      const int c = swz<D>(p, L % (D / 8));
      const uint32_t voff = static_cast<uint32_t>((pl * D * D + perm_row(p) * D + c * 8) * 2);
      dma16_cached(desc, lds_offset(pl ? dst1 : dst0) + (i * NT + w0) * 16, voff);
    }
}

// acc[mb] (output columns 32*(mb>>1) + 8g + 4*(mb&1) + e of row l16) = W . X^T for this
// wave's 16 rows; B fragments b_hi/b_lo in registers, A from the LDS planes (hi, lo).
// Passes hi.hi, + lo(W).hi(X) if W_LO, + hi(W).lo(X) if X_LO.
template <int D, bool W_LO, bool X_LO, bool DBUF = true>
__device__ __forceinline__ void row_gemm(const _Float16* __restrict__ wh, const _Float16* __restrict__ wl,
                                         const half8 (&b_hi)[D / 32], const half8 (&b_lo)[D / 32],
                                         float4v (&acc)[D / 16], int l16, int g) {
  using T = RT<D>;
#pragma unroll
  for (int mb = 0; mb < T::MB; ++mb) acc[mb] = float4v{0.f, 0.f, 0.f, 0.f};
  // groups of 4 output blocks x one k-step; the A fragments of group q + 1 are
  // read while the MFMAs of group q run (two register slots)
  constexpr int NG = T::KS * (T::MB / 4);
  half8 ah[DBUF ? 2 : 1][4], al[DBUF ? 2 : 1][W_LO ? 4 : 1];
  auto fetch = [&](int q, int slot) {
    const int ks = q / (T::MB / 4), m0 = (q % (T::MB / 4)) * 4;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int p = (m0 + u) * 16 + l16;
      const int o = p * D + swz<D>(p, ks * 4 + g) * 8;
      ah[slot][u] = *reinterpret_cast<const half8*>(wh + o);
      if constexpr (W_LO) al[slot][u] = *reinterpret_cast<const half8*>(wl + o);
    }
  };
  if constexpr (DBUF) fetch(0, 0);
#pragma unroll
  for (int q = 0; q < NG; ++q) {
    if constexpr (DBUF) {
      if (q + 1 < NG) fetch(q + 1, (q + 1) & 1);
    } else {
      fetch(q, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int ks = q / (T::MB / 4), m0 = (q % (T::MB / 4)) * 4, c = DBUF ? (q & 1) : 0;
    // passes outermost: consecutive MFMAs write different accumulators
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[m0 + u] = mfma16x16x32(ah[c][u], b_hi[ks], acc[m0 + u]);
    if constexpr (W_LO) {
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[m0 + u] = mfma16x16x32(al[c][u], b_hi[ks], acc[m0 + u]);
    }
    if constexpr (X_LO) {
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[m0 + u] = mfma16x16x32(ah[c][u], b_lo[ks], acc[m0 + u]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// value j (0..7) of k-step ks from an accumulator in the permuted layout
__device__ __forceinline__ float acc_at(const float4v* acc, int ks, int j) { return acc[2 * ks + (j >> 2)][j & 3]; }

// Quantiser table for 3-4 code bits: y -> bucket qbucket(y) = floor(clamp(120 y + 128, 0, 255)),
// a non-decreasing map (|y| <= 1.0625 stays inside the clamp), and entry k = (the boundary
// whose bucket is k, or +inf; the number of boundaries in lower buckets).  A boundary in a
// lower bucket than y lies below y and one in a higher bucket above it, so with at most one
// boundary per bucket, code = T[k] + (y > B[k]) is searchsorted-left exactly.  Entries of
// buckets holding two or more boundaries carry bit 31; the kernel then counts instead.
__device__ __forceinline__ uint32_t qbucket(float y) {
  return static_cast<uint32_t>(fminf(fmaxf(fmaf(y, 120.f, 128.f), 0.f), 255.f));
}

// searchsorted-left over the 2^BB - 1 sorted boundaries (quantize.py:334-337), times CS (the
// key path takes 4 x the code: the byte offset of its centroid in LDS).  TAB: the
// quantiser table; BB == 1: one compare; BB == 2: a two-level search (y > b1 decides the
// upper bit, then y against b2 or b0 the lower one: for sorted boundaries that is the count
// [y > b0] + [y > b1] + [y > b2]); BB >= 3 without the table: binary search of the LDS copy.
template <int BB, bool TAB, uint32_t CS = 1>
__device__ __forceinline__ uint32_t code_of(float y, const float (&br)[7], const float* bnd, const uint2* qt) {
  static_assert(CS == 1 || (BB <= 2 && !TAB), "scaled codes for 1-2 code bits");
  if constexpr (TAB) {
    const uint2 e = qt[qbucket(y)];
    return e.y + (y > __uint_as_float(e.x) ? 1u : 0u);
  } else if constexpr (BB == 1) {
    return br[0] < y ? CS : 0u;
  } else if constexpr (BB == 2) {
    const bool hi = br[1] < y;
    const bool lo = (hi ? br[2] : br[0]) < y;
    return (hi ? 2u * CS : 0u) + (lo ? CS : 0u);
  } else {
    uint32_t idx = 0;
#pragma unroll
    for (int step = 1 << (BB - 1); step; step >>= 1)
      if (bnd[idx + step - 1] < y) idx += step;
    return idx;
  }
}

// Waves per block; the weights sit in LDS (keys 128 KiB, values 64 KiB, queries 96 KiB), so
// a compute unit holds one block.  Values of bf16 / f16 rows fit 128 VGPRs with the weight
// fragments single-buffered: 16 waves (4 per SIMD) hide more latency than 8 (measured at 1M
// rows, bits 3: 101 vs 122 us).  The others need up to 256 VGPRs: 8 waves.
template <int MODE, int DT>
constexpr int row_waves() {
  return MODE == TM_VALUES && DT != TQ_F32 ? 16 : 8;
}

// LDS of one row-kernel block: the weight planes, each wave's output staging, centroids,
// boundaries and the quantiser table.  Kernels declare it as raw bytes (a union of the three
// modes' layouts in the fused append kernel).
template <int D, int MODE, int BB, int NW>
struct RowsSmem {
  static constexpr int KC = D * BB / 8;                                         // packed code bytes per row
  static constexpr int SC = D / 8;                                              // sign bytes per row
  static constexpr int NPL = MODE == TM_KEYS ? 4 : (MODE == TM_VALUES ? 2 : 3);  // weight planes resident at once
  static constexpr int STG = MODE == TM_QUERY ? 16 : 16 * (KC + (MODE == TM_KEYS ? SC : 0));  // wave staging bytes
  static constexpr bool QTAB = MODE != TM_QUERY && BB >= 3;  // quantiser table built (3-4 code bits)
  alignas(16) _Float16 wsm[NPL * D * D];
  alignas(16) uint8_t stg_all[NW * STG];
  alignas(16) float s_cent[MODE == TM_KEYS ? 16 : 1];
  alignas(16) float s_bnd[MODE == TM_QUERY ? 1 : 16];
  alignas(16) uint32_t s_qt[QTAB ? 512 : 2];  // (boundary bits, count) pairs
};

// One block of the row-owned kernels: block `block` of `nblocks` blocks that share the rows.
// MAP: outputs go to the rows out_row<true> names (a cache append); the plain form keeps the
// registers that mapping needs free for the tile loop.
template <int D, int DT, int MODE, int BB, int NW_, bool MAP>
__device__ __forceinline__ void rows_body(const TileArgs& a, RowsSmem<D, MODE, BB, NW_>& sm, int block,
                                          int nblocks) {
  using T = RT<D, NW_>;
  using SM = RowsSmem<D, MODE, BB, NW_>;
  constexpr bool DBUF = NW_ <= 8;  // weight fragments double-buffered
  constexpr int KS = T::KS, MB = T::MB, NW = T::NW;
  constexpr int KC = SM::KC, SC = SM::SC, NPL = SM::NPL, STG = SM::STG;
  constexpr bool QTAB = SM::QTAB;
  _Float16* const wsm = sm.wsm;
  uint8_t* const stg_all = sm.stg_all;
  float* const s_cent = sm.s_cent;
  float* const s_bnd = sm.s_bnd;
  uint2* const s_qt = reinterpret_cast<uint2*>(sm.s_qt);

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  uint8_t* const stg = stg_all + wave * STG;  // this wave's 16 packed rows: codes, then signs
  const int64_t ntiles = (a.n + 15) / 16;
  const int64_t nwaves = static_cast<int64_t>(nblocks) * NW;
  const int64_t gw = static_cast<int64_t>(block) * NW + wave;  // this wave's tiles: gw, gw + nwaves, ...
  float br[7] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};  // BB <= 2: the boundaries in registers
  if constexpr (MODE != TM_QUERY) {
    constexpr int NC = 1 << BB;
    // keys reconstruct with the f16-rounded centroids (compressors.py:120-122)
    if (tid < NC) {
      if constexpr (MODE == TM_KEYS) s_cent[tid] = static_cast<float>(static_cast<_Float16>(a.cent[tid]));
      if (tid < NC - 1) s_bnd[tid] = a.bounds[tid];
    }
    if constexpr (BB <= 2) {
#pragma unroll
      for (int j = 0; j < NC - 1; ++j) br[j] = a.bounds[j];
    }
    if constexpr (QTAB) {
      if (tid < 256) {
        uint32_t below = 0, inside = 0;
        float bk = __builtin_inff();
        for (int j = 0; j < NC - 1; ++j) {
          const float bj = a.bounds[j];
          const uint32_t kb = qbucket(bj);
          below += kb < static_cast<uint32_t>(tid) ? 1u : 0u;
          if (kb == static_cast<uint32_t>(tid)) {
            ++inside;
            bk = bj;
          }
        }
        s_qt[tid] = make_uint2(__float_as_uint(bk), below | (inside > 1 ? 0x80000000u : 0u));
      }
    }
  }
  // after the first block barrier: every bucket holds at most one boundary (wave-uniform)
  auto qtable_ok = [&]() {
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) bad |= (s_qt[QTAB ? 4 * lane + i : 0].y >> 31) != 0u;
    return !__any(bad);
  };
  _Float16* const P0 = wsm;
  _Float16* const P1 = wsm + D * D;
  _Float16* const P2 = wsm + (NPL > 2 ? 2 : 0) * D * D;
  _Float16* const P3 = wsm + (NPL > 3 ? 3 : 0) * D * D;

  // ---- this lane's row of tile t and its elements k = 32*ks + 8g + 0..7, fetched raw
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  constexpr int RW = DT == TQ_F32 ? 2 : 1;  // 16-byte pieces per k-step
  struct Raw {
    u32x4 v[KS][RW];
  };
  Raw raw, nxt;  // this tile's row and the next one, in flight
  auto fetch_row = [&](int64_t t, Raw& raw) {
    const int64_t gr = t * 16 + l16;
    if (t >= ntiles || gr >= a.n) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int q = 0; q < RW; ++q) raw.v[ks][q] = u32x4{0u, 0u, 0u, 0u};
      return;
    }
    const uint32_t r32 = static_cast<uint32_t>(gr);
    const uint32_t bh = a.S.div(r32), s = r32 - bh * a.S.d;
    const uint32_t bb = a.H.div(bh), h = bh - bb * a.H.d;
    const int64_t off = static_cast<int64_t>(bb) * a.sb + static_cast<int64_t>(h) * a.sh +
                        static_cast<int64_t>(s) * a.ss + 8 * g;
    constexpr int ES = DT == TQ_F32 ? 4 : 2;
    const uint8_t* base = static_cast<const uint8_t*>(a.x) + off * ES;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int q = 0; q < RW; ++q) {
        const uint8_t* p = base + (32 * ks) * ES + 16 * q;
        if (a.vec) {
          raw.v[ks][q] = *reinterpret_cast<const u32x4*>(p);
        } else {
          u32x4 v;
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            uint32_t x = 0;
            if constexpr (ES == 4) x = *reinterpret_cast<const uint32_t*>(p + 4 * w);
            else x = static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(p + 4 * w)) |
                     (static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(p + 4 * w + 2)) << 16);
            v[w] = x;
          }
          raw.v[ks][q] = v;
        }
      }
  };
  auto unpack_row = [&](const Raw& raw, float (&xv)[KS][8]) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if constexpr (DT == TQ_F32) {
          xv[ks][j] = __uint_as_float(raw.v[ks][j >> 2][j & 3]);
        } else {
          const uint32_t w = raw.v[ks][0][j >> 1];
          const uint16_t h = static_cast<uint16_t>((j & 1) ? (w >> 16) : (w & 0xffffu));
          xv[ks][j] = DT == TQ_F16 ? h2f(h) : bf16_to_f32(h);
        }
      }
  };
  half8 bh[KS], bl[KS];
  float4v acc[MB];
  float xv[KS][8];
  // sum / max over the 4 lanes of a row (lanes l16, l16+16, l16+32, l16+48), on the VALU:
  // v_permlane16_swap / v_permlane32_swap of a value with itself leave, in every lane, the
  // lane's own value in one result and its partner's (lane ^ 16, lane ^ 32) in the other
  auto xor_pair = [](float v, auto half) {
    const uint32_t u = __float_as_uint(v);
    const auto r = decltype(half)::value == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                                               : __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return float2v{__uint_as_float(r[0]), __uint_as_float(r[1])};
  };
  auto row_sum = [&](float v) {
    float2v p = xor_pair(v, std::integral_constant<int, 16>{});
    p = xor_pair(p[0] + p[1], std::integral_constant<int, 32>{});
    return p[0] + p[1];
  };
  auto row_max = [&](float v) {
    float2v p = xor_pair(v, std::integral_constant<int, 16>{});
    p = xor_pair(fmaxf(p[0], p[1]), std::integral_constant<int, 32>{});
    return fmaxf(p[0], p[1]);
  };
  auto split_row = [&](const float (&v)[KS][8], float sc, half8 (&hi)[KS], half8 (&lo)[KS]) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        _Float16 h, l;
        split_f16(v[ks][j] * sc, h, l);
        hi[ks][j] = h;
        lo[ks][j] = l;
      }
  };
  // wave-private staging is written and read by this wave only: order it within the wave
  auto wave_sync = [&]() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  // copy `bytes`-byte rows of this wave's 16 staged rows at `src` to their output rows (one
  // contiguous run when the output rows are the input rows)
  auto store_rows = [&](const uint8_t* src, uint8_t* out, int64_t row0, int bytes) {
    const int64_t nr = a.n - row0 < 16 ? a.n - row0 : 16;
    const int nd = static_cast<int>(nr) * bytes / 4;
    if (!MAP || a.ldo == 0) {
      uint32_t* dst = reinterpret_cast<uint32_t*>(out + row0 * bytes);
      for (int i = lane; i < nd; i += 64) dst[i] = reinterpret_cast<const uint32_t*>(src)[i];
    } else {
      const int wpr = bytes / 4;  // dwords per row (rows of d * b / 8 bytes, d = 64 or 128)
      for (int i = lane; i < nd; i += 64) {
        const int r = i / wpr;
        reinterpret_cast<uint32_t*>(out + out_row<MAP>(a, row0 + r) * bytes)[i - r * wpr] =
            reinterpret_cast<const uint32_t*>(src)[i];
      }
    }
  };
  // y = acc * ysc -> codes of this lane's 8 columns of k-step ks, staged at the row's packed
  // position; each(ks, j, acc value, code) sees every element
  auto quantize_ks = [&](auto tab, const float4v (&acc)[MB], float ysc, int64_t gr, int ks, auto&& each) {
    constexpr bool TAB = decltype(tab)::value;
    // keys with 1-2 code bits: codes come as 4 c, their centroid's byte offset in LDS
    constexpr uint32_t CSC = (MODE == TM_KEYS && BB <= 2 && !TAB) ? 4u : 1u;
    float4v y0, y1;
    uint32_t v = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float av = acc_at(acc, ks, j);
      const float y = av * ysc;
      if (j < 4) y0[j] = y;
      else y1[j - 4] = y;
      const uint32_t c = code_of<BB, TAB, CSC>(y, br, s_bnd, s_qt);
      v |= c << (BB * j);
      each(ks, j, av, c);
    }
    if constexpr (CSC == 4) v >>= 2;
    if (a.y_out && gr < a.n) {
      float4v* yo = reinterpret_cast<float4v*>(a.y_out + gr * D + 32 * ks + 8 * g);
      yo[0] = y0;
      yo[1] = y1;
    }
    uint8_t* dst = stg + l16 * KC + (32 * ks + 8 * g) * BB / 8;
    if constexpr (BB == 2) {
      *reinterpret_cast<uint16_t*>(dst) = static_cast<uint16_t>(v);
    } else if constexpr (BB == 4) {
      *reinterpret_cast<uint32_t*>(dst) = v;
    } else {
#pragma unroll
      for (int k = 0; k < BB; ++k) dst[k] = static_cast<uint8_t>(v >> (8 * k));
    }
  };
  auto quantize_stage = [&](auto tab, const float4v (&acc)[MB], float ysc, int64_t gr, auto&& each) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) quantize_ks(tab, acc, ysc, gr, ks, each);
  };
  // ---- vn = ||x|| and y-side product x Pi^T of this lane's row (compressors.py:108-112,
  // :274-276).  bf16 / f16 rows are exact in f16 under a power-of-two row scale 2^(15 - e)
  // (vn < 2^e; elements below ~2^-32 vn round), so x Pi^T takes the weight's hi and lo parts
  // against one x operand: 2 MFMA passes; f32 rows are split into hi + lo under 2^(10 - e):
  // 3 passes.  On return acc * xs = x Pi^T, and y = x Pi^T / (vn + 1e-8) = acc * (xs / den).
  constexpr bool XEXACT = DT != TQ_F32;
  constexpr int SX = XEXACT ? 15 : 10;
  auto front = [&](float& vn, int& e2, float& xs) {
    float ss = 0.f;
    if constexpr (XEXACT) {
      // squares of the 16-bit pairs straight from the raw words (products exact in f32)
      typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
      typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t u = raw.v[ks][0][w];
          if constexpr (DT == TQ_BF16) {
            const bf16x2 p = __builtin_bit_cast(bf16x2, u);
            ss = __builtin_amdgcn_fdot2_f32_bf16(p, p, ss, false);
          } else {
            const f16x2 p = __builtin_bit_cast(f16x2, u);
            ss = __builtin_amdgcn_fdot2(p, p, ss, false);
          }
        }
    } else {
      unpack_row(raw, xv);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = fmaf(xv[ks][j], xv[ks][j], ss);
    }
    vn = sqrtf(row_sum(ss));
    frexpf(vn, &e2);
    e2 = e2 < -100 ? -100 : e2;  // tiny rows: the scale stays finite
    const float sc = ldexpf(1.f, SX - e2);
    if constexpr (XEXACT) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t w = raw.v[ks][0][j >> 1];
          const uint16_t h = static_cast<uint16_t>((j & 1) ? (w >> 16) : (w & 0xffffu));
          const float x = DT == TQ_F16 ? h2f(h) : bf16_to_f32(h);
          bh[ks][j] = static_cast<_Float16>(x * sc);
        }
    } else {
      split_row(xv, sc, bh, bl);
    }
    row_gemm<D, true, !XEXACT, DBUF>(P0, P1, bh, bl, acc, l16, g);
    xs = ldexpf(1.f / kSplit, e2 - SX);
  };


  if constexpr (MODE == TM_QUERY) {
    load_planes<D, T::NT>(P0, P1, a.w1);
    load_planes<D, T::NT, 1>(P2, P2, a.w2);
    fetch_row(gw, raw);
    wait_vm<0>();
    wait_vm0_visible();  // the row fetched above counts as arrived inside the tile loop
    __syncthreads();
    for (int64_t t = gw; t < ntiles; t += nwaves) {
      unpack_row(raw, xv);
      fetch_row(t + nwaves, nxt);  // next tile's row, in flight during the products
      // per-row power-of-two scale so the split parts stay in range (|q| * scale < kSplit)
      float mx = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(xv[ks][j]));
      int e2;
      frexpf(row_max(mx), &e2);
      split_row(xv, ldexpf(kSplit, -e2), bh, bl);
      // q_rot = f16(q Pi^T)   (compressors.py:186)
      row_gemm<D, true, true>(P0, P1, bh, bl, acc, l16, g);
      // the tile's outputs go through range-checked buffer stores (lanes of rows past n are
      // dropped by the hardware): no branch around them, so the compiler's wait for the next
      // row at the end of the tile counts them instead of waiting for them
      const uint32_t nrows = static_cast<uint32_t>(a.n - t * 16 < 16 ? a.n - t * 16 : 16);
      const rsrc_t rq = make_rsrc(a.q_rot + t * 16 * D, nrows * D * 2);
      const rsrc_t rp = make_rsrc(a.q_proj + t * 16 * D, nrows * D * 4);
      const float inv = ldexpf(kUnsplit2, e2);
      mx = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          bh[ks][j] = static_cast<_Float16>(acc_at(acc, ks, j) * inv);
          mx = fmaxf(mx, fabsf(static_cast<float>(bh[ks][j])));
        }
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, bh[ks]), rq, (l16 * D + 32 * ks + 8 * g) * 2, 0, 0);
      }
      // q_rot holds f16 values: scaling by 2^(12-e) keeps them exact in f16
      frexpf(row_max(mx), &e2);
      const float sc2 = ldexpf(4096.f, -e2), inv2 = ldexpf(1.f / 4096.f, e2);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int j = 0; j < 8; ++j) bh[ks][j] = static_cast<_Float16>(static_cast<float>(bh[ks][j]) * sc2);
      // q_proj = q_rot S_eff^T in f32: f32 accumulation of exact f16 products, as the
      // reference's fp32 projection (kernels/attention.py:158-167, :453)
      row_gemm<D, false, false>(P2, P2, bh, bl, acc, l16, g);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        float4v o0, o1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          o0[j] = acc_at(acc, ks, j) * inv2;
          o1[j] = acc_at(acc, ks, j + 4) * inv2;
        }
        const uint32_t off = (l16 * D + 32 * ks + 8 * g) * 4;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o0), rp, off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o1), rp, off + 16, 0, 0);
      }
      raw = nxt;
    }
  } else if constexpr (MODE == TM_VALUES) {
    load_planes<D, T::NT>(P0, P1, a.w1);
    fetch_row(gw, raw);
    wait_vm<0>();
    wait_vm0_visible();  // the row fetched above counts as arrived inside the tile loop
    __syncthreads();
    auto tiles = [&](auto tab) {
      // a tile's outputs leave at the start of the next one (see the key path)
      int64_t tp = -1;
      float vn_p = 0.f;
      auto flush = [&]() {
        const int64_t grp = tp * 16 + l16;
        if (g == 0 && grp < a.n) a.vn[out_row<MAP>(a, grp)] = f2h(vn_p);
        wave_sync();
        store_rows(stg, a.codes, tp * 16, KC);
        wave_sync();
      };
      for (int64_t t = gw; t < ntiles; t += nwaves) {
        const int64_t gr = t * 16 + l16;
        fetch_row(t + nwaves, nxt);  // next tile's row, in flight during the product
        if (tp >= 0) flush();
        // ---- vn = ||x||; y = (x / (vn + 1e-8)) Pi^T; codes = searchsorted-left, packed LSB
        // first   (compressors.py:274-287)
        float vn, xs;
        int e2;
        front(vn, e2, xs);
        // the quantiser at raised priority, as in the key path (1M rows, bits 3: 103.9 vs 107.0 us)
        __builtin_amdgcn_s_setprio(1);
        quantize_stage(tab, acc, xs / (vn + 1e-8f), gr, [](int, int, float, uint32_t) {});
        __builtin_amdgcn_s_setprio(0);
        tp = t;
        vn_p = vn;
        raw = nxt;
      }
      if (tp >= 0) flush();
    };
    if constexpr (QTAB) {
      if (qtable_ok()) tiles(std::true_type{});
      else tiles(std::false_type{});
    } else {
      tiles(std::false_type{});
    }
  } else {
    // keys, one pass per tile: P0/P1 hold Pi, P2/P3 S_eff = S Pi^T (both split), resident for
    // the whole block.  The residual stays in the rotated domain:
    //   u = r Pi^T = x Pi^T - vn f16(C)[c],  rn = ||r|| = ||u||,  proj = r S^T = u S_eff^T
    // (compressors.py:120-130 form r = x - (yhat Pi) vn in the original domain: the same values
    // up to f32 rounding, without the yhat Pi product)
    load_planes<D, T::NT>(P0, P1, a.w1);
    load_planes<D, T::NT>(P2, P3, a.w3);
    fetch_row(gw, raw);
    wait_vm<0>();
    wait_vm0_visible();  // the row fetched above counts as arrived inside the tile loop
    __syncthreads();
    auto tiles = [&](auto tab) {
      // A tile's outputs (staged codes and signs, vn, rn) leave at the start of the next tile,
      // after its row fetch: the wait for that fetch at the end of the tile (vmcnt counts
      // stores too, in issue order) then finds the stores long complete instead of waiting
      // for the ones just issued.
      int64_t tp = -1;
      float vn_p = 0.f, rn_p = 0.f;
      auto flush = [&]() {
        const int64_t grp = tp * 16 + l16;
        if (g == 0 && grp < a.n) {
          const int64_t orow = out_row<MAP>(a, grp);
          a.vn[orow] = f2h(vn_p);
          a.rn[orow] = f2h(rn_p);
        }
        wave_sync();
        store_rows(stg, a.codes, tp * 16, KC);
        store_rows(stg + 16 * KC, a.signs, tp * 16, SC);
        wave_sync();
      };
      for (int64_t t = gw; t < ntiles; t += nwaves) {
        const int64_t gr = t * 16 + l16;
        fetch_row(t + nwaves, nxt);  // next tile's row, in flight during the products
        if (tp >= 0) flush();
        // ---- vn = ||x||; y = (x / (vn + 1e-8)) Pi^T; codes   (compressors.py:108-116)
        float vn, xs;
        int e2;
        front(vn, e2, xs);
        // ---- u = x Pi^T - vn f16(C)[c], carried as w = u / xs = acc - (vn / xs) f16(C)[c]
        // (xs a power of two, so u = w xs and rn = ||u|| = ||w|| xs exactly)
        const float vnw = ldexpf(vn, SX + 10 - e2);
        // |u| <= ||x|| + ||k_mse|| < 2^(e + 1): u * 2^(10 - e) = w * 2^-SX keeps both split
        // parts in range; each w is split as it is formed
        // the quantiser / residual stretch is VALU work: at raised priority it takes the SIMD
        // while the block's other wave on it runs its MFMA passes (measured at 1M rows, bits 3:
        // 201.6 vs 209.2 us median)
        __builtin_amdgcn_s_setprio(1);
        float ss = 0.f;
        float w_even = 0.f;
        uint32_t wh[KS][4], wl[KS][4];
        quantize_stage(tab, acc, xs / (vn + 1e-8f), gr, [&](int ks, int j, float av, uint32_t c) {
          // f16-rounded centroid of the code (1-2 code bits: c arrives as its byte offset)
          const float cc = BB <= 2 ? *reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(s_cent) + c)
                                   : s_cent[c];
          const float w = fmaf(-vnw, cc, av);
          ss = fmaf(w, w, ss);
          // split as (even, odd) pairs: the next product's B operand dwords
          if (j & 1) split_f16x2_scaled(w_even, w, 1.f / (1 << SX), wh[ks][j >> 1], wl[ks][j >> 1]);
          else w_even = w;
        });
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          bh[ks] = __builtin_bit_cast(half8, u32x4{wh[ks][0], wh[ks][1], wh[ks][2], wh[ks][3]});
          bl[ks] = __builtin_bit_cast(half8, u32x4{wl[ks][0], wl[ks][1], wl[ks][2], wl[ks][3]});
        }
        const float rn = sqrtf(row_sum(ss)) * xs;
        __builtin_amdgcn_s_setprio(0);
        // ---- proj = u S_eff^T; signs = (proj >= 0)   (compressors.py:128-130).  Read off the
        // accumulator's sign bits: the scale to proj is positive, and an accumulator started at
        // +0 never ends at -0
        row_gemm<D, true, true>(P2, P3, bh, bl, acc, l16, g);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          uint32_t neg = 0;  // bit j = sign of value j: v_alignbit shifts one sign bit in per value
#pragma unroll
          for (int j = 7; j >= 0; --j) neg = __builtin_amdgcn_alignbit(neg, __float_as_uint(acc_at(acc, ks, j)), 31);
          stg[16 * KC + l16 * SC + 4 * ks + g] = static_cast<uint8_t>(~neg);
        }
        if (a.proj_out && gr < a.n) {
          const float inv = ldexpf(kUnsplit2, e2);
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            float4v p0, p1;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              p0[j] = acc_at(acc, ks, j) * inv;
              p1[j] = acc_at(acc, ks, j + 4) * inv;
            }
            float4v* po = reinterpret_cast<float4v*>(a.proj_out + gr * D + 32 * ks + 8 * g);
            po[0] = p0;
            po[1] = p1;
          }
        }
        tp = t;
        vn_p = vn;
        rn_p = rn;
        raw = nxt;
      }
      if (tp >= 0) flush();
    };
    if constexpr (QTAB) {
      if (qtable_ok()) tiles(std::true_type{});
      else tiles(std::false_type{});
    } else {
      tiles(std::false_type{});
    }
    wait_vm<0>();  // no plane copy outlives the block, even with no tile to process
  }
}

template <int D, int DT, int MODE, int BB>
__global__ void __launch_bounds__((64 * row_waves<MODE, DT>())) rows_kernel(TileArgs a) {
  using SM = RowsSmem<D, MODE, BB, row_waves<MODE, DT>()>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[sizeof(SM)];
  rows_body<D, DT, MODE, BB, row_waves<MODE, DT>(), false>(a, *reinterpret_cast<SM*>(smem), blockIdx.x, gridDim.x);
}

// Few rows (a decode step's queries): blocks of 4 waves, one per SIMD, so that the rows'
// 16-row tiles spread over more compute units instead of pairing up on the SIMDs of a few
// 8-wave blocks
constexpr int kFewWaves = 4;
template <int D, int DT, int MODE, int BB>
__global__ void __launch_bounds__(64 * kFewWaves) rows_few_kernel(TileArgs a) {
  using SM = RowsSmem<D, MODE, BB, kFewWaves>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[sizeof(SM)];
  rows_body<D, DT, MODE, BB, kFewWaves, false>(a, *reinterpret_cast<SM*>(smem), blockIdx.x, gridDim.x);
}

// A cache append in one launch: blocks [0, nbk) compress the new keys, [nbk, nbk + nbv) the
// new values, the rest prepare the new queries (nbq blocks, 0 without queries).  Every block
// has 4 waves (one per SIMD: a step's few tiles spread over compute units); the LDS holds one
// mode's layout at a time.
constexpr int kAppendWaves = 4;
template <int D, int DT, int KBB, int VB>
__global__ void __launch_bounds__(64 * kAppendWaves) append_kernel(TileArgs ka, TileArgs va, TileArgs qa, int nbk,
                                                                   int nbv, int nbq) {
  constexpr int NW = kAppendWaves;
  using SK = RowsSmem<D, TM_KEYS, KBB, NW>;
  using SV = RowsSmem<D, TM_VALUES, VB, NW>;
  using SQ = RowsSmem<D, TM_QUERY, 1, NW>;
  constexpr size_t BYTES = sizeof(SK) > sizeof(SV) ? (sizeof(SK) > sizeof(SQ) ? sizeof(SK) : sizeof(SQ))
                                                   : (sizeof(SV) > sizeof(SQ) ? sizeof(SV) : sizeof(SQ));
  __shared__ __attribute__((aligned(16))) uint8_t smem[BYTES];
  const int blk = static_cast<int>(blockIdx.x);
  if (blk < nbk) rows_body<D, DT, TM_KEYS, KBB, NW, true>(ka, *reinterpret_cast<SK*>(smem), blk, nbk);
  else if (blk < nbk + nbv) rows_body<D, DT, TM_VALUES, VB, NW, true>(va, *reinterpret_cast<SV*>(smem), blk - nbk, nbv);
  else rows_body<D, DT, TM_QUERY, 1, NW, false>(qa, *reinterpret_cast<SQ*>(smem), blk - nbk - nbv, nbq);
}

// Blocks of `kernel` the device holds at once (occupancy x compute units), per device.
template <int D, int DT, int MODE, int BB>
static void launch_tile(const TileArgs& a, hipStream_t s) {
  static int cache[16] = {};
  using T = RT<D, row_waves<MODE, DT>()>;
  if constexpr (MODE == TM_QUERY) {
    static int cache_few[16] = {};
    const int64_t blocks = (a.n + 16 * kFewWaves - 1) / (16 * kFewWaves);  // one tile per wave
    const int64_t res = resident_blocks(reinterpret_cast<const void*>(&rows_few_kernel<D, DT, MODE, BB>),
                                        64 * kFewWaves, cache_few);
    if (blocks > 1 && blocks <= res) {  // all resident at once, one tile per SIMD
      rows_few_kernel<D, DT, MODE, BB><<<static_cast<unsigned>(blocks), 64 * kFewWaves, 0, s>>>(a);
      return;
    }
  }
  const int64_t blocks = (a.n + T::R - 1) / T::R;  // one 16-row tile per wave
  const int64_t res = resident_blocks(reinterpret_cast<const void*>(&rows_kernel<D, DT, MODE, BB>), T::NT, cache);
  const unsigned grid = static_cast<unsigned>(blocks < res ? blocks : res);
  rows_kernel<D, DT, MODE, BB><<<grid, T::NT, 0, s>>>(a);
}

template <int D, int MODE, int BB>
static void launch_tile_dt(const TileArgs& a, int dtype, hipStream_t s) {
  if (dtype == TQ_F32) launch_tile<D, TQ_F32, MODE, BB>(a, s);
  else if (dtype == TQ_F16) launch_tile<D, TQ_F16, MODE, BB>(a, s);
  else launch_tile<D, TQ_BF16, MODE, BB>(a, s);
}

// The row-owned kernels take head_dim 64 / 128, 1-4 code bits and fewer than
// 2^31 rows; packed outputs must be dword aligned.
static bool tile_applies(int d, int64_t n, int b) {
  return (d == 64 || d == 128) && b >= 1 && b <= 4 && n < (int64_t(1) << 31);
}
// 16-byte vector loads need every row start 16-byte aligned
static int tile_vec(const void* x, int dtype, int64_t sb, int64_t sh, int64_t ss) {
  const int64_t es = dtype == TQ_F32 ? 4 : 2;
  return (reinterpret_cast<uintptr_t>(x) % 16 == 0) && (sb * es) % 16 == 0 && (sh * es) % 16 == 0 &&
         (ss * es) % 16 == 0;
}

template <int MODE>
static void dispatch_tile(const TileArgs& a, int d, int dtype, int b, hipStream_t s) {
  switch (d * 8 + b) {
    case 64 * 8 + 1: launch_tile_dt<64, MODE, 1>(a, dtype, s); break;
    case 64 * 8 + 2: launch_tile_dt<64, MODE, 2>(a, dtype, s); break;
    case 64 * 8 + 3: launch_tile_dt<64, MODE, 3>(a, dtype, s); break;
    case 64 * 8 + 4: launch_tile_dt<64, MODE, 4>(a, dtype, s); break;
    case 128 * 8 + 1: launch_tile_dt<128, MODE, 1>(a, dtype, s); break;
    case 128 * 8 + 2: launch_tile_dt<128, MODE, 2>(a, dtype, s); break;
    case 128 * 8 + 3: launch_tile_dt<128, MODE, 3>(a, dtype, s); break;
    default: launch_tile_dt<128, MODE, 4>(a, dtype, s); break;
  }
}
template <>
void dispatch_tile<TM_QUERY>(const TileArgs& a, int d, int dtype, int, hipStream_t s) {
  if (d == 64) launch_tile_dt<64, TM_QUERY, 1>(a, dtype, s);
  else launch_tile_dt<128, TM_QUERY, 1>(a, dtype, s);
}

// ---------------------------------------------------------------- cache append (one launch)
template <int D, int DT, int KBB, int VB>
static void launch_append(const TileArgs& ka, const TileArgs& va, const TileArgs& qa, hipStream_t s) {
  static int cache[16] = {};
  constexpr int NT = 64 * kAppendWaves, RROWS = 16 * kAppendWaves;
  const int64_t res = resident_blocks(reinterpret_cast<const void*>(&append_kernel<D, DT, KBB, VB>), NT, cache);
  // a block takes rounds of RROWS rows; when the three modes need more blocks than the device
  // holds at once, they share the resident blocks by work (a key row costs about two value or
  // query rows)
  auto rounds = [](int64_t n) { return (n + RROWS - 1) / RROWS; };
  int64_t nk = rounds(ka.n), nv = rounds(va.n), nq = rounds(qa.n);
  if (nk + nv + nq > res) {
    const double wk = 2.0 * static_cast<double>(ka.n), wv = static_cast<double>(va.n);
    const double wq = static_cast<double>(qa.n), w = wk + wv + wq;
    nk = std::max<int64_t>(1, std::min<int64_t>(nk, static_cast<int64_t>(res * wk / w)));
    nv = std::max<int64_t>(1, std::min<int64_t>(nv, static_cast<int64_t>(res * wv / w)));
    nq = qa.n > 0 ? std::max<int64_t>(1, std::min<int64_t>(nq, res - nk - nv)) : 0;
  }
  append_kernel<D, DT, KBB, VB><<<static_cast<unsigned>(nk + nv + nq), NT, 0, s>>>(
      ka, va, qa, static_cast<int>(nk), static_cast<int>(nv), static_cast<int>(nq));
}

template <int D, int KBB, int VB>
static void launch_append_dt(const TileArgs& ka, const TileArgs& va, const TileArgs& qa, int dtype, hipStream_t s) {
  if (dtype == TQ_F32) launch_append<D, TQ_F32, KBB, VB>(ka, va, qa, s);
  else if (dtype == TQ_F16) launch_append<D, TQ_F16, KBB, VB>(ka, va, qa, s);
  else launch_append<D, TQ_BF16, KBB, VB>(ka, va, qa, s);
}

// head_dim 64 / 128, value bits 2-4 with key code bits one fewer (a compressor pair of one bit width)
static void dispatch_append(const TileArgs& ka, const TileArgs& va, const TileArgs& qa, int d, int dtype, int vb,
                            hipStream_t s) {
  switch (d * 8 + vb) {
    case 64 * 8 + 2: launch_append_dt<64, 1, 2>(ka, va, qa, dtype, s); break;
    case 64 * 8 + 3: launch_append_dt<64, 2, 3>(ka, va, qa, dtype, s); break;
    case 64 * 8 + 4: launch_append_dt<64, 3, 4>(ka, va, qa, dtype, s); break;
    case 128 * 8 + 2: launch_append_dt<128, 1, 2>(ka, va, qa, dtype, s); break;
    case 128 * 8 + 3: launch_append_dt<128, 2, 3>(ka, va, qa, dtype, s); break;
    default: launch_append_dt<128, 3, 4>(ka, va, qa, dtype, s); break;
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

// The tile kernel for head dim d: D = d rounded up to a multiple of 32.
#define TQ_CASE_D(FN, DD, dt, ...)                                                \
  case DD:                                                                        \
    if ((dt) == TQ_F32) FN<DD, TQ_F32>(__VA_ARGS__);                              \
    else if ((dt) == TQ_F16) FN<DD, TQ_F16>(__VA_ARGS__);                         \
    else FN<DD, TQ_BF16>(__VA_ARGS__);                                            \
    break;
#define TQ_SWITCH_DD(FN, d, dt, ...)                                              \
  switch (pad_dim(d)) {                                                           \
    TQ_CASE_D(FN, 32, dt, __VA_ARGS__)                                            \
    TQ_CASE_D(FN, 64, dt, __VA_ARGS__)                                            \
    TQ_CASE_D(FN, 96, dt, __VA_ARGS__)                                            \
    TQ_CASE_D(FN, 128, dt, __VA_ARGS__)                                           \
    TQ_CASE_D(FN, 160, dt, __VA_ARGS__)                                           \
    TQ_CASE_D(FN, 192, dt, __VA_ARGS__)                                           \
    TQ_CASE_D(FN, 224, dt, __VA_ARGS__)                                           \
    TQ_CASE_D(FN, 256, dt, __VA_ARGS__)                                           \
    default: break;                                                               \
  }

}  // namespace tq

using namespace tq;

#define TQ_CHECK_DD(what, d, dtype)                                                              \
  do {                                                                                           \
    if (!supported_dim(d)) {                                                                     \
      set_error("%s: head_dim %d not supported (multiples of 8 from 8 to 256)", what, (int)(d));  \
      return TQ_EUNSUPPORTED;                                                                    \
    }                                                                                            \
    TQ_REQUIRE((dtype) == TQ_F32 || (dtype) == TQ_F16 || (dtype) == TQ_BF16,                     \
               "%s: unknown dtype %d", what, (int)(dtype));                                     \
  } while (0)

extern "C" {

int tq_compress_keys(const void* x, int32_t dtype, int32_t B, int32_t H, int32_t S, int32_t d,
                     int64_t sxb, int64_t sxh, int64_t sxs, const uint16_t* pi_split, const uint16_t* seff_split,
                     const float* centroids, const float* bounds, int32_t b_eff, uint8_t* codes,
                     uint8_t* signs, uint16_t* rn, uint16_t* vn, float* y_out, float* proj_out,
                     void* stream) {
  TQ_CHECK_DD("tq_compress_keys", d, dtype);
  TQ_REQUIRE(b_eff >= 1 && b_eff <= 8, "tq_compress_keys: b_eff must be in [1, 8], got %d", b_eff);
  TQ_REQUIRE(B >= 0 && H >= 0 && S >= 0, "tq_compress_keys: bad shape");
  const int64_t n = static_cast<int64_t>(B) * H * S;
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(x && pi_split && seff_split && centroids && bounds && codes && signs && rn && vn,
             "tq_compress_keys: null pointer");
  if (tile_applies(d, n, b_eff) && reinterpret_cast<uintptr_t>(codes) % 4 == 0 &&
      reinterpret_cast<uintptr_t>(signs) % 4 == 0) {
    TileArgs t{};
    t.x = x; t.n = n; t.H = make_div(static_cast<uint32_t>(H)); t.S = make_div(static_cast<uint32_t>(S));
    t.sb = sxb; t.sh = sxh; t.ss = sxs; t.vec = tile_vec(x, dtype, sxb, sxh, sxs);
    t.w1 = pi_split; t.w3 = seff_split;
    t.cent = centroids; t.bounds = bounds;
    t.codes = codes; t.signs = signs; t.rn = rn; t.vn = vn; t.y_out = y_out; t.proj_out = proj_out;
    dispatch_tile<TM_KEYS>(t, d, dtype, b_eff, as_stream(stream));
    return launch_status("tq_compress_keys");
  }
  KeyArgs a{x, n, Rows4{H, S, sxb, sxh, sxs}, pi_split, seff_split, centroids, bounds, b_eff, codes, signs, rn, vn,
            y_out, proj_out, d, S, 0, 0};
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
  if (tile_applies(d, n, b) && reinterpret_cast<uintptr_t>(codes) % 4 == 0) {
    TileArgs t{};
    t.x = x; t.n = n; t.H = make_div(static_cast<uint32_t>(H)); t.S = make_div(static_cast<uint32_t>(S));
    t.sb = sxb; t.sh = sxh; t.ss = sxs; t.vec = tile_vec(x, dtype, sxb, sxh, sxs);
    t.w1 = pi_split; t.bounds = bounds;
    t.codes = codes; t.vn = vn; t.y_out = y_out;
    dispatch_tile<TM_VALUES>(t, d, dtype, b, as_stream(stream));
    return launch_status("tq_compress_values");
  }
  ValArgs a{x, n, Rows4{H, S, sxb, sxh, sxs}, pi_split, bounds, b, codes, vn, y_out, d, S, 0, 0};
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
  DecArgs a{codes, vn, n, pit_split, centroids, b, out, ld_out, d};
  TQ_SWITCH_DD(launch_decomp, d, out_dtype, a, n, as_stream(stream));
  return launch_status("tq_decompress_values");
}

int tq_query_prep(const void* q, int32_t dtype, int32_t B, int32_t Hq, int32_t Sq, int32_t d,
                  int64_t sqb, int64_t sqh, int64_t sqs, const uint16_t* pi_split,
                  const uint16_t* s_eff_f16, uint16_t* q_rot, float* q_proj, void* stream) {
  TQ_CHECK_DD("tq_query_prep", d, dtype);
  TQ_REQUIRE(B >= 0 && Hq >= 0 && Sq >= 0, "tq_query_prep: bad shape");
  const int64_t n = static_cast<int64_t>(B) * Hq * Sq;
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(q && pi_split && s_eff_f16 && q_rot && q_proj, "tq_query_prep: null pointer");
  if (tile_applies(d, n, 1) && reinterpret_cast<uintptr_t>(q_rot) % 8 == 0 &&
      reinterpret_cast<uintptr_t>(q_proj) % 16 == 0) {
    TileArgs t{};
    t.x = q; t.n = n; t.H = make_div(static_cast<uint32_t>(Hq)); t.S = make_div(static_cast<uint32_t>(Sq));
    t.sb = sqb; t.sh = sqh; t.ss = sqs; t.vec = tile_vec(q, dtype, sqb, sqh, sqs);
    t.w1 = pi_split; t.w2 = s_eff_f16; t.q_rot = q_rot; t.q_proj = q_proj;
    dispatch_tile<TM_QUERY>(t, d, dtype, 1, as_stream(stream));
    return launch_status("tq_query_prep");
  }
  PrepArgs a{q, B, Hq, Sq, sqb, sqh, sqs, pi_split, s_eff_f16, q_rot, q_proj, d};
  TQ_SWITCH_DD(launch_prep, d, dtype, a, n, as_stream(stream));
  return launch_status("tq_query_prep");
}

int tq_cache_append(const void* k, const void* v, int32_t dtype, int32_t B, int32_t H, int32_t S, int32_t d,
                    int64_t skb, int64_t skh, int64_t sks, int64_t svb, int64_t svh, int64_t svs,
                    const uint16_t* key_pi_split, const uint16_t* key_seff_split, const float* key_centroids,
                    const float* key_bounds, int32_t key_code_bits, const uint16_t* val_pi_split,
                    const float* val_bounds, int32_t val_bits, uint8_t* key_codes, uint8_t* key_signs,
                    uint16_t* key_rn, uint16_t* key_vn, uint8_t* val_codes, uint16_t* val_vn, int64_t capacity,
                    int64_t pos, const void* q, int32_t Hq, int64_t sqb, int64_t sqh, int64_t sqs,
                    const uint16_t* key_s_eff_f16, uint16_t* q_rot, float* q_proj, void* stream) {
  TQ_CHECK_DD("tq_cache_append", d, dtype);
  TQ_REQUIRE(key_code_bits >= 1 && key_code_bits <= 8 && val_bits >= 1 && val_bits <= 8,
             "tq_cache_append: bits must be in [1, 8], got key code bits %d, value bits %d", key_code_bits, val_bits);
  TQ_REQUIRE(B >= 0 && H >= 0 && S >= 0 && (!q || Hq >= 0), "tq_cache_append: bad shape");
  TQ_REQUIRE(pos >= 0 && capacity >= pos + S, "tq_cache_append: rows [%lld, %lld) do not fit a capacity of %lld",
             (long long)pos, (long long)(pos + S), (long long)capacity);
  const int64_t n = static_cast<int64_t>(B) * H * S;
  const int64_t nq = q ? static_cast<int64_t>(B) * Hq * S : 0;
  if (n == 0 && nq == 0) return TQ_OK;
  TQ_REQUIRE(n == 0 || (k && v && key_pi_split && key_seff_split && key_centroids && key_bounds && val_pi_split &&
                        val_bounds && key_codes && key_signs && key_rn && key_vn && val_codes && val_vn),
             "tq_cache_append: null pointer");
  TQ_REQUIRE(nq == 0 || (key_pi_split && key_s_eff_f16 && q_rot && q_proj), "tq_cache_append: null query pointer");
  hipStream_t st = as_stream(stream);
  const bool aligned = reinterpret_cast<uintptr_t>(key_codes) % 4 == 0 && reinterpret_cast<uintptr_t>(key_signs) % 4 == 0 &&
                       reinterpret_cast<uintptr_t>(val_codes) % 4 == 0 &&
                       (nq == 0 || (reinterpret_cast<uintptr_t>(q_rot) % 8 == 0 && reinterpret_cast<uintptr_t>(q_proj) % 16 == 0));
  if ((d == 64 || d == 128) && val_bits >= 2 && val_bits <= 4 && key_code_bits == val_bits - 1 && aligned &&
      n < (int64_t(1) << 31) && nq < (int64_t(1) << 31) && (B * static_cast<int64_t>(H) * capacity) < (int64_t(1) << 40)) {
    const uint32_t s1 = static_cast<uint32_t>(S > 0 ? S : 1);
    TileArgs ka{}, va{}, qa{};
    ka.x = k; ka.n = n; ka.H = make_div(static_cast<uint32_t>(H > 0 ? H : 1)); ka.S = make_div(s1);
    ka.sb = skb; ka.sh = skh; ka.ss = sks; ka.vec = tile_vec(k, dtype, skb, skh, sks);
    ka.w1 = key_pi_split; ka.w3 = key_seff_split; ka.cent = key_centroids; ka.bounds = key_bounds;
    ka.codes = key_codes; ka.signs = key_signs; ka.rn = key_rn; ka.vn = key_vn; ka.ldo = capacity; ka.off = pos;
    va.x = v; va.n = n; va.H = ka.H; va.S = ka.S;
    va.sb = svb; va.sh = svh; va.ss = svs; va.vec = tile_vec(v, dtype, svb, svh, svs);
    va.w1 = val_pi_split; va.bounds = val_bounds; va.codes = val_codes; va.vn = val_vn; va.ldo = capacity; va.off = pos;
    qa.n = nq;
    if (nq > 0) {
      qa.x = q; qa.H = make_div(static_cast<uint32_t>(Hq)); qa.S = make_div(s1);
      qa.sb = sqb; qa.sh = sqh; qa.ss = sqs; qa.vec = tile_vec(q, dtype, sqb, sqh, sqs);
      qa.w1 = key_pi_split; qa.w2 = key_s_eff_f16; qa.q_rot = q_rot; qa.q_proj = q_proj;
    }
    dispatch_append(ka, va, qa, d, dtype, val_bits, st);
    return launch_status("tq_cache_append");
  }
  // other head dims and bit widths: the tile kernels, writing the same mapped rows
  if (n > 0) {
    KeyArgs ka{k, n, Rows4{H, S, skb, skh, sks}, key_pi_split, key_seff_split, key_centroids, key_bounds,
               key_code_bits, key_codes, key_signs, key_rn, key_vn, nullptr, nullptr, d, S, capacity, pos};
    TQ_SWITCH_DD(launch_keys, d, dtype, ka, n, st);
    ValArgs va{v, n, Rows4{H, S, svb, svh, svs}, val_pi_split, val_bounds, val_bits, val_codes, val_vn, nullptr, d,
               S, capacity, pos};
    TQ_SWITCH_DD(launch_values, d, dtype, va, n, st);
    const int e = launch_status("tq_cache_append");
    if (e != TQ_OK) return e;
  }
  if (nq > 0)
    return tq_query_prep(q, dtype, B, Hq, S, d, sqb, sqh, sqs, key_pi_split, key_s_eff_f16, q_rot, q_proj, stream);
  return TQ_OK;
}

}  // extern "C"
