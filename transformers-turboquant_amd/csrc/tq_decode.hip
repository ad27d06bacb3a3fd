// Decode-shaped compressed attention: few query rows per head (G * Sq <= 16
// (query row, query head) columns per kv head) against long compressed
// caches.  The work is HBM-bound: every key and value record is streamed
// once per step, so the kernel is organised around the byte stream.
//
// Split-K: a block of 4 wave64 owns a chunk of keys of one (batch, kv head);
// each wave walks its own 16-key blocks straight from HBM into registers
// (prefetching the next block while computing the current one) with no LDS
// staging and no block barriers.  MFMA operands are built from the packed
// bytes through LDS lookup tables (byte -> f16 values); the k-slot order of
// each MFMA is permuted so that a lane's operand bytes are contiguous in the
// packed rows:
//   scores  S^T = K^ Q_rot^T, Sign Q_proj^T  (16x16x32): lane (key m, group g)
//           holds dims g*D/4 + ks*8 + 0..7 at k-step ks
//   values  O^T += V^T P^T (16x16x16): O^T row m of block db is dim m*(D/16)+db,
//           so a lane's value operand comes from one contiguous code field
// The (m, l, O) state of the 4 waves is merged in LDS into one partial per
// block; tq_decode_merge combines the splits, normalises and applies Pi_v.
// In scores mode each block writes its keys' f32 scores directly.
#include "tq_common.h"

namespace tq {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float4v mfma16x16x16(half4 a, half4 b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

struct DecodeArgs {
  const uint16_t *q_rot, *q_proj;
  const uint8_t *kcodes, *ksigns;
  const uint16_t *krn, *kvn, *kcent;
  const uint8_t* vcodes;
  const uint16_t* vvn;
  const float* vcent;            // f32 value centroids (tables hold their f16 values)
  int B, Hq, Hkv, Sq, Sk, G, C;  // C = G * Sq valid columns
  int nsplit, chunk;             // keys per block (multiple of 64)
  float coeff, scale;
  int causal;
  const float* mask;
  int64_t smb, smh, smq, smk;
  float* scores;                 // scores mode: f32 [B, Hq, Sq, Sk]
  float *part_o, *part_ml;       // attention mode partials
};

template <int BITS>
struct DecodeLuts {
  static constexpr int KB = BITS - 1, VB = BITS;
  // key table: KB=1 byte -> 8 values, KB=2 byte -> 4 values, KB=3 12 bits -> 4 values
  static constexpr int KENT = (KB == 3) ? 4096 : 256;
  static constexpr int KW = (KB == 1) ? 8 : 4;
  // value table: VB=2 byte -> 4, VB=3 12 bits -> 4, VB=4 byte -> 2
  static constexpr int VENT = (VB == 3) ? 4096 : 256;
  static constexpr int VW = (VB == 4) ? 2 : 4;
  static constexpr int HALVES = 256 * 8 + KENT * KW + VENT * VW;
};

template <int D, int BITS, bool SCORES>
__global__ void __launch_bounds__(256) decode_kernel(DecodeArgs a) {
  static_assert(D == 128, "decode kernel is built for head_dim 128");
  using L = DecodeLuts<BITS>;
  constexpr int KB = L::KB, VB = L::VB;
  constexpr int KS = D / 32;           // score k-steps
  constexpr int DB = D / 16;           // value row blocks
  constexpr int KC = D * KB / 8, SC = D / 8, VC = D * VB / 8;  // bytes per packed row
  constexpr int KLANE = KC / 4;        // key-code bytes per lane (4 lanes share a key row)
  constexpr float LOG2E = 1.4426950408889634f;

  // LUTs, reused as the wave-merge area once every wave is done
  constexpr int MERGE_FLOATS = 4 * 16 * (D + 2);
  constexpr int LDS_BYTES = (L::HALVES * 2 > MERGE_FLOATS * 4) ? L::HALVES * 2 : MERGE_FLOATS * 4;
  __shared__ __attribute__((aligned(16))) uint8_t lds[LDS_BYTES];
  _Float16* lutS = reinterpret_cast<_Float16*>(lds);
  _Float16* lutK = lutS + 256 * 8;
  _Float16* lutV = lutK + L::KENT * L::KW;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const int split = blockIdx.x, hkv = blockIdx.y, b = blockIdx.z;
  const int64_t bh = static_cast<int64_t>(b) * a.Hkv + hkv;

  // ---- tables
  {
    const _Float16 one = static_cast<_Float16>(1.f), mone = static_cast<_Float16>(-1.f);
    for (int i = tid; i < 256 * 8; i += 256) lutS[i] = ((i >> 3) >> (i & 7)) & 1 ? one : mone;
    for (int i = tid; i < L::KENT * L::KW; i += 256) {
      const int idx = i / L::KW, e = i % L::KW;
      lutK[i] = __builtin_bit_cast(_Float16, a.kcent[(idx >> (e * KB)) & ((1 << KB) - 1)]);
    }
    if constexpr (!SCORES) {
      for (int i = tid; i < L::VENT * L::VW; i += 256) {
        const int idx = i / L::VW, e = i % L::VW;
        lutV[i] = static_cast<_Float16>(a.vcent[(idx >> (e * VB)) & ((1 << VB) - 1)]);
      }
    }
  }

  // ---- this lane's column (query row i, head h) and q fragments (permuted k-slots)
  const int col = l16;
  const bool col_ok = col < a.C;
  const int qi = col_ok ? col / a.G : 0, h = hkv * a.G + (col_ok ? col % a.G : 0);
  half8 qr[KS], qp[KS];
  {
    const int64_t qrow = ((static_cast<int64_t>(b) * a.Hq + h) * a.Sq + qi) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d0 = lg * (D / 4) + ks * 8;
      qr[ks] = col_ok ? *reinterpret_cast<const half8*>(a.q_rot + qrow + d0) : half8{};
      qp[ks] = col_ok ? *reinterpret_cast<const half8*>(a.q_proj + qrow + d0) : half8{};
    }
  }
  __syncthreads();

  const float fa = SCORES ? 1.f : a.scale * LOG2E;
  const float fb = a.coeff * fa;
  const int lim = qi + (a.Sk - a.Sq);  // causal: keys <= lim
  const int kbeg = split * a.chunk;
  const int kend = min(a.Sk, kbeg + a.chunk);

  // per-lane registers of one 16-key block
  struct Raw {
    uint32_t k[KLANE / 4];  // key-code bytes of (key m, group g)
    uint32_t s;             // sign bytes of (key m, group g)
    uint32_t v[4];          // value-code field (VB bytes) of keys 4g+kk at dims m*8..m*8+7
    float kn[4], rn[4], vv[4];
  };
  auto load = [&](int k0, Raw& r) {
    const int key = k0 + l16;  // row of this lane's key / sign operand
    if (key < kend) {
      const uint32_t* kp = reinterpret_cast<const uint32_t*>(a.kcodes + (bh * a.Sk + key) * KC + lg * KLANE);
#pragma unroll
      for (int j = 0; j < KLANE / 4; ++j) r.k[j] = kp[j];
      r.s = *reinterpret_cast<const uint32_t*>(a.ksigns + (bh * a.Sk + key) * SC + lg * (SC / 4));
    } else {
#pragma unroll
      for (int j = 0; j < KLANE / 4; ++j) r.k[j] = 0u;
      r.s = 0u;
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int vk = k0 + lg * 4 + kk;  // key of this lane's score rows / value k-slots
      const bool ok = vk < kend;
      const int64_t row = bh * a.Sk + vk;
      r.kn[kk] = ok ? h2f(a.kvn[row]) : 0.f;
      r.rn[kk] = ok ? h2f(a.krn[row]) : 0.f;
      if constexpr (!SCORES) {
        r.vv[kk] = ok ? h2f(a.vvn[row]) : 0.f;
        uint32_t w = 0u;
        if (ok) {
          const uint8_t* vp = a.vcodes + row * VC;
          const int off = l16 * VB;  // byte offset of dims l16*8 .. +7
          const uint32_t* wp = reinterpret_cast<const uint32_t*>(vp + (off & ~3));
          const int sh = off & 3;
          w = wp[0];
          if (sh + VB > 4) w = __builtin_amdgcn_alignbyte(wp[1], w, sh);
          else if (sh) w >>= 8 * sh;
        }
        r.v[kk] = w;
      }
    }
  };

  float m_run = -INFINITY, l_run = 0.f;
  float4v oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = float4v{0.f, 0.f, 0.f, 0.f};

  Raw cur, nxt;
  int k0 = kbeg + wave * 16;
  if (k0 < kend) load(k0, cur);
  for (; k0 < kend; k0 += 64) {
    const bool more = k0 + 64 < kend;
    if (more) load(k0 + 64, nxt);

    // ---- scores: two accumulators over KS k-steps
    float4v s1 = float4v{0.f, 0.f, 0.f, 0.f}, s2 = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      half8 ka;
      if constexpr (KB == 1) {
        const uint32_t byte = (cur.k[0] >> (8 * ks)) & 0xffu;
        ka = *reinterpret_cast<const half8*>(&lutK[byte * 8]);
      } else if constexpr (KB == 2) {
        const uint32_t two = (cur.k[ks >> 1] >> (16 * (ks & 1))) & 0xffffu;
        const half4 lo = *reinterpret_cast<const half4*>(&lutK[(two & 0xffu) * 4]);
        const half4 hi = *reinterpret_cast<const half4*>(&lutK[(two >> 8) * 4]);
        ka = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      } else {
        // 24 bits of k-step ks start at bit 24*ks of the lane's 96-bit field
        const int bit = 24 * ks, wi = bit >> 5, sh = bit & 31;
        const uint32_t lo32 = cur.k[wi];
        const uint32_t hi32 = (wi + 1 < KLANE / 4) ? cur.k[wi + 1] : 0u;
        const uint32_t f = sh ? __builtin_amdgcn_alignbit(hi32, lo32, sh) : lo32;
        const half4 lo = *reinterpret_cast<const half4*>(&lutK[(f & 0xfffu) * 4]);
        const half4 hi = *reinterpret_cast<const half4*>(&lutK[((f >> 12) & 0xfffu) * 4]);
        ka = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
      const half8 sa = *reinterpret_cast<const half8*>(&lutS[((cur.s >> (8 * ks)) & 0xffu) * 8]);
      s1 = mfma16x16x32(ka, qr[ks], s1);
      s2 = mfma16x16x32(sa, qp[ks], s2);
    }

    if constexpr (SCORES) {
      if (col_ok) {
        float* orow = a.scores + ((static_cast<int64_t>(b) * a.Hq + h) * a.Sq + qi) * a.Sk;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = k0 + lg * 4 + e;
          if (key < kend) orow[key] = s1[e] * (fa * cur.kn[e]) + s2[e] * (fb * cur.rn[e]);
        }
      }
    } else {
      // ---- online softmax (log2 units, lazily rescaled)
      float sc[4];
      float tmax = -INFINITY;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = k0 + lg * 4 + e;
        float v = s1[e] * (fa * cur.kn[e]) + s2[e] * (fb * cur.rn[e]);
        if (a.mask && col_ok && key < kend)
          v += fmaxf(a.mask[b * a.smb + h * a.smh + static_cast<int64_t>(qi) * a.smq +
                            static_cast<int64_t>(key) * a.smk] * LOG2E,
                     -3.0e38f);
        if (key >= kend || (a.causal && key > lim)) v = -INFINITY;
        sc[e] = v;
        tmax = fmaxf(tmax, v);
      }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const bool grow = tmax > m_run + 8.0f;
      if (__any(grow)) {
        const float m_new = grow ? tmax : m_run;
        const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) oacc[db] *= alpha;
      }
      // p = 2^(s - m_run - TAU) <= 1, so P * vn stays inside f16 range for any f16 norm;
      // (m_run + TAU) is the reference the partial's (O, l) are scaled to
      const float m_use = (m_run == -INFINITY) ? 0.f : m_run + 8.0f;
      half4 ph, pl;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float p = __builtin_amdgcn_exp2f(sc[e] - m_use);
        l_run += p;
        const float pv = p * cur.vv[e];
        const _Float16 hh = static_cast<_Float16>(pv);
        ph[e] = hh;
        pl[e] = static_cast<_Float16>(pv - static_cast<float>(hh));
      }
      // ---- value operands: per key kk the 8 values of dims l16*8 + db, db = 0..7
      half8 vals[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const uint32_t w = cur.v[kk];
        if constexpr (VB == 2) {
          const half4 lo = *reinterpret_cast<const half4*>(&lutV[(w & 0xffu) * 4]);
          const half4 hi = *reinterpret_cast<const half4*>(&lutV[((w >> 8) & 0xffu) * 4]);
          vals[kk] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        } else if constexpr (VB == 3) {
          const half4 lo = *reinterpret_cast<const half4*>(&lutV[(w & 0xfffu) * 4]);
          const half4 hi = *reinterpret_cast<const half4*>(&lutV[((w >> 12) & 0xfffu) * 4]);
          vals[kk] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        } else {
          half8 v8;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const half2v t = *reinterpret_cast<const half2v*>(&lutV[((w >> (8 * q)) & 0xffu) * 2]);
            v8[2 * q] = t[0];
            v8[2 * q + 1] = t[1];
          }
          vals[kk] = v8;
        }
      }
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const half4 va = half4{vals[0][db], vals[1][db], vals[2][db], vals[3][db]};
        oacc[db] = mfma16x16x16(va, ph, oacc[db]);
        oacc[db] = mfma16x16x16(va, pl, oacc[db]);
      }
    }
    if (more) cur = nxt;
  }

  if constexpr (!SCORES) {
    // ---- merge the 4 waves of the block in LDS, write one partial per block
    __syncthreads();  // all waves done with the tables
    float* mrg = reinterpret_cast<float*>(lds);  // [wave][col][D + 2]
    float l = l_run;
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    float* mine = mrg + (wave * 16 + col) * (D + 2);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int e = 0; e < 4; ++e) mine[(lg * 4 + e) * (D / 16) + db] = oacc[db][e];
    if (lg == 0) {
      mine[D] = (m_run == -INFINITY) ? m_run : m_run + 8.0f;
      mine[D + 1] = l;
    }
    __syncthreads();
    const int64_t pbase = (bh * a.nsplit + split) * a.C;
    for (int it = tid; it < a.C * D; it += 256) {
      const int c = it / D, d = it % D;
      float mx = -INFINITY;
#pragma unroll
      for (int w = 0; w < 4; ++w) mx = fmaxf(mx, mrg[(w * 16 + c) * (D + 2) + D]);
      float o = 0.f, ls = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float* src = mrg + (w * 16 + c) * (D + 2);
        const float sc = (src[D] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(src[D] - mx);
        o += sc * src[d];
        ls += sc * src[D + 1];
      }
      a.part_o[(pbase + c) * D + d] = o;
      if (d == 0) {
        a.part_ml[(pbase + c) * 2] = mx;
        a.part_ml[(pbase + c) * 2 + 1] = ls;
      }
    }
  }
}

struct MergeArgs {
  const float *part_o, *part_ml;
  const uint16_t* vpit;  // split Pi_v^T
  int B, Hq, Hkv, Sq, G, C, nsplit;
  void* out;
  int out_dtype;
  int64_t sob, soh, sos;
};

// One block per (batch, kv head): combine the splits of its C columns, normalise,
// rotate back with Pi_v (read once per block) and store.
template <int D>
__global__ void __launch_bounds__(256) decode_merge_kernel(MergeArgs a) {
  constexpr int SW = 64;  // splits per weight batch
  __shared__ float o_rot[16 * D];
  __shared__ float s_w[16 * SW];
  __shared__ float s_red[16 * 16];
  __shared__ float s_mx[16], s_l[16];
  const int hkv = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int C = a.C, ns = a.nsplit;
  const int64_t base = (static_cast<int64_t>(b) * a.Hkv + hkv) * ns;  // first split record
  auto ml = [&](int s, int c, int k) { return a.part_ml[((base + s) * C + c) * 2 + k]; };

  // column maxima: thread (c, r) scans splits r, r + 16, ...
  {
    const int c = tid & 15, r = tid >> 4;
    float mx = -INFINITY;
    if (c < C)
      for (int s = r; s < ns; s += 16) mx = fmaxf(mx, ml(s, c, 0));
    s_red[r * 16 + c] = mx;
    __syncthreads();
    if (tid < 16) {
      float m = -INFINITY;
      for (int i = 0; i < 16; ++i) m = fmaxf(m, s_red[i * 16 + tid]);
      s_mx[tid] = m;
      s_l[tid] = 0.f;
    }
    __syncthreads();
  }

  // weighted sum of the splits; thread owns outputs it, it + 256, ... of the C x D tile
  constexpr int PER = 16 * D / 256;
  float acc[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) acc[k] = 0.f;
  for (int s0 = 0; s0 < ns; s0 += SW) {
    const int nb = min(SW, ns - s0);
    for (int i = tid; i < C * SW; i += 256) {
      const int c = i / SW, s = i % SW;
      float w = 0.f;
      if (s < nb) {
        const float m = ml(s0 + s, c, 0);
        w = (m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - s_mx[c]);
      }
      s_w[c * SW + s] = w;
    }
    __syncthreads();
    if (tid < C) {
      float l = s_l[tid];
      for (int s = 0; s < nb; ++s) l += s_w[tid * SW + s] * ml(s0 + s, tid, 1);
      s_l[tid] = l;
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int it = tid + 256 * k, c = it / D, j = it % D;
      if (c < C) {
        const float* src = a.part_o + ((base + s0) * C + c) * D + j;
        float o = acc[k];
        for (int s = 0; s < nb; ++s) o += s_w[c * SW + s] * src[static_cast<int64_t>(s) * C * D];
        acc[k] = o;
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int it = tid + 256 * k, c = it / D, j = it % D;
    if (c < C) o_rot[c * D + j] = (s_l[c] > 0.f) ? acc[k] / s_l[c] : 0.f;
  }
  __syncthreads();

  // out[c][j] = sum_i o_rot[c][i] * Pi_v[i][j] = sum_i o_rot[c][i] * Pi_v^T[j][i], Pi_v^T = (hi + lo) / 1024
  const int j = tid % D, c0 = tid / D;
  const _Float16* ph = reinterpret_cast<const _Float16*>(a.vpit) + j * D;
  const _Float16* pl = ph + D * D;
  constexpr int CS = 256 / D;  // columns handled per pass
  for (int cb = 0; cb < C; cb += 4 * CS) {
    float r[4] = {0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < D; i += 8) {
      const half8 h = *reinterpret_cast<const half8*>(ph + i);
      const half8 l = *reinterpret_cast<const half8*>(pl + i);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float w = (static_cast<float>(h[e]) + static_cast<float>(l[e])) * (1.f / kSplit);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int c = cb + c0 + q * CS;
          if (c < C) r[q] += o_rot[c * D + i + e] * w;
        }
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = cb + c0 + q * CS;
      if (c >= C) continue;
      const int qi = c / a.G, h = hkv * a.G + c % a.G;
      const int64_t off = static_cast<int64_t>(b) * a.sob + static_cast<int64_t>(h) * a.soh +
                          static_cast<int64_t>(qi) * a.sos + j;
      if (a.out_dtype == TQ_BF16) store_act<TQ_BF16>(a.out, off, r[q]);
      else if (a.out_dtype == TQ_F16) store_act<TQ_F16>(a.out, off, r[q]);
      else store_act<TQ_F32>(a.out, off, r[q]);
    }
  }
}

// ---------------------------------------------------------------- planning
struct DecodePlan {
  bool use;
  int nsplit, chunk;
  int64_t ws_bytes;
};

static DecodePlan plan_decode(int B, int Hq, int Hkv, int Sq, int Sk, int d, int bits) {
  DecodePlan p{false, 0, 0, 0};
  if (d != 128 || bits < 2 || bits > 4 || Hkv <= 0 || Hq % Hkv) return p;
  const int C = (Hq / Hkv) * Sq;
  if (C > 16 || Sk < 1) return p;
  const int64_t groups = static_cast<int64_t>(B) * Hkv;
  int nsplit = static_cast<int>((1024 + groups - 1) / groups);
  const int max_split = (Sk + 255) / 256;
  if (nsplit > max_split) nsplit = max_split;
  if (nsplit > 1024) nsplit = 1024;
  if (nsplit < 1) nsplit = 1;
  int chunk = (Sk + nsplit - 1) / nsplit;
  chunk = (chunk + 63) / 64 * 64;
  nsplit = (Sk + chunk - 1) / chunk;
  p.use = true;
  p.nsplit = nsplit;
  p.chunk = chunk;
  p.ws_bytes = groups * nsplit * C * static_cast<int64_t>(d + 2) * 4;
  return p;
}

}  // namespace tq

using namespace tq;

// Used by tq_attn.hip's entry points.
namespace tq {

int64_t decode_workspace_bytes(int B, int Hq, int Hkv, int Sq, int Sk, int d, int bits) {
  const DecodePlan p = plan_decode(B, Hq, Hkv, Sq, Sk, d, bits);
  return p.use ? p.ws_bytes : 0;
}

bool decode_applies(int B, int Hq, int Hkv, int Sq, int Sk, int d, int bits) {
  return plan_decode(B, Hq, Hkv, Sq, Sk, d, bits).use;
}

template <int BITS, bool SCORES>
static void launch_decode(const DecodeArgs& a, hipStream_t s) {
  dim3 grid(a.nsplit, a.Hkv, a.B);
  decode_kernel<128, BITS, SCORES><<<grid, 256, 0, s>>>(a);
}

int decode_scores(const uint16_t* q_rot, const uint16_t* q_proj, const uint8_t* kcodes,
                  const uint8_t* ksigns, const uint16_t* krn, const uint16_t* kvn, const uint16_t* kcent,
                  int B, int Hq, int Hkv, int Sq, int Sk, int d, int bits, float coeff, float* out,
                  hipStream_t s) {
  const DecodePlan p = plan_decode(B, Hq, Hkv, Sq, Sk, d, bits);
  DecodeArgs a{};
  a.q_rot = q_rot;
  a.q_proj = q_proj;
  a.kcodes = kcodes;
  a.ksigns = ksigns;
  a.krn = krn;
  a.kvn = kvn;
  a.kcent = kcent;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.Sq = Sq;
  a.Sk = Sk;
  a.G = Hq / Hkv;
  a.C = a.G * Sq;
  a.nsplit = p.nsplit;
  a.chunk = p.chunk;
  a.coeff = coeff;
  a.scale = 1.f;
  a.scores = out;
  if (bits == 2) launch_decode<2, true>(a, s);
  else if (bits == 3) launch_decode<3, true>(a, s);
  else launch_decode<4, true>(a, s);
  return launch_status("tq_attention_scores (decode)");
}

int decode_attention(const uint16_t* q_rot, const uint16_t* q_proj, const uint8_t* kcodes,
                     const uint8_t* ksigns, const uint16_t* krn, const uint16_t* kvn, const uint16_t* kcent,
                     int bits, const uint8_t* vcodes, const uint16_t* vvn, const float* vcent32,
                     const uint16_t* vpit, int B, int Hq, int Hkv, int Sq, int Sk, int d, float coeff,
                     float scale, int causal, const float* mask, int64_t smb, int64_t smh, int64_t smq,
                     int64_t smk, void* out, int out_dtype, int64_t sob, int64_t soh, int64_t sos,
                     void* workspace, hipStream_t s) {
  const DecodePlan p = plan_decode(B, Hq, Hkv, Sq, Sk, d, bits);
  DecodeArgs a{};
  a.q_rot = q_rot;
  a.q_proj = q_proj;
  a.kcodes = kcodes;
  a.ksigns = ksigns;
  a.krn = krn;
  a.kvn = kvn;
  a.kcent = kcent;
  a.vcodes = vcodes;
  a.vvn = vvn;
  a.vcent = vcent32;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.Sq = Sq;
  a.Sk = Sk;
  a.G = Hq / Hkv;
  a.C = a.G * Sq;
  a.nsplit = p.nsplit;
  a.chunk = p.chunk;
  a.coeff = coeff;
  a.scale = scale;
  a.causal = causal;
  a.mask = mask;
  a.smb = smb;
  a.smh = smh;
  a.smq = smq;
  a.smk = smk;
  float* ws = static_cast<float*>(workspace);
  const int64_t n_part = static_cast<int64_t>(B) * Hkv * p.nsplit * a.C;
  a.part_o = ws;
  a.part_ml = ws + n_part * d;
  if (bits == 2) launch_decode<2, false>(a, s);
  else if (bits == 3) launch_decode<3, false>(a, s);
  else launch_decode<4, false>(a, s);
  int st = launch_status("tq_attention_fwd (decode)");
  if (st != TQ_OK) return st;
  MergeArgs m{};
  m.part_o = a.part_o;
  m.part_ml = a.part_ml;
  m.vpit = vpit;
  m.B = B;
  m.Hq = Hq;
  m.Hkv = Hkv;
  m.Sq = Sq;
  m.G = a.G;
  m.C = a.C;
  m.nsplit = p.nsplit;
  m.out = out;
  m.out_dtype = out_dtype;
  m.sob = sob;
  m.soh = soh;
  m.sos = sos;
  dim3 grid(Hkv, B);
  decode_merge_kernel<128><<<grid, 256, 0, s>>>(m);
  return launch_status("tq_attention_fwd (decode merge)");
}

}  // namespace tq
