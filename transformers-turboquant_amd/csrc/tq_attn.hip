// Compressed-domain attention on gfx950: asymmetric scores from packed keys,
// online softmax, and P.V over packed values, in one kernel.  This tiled kernel
// serves every head dim that is a multiple of 8 up to 256 (the prefill and
// split-K decode kernels cover head_dim 64 and 128 at their shapes).
//
// Scores follow the reference estimator (kernels/attention.py:380-461,
// compressors.py:178-200):
//   s(q, k) = vn_k * <q_rot, Ck[codes_k]> + coeff * rn_k * <q_proj, 2*sign_k - 1>
// with q_rot = f16(q Pi^T) and q_proj = q_rot S_eff^T (f32) from tq_query_prep;
// q_proj enters as f16 hi + lo (two MFMAs against the exact +-1 operand, ~2^-22
// of f32), as the reference keeps it in fp32 (attention.py:158-167).
// Both inner products run as v_mfma_f32_16x16x32_f16 chains with exact f16
// key operands (f16 centroids, +-1), so term 1 is exactly the reference's f32
// accumulation of f16 products; the per-key factors vn and coeff * rn are
// applied in f32 to the two accumulators.
//
// Work decomposition: a block of 4 wave64 owns one (batch, kv head) and BR
// (query row, query head) columns -- all G = Hq/Hkv heads of the group share
// each key tile (the reference expands K/V with repeat_interleave instead,
// families/qwen2.py:101-102).  Key tiles of KT keys are streamed through LDS
// as raw packed byte streams (rows of d*b/8 bytes; software pipelined: the next
// tile's planes are loaded into registers while the current tile computes) and
// decoded once per tile into f16 K^, sign and V^T tiles through byte-indexed
// lookup tables.  Head dims are padded to a multiple of 32 with zeros.  S^T's
// accumulator layout (4 consecutive keys of one column per lane) is the
// B-operand layout P^T needs for O^T += V^T P^T, so P stays in registers.
// Values stay in the rotated domain:
// O = (sum_j p_j vn_j Cv[c_j]) Pi_v, with Pi_v applied once per output row.
// P enters the P.V product as an f16 (hi, lo) pair, so the only f16 rounding
// on the value side is that of the decoded V^ = f16(Cv * vn).
#include "tq_common.h"

#include <mutex>

namespace tq {

constexpr int kAttnWaves = 4;      // waves per block
constexpr int kAttnKeys = 32;      // keys per tile
constexpr float kAttnTau = 8.0f;   // lazy-rescale headroom of the online softmax (log2 units)

// D is the head dim padded to a multiple of 32 (the MFMA k-step); the real head dim d
// (a multiple of 8) comes at run time.  Query fragments, decoded key / sign / value tiles
// and Pi_v read zero past d, so the padding adds nothing to any product.
template <int D, bool SCORES>
struct ATile {
  static constexpr int NW = kAttnWaves;          // waves per block
  static constexpr int NT = 64 * NW;             // threads per block
  static constexpr int KT = kAttnKeys;           // keys per tile
  // 16-column blocks per wave: two where the q_rot / q_proj (hi, lo) fragments and, in
  // attention mode, the O^T accumulators of both fit in registers
  static constexpr int NBW = SCORES ? (D <= 128 ? 2 : 1) : (D <= 64 ? 2 : 1);
  static constexpr int BR = NW * 16 * NBW;       // (query, head) columns per block
  static constexpr int KS = D / 32;              // k-steps of the score MFMAs
  static constexpr int MBK = KT / 16;            // 16-key blocks per tile
  static constexpr int DB = D / 16;              // 16-dim blocks
  static constexpr int LDK = D + 8;              // f16 row stride of decoded key / sign tiles
  static constexpr int LDV = KT + 8;             // f16 row stride of the V^T tile
  // raw planes of a tile in LDS, either as rows padded by one dword (head dims that are a
  // multiple of 32: dword-aligned rows, and the pad spreads the decode's row-strided reads
  // over the banks) or as a byte stream (other head dims: rows of d*b/8 bytes, staged from
  // the dword at or below the tile's first byte); slack covers the stream's shift and the
  // dword-pair reads of the last row
  static constexpr int KRAW = KT * (D * 3 / 8 + 4) + 8, SRAW = KT * (D / 8 + 4) + 8, VRAW = KT * (D * 4 / 8 + 4) + 8;
  static constexpr int KREG = (KRAW / 4 + NT - 1) / NT;  // per-thread dwords of a tile
  static constexpr int SREG = (SRAW / 4 + NT - 1) / NT;
  static constexpr int VREG = (VRAW / 4 + NT - 1) / NT;
};

struct AttnArgs {
  const uint16_t* q_rot;
  const float* q_proj;  // f32, taken as f16 hi + lo operands (two MFMAs against the exact +-1 signs)
  const uint8_t *kcodes, *ksigns;
  const uint16_t *krn, *kvn, *kcent;
  const uint8_t* vcodes;
  const uint16_t *vvn, *vpit;
  const float* vcent32;
  int vb;
  int d;  // head dim (multiple of 8, <= D)
  int B, Hq, Hkv, Sq, Sk, G, QT, nqb;
  int64_t ldk;  // rows between consecutive (batch, kv head) planes (>= Sk)
  float coeff, scale;
  int causal;
  const float* mask;
  int64_t smb, smh, smq, smk;
  void* out;
  int out_dtype;
  int64_t sob, soh, sos;
  float* scores;  // scores-only mode output f32 [B, Hq, Sq, Sk]
  // split over keys (nsplit > 1): block (x, split) takes keys [split * chunk, (split + 1) *
  // chunk); in scores mode it writes their scores, in attention mode (part_o) its columns'
  // partial O (unnormalised, rotated value domain, rows of dp floats), reference maximum and
  // sum for attn_merge_kernel
  float *part_o, *part_ml;
  int nsplit, chunk, C, dp;
};

__device__ __forceinline__ half8 cat8(half4 a, half4 b) {
  return half8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// 32 bits of a byte stream from byte `off` on (base 4-byte aligned, one readable dword
// past the dword holding byte off + 3).
__device__ __forceinline__ uint32_t bits32_at(const uint8_t* base, int off) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(base + (off & ~3));
  return __builtin_amdgcn_alignbyte(w[1], w[0], off & 3);
}

template <int DT>
__device__ __forceinline__ void store4(void* out, int64_t o, float4v v, int n) {
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (e < n) store_act<DT>(out, o + e, v[e]);
}

// STREAM: head dims that are not a multiple of 32 (byte-stream staging, run-time d); otherwise
// d = D and rows are staged padded
template <int D, int KB, bool SCORES, bool MASK, bool STREAM>
__global__ void __launch_bounds__(64 * kAttnWaves, 2) attn_kernel(AttnArgs a) {
  using T = ATile<D, SCORES>;
  constexpr int KT = T::KT, NBW = T::NBW, KS = T::KS, MBK = T::MBK, DB = T::DB, NT = T::NT;
  constexpr int LUTK_W = (KB == 1) ? 8 : 4;  // f16 values per key-LUT entry (KB <= 2)
  constexpr int KITEMS = KT * (D / 8);       // (key, 8-dim group) decode items
  constexpr int VITEMS = (D / 8) * (KT / 4);  // (8-dim group, 4-key quad) decode items

  // double-buffered raw planes (byte streams), decoded tiles, lookup tables
  __shared__ __attribute__((aligned(16))) uint8_t rawK[2][T::KRAW];
  __shared__ __attribute__((aligned(16))) uint8_t rawS[2][T::SRAW];
  __shared__ __attribute__((aligned(16))) uint8_t rawV[SCORES ? 1 : 2][SCORES ? 4 : T::VRAW];
  __shared__ __attribute__((aligned(16))) float skA[2][KT];      // vn * scale * log2(e)
  __shared__ __attribute__((aligned(16))) float skB[2][KT];      // coeff * rn * scale * log2(e)
  __shared__ __attribute__((aligned(16))) float svv[2][KT];      // value norms
  __shared__ __attribute__((aligned(16))) _Float16 sK[KT * T::LDK];
  __shared__ __attribute__((aligned(16))) _Float16 sS[KT * T::LDK];
  __shared__ __attribute__((aligned(16))) _Float16 sVt[SCORES ? 8 : D * T::LDV];
  __shared__ __attribute__((aligned(16))) _Float16 lutS[256 * 8];
  __shared__ __attribute__((aligned(16))) _Float16 lutK[(KB == 3) ? 8 : 256 * LUTK_W];
  __shared__ float lutV[16];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  // blocks in order of decreasing causal work across every (batch, kv head): block i takes query
  // block nqb - 1 - i / (B Hkv) of group i % (B Hkv), so the longest blocks of all groups start
  // first and the grid's tail is short ones (the per-group order, all of one group's query
  // blocks before the next group's, left a 23% longer schedule at 8 kv heads); consecutive
  // blocks are different groups, so each XCD (blocks dealt round-robin) keeps to a fixed set of
  // groups and their K / V planes in its L2
  const int nbh = a.B * a.Hkv;
  const int qblk = a.nqb - 1 - static_cast<int>(blockIdx.x) / nbh;
  const int bhi = static_cast<int>(blockIdx.x) % nbh;
  const int hkv = bhi % a.Hkv, b = bhi / a.Hkv;
  const int q0 = qblk * a.QT;
  const bool split_k = a.nsplit > 1;
  const int split = split_k ? static_cast<int>(blockIdx.y) : 0;
  const int d = STREAM ? a.d : D;
  const int KC = d * KB / 8, SC = d / 8, vc = d * a.vb / 8;  // bytes per packed row
  const int ng = d / 8;                                       // real 8-dim groups
  const int64_t bh_kv = static_cast<int64_t>(b) * a.Hkv + hkv;

  // ---- lookup tables: byte -> 8 x (+-1); byte -> key centroids; value centroids (f32)
  {
    const _Float16 one = static_cast<_Float16>(1.f), mone = static_cast<_Float16>(-1.f);
    for (int i = tid; i < 256 * 8; i += NT) lutS[i] = ((i >> 3) >> (i & 7)) & 1 ? one : mone;
    if constexpr (KB == 3) {
      if (tid < 8) lutK[tid] = __builtin_bit_cast(_Float16, a.kcent[tid]);
    } else {
      for (int i = tid; i < 256 * LUTK_W; i += NT) {
        const int byte = i / LUTK_W, e = i % LUTK_W;
        lutK[i] = __builtin_bit_cast(_Float16, a.kcent[(byte >> (e * KB)) & ((1 << KB) - 1)]);
      }
    }
    if (!SCORES && tid < (1 << a.vb)) lutV[tid] = a.vcent32[tid];
  }

  // ---- this lane's columns and their q fragments (B operands): q_rot, q_proj hi and lo
  int col_i[NBW], col_h[NBW];
  bool col_ok[NBW];
  half8 qr[KS][NBW], qp[KS][NBW], qlo[KS][NBW];
  int64_t qrow[NBW];
  float qmax = 0.f;  // largest |q_proj| of the block's columns: the scale of its (hi, lo) split
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
    const int r = (wave * NBW + nb) * 16 + l16;
    const int ql = r / a.G, gi = r % a.G;
    col_i[nb] = q0 + ql;
    col_h[nb] = hkv * a.G + gi;
    col_ok[nb] = (ql < a.QT) && (col_i[nb] < a.Sq);
    qrow[nb] = ((static_cast<int64_t>(b) * a.Hq + col_h[nb]) * a.Sq + col_i[nb]) * d;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      if (col_ok[nb] && ks * 32 + lg * 8 < d) qmax = fmaxf(qmax, absmax8(a.q_proj + qrow[nb] + ks * 32 + lg * 8));
  }
  __shared__ float s_qmax[T::NW];
  qmax = wave_max(qmax);
  if (lane == 0) s_qmax[wave] = qmax;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < T::NW; ++w) qmax = fmaxf(qmax, s_qmax[w]);
  const float qs = qproj_split_scale(qmax);
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d0 = ks * 32 + lg * 8;
      const bool ok = col_ok[nb] && d0 < d;  // d % 8 == 0: the 8 dims from d0 are all real or all padding
      qr[ks][nb] = ok ? *reinterpret_cast<const half8*>(a.q_rot + qrow[nb] + d0) : half8{};
      half8 hi = half8{}, lo = half8{};
      if (ok) split8s(a.q_proj + qrow[nb] + d0, qs, hi, lo);
      qp[ks][nb] = hi;
      qlo[ks][nb] = lo;
    }
  }
  const float coeff_q = a.coeff * (1.f / qs);  // q_proj's operands carry qs

  // key range this block needs; tiles past `kfull` need per-element masking.  A split ends
  // on a tile boundary (chunk is a multiple of KT), so only the keys' own end needs masking.
  int kend = a.Sk;
  int kfull = a.Sk;
  if (a.causal) {
    const int imax = min(q0 + a.QT - 1, a.Sq - 1);
    kend = min(a.Sk, imax + (a.Sk - a.Sq) + 1);
    kfull = min(kfull, q0 + (a.Sk - a.Sq) + 1);
  }
  int kbeg = 0;
  if (split_k) {
    kbeg = split * a.chunk;
    kend = min(kend, kbeg + a.chunk);
  }
  constexpr float LOG2E = 1.4426950408889634f;
  const float fa = SCORES ? 1.f : a.scale * LOG2E;  // scores kept in log2 units

  // byte offset of tile k0's first row in a plane of `rowbytes`-byte rows, and that byte's
  // position within its dword (the staged stream starts at the dword)
  auto plane_off = [&](int k0, int rowbytes) { return (bh_kv * a.ldk + k0) * rowbytes; };
  auto shift_of = [&](const uint8_t* plane, int k0, int rowbytes) {
    return static_cast<int>((reinterpret_cast<uintptr_t>(plane) + plane_off(k0, rowbytes)) & 3);
  };

  // ---- register staging of one tile's planes: dwords from the aligned start on
  uint32_t rk[T::KREG], rs[T::SREG], rv[SCORES ? 1 : T::VREG];
  float r_a = 0.f, r_b = 0.f, r_v = 0.f;
  auto fetch_stream = [&](const uint8_t* plane, int k0, int rowbytes, int bytes, uint32_t* regs, int nreg) {
    // STREAM: from the dword holding the tile's first byte; otherwise rows are whole dwords
    const int shift = STREAM ? shift_of(plane, k0, rowbytes) : 0;
    const uint32_t* g = reinterpret_cast<const uint32_t*>(plane + (plane_off(k0, rowbytes) - shift));
    const int ndw = (shift + bytes + 3) >> 2;  // dwords holding the tile's bytes
    for (int j = 0; j < nreg; ++j) {
      const int w = tid + j * NT;
      regs[j] = (w < ndw) ? g[w] : 0u;
    }
  };
  // staged dwords -> LDS: contiguous (STREAM) or rows of `rowbytes` padded to rowbytes + 4
  auto stash_stream = [&](uint8_t* dst, int rowbytes, int raw_bytes, const uint32_t* regs, int nreg) {
    for (int j = 0; j < nreg; ++j) {
      const int w = tid + j * NT;
      if constexpr (STREAM) {
        if (w < raw_bytes / 4) reinterpret_cast<uint32_t*>(dst)[w] = regs[j];
      } else {
        const int wpr = rowbytes / 4;
        if (w < KT * wpr) {
          const int row = w / wpr, col = w - row * wpr;
          *reinterpret_cast<uint32_t*>(dst + row * (rowbytes + 4) + col * 4) = regs[j];
        }
      }
    }
  };
  auto fetch = [&](int k0) {
    const int nk = min(KT, a.Sk - k0);
    fetch_stream(a.kcodes, k0, KC, nk * KC, rk, T::KREG);
    fetch_stream(a.ksigns, k0, SC, nk * SC, rs, T::SREG);
    if constexpr (!SCORES) fetch_stream(a.vcodes, k0, vc, nk * vc, rv, T::VREG);
    if (tid < KT) {
      const int64_t kr = bh_kv * a.ldk + k0 + tid;
      const bool ok = tid < nk;
      const float vn = ok ? h2f(a.kvn[kr]) : 0.f;
      const float rn = ok ? h2f(a.krn[kr]) : 0.f;
      r_a = fa * vn;
      r_b = fa * coeff_q * rn;
      if constexpr (!SCORES) r_v = ok ? h2f(a.vvn[kr]) : 0.f;
    }
  };
  auto stash = [&](int buf) {
    stash_stream(rawK[buf], KC, T::KRAW, rk, T::KREG);
    stash_stream(rawS[buf], SC, T::SRAW, rs, T::SREG);
    if constexpr (!SCORES) stash_stream(rawV[buf], vc, T::VRAW, rv, T::VREG);
    if (tid < KT) {
      skA[buf][tid] = r_a;
      skB[buf][tid] = r_b;
      if constexpr (!SCORES) svv[buf][tid] = r_v;
    }
  };

  float m_run[NBW], l_run[NBW];
  float4v oacc[SCORES ? 1 : DB][NBW];
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
    m_run[nb] = -INFINITY;
    l_run[nb] = 0.f;
    if constexpr (!SCORES) {
#pragma unroll
      for (int db = 0; db < DB; ++db) oacc[db][nb] = float4v{0.f, 0.f, 0.f, 0.f};
    }
  }

  if (kend > kbeg) {
    fetch(kbeg);
    stash(0);
  }
  int cur = 0;
  for (int k0 = kbeg; k0 < kend; k0 += KT) {
    __syncthreads();  // tile k0 staged in buffer `cur`; previous tile's decoded tiles consumed
    // ---- decode this tile once per block: K^ and sign tiles [key][dim], V^T [dim][key];
    // groups past d decode to zeros
    // row r of a plane starts at byte sh + r * rp of its staged copy
    const int shk = STREAM ? shift_of(a.kcodes, k0, KC) : 0, rpk = STREAM ? KC : KC + 4;
    const int shs = STREAM ? shift_of(a.ksigns, k0, SC) : 0, rps = STREAM ? SC : SC + 4;
#pragma unroll
    for (int j = 0; j < (KITEMS + NT - 1) / NT; ++j) {
      const int it = tid + j * NT;
      if (KITEMS % NT == 0 || it < KITEMS) {
        const int key = it / (D / 8), dg = it % (D / 8);
        half8 kv = half8{}, sv = half8{};
        if (!STREAM || dg < ng) {
          const int ko = shk + key * rpk + dg * KB;  // the group's KB bytes
          if constexpr (KB == 1) {
            kv = *reinterpret_cast<const half8*>(&lutK[rawK[cur][ko] * 8]);
          } else if constexpr (KB == 2) {
            uint32_t two;  // the group's two code bytes (an aligned u16 in the padded rows)
            if constexpr (STREAM) two = rawK[cur][ko] | (static_cast<uint32_t>(rawK[cur][ko + 1]) << 8);
            else two = *reinterpret_cast<const uint16_t*>(&rawK[cur][ko]);
            kv = cat8(*reinterpret_cast<const half4*>(&lutK[(two & 0xffu) * 4]),
                      *reinterpret_cast<const half4*>(&lutK[(two >> 8) * 4]));
          } else {
            const uint32_t w = bits32_at(rawK[cur], ko);
#pragma unroll
            for (int e = 0; e < 8; ++e) kv[e] = lutK[(w >> (e * 3)) & 7u];
          }
          sv = *reinterpret_cast<const half8*>(&lutS[rawS[cur][shs + key * rps + dg] * 8]);
        }
        *reinterpret_cast<half8*>(&sK[key * T::LDK + dg * 8]) = kv;
        *reinterpret_cast<half8*>(&sS[key * T::LDK + dg * 8]) = sv;
      }
    }
    if constexpr (!SCORES) {
      // V^ = f16(Cv[code] * vn_v); item = (8-dim group dg, 4-key quad kq)
      const uint32_t mv = (1u << a.vb) - 1u;
      const int shv = STREAM ? shift_of(a.vcodes, k0, vc) : 0, rpv = STREAM ? vc : vc + 4;
#pragma unroll
      for (int j = 0; j < (VITEMS + NT - 1) / NT; ++j) {
        const int it = tid + j * NT;
        if (VITEMS % NT == 0 || it < VITEMS) {
          const int kq = it % (KT / 4), dg = it / (KT / 4);
          const float4v vn4 = *reinterpret_cast<const float4v*>(&svv[cur][kq * 4]);
          half4 col[8];
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) {
            const bool real = !STREAM || dg < ng;
            const uint32_t w = real ? bits32_at(rawV[cur], shv + (kq * 4 + kk) * rpv + dg * a.vb) : 0u;
#pragma unroll
            for (int e = 0; e < 8; ++e)
              col[e][kk] = real ? static_cast<_Float16>(lutV[(w >> (e * a.vb)) & mv] * vn4[kk])
                                : static_cast<_Float16>(0.f);
          }
#pragma unroll
          for (int e = 0; e < 8; ++e)
            *reinterpret_cast<half4*>(&sVt[(dg * 8 + e) * T::LDV + kq * 4]) = col[e];
        }
      }
    }
    const bool more = k0 + KT < kend;
    if (more) fetch(k0 + KT);  // global loads in flight during this tile's math
    __syncthreads();

    // ---- S^T = K^ Q_rot^T (term 1) and Sign (Q_proj hi + lo)^T (term 2)
    float4v sacc[MBK][NBW], tacc[MBK][NBW];
#pragma unroll
    for (int mb = 0; mb < MBK; ++mb)
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        sacc[mb][nb] = float4v{0.f, 0.f, 0.f, 0.f};
        tacc[mb][nb] = float4v{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int mb = 0; mb < MBK; ++mb) {
        const int off = (mb * 16 + l16) * T::LDK + ks * 32 + lg * 8;
        const half8 ka = *reinterpret_cast<const half8*>(&sK[off]);
        const half8 sa = *reinterpret_cast<const half8*>(&sS[off]);
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) {
          sacc[mb][nb] = mfma16x16x32(ka, qr[ks][nb], sacc[mb][nb]);
          tacc[mb][nb] = mfma16x16x32(sa, qp[ks][nb], tacc[mb][nb]);
          tacc[mb][nb] = mfma16x16x32(sa, qlo[ks][nb], tacc[mb][nb]);
        }
      }
    }

    if constexpr (SCORES) {
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        if (!col_ok[nb]) continue;
        float* orow = a.scores + ((static_cast<int64_t>(b) * a.Hq + col_h[nb]) * a.Sq + col_i[nb]) * a.Sk;
#pragma unroll
        for (int mb = 0; mb < MBK; ++mb) {
          const int kk = mb * 16 + lg * 4;
          const float4v ka4 = *reinterpret_cast<const float4v*>(&skA[cur][kk]);
          const float4v kb4 = *reinterpret_cast<const float4v*>(&skB[cur][kk]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int key = k0 + kk + e;
            if (key < a.Sk) orow[key] = sacc[mb][nb][e] * ka4[e] + tacc[mb][nb][e] * kb4[e];
          }
        }
      }
    } else {
      // ---- online softmax in log2 units, lazily rescaled: a column's reference
      // maximum only moves when its running maximum grows by more than TAU, so
      // p <= 2^TAU and the accumulator is rescaled on few tiles
      const bool edge = (k0 + KT > kfull);
      half8 pb[MBK / 2][NBW], pl[MBK / 2][NBW];  // P = hi + lo (f16 pair, 2^-22 accurate)
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        float sc[MBK][4];
        float tmax = -INFINITY;
        const int lim = col_i[nb] + (a.Sk - a.Sq);
#pragma unroll
        for (int mb = 0; mb < MBK; ++mb) {
          const int kk = mb * 16 + lg * 4;
          const float4v ka4 = *reinterpret_cast<const float4v*>(&skA[cur][kk]);
          const float4v kb4 = *reinterpret_cast<const float4v*>(&skB[cur][kk]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float v = sacc[mb][nb][e] * ka4[e] + tacc[mb][nb][e] * kb4[e];
            const int key = k0 + kk + e;
            if constexpr (MASK) {
              if (col_ok[nb] && key < a.Sk)
                v += fmaxf(a.mask[b * a.smb + col_h[nb] * a.smh + static_cast<int64_t>(col_i[nb]) * a.smq +
                                  static_cast<int64_t>(key) * a.smk] * LOG2E,
                           -3.0e38f);
            }
            if (edge && (key >= a.Sk || (a.causal && key > lim))) v = -INFINITY;
            sc[mb][e] = v;
            tmax = fmaxf(tmax, v);
          }
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const bool grow = tmax > m_run[nb] + kAttnTau;
        if (__any(grow)) {
          const float m_new = grow ? tmax : m_run[nb];
          const float alpha = (m_run[nb] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run[nb] - m_new);
          m_run[nb] = m_new;
          l_run[nb] *= alpha;
#pragma unroll
          for (int db = 0; db < DB; ++db) oacc[db][nb] *= alpha;
        }
        const float m_use = (m_run[nb] == -INFINITY) ? 0.f : m_run[nb];
        float psum = 0.f;
#pragma unroll
        for (int mb = 0; mb < MBK; ++mb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float p = __builtin_amdgcn_exp2f(sc[mb][e] - m_use);
            psum += p;
            const _Float16 ph = static_cast<_Float16>(p);
            pb[mb / 2][nb][(mb & 1) * 4 + e] = ph;
            pl[mb / 2][nb][(mb & 1) * 4 + e] = static_cast<_Float16>(p - static_cast<float>(ph));
          }
        l_run[nb] += psum;
      }
      // ---- O^T += V^T P^T ; k-slots 8*lg+0..3 <-> keys 32c+4lg+0..3, 8*lg+4..7 <-> 32c+16+4lg+0..3
#pragma unroll
      for (int c = 0; c < MBK / 2; ++c) {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const int row = (db * 16 + l16) * T::LDV + c * 32 + lg * 4;
          const half8 va = cat8(*reinterpret_cast<const half4*>(&sVt[row]),
                                *reinterpret_cast<const half4*>(&sVt[row + 16]));
#pragma unroll
          for (int nb = 0; nb < NBW; ++nb) {
            oacc[db][nb] = mfma16x16x32(va, pb[c][nb], oacc[db][nb]);
            oacc[db][nb] = mfma16x16x32(va, pl[c][nb], oacc[db][nb]);
          }
        }
      }
    }
    if (more) stash(cur ^ 1);  // other buffer: last read before this tile's first barrier
    cur ^= 1;
  }

  if constexpr (!SCORES) {
    if (split_k) {  // attention mode splits only with part_o set
      // ---- split-K partial of each column: O (dims 16 db + 4 lg + e), the reference maximum
      // its weights are relative to (-inf when the split saw no finite score) and their sum
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        float l = l_run[nb];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        if (col_ok[nb]) {
          const int c = col_i[nb] * a.G + (col_h[nb] - hkv * a.G);
          const int64_t rec = (bh_kv * a.nsplit + split) * a.C + c;
          float* po = a.part_o + rec * a.dp;
#pragma unroll
          for (int db = 0; db < DB; ++db) *reinterpret_cast<float4v*>(po + db * 16 + lg * 4) = oacc[db][nb];
          if (lg == 0) {
            a.part_ml[rec * 2] = m_run[nb];
            a.part_ml[rec * 2 + 1] = l;
          }
        }
      }
      return;
    }
    // ---- normalise and rotate back: out = (O^T / l)^T Pi_v, Pi_v^T [2][d][d] as A operand
    // (rows and columns past d read as zero)
    const half4* Ph = reinterpret_cast<const half4*>(a.vpit);
    const half4* Pl = reinterpret_cast<const half4*>(a.vpit + static_cast<int64_t>(d) * d);
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) {
      float l = l_run[nb];
      l += __shfl_xor(l, 16, 64);
      l += __shfl_xor(l, 32, 64);
      const float inv_l = (l > 0.f) ? 1.f / l : 0.f;
      float mx = 0.f;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        oacc[db][nb] *= inv_l;
#pragma unroll
        for (int e = 0; e < 4; ++e) mx = fmaxf(mx, fabsf(oacc[db][nb][e]));
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      int ex;
      frexpf(mx, &ex);
      const float up = ldexpf(kSplit, -ex), down = ldexpf(kUnsplit2, ex);
      half8 bh[DB / 2], bl[DB / 2];
#pragma unroll
      for (int c = 0; c < DB / 2; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          _Float16 h, lo;
          split_f16(oacc[2 * c][nb][e] * up, h, lo);
          bh[c][e] = h;
          bl[c][e] = lo;
          split_f16(oacc[2 * c + 1][nb][e] * up, h, lo);
          bh[c][4 + e] = h;
          bl[c][4 + e] = lo;
        }
      const int qi = col_i[nb], h = col_h[nb];
#pragma unroll 1
      for (int ib = 0; ib < DB; ++ib) {
        float4v f = float4v{0.f, 0.f, 0.f, 0.f};
        const int i = ib * 16 + l16;
#pragma unroll
        for (int c = 0; c < DB / 2; ++c) {
          const int j0 = c * 32 + lg * 4;
          // d % 8 == 0: each 4-column run is all real or all padding
          const bool r0 = i < d && j0 < d, r1 = i < d && j0 + 16 < d;
          const int64_t p0 = (static_cast<int64_t>(i) * d + j0) / 4, p1 = (static_cast<int64_t>(i) * d + j0 + 16) / 4;
          const half4 z = half4{};
          const half8 ah = cat8(r0 ? Ph[p0] : z, r1 ? Ph[p1] : z);
          const half8 al = cat8(r0 ? Pl[p0] : z, r1 ? Pl[p1] : z);
          f = mfma16x16x32(ah, bh[c], f);
          f = mfma16x16x32(al, bh[c], f);
          f = mfma16x16x32(ah, bl[c], f);
        }
        const int c0 = ib * 16 + lg * 4;
        if (col_ok[nb] && c0 < d) {
          const int64_t o = static_cast<int64_t>(b) * a.sob + static_cast<int64_t>(h) * a.soh +
                            static_cast<int64_t>(qi) * a.sos + c0;
          const float4v fo = f * down;
          const int n = min(4, d - c0);
          if (a.out_dtype == TQ_BF16) store4<TQ_BF16>(a.out, o, fo, n);
          else if (a.out_dtype == TQ_F16) store4<TQ_F16>(a.out, o, fo, n);
          else store4<TQ_F32>(a.out, o, fo, n);
        }
      }
    }
  }
}

template <int D, int KB, bool SCORES, bool STREAM>
static void launch_attn_st(const AttnArgs& a, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(a.nqb) * a.Hkv * a.B),  // see the kernel
                  static_cast<unsigned>(a.nsplit > 1 ? a.nsplit : 1));
  if (!SCORES && a.mask) attn_kernel<D, KB, SCORES, !SCORES, STREAM><<<grid, ATile<D, SCORES>::NT, 0, s>>>(a);
  else attn_kernel<D, KB, SCORES, false, STREAM><<<grid, ATile<D, SCORES>::NT, 0, s>>>(a);
}
template <int D, int KB, bool SCORES>
static void launch_attn(const AttnArgs& a, hipStream_t s) {
  if (a.d == D) launch_attn_st<D, KB, SCORES, false>(a, s);
  else launch_attn_st<D, KB, SCORES, true>(a, s);
}

// the tiled kernel for head dim d: D = d rounded up to a multiple of 32
template <bool SCORES>
static void dispatch_attn(int d, int kb, const AttnArgs& a, hipStream_t s) {
#define TQ_KB_CASES(DD)                                 \
  case DD:                                              \
    if (kb == 1) launch_attn<DD, 1, SCORES>(a, s);      \
    else if (kb == 2) launch_attn<DD, 2, SCORES>(a, s); \
    else launch_attn<DD, 3, SCORES>(a, s);              \
    break;
  switch (pad_dim(d)) {
    TQ_KB_CASES(32)
    TQ_KB_CASES(64)
    TQ_KB_CASES(96)
    TQ_KB_CASES(128)
    TQ_KB_CASES(160)
    TQ_KB_CASES(192)
    TQ_KB_CASES(224)
    default: TQ_KB_CASES(256)
  }
#undef TQ_KB_CASES
}

// (query row, query head) columns per block of the tiled kernel: the largest GQA group it serves
static int block_rows(int d, bool scores) {
  switch (pad_dim(d)) {
    case 32: return scores ? ATile<32, true>::BR : ATile<32, false>::BR;
    case 64: return scores ? ATile<64, true>::BR : ATile<64, false>::BR;
    case 96: return scores ? ATile<96, true>::BR : ATile<96, false>::BR;
    case 128: return scores ? ATile<128, true>::BR : ATile<128, false>::BR;
    case 160: return scores ? ATile<160, true>::BR : ATile<160, false>::BR;
    case 192: return scores ? ATile<192, true>::BR : ATile<192, false>::BR;
    case 224: return scores ? ATile<224, true>::BR : ATile<224, false>::BR;
    default: return scores ? ATile<256, true>::BR : ATile<256, false>::BR;
  }
}

// ---------------------------------------------------------------- split-K merge, any head dim
// Combines the tiled kernel's split-K partials (rows of DP floats, DP = 64, 128 or 256 >= the
// padded head dim) with log-sum-exp weights and applies Pi_v (Pi_v^T [2][d][d] split f16,
// rows and columns past d read as zero) on MFMA, hi.hi + lo.hi + hi.lo.  One block per (kv
// head, batch, group of 4 columns); wave w combines column 4 blockIdx.z + w (PL = DP / 64 dims
// per lane, the loads of 16 splits issued together), then owns output row blocks
// NRB w .. NRB w + NRB - 1 of the product.  Latency-bound like the head_dim-128 merge.
struct SplitMergeArgs {
  const float *part_o, *part_ml;
  const uint16_t* vpit;
  int B, Hq, Hkv, Sq, G, C, nsplit, d, dpad;
  void* out;
  int out_dtype;
  int64_t sob, soh, sos;
};

template <int DP>
__global__ void __launch_bounds__(256) attn_merge_kernel(SplitMergeArgs a) {
  static_assert(DP == 64 || DP == 128 || DP == 256, "partial rows of 64, 128 or 256 floats");
  constexpr int PL = DP / 64;    // dims per lane in the combine
  constexpr int NRB = DP / 64;   // 16-row output blocks per wave
  constexpr int KS = DP / 32;    // k-steps of the product
  constexpr int NB = 16;         // splits per load batch
  constexpr int SW = 64;         // splits per weight batch (one per lane)
  __shared__ __attribute__((aligned(16))) float o_s[4][DP];
  __shared__ float s_w[4][SW];
  __shared__ float s_up[4];
  const int hkv = blockIdx.x, b = blockIdx.y, c0 = blockIdx.z * 4, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, l16 = lane & 15, lg = lane >> 4;
  const int C = a.C, ns = a.nsplit, d = a.d;
  const int64_t base = (static_cast<int64_t>(b) * a.Hkv + hkv) * ns;
  typedef float floatPL __attribute__((ext_vector_type(PL)));

  // ---- column c = c0 + wave: o = sum_s w_s o_s / sum_s w_s l_s
  {
    const int c = c0 + wave;
    float* oc = o_s[wave];
    if (c >= C) {
#pragma unroll
      for (int e = 0; e < PL; ++e) oc[PL * lane + e] = 0.f;
      if (lane == 0) s_up[wave] = 1.f;
    } else {
      auto ml = [&](int sp, int k) { return a.part_ml[((base + sp) * C + c) * 2 + k]; };
      const int64_t step = static_cast<int64_t>(C) * DP;
      const float* src0 = a.part_o + (base * C + c) * DP + PL * lane;
      const bool real = PL * lane < a.dpad;  // dims past the padded head dim are not written
      auto load = [&](int sp) {
        floatPL v;
        if (real) {
          v = *reinterpret_cast<const floatPL*>(src0 + sp * step);
        } else {
#pragma unroll
          for (int e = 0; e < PL; ++e) v[e] = 0.f;
        }
        return v;
      };
      floatPL v0[NB];
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        if (u < ns) {
          v0[u] = load(u);
        } else {
#pragma unroll
          for (int e = 0; e < PL; ++e) v0[u][e] = 0.f;
        }
      }
      const float m_first = lane < ns ? ml(lane, 0) : -INFINITY;
      const float l_first = lane < ns ? ml(lane, 1) : 0.f;
      float mx = m_first;
      for (int sp = lane + SW; sp < ns; sp += SW) mx = fmaxf(mx, ml(sp, 0));
#pragma unroll
      for (int sh = 32; sh >= 1; sh >>= 1) mx = fmaxf(mx, __shfl_xor(mx, sh, 64));
      float lsum = 0.f;
      float o[PL];
#pragma unroll
      for (int e = 0; e < PL; ++e) o[e] = 0.f;
      for (int s0 = 0; s0 < ns; s0 += SW) {
        const int sp = s0 + lane;
        float w = 0.f;
        if (sp < ns) {
          const float m = s0 == 0 ? m_first : ml(sp, 0);
          w = (m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - mx);
          lsum += w * (s0 == 0 ? l_first : ml(sp, 1));
        }
        s_w[wave][lane] = w;  // read back by the same wave only: LDS order suffices
        const int nb = min(SW, ns - s0);
        int k = 0;
        if (s0 == 0) {
#pragma unroll
          for (int u = 0; u < NB; ++u) {
            const float ww = u < nb ? s_w[wave][u] : 0.f;
#pragma unroll
            for (int e = 0; e < PL; ++e) o[e] = fmaf(ww, v0[u][e], o[e]);
          }
          k = min(NB, nb);
        }
        for (; k < nb; k += NB) {
          floatPL v[NB];
#pragma unroll
          for (int u = 0; u < NB; ++u) {
            if (k + u < nb) {
              v[u] = load(s0 + k + u);
            } else {
#pragma unroll
              for (int e = 0; e < PL; ++e) v[u][e] = 0.f;
            }
          }
#pragma unroll
          for (int u = 0; u < NB; ++u) {
            const float ww = k + u < nb ? s_w[wave][k + u] : 0.f;
#pragma unroll
            for (int e = 0; e < PL; ++e) o[e] = fmaf(ww, v[u][e], o[e]);
          }
        }
      }
#pragma unroll
      for (int sh = 32; sh >= 1; sh >>= 1) lsum += __shfl_xor(lsum, sh, 64);
      const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
      float m = 0.f;
#pragma unroll
      for (int e = 0; e < PL; ++e) {
        o[e] *= inv;
        oc[PL * lane + e] = o[e];
        m = fmaxf(m, fabsf(o[e]));
      }
#pragma unroll
      for (int sh = 32; sh >= 1; sh >>= 1) m = fmaxf(m, __shfl_xor(m, sh, 64));
      if (lane == 0) {
        int ex;
        frexpf(m, &ex);
        s_up[wave] = ldexpf(kSplit, -ex);  // scaled |o| < kSplit
      }
    }
  }
  __syncthreads();

  // ---- out^T[i][c] = sum_j Pi_v^T[i][j] o[c][j]; MFMA column l16 < 4 is column c0 + l16
  const float up = s_up[l16 & 3];
  half8 bh[KS], bl[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const float* src = o_s[l16 & 3] + ks * 32 + lg * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      _Float16 hh, lo;
      split_f16(src[e] * up, hh, lo);
      bh[ks][e] = hh;
      bl[ks][e] = lo;
    }
  }
  const bool col_ok = l16 < 4 && c0 + l16 < C;
  const int qi = col_ok ? (c0 + l16) / a.G : 0, h = hkv * a.G + (col_ok ? (c0 + l16) % a.G : 0);
  const float down = kUnsplit2 / up;
  const _Float16* Ph = reinterpret_cast<const _Float16*>(a.vpit);
  const _Float16* Pl = Ph + static_cast<int64_t>(d) * d;
#pragma unroll
  for (int r = 0; r < NRB; ++r) {
    const int i = (wave * NRB + r) * 16 + l16;
    float4v f = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int j0 = ks * 32 + lg * 8;
      const bool ok = i < d && j0 < d;  // d % 8 == 0: the 8 columns from j0 are all real or all padding
      const int64_t pofs = static_cast<int64_t>(i) * d + j0;
      const half8 ah = ok ? *reinterpret_cast<const half8*>(Ph + pofs) : half8{};
      const half8 al = ok ? *reinterpret_cast<const half8*>(Pl + pofs) : half8{};
      f = mfma16x16x32(ah, bh[ks], f);
      f = mfma16x16x32(al, bh[ks], f);
      f = mfma16x16x32(ah, bl[ks], f);
    }
    const int row0 = (wave * NRB + r) * 16 + lg * 4;
    if (col_ok && row0 < d) {
      const int64_t off = static_cast<int64_t>(b) * a.sob + static_cast<int64_t>(h) * a.soh +
                          static_cast<int64_t>(qi) * a.sos + row0;
      const float4v fo = f * (down * kSplit);
      const int n = min(4, d - row0);
      if (a.out_dtype == TQ_BF16) store4<TQ_BF16>(a.out, off, fo, n);
      else if (a.out_dtype == TQ_F16) store4<TQ_F16>(a.out, off, fo, n);
      else store4<TQ_F32>(a.out, off, fo, n);
    }
  }
}

// Split-K plan of the tiled kernel for few query rows per kv head (one query block) over long
// key ranges: about kSplitBlocks blocks (two resident per CU), splits of whole 32-key tiles and
// at least kSplitMinKeys keys each.  Not used when the split-K decode kernels apply.
constexpr int kSplitBlocks = 512;
constexpr int kSplitMinKeys = 256;
struct SplitPlan {
  int nsplit = 0, chunk = 0, dp = 0;
  int64_t bytes = 0;
};
static int split_row_floats(int d) {
  const int dpad = pad_dim(d);
  return dpad <= 64 ? 64 : (dpad <= 128 ? 128 : 256);
}
static SplitPlan tiled_split_plan(int B, int Hq, int Hkv, int Sq, int Sk, int d, bool scores = false) {
  SplitPlan p;
  if (!supported_dim(d) || Hkv <= 0 || Hq % Hkv || B <= 0 || Sq <= 0) return p;
  const int G = Hq / Hkv;
  const int64_t cols = block_rows(d, scores);
  if (static_cast<int64_t>(G) * Sq > cols) return p;  // one query block per kv head
  if (Sk < 2 * kSplitMinKeys) return p;
  const int64_t groups = static_cast<int64_t>(B) * Hkv;
  int64_t ns = (kSplitBlocks + groups - 1) / groups;
  const int64_t max_split = Sk / kSplitMinKeys;
  if (ns > max_split) ns = max_split;
  if (ns > 1024) ns = 1024;
  if (ns < 2) return p;
  int chunk = static_cast<int>((Sk + ns - 1) / ns);
  chunk = (chunk + kAttnKeys - 1) / kAttnKeys * kAttnKeys;
  p.nsplit = (Sk + chunk - 1) / chunk;
  if (p.nsplit < 2) return SplitPlan{};
  p.chunk = chunk;
  p.dp = split_row_floats(d);
  const int64_t C = static_cast<int64_t>(G) * Sq;
  p.bytes = groups * p.nsplit * C * (p.dp + 2) * 4;
  return p;
}

static void launch_split_merge(const SplitMergeArgs& m, int dp, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(m.Hkv), static_cast<unsigned>(m.B), static_cast<unsigned>((m.C + 3) / 4));
  if (dp == 64) attn_merge_kernel<64><<<grid, 256, 0, s>>>(m);
  else if (dp == 128) attn_merge_kernel<128><<<grid, 256, 0, s>>>(m);
  else attn_merge_kernel<256><<<grid, 256, 0, s>>>(m);
}

int merge_key_splits(const float* part_o, const float* part_ml, const uint16_t* vpit, int B, int Hq, int Hkv,
                     int Sq, int C, int nsplit, int d, void* out, int out_dtype, int64_t sob, int64_t soh,
                     int64_t sos, hipStream_t s) {
  SplitMergeArgs m{};
  m.part_o = part_o;
  m.part_ml = part_ml;
  m.vpit = vpit;
  m.B = B;
  m.Hq = Hq;
  m.Hkv = Hkv;
  m.Sq = Sq;
  m.G = Hq / Hkv;
  m.C = C;
  m.nsplit = nsplit;
  m.d = d;
  m.dpad = pad_dim(d);
  m.out = out;
  m.out_dtype = out_dtype;
  m.sob = sob;
  m.soh = soh;
  m.sos = sos;
  launch_split_merge(m, split_row_floats(d), s);
  return launch_status("tq_attention_fwd (split merge)");
}

}  // namespace tq

using namespace tq;

namespace tq {
int64_t decode_workspace_bytes(int B, int Hq, int Hkv, int Sq, int Sk, int d, int bits);
bool decode_applies(int B, int Hq, int Hkv, int Sq, int Sk, int d, int bits);
bool prefill_applies(int Hq, int Hkv, int d, int bits, int val_bits, bool masked);
bool prefill_split_applies(int Hq, int Hkv, int Sq, int d, int bits, int val_bits, bool masked);
int prefill_attention(int64_t ldk, const uint16_t* q_rot, const float* q_proj, const uint8_t* kcodes,
                      const uint8_t* ksigns, const uint16_t* krn, const uint16_t* kvn, const uint16_t* kcent,
                      int bits, const uint8_t* vcodes, const uint16_t* vvn, const float* vcent,
                      const uint16_t* vpit, int B, int Hq, int Hkv, int Sq, int Sk, int d, float coeff, float scale,
                      int causal, const float* mask, int64_t smb, int64_t smh, int64_t smq, int64_t smk, void* out,
                      int out_dtype, int64_t sob, int64_t soh, int64_t sos, hipStream_t s, float* part_o = nullptr,
                      float* part_ml = nullptr, int nsplit = 0, int chunk = 0, int C = 0, int dp = 0);
int decode_scores(int64_t ldk, const uint16_t* q_rot, const float* q_proj, const uint8_t* kcodes,
                  const uint8_t* ksigns, const uint16_t* krn, const uint16_t* kvn, const uint16_t* kcent,
                  int B, int Hq, int Hkv, int Sq, int Sk, int d, int bits, float coeff, float* out,
                  hipStream_t s);
int decode_attention(int64_t ldk, const uint16_t* q_rot, const float* q_proj, const uint8_t* kcodes,
                     const uint8_t* ksigns, const uint16_t* krn, const uint16_t* kvn, const uint16_t* kcent,
                     int bits, const uint8_t* vcodes, const uint16_t* vvn, const float* vcent32,
                     const uint16_t* vpit, int B, int Hq, int Hkv, int Sq, int Sk, int d, float coeff,
                     float scale, int causal, const float* mask, int64_t smb, int64_t smh, int64_t smq,
                     int64_t smk, void* out, int out_dtype, int64_t sob, int64_t soh, int64_t sos,
                     void* workspace, hipStream_t s);
}  // namespace tq

static int check_common(const char* what, int32_t B, int32_t Hq, int32_t Hkv, int32_t Sq, int32_t Sk,
                        int32_t d, int32_t bits) {
  if (!supported_dim(d)) {
    set_error("%s: head_dim %d not supported (multiples of 8 from 8 to 256)", what, (int)d);
    return TQ_EUNSUPPORTED;
  }
  TQ_REQUIRE(bits >= 2 && bits <= 4, "%s: key bits must be in [2, 4], got %d", what, (int)bits);
  TQ_REQUIRE(B >= 0 && Hq >= 0 && Hkv >= 1 && Sq >= 0 && Sk >= 0, "%s: bad shape", what);
  TQ_REQUIRE(Hq % Hkv == 0, "%s: Hq=%d is not a multiple of Hkv=%d", what, (int)Hq, (int)Hkv);
  return TQ_OK;
}

// the tiled kernel serves GQA groups of at most block_rows(d, scores) query heads
static int check_group(const char* what, int32_t Hq, int32_t Hkv, int32_t d, bool scores) {
  TQ_REQUIRE(Hq / Hkv <= block_rows(d, scores), "%s: group size %d exceeds %d at head_dim %d", what,
             (int)(Hq / Hkv), block_rows(d, scores), (int)d);
  return TQ_OK;
}

static void fill_common(AttnArgs& a, int32_t B, int32_t Hq, int32_t Hkv, int32_t Sq, int32_t Sk, int64_t ldk,
                        int32_t d, bool scores) {
  a.d = d;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.Sq = Sq;
  a.Sk = Sk;
  a.ldk = ldk;
  a.G = Hq / Hkv;
  a.QT = block_rows(d, scores) / a.G;
  a.nqb = (Sq + a.QT - 1) / a.QT;
}

extern "C" {

int64_t tq_attention_workspace_size(int32_t B, int32_t Hq, int32_t Hkv, int32_t Sq, int32_t Sk, int32_t d,
                                    int32_t bits) {
  // the split-K decode kernels' partials, or the tiled kernel's split over keys (value bits
  // other than the key bits, head dims other than 128, larger groups): enough for either
  const int64_t dec = decode_workspace_bytes(B, Hq, Hkv, Sq, Sk, d, bits);
  const int64_t til = tiled_split_plan(B, Hq, Hkv, Sq, Sk, d).bytes;
  return dec > til ? dec : til;
}

int tq_attention_scores_kv(const uint16_t* q_rot, const float* q_proj, const uint8_t* key_codes,
                           const uint8_t* key_signs, const uint16_t* key_rn, const uint16_t* key_vn,
                           const uint16_t* centroids_f16, int32_t B, int32_t Hq, int32_t Hkv, int32_t Sq,
                           int32_t Sk, int64_t kv_stride, int32_t d, int32_t bits, float coeff, float* out,
                           void* stream) {
  int st = check_common("tq_attention_scores", B, Hq, Hkv, Sq, Sk, d, bits);
  if (st != TQ_OK) return st;
  const int64_t ldk = kv_stride > 0 ? kv_stride : Sk;
  TQ_REQUIRE(ldk >= Sk, "tq_attention_scores: kv_stride %lld < Sk %d", (long long)kv_stride, (int)Sk);
  if (static_cast<int64_t>(B) * Hq * Sq * Sk == 0) return TQ_OK;
  TQ_REQUIRE(q_rot && q_proj && key_codes && key_signs && key_rn && key_vn && centroids_f16 && out,
             "tq_attention_scores: null pointer");
  if (decode_applies(B, Hq, Hkv, Sq, Sk, d, bits))
    return decode_scores(ldk, q_rot, q_proj, key_codes, key_signs, key_rn, key_vn, centroids_f16, B, Hq, Hkv,
                         Sq, Sk, d, bits, coeff, out, as_stream(stream));
  st = check_group("tq_attention_scores", Hq, Hkv, d, true);
  if (st != TQ_OK) return st;
  AttnArgs a{};
  a.q_rot = q_rot;
  a.q_proj = q_proj;
  a.kcodes = key_codes;
  a.ksigns = key_signs;
  a.krn = key_rn;
  a.kvn = key_vn;
  a.kcent = centroids_f16;
  a.vb = 1;
  fill_common(a, B, Hq, Hkv, Sq, Sk, ldk, d, true);
  TQ_REQUIRE(static_cast<int64_t>(a.nqb) * Hkv * B < (int64_t(1) << 31), "%s: %lld query blocks exceed one grid",
             "tq_attention", (long long)(static_cast<int64_t>(a.nqb) * Hkv * B));
  a.coeff = coeff;
  a.scale = 1.f;
  a.scores = out;
  // few query rows per kv head over a long key range: blocks split the keys (each writes its
  // own keys' scores, nothing to merge)
  const SplitPlan sp = tiled_split_plan(B, Hq, Hkv, Sq, Sk, d, true);
  if (sp.nsplit > 1) {
    a.nsplit = sp.nsplit;
    a.chunk = sp.chunk;
  }
  dispatch_attn<true>(d, bits - 1, a, as_stream(stream));
  return launch_status("tq_attention_scores");
}

int tq_attention_fwd_kv(const uint16_t* q_rot, const float* q_proj, const uint8_t* key_codes,
                        const uint8_t* key_signs, const uint16_t* key_rn, const uint16_t* key_vn,
                        const uint16_t* key_centroids_f16, int32_t bits, const uint8_t* val_codes,
                        const uint16_t* val_vn, const float* val_centroids, int32_t val_bits,
                        const uint16_t* val_pit_split, int32_t B, int32_t Hq, int32_t Hkv, int32_t Sq,
                        int32_t Sk, int64_t kv_stride, int32_t d, float coeff, float scale, int32_t causal,
                        const float* mask, int64_t smb, int64_t smh, int64_t smq, int64_t smk,
                        void* out, int32_t out_dtype, int64_t sob, int64_t soh, int64_t sos,
                        void* workspace, int64_t workspace_bytes, void* stream) {
  int st = check_common("tq_attention_fwd", B, Hq, Hkv, Sq, Sk, d, bits);
  if (st != TQ_OK) return st;
  const int64_t ldk = kv_stride > 0 ? kv_stride : Sk;
  TQ_REQUIRE(ldk >= Sk, "tq_attention_fwd: kv_stride %lld < Sk %d", (long long)kv_stride, (int)Sk);
  TQ_REQUIRE(val_bits >= 1 && val_bits <= 4, "tq_attention_fwd: value bits must be in [1, 4], got %d",
             (int)val_bits);
  TQ_REQUIRE(out_dtype == TQ_F32 || out_dtype == TQ_F16 || out_dtype == TQ_BF16,
             "tq_attention_fwd: unknown out dtype %d", (int)out_dtype);
  TQ_REQUIRE(!causal || Sk >= Sq, "tq_attention_fwd: causal needs Sk >= Sq");
  if (static_cast<int64_t>(B) * Hq * Sq == 0) return TQ_OK;
  TQ_REQUIRE(q_rot && q_proj && val_pit_split && out && key_centroids_f16 && val_centroids,
             "tq_attention_fwd: null pointer");
  TQ_REQUIRE(Sk == 0 || (key_codes && key_signs && key_rn && key_vn && val_codes && val_vn),
             "tq_attention_fwd: null key/value plane");
  const int64_t need = decode_workspace_bytes(B, Hq, Hkv, Sq, Sk, d, bits);
  if (need > 0 && val_bits == bits && workspace && workspace_bytes >= need)
    return decode_attention(ldk, q_rot, q_proj, key_codes, key_signs, key_rn, key_vn, key_centroids_f16, bits,
                            val_codes, val_vn, val_centroids, val_pit_split, B, Hq, Hkv, Sq, Sk, d, coeff,
                            scale, causal, mask, smb, smh, smq, smk, out, out_dtype, sob, soh, sos,
                            workspace, as_stream(stream));
  // few query rows per kv head over a long key range: the tiled kernel split over keys, then a
  // merge (the decode kernels above take head_dim 64 / 128 with at most 16 columns and key
  // bits = value bits)
  const SplitPlan sp = tiled_split_plan(B, Hq, Hkv, Sq, Sk, d);
  const bool split = sp.nsplit > 0 && workspace && workspace_bytes >= sp.bytes &&
                     reinterpret_cast<uintptr_t>(workspace) % 16 == 0;
  auto merge_split = [&](float* part_o, float* part_ml, int C) {
    return merge_key_splits(part_o, part_ml, val_pit_split, B, Hq, Hkv, Sq, C, sp.nsplit, d, out, out_dtype, sob,
                            soh, sos, as_stream(stream));
  };
  if (split && prefill_split_applies(Hq, Hkv, Sq, d, bits, val_bits, mask != nullptr)) {
    // head_dim 64 / 128: the prefill kernel split over keys
    const int C = (Hq / Hkv) * Sq;
    float* part_o = static_cast<float*>(workspace);
    float* part_ml = part_o + static_cast<int64_t>(B) * Hkv * sp.nsplit * C * sp.dp;
    st = prefill_attention(ldk, q_rot, q_proj, key_codes, key_signs, key_rn, key_vn, key_centroids_f16, bits,
                           val_codes, val_vn, val_centroids, val_pit_split, B, Hq, Hkv, Sq, Sk, d, coeff, scale,
                           causal, mask, smb, smh, smq, smk, out, out_dtype, sob, soh, sos, as_stream(stream), part_o,
                           part_ml, sp.nsplit, sp.chunk, C, sp.dp);
    if (st != TQ_OK) return st;
    return merge_split(part_o, part_ml, C);
  }
  if (!split && prefill_applies(Hq, Hkv, d, bits, val_bits, mask != nullptr))
    return prefill_attention(ldk, q_rot, q_proj, key_codes, key_signs, key_rn, key_vn, key_centroids_f16, bits,
                             val_codes, val_vn, val_centroids, val_pit_split, B, Hq, Hkv, Sq, Sk, d, coeff, scale,
                             causal, mask, smb, smh, smq, smk, out, out_dtype, sob, soh, sos, as_stream(stream));
  st = check_group("tq_attention_fwd", Hq, Hkv, d, false);
  if (st != TQ_OK) return st;
  AttnArgs a{};
  a.q_rot = q_rot;
  a.q_proj = q_proj;
  a.kcodes = key_codes;
  a.ksigns = key_signs;
  a.krn = key_rn;
  a.kvn = key_vn;
  a.kcent = key_centroids_f16;
  a.vcodes = val_codes;
  a.vvn = val_vn;
  a.vcent32 = val_centroids;
  a.vpit = val_pit_split;
  a.vb = val_bits;
  fill_common(a, B, Hq, Hkv, Sq, Sk, ldk, d, false);
  TQ_REQUIRE(static_cast<int64_t>(a.nqb) * Hkv * B < (int64_t(1) << 31), "%s: %lld query blocks exceed one grid",
             "tq_attention", (long long)(static_cast<int64_t>(a.nqb) * Hkv * B));
  a.coeff = coeff;
  a.scale = scale;
  a.causal = causal;
  a.mask = mask;
  a.smb = smb;
  a.smh = smh;
  a.smq = smq;
  a.smk = smk;
  a.out = out;
  a.out_dtype = out_dtype;
  a.sob = sob;
  a.soh = soh;
  a.sos = sos;
  if (split) {
    const int C = (Hq / Hkv) * Sq;
    const int64_t n_part = static_cast<int64_t>(B) * Hkv * sp.nsplit * C;
    a.part_o = static_cast<float*>(workspace);
    a.part_ml = a.part_o + n_part * sp.dp;
    a.nsplit = sp.nsplit;
    a.chunk = sp.chunk;
    a.C = C;
    a.dp = sp.dp;
  }
  dispatch_attn<false>(d, bits - 1, a, as_stream(stream));
  if (!split) return launch_status("tq_attention_fwd");
  st = launch_status("tq_attention_fwd (keys split)");
  if (st != TQ_OK) return st;
  return merge_split(a.part_o, a.part_ml, a.C);
}

}  // extern "C"

// ---------------------------------------------------------------- allocation-free variant
// The split-K decode partials of tq_attention_fwd_kv_noalloc live in this array, one copy
// per GPU, held until the process ends.  Host code never passes `scratch` itself to a
// kernel (in host code the name is a host-side stand-in, not a device address): the
// device address comes from hipGetSymbolAddress, once per device, with that device current.
namespace {
constexpr int64_t kScratchBytes = TQ_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// device address of this GPU's scratch array (nullptr after setting the error message)
void* device_scratch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("tq_attention_fwd_kv_noalloc: no current HIP device (or device index >= %d)", kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("tq_attention_fwd_kv_noalloc: hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" {

int64_t tq_noalloc_scratch_bytes(void) { return kScratchBytes; }

int tq_attention_fwd_kv_noalloc(const uint16_t* q_rot, const float* q_proj, const uint8_t* key_codes,
                                const uint8_t* key_signs, const uint16_t* key_rn, const uint16_t* key_vn,
                                const uint16_t* key_centroids_f16, int32_t bits, const uint8_t* val_codes,
                                const uint16_t* val_vn, const float* val_centroids, int32_t val_bits,
                                const uint16_t* val_pit_split, int32_t B, int32_t Hq, int32_t Hkv, int32_t Sq,
                                int32_t Sk, int64_t kv_stride, int32_t d, float coeff, float scale,
                                int32_t causal, const float* mask, int64_t smb, int64_t smh, int64_t smq,
                                int64_t smk, void* out, int32_t out_dtype, int64_t sob, int64_t soh,
                                int64_t sos, void* stream) {
  int st = check_common("tq_attention_fwd_kv_noalloc", B, Hq, Hkv, Sq, Sk, d, bits);
  if (st != TQ_OK) return st;
  void* ws = nullptr;
  int64_t ws_bytes = 0;
  const int64_t dec = (val_bits == bits && static_cast<int64_t>(B) * Hq * Sq > 0)
                          ? decode_workspace_bytes(B, Hq, Hkv, Sq, Sk, d, bits) : 0;
  if (dec > 0) {
    TQ_REQUIRE(dec <= kScratchBytes,
               "tq_attention_fwd_kv_noalloc: this shape's split-K partials need %lld bytes, more than the "
               "%lld-byte scratch array; use tq_attention_fwd_kv with a caller workspace",
               (long long)dec, (long long)kScratchBytes);
    ws = device_scratch();
    if (!ws) return TQ_EHIP;
    ws_bytes = dec;
  } else if (static_cast<int64_t>(B) * Hq * Sq > 0) {
    // the tiled kernel's split over keys when its partials fit the array; otherwise it runs
    // unsplit (no workspace), which needs none
    const int64_t til = tiled_split_plan(B, Hq, Hkv, Sq, Sk, d).bytes;
    if (til > 0 && til <= kScratchBytes) {
      ws = device_scratch();
      if (!ws) return TQ_EHIP;
      ws_bytes = til;
    }
  }
  // every split record is written in full before the merge reads it: nothing to clear
  return tq_attention_fwd_kv(q_rot, q_proj, key_codes, key_signs, key_rn, key_vn, key_centroids_f16, bits,
                             val_codes, val_vn, val_centroids, val_bits, val_pit_split, B, Hq, Hkv, Sq, Sk,
                             kv_stride, d, coeff, scale, causal, mask, smb, smh, smq, smk, out, out_dtype, sob,
                             soh, sos, ws, ws_bytes, stream);
}

int tq_attention_scores(const uint16_t* q_rot, const float* q_proj, const uint8_t* key_codes,
                        const uint8_t* key_signs, const uint16_t* key_rn, const uint16_t* key_vn,
                        const uint16_t* centroids_f16, int32_t B, int32_t Hq, int32_t Hkv, int32_t Sq,
                        int32_t Sk, int32_t d, int32_t bits, float coeff, float* out, void* stream) {
  return tq_attention_scores_kv(q_rot, q_proj, key_codes, key_signs, key_rn, key_vn, centroids_f16, B, Hq, Hkv,
                                Sq, Sk, Sk, d, bits, coeff, out, stream);
}

int tq_attention_fwd(const uint16_t* q_rot, const float* q_proj, const uint8_t* key_codes,
                     const uint8_t* key_signs, const uint16_t* key_rn, const uint16_t* key_vn,
                     const uint16_t* key_centroids_f16, int32_t bits, const uint8_t* val_codes,
                     const uint16_t* val_vn, const float* val_centroids, int32_t val_bits,
                     const uint16_t* val_pit_split, int32_t B, int32_t Hq, int32_t Hkv, int32_t Sq,
                     int32_t Sk, int32_t d, float coeff, float scale, int32_t causal,
                     const float* mask, int64_t smb, int64_t smh, int64_t smq, int64_t smk,
                     void* out, int32_t out_dtype, int64_t sob, int64_t soh, int64_t sos,
                     void* workspace, int64_t workspace_bytes, void* stream) {
  return tq_attention_fwd_kv(q_rot, q_proj, key_codes, key_signs, key_rn, key_vn, key_centroids_f16, bits,
                             val_codes, val_vn, val_centroids, val_bits, val_pit_split, B, Hq, Hkv, Sq, Sk, Sk, d,
                             coeff, scale, causal, mask, smb, smh, smq, smk, out, out_dtype, sob, soh, sos,
                             workspace, workspace_bytes, stream);
}

}  // extern "C"
