// Compressed-domain attention on gfx950: asymmetric scores from packed keys,
// online softmax, and P.V over packed values, in one kernel.
//
// Scores follow the reference estimator (kernels/attention.py:380-461,
// compressors.py:178-200):
//   s(q, k) = vn_k * <q_rot, Ck[codes_k]> + coeff * rn_k * <q_proj, 2*sign_k - 1>
// with q_rot = f16(q Pi^T) and q_proj = f16(q_rot S_eff^T) from tq_query_prep.
// Both inner products run as v_mfma_f32_16x16x32_f16 with the decoded key
// operands (f16 centroids, +-1 signs) exact in f16, so term 1 is exactly the
// reference's f32 accumulation of f16 products.
//
// Work decomposition: a block of 4 wave64 owns one (batch, kv head) and BR
// (query row, query head) pairs -- all G = Hq/Hkv heads of the group share each
// decoded key tile (the reference expands K/V with repeat_interleave instead,
// families/qwen2.py:101-102).  Per key tile of KT keys the block stages the
// packed planes in LDS with dword loads, decodes keys once into f16 tiles
// (K^, sign, V^T), and each wave computes S^T = K^ Q^T for its 16..32 columns.
// S^T's accumulator layout (4 consecutive keys of one column per lane) is
// exactly the B-operand layout P^T needs for O^T += V^T P^T, so P never leaves
// registers.  Values stay in the rotated domain: O = (sum_j p_j vn_j Cv[c_j]) Pi_v,
// with the final Pi_v applied once per query row (f16 hi/lo split MFMA).
#include "tq_common.h"

namespace tq {

template <int D>
struct ATile {
  static constexpr int KT = (D == 256) ? 32 : 64;   // keys per tile
  static constexpr int NBW = (D == 256) ? 1 : 2;    // 16-column blocks per wave
  static constexpr int BR = 4 * 16 * NBW;           // (query, head) rows per block
  static constexpr int KS = D / 32;                 // k-steps of the score MFMAs
  static constexpr int MBK = KT / 16;               // 16-key blocks per tile
  static constexpr int DB = D / 16;                 // 16-dim blocks
  static constexpr int LDK = D + 8;                 // padded f16 row stride of K^ / sign tiles
  static constexpr int LDV = KT + 8;                // padded f16 row stride of V^T tile
  static constexpr int KC_MAX = D * 3 / 8;          // key code bytes/row (bits <= 4)
  static constexpr int VC_MAX = D * 4 / 8;          // value code bytes/row (bits <= 4)
};

struct AttnArgs {
  const uint16_t *q_rot, *q_proj;
  const uint8_t *kcodes, *ksigns;
  const uint16_t *krn, *kvn, *kcent;
  int kb;
  const uint8_t* vcodes;
  const uint16_t *vvn, *vcent, *vpit;
  int vb;
  int B, Hq, Hkv, Sq, Sk, G, QT, nqb;
  float coeff, scale;
  int causal;
  const float* mask;
  int64_t smb, smh, smq, smk;
  void* out;
  int64_t sob, soh, sos;
  float* scores;  // scores-only mode output f32 [B, Hq, Sq, Sk]
};

__device__ __forceinline__ half8 cat8(half4 a, half4 b) {
  return half8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// 8 codes of `bits` bits starting at a byte boundary (little endian bytes).
__device__ __forceinline__ uint64_t load_group(const uint8_t* p, int bits) {
  uint64_t w = 0;
  for (int i = 0; i < bits; ++i) w |= static_cast<uint64_t>(p[i]) << (8 * i);
  return w;
}

template <int D, int DT, bool SCORES>
__global__ void __launch_bounds__(256) attn_kernel(AttnArgs a) {
  using T = ATile<D>;
  constexpr int KT = T::KT, NBW = T::NBW, KS = T::KS, MBK = T::MBK, DB = T::DB;
  __shared__ _Float16 sK[KT * T::LDK];
  __shared__ _Float16 sS[KT * T::LDK];
  __shared__ _Float16 sVt[SCORES ? 1 : D * T::LDV];
  __shared__ uint32_t rawK[KT * T::KC_MAX / 4];
  __shared__ uint32_t rawS[KT * D / 32];
  __shared__ uint32_t rawV[SCORES ? 1 : KT * T::VC_MAX / 4];
  __shared__ _Float16 lutK[8], lutV[16];
  __shared__ float skv[KT], skr[KT], svv[KT];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const int qblk = a.nqb - 1 - static_cast<int>(blockIdx.x);  // heavy causal blocks first
  const int hkv = blockIdx.y, b = blockIdx.z;
  const int q0 = qblk * a.QT;
  const int kc = D * a.kb / 8, vc = D * a.vb / 8;
  const int64_t bh_kv = static_cast<int64_t>(b) * a.Hkv + hkv;

  if (tid < (1 << a.kb)) lutK[tid] = __builtin_bit_cast(_Float16, a.kcent[tid]);
  if (!SCORES && tid < (1 << a.vb)) lutV[tid] = __builtin_bit_cast(_Float16, a.vcent[tid]);

  // ---- this lane's columns: (query position, head) and its q fragments
  int col_i[NBW], col_h[NBW];
  bool col_ok[NBW];
  half8 qr[KS][NBW], qp[KS][NBW];
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
    const int r = (wave * NBW + nb) * 16 + l16;
    const int ql = r / a.G, gi = r % a.G;
    col_i[nb] = q0 + ql;
    col_h[nb] = hkv * a.G + gi;
    col_ok[nb] = (ql < a.QT) && (col_i[nb] < a.Sq);
    const int64_t qrow = ((static_cast<int64_t>(b) * a.Hq + col_h[nb]) * a.Sq + col_i[nb]) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d0 = ks * 32 + lg * 8;
      if (col_ok[nb]) {
        qr[ks][nb] = *reinterpret_cast<const half8*>(a.q_rot + qrow + d0);
        qp[ks][nb] = *reinterpret_cast<const half8*>(a.q_proj + qrow + d0);
      } else {
        qr[ks][nb] = half8{};
        qp[ks][nb] = half8{};
      }
    }
  }

  // key range this block needs
  int kend = a.Sk;
  if (a.causal) {
    const int imax = min(q0 + a.QT - 1, a.Sq - 1);
    kend = min(a.Sk, imax + (a.Sk - a.Sq) + 1);
  }

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
  constexpr float LOG2E = 1.4426950408889634f;

  for (int k0 = 0; k0 < kend; k0 += KT) {
    const int nk = min(KT, a.Sk - k0);
    __syncthreads();  // previous tile fully consumed
    // ---- stage packed planes (dword loads; rows are 4-byte aligned)
    {
      const uint32_t* gk = reinterpret_cast<const uint32_t*>(a.kcodes + (bh_kv * a.Sk + k0) * kc);
      for (int w = tid; w < nk * kc / 4; w += 256) rawK[w] = gk[w];
      const uint32_t* gs = reinterpret_cast<const uint32_t*>(a.ksigns + (bh_kv * a.Sk + k0) * (D / 8));
      for (int w = tid; w < nk * D / 32; w += 256) rawS[w] = gs[w];
      if constexpr (!SCORES) {
        const uint32_t* gv = reinterpret_cast<const uint32_t*>(a.vcodes + (bh_kv * a.Sk + k0) * vc);
        for (int w = tid; w < nk * vc / 4; w += 256) rawV[w] = gv[w];
      }
      if (tid < KT) {
        const int64_t kr = bh_kv * a.Sk + k0 + tid;
        const bool ok = tid < nk;
        skv[tid] = ok ? h2f(a.kvn[kr]) : 0.f;
        skr[tid] = ok ? a.coeff * h2f(a.krn[kr]) : 0.f;
        if constexpr (!SCORES) svv[tid] = ok ? h2f(a.vvn[kr]) : 0.f;
      }
    }
    __syncthreads();
    // ---- decode K^ and signs: one 8-dim group per item
    {
      const uint8_t* rk = reinterpret_cast<const uint8_t*>(rawK);
      const uint8_t* rs = reinterpret_cast<const uint8_t*>(rawS);
      for (int it = tid; it < KT * (D / 8); it += 256) {
        const int key = it / (D / 8), dg = it % (D / 8);
        half8 kv, sv;
        if (key < nk) {
          const uint64_t w = load_group(rk + key * kc + dg * a.kb, a.kb);
          const uint32_t sb = rs[key * (D / 8) + dg];
          const uint32_t mk = (1u << a.kb) - 1u;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            kv[e] = lutK[static_cast<uint32_t>(w >> (e * a.kb)) & mk];
            sv[e] = ((sb >> e) & 1u) ? static_cast<_Float16>(1.0f) : static_cast<_Float16>(-1.0f);
          }
        } else {
          kv = half8{};
          sv = half8{};
        }
        *reinterpret_cast<half8*>(&sK[key * T::LDK + dg * 8]) = kv;
        *reinterpret_cast<half8*>(&sS[key * T::LDK + dg * 8]) = sv;
      }
      if constexpr (!SCORES) {
        // V^T: item = (8-dim group, 4-key quad)
        const uint8_t* rv = reinterpret_cast<const uint8_t*>(rawV);
        const uint32_t mv = (1u << a.vb) - 1u;
        for (int it = tid; it < (D / 8) * (KT / 4); it += 256) {
          const int dg = it % (D / 8), kq = it / (D / 8);
          half4 col[8];
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) {
            const int key = kq * 4 + kk;
            uint64_t w = 0;
            if (key < nk) w = load_group(rv + key * vc + dg * a.vb, a.vb);
#pragma unroll
            for (int e = 0; e < 8; ++e)
              col[e][kk] = (key < nk) ? lutV[static_cast<uint32_t>(w >> (e * a.vb)) & mv]
                                      : static_cast<_Float16>(0.f);
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) *reinterpret_cast<half4*>(&sVt[(dg * 8 + e) * T::LDV + kq * 4]) = col[e];
        }
      }
    }
    __syncthreads();

    // ---- S^T = K^ Q^T (term 1) and Sign Q_proj^T (term 2)
    float4v s1[MBK][NBW], s2[MBK][NBW];
#pragma unroll
    for (int mb = 0; mb < MBK; ++mb)
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        s1[mb][nb] = float4v{0.f, 0.f, 0.f, 0.f};
        s2[mb][nb] = float4v{0.f, 0.f, 0.f, 0.f};
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
          s1[mb][nb] = mfma16x16x32(ka, qr[ks][nb], s1[mb][nb]);
          s2[mb][nb] = mfma16x16x32(sa, qp[ks][nb], s2[mb][nb]);
        }
      }
    }

    // ---- combine: s = vn * t1 + coeff * rn * t2
    float sc[MBK][NBW][4];
#pragma unroll
    for (int mb = 0; mb < MBK; ++mb) {
      const int kk = mb * 16 + lg * 4;
      const float4v kv = *reinterpret_cast<const float4v*>(&skv[kk]);
      const float4v kr = *reinterpret_cast<const float4v*>(&skr[kk]);
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb)
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[mb][nb][e] = s1[mb][nb][e] * kv[e] + s2[mb][nb][e] * kr[e];
    }

    if constexpr (SCORES) {
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        if (!col_ok[nb]) continue;
        float* orow = a.scores + ((static_cast<int64_t>(b) * a.Hq + col_h[nb]) * a.Sq + col_i[nb]) * a.Sk;
#pragma unroll
        for (int mb = 0; mb < MBK; ++mb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int key = k0 + mb * 16 + lg * 4 + e;
            if (key < a.Sk) orow[key] = sc[mb][nb][e];
          }
      }
    } else {
      // ---- online softmax (natural-log units; exp via exp2)
      half8 pb[MBK / 2][NBW];
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        const int qi = col_i[nb];
        const int lim = qi + (a.Sk - a.Sq);  // causal: keys <= lim
        const float* mrow = a.mask ? a.mask + b * a.smb + col_h[nb] * a.smh + static_cast<int64_t>(qi) * a.smq
                                   : nullptr;
        float tmax = -INFINITY;
#pragma unroll
        for (int mb = 0; mb < MBK; ++mb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int key = k0 + mb * 16 + lg * 4 + e;
            float v = sc[mb][nb][e] * a.scale;
            if (mrow && key < a.Sk && col_ok[nb]) v += mrow[key * a.smk];
            const bool dead = key >= a.Sk || (a.causal && key > lim) || !col_ok[nb];
            v = dead ? -INFINITY : v;
            sc[mb][nb][e] = v;
            tmax = fmaxf(tmax, v);
          }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float m_new = fmaxf(m_run[nb], tmax);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        const float alpha = (m_run[nb] == -INFINITY) ? 0.f : exp2f((m_run[nb] - m_use) * LOG2E);
        m_run[nb] = m_new;
        float psum = 0.f;
#pragma unroll
        for (int mb = 0; mb < MBK; ++mb) {
          const int kk = mb * 16 + lg * 4;
          const float4v vv = *reinterpret_cast<const float4v*>(&svv[kk]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float p = exp2f((sc[mb][nb][e] - m_use) * LOG2E);
            psum += p;
            pb[mb / 2][nb][(mb & 1) * 4 + e] = static_cast<_Float16>(p * vv[e]);
          }
        }
        l_run[nb] = l_run[nb] * alpha + psum;
#pragma unroll
        for (int db = 0; db < DB; ++db) oacc[db][nb] *= alpha;
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
          for (int nb = 0; nb < NBW; ++nb) oacc[db][nb] = mfma16x16x32(va, pb[c][nb], oacc[db][nb]);
        }
      }
    }
  }

  if constexpr (!SCORES) {
    // ---- normalise and rotate back: out = (O^T / l)^T Pi_v, Pi_v^T as A operand
    const half4* Ph = reinterpret_cast<const half4*>(a.vpit);
    const half4* Pl = reinterpret_cast<const half4*>(a.vpit + D * D);
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
      const float up = ldexpf(64.f, -ex), down = ldexpf(1.f / 4096.f, ex);
      // B operand chunks (hi/lo) of O_rot^T
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
#pragma unroll
      for (int ib = 0; ib < DB; ++ib) {
        float4v f = float4v{0.f, 0.f, 0.f, 0.f};
        const int i = ib * 16 + l16;
#pragma unroll
        for (int c = 0; c < DB / 2; ++c) {
          const int j0 = c * 32 + lg * 4;
          const half8 ah = cat8(Ph[(i * D + j0) / 4], Ph[(i * D + j0 + 16) / 4]);
          const half8 al = cat8(Pl[(i * D + j0) / 4], Pl[(i * D + j0 + 16) / 4]);
          f = mfma16x16x32(ah, bh[c], f);
          f = mfma16x16x32(al, bh[c], f);
          f = mfma16x16x32(ah, bl[c], f);
        }
        if (col_ok[nb]) {
          const int64_t o = static_cast<int64_t>(b) * a.sob + static_cast<int64_t>(h) * a.soh +
                            static_cast<int64_t>(qi) * a.sos + ib * 16 + lg * 4;
#pragma unroll
          for (int e = 0; e < 4; ++e) store_act<DT>(a.out, o + e, f[e] * down);
        }
      }
    }
  }
}

template <int D, int DT, bool SCORES>
static void launch_attn(AttnArgs a, hipStream_t s) {
  dim3 grid(a.nqb, a.Hkv, a.B);
  attn_kernel<D, DT, SCORES><<<grid, 256, 0, s>>>(a);
}

#define TQ_ATTN_SWITCH(d, dt, SC, a, s)                                \
  switch ((d) * 4 + (dt)) {                                            \
    case 32 * 4 + TQ_F32: launch_attn<32, TQ_F32, SC>(a, s); break;    \
    case 32 * 4 + TQ_F16: launch_attn<32, TQ_F16, SC>(a, s); break;    \
    case 32 * 4 + TQ_BF16: launch_attn<32, TQ_BF16, SC>(a, s); break;  \
    case 64 * 4 + TQ_F32: launch_attn<64, TQ_F32, SC>(a, s); break;    \
    case 64 * 4 + TQ_F16: launch_attn<64, TQ_F16, SC>(a, s); break;    \
    case 64 * 4 + TQ_BF16: launch_attn<64, TQ_BF16, SC>(a, s); break;  \
    case 128 * 4 + TQ_F32: launch_attn<128, TQ_F32, SC>(a, s); break;  \
    case 128 * 4 + TQ_F16: launch_attn<128, TQ_F16, SC>(a, s); break;  \
    case 128 * 4 + TQ_BF16: launch_attn<128, TQ_BF16, SC>(a, s); break;\
    case 256 * 4 + TQ_F32: launch_attn<256, TQ_F32, SC>(a, s); break;  \
    case 256 * 4 + TQ_F16: launch_attn<256, TQ_F16, SC>(a, s); break;  \
    case 256 * 4 + TQ_BF16: launch_attn<256, TQ_BF16, SC>(a, s); break;\
    default: break;                                                    \
  }

static int block_rows(int d) {
  switch (d) {
    case 32: return ATile<32>::BR;
    case 64: return ATile<64>::BR;
    case 128: return ATile<128>::BR;
    default: return ATile<256>::BR;
  }
}

}  // namespace tq

using namespace tq;

static int check_common(const char* what, int32_t B, int32_t Hq, int32_t Hkv, int32_t Sq, int32_t Sk,
                        int32_t d, int32_t bits) {
  if (!supported_dim(d)) {
    set_error("%s: head_dim %d not built (supported: 32, 64, 128, 256)", what, (int)d);
    return TQ_EUNSUPPORTED;
  }
  TQ_REQUIRE(bits >= 2 && bits <= 4, "%s: key bits must be in [2, 4], got %d", what, (int)bits);
  TQ_REQUIRE(B >= 0 && Hq >= 0 && Hkv >= 1 && Sq >= 0 && Sk >= 0, "%s: bad shape", what);
  TQ_REQUIRE(Hq % Hkv == 0, "%s: Hq=%d is not a multiple of Hkv=%d", what, (int)Hq, (int)Hkv);
  TQ_REQUIRE(Hq / Hkv <= block_rows(d), "%s: group size %d exceeds %d", what, (int)(Hq / Hkv),
             block_rows(d));
  return TQ_OK;
}

extern "C" {

int tq_attention_scores(const uint16_t* q_rot, const uint16_t* q_proj, const uint8_t* key_codes,
                        const uint8_t* key_signs, const uint16_t* key_rn, const uint16_t* key_vn,
                        const uint16_t* centroids_f16, int32_t B, int32_t Hq, int32_t Hkv, int32_t Sq,
                        int32_t Sk, int32_t d, int32_t bits, float coeff, float* out, void* stream) {
  int st = check_common("tq_attention_scores", B, Hq, Hkv, Sq, Sk, d, bits);
  if (st != TQ_OK) return st;
  if (static_cast<int64_t>(B) * Hq * Sq * Sk == 0) return TQ_OK;
  TQ_REQUIRE(q_rot && q_proj && key_codes && key_signs && key_rn && key_vn && centroids_f16 && out,
             "tq_attention_scores: null pointer");
  AttnArgs a{};
  a.q_rot = q_rot;
  a.q_proj = q_proj;
  a.kcodes = key_codes;
  a.ksigns = key_signs;
  a.krn = key_rn;
  a.kvn = key_vn;
  a.kcent = centroids_f16;
  a.kb = bits - 1;
  a.vb = 1;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.Sq = Sq;
  a.Sk = Sk;
  a.G = Hq / Hkv;
  a.QT = block_rows(d) / a.G;
  a.nqb = (Sq + a.QT - 1) / a.QT;
  a.coeff = coeff;
  a.scale = 1.f;
  a.scores = out;
  TQ_ATTN_SWITCH(d, TQ_F32, true, a, as_stream(stream));
  return launch_status("tq_attention_scores");
}

int tq_attention_fwd(const uint16_t* q_rot, const uint16_t* q_proj, const uint8_t* key_codes,
                     const uint8_t* key_signs, const uint16_t* key_rn, const uint16_t* key_vn,
                     const uint16_t* key_centroids_f16, int32_t bits, const uint8_t* val_codes,
                     const uint16_t* val_vn, const uint16_t* val_centroids_f16, int32_t val_bits,
                     const uint16_t* val_pit_split, int32_t B, int32_t Hq, int32_t Hkv, int32_t Sq,
                     int32_t Sk, int32_t d, float coeff, float scale, int32_t causal,
                     const float* mask, int64_t smb, int64_t smh, int64_t smq, int64_t smk,
                     void* out, int32_t out_dtype, int64_t sob, int64_t soh, int64_t sos,
                     void* stream) {
  int st = check_common("tq_attention_fwd", B, Hq, Hkv, Sq, Sk, d, bits);
  if (st != TQ_OK) return st;
  TQ_REQUIRE(val_bits >= 1 && val_bits <= 4, "tq_attention_fwd: value bits must be in [1, 4], got %d",
             (int)val_bits);
  TQ_REQUIRE(out_dtype == TQ_F32 || out_dtype == TQ_F16 || out_dtype == TQ_BF16,
             "tq_attention_fwd: unknown out dtype %d", (int)out_dtype);
  TQ_REQUIRE(!causal || Sk >= Sq, "tq_attention_fwd: causal needs Sk >= Sq");
  if (static_cast<int64_t>(B) * Hq * Sq == 0) return TQ_OK;
  TQ_REQUIRE(q_rot && q_proj && val_pit_split && out && key_centroids_f16 && val_centroids_f16,
             "tq_attention_fwd: null pointer");
  TQ_REQUIRE(Sk == 0 || (key_codes && key_signs && key_rn && key_vn && val_codes && val_vn),
             "tq_attention_fwd: null key/value plane");
  AttnArgs a{};
  a.q_rot = q_rot;
  a.q_proj = q_proj;
  a.kcodes = key_codes;
  a.ksigns = key_signs;
  a.krn = key_rn;
  a.kvn = key_vn;
  a.kcent = key_centroids_f16;
  a.kb = bits - 1;
  a.vcodes = val_codes;
  a.vvn = val_vn;
  a.vcent = val_centroids_f16;
  a.vpit = val_pit_split;
  a.vb = val_bits;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.Sq = Sq;
  a.Sk = Sk;
  a.G = Hq / Hkv;
  a.QT = block_rows(d) / a.G;
  a.nqb = (Sq + a.QT - 1) / a.QT;
  a.coeff = coeff;
  a.scale = scale;
  a.causal = causal;
  a.mask = mask;
  a.smb = smb;
  a.smh = smh;
  a.smq = smq;
  a.smk = smk;
  a.out = out;
  a.sob = sob;
  a.soh = soh;
  a.sos = sos;
  TQ_ATTN_SWITCH(d, out_dtype, false, a, as_stream(stream));
  return launch_status("tq_attention_fwd");
}

}  // extern "C"
