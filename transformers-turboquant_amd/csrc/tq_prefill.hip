// Fused compressed-domain attention for many query rows (prefill), head_dim 64 and 128.
//
// Same estimator and output as tq_attn.hip's tiled kernel (scores from packed
// keys, online softmax, P.V over packed values, Pi_v applied once per output
// row), organised so that no phase waits on another:
//
//  * Raw packed planes of each 32-key tile (codes, signs, value codes, the
//    three norm planes) are copied straight into an R-slot LDS ring with
//    direct-to-LDS buffer loads issued R-1 tiles ahead (no register staging).
//  * Each tile is decoded once per block into f16 tiles: K^ = Ck[codes] and
//    the +-1 sign tile as [key][dim] rows, and V^T = Cv[codes] as [dim][key]
//    rows (dims permuted so that the epilogue's Pi_v^T fragments are 16-byte runs),
//    V^ = f16(Cv[code] * vn) with the value norm applied by a packed f16
//    multiply of each (key, key+1) dword.  Decoding uses small
//    LDS tables indexed by nibbles / bit fields (conflict-free for <= 32
//    entries); the value table is indexed by the codes of two keys at one dim,
//    so each lookup yields the (key, key+1) pair the MFMA operand needs and no
//    transposition is done.
//  * The decoded tiles are double-buffered: in one pass between two barriers
//    every wave decodes its share of tile t+1 and runs the MFMAs and softmax of
//    tile t, one block barrier per tile.
//  * A block of 4 wave64 owns 128 (query row, query head) columns of one
//    (batch, kv head); each wave owns two 16-column blocks (one, 64 columns per
//    block, when an additive mask is applied: its loads and addresses do not fit
//    the 256 VGPRs of the two-block form, which spilled ~56 of them).  S^T = K^ Q^T comes
//    out of v_mfma_f32_16x16x32_f16 with 4 consecutive keys of one column per
//    lane, the P^T operand layout of O^T += V^T P^T, so P stays in registers.
//    P = f16(2^(s - m)) enters the P.V product (one f16 rounding, P <= 2^TAU).
//  * q_proj enters the QJL term as f16 hi + lo (two MFMAs against the exact +-1 signs, f32
//    grade).  The hi fragments stay in registers.  The lo fragments stay in registers where
//    they fit (head_dim 64, or one column block per wave).  At head_dim 128 with two column
//    blocks per wave they live in LDS: each wave holds its own 8 KB of them and reads each one
//    once per tile.  Their LDS comes from the +-1 sign tiles, which that form does not decode:
//    its sign operands come straight from the raw sign bits through a 16-entry table, and the
//    QJL term's k-slots are permuted so that one dword of a key's sign row serves all four
//    k-steps.
#include "tq_common.h"
#include "tq_stream.h"

#include <type_traits>


namespace tq {

constexpr int kPfRing = 2;   // raw tiles in the LDS ring (one in flight while one is decoded)
constexpr int kPfWaves = 4;  // waves per block, each with two 16-column blocks: 128 columns
// 16-column MFMA blocks per wave: 2, or 1 with an additive mask
template <bool MASK>
constexpr int pf_nbw() { return MASK ? 1 : 2; }
// where q_proj's lo fragments live: registers where they fit, otherwise LDS (two column
// blocks per wave at head_dim 128)
template <int D, bool MASK>
constexpr bool pf_qlo_lds() { return D > 64 && pf_nbw<MASK>() > 1; }

struct PrefillArgs {
  const uint16_t* q_rot;
  const float* q_proj;  // f32, taken as f16 hi + lo operands
  const uint8_t *kcodes, *ksigns;
  const uint16_t *krn, *kvn, *kcent;  // f16 key centroids
  const uint8_t* vcodes;
  const uint16_t *vvn, *vpit;         // vpit: split Pi_v^T (hi, lo)
  const float* vcent;                 // f32 value centroids
  int B, Hq, Hkv, Sq, Sk, G, QT, nqb;
  int64_t ldk;                        // rows between consecutive (batch, kv head) planes
  float coeff, scale;
  int causal;
  const float* mask;
  int64_t smb, smh, smq, smk;
  void* out;
  int out_dtype;
  int64_t sob, soh, sos;
  // split-K (part_o != nullptr, one query block per kv head): block (x, split) attends keys
  // [split * chunk, (split + 1) * chunk) and writes its columns' partial O (unnormalised,
  // rotated value domain, rows of dp floats), reference maximum and sum for a merge
  float *part_o, *part_ml;
  int nsplit, chunk, C, dp;
};

template <int D_, int BITS>
struct PfCfg {
  static constexpr int D = D_, KT = 32, R = kPfRing, NW = kPfWaves, NT = 64 * NW;
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static_assert(NW == 4 || NW == 8, "4 or 8 waves per block");
  static constexpr int KB = BITS - 1, VB = BITS;
  static constexpr int KC = D * KB / 8, SC = D / 8, VC = D * VB / 8;  // bytes per packed row
  // raw slot: code planes, sign plane, value codes (+16 so that dword-pair reads of the
  // last row stay inside the slot), three norm planes of one dword per key
  static constexpr int OFF_K = 0, OFF_S = OFF_K + KT * KC, OFF_V = OFF_S + KT * SC;
  static constexpr int OFF_N = OFF_V + KT * VC + 16;
  static constexpr int NRM = KT * 4;
  static constexpr int SLOT = OFF_N + 3 * NRM;
  static constexpr int NKD = (KT * KC + 1023) / 1024, NSD = (KT * SC + 1023) / 1024, NVD = (KT * VC + 1023) / 1024;
  static constexpr int NDMA = NKD + NSD + NVD + 3;  // DMA instructions per tile (issued by wave 0)
  static constexpr int LDK = D + 8;   // f16 stride of K^ / sign rows: 8-lane b128 reads hit distinct banks
  static constexpr int LDV = KT + 8;  // f16 stride of V^T rows: 8-lane b128 reads hit distinct banks
  // lookup tables: signs 16 x half4; keys KB=1 16 x half4, KB=2 16 x half2, KB=3 64 x half2;
  // value pairs (C[x], C[y]) indexed by x | y << VB: 16 / 64 / 256 x half2
  static constexpr int T_SGN = 0, T_KEY = 128;
  static constexpr int T_VAL = T_KEY + (KB == 1 ? 128 : (KB == 2 ? 64 : 256));
  static constexpr int T_BYTES = T_VAL + (VB == 2 ? 64 : (VB == 3 ? 256 : 1024));
  static_assert((KT * KC) % 256 == 0 && (KT * SC) % 256 == 0 && (KT * VC) % 256 == 0,
                "planes of whole 16-byte chunks per lane");
};

// 32 bits of a packed row from byte `off` on: the dword pair around it, byte-aligned
// without a branch (a shift of 0 returns the low dword)
__device__ __forceinline__ uint32_t field32(const uint8_t* row, int off) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(row + (off & ~3));
  return __builtin_amdgcn_alignbyte(w[1], w[0], off & 3);
}

// odd VB-bit fields of 8 consecutive fields
template <int VB>
constexpr uint32_t odd_fields() {
  return VB == 2 ? 0xCCCCu : (VB == 3 ? 0xE38E38u : 0xF0F0F0F0u);
}

template <int D_, int BITS, bool MASK>
__global__ void __launch_bounds__(64 * kPfWaves) __attribute__((amdgpu_waves_per_eu(2))) prefill_kernel(PrefillArgs a) {
  using C = PfCfg<D_, BITS>;
  constexpr int D = C::D, KT = C::KT, R = C::R, KB = C::KB, VB = C::VB;
  constexpr bool QLDS = pf_qlo_lds<D_, MASK>();  // lo fragments in LDS, signs from the raw bits
  constexpr int KC = C::KC, SC = C::SC, VC = C::VC, LDK = C::LDK, LDV = C::LDV;
  constexpr int KS = D / 32, DB = D / 16, NT = C::NT, NBW = pf_nbw<MASK>();  // 16 columns per block
  constexpr float LOG2E = 1.4426950408889634f;
  constexpr float TAU = 8.0f;  // lazy-rescale headroom (log2 units)

  __shared__ __attribute__((aligned(16))) uint8_t luts[C::T_BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t ring[R * C::SLOT];
  __shared__ __attribute__((aligned(16))) _Float16 sK0[KT * LDK], sK1[KT * LDK];
  __shared__ __attribute__((aligned(16))) _Float16 sS0[QLDS ? 8 : KT * LDK], sS1[QLDS ? 8 : KT * LDK];
  // lo fragments of q_proj, per wave [k-step][column block][lane] (QLDS only)
  __shared__ __attribute__((aligned(16))) half8 sQlo[QLDS ? kPfWaves * KS * NBW * 64 : 1];
  __shared__ __attribute__((aligned(16))) _Float16 sV0[D * LDV], sV1[D * LDV];
  __shared__ __attribute__((aligned(16))) float fac0[3][KT], fac1[3][KT];  // fa*vn_k, fa*coeff*rn_k, unused
  const uint8_t* tS = luts + C::T_SGN;
  const uint8_t* tK = luts + C::T_KEY;
  const uint8_t* tV = luts + C::T_VAL;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
  const int64_t bh = static_cast<int64_t>(b) * a.Hkv + hkv;

  // ---- lookup tables
  {
    auto kc = [&](int i) { return __builtin_bit_cast(_Float16, a.kcent[i]); };
    auto vc = [&](int i) { return static_cast<_Float16>(a.vcent[i]); };
    if (tid < 16) {
      half4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = ((tid >> j) & 1) ? static_cast<_Float16>(1.f) : static_cast<_Float16>(-1.f);
      *reinterpret_cast<half4*>(luts + C::T_SGN + tid * 8) = v;
    }
    if constexpr (KB == 1) {
      if (tid < 16) {
        half4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = kc((tid >> j) & 1);
        *reinterpret_cast<half4*>(luts + C::T_KEY + tid * 8) = v;
      }
    } else {
      constexpr int N = (KB == 2) ? 16 : 64;
      if (tid < N) {
        half2v v;
        v[0] = kc(tid & ((1 << KB) - 1));
        v[1] = kc(tid >> KB);
        *reinterpret_cast<half2v*>(luts + C::T_KEY + tid * 4) = v;
      }
    }
    constexpr int NV = 1 << (2 * VB);
    if (tid < NV) {
      half2v v;
      v[0] = vc(tid & ((1 << VB) - 1));
      v[1] = vc(tid >> VB);
      *reinterpret_cast<half2v*>(luts + C::T_VAL + tid * 4) = v;
    }
  }

  // ---- this lane's columns and their query fragments (B operands)
  int col_i[NBW], col_h[NBW];
  bool col_ok[NBW];
  half8 qr[KS][NBW], qp[KS][NBW];
  [[maybe_unused]] half8 qlo[QLDS ? 1 : KS][NBW];
  half8* const wlo = sQlo + wave * (KS * NBW * 64) + lane;  // this lane's lo fragments (QLDS)
  int64_t qrow[NBW];
  float qmax = 0.f;  // largest |q_proj| of the block's columns: the scale of its (hi, lo) split
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
    const int r = (wave * NBW + nb) * 16 + l16;
    const int ql = r / a.G, gi = r % a.G;
    col_i[nb] = q0 + ql;
    col_h[nb] = hkv * a.G + gi;
    col_ok[nb] = (ql < a.QT) && (col_i[nb] < a.Sq);
    qrow[nb] = ((static_cast<int64_t>(b) * a.Hq + col_h[nb]) * a.Sq + (col_ok[nb] ? col_i[nb] : 0)) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      if (col_ok[nb]) qmax = fmaxf(qmax, absmax8(a.q_proj + qrow[nb] + ks * 32 + lg * 8));
  }
  __shared__ float s_qmax[kPfWaves];
  qmax = wave_max(qmax);
  if (lane == 0) s_qmax[wave] = qmax;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kPfWaves; ++w) qmax = fmaxf(qmax, s_qmax[w]);
  const float qs = qproj_split_scale(qmax);
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d0 = ks * 32 + lg * 8;
      qr[ks][nb] = col_ok[nb] ? *reinterpret_cast<const half8*>(a.q_rot + qrow[nb] + d0) : half8{};
      // the QJL term's k-slots: lane group lg, k-step ks <-> dims 32 lg + 8 ks + 0..7 where the
      // sign operands come from the raw bits (byte 4 lg + ks of the key's sign row)
      const int dp = QLDS ? lg * 32 + ks * 8 : d0;
      half8 hi = half8{}, lo = half8{};
      if (col_ok[nb]) split8s(a.q_proj + qrow[nb] + dp, qs, hi, lo);
      qp[ks][nb] = hi;
      if constexpr (QLDS) wlo[(ks * NBW + nb) * 64] = lo;
      else qlo[ks][nb] = lo;
    }
  }
  // additive-mask rows of this lane's columns (row 0 for padding columns, whose scores are
  // never written).  A lane's keys 4lg + 0..3 of a 16-key block are consecutive: one 16-byte
  // load when the rows are contiguous in keys and 16-byte aligned (wave-uniform test)
  const float* mrow[NBW];
  bool mvec = false;
  if constexpr (MASK) {
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb)
      mrow[nb] = a.mask + static_cast<int64_t>(b) * a.smb + static_cast<int64_t>(col_h[nb]) * a.smh +
                 static_cast<int64_t>(col_ok[nb] ? col_i[nb] : 0) * a.smq;
    mvec = a.smk == 1 && (reinterpret_cast<uintptr_t>(a.mask) & 15) == 0 && ((a.smb | a.smh | a.smq) & 3) == 0;
  }

  // keys this block needs; tiles past `kfull` need per-element masking.  A split starts and
  // ends on tile boundaries (chunk is a multiple of KT); tb is its first tile.
  const bool split_k = a.part_o != nullptr;
  const int split = split_k ? static_cast<int>(blockIdx.y) : 0;
  int kend = a.Sk, kfull = a.Sk;
  if (a.causal) {
    const int imax = min(q0 + a.QT - 1, a.Sq - 1);
    kend = min(a.Sk, imax + (a.Sk - a.Sq) + 1);
    kfull = min(kfull, q0 + (a.Sk - a.Sq) + 1);
  }
  int tb = 0;
  if (split_k) {
    tb = split * (a.chunk / KT);
    kend = min(kend, (tb * KT) + a.chunk);
  }
  const int nt = kend > tb * KT ? (kend - tb * KT + KT - 1) / KT : 0;  // tiles tb .. tb + nt - 1
  const float fa = a.scale * LOG2E;  // scores kept in log2 units
  const float fb = fa * a.coeff * (1.f / qs);  // q_proj's operands carry qs

  // ---- raw ring: wave 0 copies tile j's planes into slot j % R
  const int64_t g0 = bh * a.ldk;
  const uint8_t* pk = a.kcodes + g0 * KC;
  const uint8_t* ps = a.ksigns + g0 * SC;
  const uint8_t* pv = a.vcodes + g0 * VC;
  const uint16_t* pkn = a.kvn + g0;
  const uint16_t* prn = a.krn + g0;
  const uint16_t* pvn = a.vvn + g0;
  const uint32_t ring_lds = lds_offset(ring);
  auto copy_plane = [&](const i32x4& r, uint32_t dst, int bytes, int nrounds) __attribute__((always_inline)) {
    const uint32_t lo = lane * 16;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (c >= nrounds) break;
      // whole rounds need no lane test; a partial round's lanes cover its remaining bytes
      if ((c + 1) * 1024 <= bytes || lane * 16 < bytes - c * 1024) dma16(r, dst + c * 1024, lo + c * 1024);
    }
  };
  auto issue = [&](int j) __attribute__((always_inline)) {  // wave 0 only
    const int kb = (tb + j) * KT;
    const uint32_t dst = ring_lds + (j % R) * C::SLOT;
    copy_plane(rows_desc(pk, KC, kb, kend), dst + C::OFF_K, KT * KC, C::NKD);
    copy_plane(rows_desc(ps, SC, kb, kend), dst + C::OFF_S, KT * SC, C::NSD);
    copy_plane(rows_desc(pv, VC, kb, kend), dst + C::OFF_V, KT * VC, C::NVD);
    if (lane < 32) {
      dma_u16(rows_desc(pkn, 2, kb, kend), dst + C::OFF_N, lane * 2);
      dma_u16(rows_desc(prn, 2, kb, kend), dst + C::OFF_N + C::NRM, lane * 2);
      dma_u16(rows_desc(pvn, 2, kb, kend), dst + C::OFF_N + 2 * C::NRM, lane * 2);
    }
  };
  // wave 0: wait until tile j has landed, `later` tiles having been issued after it
  auto wait_tile = [&](int later) __attribute__((always_inline)) {
    static_assert(R >= 2 && R <= 4, "ring of 2 to 4 tiles");
    if (later >= 2) wait_vm<(R >= 4 ? 2 * C::NDMA : 0)>();
    else if (later == 1) wait_vm<(R >= 3 ? C::NDMA : 0)>();
    else wait_vm<0>();
  };

  // ---- decode tile j (raw slot j % R): every thread one item of each kind, branch-free (a
  // slot past the last tile decodes stale bytes into a buffer nobody reads)
  auto decode_ks = [&](int j, _Float16* dK, _Float16* dS) __attribute__((always_inline)) {  // item (key, 8-dim group)
    const uint8_t* raw = ring + (j % R) * C::SLOT;
    constexpr int NG = D / 8;  // 8-dim groups per row
#pragma unroll
    for (int rep = 0; rep < KT * NG / NT; ++rep) {
      const int i = tid + rep * NT, key = i / NG, g = i % NG;  // NG a power of two: shifts
      half8 kv;
      if constexpr (KB == 1) {
        kv = nib2x4<0>(tK, raw[C::OFF_K + key * KC + g]);
      } else if constexpr (KB == 2) {
        kv = nib4x2<0>(tK, *reinterpret_cast<const uint16_t*>(raw + C::OFF_K + key * KC + 2 * g));
      } else {
        kv = six4x2(tK, field32(raw + C::OFF_K + key * KC, 3 * g));
      }
      *reinterpret_cast<half8*>(dK + key * LDK + 8 * g) = kv;
      if constexpr (!QLDS) {
        const half8 sv = nib2x4<0>(tS, raw[C::OFF_S + key * SC + g]);
        *reinterpret_cast<half8*>(dS + key * LDK + 8 * g) = sv;
      }
    }
  };
  auto decode_v = [&](int j, _Float16* dV, float (*dF)[KT]) __attribute__((always_inline)) {
    const uint8_t* raw = ring + (j % R) * C::SLOT;
    constexpr int NG = D / 8;  // 8-dim groups per row
#pragma unroll
    for (int rep = 0; rep < 2 * (KT / 2) * NG / NT; ++rep) {
      // values: item (key pair kp, 8-dim group dg, parity par) -> dwords (C[code 2kp], C[code 2kp+1])
      // of the even (par 0) or odd (par 1) dims of the group
      static_assert(NT == 256, "items i = tid + 256 rep: kp = i % 16, dg = (i / 16) % NG, par = i / (16 NG)");
      const int i = tid + rep * NT;
      // (tid < 256: at head_dim 128 the item is (tid & 15, tid >> 4, rep))
      const int kp = tid & 15, dg = NG == 16 ? (tid >> 4) : ((i >> 4) % NG), par = NG == 16 ? rep : ((i >> 4) / NG);
      const uint8_t* r0 = raw + C::OFF_V + (2 * kp) * VC;
      const uint32_t w0 = field32(r0, dg * VB), w1 = field32(r0 + VC, dg * VB);
      constexpr uint32_t M = odd_fields<VB>();
      const uint32_t x = par ? (w0 >> VB) : w0, y = par ? w1 : (w1 << VB);
      const uint32_t f = bfi32(M, y, x);
      half8 pv8;
      if constexpr (VB == 2) pv8 = nib4x2<0>(tV, f);
      else if constexpr (VB == 3) pv8 = six4x2(tV, f);
      else pv8 = byte4x2(tV, f);
      // V^ = f16(Cv[code] * vn): the pair's two value norms scale their halves of each dword
      const uint32_t* vnr = reinterpret_cast<const uint32_t*>(raw + C::OFF_N + 2 * C::NRM) + 2 * kp;
      const uint32_t vnw = (vnr[0] & 0xffffu) | (vnr[1] << 16);
      const half2v vn2 = __builtin_bit_cast(half2v, vnw);
      // V^T column order: key 16h + 4g + e sits at position 8g + 4h + e, so the 8 keys of one
      // P.V k-group (4g..4g+3 and 16+4g..16+4g+3) are one 16-byte run of a row
      const int pos = 8 * ((kp >> 1) & 3) + 4 * (kp >> 3) + 2 * (kp & 1);
      // V^T row order: dim 32c + 8g + 4h + e sits in row 16(2c + h) + 4g + e, so that lane group g
      // of O^T blocks 2c, 2c+1 holds dims 32c + 8g + 0..7 (one 16-byte run of a Pi_v^T row in the
      // epilogue); this item's dims 8dg + par + 2e land in rows vrow + {0, 2, 16, 18}
      const int vrow = 32 * (dg >> 2) + 4 * (dg & 3) + par;
      half2v* vcol = reinterpret_cast<half2v*>(dV + vrow * LDV + pos);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const half2v c2 = half2v{pv8[2 * e], pv8[2 * e + 1]};
        vcol[(16 * (e >> 1) + 2 * (e & 1)) * (LDV / 2)] = c2 * vn2;
      }
    }
    {  // per-key score factors from the key norm planes; threads past them write row 2 (unused)
      const uint32_t* nrm = reinterpret_cast<const uint32_t*>(raw + C::OFF_N);
      const int which = min(tid >> 5, 2), k = tid & 31;
      dF[which][k] = (which == 0 ? fa : fb) * h2f(static_cast<uint16_t>(nrm[min(which, 1) * KT + k]));
    }
  };

  // per column: the reference maximum mref (0 until the column has one) and the threshold a
  // lane's score (relative to mref) must exceed to move it: -inf until then, TAU after
  float mref[NBW], thr[NBW], l_run[NBW];
  float4v oacc[DB][NBW];
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
    mref[nb] = 0.f;
    thr[nb] = -INFINITY;
    l_run[nb] = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db][nb] = float4v{0.f, 0.f, 0.f, 0.f};
  }

  // ---- scores of tile j: S^T = K^ Q_rot^T (term 1) and Sign Q_proj^T (term 2).  `sw` (QLDS):
  // sign dword lg of the rows of keys l16 and 16 + l16 (raw bits of the tile)
  auto scores = [&](const _Float16* cK, const _Float16* cS, const uint32_t (&sw)[2], float4v (&sacc)[2][NBW],
                    float4v (&tacc)[2][NBW]) __attribute__((always_inline)) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        sacc[mb][nb] = float4v{0.f, 0.f, 0.f, 0.f};
        tacc[mb][nb] = float4v{0.f, 0.f, 0.f, 0.f};
      }
    // K^ and sign fragments one (k-step, key block) step ahead of their MFMAs; lo fragments
    // (QLDS) one k-step ahead
    half8 ka[2], sa[2];
    [[maybe_unused]] half8 la[2][NBW];
    auto frag = [&](auto I, int slot) __attribute__((always_inline)) {
      constexpr int i = decltype(I)::value;
      const int off = ((i & 1) * 16 + l16) * LDK + (i >> 1) * 32 + lg * 8;
      ka[slot] = *reinterpret_cast<const half8*>(cK + off);
      if constexpr (QLDS) sa[slot] = nib2x4<(i >> 1)>(tS, sw[i & 1]);
      else sa[slot] = *reinterpret_cast<const half8*>(cS + off);
    };
    auto lofrag = [&](int ks) __attribute__((always_inline)) {
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) la[ks & 1][nb] = wlo[(ks * NBW + nb) * 64];
    };
    frag(std::integral_constant<int, 0>{}, 0);
    if constexpr (QLDS) lofrag(0);
    static_for<2 * KS>([&](auto I) __attribute__((always_inline)) {
      constexpr int i = decltype(I)::value;
      constexpr int ks = i >> 1, mb = i & 1, c = i & 1;
      if constexpr (i + 1 < 2 * KS) frag(std::integral_constant<int, i + 1>{}, c ^ 1);
      if constexpr (QLDS && mb == 0 && ks + 1 < KS) lofrag(ks + 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        sacc[mb][nb] = mfma16x16x32(ka[c], qr[ks][nb], sacc[mb][nb]);
        tacc[mb][nb] = mfma16x16x32(sa[c], qp[ks][nb], tacc[mb][nb]);
        if constexpr (QLDS) tacc[mb][nb] = mfma16x16x32(sa[c], la[ks & 1][nb], tacc[mb][nb]);
        else tacc[mb][nb] = mfma16x16x32(sa[c], qlo[ks][nb], tacc[mb][nb]);
      }
    });
  };
  // ---- log2-domain scores with masking, column maxima, lazy rescale (one rare branch per tile)
  auto softmax_max = [&](int j, const float (*cF)[KT], const float4v (&sacc)[2][NBW],
                         const float4v (&tacc)[2][NBW], float (&sc)[NBW][2][4]) __attribute__((always_inline)) {
    const int k0 = (tb + j) * KT;
    const float4v fA0 = *reinterpret_cast<const float4v*>(&cF[0][4 * lg]);
    const float4v fA1 = *reinterpret_cast<const float4v*>(&cF[0][16 + 4 * lg]);
    const float4v fB0 = *reinterpret_cast<const float4v*>(&cF[1][4 * lg]);
    const float4v fB1 = *reinterpret_cast<const float4v*>(&cF[1][16 + 4 * lg]);
    const bool edge = k0 + KT > kfull;
    float lmax[NBW];
    bool grow_any = false;
    float4v mk[NBW][2];  // mask values of keys k0 + 16mb + 4lg + e (0 past Sk)
    if constexpr (MASK) {
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb)
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
          const int kb = k0 + mb * 16 + 4 * lg;
          if (mvec && kb + 4 <= a.Sk) {
            mk[nb][mb] = *reinterpret_cast<const float4v*>(mrow[nb] + kb);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              mk[nb][mb][e] = kb + e < a.Sk ? mrow[nb][static_cast<int64_t>(kb + e) * a.smk] : 0.f;
          }
        }
    }
    // scores leave here relative to the column's reference maximum: s - m in the same two
    // fmas, so P = 2^(s - m) needs no subtraction per score.  Under an additive mask they stay
    // absolute until the rescale test and are made relative after it: folding -m into the
    // fmas is exact only while m is of the order of real scores, and a column whose first
    // tile is masked with finfo.min (clamped to -3e38) would set m to -3e38, after which
    // s - m would round every real score of the next tile to the same value
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v;
          if constexpr (MASK)
            v = fmaf(tacc[mb][nb][e], mb ? fB1[e] : fB0[e], sacc[mb][nb][e] * (mb ? fA1[e] : fA0[e])) +
                fmaxf(mk[nb][mb][e] * LOG2E, -3.0e38f);
          else
            v = fmaf(tacc[mb][nb][e], mb ? fB1[e] : fB0[e], fmaf(sacc[mb][nb][e], mb ? fA1[e] : fA0[e], -mref[nb]));
          sc[nb][mb][e] = v;
        }
    }
    if (edge) {  // wave-uniform: only the block's last tiles reach past the causal edge or Sk
      asm volatile("; edge");  // a side effect keeps this a branch instead of selects on every tile
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        const int lim = a.causal ? col_i[nb] + (a.Sk - a.Sq) : a.Sk - 1;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int key = k0 + mb * 16 + 4 * lg + e;
            if (key >= a.Sk || key > lim) sc[nb][mb][e] = -INFINITY;
          }
      }
    }
    // the reference maximum of a column moves only when one of its scores exceeds it by
    // more than TAU: each lane tests its own scores, the exact column maxima are formed
    // (cross-lane) only when some lane triggers
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) {
      lmax[nb] = max8_raw(sc[nb][0][0], sc[nb][0][1], sc[nb][0][2], sc[nb][0][3], sc[nb][1][0], sc[nb][1][1],
                          sc[nb][1][2], sc[nb][1][3]);
      grow_any = grow_any || ((MASK ? lmax[nb] - mref[nb] : lmax[nb]) > thr[nb]);
    }
    if (__any(grow_any)) {
      asm volatile("; rescale");  // a side effect: the rare rescale stays a branch, never speculated
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        float tmax = lmax[nb];
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const bool grow = (MASK ? tmax - mref[nb] : tmax) > thr[nb];
        const float m_new = grow ? (MASK ? tmax : tmax + mref[nb]) : mref[nb];
        // O and l of a column without a reference are still zero
        const float alpha = (grow && thr[nb] != -INFINITY) ? __builtin_amdgcn_exp2f(mref[nb] - m_new) : 1.f;
        if constexpr (!MASK) {  // the tile's scores move to the new reference
          const float shift = m_new - mref[nb];
#pragma unroll
          for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int e = 0; e < 4; ++e) sc[nb][mb][e] -= shift;
        }
        mref[nb] = m_new;
        thr[nb] = grow ? TAU : thr[nb];
        l_run[nb] *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) oacc[db][nb] *= alpha;
      }
    }
    if constexpr (MASK) {
      // relative to the settled reference: a column that has seen only masked keys (all at
      // -3e38) gives them equal weights, as the reference's softmax of equal scores does
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb)
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int e = 0; e < 4; ++e) sc[nb][mb][e] -= mref[nb];
    }
  };
  // ---- P = f16(2^(s - m)) (<= 2^TAU), row sums, O^T += V^T P^T
  auto pv_tile = [&](const _Float16* cV, const float (&sc)[NBW][2][4]) __attribute__((always_inline)) {
    half8 pb[NBW];
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e) pb[nb][mb * 4 + e] = static_cast<_Float16>(__builtin_amdgcn_exp2f(sc[nb][mb][e]));
      // the row sums add the f16 weights that enter the product, two per v_dot2_f32_f16
      const half2v one2 = {static_cast<_Float16>(1.f), static_cast<_Float16>(1.f)};
      float l = l_run[nb];
#pragma unroll
      for (int q = 0; q < 4; ++q) l = __builtin_amdgcn_fdot2(half2v{pb[nb][2 * q], pb[nb][2 * q + 1]}, one2, l, false);
      l_run[nb] = l;
    }
    // k-slots 8*lg+0..3 <-> keys 4lg+0..3, 8*lg+4..7 <-> keys 16+4lg+0..3: positions 8lg..8lg+7
    // V^T fragments two blocks ahead of their MFMAs
    constexpr int PD = 2;
    half8 va[PD + 1];
#pragma unroll
    for (int q = 0; q < PD; ++q) va[q] = *reinterpret_cast<const half8*>(cV + (q * 16 + l16) * LDV + 8 * lg);
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      if (db + PD < DB) va[(db + PD) % (PD + 1)] = *reinterpret_cast<const half8*>(cV + ((db + PD) * 16 + l16) * LDV + 8 * lg);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) oacc[db][nb] = mfma16x16x32(va[db % (PD + 1)], pb[nb], oacc[db][nb]);
    }
  };

  // sign dword lg of keys l16 and 16 + l16 of raw tile j (QLDS)
  uint32_t swc[2] = {0u, 0u}, swn[2] = {0u, 0u};
  auto sign_words = [&](int j, uint32_t (&w)[2]) __attribute__((always_inline)) {
    const uint8_t* raw = ring + (j % R) * C::SLOT + C::OFF_S + lg * 4;
    w[0] = *reinterpret_cast<const uint32_t*>(raw + l16 * SC);
    w[1] = *reinterpret_cast<const uint32_t*>(raw + (16 + l16) * SC);
  };

  // ---- pipeline: tiles 0..R-1 in flight, tile 0 decoded, then one barrier per tile
  __builtin_amdgcn_s_waitcnt(0);  // q fragments landed: the ring's vmcnt waits count DMAs only
  if (nt > 0) {
    if (wave == 0) {
#pragma unroll
      for (int j = 0; j < R; ++j)
        if (j < nt) issue(j);
      wait_tile(min(nt, R) - 1);
    }
    __syncthreads();  // tables and raw tile 0 visible
    decode_ks(0, sK0, sS0);
    decode_v(0, sV0, fac0);
    if constexpr (QLDS) sign_words(0, swc);
  }
  auto iter = [&](int t, const _Float16* cK, const _Float16* cS, const _Float16* cV, const float (*cF)[KT],
                  _Float16* nK, _Float16* nS, _Float16* nV, float (*nF)[KT]) __attribute__((always_inline)) {
    if (wave == 0 && t + 1 < nt) wait_tile(max(0, min(nt, t + R) - (t + 2)));
    __syncthreads();  // tile t decoded by all waves; raw tile t+1 landed; buffers of tile t-1 free
    if (wave == 0 && t + R < nt) issue(t + R);
    float4v sacc[2][NBW], tacc[2][NBW];
    float sc[NBW][2][4];
    // the wave's priority is raised while it issues MFMAs
    decode_ks(t + 1, nK, nS);  // overlaps the score MFMAs
    if constexpr (QLDS) sign_words(t + 1, swn);  // raw tile t + 1 is overwritten at the next barrier
    __builtin_amdgcn_s_setprio(1);
    scores(cK, cS, swc, sacc, tacc);
    __builtin_amdgcn_s_setprio(0);
    softmax_max(t, cF, sacc, tacc, sc);
    __builtin_amdgcn_s_setprio(1);
    pv_tile(cV, sc);
    __builtin_amdgcn_s_setprio(0);
    decode_v(t + 1, nV, nF);   // overlaps the P.V MFMAs
    if constexpr (QLDS) {
      swc[0] = swn[0];
      swc[1] = swn[1];
    }
  };
  for (int t = 0; t < nt; t += 2) {
    iter(t, sK0, sS0, sV0, fac0, sK1, sS1, sV1, fac1);
    if (t + 1 < nt) iter(t + 1, sK1, sS1, sV1, fac1, sK0, sS0, sV0, fac0);
  }

  if (split_k) {
    // ---- split-K partial of each column: O in dim order (O^T row 16 db + 4 lg + e holds dim
    // 32 (db >> 1) + 8 lg + 4 (db & 1) + e), the reference its weights are relative to (-inf
    // while the column has none) and their sum
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) {
      float l = l_run[nb];
      l += __shfl_xor(l, 16, 64);
      l += __shfl_xor(l, 32, 64);
      if (col_ok[nb]) {
        const int c = col_i[nb] * a.G + (col_h[nb] - hkv * a.G);
        const int64_t rec = (bh * a.nsplit + split) * a.C + c;
        float* po = a.part_o + rec * a.dp;
#pragma unroll
        for (int db = 0; db < DB; ++db)
          *reinterpret_cast<float4v*>(po + 32 * (db >> 1) + 8 * lg + 4 * (db & 1)) = oacc[db][nb];
        if (lg == 0) {
          a.part_ml[rec * 2] = (thr[nb] == -INFINITY) ? -INFINITY : mref[nb];
          a.part_ml[rec * 2 + 1] = l;
        }
      }
    }
    return;
  }
  // ---- normalise and rotate back: out = (O^T / l)^T Pi_v, Pi_v^T as split-f16 A operand.
  // Lane group g of O^T blocks 2c, 2c+1 holds dims 32c + 8g + 0..7 (the V^T row order), so
  // each A fragment is one 16-byte run of a Pi_v^T row, read once for both column blocks.
  half8 oh[DB / 2][NBW], ol[DB / 2][NBW];  // split (hi, lo) B operands
  float down[NBW];
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
    const float up = ldexpf(kSplit, -ex);
    down[nb] = ldexpf(kUnsplit2, ex);
#pragma unroll
    for (int c = 0; c < DB / 2; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        _Float16 h, lo;
        split_f16(oacc[2 * c][nb][e] * up, h, lo);
        oh[c][nb][e] = h;
        ol[c][nb][e] = lo;
        split_f16(oacc[2 * c + 1][nb][e] * up, h, lo);
        oh[c][nb][4 + e] = h;
        ol[c][nb][4 + e] = lo;
      }
  }
  const _Float16* Ph = reinterpret_cast<const _Float16*>(a.vpit);
  const _Float16* Pl = Ph + D * D;
#pragma unroll 2
  for (int ib = 0; ib < DB; ++ib) {
    const int i = ib * 16 + l16;
    half8 ah[DB / 2], al[DB / 2];
#pragma unroll
    for (int c = 0; c < DB / 2; ++c) {
      ah[c] = *reinterpret_cast<const half8*>(Ph + i * D + c * 32 + lg * 8);
      al[c] = *reinterpret_cast<const half8*>(Pl + i * D + c * 32 + lg * 8);
    }
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) {
      float4v f = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < DB / 2; ++c) {
        f = mfma16x16x32(ah[c], oh[c][nb], f);
        f = mfma16x16x32(al[c], oh[c][nb], f);
        f = mfma16x16x32(ah[c], ol[c][nb], f);
      }
      if (col_ok[nb]) {
        const int64_t o = static_cast<int64_t>(b) * a.sob + static_cast<int64_t>(col_h[nb]) * a.soh +
                          static_cast<int64_t>(col_i[nb]) * a.sos + ib * 16 + lg * 4;
        const float4v fo = f * down[nb];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (a.out_dtype == TQ_BF16) store_act<TQ_BF16>(a.out, o + e, fo[e]);
          else if (a.out_dtype == TQ_F16) store_act<TQ_F16>(a.out, o + e, fo[e]);
          else store_act<TQ_F32>(a.out, o + e, fo[e]);
        }
      }
    }
  }
}

// Used by tq_attn.hip's entry points.
bool prefill_applies(int Hq, int Hkv, int d, int bits, int val_bits, bool masked) {
  const int cols = kPfWaves * 16 * (masked ? pf_nbw<true>() : pf_nbw<false>());
  return (d == 64 || d == 128) && bits >= 2 && bits <= 4 && val_bits == bits && Hq / Hkv <= cols;
}
// the split-K form: the kv head's columns (query rows x group) in one block
bool prefill_split_applies(int Hq, int Hkv, int Sq, int d, int bits, int val_bits, bool masked) {
  const int cols = kPfWaves * 16 * (masked ? pf_nbw<true>() : pf_nbw<false>());
  return prefill_applies(Hq, Hkv, d, bits, val_bits, masked) && static_cast<int64_t>(Hq / Hkv) * Sq <= cols;
}

int prefill_attention(int64_t ldk, const uint16_t* q_rot, const float* q_proj, const uint8_t* kcodes,
                      const uint8_t* ksigns, const uint16_t* krn, const uint16_t* kvn, const uint16_t* kcent,
                      int bits, const uint8_t* vcodes, const uint16_t* vvn, const float* vcent,
                      const uint16_t* vpit, int B, int Hq, int Hkv, int Sq, int Sk, int d, float coeff, float scale,
                      int causal, const float* mask, int64_t smb, int64_t smh, int64_t smq, int64_t smk, void* out,
                      int out_dtype, int64_t sob, int64_t soh, int64_t sos, hipStream_t s, float* part_o,
                      float* part_ml, int nsplit, int chunk, int C, int dp) {
  PrefillArgs a{};
  a.q_rot = q_rot;
  a.q_proj = q_proj;
  a.kcodes = kcodes;
  a.ksigns = ksigns;
  a.krn = krn;
  a.kvn = kvn;
  a.kcent = kcent;
  a.vcodes = vcodes;
  a.vvn = vvn;
  a.vcent = vcent;
  a.vpit = vpit;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.Sq = Sq;
  a.Sk = Sk;
  a.G = Hq / Hkv;
  a.QT = kPfWaves * 16 * (mask ? pf_nbw<true>() : pf_nbw<false>()) / a.G;  // query rows per block
  a.nqb = (Sq + a.QT - 1) / a.QT;
  a.ldk = ldk;
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
  // one block per (query block, batch, kv head), query blocks heavy first across all groups;
  // split-K: one query block, grid.y = splits
  if (part_o) {
    a.part_o = part_o;
    a.part_ml = part_ml;
    a.nsplit = nsplit;
    a.chunk = chunk;
    a.C = C;
    a.dp = dp;
  }
  const int64_t nblocks = static_cast<int64_t>(a.nqb) * Hkv * B;
  TQ_REQUIRE(nblocks < (int64_t(1) << 31), "tq_attention_fwd: %lld query blocks exceed one grid",
             (long long)nblocks);
  TQ_REQUIRE(!part_o || (a.nqb == 1 && chunk % PfCfg<128, 3>::KT == 0), "tq_attention_fwd: bad split plan");
  const dim3 grid(static_cast<unsigned>(nblocks), static_cast<unsigned>(part_o ? nsplit : 1));
#define TQ_PF_LAUNCH(DD, BB)                                                       \
  if (mask) prefill_kernel<DD, BB, true><<<grid, PfCfg<DD, BB>::NT, 0, s>>>(a);  \
  else prefill_kernel<DD, BB, false><<<grid, PfCfg<DD, BB>::NT, 0, s>>>(a);
  if (d == 64) {
    if (bits == 2) { TQ_PF_LAUNCH(64, 2) }
    else if (bits == 3) { TQ_PF_LAUNCH(64, 3) }
    else { TQ_PF_LAUNCH(64, 4) }
  } else {
    if (bits == 2) { TQ_PF_LAUNCH(128, 2) }
    else if (bits == 3) { TQ_PF_LAUNCH(128, 3) }
    else { TQ_PF_LAUNCH(128, 4) }
  }
#undef TQ_PF_LAUNCH
  return launch_status("tq_attention_fwd (prefill)");
}

}  // namespace tq
