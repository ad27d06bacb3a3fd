// Decode-shaped fused attention (split-K over keys) and the merge of the splits;
// the shared argument block, lookup tables and split planning are in tq_decode.h.
#include "tq_decode.h"

namespace tq {

// Fused decode attention, LDS-staged.  Each wave streams 64-key slabs of the key
// codes, sign bits, value codes and the three norm planes straight into its own
// LDS ring (R slots) with direct-to-LDS buffer loads, so many KB per wave are in
// flight without holding registers; lanes then gather their MFMA operands from
// the slot.  Lane (column l16, group lg) ends each 16-key block with the scores
// of keys 4*lg + e for its own column, which is the P^T operand layout of the
// value MFMA, so P never leaves registers.
template <int D, int BITS, int NBS, int R, bool PACK>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(PACK ? 4 : 3)))
decode_attn_lds_kernel(DecodeArgs a) {
  static_assert(D == 64 || D == 128, "decode kernel is built for head_dim 64 or 128");
  using L = SmallLuts<BITS>;
  constexpr int KB = L::KB, VB = L::VB;
  constexpr int KS = D / 32;           // score k-steps
  constexpr int DB = D / 16;           // value row blocks: lane l16 holds dims DB l16 .. DB l16 + DB - 1
  constexpr int NPAIR = D / 32;        // pair-table groups per parity
  constexpr int KC = D * KB / 8, SC = D / 8, VC = D * VB / 8;  // bytes per packed row
  constexpr int KLANE = KC / 4;        // key-code bytes per lane (4 lanes share a key row)
  constexpr int KW32 = (KLANE + 3) / 4;
  constexpr int SLANE = SC / 4;        // sign bytes per lane
  constexpr int VFB = DB * VB;         // value field bits of a lane
  constexpr int VW32 = (VB == 3) ? 2 : 1;  // dwords holding a lane's value field
  constexpr int NK = 16 * NBS;         // keys per wave slab
  constexpr int SLAB = 4 * NK;         // keys per block slab
  constexpr int OFF_K = 0, OFF_S = NK * KC, OFF_V = OFF_S + NK * SC, OFF_N = OFF_V + NK * VC;
  constexpr int NRM = NK * 4;          // one norm plane: a dword per key
  constexpr int SLOT = OFF_N + 3 * NRM;
  constexpr int STAGE = 4 * R * SLOT;
  constexpr int MERGE = 4 * 16 * (D + 2) * 4;
  static_assert(NBS == 2 || NBS == 4, "slabs of 32 or 64 keys");
  constexpr float LOG2E = 1.4426950408889634f;
  constexpr float TAU = 8.0f;          // lazy-rescale headroom (log2 units)
  // p = 2^(s - m_run + PUP) <= 2^(TAU + PUP): the top weight of a column sits near 2^6 ..
  // 2^14, so keys down to ~2^-31 of it still reach the f16 P operand (the f16 subnormal
  // floor is 2^-24), and p * vn / vcap <= 2^14 stays far from the f16 maximum
  constexpr float PUP = 6.0f;

  __shared__ __attribute__((aligned(16))) uint8_t luts[L::BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t stage[STAGE > MERGE ? STAGE : MERGE];
  // per-wave f32 key factors of the current slab: fa*vn_k, fb*rn_k, vn_v (one pass per key
  // instead of one per (key, column) lane)
  __shared__ __attribute__((aligned(16))) float fac[4][3][NK];
  const uint8_t* tS = luts + L::SGN_OFF;
  const uint8_t* tK = luts + L::KEY_OFF;
  const uint8_t* tV = luts + L::VAL_OFF;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int split = blockIdx.x, hkv = blockIdx.y, b = blockIdx.z;
  const int64_t bh = static_cast<int64_t>(b) * a.Hkv + hkv;

  build_small_luts<BITS, true>(a, luts, tid);

  // q_proj enters term 2 as f16 hi + lo.  PACK (C <= 8): B column l16 < 8 carries query
  // column l16 (q_rot, hi), column l16 + 8 carries the same column's lo part (q_rot zero);
  // after the MFMAs lane l16 adds lane l16 + 8's term 2 (DPP row rotate by 8).  Otherwise
  // the lo parts take a second MFMA per k-step.
  const int c = PACK ? (l16 & 7) : l16;
  const bool lo_col = PACK && l16 >= 8;
  const bool c_ok = c < a.C;
  const bool col_ok = c_ok && !lo_col;
  const int qi = c_ok ? c / a.G : 0, h = hkv * a.G + (c_ok ? c % a.G : 0);
  half8 qr[KS], qp[KS];
  [[maybe_unused]] half8 ql[PACK ? 1 : KS];
  {
    const int64_t qrow = ((static_cast<int64_t>(b) * a.Hq + h) * a.Sq + qi) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d0 = lg * (D / 4) + ks * 8;
      half8 hi = half8{}, lo = half8{};
      if (c_ok) split8(a.q_proj + qrow + d0, hi, lo);
      qr[ks] = (c_ok && !lo_col) ? *reinterpret_cast<const half8*>(a.q_rot + qrow + d0) : half8{};
      if constexpr (PACK) {
        qp[ks] = lo_col ? lo : hi;
      } else {
        qp[ks] = hi;
        ql[ks] = lo;
      }
    }
  }

  const float fa = a.scale * LOG2E;
  const float fb = a.coeff * fa;
  const int lim = a.causal ? qi + (a.Sk - a.Sq) : 0x7fffffff;  // keys <= lim are visible
  const int causal_from = a.causal ? a.Sk - a.Sq : 0x7fffffff;  // smallest lim of any column
  const int kbeg = split * a.chunk;
  const int kend = min(a.Sk, kbeg + a.chunk);

  // this lane's value field: VFB bits from bit l16 * VFB of the row, read as the dword (pair)
  // from byte vbase (the pair may run past the row end into the next row or the slot's norm
  // area; those bits are not used)
  const int vbit = l16 * VFB;
  const int vbase = (vbit >> 5) * 4;
  const int vshift = vbit & 31;

  const int64_t g0 = bh * a.ldk;
  const uint8_t* pk = a.kcodes + g0 * KC;
  const uint8_t* ps = a.ksigns + g0 * SC;
  const uint16_t* pkn = a.kvn + g0;
  const uint16_t* prn = a.krn + g0;
  const uint16_t* pvn = a.vvn + g0;
  const uint8_t* pv = a.vcodes + g0 * VC;

  uint8_t* mine = stage + wave * (R * SLOT);
  const uint32_t mine_lds = lds_offset(mine);
  constexpr int NKD = (NK * KC + 1023) / 1024, NSD = (NK * SC + 1023) / 1024, NVD = (NK * VC + 1023) / 1024;
  constexpr int NDMA = NKD + NSD + NVD + 3;  // DMA instructions per slot
  // a plane of `bytes` (a multiple of 16) moves in 1 KB rounds of 64 lanes x 16 B; a final
  // partial round uses the lanes it needs
  auto copy_plane = [&](const i32x4& r, uint32_t dst, int bytes, int nrounds) {
    const uint32_t lo = lane * 16;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (c >= nrounds) break;
      if ((c + 1) * 1024 <= bytes || lane * 16 < bytes - c * 1024) dma16(r, dst + c * 1024, lo + c * 1024);
    }
  };
  // DMA the wave's slab of keys [kb, kb + NK) into ring slot `slot`; rows past kend read zero
  auto issue = [&](int kb, int slot) {
    const uint32_t dst = mine_lds + slot * SLOT;
    wait_lds();  // earlier reads of this slot have landed
    copy_plane(rows_desc(pk, KC, kb, kend), dst + OFF_K, NK * KC, NKD);
    copy_plane(rows_desc(ps, SC, kb, kend), dst + OFF_S, NK * SC, NSD);
    copy_plane(rows_desc(pv, VC, kb, kend), dst + OFF_V, NK * VC, NVD);
    if (NK == 64 || lane < 32) {
      dma_u16(rows_desc(pkn, 2, kb, kend), dst + OFF_N, lane * 2);
      dma_u16(rows_desc(prn, 2, kb, kend), dst + OFF_N + NRM, lane * 2);
      dma_u16(rows_desc(pvn, 2, kb, kend), dst + OFF_N + 2 * NRM, lane * 2);
    }
  };
  // wait until the slot issued `later` slots ago has landed
  auto wait_slot = [&](int later) {
    static_assert(R <= 3, "ring of at most 3 slots");
    if (later >= 2) wait_vm<(R >= 3 ? 2 * NDMA : 0)>();
    else if (later == 1) wait_vm<NDMA>();
    else wait_vm<0>();
  };

  float m_run = -INFINITY, l_run = 0.f;
  // value norms enter P as vn / vcap <= 1; vcap is a power of two that only grows
  // (oacc is rescaled when it does) and multiplies oacc back before the merge
  float vcap = 0x1p-24f, inv_vcap = 0x1p24f;
  float4v oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = float4v{0.f, 0.f, 0.f, 0.f};

  // one NK-key slab in four phases (scores of all 4 blocks, scaling and edge
  // masking, one lazy-softmax step, values), giving the scheduler long
  // branch-free stretches; rows 16j .. 16j+15 of the slot are keys ks0 + 16j ..
  float (*fw)[NK] = fac[wave];
  auto slab = [&](const uint8_t* src, int ks0) {
    // ---- per-key factors fa*vn_k, fb*rn_k, vn_v/vcap: 3*NK values, one per lane and pass
#pragma unroll
    for (int i0 = 0; i0 < 3 * NK; i0 += 64) {
      const int i = i0 + lane, which = i / NK, k = i % NK;
      const float v = (i < 3 * NK)
          ? h2f(static_cast<uint16_t>(*reinterpret_cast<const uint32_t*>(src + OFF_N + which * NRM + k * 4)))
          : 0.f;
      if (i0 + 63 >= 2 * NK) {  // this pass holds value norms: keep them <= vcap
        const float vv = (which == 2) ? v : 0.f;
        if (__any(vv > vcap)) {
          float t = vv;
#pragma unroll
          for (int sh = 32; sh >= 1; sh >>= 1) t = fmaxf(t, __shfl_xor(t, sh, 64));
          int ex;
          frexpf(t, &ex);  // t < 2^ex; every lane holds the same t, so ex is wave-uniform
          ex = __builtin_amdgcn_readfirstlane(ex);
          const float cap = ldexpf(1.f, ex);
          const float shrink = vcap / cap;
#pragma unroll
          for (int db = 0; db < DB; ++db) oacc[db] *= shrink;
          vcap = cap;
          inv_vcap = ldexpf(1.f, -ex);
        }
      }
      if (i < 3 * NK) fw[which][k] = (which == 0) ? fa * v : (which == 1 ? fb * v : v * inv_vcap);
    }
    // ---- scores S^T = K^ Q^T (term 1) and Sign Q_proj^T (term 2), NBS blocks
    float4v s1[NBS], s2[NBS];
#pragma unroll
    for (int j = 0; j < NBS; ++j) {
      uint32_t kw[KW32];
      load_key_field<KLANE>(src + OFF_K + (16 * j + l16) * KC + lg * KLANE, kw);
      const uint32_t sw = load_sign_field<D>(src + OFF_S + (16 * j + l16) * SC + lg * SLANE);
      s1[j] = float4v{0.f, 0.f, 0.f, 0.f};
      s2[j] = float4v{0.f, 0.f, 0.f, 0.f};
      static_for<KS>([&](auto cc) {
        constexpr int ks = decltype(cc)::value;
        s1[j] = mfma16x16x32(key_operand<KB, KW32, ks>(tK, kw), qr[ks], s1[j]);
        const half8 sg = nib2x4<ks>(tS, sw);
        s2[j] = mfma16x16x32(sg, qp[ks], s2[j]);
        if constexpr (!PACK) s2[j] = mfma16x16x32(sg, ql[ks], s2[j]);
      });
      if constexpr (PACK) {
#pragma unroll
        for (int e = 0; e < 4; ++e) s2[j][e] += dpp_row_ror8(s2[j][e]);
      }
    }
    // ---- log2-domain scores of keys ks0 + 16j + 4lg + e for this column
    float sc[NBS][4];
#pragma unroll
    for (int j = 0; j < NBS; ++j) {
      const float4v ka = *reinterpret_cast<const float4v*>(&fw[0][16 * j + 4 * lg]);
      const float4v kb2 = *reinterpret_cast<const float4v*>(&fw[1][16 * j + 4 * lg]);
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[j][e] = fmaf(s2[j][e], kb2[e], s1[j][e] * ka[e]);
    }
    if (ks0 + NK > kend || ks0 + NK - 1 > causal_from || a.mask) {  // wave-uniform edge test
#pragma unroll
      for (int j = 0; j < NBS; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = ks0 + 16 * j + 4 * lg + e;
          if (a.mask && col_ok && key < kend)
            sc[j][e] += fmaxf(a.mask[b * a.smb + h * a.smh + static_cast<int64_t>(qi) * a.smq +
                                     static_cast<int64_t>(key) * a.smk] * LOG2E,
                              -3.0e38f);
          if (key >= kend || key > lim) sc[j][e] = -INFINITY;
        }
    }
    // ---- lazy online softmax over the slab: the column reference m_run moves only
    // when a score exceeds it by more than TAU; p = 2^(s - m_run + PUP)
    float lmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < NBS; ++j) lmax = max3_raw(lmax, max3_raw(sc[j][0], sc[j][1], sc[j][2]), sc[j][3]);
    if (__any(lmax > m_run + TAU)) {
      float t = lmax;
      t = fmaxf(t, __shfl_xor(t, 16, 64));
      t = fmaxf(t, __shfl_xor(t, 32, 64));
      if (t > m_run + TAU) {
        const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - t);
        m_run = t;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) oacc[db] *= alpha;
      }
    }
    const float m_use = (m_run == -INFINITY) ? 0.f : m_run - PUP;
    // ---- values: O^T += V^T (P * vn)^T, two 16-key blocks per 16x16x32 MFMA.  K-slot
    // 8lg + 4h + e of block pair jp is key 16(2jp + h) + 4lg + e: the B operand is the lane's
    // own P values of both blocks, and each A dword is one dim of a key pair (2c, 2c + 1),
    // read from the pair table after interleaving the two keys' code fields
    constexpr uint32_t M = odd_fields<VB>();
#pragma unroll
    for (int jp = 0; jp < NBS / 2; ++jp) {
      half8 pb;
      uint32_t w[2][4];  // value fields of keys 16(2jp + h) + 4lg + kk
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int j = 2 * jp + h;
        const float4v nv = *reinterpret_cast<const float4v*>(&fw[2][16 * j + 4 * lg]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p = __builtin_amdgcn_exp2f(sc[j][e] - m_use);
          l_run += p;
          pb[4 * h + e] = static_cast<_Float16>(p * nv[e]);
        }
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const uint32_t* vp = reinterpret_cast<const uint32_t*>(src + OFF_V + (16 * j + 4 * lg + kk) * VC + vbase);
          if constexpr (VW32 == 2)
            w[h][kk] = __builtin_amdgcn_alignbit(vp[1], vp[0], vshift);
          else
            w[h][kk] = vp[0] >> vshift;
        }
      }
      // parity 0: even dims (fields of key 2c, fields of key 2c + 1 shifted into the odd slots);
      // parity 1: odd dims.  Pair field i of a merged word is dim 2i + parity of the key pair.
#pragma unroll
      for (int par = 0; par < 2; ++par) {
        uint32_t f[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const uint32_t wa = w[h][2 * c], wb = w[h][2 * c + 1];
            f[h][c] = par ? bfi32(M, wb, wa >> VB) : bfi32(M, wb << VB, wa);
          }
        static_for<NPAIR>([&](auto ic) {
          constexpr int i = decltype(ic)::value;
          const int db = 2 * i + par;
          const half8 va = __builtin_bit_cast(half8, u32x4{value_pair<VB, i>(tV, f[0][0]), value_pair<VB, i>(tV, f[0][1]),
                                                           value_pair<VB, i>(tV, f[1][0]), value_pair<VB, i>(tV, f[1][1])});
          oacc[db] = mfma16x16x32(va, pb, oacc[db]);
        });
      }
    }
  };

  // the q fragments (the compiler's only outstanding loads) land before the ring
  // starts, so none of its own waits inside the loop reach back past a DMA
  __builtin_amdgcn_s_waitcnt(0);
  const int k0w = kbeg + wave * NK;
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (k0w + r * SLAB < kend) issue(k0w + r * SLAB, r);
  __syncthreads();  // tables built
  for (int k0 = k0w; k0 < kend; k0 += R * SLAB) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int ks0 = k0 + r * SLAB;
      if (ks0 < kend) {
        // slots issued after this one: those of the next R-1 slabs that exist
        int later = 0;
#pragma unroll
        for (int q = 1; q < R; ++q) later += (ks0 + q * SLAB < kend) ? 1 : 0;
        wait_slot(later);
        slab(mine + r * SLOT, ks0);
        if (ks0 + R * SLAB < kend) issue(ks0 + R * SLAB, r);
      }
    }
  }

  // ---- merge the 4 waves of the block in LDS (reusing the staging area)
  __syncthreads();
  float* mrg = reinterpret_cast<float*>(stage);  // [wave][col][D + 2]
  float l = l_run;
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  float* my = mrg + (wave * 16 + l16) * (D + 2);
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int e = 0; e < 4; ++e) my[(lg * 4 + e) * (D / 16) + db] = oacc[db][e] * vcap;
  if (lg == 0) {
    my[D] = (m_run == -INFINITY) ? m_run : m_run - PUP;
    my[D + 1] = l;
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
      const float* srcm = mrg + (w * 16 + c) * (D + 2);
      const float scw = (srcm[D] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(srcm[D] - mx);
      o += scw * srcm[d];
      ls += scw * srcm[D + 1];
    }
    a.part_o[(pbase + c) * D + d] = o;
    if (d == 0) {
      a.part_ml[(pbase + c) * 2] = mx;
      a.part_ml[(pbase + c) * 2 + 1] = ls;
    }
  }
}

// Materialised scores on the integer MFMA (bit-plane form, PlaneQuery in tq_decode.h), with
// the MFMA accumulators in VGPRs like every kernel of this file: columns lg + 4g (NCG groups
// of 4) per lane group, keys on the N side; unit u of a 32-key slab scores keys 2n + u
// (n = l16), so each lane ends with two adjacent keys of its columns and a score row's 32
// values leave as one 128-byte run.
template <int KB, int R, int NCG, int D>
__global__ void __launch_bounds__(256) decode_scores_i8_kernel(DecodeArgs a) {
  static_assert(R >= 2 && R <= 4, "ring of 2 to 4 slots");
  using PQ = PlaneQuery<KB, NCG, D>;
  constexpr int NK = 32;
  constexpr int KC = D * KB / 8, SC = D / 8;
  constexpr int KLANE = KC / 4, SLANE = SC / 4;  // a lane group's quarter of a code / sign row
  constexpr int SLAB = 4 * NK;
  constexpr int OFF_K = 0, OFF_S = NK * KC, OFF_N = OFF_S + NK * SC;
  constexpr int NRM = NK * 4;
  constexpr int SLOT = OFF_N + 2 * NRM;
  // ring slot r of wave w at (r * 4 + w) * SLOT; the last NSTG slots of the four waves
  // (issued after the query set-up) first serve as the set-up's staging area
  constexpr int STG = 4 * SLOT;
  constexpr int NSTG = (PQ::STAGE_BYTES + STG - 1) / STG;
  static_assert(NSTG < R, "set-up staging fits in the ring and leaves a slot to prefetch");

  __shared__ __attribute__((aligned(16))) uint8_t stage[R * STG];
  uint8_t* const stg = stage + (R - NSTG) * STG;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int split = blockIdx.x, hkv = blockIdx.y, b = blockIdx.z;
  const int64_t bh = static_cast<int64_t>(b) * a.Hkv + hkv;
  const int kbeg = split * a.chunk;
  const int kend = min(a.Sk, kbeg + a.chunk);

  const int64_t g0 = bh * a.ldk;
  const uint8_t* pk = a.kcodes + g0 * KC;
  const uint8_t* ps = a.ksigns + g0 * SC;
  const uint16_t* pkn = a.kvn + g0;
  const uint16_t* prn = a.krn + g0;
  const uint32_t ring_lds = lds_offset(stage) + wave * SLOT;
  constexpr int NKD = (NK * KC + 1023) / 1024, NSD = (NK * SC + 1023) / 1024;
  constexpr int NDMA = NKD + NSD + 2;
  // 16 bytes per lane and round; the plane sizes (256 to 1536 bytes) are multiples of 16
  auto copy_plane = [&](const i32x4& r, uint32_t dst, int bytes, int nrounds) {
    const uint32_t lo = lane * 16;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (c >= nrounds) break;
      if ((c + 1) * 1024 <= bytes || lane * 16 < bytes - c * 1024) dma16(r, dst + c * 1024, lo + c * 1024);
    }
  };
  auto issue = [&](int kb, int slot) {
    const uint32_t dst = ring_lds + slot * STG;
    wait_lds();
    copy_plane(rows_desc(pk, KC, kb, kend), dst + OFF_K, NK * KC, NKD);
    copy_plane(rows_desc(ps, SC, kb, kend), dst + OFF_S, NK * SC, NSD);
    if (lane < 32) {
      dma_u16(rows_desc(pkn, 2, kb, kend), dst + OFF_N, lane * 2);
      dma_u16(rows_desc(prn, 2, kb, kend), dst + OFF_N + NRM, lane * 2);
    }
  };
  auto wait_slot = [&](int later) {
    if (later >= 3) wait_vm<(R >= 4 ? 3 * NDMA : 0)>();
    else if (later == 2) wait_vm<(R >= 3 ? 2 * NDMA : 0)>();
    else if (later == 1) wait_vm<NDMA>();
    else wait_vm<0>();
  };
  // slots 0 .. R-NSTG-1 stream while the queries are set up
  const int k0w = kbeg + wave * NK;
#pragma unroll
  for (int r = 0; r < R - NSTG; ++r)
    if (k0w + r * SLAB < kend) issue(k0w + r * SLAB, r);

  PQ pq;
  pq.setup(a, b, hkv, stg, tid);
  const float* pout = a.scores + (static_cast<int64_t>(b) * a.Hq + hkv * a.G) * a.Sq * a.Sk;
  const uint32_t out_bytes = static_cast<uint32_t>(a.C) * a.Sk * 4;
  uint32_t oo[NCG];
#pragma unroll
  for (int g = 0; g < NCG; ++g) {
    const int c = lg + 4 * g;
    oo[g] = c < a.C ? static_cast<uint32_t>((c % a.G) * a.Sq + c / a.G) * a.Sk * 4 + 8 * l16 : kOutOfRange;
  }
  const float fb = a.coeff;
  __syncthreads();  // every wave holds its fragments: the staging slots join the ring
#pragma unroll
  for (int r = R - NSTG; r < R; ++r)
    if (k0w + r * SLAB < kend) issue(k0w + r * SLAB, r);

  auto slab = [&](const uint8_t* src, int ks0) {
    float sc[NCG][2], t1[2][NCG], t2[2][NCG];
    pq.dots2(src + OFF_K + (2 * l16) * KC + lg * KLANE, src + OFF_S + (2 * l16) * SC + lg * SLANE,
             src + OFF_K + (2 * l16 + 1) * KC + lg * KLANE, src + OFF_S + (2 * l16 + 1) * SC + lg * SLANE, t1, t2);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int row = 2 * l16 + u;
      const float kn = h2f(static_cast<uint16_t>(*reinterpret_cast<const uint32_t*>(src + OFF_N + row * 4)));
      const float rn = fb * h2f(static_cast<uint16_t>(*reinterpret_cast<const uint32_t*>(src + OFF_N + NRM + row * 4)));
#pragma unroll
      for (int g = 0; g < NCG; ++g) sc[g][u] = fmaf(t1[u][g], kn, t2[u][g] * rn);
    }
    const int key = ks0 + 2 * l16;
    if (key < kend) {
      const rsrc_t ro = make_rsrc(pout + ks0, out_bytes - static_cast<uint32_t>(ks0) * 4);
#pragma unroll
      for (int g = 0; g < NCG; ++g) {
        if (key + 1 < kend)
          __builtin_amdgcn_raw_buffer_store_b64(
              u32x2{__builtin_bit_cast(uint32_t, sc[g][0]), __builtin_bit_cast(uint32_t, sc[g][1])}, ro, oo[g], 0, 2);
        else
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, sc[g][0]), ro, oo[g], 0, 2);
      }
    }
  };

  // every outstanding load of the compiler's own (the query reads) has landed at the
  // barriers above, so its waits inside the loop never reach back past a DMA
  for (int k0 = k0w; k0 < kend; k0 += R * SLAB) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int ks0 = k0 + r * SLAB;
      if (ks0 < kend) {
        int later = 0;
#pragma unroll
        for (int q = 1; q < R; ++q) later += (ks0 + q * SLAB < kend) ? 1 : 0;
        wait_slot(later);
        slab(stage + r * STG + wave * SLOT, ks0);
        if (ks0 + R * SLAB < kend) issue(ks0 + R * SLAB, r);
      }
    }
  }
}

template <int D>
static void launch_scores_planes_d(const DecodeArgs& a, int bits, hipStream_t s) {
  // head_dim 64 with 1-bit codes and two column groups stages its set-up over 3 ring slots
  constexpr int R = D == 64 ? 4 : 3;
  const dim3 grid(a.nsplit, a.Hkv, a.B);
  if (a.C > 4) {
    if (bits == 2) decode_scores_i8_kernel<1, R, 2, D><<<grid, 256, 0, s>>>(a);
    else decode_scores_i8_kernel<2, R, 2, D><<<grid, 256, 0, s>>>(a);
  } else {
    if (bits == 2) decode_scores_i8_kernel<1, R, 1, D><<<grid, 256, 0, s>>>(a);
    else decode_scores_i8_kernel<2, R, 1, D><<<grid, 256, 0, s>>>(a);
  }
}

void launch_scores_planes(const DecodeArgs& a, int bits, int d, hipStream_t s) {
  if (d == 64) launch_scores_planes_d<64>(a, bits, s);
  else launch_scores_planes_d<128>(a, bits, s);
}

// Fused decode attention for 1- and 2-bit key codes and at most 8 columns, scores on the
// integer MFMA in bit-plane form (PlaneQuery, tq_decode.h) with the keys on the N side:
// lane (key n, group g) scores key n of each 16-key block for columns g, g + 4 (NCG column
// groups of 4), so the softmax runs once per (column, key) instead of once per MFMA column.
// P goes through a small per-wave LDS tile into the P^T operand of the value MFMA (the same
// O^T += V^T P^T step as decode_attn_lds_kernel, with column n of O^T serving column
// n & (4 NCG - 1)); the value decode is shared by all of a kv head's columns.
//
// MASK (an additive mask is applied): scores stay absolute until the column maximum is
// settled and are made relative to it after the rescale test.  The unmasked form folds the
// reference into the score fmas (s - mref), which is exact only while mref is of the order
// of real scores: a leading slab masked with finfo.min (clamped to -3e38) would set mref to
// -3e38, and s - mref would then round every later real score to the same value.
template <int KB, int R, bool MASK, int NCG, int D>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NCG == 1 ? 4 : 3)))
decode_attn_i8_kernel(DecodeArgs a) {
  constexpr int BITS = KB + 1;
  using L = SmallLuts<BITS>;
  using PQ = PlaneQuery<KB, NCG, D>;
  constexpr int NC = PQ::NC;
  constexpr int VB = L::VB;
  constexpr int DB = D / 16;    // value-MFMA row blocks: lane l16 holds dims DB l16 .. DB l16 + DB - 1
  constexpr int NPAIR = D / 32; // pair-table groups per parity
  constexpr int KC = D * KB / 8, SC = D / 8, VC = D * VB / 8;
  constexpr int KLANE = KC / 4, SLANE = SC / 4;
  constexpr int VFB = DB * VB;  // value field bits of a lane
  constexpr int VW32 = (VB == 3) ? 2 : 1;  // 3-bit fields may straddle a dword
  constexpr int NK = 32;
  constexpr int SLAB = 4 * NK;
  constexpr int OFF_K = 0, OFF_S = NK * KC, OFF_V = OFF_S + NK * SC, OFF_N = OFF_V + NK * VC;
  constexpr int NRM = NK * 4;
  constexpr int SLOT = OFF_N + 3 * NRM;
  // slot r of the four waves at r * STG; the last NSTG slots (issued after the query set-up)
  // first serve as the set-up's staging area
  constexpr int STG = 4 * SLOT;
  constexpr int NSTG = (PQ::STAGE_BYTES + STG - 1) / STG;
  constexpr int MERGE = 4 * NC * (D + 2) * 4;
  constexpr int STAGE = R * STG > MERGE ? R * STG : MERGE;
  static_assert(NSTG < R, "set-up staging fits in the ring and leaves a slot to prefetch");
  static_assert(R >= 2 && R <= 3, "ring of 2 or 3 slots");
  constexpr float LOG2E = 1.4426950408889634f;
  constexpr float TAU = 8.0f;
  constexpr float PUP = 6.0f;  // the same weight scaling as decode_attn_lds_kernel

  __shared__ __attribute__((aligned(16))) uint8_t luts[L::BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t stage[STAGE];
  __shared__ __attribute__((aligned(16))) _Float16 ptile[4][NC][NK];  // per wave: P [column][key]
  const uint8_t* tV = luts + L::VAL_OFF;
  uint8_t* const stg = stage + (R - NSTG) * STG;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int split = blockIdx.x, hkv = blockIdx.y, b = blockIdx.z;
  const int64_t bh = static_cast<int64_t>(b) * a.Hkv + hkv;

  build_small_luts<BITS, true>(a, luts, tid);

  // this lane's score columns lg + 4g
  bool c_ok[NCG];
  int lim[NCG];
  const float* mrow[NCG];  // MASK: the column's mask row (key 0)
#pragma unroll
  for (int g = 0; g < NCG; ++g) {
    const int c = lg + 4 * g;
    c_ok[g] = c < a.C;
    const int qi = c_ok[g] ? c / a.G : 0, h = hkv * a.G + (c_ok[g] ? c % a.G : 0);
    lim[g] = a.causal ? qi + (a.Sk - a.Sq) : 0x7fffffff;
    mrow[g] = MASK ? a.mask + (b * a.smb + h * a.smh + static_cast<int64_t>(qi) * a.smq) : nullptr;
  }
  const float fa = a.scale * LOG2E;
  const float fb = a.coeff * fa;
  const int causal_from = a.causal ? a.Sk - a.Sq : 0x7fffffff;
  const int kbeg = split * a.chunk;
  const int kend = min(a.Sk, kbeg + a.chunk);

  // value field of the lane (value-MFMA row l16): VFB bits from bit l16 * VFB of the row
  const int vbit = l16 * VFB;
  const int vbase = (vbit >> 5) * 4;
  const int vshift = vbit & 31;

  const int64_t g0 = bh * a.ldk;
  const uint8_t* pk = a.kcodes + g0 * KC;
  const uint8_t* ps = a.ksigns + g0 * SC;
  const uint16_t* pkn = a.kvn + g0;
  const uint16_t* prn = a.krn + g0;
  const uint16_t* pvn = a.vvn + g0;
  const uint8_t* pv = a.vcodes + g0 * VC;
  const uint32_t ring_lds = lds_offset(stage) + wave * SLOT;
  constexpr int NKD = (NK * KC + 1023) / 1024, NSD = (NK * SC + 1023) / 1024, NVD = (NK * VC + 1023) / 1024;
  constexpr int NDMA = NKD + NSD + NVD + 3;
  // 16 bytes per lane and round; the plane sizes (256 to 1536 bytes) are multiples of 16
  auto copy_plane = [&](const i32x4& r, uint32_t dst, int bytes, int nrounds) {
    const uint32_t lo = lane * 16;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (c >= nrounds) break;
      if ((c + 1) * 1024 <= bytes || lane * 16 < bytes - c * 1024) dma16(r, dst + c * 1024, lo + c * 1024);
    }
  };
  auto issue = [&](int kb, int slot) {
    const uint32_t dst = ring_lds + slot * STG;
    wait_lds();
    copy_plane(rows_desc(pk, KC, kb, kend), dst + OFF_K, NK * KC, NKD);
    copy_plane(rows_desc(ps, SC, kb, kend), dst + OFF_S, NK * SC, NSD);
    copy_plane(rows_desc(pv, VC, kb, kend), dst + OFF_V, NK * VC, NVD);
    if (lane < 32) {
      dma_u16(rows_desc(pkn, 2, kb, kend), dst + OFF_N, lane * 2);
      dma_u16(rows_desc(prn, 2, kb, kend), dst + OFF_N + NRM, lane * 2);
      dma_u16(rows_desc(pvn, 2, kb, kend), dst + OFF_N + 2 * NRM, lane * 2);
    }
  };
  auto wait_slot = [&](int later) {
    if (later >= 2) wait_vm<(R >= 3 ? 2 * NDMA : 0)>();
    else if (later == 1) wait_vm<NDMA>();
    else wait_vm<0>();
  };
  const int k0w = kbeg + wave * NK;
#pragma unroll
  for (int r = 0; r < R - NSTG; ++r)
    if (k0w + r * SLAB < kend) issue(k0w + r * SLAB, r);

  PQ pq;
  pq.setup(a, b, hkv, stg, tid);
  __syncthreads();  // fragments held (and tables built): the staging slots join the ring
#pragma unroll
  for (int r = R - NSTG; r < R; ++r)
    if (k0w + r * SLAB < kend) issue(k0w + r * SLAB, r);

  // column lg + 4g: reference mref = m - PUP (0 until the column has a maximum m) and the
  // threshold a score relative to mref must exceed to move it (-inf until then, TAU + PUP after)
  float mref[NCG], thr[NCG], l_run[NCG];
#pragma unroll
  for (int g = 0; g < NCG; ++g) {
    mref[g] = 0.f;
    thr[g] = -INFINITY;
    l_run[g] = 0.f;
  }
  float vcap = 0x1p-24f, inv_vcap = 0x1p24f;
  float4v oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = float4v{0.f, 0.f, 0.f, 0.f};
  _Float16* const pt = &ptile[wave][0][0];

  auto slab = [&](const uint8_t* src, int ks0) {
    // ---- scores of keys ks0 + 16j + l16 (j = 0, 1) for columns lg + 4g, log2 domain
    float sc[NCG][2], nv[2], t1[2][NCG], t2[2][NCG];
    pq.dots2(src + OFF_K + l16 * KC + lg * KLANE, src + OFF_S + l16 * SC + lg * SLANE,
             src + OFF_K + (16 + l16) * KC + lg * KLANE, src + OFF_S + (16 + l16) * SC + lg * SLANE, t1, t2);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int row = 16 * j + l16;
      const float kn = h2f(static_cast<uint16_t>(*reinterpret_cast<const uint32_t*>(src + OFF_N + row * 4)));
      const float rn = h2f(static_cast<uint16_t>(*reinterpret_cast<const uint32_t*>(src + OFF_N + NRM + row * 4)));
      nv[j] = h2f(static_cast<uint16_t>(*reinterpret_cast<const uint32_t*>(src + OFF_N + 2 * NRM + row * 4)));
      const float ka = fa * kn, kb = fb * rn;
      // s - mref; absolute s under a mask (made relative after the rescale test)
#pragma unroll
      for (int g = 0; g < NCG; ++g)
        sc[g][j] = fmaf(t1[j][g], ka, MASK ? t2[j][g] * kb : fmaf(t2[j][g], kb, -mref[g]));
    }
    // ---- value norms enter P as vn / vcap <= 1; vcap is a power of two that only grows
    {
      const float vmx = max_raw(nv[0], nv[1]);
      if (__any(vmx > vcap)) {
        float t = vmx;
#pragma unroll
        for (int sh = 32; sh >= 1; sh >>= 1) t = fmaxf(t, __shfl_xor(t, sh, 64));
        int ex;
        frexpf(t, &ex);
        ex = __builtin_amdgcn_readfirstlane(ex);
        const float cap = ldexpf(1.f, ex);
        const float shrink = vcap / cap;
#pragma unroll
        for (int db = 0; db < DB; ++db) oacc[db] *= shrink;
        vcap = cap;
        inv_vcap = ldexpf(1.f, -ex);
      }
    }
    if (MASK || ks0 + NK > kend || ks0 + NK - 1 > causal_from) {  // wave-uniform edge test
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int key = ks0 + 16 * j + l16;
#pragma unroll
        for (int g = 0; g < NCG; ++g) {
          if (MASK && c_ok[g] && key < kend)
            sc[g][j] += fmaxf(mrow[g][static_cast<int64_t>(key) * a.smk] * LOG2E, -3.0e38f);
          if (key >= kend || key > lim[g]) sc[g][j] = -INFINITY;
        }
      }
    }
    // ---- lazy online softmax: column c's maximum m (uniform over the 16 lanes of the column)
    // moves only when a score exceeds it by more than TAU; p = 2^(s - m + PUP) = 2^sc
    float lmax[NCG];
    bool hit = false;
#pragma unroll
    for (int g = 0; g < NCG; ++g) {
      lmax[g] = max_raw(sc[g][0], sc[g][1]);
      hit = hit || (MASK ? lmax[g] - mref[g] : lmax[g]) > thr[g];
    }
    if (__any(hit)) {
      float alpha[NCG];
#pragma unroll
      for (int g = 0; g < NCG; ++g) {
        float t = lmax[g];
#pragma unroll
        for (int sh = 8; sh >= 1; sh >>= 1) t = fmaxf(t, __shfl_xor(t, sh, 64));
        alpha[g] = 1.f;
        if ((MASK ? t - mref[g] : t) > thr[g]) {
          const float mref_new = (MASK ? t : t + mref[g]) - PUP;
          alpha[g] = (thr[g] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mref[g] - mref_new);
          if constexpr (!MASK) {
            const float shift = mref_new - mref[g];
            sc[g][0] -= shift;
            sc[g][1] -= shift;
          }
          mref[g] = mref_new;
          thr[g] = TAU + PUP;
          l_run[g] *= alpha[g];
        }
      }
      // O^T column l16 serves column l16 & (NC - 1), held by lane group l16 & 3
      float ac = __shfl(alpha[0], 16 * (l16 & 3), 64);
      if constexpr (NCG == 2) {
        const float a1 = __shfl(alpha[1], 16 * (l16 & 3), 64);
        ac = (l16 & 4) ? a1 : ac;
      }
#pragma unroll
      for (int db = 0; db < DB; ++db) oacc[db] *= ac;
    }
    if constexpr (MASK) {
      // relative to the settled reference: a column that has seen only masked keys (all at
      // -3e38) gives them equal weights, as the reference's softmax of equal scores does
#pragma unroll
      for (int g = 0; g < NCG; ++g) {
        sc[g][0] -= mref[g];
        sc[g][1] -= mref[g];
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float vs = nv[j] * inv_vcap;
#pragma unroll
      for (int g = 0; g < NCG; ++g) {
        const float p = __builtin_amdgcn_exp2f(sc[g][j]);
        l_run[g] += p;
        pt[(lg + 4 * g) * NK + 16 * j + l16] = static_cast<_Float16>(p * vs);
      }
    }
    // ---- values: O^T += V^T (P * vn)^T over the slab's 32 keys in one 16x16x32 MFMA per row
    // block: K-slot 8lg + 4j + e is key 16j + 4lg + e; the B operand (column l16) reads
    // column l16 & (NC - 1) of the P tile
    half8 pb;
    {
      const _Float16* pr = pt + (l16 & (NC - 1)) * NK + 4 * lg;
      const u32x2 p0 = *reinterpret_cast<const u32x2*>(pr);
      const u32x2 p1 = *reinterpret_cast<const u32x2*>(pr + 16);
      pb = __builtin_bit_cast(half8, u32x4{p0[0], p0[1], p1[0], p1[1]});
    }
    constexpr uint32_t M = odd_fields<VB>();
    uint32_t w[2][4];  // value fields of keys 16j + 4lg + kk
    // the 8 row reads issued as one batch (the compiler otherwise reuses one register pair and
    // waits after each)
    uint32_t r0[2][4], r1[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const uint32_t* vp = reinterpret_cast<const uint32_t*>(src + OFF_V + (16 * j + 4 * lg + kk) * VC + vbase);
        r0[j][kk] = vp[0];
        if constexpr (VW32 == 2) r1[j][kk] = vp[1];
      }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if constexpr (VW32 == 2)
          w[j][kk] = __builtin_amdgcn_alignbit(r1[j][kk], r0[j][kk], vshift);
        else
          w[j][kk] = r0[j][kk] >> vshift;
      }
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      uint32_t f[2][2];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const uint32_t wa = w[j][2 * c], wb = w[j][2 * c + 1];
          f[j][c] = par ? bfi32(M, wb, wa >> VB) : bfi32(M, wb << VB, wa);
        }
      // pair-table lookups one MFMA ahead: group i + 1 is read while the MFMA of group i runs
      auto look = [&](auto ic) {
        constexpr int i = decltype(ic)::value;
        return __builtin_bit_cast(half8, u32x4{value_pair<VB, i>(tV, f[0][0]), value_pair<VB, i>(tV, f[0][1]),
                                               value_pair<VB, i>(tV, f[1][0]), value_pair<VB, i>(tV, f[1][1])});
      };
      half8 va = look(std::integral_constant<int, 0>{});
      static_for<NPAIR>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        half8 vn = va;
        if constexpr (i + 1 < NPAIR) vn = look(std::integral_constant<int, i + 1>{});
        __builtin_amdgcn_sched_barrier(0);
        oacc[2 * i + par] = mfma16x16x32(va, pb, oacc[2 * i + par]);
        va = vn;
      });
    }
  };

  for (int k0 = k0w; k0 < kend; k0 += R * SLAB) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int ks0 = k0 + r * SLAB;
      if (ks0 < kend) {
        int later = 0;
#pragma unroll
        for (int q = 1; q < R; ++q) later += (ks0 + q * SLAB < kend) ? 1 : 0;
        wait_slot(later);
        slab(stage + r * STG + wave * SLOT, ks0);
        if (ks0 + R * SLAB < kend) issue(ks0 + R * SLAB, r);
      }
    }
  }

  // ---- merge the 4 waves of the block in LDS (reusing the staging area)
  __syncthreads();
  float* mrg = reinterpret_cast<float*>(stage);  // [wave][column < NC][D + 2]
  float l[NCG];
#pragma unroll
  for (int g = 0; g < NCG; ++g) {
    l[g] = l_run[g];
#pragma unroll
    for (int sh = 8; sh >= 1; sh >>= 1) l[g] += __shfl_xor(l[g], sh, 64);
  }
  if (l16 < NC) {
    float* my = mrg + (wave * NC + l16) * (D + 2);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int e = 0; e < 4; ++e) my[(lg * 4 + e) * (D / 16) + db] = oacc[db][e] * vcap;
  }
  if (l16 == 0) {
#pragma unroll
    for (int g = 0; g < NCG; ++g) {
      float* my = mrg + (wave * NC + lg + 4 * g) * (D + 2);
      my[D] = (thr[g] == -INFINITY) ? -INFINITY : mref[g];
      my[D + 1] = l[g];
    }
  }
  __syncthreads();
  const int64_t pbase = (bh * a.nsplit + split) * a.C;
  for (int it = tid; it < a.C * D; it += 256) {
    const int c = it / D, d = it % D;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) mx = fmaxf(mx, mrg[(w * NC + c) * (D + 2) + D]);
    float o = 0.f, ls = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float* srcm = mrg + (w * NC + c) * (D + 2);
      const float scw = (srcm[D] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(srcm[D] - mx);
      o += scw * srcm[d];
      ls += scw * srcm[D + 1];
    }
    a.part_o[(pbase + c) * D + d] = o;
    if (d == 0) {
      a.part_ml[(pbase + c) * 2] = mx;
      a.part_ml[(pbase + c) * 2 + 1] = ls;
    }
  }
}

// splits the one-wave-per-column merge loads in its first round trip; shapes with more take
// decode_merge_split_kernel (measured, C ABI, bits 3: 32/8 heads B1 x 32k keys, 128 splits,
// 25.7 -> 21.9 us for attention + merge; at 8 splits, B16 x 32k, the per-column blocks'
// extra Pi_v fragment reads made it 4% slower)
constexpr int kMergeSplitsPerWave = 16;

struct MergeArgs {
  const float *part_o, *part_ml;
  const uint16_t* vpit;  // split Pi_v^T
  int B, Hq, Hkv, Sq, G, C, nsplit;
  void* out;
  int out_dtype;
  int64_t sob, soh, sos;
};

// One block per (batch, kv head, group of 4 columns): combine the splits of its columns with
// log-sum-exp weights into o[c][:] (LDS), then out^T = Pi_v^T o^T on MFMA with
// Pi_v^T as the split-f16 A operand (rows i = output dim) and o^T as split-f16 B
// operand (columns c, scaled per column by a power of two), hi.hi + lo.hi + hi.lo.
// The kernel is latency-bound (a few KB per block), so it is laid out as few dependent
// round trips as possible: each wave first issues the loads of its Pi_v^T fragments,
// then combines one whole column (c = 4 blockIdx.z + wave) on its own: split maxima and
// weights by wave reductions, and 2 dims per lane summed over all splits with the loads
// of a batch issued together; one block barrier precedes the Pi_v product.  Columns beyond
// the first 4 of a kv head go to further blocks rather than further rounds of a wave.
template <int D>
__global__ void __launch_bounds__(256) decode_merge_kernel(MergeArgs a) {
  static_assert(D == 128, "merge is built for head_dim 128");
  constexpr int SW = 64;  // splits per weight batch (one per lane)
  __shared__ float o_s[4 * D];
  __shared__ float s_w[4][SW];
  __shared__ float s_up[4];
  const int hkv = blockIdx.x, b = blockIdx.y, c0 = blockIdx.z * 4, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, l16 = lane & 15, lg = lane >> 4;
  const int C = a.C, ns = a.nsplit;
  const int64_t base = (static_cast<int64_t>(b) * a.Hkv + hkv) * ns;  // first split record

  // ---- Pi_v^T fragments of this wave's output rows 32w .. 32w+31 (in flight meanwhile)
  const _Float16* Ph = reinterpret_cast<const _Float16*>(a.vpit);
  const _Float16* Pl = Ph + D * D;
  half8 ah[2][D / 32], al[2][D / 32];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int i = wave * 32 + rb * 16 + l16;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      ah[rb][ks] = *reinterpret_cast<const half8*>(Ph + i * D + ks * 32 + lg * 8);
      al[rb][ks] = *reinterpret_cast<const half8*>(Pl + i * D + ks * 32 + lg * 8);
    }
  }

  // ---- column c = c0 + wave: o[c] = sum_s w_s o_s / sum_s w_s l_s
  for (int c = c0 + wave; c < c0 + 4; c += 4) {
    float* oc = o_s + (c - c0) * D;
    if (c >= C) {
      oc[2 * lane] = 0.f;
      oc[2 * lane + 1] = 0.f;
      if (lane == 0) s_up[c - c0] = 1.f;
      continue;
    }
    auto ml = [&](int s, int k) { return a.part_ml[((base + s) * C + c) * 2 + k]; };
    const int64_t step = static_cast<int64_t>(C) * D;
    const float* src0 = a.part_o + (base * C + c) * D + 2 * lane;
    // one memory round trip for up to NB0 splits (the decode shapes: 8 at 16 sequences x 32k
    // keys, 16 at one sequence x 4k): the first NB0 splits' partial o and this lane's split
    // maximum and sum are all issued before any is used
    constexpr int NB0 = kMergeSplitsPerWave;
    float2 v0[NB0];
#pragma unroll
    for (int u = 0; u < NB0; ++u)
      v0[u] = u < ns ? *reinterpret_cast<const float2*>(src0 + u * step) : float2{0.f, 0.f};
    const float m_first = lane < ns ? ml(lane, 0) : -INFINITY;
    const float l_first = lane < ns ? ml(lane, 1) : 0.f;
    float mx = m_first;
    for (int s = lane + SW; s < ns; s += SW) mx = fmaxf(mx, ml(s, 0));
#pragma unroll
    for (int sh = 32; sh >= 1; sh >>= 1) mx = fmaxf(mx, __shfl_xor(mx, sh, 64));
    float lsum = 0.f, o0 = 0.f, o1 = 0.f;
    for (int s0 = 0; s0 < ns; s0 += SW) {
      const int s = s0 + lane;
      float w = 0.f;
      if (s < ns) {
        const float m = s0 == 0 ? m_first : ml(s, 0);
        w = (m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - mx);
        lsum += w * (s0 == 0 ? l_first : ml(s, 1));
      }
      s_w[wave][lane] = w;  // read back by the same wave only: LDS order suffices
      const int nb = min(SW, ns - s0);
      const float* src = src0 + s0 * step;
      int k = 0;
      if (s0 == 0) {
        // the preloaded first batch (splits past ns hold zeros and weight 0)
#pragma unroll
        for (int u = 0; u < NB0; ++u) {
          const float ww = u < nb ? s_w[wave][u] : 0.f;
          o0 = fmaf(ww, v0[u].x, o0);
          o1 = fmaf(ww, v0[u].y, o1);
        }
        k = min(NB0, nb);
      }
      for (; k + 16 <= nb; k += 16) {
        float2 v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = *reinterpret_cast<const float2*>(src + (k + u) * step);
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const float ww = s_w[wave][k + u];
          o0 = fmaf(ww, v[u].x, o0);
          o1 = fmaf(ww, v[u].y, o1);
        }
      }
      for (; k < nb; ++k) {
        const float2 v = *reinterpret_cast<const float2*>(src + k * step);
        const float ww = s_w[wave][k];
        o0 = fmaf(ww, v.x, o0);
        o1 = fmaf(ww, v.y, o1);
      }
    }
#pragma unroll
    for (int sh = 32; sh >= 1; sh >>= 1) lsum += __shfl_xor(lsum, sh, 64);
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    o0 *= inv;
    o1 *= inv;
    oc[2 * lane] = o0;
    oc[2 * lane + 1] = o1;
    float m = fmaxf(fabsf(o0), fabsf(o1));
#pragma unroll
    for (int sh = 32; sh >= 1; sh >>= 1) m = fmaxf(m, __shfl_xor(m, sh, 64));
    if (lane == 0) {
      int ex;
      frexpf(m, &ex);
      s_up[c - c0] = ldexpf(kSplit, -ex);  // scaled |o| < kSplit
    }
  }
  __syncthreads();

  // ---- out^T[i][c] = sum_j Pi_v^T[i][j] o[c][j]; wave w owns output rows 32w .. 32w+31;
  // MFMA column l16 < 4 is column c0 + l16 (the other 12 repeat them and are not stored)
  const float up = s_up[l16 & 3];
  half8 bh[D / 32], bl[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
    const float* src = o_s + (l16 & 3) * D + ks * 32 + lg * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      _Float16 h, lo;
      split_f16(src[e] * up, h, lo);
      bh[ks][e] = h;
      bl[ks][e] = lo;
    }
  }
  const bool col_ok = l16 < 4 && c0 + l16 < C;
  const int qi = col_ok ? (c0 + l16) / a.G : 0, h = hkv * a.G + (col_ok ? (c0 + l16) % a.G : 0);
  const float down = kUnsplit2 / up;  // 1/(kSplit * up) * (1/kSplit) for Pi_v^T's scale
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    float4v f = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      f = mfma16x16x32(ah[rb][ks], bh[ks], f);
      f = mfma16x16x32(al[rb][ks], bh[ks], f);
      f = mfma16x16x32(ah[rb][ks], bl[ks], f);
    }
    if (col_ok) {
      const int64_t off = static_cast<int64_t>(b) * a.sob + static_cast<int64_t>(h) * a.soh +
                          static_cast<int64_t>(qi) * a.sos + wave * 32 + rb * 16 + lg * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = f[e] * (down * kSplit);
        if (a.out_dtype == TQ_BF16) store_act<TQ_BF16>(a.out, off + e, v);
        else if (a.out_dtype == TQ_F16) store_act<TQ_F16>(a.out, off + e, v);
        else store_act<TQ_F32>(a.out, off + e, v);
      }
    }
  }
}

// The same merge for many splits (decode_merge_kernel walks a column's splits in one wave,
// a batch of 16 per memory round trip): one block per (column, kv head, batch) combines the
// column's splits with log-sum-exp
// weights into o[:], then out = Pi_v^T o on MFMA with Pi_v^T as the split-f16 A operand
// (rows i = output dim) and o as split-f16 B operand (scaled by a power of two; every MFMA
// column holds it, column 0 is stored), hi.hi + lo.hi + hi.lo.  The kernel is latency-bound
// (a few KB per block), so it is laid out as few dependent round trips as possible: each wave
// issues the loads of its Pi_v^T fragments, of the partial o of its splits (wave w takes
// splits w, w + 4, ..., up to NB of them per batch) and of their maxima and sums together;
// the block maximum crosses one barrier, each wave sums its splits (2 dims per lane), and
// the waves' partial sums cross a second barrier before the Pi_v product.
template <int D>
__global__ void __launch_bounds__(256) decode_merge_split_kernel(MergeArgs a) {
  static_assert(D == 64 || D == 128, "merge is built for head_dim 64 or 128");
  constexpr int NB = 16;       // splits per wave per load batch
  constexpr int PL = D / 64;   // dims per lane in the combine
  constexpr int RB = D / 64;   // 16-row output blocks per wave
  typedef float floatPL __attribute__((ext_vector_type(PL)));
  __shared__ float s_m[4], s_l[4];
  __shared__ __attribute__((aligned(16))) float s_o[4][D];
  const int c = blockIdx.x, hkv = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, l16 = lane & 15, lg = lane >> 4;
  const int C = a.C, ns = a.nsplit;
  const int64_t base = (static_cast<int64_t>(b) * a.Hkv + hkv) * ns;  // first split record

  // ---- Pi_v^T fragments of this wave's output rows (D / 4) w .. (D / 4) w + D / 4 - 1 (in
  // flight meanwhile)
  const _Float16* Ph = reinterpret_cast<const _Float16*>(a.vpit);
  const _Float16* Pl = Ph + D * D;
  half8 ah[RB][D / 32], al[RB][D / 32];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int i = wave * (D / 4) + rb * 16 + l16;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      ah[rb][ks] = *reinterpret_cast<const half8*>(Ph + i * D + ks * 32 + lg * 8);
      al[rb][ks] = *reinterpret_cast<const half8*>(Pl + i * D + ks * 32 + lg * 8);
    }
  }

  // ---- this wave's splits w + 4u, u < nw: partial o (first batch), maxima and sums
  const int nw = ns > wave ? (ns - wave + 3) / 4 : 0;
  const int64_t ostep = 4 * static_cast<int64_t>(C) * D;  // floats between the wave's splits
  const int64_t mstep = 4 * 2 * static_cast<int64_t>(C);
  const float* src0 = a.part_o + ((base + wave) * C + c) * D + PL * lane;
  const float* ml0 = a.part_ml + ((base + wave) * C + c) * 2;
  auto load = [&](int64_t off) { return *reinterpret_cast<const floatPL*>(src0 + off); };
  floatPL v0[NB];
#pragma unroll
  for (int u = 0; u < NB; ++u) v0[u] = u < nw ? load(u * ostep) : floatPL{};
  const float m_first = lane < nw ? ml0[lane * mstep] : -INFINITY;
  const float l_first = lane < nw ? ml0[lane * mstep + 1] : 0.f;
  float mx = m_first;
  for (int u = lane + 64; u < nw; u += 64) mx = fmaxf(mx, ml0[u * mstep]);
#pragma unroll
  for (int sh = 32; sh >= 1; sh >>= 1) mx = fmaxf(mx, __shfl_xor(mx, sh, 64));
  if (lane == 0) s_m[wave] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));

  // ---- o_w = sum_u wt_u o_u, l_w = sum_u wt_u l_u, wt_u = 2^(m_u - M); lane u holds wt_u of
  // its batch of 64 and every lane reads it back with v_readlane
  floatPL o = floatPL{};
  float lsum = 0.f;
  for (int s0 = 0; s0 < nw; s0 += 64) {
    const int u = s0 + lane;
    float w = 0.f;
    if (u < nw) {
      const float m = s0 == 0 ? m_first : ml0[u * mstep];
      w = (m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - M);
      lsum += w * (s0 == 0 ? l_first : ml0[u * mstep + 1]);
    }
    const int nb = min(64, nw - s0);
    int k = 0;
    if (s0 == 0) {
      // the first batch, loaded above (splits past nw hold zeros and weight 0)
#pragma unroll
      for (int uu = 0; uu < NB; ++uu) {
        const float ww = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), uu));
#pragma unroll
        for (int e = 0; e < PL; ++e) o[e] = fmaf(ww, v0[uu][e], o[e]);
      }
      k = NB;
    }
    for (; k < nb; k += NB) {
      floatPL v[NB];
#pragma unroll
      for (int uu = 0; uu < NB; ++uu) v[uu] = k + uu < nb ? load((s0 + k + uu) * ostep) : floatPL{};
#pragma unroll
      for (int uu = 0; uu < NB; ++uu) {
        const float ww = k + uu < 64 ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), k + uu)) : 0.f;
#pragma unroll
        for (int e = 0; e < PL; ++e) o[e] = fmaf(ww, v[uu][e], o[e]);
      }
    }
  }
#pragma unroll
  for (int sh = 32; sh >= 1; sh >>= 1) lsum += __shfl_xor(lsum, sh, 64);
  *reinterpret_cast<floatPL*>(&s_o[wave][PL * lane]) = o;
  if (lane == 0) s_l[wave] = lsum;
  __syncthreads();

  // ---- o = sum_w o_w / sum_w l_w as this lane's B operand dims ks*32 + lg*8 + e, scaled so
  // that |o| < kSplit (the same scale in every wave: every wave builds the same operand)
  const float L = (s_l[0] + s_l[1]) + (s_l[2] + s_l[3]);
  const float inv = L > 0.f ? 1.f / L : 0.f;
  float ov[D / 32][8];
  float om = 0.f;
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
    const int d0 = ks * 32 + lg * 8;
#pragma unroll
    for (int h4 = 0; h4 < 2; ++h4) {
      float4 t = *reinterpret_cast<const float4*>(&s_o[0][d0 + 4 * h4]);
#pragma unroll
      for (int w = 1; w < 4; ++w) {
        const float4 x = *reinterpret_cast<const float4*>(&s_o[w][d0 + 4 * h4]);
        t.x += x.x;
        t.y += x.y;
        t.z += x.z;
        t.w += x.w;
      }
      ov[ks][4 * h4 + 0] = t.x * inv;
      ov[ks][4 * h4 + 1] = t.y * inv;
      ov[ks][4 * h4 + 2] = t.z * inv;
      ov[ks][4 * h4 + 3] = t.w * inv;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) om = fmaxf(om, fabsf(ov[ks][e]));
  }
#pragma unroll
  for (int sh = 32; sh >= 16; sh >>= 1) om = fmaxf(om, __shfl_xor(om, sh, 64));  // over lane groups
  int ex;
  frexpf(om, &ex);
  const float up = ldexpf(kSplit, -ex);  // scaled |o| < kSplit
  half8 bh[D / 32], bl[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      _Float16 hh, lo;
      split_f16(ov[ks][e] * up, hh, lo);
      bh[ks][e] = hh;
      bl[ks][e] = lo;
    }
  }
  // ---- out[i] = sum_j Pi_v^T[i][j] o[j]; wave w owns output rows (D / 4) w .. (D / 4) w + D / 4 - 1
  const int qi = c / a.G, h = hkv * a.G + c % a.G;
  const float down = kUnsplit2 / up;  // 1/(kSplit * up) * (1/kSplit) for Pi_v^T's scale
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    float4v f = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      f = mfma16x16x32(ah[rb][ks], bh[ks], f);
      f = mfma16x16x32(al[rb][ks], bh[ks], f);
      f = mfma16x16x32(ah[rb][ks], bl[ks], f);
    }
    if (l16 == 0) {
      const int64_t off = static_cast<int64_t>(b) * a.sob + static_cast<int64_t>(h) * a.soh +
                          static_cast<int64_t>(qi) * a.sos + wave * (D / 4) + rb * 16 + lg * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = f[e] * (down * kSplit);
        if (a.out_dtype == TQ_BF16) store_act<TQ_BF16>(a.out, off + e, v);
        else if (a.out_dtype == TQ_F16) store_act<TQ_F16>(a.out, off + e, v);
        else store_act<TQ_F32>(a.out, off + e, v);
      }
    }
  }
}

// bit-plane kernel for 1- and 2-bit key codes and at most 8 columns (one or two groups of 4)
static bool attn_planes(int bits, int C) { return bits <= 3 && C <= 8; }
// ring slots: head_dim 128 stages the query set-up in one slot, head_dim 64 (smaller slots)
// in up to two
template <int D>
constexpr int attn_plane_ring() {
  return D == 64 ? 3 : 2;
}

template <int KB, int NCG, int D>
static const void* attn_i8_kernel() {
  return reinterpret_cast<const void*>(&decode_attn_i8_kernel<KB, attn_plane_ring<D>(), false, NCG, D>);
}

// grid target of the fused decode attention: one round of resident blocks
static int attn_target_blocks(int bits, int C, int d) {
  static int cache[14][16] = {};
  if (attn_planes(bits, C)) {
    const bool two = C > 4;
    const void* k;
    if (d == 64)
      k = bits == 2 ? (two ? attn_i8_kernel<1, 2, 64>() : attn_i8_kernel<1, 1, 64>())
                    : (two ? attn_i8_kernel<2, 2, 64>() : attn_i8_kernel<2, 1, 64>());
    else
      k = bits == 2 ? (two ? attn_i8_kernel<1, 2, 128>() : attn_i8_kernel<1, 1, 128>())
                    : (two ? attn_i8_kernel<2, 2, 128>() : attn_i8_kernel<2, 1, 128>());
    return resident_blocks(k, 256, cache[bits + 1 + (two ? 2 : 0) + (d == 64 ? 4 : 0)]);
  }
  if (d == 64) {
    const void* k = bits == 2 ? reinterpret_cast<const void*>(&decode_attn_lds_kernel<64, 2, kAttnNbs, kAttnRing, true>)
                  : bits == 3 ? reinterpret_cast<const void*>(&decode_attn_lds_kernel<64, 3, kAttnNbs, kAttnRing, true>)
                              : reinterpret_cast<const void*>(&decode_attn_lds_kernel<64, 4, kAttnNbs, kAttnRing, true>);
    return resident_blocks(k, 256, cache[11 + bits - 2]);
  }
  const void* k = bits == 2 ? reinterpret_cast<const void*>(&decode_attn_lds_kernel<128, 2, kAttnNbs, kAttnRing, true>)
                : bits == 3 ? reinterpret_cast<const void*>(&decode_attn_lds_kernel<128, 3, kAttnNbs, kAttnRing, true>)
                            : reinterpret_cast<const void*>(&decode_attn_lds_kernel<128, 4, kAttnNbs, kAttnRing, true>);
  return resident_blocks(k, 256, cache[bits - 2]);
}

static DecodePlan plan_decode(int B, int Hq, int Hkv, int Sq, int Sk, int d, int bits) {
  if (!decode_shape(Hq, Hkv, Sq, Sk, d, bits)) return DecodePlan{false, 0, 0, 0};
  constexpr int slab = 64 * kAttnNbs;  // 4 waves x 32 keys for both kernels
  const int C = (Hq / Hkv) * Sq;
  DecodePlan p = plan_split(B, Hkv, Sk, attn_target_blocks(bits, C, d), slab, 2 * slab);
  p.ws_bytes = static_cast<int64_t>(B) * Hkv * p.nsplit * C * static_cast<int64_t>(d + 2) * 4;
  return p;
}

}  // namespace tq

using namespace tq;

namespace tq {

int64_t decode_workspace_bytes(int B, int Hq, int Hkv, int Sq, int Sk, int d, int bits) {
  const DecodePlan p = plan_decode(B, Hq, Hkv, Sq, Sk, d, bits);
  return p.use ? p.ws_bytes : 0;
}

bool decode_applies(int B, int Hq, int Hkv, int Sq, int Sk, int d, int bits) {
  return plan_decode(B, Hq, Hkv, Sq, Sk, d, bits).use;
}

template <int BITS, int D>
static void launch_decode_attn(const DecodeArgs& a, hipStream_t s) {
  dim3 grid(a.nsplit, a.Hkv, a.B);
  if constexpr (BITS <= 3) {
    if (attn_planes(BITS, a.C)) {
      constexpr int R = attn_plane_ring<D>();
      if (a.C > 4) {
        if (a.mask) decode_attn_i8_kernel<BITS - 1, R, true, 2, D><<<grid, 256, 0, s>>>(a);
        else decode_attn_i8_kernel<BITS - 1, R, false, 2, D><<<grid, 256, 0, s>>>(a);
      } else {
        if (a.mask) decode_attn_i8_kernel<BITS - 1, R, true, 1, D><<<grid, 256, 0, s>>>(a);
        else decode_attn_i8_kernel<BITS - 1, R, false, 1, D><<<grid, 256, 0, s>>>(a);
      }
      return;
    }
  }
  if (a.C <= 8) decode_attn_lds_kernel<D, BITS, kAttnNbs, kAttnRing, true><<<grid, 256, 0, s>>>(a);
  else decode_attn_lds_kernel<D, BITS, kAttnNbs, kAttnRing, false><<<grid, 256, 0, s>>>(a);
}

int decode_attention(int64_t ldk, const uint16_t* q_rot, const float* q_proj, const uint8_t* kcodes,
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
  a.ldk = ldk;
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
  if (d == 64) {
    if (bits == 2) launch_decode_attn<2, 64>(a, s);
    else if (bits == 3) launch_decode_attn<3, 64>(a, s);
    else launch_decode_attn<4, 64>(a, s);
  } else {
    if (bits == 2) launch_decode_attn<2, 128>(a, s);
    else if (bits == 3) launch_decode_attn<3, 128>(a, s);
    else launch_decode_attn<4, 128>(a, s);
  }
  int st = launch_status("tq_attention_fwd (decode)");
  if (st != TQ_OK) return st;
  // head_dim 64, few splits: the split merge of any head dim (tq_attn.hip: a wave per column,
  // partial rows of 64 floats)
  if (d == 64 && p.nsplit <= kMergeSplitsPerWave)
    return merge_key_splits(a.part_o, a.part_ml, vpit, B, Hq, Hkv, Sq, a.C, p.nsplit, d, out, out_dtype, sob, soh,
                            sos, s);
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
  if (p.nsplit > kMergeSplitsPerWave) {
    if (d == 64) decode_merge_split_kernel<64><<<dim3(a.C, Hkv, B), 256, 0, s>>>(m);
    else decode_merge_split_kernel<128><<<dim3(a.C, Hkv, B), 256, 0, s>>>(m);
  } else {
    decode_merge_kernel<128><<<dim3(Hkv, B, (a.C + 3) / 4), 256, 0, s>>>(m);
  }
  return launch_status("tq_attention_fwd (decode merge)");
}

}  // namespace tq
