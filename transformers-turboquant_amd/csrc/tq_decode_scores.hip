// Decode-shaped materialised scores (split-K over keys) through lookup tables, head_dim 64
// and 128, for bits 4 and 9-16 columns (the bit-plane kernel for bits 2-3 and at most 8 columns is in
// tq_decode.hip); the shared argument block, lookup tables and split planning are in
// tq_decode.h.  Built without -amdgpu-mfma-vgpr-form: with MFMA accumulators in VGPRs the
// compiler gave wrong scores from the second ring slot on when part of an accumulator is
// dead (the two-columns-per-lane layout below), measured on MI355X.
#include "tq_decode.h"

namespace tq {

// Scores: each wave DMAs NK-key slabs of the code, sign and norm planes into its
// own R-slot LDS ring (16 B per lane; nothing is held in registers while in
// flight) and scores them with the keys on the MFMA's N side, so lane (key l16,
// group lg) ends with columns 4*lg + e of its own key: the two norms are
// per-lane scalars and each column's 16 scores leave as one 64-byte run.
template <int D, int BITS, int R, int NK, bool PACK>
__global__ void __launch_bounds__(256) decode_scores_kernel(DecodeArgs a) {
  static_assert(D == 64 || D == 128, "decode kernel is built for head_dim 64 or 128");
  static_assert(R >= 2 && R <= 4, "ring of 2 to 4 slots");
  static_assert(NK == 32 || NK == 64, "slabs of 32 or 64 keys");
  using L = SmallLuts<BITS>;
  constexpr int KB = L::KB;
  constexpr int KS = D / 32;
  constexpr int KC = D * KB / 8, SC = D / 8;
  constexpr int KLANE = KC / 4;
  constexpr int KW32 = (KLANE + 3) / 4;
  constexpr int SLANE = SC / 4;
  constexpr int NBS = NK / 16;
  constexpr int SLAB = 4 * NK;           // keys per block slab
  constexpr int OFF_K = 0, OFF_S = NK * KC, OFF_N = OFF_S + NK * SC;
  constexpr int NRM = NK * 4;            // one norm plane: a dword per key
  constexpr int SLOT = OFF_N + 2 * NRM;

  __shared__ __attribute__((aligned(16))) uint8_t luts[L::BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t stage[4 * R * SLOT];
  const uint8_t* tS = luts + L::SGN_OFF;
  const uint8_t* tK = luts + L::KEY_OFF;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int split = blockIdx.x, hkv = blockIdx.y, b = blockIdx.z;
  const int64_t bh = static_cast<int64_t>(b) * a.Hkv + hkv;

  build_small_luts<BITS, false>(a, luts, tid);

  // A operand row l16, dims lg*D/4 + ks*8 + 0..7.  q_proj enters term 2 as f16 hi + lo.
  // PACK (C <= 8): row 4g + e carries column 2g + (e & 1): q_rot and hi(q_proj) for e < 2,
  // zero and lo(q_proj) for e >= 2, so lane (key, g) ends with both parts of columns 2g and
  // 2g + 1 and adds them.  Otherwise row l16 is column l16 and the lo parts take a second
  // MFMA per k-step.
  constexpr int NOUT = PACK ? 2 : 4;  // columns per lane
  half8 qr[KS], qp[KS];
  [[maybe_unused]] half8 ql[PACK ? 1 : KS];
  {
    const int c = PACK ? 2 * (l16 >> 2) + (l16 & 1) : l16;
    const bool lo_row = PACK && (l16 & 2);
    const bool ok = c < a.C;
    const int qi = ok ? c / a.G : 0, h = hkv * a.G + (ok ? c % a.G : 0);
    const int64_t qrow = ((static_cast<int64_t>(b) * a.Hq + h) * a.Sq + qi) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d0 = lg * (D / 4) + ks * 8;
      half8 hi = half8{}, lo = half8{};
      if (ok) split8(a.q_proj + qrow + d0, hi, lo);
      qr[ks] = (ok && !lo_row) ? *reinterpret_cast<const half8*>(a.q_rot + qrow + d0) : half8{};
      if constexpr (PACK) {
        qp[ks] = lo_row ? lo : hi;
      } else {
        qp[ks] = hi;
        ql[ks] = lo;
      }
    }
  }

  const int kbeg = split * a.chunk;
  const int kend = min(a.Sk, kbeg + a.chunk);
  const float fb = a.coeff;

  // output: the C score rows of this (b, kv head) are contiguous [C][Sk] f32
  // (head h = hkv*G + c%G, query row c/G); invalid columns aim past the end and
  // are dropped by the store's range check
  const float* pout = a.scores + (static_cast<int64_t>(b) * a.Hq + hkv * a.G) * a.Sq * a.Sk;
  const uint32_t out_bytes = static_cast<uint32_t>(a.C) * a.Sk * 4;
  uint32_t oo[NOUT];
#pragma unroll
  for (int e = 0; e < NOUT; ++e) {
    const int c = NOUT * lg + e;
    oo[e] = c < a.C ? static_cast<uint32_t>((c % a.G) * a.Sq + c / a.G) * a.Sk * 4 + 4 * l16 : kOutOfRange;
  }

  const int64_t g0 = bh * a.ldk;
  const uint8_t* pk = a.kcodes + g0 * KC;
  const uint8_t* ps = a.ksigns + g0 * SC;
  const uint16_t* pkn = a.kvn + g0;
  const uint16_t* prn = a.krn + g0;

  uint8_t* mine = stage + wave * (R * SLOT);
  const uint32_t mine_lds = lds_offset(mine);
  constexpr int NKD = (NK * KC + 1023) / 1024, NSD = (NK * SC + 1023) / 1024;
  constexpr int NDMA = NKD + NSD + 2;  // DMA instructions per slot
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
    if (NK == 64 || lane < 32) {
      dma_u16(rows_desc(pkn, 2, kb, kend), dst + OFF_N, lane * 2);
      dma_u16(rows_desc(prn, 2, kb, kend), dst + OFF_N + NRM, lane * 2);
    }
  };
  // wait until the slot issued `later` slots ago has landed (score stores issued
  // in between only make the wait stronger: loads complete in issue order)
  auto wait_slot = [&](int later) {
    if (later >= 3) wait_vm<(R >= 4 ? 3 * NDMA : 0)>();
    else if (later == 2) wait_vm<(R >= 3 ? 2 * NDMA : 0)>();
    else if (later == 1) wait_vm<NDMA>();
    else wait_vm<0>();
  };

  auto slab = [&](const uint8_t* src, int ks0) {
#pragma unroll
    for (int j = 0; j < NBS; ++j) {
      uint32_t kw[KW32];
      load_key_field<KLANE>(src + OFF_K + (16 * j + l16) * KC + lg * KLANE, kw);
      const uint32_t sw = load_sign_field<D>(src + OFF_S + (16 * j + l16) * SC + lg * SLANE);
      float4v s1 = float4v{0.f, 0.f, 0.f, 0.f}, s2 = float4v{0.f, 0.f, 0.f, 0.f};
      static_for<KS>([&](auto c) {
        constexpr int ks = decltype(c)::value;
        s1 = mfma16x16x32(qr[ks], key_operand<KB, KW32, ks>(tK, kw), s1);
        const half8 sg = nib2x4<ks>(tS, sw);
        s2 = mfma16x16x32(qp[ks], sg, s2);
        if constexpr (!PACK) s2 = mfma16x16x32(ql[ks], sg, s2);
      });
      const float kn = h2f(static_cast<uint16_t>(*reinterpret_cast<const uint32_t*>(src + OFF_N + (16 * j + l16) * 4)));
      const float rn =
          fb * h2f(static_cast<uint16_t>(*reinterpret_cast<const uint32_t*>(src + OFF_N + NRM + (16 * j + l16) * 4)));
      const int kb = ks0 + 16 * j;
      if (kb + l16 < kend) {
        const rsrc_t ro = make_rsrc(pout + kb, out_bytes - static_cast<uint32_t>(kb) * 4);
#pragma unroll
        for (int e = 0; e < NOUT; ++e) {
          const float t2 = PACK ? s2[e] + s2[e + 2] : s2[e];
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, s1[e] * kn + t2 * rn), ro, oo[e], 0, 2);
        }
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
}

template <int D>
static void launch_scores_tables(const DecodeArgs& a, int bits, hipStream_t s) {
  const dim3 grid(a.nsplit, a.Hkv, a.B);
  if (a.C <= 8) {
    if (bits == 2) decode_scores_kernel<D, 2, score_ring(2), score_slab_keys(2), true><<<grid, 256, 0, s>>>(a);
    else if (bits == 3) decode_scores_kernel<D, 3, score_ring(3), score_slab_keys(3), true><<<grid, 256, 0, s>>>(a);
    else decode_scores_kernel<D, 4, score_ring(4), score_slab_keys(4), true><<<grid, 256, 0, s>>>(a);
  } else {
    if (bits == 2) decode_scores_kernel<D, 2, score_ring(2), score_slab_keys(2), false><<<grid, 256, 0, s>>>(a);
    else if (bits == 3) decode_scores_kernel<D, 3, score_ring(3), score_slab_keys(3), false><<<grid, 256, 0, s>>>(a);
    else decode_scores_kernel<D, 4, score_ring(4), score_slab_keys(4), false><<<grid, 256, 0, s>>>(a);
  }
}

static DecodePlan plan_scores(int B, int Hq, int Hkv, int Sq, int Sk, int d, int bits) {
  if (!decode_shape(Hq, Hkv, Sq, Sk, d, bits)) return DecodePlan{false, 0, 0, 0};
  const int slab = 4 * score_slab_keys(bits);
  // the two-column-group bit-plane kernel (5-8 columns) costs more per block to set up:
  // fewer, longer splits (measured: 512 blocks against 4096, B16 x 32k keys, 16/2 heads,
  // bits 3: 22.0 vs 39.4 us)
  const int C = (Hq / Hkv) * Sq;
  return plan_split(B, Hkv, Sk, (bits <= 3 && C > 4) ? kScoreBlocks2 : kScoreBlocks, slab, 2 * slab);
}


int decode_scores(int64_t ldk, const uint16_t* q_rot, const float* q_proj, const uint8_t* kcodes,
                  const uint8_t* ksigns, const uint16_t* krn, const uint16_t* kvn, const uint16_t* kcent,
                  int B, int Hq, int Hkv, int Sq, int Sk, int d, int bits, float coeff, float* out,
                  hipStream_t s) {
  const DecodePlan p = plan_scores(B, Hq, Hkv, Sq, Sk, d, bits);
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
  a.ldk = ldk;
  a.G = Hq / Hkv;
  a.C = a.G * Sq;
  a.nsplit = p.nsplit;
  a.chunk = p.chunk;
  a.coeff = coeff;
  a.scale = 1.f;
  a.scores = out;
  if (bits <= 3 && a.C <= 8) {
    launch_scores_planes(a, bits, d, s);  // tq_decode.hip
    return launch_status("tq_attention_scores (decode, bit planes)");
  }
  if (d == 64) launch_scores_tables<64>(a, bits, s);
  else launch_scores_tables<128>(a, bits, s);
  return launch_status("tq_attention_scores (decode)");
}

}  // namespace tq
