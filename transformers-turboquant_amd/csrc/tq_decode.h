// Declarations shared by the decode-shaped kernels (tq_decode.hip: fused attention
// and merge; tq_decode_scores.hip: materialised scores).
#pragma once
#include "tq_common.h"
#include "tq_stream.h"

// Decode-shaped compressed attention: few query rows per head (G * Sq <= 16
// (query row, query head) columns per kv head) against long compressed
// caches.  The work is HBM-bound: every key and value record is streamed
// once per step, so the kernels are organised around the byte stream.
//
// Split-K: a block of 4 wave64 owns a chunk of keys of one (batch, kv head).
// Each wave streams its own slabs of the packed planes into a private LDS ring
// with direct-to-LDS buffer loads (16 B per lane, several slabs in flight, no
// block barriers) and builds MFMA operands from the packed bytes through small
// LDS lookup tables; the k-slot order of each MFMA is permuted so that a lane's
// operand bytes are one contiguous field of a packed row:
//   scores     S = Q K^T (16x16x32), keys on the N side: lane (key n, group g)
//              supplies dims g*D/4 + ks*8 + 0..7 of its key at k-step ks and
//              ends with 2 (at most 8 columns) or 4 columns of its own key
//   attention  S^T = K Q^T (16x16x32), keys on the M side, so the accumulator
//              is the P^T operand of O^T += V^T P^T (16x16x32 over key pairs)
// q_proj (f32) enters term 2 as f16 hi + lo parts; with at most 8 columns the lo
// parts ride in the MFMA rows / columns the queries leave empty, otherwise they
// take a second MFMA per k-step.
// In attention mode the (m, l, O) state of the 4 waves is merged in LDS into
// one partial per block; decode_merge_kernel combines the splits, normalises
// and applies Pi_v.  In scores mode each block writes its keys' f32 scores.

// Launch shapes (measured on MI355X at 16 x 32k keys, bits 3):
//   scores     wave slabs of score_slab_keys(bits) keys, score_ring(bits) slots in
//              flight, grids of about kScoreBlocks blocks: many short blocks balance
//              the last round better than one persistent stream per CU (57 vs 62-66 us)
//   attention  wave slabs of 16 * kAttnNbs keys in kAttnRing slots, a grid of one
//              round of resident blocks (4 per CU at 128 VGPRs: 1024 on 256 CUs,
//              8% faster than 768 blocks at 3 waves per SIMD)
// Scores: 32-key slabs in a 3-slot ring at bits 3-4 (22 KB of LDS, 6 blocks per CU),
// 64-key slabs in 2 slots at bits 2, where the shorter slabs' per-slab overhead is a
// larger share of the lighter decode: bits 3 56.3 vs 57.8 us, bits 4 68.2 vs 69.1 us,
// bits 2 48.0 vs 46.5 us for 32/3 against 64/2.

namespace tq {

constexpr int kScoreBlocks = 4096;
constexpr int kScoreBlocks2 = 512;  // the bit-plane kernel's two-column-group form
constexpr int kAttnNbs = 2;
constexpr int kAttnRing = 2;
constexpr int score_ring(int bits) { return bits == 2 ? 2 : 3; }
constexpr int score_slab_keys(int bits) { return bits == 2 ? 64 : 32; }


struct DecodeArgs {
  const uint16_t* q_rot;
  const float* q_proj;           // f32, split into f16 hi + lo operands
  const uint8_t *kcodes, *ksigns;
  const uint16_t *krn, *kvn, *kcent;
  const uint8_t* vcodes;
  const uint16_t* vvn;
  const float* vcent;            // f32 value centroids (tables hold their f16 values)
  int B, Hq, Hkv, Sq, Sk, G, C;  // C = G * Sq valid columns
  int64_t ldk;                   // rows between consecutive (batch, kv head) planes (>= Sk)
  int nsplit, chunk;             // keys per block (multiple of 64)
  float coeff, scale;
  int causal;
  const float* mask;
  int64_t smb, smh, smq, smk;
  float* scores;                 // scores mode: f32 [B, Hq, Sq, Sk]
  float *part_o, *part_ml;       // attention mode partials
};


// odd VB-bit fields of 8 consecutive fields
template <int VB>
constexpr uint32_t odd_fields() {
  return VB == 2 ? 0xCCCCu : (VB == 3 ? 0xE38E38u : 0xF0F0F0F0u);
}

// Pair-table entry I (two f16 values) of a value word whose fields are VB bits each, LSB
// first: the fields nib4x2 (VB 2), six4x2 (VB 3) and byte4x2 (VB 4) read as entry I
template <int VB, int I>
__device__ __forceinline__ uint32_t value_pair(const uint8_t* t, uint32_t w) {
  static_assert(I >= 0 && I < 4, "four pair fields per word");
  if constexpr (VB == 2) {
    constexpr uint32_t m = 0x3Cu;
    return lds32(t, and_byte<I / 2>(m, (I & 1) ? (w >> 2) : (w << 2)));
  } else if constexpr (VB == 3) {
    constexpr uint32_t m = 0xFCu;
    if constexpr (I == 0) return lds32(t, and_byte<0>(m, w << 2));
    else if constexpr (I == 1) return lds32(t, and_byte<0>(m, w >> 4));
    else if constexpr (I == 2) return lds32(t, and_byte<1>(m, w >> 2));
    else return lds32(t, and_byte<2>(m, w));
  } else {
    return lds32(t, byte_x4<I>(w));
  }
}

// ---------------------------------------------------------------- small tables
// Lookup tables of at most 32 dwords give every entry its own LDS bank, so the
// data-dependent lookups of a wave never conflict (64-entry tables share a bank
// between two entries).  Entries are indexed by nibbles / 6-bit fields of the
// packed rows:
//   sign table   16 x half4: 4 sign bits -> 4 x (+-1)
//   key table    KB=1: 16 x half4 (4 codes) | KB=2: 16 x half2 (2 codes) | KB=3: 64 x half2
//   value table  VB=2: 16 x half2 | VB=3: 64 x half2 | VB=4: 256 x half2
template <int BITS>
struct SmallLuts {
  static constexpr int KB = BITS - 1, VB = BITS;
  static constexpr int SGN_BYTES = 16 * 8;
  static constexpr int KEY_BYTES = (KB == 1) ? 16 * 8 : (KB == 2 ? 16 * 4 : 64 * 4);
  static constexpr int VAL_BYTES = (VB == 2) ? 16 * 4 : (VB == 3 ? 64 * 4 : 256 * 4);
  static constexpr int SGN_OFF = 0, KEY_OFF = SGN_BYTES, VAL_OFF = SGN_BYTES + KEY_BYTES;
  static constexpr int BYTES = VAL_OFF + VAL_BYTES;
};

template <int BITS, bool VALUES>
__device__ __forceinline__ void build_small_luts(const DecodeArgs& a, uint8_t* t, int tid) {
  using L = SmallLuts<BITS>;
  constexpr int KB = L::KB, VB = L::VB;
  if (tid < 16) {
    half4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = ((tid >> j) & 1) ? static_cast<_Float16>(1.f) : static_cast<_Float16>(-1.f);
    *reinterpret_cast<half4*>(t + L::SGN_OFF + tid * 8) = v;
  }
  auto kc = [&](int i) { return __builtin_bit_cast(_Float16, a.kcent[i]); };
  if constexpr (KB == 1) {
    if (tid < 16) {
      half4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = kc((tid >> j) & 1);
      *reinterpret_cast<half4*>(t + L::KEY_OFF + tid * 8) = v;
    }
  } else {
    constexpr int N = (KB == 2) ? 16 : 64;
    if (tid < N) {
      half2v v;
      v[0] = kc(tid & ((1 << KB) - 1));
      v[1] = kc(tid >> KB);
      *reinterpret_cast<half2v*>(t + L::KEY_OFF + tid * 4) = v;
    }
  }
  if constexpr (VALUES) {
    constexpr int N = (VB == 2) ? 16 : (VB == 3 ? 64 : 256);
    if (tid < N) {
      half2v v;
      v[0] = static_cast<_Float16>(a.vcent[tid & ((1 << VB) - 1)]);
      v[1] = static_cast<_Float16>(a.vcent[tid >> VB]);
      *reinterpret_cast<half2v*>(t + L::VAL_OFF + tid * 4) = v;
    }
  }
}

// A lane group's quarter of a packed key row (KLANE = D * KB / 32 bytes from byte
// lg * KLANE) as dwords, LSB first.  Head_dim 64 gives fields that are not dword multiples
// (2 bytes at 1 code bit, 6 at 3 bits), read as 2-byte pieces: their rows are only 2-byte
// aligned.
template <int KLANE>
__device__ __forceinline__ void load_key_field(const uint8_t* kp, uint32_t (&kw)[(KLANE + 3) / 4]) {
  if constexpr (KLANE == 2) {
    kw[0] = *reinterpret_cast<const uint16_t*>(kp);
  } else if constexpr (KLANE == 6) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(kp);
    kw[0] = static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16);
    kw[1] = h[2];
  } else if constexpr (KLANE == 8) {
    const u32x2 t = *reinterpret_cast<const u32x2*>(kp);
    kw[0] = t[0];
    kw[1] = t[1];
  } else {
    static_assert(KLANE % 4 == 0, "dword fields");
#pragma unroll
    for (int w = 0; w < KLANE / 4; ++w) kw[w] = reinterpret_cast<const uint32_t*>(kp)[w];
  }
}
// a lane group's sign bits (D / 4 of them, from byte lg * D / 32 of the sign row)
template <int D>
__device__ __forceinline__ uint32_t load_sign_field(const uint8_t* sp) {
  if constexpr (D == 64) return *reinterpret_cast<const uint16_t*>(sp);
  else return *reinterpret_cast<const uint32_t*>(sp);
}

// Key operand of k-step KS: dims KS*8 .. KS*8+7 of the lane's field (D / 4 dims)
template <int KB, int KW32, int KS>
__device__ __forceinline__ half8 key_operand(const uint8_t* t, const uint32_t (&k)[KW32]) {
  if constexpr (KB == 1) {
    return nib2x4<KS>(t, k[0]);
  } else if constexpr (KB == 2) {
    return nib4x2<2 * (KS & 1)>(t, k[KS >> 1]);
  } else {
    constexpr int bit = 24 * KS, wi = bit >> 5, sh = bit & 31;
    const uint32_t lo32 = k[wi];
    const uint32_t hi32 = (wi + 1 < KW32) ? k[wi + 1] : 0u;
    return six4x2(t, sh ? __builtin_amdgcn_alignbit(hi32, lo32, sh) : lo32);
  }
}

// ---------------------------------------------------------------- bit-plane scores
// Scores on the integer MFMA for 1- and 2-bit key codes and at most 8 columns.
// Both terms are sums of query values over the set bits of key bit-planes:
//   term 1: f16(C)[code] = c0 + (c1 - c0) b0 [+ (c2 - c0) b1 + (c3 - c2 - c1 + c0) b0 b1]
//           (b0, b1: low / high code bit), so q_rot . f16(C)[codes] =
//           c0 sum(q_rot) + sum over planes of (coefficient q_rot) . plane
//   term 2: q_proj . (2 s - 1) = (2 q_proj) . s - sum(q_proj)
// (attention.py:419-461).  A plane operand needs no lookup: byte j of
// w & (0x01010101 << i) is bit 8j + i of the packed word w, weighted 2^i (i = 7: -128
// as int8), and feeds v_mfma_i32_16x16x64_i8 as is.  The query side carries, for the
// K slot of bit i, W 2^(7 - i) (i = 7: -W), W = rint(v 2^F) with F per (query, term)
// such that |W| <= 2^23; the int32 A values are split into four signed base-256
// digits, and the 16 MFMA rows of a row group are 4 queries x 4 digits, so lane (key n,
// group g) ends with the 4 digit sums of query g and of its own key:
//   dot = 2^(-7 - F) (acc0 + 2^8 acc1 + 2^16 acc2 + 2^24 acc3)
// exact up to the rounding of v to 24 significant bits of the largest |v|, i.e. f32
// grade for q_proj as well.  The interaction plane b0 b1 is only used when the
// codebook is not affine in its bits (every Lloyd-Max codebook is odd, hence affine).
typedef int i32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i32x4v mfma_i8(i32x4v a, i32x4v b, i32x4v c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
// plane dwords i0 .. i0 + 3 of word w: byte j of element e is bit 8j + i0 + e
template <int I0>
__device__ __forceinline__ i32x4v planes4(uint32_t w) {
  constexpr uint32_t m = 0x01010101u;
  return i32x4v{static_cast<int>(w & (m << I0)), static_cast<int>(w & (m << (I0 + 1))),
                static_cast<int>(w & (m << (I0 + 2))), static_cast<int>(w & (m << (I0 + 3)))};
}
// even bit positions 0, 2, 4, 6 of each byte
__device__ __forceinline__ i32x4v planes_even(uint32_t w) {
  constexpr uint32_t m = 0x01010101u;
  return i32x4v{static_cast<int>(w & m), static_cast<int>(w & (m << 2)), static_cast<int>(w & (m << 4)),
                static_cast<int>(w & (m << 6))};
}
// digit sums -> f32: (acc3 2^8 + acc2) 2^16 + (acc1 2^8 + acc0), both halves exact in int32
__device__ __forceinline__ float digits_f32(i32x4v acc) {
  const int hi = (acc[3] << 8) + acc[2], lo = (acc[1] << 8) + acc[0];
  return fmaf(static_cast<float>(hi), 65536.f, static_cast<float>(lo));
}

// The query side of a block: column c of the block's kv head is MFMA row group c & 3 (rows
// 4 (c & 3) + t, t = digit) of column group c >> 2, so a lane of group lg holds the digits of
// columns lg, lg + 4, ... (one set of A fragments per column group) and, after the MFMAs over
// a 16-key block on the N side, the digit sums of those columns against its own key (lane
// l16).  The key-side plane operands are built once per key and serve every column group.
// STAGE_BYTES of LDS serve as staging during setup().
template <int KB, int NCG = 1, int D_ = 128>
struct PlaneQuery {
  static_assert(KB == 1 || KB == 2, "1- or 2-bit key codes");
  static_assert(NCG == 1 || NCG == 2, "4 or 8 columns");
  static_assert(D_ == 64 || D_ == 128, "head_dim 64 or 128");
  static constexpr int D = D_;
  static constexpr int LW = D / 4;                 // dims per lane group (a quarter of a key row)
  static constexpr int KWD = (LW * KB + 31) / 32;  // code dwords per lane (head_dim 64, 1 bit: half a dword)
  static constexpr int NC = 4 * NCG;               // columns served
  static constexpr int NT1 = 2 * KWD;              // code-plane fragments (MFMAs per 16 keys)
  static constexpr int NFM = NT1 + 2;              // then the two sign-plane fragments
  static constexpr int NDL = KB == 2 ? KWD : 0;    // interaction-plane fragments
  static constexpr int NF = NFM + NDL;
  static constexpr int STAGE_BYTES =
      (NC * 2 * D * 4 > NCG * NFM * 1024) ? NC * 2 * D * 4 : NCG * NFM * 1024;
  // with two column groups the interaction-plane fragments (used only by codebooks that are
  // not affine in their bits) stay in LDS instead of registers
  static constexpr bool INTER_LDS = NCG > 1 && NDL > 0;
  i32x4v A[NCG][INTER_LDS ? NFM : NF];
  const i32x4v* aint;      // INTER_LDS: this lane's interaction fragments, [g * NDL + w] * 64
  int x1[NCG], x2[NCG];    // column lg + 4g: dot = 2^x digits_f32(acc)
  float k1[NCG], k2[NCG];  // column lg + 4g: c0 sum(q_rot), sum(q_proj)
  bool inter;              // the codebook needs the interaction plane (block-uniform)

  // Every thread of the block calls this (it holds barriers); the staging area may be
  // reused once the caller has passed another barrier.
  __device__ __forceinline__ void setup(const DecodeArgs& a, int b, int hkv, uint8_t* stg, int tid) {
    __shared__ float st_k1[NC], st_k2[NC];
    __shared__ int st_f1[NC], st_f2[NC];
    __shared__ i32x4v s_int[INTER_LDS ? NCG * NDL * 64 : 1];
    const int lane = tid & 63, wave = tid >> 6, lg = lane >> 4;
    // codebook in plane form: c(b0, b1) = c0 + alo b0 + ahi b1 + adl b0 b1
    const float c0 = h2f(a.kcent[0]), alo = h2f(a.kcent[1]) - c0;
    const float ahi = KB == 2 ? h2f(a.kcent[2]) - c0 : 0.f;
    const float adl = KB == 2 ? (h2f(a.kcent[3]) - h2f(a.kcent[2])) - alo : 0.f;
    inter = adl != 0.f;

    // phase 1: wave w stages columns w, w + 4, ... (f32) and finds their scales
    float* const qst = reinterpret_cast<float*>(stg);  // [NC][2][D]: q_rot, q_proj
    const float cmax = fmaxf(fabsf(alo), fmaxf(fabsf(ahi), fabsf(adl)));
#pragma unroll
    for (int g = 0; g < NCG; ++g) {
      const int c = wave + 4 * g;
      float r0 = 0.f, r1 = 0.f, p0 = 0.f, p1 = 0.f;
      const bool dim_ok = 2 * lane < D;  // head_dim 64: lanes 0-31 hold the row
      if (c < a.C && dim_ok) {
        const int qi = c / a.G, h = hkv * a.G + c % a.G;
        const int64_t qrow = ((static_cast<int64_t>(b) * a.Hq + h) * a.Sq + qi) * D + 2 * lane;
        const uint32_t rr = *reinterpret_cast<const uint32_t*>(a.q_rot + qrow);
        r0 = h2f(static_cast<uint16_t>(rr));
        r1 = h2f(static_cast<uint16_t>(rr >> 16));
        const float2 pp = *reinterpret_cast<const float2*>(a.q_proj + qrow);
        p0 = pp.x;
        p1 = pp.y;
      }
      if (dim_ok) {
        *reinterpret_cast<float2*>(qst + (c * 2) * D + 2 * lane) = float2{r0, r1};
        *reinterpret_cast<float2*>(qst + (c * 2 + 1) * D + 2 * lane) = float2{p0, p1};
      }
      float mr = fmaxf(fabsf(r0), fabsf(r1)), mp = fmaxf(fabsf(p0), fabsf(p1));
      float sr = r0 + r1, sp = p0 + p1;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        mr = fmaxf(mr, __shfl_xor(mr, o));
        mp = fmaxf(mp, __shfl_xor(mp, o));
        sr += __shfl_xor(sr, o);
        sp += __shfl_xor(sp, o);
      }
      if (lane == 0) {
        int e1 = 0, e2 = 0;
        frexpf(mr * cmax, &e1);
        frexpf(2.f * mp, &e2);
        st_f1[c] = mr * cmax > 0.f ? 23 - e1 : 0;
        st_f2[c] = mp > 0.f ? 23 - e2 : 0;
        st_k1[c] = c0 * sr;
        st_k2[c] = sp;
      }
    }
    __syncthreads();

    // phase 2: each thread builds dword groups (column group g, fragment f, column 4 g + cq,
    // lane group lg', element e): 4 A values (bytes j = 0..3) -> one dword per digit row
    // 4 cq + t
    constexpr int PER = (NCG * NF * 64 + 255) / 256;
    uint32_t outw[PER][4];
    int oaddr[PER], ofrag[PER];
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int gi = tid + 256 * r;
      const int e = gi & 3, lgp = (gi >> 2) & 3, cq = (gi >> 4) & 3, gf = gi >> 6;
      const int g = gf / NF, f = gf % NF;
      ofrag[r] = g < NCG ? f : NF;
      int i = 0, m0 = 0, mstep = 8, term = 1;  // slot bit i; lane-group dims m0 + j * mstep
      float coef = 0.f;
      if (f < NT1) {
        const int w = f >> 1;
        i = 4 * (f & 1) + e;
        const int p0 = 32 * w + i;  // + 8j
        m0 = KB == 1 ? p0 : (p0 >> 1);
        mstep = KB == 1 ? 8 : 4;
        coef = (KB == 2 && (i & 1)) ? ahi : alo;
      } else if (f < NFM) {
        i = 4 * (f - NT1) + e;
        m0 = i;
        coef = 2.f;
        term = 2;
      } else {
        const int w = f - NFM;
        i = 2 * e;
        m0 = 16 * w + e;
        mstep = 4;
        coef = adl;
      }
      const int c = 4 * (g < NCG ? g : 0) + cq;
      const int F = term == 1 ? st_f1[c] : st_f2[c];
      const float* qv = qst + (c * 2 + (term - 1)) * D + LW * lgp;
      uint32_t u[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // slots past the lane group's dims (head_dim 64: the upper half of a 1-bit code or
        // sign dword) carry zero, so the bits read there add nothing
        const int m = m0 + j * mstep;
        const int wv = (g < NCG && m < LW) ? __float2int_rn(ldexpf(coef * qv[m], F)) : 0;
        const int av = i < 7 ? wv * (1 << (7 - i)) : -wv;
        u[j] = (static_cast<uint32_t>(av) + 0x808080u) ^ 0x808080u;
      }
#pragma unroll
      for (int t = 0; t < 4; ++t)
        outw[r][t] = ((u[0] >> (8 * t)) & 0xFFu) | (((u[1] >> (8 * t)) & 0xFFu) << 8) |
                     (((u[2] >> (8 * t)) & 0xFFu) << 16) | (((u[3] >> (8 * t)) & 0xFFu) << 24);
      const int slot = f < NFM ? g * NFM + f : g * NDL + (f - NFM);
      oaddr[r] = ((slot * 64 + 4 * cq + 16 * lgp) * 4 + e) * 4;
    }
    // the staged queries are read; fragments overwrite them (row 4 cq + t = lane + t)
    auto put = [&](bool second, uint8_t* dst) {
#pragma unroll
      for (int r = 0; r < PER; ++r) {
        if (ofrag[r] < NF && (ofrag[r] >= NFM) == second) {
#pragma unroll
          for (int t = 0; t < 4; ++t) *reinterpret_cast<uint32_t*>(dst + oaddr[r] + t * 16) = outw[r][t];
        }
      }
    };
    __syncthreads();
    put(false, stg);
    if constexpr (INTER_LDS) {
      if (inter) put(true, reinterpret_cast<uint8_t*>(s_int));
    }
    aint = s_int + lane;
    __syncthreads();

    // phase 3: the lane's fragments and its columns' constants
#pragma unroll
    for (int g = 0; g < NCG; ++g)
#pragma unroll
      for (int f = 0; f < NFM; ++f) A[g][f] = *reinterpret_cast<const i32x4v*>(stg + ((g * NFM + f) * 64 + lane) * 16);
    if constexpr (NDL > 0 && !INTER_LDS) {
      if (inter) {
        __syncthreads();
        put(true, stg);
        __syncthreads();
#pragma unroll
        for (int g = 0; g < NCG; ++g)
#pragma unroll
          for (int f = NFM; f < NF; ++f)
            A[g][f] = *reinterpret_cast<const i32x4v*>(stg + ((g * NDL + f - NFM) * 64 + lane) * 16);
      } else {
#pragma unroll
        for (int g = 0; g < NCG; ++g)
#pragma unroll
          for (int f = NFM; f < NF; ++f) A[g][f] = i32x4v{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int g = 0; g < NCG; ++g) {
      x1[g] = -7 - st_f1[lg + 4 * g];
      x2[g] = -7 - st_f2[lg + 4 * g];
      k1[g] = st_k1[lg + 4 * g];
      k2[g] = st_k2[lg + 4 * g];
    }
  }

  // term 1 (q_rot . f16(C)[codes]) and term 2 (q_proj . (2 s - 1)) of columns lg + 4g against
  // two keys, whose code fields (KB dwords each) and sign fields (one dword each) this lane
  // reads from LDS.  Both keys' fields are read before any MFMA, and the (block-uniform, rare)
  // interaction-plane branch is taken once for both, so that it does not split the keys'
  // work into separate basic blocks; each plane operand feeds the MFMAs of every column group.
  __device__ __forceinline__ void dots2(const uint8_t* kp0, const uint8_t* sp0, const uint8_t* kp1,
                                        const uint8_t* sp1, float (&t1)[2][NCG], float (&t2)[2][NCG]) const {
    uint32_t kw[2][KWD], sw[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint8_t* kp = j ? kp1 : kp0;
      if constexpr (KWD == 2) {
        const u32x2 t = *reinterpret_cast<const u32x2*>(kp);
        kw[j][0] = t[0];
        kw[j][1] = t[1];
      } else if constexpr (LW * KB == 16) {
        kw[j][0] = *reinterpret_cast<const uint16_t*>(kp);  // a 2-byte field
      } else {
        kw[j][0] = *reinterpret_cast<const uint32_t*>(kp);
      }
      const uint8_t* sp = j ? sp1 : sp0;
      if constexpr (LW == 16) sw[j] = *reinterpret_cast<const uint16_t*>(sp);
      else sw[j] = *reinterpret_cast<const uint32_t*>(sp);
    }
    if constexpr (NCG == 1) {
      i32x4v s1[2], s2[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        s1[j] = i32x4v{0, 0, 0, 0};
        s2[j] = i32x4v{0, 0, 0, 0};
        static_for<NT1>([&](auto ff) {
          constexpr int f = decltype(ff)::value;
          s1[j] = mfma_i8(A[0][f], planes4<4 * (f & 1)>(kw[j][f >> 1]), s1[j]);
        });
        static_for<2>([&](auto ff) {
          constexpr int f = decltype(ff)::value;
          s2[j] = mfma_i8(A[0][NT1 + f], planes4<4 * f>(sw[j]), s2[j]);
        });
      }
      if constexpr (NDL > 0) {
        if (inter) {
#pragma unroll
          for (int j = 0; j < 2; ++j)
            static_for<NDL>([&](auto ff) {
              constexpr int w = decltype(ff)::value;
              s1[j] = mfma_i8(A[0][NFM + w], planes_even(kw[j][w] & (kw[j][w] >> 1)), s1[j]);
            });
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        t1[j][0] = ldexpf(digits_f32(s1[j]), x1[0]) + k1[0];
        t2[j][0] = ldexpf(digits_f32(s2[j]), x2[0]) - k2[0];
      }
    } else {
      // one key at a time (its accumulators die at its conversion); each plane operand feeds
      // the MFMAs of both column groups
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        i32x4v s1[NCG], s2[NCG];
#pragma unroll
        for (int g = 0; g < NCG; ++g) {
          s1[g] = i32x4v{0, 0, 0, 0};
          s2[g] = i32x4v{0, 0, 0, 0};
        }
        static_for<NT1>([&](auto ff) {
          constexpr int f = decltype(ff)::value;
          const i32x4v op = planes4<4 * (f & 1)>(kw[j][f >> 1]);
#pragma unroll
          for (int g = 0; g < NCG; ++g) s1[g] = mfma_i8(A[g][f], op, s1[g]);
        });
        static_for<2>([&](auto ff) {
          constexpr int f = decltype(ff)::value;
          const i32x4v op = planes4<4 * f>(sw[j]);
#pragma unroll
          for (int g = 0; g < NCG; ++g) s2[g] = mfma_i8(A[g][NT1 + f], op, s2[g]);
        });
        if constexpr (NDL > 0) {
          if (inter) {
            static_for<NDL>([&](auto ff) {
              constexpr int w = decltype(ff)::value;
              const i32x4v op = planes_even(kw[j][w] & (kw[j][w] >> 1));
#pragma unroll
              for (int g = 0; g < NCG; ++g) s1[g] = mfma_i8(aint[(g * NDL + w) * 64], op, s1[g]);
            });
          }
        }
#pragma unroll
        for (int g = 0; g < NCG; ++g) {
          t1[j][g] = ldexpf(digits_f32(s1[g]), x1[g]) + k1[g];
          t2[j][g] = ldexpf(digits_f32(s2[g]), x2[g]) - k2[g];
        }
      }
    }
  }
};

// materialised scores for bits 2-3 and at most 8 columns, head_dim d = 64 or 128
// (tq_decode.hip), on a plan of tq_decode_scores.hip
void launch_scores_planes(const DecodeArgs& a, int bits, int d, hipStream_t s);

// Log-sum-exp merge of per-split partial rows (unnormalised o in the rotated value domain,
// d floats for d = 64, then [maximum (log2), sum] per row at part_ml) and the Pi_v product,
// for any supported head dim (tq_attn.hip)
int merge_key_splits(const float* part_o, const float* part_ml, const uint16_t* vpit, int B, int Hq, int Hkv,
                     int Sq, int C, int nsplit, int d, void* out, int out_dtype, int64_t sob, int64_t soh,
                     int64_t sos, hipStream_t s);

// ---------------------------------------------------------------- planning
struct DecodePlan {
  bool use;
  int nsplit, chunk;
  int64_t ws_bytes;
};


// Split S_k so that about `target` blocks cover the (batch, kv head) groups, each
// split a multiple of `quantum` keys and no shorter than `min_chunk`.
inline DecodePlan plan_split(int B, int Hkv, int Sk, int target, int quantum, int min_chunk) {
  DecodePlan p{true, 0, 0, 0};
  const int64_t groups = static_cast<int64_t>(B) * Hkv;
  int nsplit = static_cast<int>((target + groups - 1) / groups);
  const int max_split = (Sk + min_chunk - 1) / min_chunk;
  if (nsplit > max_split) nsplit = max_split;
  if (nsplit > 1024) nsplit = 1024;
  if (nsplit < 1) nsplit = 1;
  int chunk = (Sk + nsplit - 1) / nsplit;
  chunk = (chunk + quantum - 1) / quantum * quantum;
  p.nsplit = (Sk + chunk - 1) / chunk;
  p.chunk = chunk;
  return p;
}

// head_dim 64 or 128, bits 2-4, at most 16 query columns per kv head; S_k below 2^24
// keeps every per-group byte offset of the planes and score rows under 2^31
inline bool decode_shape(int Hq, int Hkv, int Sq, int Sk, int d, int bits) {
  if ((d != 64 && d != 128) || bits < 2 || bits > 4 || Hkv <= 0 || Hq % Hkv) return false;
  return (Hq / Hkv) * Sq <= 16 && Sk >= 1 && Sk < (1 << 24);
}

}  // namespace tq
