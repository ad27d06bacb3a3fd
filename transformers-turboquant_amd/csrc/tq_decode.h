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

// Key operand of k-step KS: dims KS*8 .. KS*8+7 of the lane's 32-dim field
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

// head_dim 128, bits 2-4, at most 16 query columns per kv head; S_k below 2^24
// keeps every per-group byte offset of the planes and score rows under 2^31
inline bool decode_shape(int Hq, int Hkv, int Sq, int Sk, int d, int bits) {
  if (d != 128 || bits < 2 || bits > 4 || Hkv <= 0 || Hq % Hkv) return false;
  return (Hq / Hkv) * Sq <= 16 && Sk >= 1 && Sk < (1 << 24);
}

}  // namespace tq
