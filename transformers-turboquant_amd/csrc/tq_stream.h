// Streaming helpers shared by the gfx950 attention kernels: compile-time loops,
// buffer resources over packed planes, direct-to-LDS buffer loads with explicit
// vmcnt waits, and MFMA operand builders that index small LDS lookup tables with
// SDWA byte selects.  Everything here is wave-level device code.
#pragma once
#include "tq_common.h"

#include <type_traits>

namespace tq {

// compile-time loop: f(std::integral_constant<int, I>) for I = 0 .. N-1
template <int I, int N, typename F>
__device__ __forceinline__ void static_for_impl(F& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for_impl<I + 1, N>(f);
  }
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl<0, N>(f);
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float4v mfma16x16x16(half4 a, half4 b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// Raw buffer loads: each 16-key block of a plane is read through a resource
// whose base is the block's first row and whose record count ends at the
// split's last key, so lanes past it read zero (the range check covers the
// per-lane offset only, hence the per-block base).  Lanes carry constant offsets;
// the base and count are wave-uniform scalar arithmetic.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x3 __attribute__((ext_vector_type(3)));

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}
// resource over rows [kb, kend) of a plane with `rb`-byte rows
__device__ __forceinline__ rsrc_t rows_rsrc(const void* plane, int rb, int kb, int kend) {
  return make_rsrc(static_cast<const uint8_t*>(plane) + static_cast<int64_t>(kb) * rb,
                   static_cast<uint32_t>(kend - kb) * rb);
}
constexpr uint32_t kOutOfRange = 0x80000000u;  // lane offset that every resource here rejects
// Streamed planes are read once per step: loads carry the non-temporal hint.
constexpr int kStream = 2;
template <int N>
__device__ __forceinline__ void bload(rsrc_t r, uint32_t voff, uint32_t soff, uint32_t (&out)[N]) {
  if constexpr (N == 1) {
    out[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, kStream);
  } else if constexpr (N == 2) {
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, kStream);
    out[0] = v[0]; out[1] = v[1];
  } else {
    static_assert(N == 3, "1-3 dwords");
    const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(r, voff, soff, kStream);
    out[0] = v[0]; out[1] = v[1]; out[2] = v[2];
  }
}
__device__ __forceinline__ uint32_t bload16(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, kStream);
}
// Direct-to-LDS copies (buffer_load ... lds): every lane moves 16 bytes (or one
// u16, zero-extended to a dword) from its resource offset into LDS at
// M0 + lane*16 (lane*4).  They are issued through inline asm so that the compiler
// does not serialise them against LDS reads of other ring slots; the kernel waits
// for a slot itself with wait_vm<N>() (vmcnt completes in issue order, so DMAs the
// compiler does not count only make its own waits stronger).  The kernel keeps
// no value of its own in M0.
typedef __attribute__((address_space(3))) void* lds_void_t;
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t)(const_cast<void*>(p))));
}
__device__ __forceinline__ i32x4 rows_desc(const void* plane, int rb, int kb, int kend) {
  const uint64_t base = reinterpret_cast<uint64_t>(static_cast<const uint8_t*>(plane) + static_cast<int64_t>(kb) * rb);
  return i32x4{static_cast<int>(static_cast<uint32_t>(base)), static_cast<int>(static_cast<uint32_t>(base >> 32) & 0xffffu),
               static_cast<int>(static_cast<uint32_t>(kend > kb ? kend - kb : 0) * rb), 0x00020000};
}
// descriptor and LDS address are wave-uniform; readfirstlane lets the compiler
// prove it where the call sits under a lane-dependent branch
__device__ __forceinline__ i32x4 uniform4(i32x4 r) {
  return i32x4{__builtin_amdgcn_readfirstlane(r[0]), __builtin_amdgcn_readfirstlane(r[1]),
               __builtin_amdgcn_readfirstlane(r[2]), __builtin_amdgcn_readfirstlane(r[3])};
}
// M0 is written here only; the compiler keeps nothing of its own in it in these kernels
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(i32x4 r, uint32_t lds, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
               :: "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(uniform4(r)) : "memory", "m0");
}
// the same copy without the non-temporal hint, for data that many blocks re-read (weights)
__device__ __forceinline__ void dma16_cached(i32x4 r, uint32_t lds, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(uniform4(r)) : "memory", "m0");
}
__device__ __forceinline__ void dma_u16(i32x4 r, uint32_t lds, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_ushort %1, %2, 0 offen nt lds"
               :: "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(uniform4(r)) : "memory", "m0");
}
#pragma clang diagnostic pop
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}
// vmcnt(0) as a compiler-visible s_waitcnt (vmcnt 0, expcnt and lgkmcnt unconstrained).  The
// compiler's wait-insertion pass does not read inline asm, so after wait_vm<0>() it still takes
// earlier loads as pending and waits again at their first use, which inside a loop means every
// iteration (with the loads issued in between included); after this one they count as done.
__device__ __forceinline__ void wait_vm0_visible() { __builtin_amdgcn_s_waitcnt(0x0F70); }
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t lds32(const uint8_t* t, uint32_t off) {
  return *reinterpret_cast<const uint32_t*>(t + off);
}
__device__ __forceinline__ u32x2 lds64(const uint8_t* t, uint32_t off) {
  return *reinterpret_cast<const u32x2*>(t + off);
}
// Table offsets are built with SDWA byte selects: (byte K of x) & mask in one
// instruction, on copies of the packed word pre-shifted so that each field lands
// at the entry stride (x4 or x8 bytes) inside a byte.
// (y & mask) | (x & ~mask) in one v_bfi_b32: for x = w >> k the compiler folds ~mask into
// a narrower constant first and then emits a shift, an and and an and-or
__device__ __forceinline__ uint32_t bfi32(uint32_t mask, uint32_t y, uint32_t x) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(mask), "v"(y), "v"(x));
  return r;
}
template <int K>
__device__ __forceinline__ uint32_t and_byte(uint32_t mask, uint32_t x) {
  static_assert(K >= 0 && K < 4, "byte select");
  uint32_t r;
  if constexpr (K == 0)
    asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
        : "=v"(r) : "v"(mask), "v"(x));
  else if constexpr (K == 1)
    asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
        : "=v"(r) : "v"(mask), "v"(x));
  else if constexpr (K == 2)
    asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
        : "=v"(r) : "v"(mask), "v"(x));
  else
    asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
        : "=v"(r) : "v"(mask), "v"(x));
  return r;
}
// (byte K of x) << 2 in one instruction
template <int K>
__device__ __forceinline__ uint32_t byte_x4(uint32_t x) {
  static_assert(K >= 0 && K < 4, "byte select");
  uint32_t r;
  if constexpr (K == 0)
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0" : "=v"(r) : "v"(x));
  else if constexpr (K == 1)
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1" : "=v"(r) : "v"(x));
  else if constexpr (K == 2)
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2" : "=v"(r) : "v"(x));
  else
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3" : "=v"(r) : "v"(x));
  return r;
}

// 8 halves from two half4 entries (x8 bytes) indexed by the two nibbles of byte K of w
template <int K>
__device__ __forceinline__ half8 nib2x4(const uint8_t* t, uint32_t w) {
  const uint32_t m = 0x78u;
  const u32x2 lo = lds64(t, and_byte<K>(m, w << 3)), hi = lds64(t, and_byte<K>(m, w >> 1));
  return __builtin_bit_cast(half8, u32x4{lo[0], lo[1], hi[0], hi[1]});
}
// 8 halves from four half2 entries (x4 bytes) indexed by the nibbles of bytes K, K+1 of w
template <int K>
__device__ __forceinline__ half8 nib4x2(const uint8_t* t, uint32_t w) {
  const uint32_t m = 0x3Cu;
  const uint32_t a = w << 2, b = w >> 2;
  return __builtin_bit_cast(half8, u32x4{lds32(t, and_byte<K>(m, a)), lds32(t, and_byte<K>(m, b)),
                                         lds32(t, and_byte<K + 1>(m, a)), lds32(t, and_byte<K + 1>(m, b))});
}
// 8 halves from four half2 entries indexed by the four 6-bit fields of the low 24 bits of f
__device__ __forceinline__ half8 six4x2(const uint8_t* t, uint32_t f) {
  const uint32_t m = 0xFCu;
  return __builtin_bit_cast(half8, u32x4{lds32(t, and_byte<0>(m, f << 2)), lds32(t, and_byte<0>(m, f >> 4)),
                                         lds32(t, and_byte<1>(m, f >> 2)), lds32(t, and_byte<2>(m, f))});
}
// 8 halves from four half2 entries indexed by the four bytes of w
__device__ __forceinline__ half8 byte4x2(const uint8_t* t, uint32_t w) {
  return __builtin_bit_cast(half8, u32x4{lds32(t, byte_x4<0>(w)), lds32(t, byte_x4<1>(w)),
                                         lds32(t, byte_x4<2>(w)), lds32(t, byte_x4<3>(w))});
}


}  // namespace tq
