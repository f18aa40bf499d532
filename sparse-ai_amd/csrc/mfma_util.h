// Shared pieces of the MFMA kernels (gfx950): operand types, the 32x32x16
// MFMA wrappers, explicit vector-memory waits, a fence-free barrier and the
// direct-to-LDS loads with their pipeline waits.
#pragma once

#include "sa_internal.h"

namespace sa {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <typename T> struct Mma;
template <> struct Mma<bf16_t> {
  typedef bf16x8_t vec;
  static __device__ __forceinline__ f32x16_t mma(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(vec, a),
                                                   __builtin_bit_cast(vec, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_bf16x2(lo, hi); }
};
template <> struct Mma<f16_t> {
  typedef f16x8_t vec;
  static __device__ __forceinline__ f32x16_t mma(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(vec, a),
                                                  __builtin_bit_cast(vec, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_f16x2(lo, hi); }
};

// 16x16 tiles: k32 = v_mfma_f32_16x16x32 (lane l holds 8 consecutive k of
// row / column l % 16, k-group l / 16), k16 = v_mfma_f32_16x16x16 (4
// consecutive k per lane). The 16x16 result: lane l holds rows 4 (l / 16) + i,
// i < 4, of column l % 16.
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef short s16x4v_t __attribute__((ext_vector_type(4)));
template <typename T> struct Mma16;
template <> struct Mma16<bf16_t> {
  static __device__ __forceinline__ f32x4_t k32(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4_t k16(u32x2_t a, u32x2_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4v_t, a),
                                                     __builtin_bit_cast(s16x4v_t, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_bf16x2(lo, hi); }
};
template <> struct Mma16<f16_t> {
  static __device__ __forceinline__ f32x4_t k32(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  }
  static __device__ __forceinline__ f32x4_t k16(u32x2_t a, u32x2_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a), __builtin_bit_cast(f16x4_t, b), c,
                                                 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_f16x2(lo, hi); }
};

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14, expcnt / lgkmcnt left at
// their "no wait" maxima).
template <int VM>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(VM >= 0 && VM < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (15 << 8));
}
// Workgroup barrier without the release/acquire fences of __syncthreads():
// the fence would wait for every in-flight direct-to-LDS load of the
// pipeline. The kernel orders its own LDS traffic with explicit waits.
__device__ __forceinline__ void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

typedef short s16x4_t __attribute__((ext_vector_type(4)));
#define SA_LDS __attribute__((address_space(3)))

// Direct-to-LDS loads of 16 bytes per lane: lane L's bytes land at LDS
// address lds_addr + 16 L. Issued through inline asm so that the compiler
// does not track them: its own wait insertion would otherwise drain every
// in-flight load before any LDS read. The kernel waits for these loads with
// explicit vmcnt counts before the barrier that publishes a stage.
//   dma16:   64-bit per-lane address.
//   dma16_s: uniform 64-bit base in SGPRs + 32-bit per-lane byte offset.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
               :: "s"(lds_addr), "v"(src) : "memory", "m0");
}
// A pointer that is the same in every lane, moved to scalar registers.
__device__ __forceinline__ const char* uniform_ptr(const char* x) {
  const uint64_t v = reinterpret_cast<uint64_t>(x);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const char*>((static_cast<uint64_t>(hi) << 32) | lo);
}
__device__ __forceinline__ void dma16_s(const void* base, uint32_t off, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
               :: "s"(lds_addr), "v"(off), "s"(uniform_ptr(static_cast<const char*>(base))) : "memory", "m0");
}

// Wait until at most `ahead` pipeline tiles (LPW loads each) are in flight:
// `ahead` is the number of tiles issued after the one about to be computed.
template <int LPW, int MAXA>
__device__ __forceinline__ void wait_tiles(int ahead) {
  static_assert(MAXA >= 1 && MAXA <= 3, "pipeline depth");
  if constexpr (MAXA >= 3) {
    if (ahead >= 3) {
      wait_vmcnt<3 * LPW>();
      return;
    }
  }
  if constexpr (MAXA >= 2) {
    if (ahead >= 2) {
      wait_vmcnt<2 * LPW>();
      return;
    }
  }
  if (ahead >= 1) wait_vmcnt<LPW>();
  else wait_vmcnt<0>();
}

// Direct-to-LDS load of 4 bytes per lane (lane L's dword lands at lds_addr + 4 L).
__device__ __forceinline__ void dma4(const void* src, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off"
               :: "s"(lds_addr), "v"(src) : "memory", "m0");
}

}  // namespace sa
