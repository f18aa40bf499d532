// Internal helpers shared by the HIP translation units of libsparseattn.so.
// gfx950 only: wave64, 32x32 MFMA tiles, DPP row operations.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <string>

#include "../../include/sparse_attn.h"

namespace sa {

// ---- host-side error plumbing -------------------------------------------------
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool is_pow2(long long x) { return x > 0 && (x & (x - 1)) == 0; }

// ---- element conversion --------------------------------------------------------
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__device__ __forceinline__ float bf16_bits_to_float(uint32_t b) {
  return __uint_as_float(b << 16);
}
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Round-to-nearest-even conversions on gfx950's packed converters
// (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), f16x2_t));
}
__device__ __forceinline__ uint32_t float_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ float f16_bits_to_float(uint32_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
}
__device__ __forceinline__ uint32_t float_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <typename T> struct Elem;
template <> struct Elem<float> {
  __device__ static float load(const float* p) { return *p; }
  __device__ static void store(float* p, float v) { *p = v; }
};
template <> struct Elem<bf16_t> {
  __device__ static float load(const bf16_t* p) { return bf16_bits_to_float(p->bits); }
  __device__ static void store(bf16_t* p, float v) {
    p->bits = static_cast<uint16_t>(float_to_bf16_bits(v));
  }
};
template <> struct Elem<f16_t> {
  __device__ static float load(const f16_t* p) { return f16_bits_to_float(p->bits); }
  __device__ static void store(f16_t* p, float v) {
    p->bits = static_cast<uint16_t>(float_to_f16_bits(v));
  }
};

// ---- wave64 / DPP helpers ------------------------------------------------------
// dpp_ctrl encodings (GCN/CDNA DPP): quad_perm = a | b<<2 | c<<4 | d<<6,
// row_mirror = 0x140, row_half_mirror = 0x141.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
// Sum / max over each aligned group of 16 lanes (a DPP "row"); every lane of
// the row receives the result.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f<0xB1>(x);   // quad_perm(1,0,3,2)
  x += dpp_f<0x4E>(x);   // quad_perm(2,3,0,1)
  x += dpp_f<0x141>(x);  // row_half_mirror
  x += dpp_f<0x140>(x);  // row_mirror
  return x;
}
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp_f<0xB1>(x));
  x = fmaxf(x, dpp_f<0x4E>(x));
  x = fmaxf(x, dpp_f<0x141>(x));
  x = fmaxf(x, dpp_f<0x140>(x));
  return x;
}

// XCD-aware work index: the dispatcher places workgroup b on XCD b % 8 (MI355X
// has 8 XCDs, each with its own L2); give each XCD a contiguous range of the T
// work items so that neighbouring items share an L2.
__device__ __forceinline__ int xcd_remap(int b, int T) {
  const int xcd = b & 7, slot = b >> 3;
  const int q8 = T >> 3, r8 = T & 7;
  return xcd < r8 ? xcd * (q8 + 1) + slot : r8 * (q8 + 1) + (xcd - r8) * q8 + slot;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

}  // namespace sa
