// Shared device/host helpers for the QStore gfx950 kernels.
//
// Everything here is CDNA4 (gfx950) specific: wave64, MFMA operand layouts of the
// 16x16 families, hardware RNE fp32->bf16 conversion (v_cvt_pk_bf16_f32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/qstore_hip.h"

namespace qs {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------------
// host-side error plumbing: every entry point returns a qs_status and records a
// human-readable message retrievable with qs_last_error().
// ---------------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int fail(int status, const char* fmt, ...);
int hip_check(hipError_t e, const char* what);

inline bool aligned(const void* p, int bytes) {
  return (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(bytes)) == 0;
}
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------------

// int8 code (byte b of a dword) -> exact fp32. Compiles to v_cvt_f32_i32_sdwa sext.
__device__ __forceinline__ float byte_f32(int d, int b) {
  return static_cast<float>(static_cast<signed char>(d >> (8 * b)));
}

// float(signed byte B of d) as ONE v_cvt_f32_i32 with an SDWA sign-extending byte
// select.  byte_f32 computes the same value, but whether the compiler folds the byte
// extraction into the conversion depends on the surrounding code (when it does not, each
// code costs a v_bfe_i32 more, about one VALU op per weight byte on the GEMV paths).
template <int B>
__device__ __forceinline__ float sbyte_f32(int d) {
  static_assert(B >= 0 && B < 4, "byte index");
  float r;
  if constexpr (B == 0)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(d));
  else if constexpr (B == 1)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(d));
  else if constexpr (B == 2)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(d));
  else
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(d));
  return r;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float v) {
  __bf16 b = static_cast<__bf16>(v);  // hardware RNE
  return __builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
  _Float16 h = static_cast<_Float16>(v);  // RNE
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

// Dequantize 16 int8 codes held in one 128-bit register group with one fp32 row
// scale, rounding each fp32 product to bf16 (the W8A16 weight contract
// bf16(float(code) * scale)).  Element e of the 16 lands in lo[e] / hi[e-8].
__device__ __forceinline__ void deq16_bf16(i32x4 w, float s, bf16x8& lo, bf16x8& hi) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int a = w[j], b = w[j + 2];
    lo[4 * j + 0] = static_cast<__bf16>(sbyte_f32<0>(a) * s);
    lo[4 * j + 1] = static_cast<__bf16>(sbyte_f32<1>(a) * s);
    lo[4 * j + 2] = static_cast<__bf16>(sbyte_f32<2>(a) * s);
    lo[4 * j + 3] = static_cast<__bf16>(sbyte_f32<3>(a) * s);
    hi[4 * j + 0] = static_cast<__bf16>(sbyte_f32<0>(b) * s);
    hi[4 * j + 1] = static_cast<__bf16>(sbyte_f32<1>(b) * s);
    hi[4 * j + 2] = static_cast<__bf16>(sbyte_f32<2>(b) * s);
    hi[4 * j + 3] = static_cast<__bf16>(sbyte_f32<3>(b) * s);
  }
}

__device__ __forceinline__ void deq16_f16(i32x4 w, float s, f16x8& lo, f16x8& hi) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int a = w[j], b = w[j + 2];
    lo[4 * j + 0] = static_cast<_Float16>(sbyte_f32<0>(a) * s);
    lo[4 * j + 1] = static_cast<_Float16>(sbyte_f32<1>(a) * s);
    lo[4 * j + 2] = static_cast<_Float16>(sbyte_f32<2>(a) * s);
    lo[4 * j + 3] = static_cast<_Float16>(sbyte_f32<3>(a) * s);
    hi[4 * j + 0] = static_cast<_Float16>(sbyte_f32<0>(b) * s);
    hi[4 * j + 1] = static_cast<_Float16>(sbyte_f32<1>(b) * s);
    hi[4 * j + 2] = static_cast<_Float16>(sbyte_f32<2>(b) * s);
    hi[4 * j + 3] = static_cast<_Float16>(sbyte_f32<3>(b) * s);
  }
}

// Full-wave sum with a fixed butterfly order (deterministic, identical for every
// call with the same operand).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Full-wave sum on DPP lane moves (quad swaps, half-row and row mirrors, row
// broadcasts): a fixed association order, no LDS round trips.  The total is read from
// lane 63 and returned in every lane.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
  const int t = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf, false);
  return v + __builtin_bit_cast(float, t);
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = dpp_add<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141, 0xf>(v);  // row_half_mirror
  v = dpp_add<0x140, 0xf>(v);  // row_mirror: every lane holds its row's sum
  v = dpp_add<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v = dpp_add<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3: lane 63 holds the total
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Non-contracted fp32 product / sum (keeps the reference's separate roundings).
__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float add_rn(float a, float b) { return __fadd_rn(a, b); }

// x / s for a bf16 x, |x| <= 127 s, with r = RN(1 / s): Markstein's corrected quotient
// (y0 = RN(x r), rem = fma(-y0, s, x), RN(rem r + y0); P. Markstein, IBM J. Res. Dev.
// 34(1), 1990).  For every bf16 amax with s = amax / 127 >= 2^-120 and every bf16 x with
// |x| <= amax, clamp(rint(.)) of it equals that of the correctly rounded x / s (checked
// exhaustively over all 1.07e9 such pairs by tests/quant_division_check.c); 3 VALU
// operations instead of a full division.
__device__ __forceinline__ float quot_markstein(float x, float s, float r) {
  const float y0 = mul_rn(x, r);
  return __builtin_fmaf(__builtin_fmaf(-y0, s, x), r, y0);
}

}  // namespace qs
