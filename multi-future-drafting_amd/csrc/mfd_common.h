// Shared device helpers for the gfx950 (CDNA4) kernels of the MFD hot path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mfd_hip.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

#define MFD_WAVE 64

// v_mfma_f32_32x32x16_bf16: C[32x32] += A[32x16] B[16x32]. Lane l holds row/col (l % 32) of A/B and
// eight k values; any k assignment works as long as A and B use the same one. C register r of lane l
// is row 8*(r/4) + 4*(l/32) + r%4, column l%32.
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// v_mfma_f32_16x16x32_bf16: C[16x16] += A[16x32] B[32x16]; C register r of lane l is row 4*(l/16) + r,
// column l%16.
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }
__device__ __forceinline__ uint16_t f2bf_bits(float f) {
  __bf16 h = (__bf16)f;
  return __builtin_bit_cast(uint16_t, h);
}
// fp32 -> (hi, lo) bf16 pair with hi + lo == x to about 2^-17 relative.
__device__ __forceinline__ void split_bf16(float x, __bf16& hi, __bf16& lo) {
  hi = (__bf16)x;
  lo = (__bf16)(x - (float)hi);
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
// Two fp32 values -> packed bf16 hi pair and packed bf16 lo pair (element 0 in the low half), hi + lo == x
// to about 2^-17 relative; the rounding is round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ void split2_bf16(float x0, float x1, uint32_t& hi2, uint32_t& lo2) {
  hi2 = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x0, x1}, bf16x2));
  const float h0 = __uint_as_float(hi2 << 16);
  const float h1 = __uint_as_float(hi2 & 0xffff0000u);
  lo2 = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x0 - h0, x1 - h1}, bf16x2));
}

__device__ __forceinline__ bf16x8 as_bf16x8(u16x8 v) { return __builtin_bit_cast(bf16x8, v); }

// Orderable 32-bit key of a float (larger float -> larger unsigned key; -0 < +0 is irrelevant here).
__device__ __forceinline__ uint32_t float_order_key(float f) {
  uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

#define MFD_CHECK_LAUNCH()                                  \
  do {                                                      \
    hipError_t _e = hipGetLastError();                      \
    if (_e != hipSuccess) return mfd_set_hip_error(_e);     \
  } while (0)

// implemented in mfd_api.hip
int mfd_set_error(int code, const char* fmt, ...);
int mfd_set_hip_error(hipError_t e);
// compute units of the current device (cached per device; 256 if the query fails)
int mfd_num_cus();
// Raise kernel fn's dynamic LDS limit to bytes on the current device, once per (device, kernel, bytes); first calls
// from several host threads serialise on a lock. Returns MFD_OK or the HIP error code through mfd_set_hip_error.
int mfd_set_max_lds(const void* fn, int bytes);
