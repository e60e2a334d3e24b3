// Shared device helpers of the MI355X W8A8 linear path: element conversions with
// round-to-nearest-even, the canonical transcendental definitions the quantizers use, and
// the library's error state.  Compiled only for gfx950 with -ffp-contract=off, so every
// float expression below is evaluated exactly as written (no fused multiply-add unless a
// builtin fma is spelled out).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/int8_linear_amd.h"

namespace i8l {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------- conversions
// float -> bf16, round to nearest even; NaN becomes the quiet NaN 0x7FC0 (torch's rule).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// float -> IEEE half, round to nearest even, with subnormals and overflow to infinity.
// (_Float16 conversion is v_cvt_f16_f32, which rounds to nearest even; fp16 denormals are
// kept on gfx950.)
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Round a float through an activation dtype and back (the reference's `.to(dtype).to(f32)`).
__device__ __forceinline__ float round_through(float v, int dtype) {
  if (dtype == I8L_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  return f16_bits_to_f32(f32_to_f16_bits(v));
}
__device__ __forceinline__ float act_to_f32(uint32_t bits, int dtype) {
  return dtype == I8L_BF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
}
__device__ __forceinline__ uint16_t f32_to_act(float v, int dtype) {
  return dtype == I8L_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
}

// ---------------------------------------------------------------- canonical math
// exp(x) for float x, defined so that host and device give identical bits: Cody-Waite
// range reduction x = k*ln2 + r (k = rne(x*log2(e)), ln2 split in a short head and a
// tail, each subtraction a single fma), then e^r from its Taylor series to degree 7 in
// Horner form with fma, scaled by 2^k.  |r| <= 0.35, so the truncation error is below
// 6e-9 relative.  Results below the normal range (x < -87) are returned as 0; above
// FLT_MAX they overflow to +inf.  Only IEEE add/mul/fma/rint are used.
__device__ __forceinline__ float canon_expf(float x) {
  if (x != x) return x;
  if (x > 89.0f) return __builtin_inff();
  if (x < -87.0f) return 0.0f;
  const float kf = __builtin_rintf(x * 0x1.715476p+0f);
  float r = __builtin_fmaf(kf, -0x1.62e4p-1f, x);
  r = __builtin_fmaf(kf, -0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;                  // 1/5040
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);  // 1/720
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);   // 1/120
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);   // 1/24
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);   // 1/6
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int k = (int)kf;
  if (k > 127) return (p * 0x1p127f) * 2.0f;
  return p * __uint_as_float((uint32_t)(k + 127) << 23);
}

// 1/sqrt(v) as the correctly rounded double result rounded once more to float.
__device__ __forceinline__ float canon_rsqrtf(float v) {
  return (float)(1.0 / __builtin_sqrt((double)v));
}

// ---------------------------------------------------------------- errors
void set_error(const char* fmt, ...);
int hip_status(hipError_t e, const char* where);

}  // namespace i8l
