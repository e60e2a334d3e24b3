// Shared device helpers of the MI355X W8A8 linear path: element conversions with
// round-to-nearest-even, the canonical transcendental definitions the quantizers use, and
// the library's error state.  Compiled only for gfx950 with -ffp-contract=off, so every
// float expression below is evaluated exactly as written (no fused multiply-add unless a
// builtin fma is spelled out).
#pragma once

#include <hip/hip_runtime.h>
#include <type_traits>
#include <stdint.h>

#include "../../include/int8_linear_amd.h"

namespace i8l {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------- conversions
// float -> bf16, round to nearest even, by the hardware conversion (v_cvt_pk_bf16_f32).
// For every non-NaN float it equals the bit-level RNE rule, subnormals included; a NaN
// becomes the quiet NaN (u >> 16) | 0x40, keeping its sign and top payload bits.  Both
// facts were checked on gfx950 over all 2^32 inputs; the CPU oracle uses the same rule.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
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

// Activation dtype as a compile-time parameter (I8L_BF16 or I8L_F16).
template <int DT>
__device__ __forceinline__ float act_to_f32(uint32_t bits) {
  return DT == I8L_BF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
}
template <int DT>
__device__ __forceinline__ uint16_t f32_to_act(float v) {
  return DT == I8L_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
}
// Round a float through an activation dtype and back (the reference's `.to(dtype).to(f32)`).
template <int DT>
__device__ __forceinline__ float round_through(float v) {
  if (DT == I8L_BF16) return (float)(__bf16)v;
  return (float)(_Float16)v;
}

// Two values rounded through bf16 with one conversion instruction.
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){a, b}, v2bf));
}
template <int DT>
__device__ __forceinline__ uint32_t f32x2_to_act2(float a, float b) {
  if (DT == I8L_BF16) return f32x2_to_bf16x2_bits(a, b);
  return f32_to_f16_bits(a) | ((uint32_t)f32_to_f16_bits(b) << 16);
}
template <int DT>
__device__ __forceinline__ void round_through2(float& a, float& b) {
  if (DT == I8L_BF16) {
    const uint32_t p = f32x2_to_bf16x2_bits(a, b);
    a = __uint_as_float(p << 16);
    b = __uint_as_float(p & 0xffff0000u);
  } else {
    a = round_through<DT>(a);
    b = round_through<DT>(b);
  }
}

// Runtime-dtype forms, for code outside the per-element hot loops.
__device__ __forceinline__ float act_to_f32(uint32_t bits, int dtype) {
  return dtype == I8L_BF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
}

// ---------------------------------------------------------------- kernel arguments
// Kernel arguments into SGPRs, all at once.  The compiler loads each argument where it is
// first used, and a branch on one (on gridDim, on a size) makes every load after it wait for
// it: a round trip to the argument segment per branch, each 0.2-0.3 us at a kernel's start
// (the segment is cold), before the first copy is requested.  Naming the arguments in one
// empty asm statement issues their loads together, waited for once; later uses read the same
// registers.  (Each asm statement bounds the scheduling of the loads that feed it, so one
// statement takes them all.)
template <typename T>
__device__ __forceinline__ int64_t pin_value(T v) {
  if constexpr (std::is_pointer_v<T>)
    return (int64_t)(uintptr_t)v;
  else if constexpr (std::is_same_v<T, float>)
    return __float_as_int(v);                // the bits: no conversion instruction
  else
    return (int64_t)v;
}
// The grid size and up to 14 arguments.
template <typename... T>
__device__ __forceinline__ void pin_vals(T... v) {
  static_assert(sizeof...(T) <= 14, "at most 14 arguments");
  const int64_t x[14] = {pin_value(v)...};
  asm volatile("" ::"s"((int)gridDim.x), "s"((int)gridDim.y), "s"((int)gridDim.z), "s"(x[0]),
               "s"(x[1]), "s"(x[2]), "s"(x[3]), "s"(x[4]), "s"(x[5]), "s"(x[6]), "s"(x[7]),
               "s"(x[8]), "s"(x[9]), "s"(x[10]), "s"(x[11]), "s"(x[12]), "s"(x[13]));
}

// ---------------------------------------------------------------- canonical math
// clamp(rint(v), -128, 127) as the low byte of the result (the byte an int8 code is stored
// as), without a float-to-int conversion: the clamp is taken first, which gives the same
// integer since both bounds are integers, and adding 1.5 * 2^23 rounds it to an integer in
// that one IEEE addition (round half to even, as rint), leaving it in the low mantissa bits
// of a float whose exponent is fixed: bits = 0x4B400000 + rint(v), two's complement in the
// low byte for negative codes.
__device__ __forceinline__ uint32_t code_rne(float v) {
  const float t = fminf(fmaxf(v, -128.0f), 127.0f) + 12582912.0f;
  return __float_as_uint(t) & 0xffu;
}

// exp(x) for float x, defined so that host and device give identical bits: Cody-Waite
// range reduction x = k*ln2 + r (k = rne(x*log2(e)), ln2 split in a short head and a
// tail, each subtraction a single fma), then e^r from its Taylor series to degree 7 in
// Horner form with fma, scaled by 2^k.  |r| <= 0.35, so the truncation error is below
// 6e-9 relative.  Results below the normal range (x < -87) are returned as 0; above
// FLT_MAX they overflow to +inf; NaN returns itself.  Only IEEE add/mul/fma/rint/ldexp
// are used.  Written without branches: the input is clamped to [-87.5, 89.5] so that
// k stays within [-127, 130], the scaling by 2^k is one ldexp (exact for the normal
// results of the kept range, and the same single rounding to inf on overflow as the
// oracle's two-step product), and the special ranges are selected at the end.  This
// branch-free form gives the oracle's bits for all 2^32 inputs (checked on gfx950).
// The polynomial part for x already in [-87.5, 89.5]: the value before the range selects.
__device__ __forceinline__ float canon_expf_core(float xc) {
  const float kf = __builtin_rintf(xc * 0x1.715476p+0f);
  float r = __builtin_fmaf(kf, -0x1.62e4p-1f, xc);
  r = __builtin_fmaf(kf, -0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;                  // 1/5040
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);  // 1/720
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);   // 1/120
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);   // 1/24
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);   // 1/6
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, (int)kf);
}
// Above 89 the clamped input already overflows to +inf, so only the low range is selected.
__device__ __forceinline__ float canon_expf(float x) {
  const float e = canon_expf_core(__builtin_amdgcn_fmed3f(x, -87.5f, 89.5f));
  return x != x ? x : x < -87.0f ? 0.0f : e;
}

// 1/sqrt(v) as the correctly rounded double result rounded once more to float.
__device__ __forceinline__ float canon_rsqrtf(float v) {
  return (float)(1.0 / __builtin_sqrt((double)v));
}

// ---------------------------------------------------------------- cross-lane moves
// DPP controls (gfx9): quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror, row_mirror.
constexpr int kQuadSwap1 = 0xB1, kQuadSwap2 = 0x4E, kHalfMirror = 0x141, kRowMirror = 0x140;
// ds_swizzle bitmask mode: lane ^ 16 within each 32-lane half.
constexpr int kSwizzleXor16 = 0x401F;

// Every control used is a full permutation, so no lane reads an invalid source.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}

// Maximum over each aligned group of G lanes (G = 16, 32 or 64); every lane returns its
// group's.  Four DPP steps cover a 16-lane row; a swizzle and a permute cover 32 and 64.
template <int G>
__device__ __forceinline__ float group_max(float v) {
  static_assert(G == 16 || G == 32 || G == 64, "groups of 16, 32 or 64 lanes");
  v = fmaxf(v, __int_as_float(dpp_i<kQuadSwap1>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_i<kQuadSwap2>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_i<kHalfMirror>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_i<kRowMirror>(__float_as_int(v))));
  if constexpr (G >= 32)
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), kSwizzleXor16)));
  if constexpr (G == 64) v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

// Doubles moved across lanes as two 32-bit halves.
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const int lo = dpp_i<CTRL>((int)(uint32_t)u), hi = dpp_i<CTRL>((int)(uint32_t)(u >> 32));
  return __builtin_bit_cast(double, (uint64_t)(uint32_t)lo | ((uint64_t)(uint32_t)hi << 32));
}
__device__ __forceinline__ double swz16_d(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_ds_swizzle((int)(uint32_t)u, kSwizzleXor16);
  const int hi = __builtin_amdgcn_ds_swizzle((int)(uint32_t)(u >> 32), kSwizzleXor16);
  return __builtin_bit_cast(double, (uint64_t)(uint32_t)lo | ((uint64_t)(uint32_t)hi << 32));
}
__device__ __forceinline__ double readlane_d(double v, int lane) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_readlane((int)(uint32_t)u, lane);
  const int hi = __builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
  return __builtin_bit_cast(double, (uint64_t)(uint32_t)lo | ((uint64_t)(uint32_t)hi << 32));
}

// Sum over each aligned group of G lanes (G = 16, 32 or 64) as a perfect binary tree, lane
// i of the group being leaf i; every lane returns its group's sum.  Pairs, quads, then (each
// quad being uniform) a mirror within 8 lanes and within 16 pairs the blocks below them, a
// swizzle pairs the 16-lane halves of 32, and the two 32-lane halves are read back last.
// IEEE addition is commutative, so both partners of each step hold the same node.
template <int G>
__device__ __forceinline__ double group_tree_sum(double v) {
  static_assert(G == 16 || G == 32 || G == 64, "groups of 16, 32 or 64 lanes");
  v = v + dpp_d<kQuadSwap1>(v);    // pairs
  v = v + dpp_d<kQuadSwap2>(v);    // quads
  v = v + dpp_d<kHalfMirror>(v);   // 8 lanes
  v = v + dpp_d<kRowMirror>(v);    // 16 lanes
  if constexpr (G >= 32) v = v + swz16_d(v);   // 32 lanes
  if constexpr (G == 64) v = readlane_d(v, 0) + readlane_d(v, 32);
  return v;
}

// group_tree_sum of N independent values, level by level across the values, so that the
// cross-lane moves of one value overlap the additions of the others (each value's sum is
// the same tree, bit for bit).
template <int G, int N>
__device__ __forceinline__ void group_tree_sum_n(double (&v)[N]) {
  static_assert(G == 16 || G == 32 || G == 64, "groups of 16, 32 or 64 lanes");
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = v[i] + dpp_d<kQuadSwap1>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = v[i] + dpp_d<kQuadSwap2>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = v[i] + dpp_d<kHalfMirror>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = v[i] + dpp_d<kRowMirror>(v[i]);
  if constexpr (G >= 32) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = v[i] + swz16_d(v[i]);
  }
  if constexpr (G == 64) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = readlane_d(v[i], 0) + readlane_d(v[i], 32);
  }
}

// group_max of N independent values, level by level across the values.
template <int G, int N>
__device__ __forceinline__ void group_max_n(float (&v)[N]) {
  static_assert(G == 16 || G == 32 || G == 64, "groups of 16, 32 or 64 lanes");
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = fmaxf(v[i], __int_as_float(dpp_i<kQuadSwap1>(__float_as_int(v[i]))));
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = fmaxf(v[i], __int_as_float(dpp_i<kQuadSwap2>(__float_as_int(v[i]))));
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = fmaxf(v[i], __int_as_float(dpp_i<kHalfMirror>(__float_as_int(v[i]))));
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = fmaxf(v[i], __int_as_float(dpp_i<kRowMirror>(__float_as_int(v[i]))));
  if constexpr (G >= 32) {
#pragma unroll
    for (int i = 0; i < N; ++i)
      v[i] = fmaxf(v[i], __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v[i]), kSwizzleXor16)));
  }
  if constexpr (G == 64) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = fmaxf(v[i], __shfl_xor(v[i], 32));
  }
}

// ---------------------------------------------------------------- errors
void set_error(const char* fmt, ...);
int hip_status(hipError_t e, const char* where);

}  // namespace i8l
