// Fused per-token int8 quantizers for MI355X (gfx950): add+RMSNorm+quantize,
// SiLU-and-mul+quantize and the plain per-token quantizer.  One workgroup per token row.
//
// Arithmetic follows the reference's Triton kernels step for step
// (AshrithaG/int8-linear, int8_linear/fused_quant.py): the residual add and the norm in
// fp32 (60-69), the normalized value rounded to the weight dtype, multiplied by the weight
// and rounded to the activation dtype (72), the SiLU and its rounding (84-87), and the
// quantizer _quantize_row (41-53):
//     scale = absmax / 127;  inv = absmax == 0 ? 0 : 127 / absmax;
//     q = clamp(rne(y * inv), -128, 127)
// Three points the reference leaves to Triton/libdevice are fixed here so that the CPU
// oracle reproduces every bit:
//   * sum(x^2) is a pairwise tree in double over the row padded with zeros to a power of
//     two, leaf i = x_i^2 (exact in double); thread t owns the contiguous leaves
//     [E*t, E*t+E), wave lanes combine by xor-butterfly and waves in pairwise order, which
//     is the same perfect binary tree for every launch shape;  var = f32(sum / H);
//   * rsqrt(v) = f32(1 / sqrt(double(v))) (IEEE double sqrt and divide);
//   * exp is canon_expf (Cody-Waite + degree-7 Taylor with explicit fma).
// Compiled with -ffp-contract=off: every other operation is the single IEEE fp32 op written.
#include "i8l_common.h"

namespace i8l {

namespace {

__device__ __forceinline__ void unpack8(uint4 v, int dtype, float* o) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = act_to_f32(w[i] & 0xffffu, dtype);
    o[2 * i + 1] = act_to_f32(w[i] >> 16, dtype);
  }
}

// Load E consecutive elements [base, base+E) of a row of length n (zeros past the end).
template <int E>
__device__ __forceinline__ void load_row(const uint16_t* p, int base, int n, int dtype, bool vec,
                                         float* o) {
  if (vec) {
#pragma unroll
    for (int j = 0; j < E; j += 8) {
      if (base + j < n) {
        unpack8(*(const uint4*)(p + base + j), dtype, o + j);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[j + i] = 0.0f;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < E; ++j) o[j] = base + j < n ? act_to_f32(p[base + j], dtype) : 0.0f;
  }
}

template <int E>
__device__ __forceinline__ void store_act(uint16_t* p, int base, int n, int dtype, bool vec,
                                          const float* v) {
  if (vec) {
#pragma unroll
    for (int j = 0; j < E; j += 8) {
      if (base + j < n) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          w[i] = f32_to_act(v[j + 2 * i], dtype) | ((uint32_t)f32_to_act(v[j + 2 * i + 1], dtype) << 16);
        *(uint4*)(p + base + j) = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < E; ++j)
      if (base + j < n) p[base + j] = f32_to_act(v[j], dtype);
  }
}

// Block-wide max of non-negative floats (exact: max is order-free).
__device__ __forceinline__ float block_max(float v, float* sh) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  const int nw = blockDim.x >> 6, wave = threadIdx.x >> 6;
  if (nw == 1) return v;
  __syncthreads();  // sh may still be read by a previous reduction
  if ((threadIdx.x & 63) == 0) sh[wave] = v;
  __syncthreads();
  float m = sh[0];
  for (int w = 1; w < nw; ++w) m = fmaxf(m, sh[w]);
  return m;
}

// Quantize E values of one row and store the codes; thread 0 stores the scale.
template <int E>
__device__ __forceinline__ void quantize_store(const float* y, int base, int n, int8_t* qrow,
                                               float* scale_out, bool vec, int precise,
                                               float* sh) {
  float am = 0.0f;
#pragma unroll
  for (int j = 0; j < E; ++j) am = fmaxf(am, fabsf(y[j]));
  const float absmax = block_max(am, sh);
  float scale, inv;
  if (precise) {
    scale = absmax / 127.0f;
    inv = absmax == 0.0f ? 0.0f : 127.0f / absmax;
  } else {
    scale = absmax * (1.0f / 127.0f);
    inv = absmax == 0.0f ? 0.0f : 127.0f * (1.0f / absmax);
  }
  if (threadIdx.x == 0) *scale_out = scale;
  int8_t c[E];
#pragma unroll
  for (int j = 0; j < E; ++j) {
    float v = __builtin_rintf(y[j] * inv);
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    c[j] = (int8_t)(int)v;
  }
  if (vec) {
#pragma unroll
    for (int j = 0; j < E; j += 8) {
      if (base + j < n) {
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lo |= (uint32_t)(uint8_t)c[j + i] << (8 * i);
          hi |= (uint32_t)(uint8_t)c[j + 4 + i] << (8 * i);
        }
        *(uint2*)(qrow + base + j) = make_uint2(lo, hi);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < E; ++j)
      if (base + j < n) qrow[base + j] = c[j];
  }
}

// ------------------------------------------------------------------ add + RMSNorm + quant
template <int E>
__global__ void __launch_bounds__(1024)
add_rmsnorm_quant_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ res,
                         const uint16_t* __restrict__ w, float eps, int8_t* __restrict__ q,
                         float* __restrict__ scale, uint16_t* __restrict__ rout, int H, int act,
                         int wdt, int precise, int vec) {
  __shared__ double dsh[16];
  __shared__ float fsh[16];
  const int64_t row = blockIdx.x;
  const int base = threadIdx.x * E;
  float xv[E];
  load_row<E>(x + row * H, base, H, act, vec, xv);
  if (res) {
    float rv[E];
    load_row<E>(res + row * H, base, H, act, vec, rv);
#pragma unroll
    for (int j = 0; j < E; ++j) xv[j] = xv[j] + rv[j];
    store_act<E>(rout + row * H, base, H, act, vec, xv);
  }
  // pairwise tree of x^2 in double: thread-local subtree, then lanes, then waves
  double s[E];
#pragma unroll
  for (int j = 0; j < E; ++j) s[j] = (double)xv[j] * (double)xv[j];
#pragma unroll
  for (int st = 1; st < E; st <<= 1)
#pragma unroll
    for (int j = 0; j < E; j += 2 * st) s[j] = s[j] + s[j + st];
  double tot = s[0];
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) tot = tot + __shfl_xor(tot, o);
  const int nw = blockDim.x >> 6;
  if (nw > 1) {
    if ((threadIdx.x & 63) == 0) dsh[threadIdx.x >> 6] = tot;
    __syncthreads();
    double v[16];
    for (int i = 0; i < nw; ++i) v[i] = dsh[i];
    for (int st = 1; st < nw; st <<= 1)
      for (int i = 0; i < nw; i += 2 * st) v[i] = v[i] + v[i + st];
    tot = v[0];
  }
  const float var = (float)(tot / (double)H);
  const float rs = canon_rsqrtf(var + eps);
  float wv[E];
  load_row<E>(w, base, H, wdt, vec, wv);
  float y[E];
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const float xn = xv[j] * rs;
    y[j] = round_through(round_through(xn, wdt) * wv[j], act);
  }
  quantize_store<E>(y, base, H, q + row * H, scale + row, vec, precise, fsh);
}

// ------------------------------------------------------------------ SiLU-and-mul + quant
template <int E>
__global__ void __launch_bounds__(1024)
silu_mul_quant_kernel(const uint16_t* __restrict__ gu, int8_t* __restrict__ q,
                      float* __restrict__ scale, int I, int act, int round_silu, int precise,
                      int vec) {
  __shared__ float fsh[16];
  const int64_t row = blockIdx.x;
  const int base = threadIdx.x * E;
  float g[E], u[E], y[E];
  load_row<E>(gu + row * 2 * I, base, I, act, vec, g);
  load_row<E>(gu + row * 2 * I + I, base, I, act, vec, u);
#pragma unroll
  for (int j = 0; j < E; ++j) {
    float a = g[j] / (1.0f + canon_expf(-g[j]));
    if (round_silu) a = round_through(a, act);
    y[j] = round_through(a * u[j], act);
  }
  quantize_store<E>(y, base, I, q + row * I, scale + row, vec, precise, fsh);
}

// ------------------------------------------------------------------ plain per-token quant
template <int E>
__global__ void __launch_bounds__(1024)
quant_kernel(const uint16_t* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ scale,
             int H, int act, int precise, int vec) {
  __shared__ float fsh[16];
  const int64_t row = blockIdx.x;
  const int base = threadIdx.x * E;
  float y[E];
  load_row<E>(x + row * H, base, H, act, vec, y);
  quantize_store<E>(y, base, H, q + row * H, scale + row, vec, precise, fsh);
}

bool a16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

bool act_ok(int dt) { return dt == I8L_BF16 || dt == I8L_F16; }

// elements per thread: 8 up to 8192 elements a row, then 16, 32
int pick_e(int n) { return n <= 8192 ? 8 : n <= 16384 ? 16 : 32; }

}  // namespace
}  // namespace i8l

using namespace i8l;

#define I8L_DISPATCH_E(E_, KERNEL, GRID, BLOCK, STREAM, ...)                               \
  do {                                                                                    \
    if (E_ == 8)                                                                          \
      hipLaunchKernelGGL(KERNEL<8>, GRID, BLOCK, 0, STREAM, __VA_ARGS__);                  \
    else if (E_ == 16)                                                                    \
      hipLaunchKernelGGL(KERNEL<16>, GRID, BLOCK, 0, STREAM, __VA_ARGS__);                 \
    else                                                                                  \
      hipLaunchKernelGGL(KERNEL<32>, GRID, BLOCK, 0, STREAM, __VA_ARGS__);                 \
  } while (0)

extern "C" int i8l_add_rmsnorm_quant(const void* x, const void* residual, const void* weight,
                                     float eps, int8_t* q, float* scale, void* residual_out,
                                     int64_t M, int64_t H, int32_t act_dtype, int32_t w_dtype,
                                     int32_t precise_div, void* stream) {
  if (M < 0 || H <= 0) {
    set_error("add_rmsnorm_quant: bad sizes M=%lld H=%lld", (long long)M, (long long)H);
    return I8L_INVALID_ARG;
  }
  if (!act_ok(act_dtype) || !act_ok(w_dtype)) {
    set_error("add_rmsnorm_quant: activations and weight must be bf16 or fp16");
    return I8L_UNSUPPORTED;
  }
  if ((residual == nullptr) != (residual_out == nullptr)) {
    set_error("add_rmsnorm_quant: residual and residual_out must both be given or both NULL");
    return I8L_INVALID_ARG;
  }
  if (H > 32768 || M > INT32_MAX) {
    set_error("add_rmsnorm_quant: rows longer than 32768 or more than 2^31 rows");
    return I8L_UNSUPPORTED;
  }
  if (M == 0) return I8L_OK;
  const int h = (int)H, P = next_pow2(h), E = pick_e(P);
  const int T = P / E < 64 ? 64 : P / E;
  const bool vec = h % 8 == 0 && a16(x) && a16(weight) && a16(q) && (!residual || (a16(residual) && a16(residual_out)));
  I8L_DISPATCH_E(E, add_rmsnorm_quant_kernel, dim3((unsigned)M), dim3(T), (hipStream_t)stream,
                 (const uint16_t*)x, (const uint16_t*)residual, (const uint16_t*)weight, eps, q,
                 scale, (uint16_t*)residual_out, h, act_dtype, w_dtype, precise_div, (int)vec);
  return hip_status(hipGetLastError(), "add_rmsnorm_quant launch");
}

extern "C" int i8l_silu_mul_quant(const void* gate_up, int8_t* q, float* scale, int64_t M,
                                  int64_t I, int32_t act_dtype, int32_t round_silu,
                                  int32_t precise_div, void* stream) {
  if (M < 0 || I <= 0) {
    set_error("silu_mul_quant: bad sizes M=%lld I=%lld", (long long)M, (long long)I);
    return I8L_INVALID_ARG;
  }
  if (!act_ok(act_dtype)) {
    set_error("silu_mul_quant: activations must be bf16 or fp16");
    return I8L_UNSUPPORTED;
  }
  if (I > 32768 || M > INT32_MAX) {
    set_error("silu_mul_quant: rows longer than 32768 or more than 2^31 rows");
    return I8L_UNSUPPORTED;
  }
  if (M == 0) return I8L_OK;
  const int i = (int)I, E = pick_e(i);
  int T = (i + E - 1) / E;
  T = (T + 63) / 64 * 64;
  const bool vec = i % 8 == 0 && a16(gate_up) && a16(q);
  I8L_DISPATCH_E(E, silu_mul_quant_kernel, dim3((unsigned)M), dim3(T), (hipStream_t)stream,
                 (const uint16_t*)gate_up, q, scale, i, act_dtype, round_silu, precise_div,
                 (int)vec);
  return hip_status(hipGetLastError(), "silu_mul_quant launch");
}

extern "C" int i8l_quant_per_token(const void* x, int8_t* q, float* scale, int64_t M, int64_t H,
                                   int32_t act_dtype, int32_t precise_div, void* stream) {
  if (M < 0 || H <= 0) {
    set_error("quant_per_token: bad sizes M=%lld H=%lld", (long long)M, (long long)H);
    return I8L_INVALID_ARG;
  }
  if (!act_ok(act_dtype)) {
    set_error("quant_per_token: activations must be bf16 or fp16");
    return I8L_UNSUPPORTED;
  }
  if (H > 32768 || M > INT32_MAX) {
    set_error("quant_per_token: rows longer than 32768 or more than 2^31 rows");
    return I8L_UNSUPPORTED;
  }
  if (M == 0) return I8L_OK;
  const int h = (int)H, E = pick_e(h);
  int T = (h + E - 1) / E;
  T = (T + 63) / 64 * 64;
  const bool vec = h % 8 == 0 && a16(x) && a16(q);
  I8L_DISPATCH_E(E, quant_kernel, dim3((unsigned)M), dim3(T), (hipStream_t)stream,
                 (const uint16_t*)x, q, scale, h, act_dtype, precise_div, (int)vec);
  return hip_status(hipGetLastError(), "quant_per_token launch");
}
