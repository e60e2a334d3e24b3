/*
 * CPU oracle of the W8A8 linear path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's arithmetic (AshrithaG/int8-linear), used by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker.  The
 * product library never links, loads or calls this file.
 *
 * Built with gcc -O3 -ffp-contract=off (no fast-math): every float expression is the IEEE
 * operation written, rounded to nearest even, so results are bit-reproducible.
 *
 * What pins each function (tests/test_oracle.py):
 *   or_gemm_i32         float64 matmul of the int8 operands (exact below 2^53); brute force
 *   or_epilogue         float64 reference within 1 bf16 ulp / the reference's rel. tolerance;
 *                       exact results for power-of-two scales
 *   or_f32_to_bf16/f16  torch's .to(bfloat16/float16) on edge values (ties, NaN, inf, subnormal)
 *   or_expf             math.exp rounded to float32, within 1 ulp over a dense sweep
 *   or_rsqrtf           decimal-module 1/sqrt to 40 digits, rounded to float32
 *   or_quantize_row     zero row, row max -> +-127, hand-built half-way ties (RNE)
 *   or_add_rmsnorm_quant, or_silu_mul_quant, or_quant_per_token
 *                       the reference's own torch restatements (tests/test_fused_quant.py:26-51)
 *                       under its tolerance, residual bit-exact; closed forms (constant rows)
 *   or_quant_rows_div   torch restatement of bench/bench_linear.py:146-150, bit-exact
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_BF16 1
#define OR_F16 2
#define OR_F32 3
#define OR_I32 4

/* ------------------------------------------------------------------ conversions */
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* float -> bf16 bits, round to nearest even (torch's rule for every non-NaN value).  A NaN
 * becomes the quiet NaN (u >> 16) | 0x40, keeping its sign and top payload bits: the rule
 * of the gfx950 conversion instruction the device code uses (torch writes 0x7FC0 for every
 * NaN, NVIDIA hardware 0x7FFF; no reference result depends on the payload). */
uint16_t or_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if (f != f) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
float or_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* float -> IEEE binary16 bits, round to nearest even, subnormals, overflow to inf. */
uint16_t or_f32_to_f16(float f) {
  const uint32_t x = f2u(f);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return sign | 0x7e00u;      /* NaN */
  if (ax >= 0x477ff000u) return sign | 0x7c00u;     /* >= 65520 rounds to inf */
  if (ax < 0x38800000u) {                           /* below 2^-14: subnormal half */
    const float t = u2f(ax) * 16777216.0f;          /* exact: scale by 2^24 */
    return sign | (uint16_t)rintf(t);
  }
  uint32_t h = ((((ax >> 23) - 127u + 15u)) << 10) | ((ax & 0x7fffffu) >> 13);
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return sign | (uint16_t)h;
}
float or_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
  if (e == 0) {                                     /* zero / subnormal: m * 2^-24, exact */
    const float v = (float)m * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
  return u2f(sign | ((e - 15 + 127) << 23) | (m << 13));
}

static float act_load(const void* p, int64_t i, int dt) {
  const uint16_t h = ((const uint16_t*)p)[i];
  return dt == OR_BF16 ? or_bf16_to_f32(h) : or_f16_to_f32(h);
}
static uint16_t act_bits(float v, int dt) { return dt == OR_BF16 ? or_f32_to_bf16(v) : or_f32_to_f16(v); }
/* `.to(dtype).to(float32)` */
static float round_through(float v, int dt) {
  return dt == OR_BF16 ? or_bf16_to_f32(or_f32_to_bf16(v)) : or_f16_to_f32(or_f32_to_f16(v));
}

/* ------------------------------------------------------------------ canonical math */
/* exp(x): Cody-Waite reduction x = k ln2 + r, degree-7 Taylor polynomial of e^r in Horner
 * form with fma, scaled by 2^k; 0 below x = -87, +inf above FLT_MAX.  The same definition
 * as the device library's, so both give the same bits; the accuracy pin is math.exp. */
float or_expf(float x) {
  if (x != x) return x;
  if (x > 89.0f) return INFINITY;
  if (x < -87.0f) return 0.0f;
  const float kf = rintf(x * 0x1.715476p+0f);
  float r = fmaf(kf, -0x1.62e4p-1f, x);
  r = fmaf(kf, -0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;
  p = fmaf(p, r, 0x1.6c16c2p-10f);
  p = fmaf(p, r, 0x1.111112p-7f);
  p = fmaf(p, r, 0x1.555556p-5f);
  p = fmaf(p, r, 0x1.555556p-3f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int k = (int)kf;
  if (k > 127) return (p * 0x1p127f) * 2.0f;
  return p * u2f((uint32_t)(k + 127) << 23);
}

/* 1/sqrt(v): IEEE double sqrt and divide, rounded once more to float. */
float or_rsqrtf(float v) { return (float)(1.0 / sqrt((double)v)); }

/* ------------------------------------------------------------------ quantizer */
/* int8_linear/fused_quant.py:41-53 (_quantize_row): absmax, scale = absmax/127 (IEEE when
 * PRECISE_DIV, 45-46), inv = absmax == 0 ? 0 : 127/absmax, q = clamp(rint(y*inv), -128, 127).
 * precise_div == 0 stands for the non-IEEE division: multiply by the IEEE reciprocal. */
void or_quantize_row(const float* y, int64_t n, int precise_div, int8_t* q, float* scale) {
  float absmax = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    const float a = fabsf(y[i]);
    if (a > absmax) absmax = a;
  }
  float s, inv;
  if (precise_div) {
    s = absmax / 127.0f;
    inv = absmax == 0.0f ? 0.0f : 127.0f / absmax;
  } else {
    s = absmax * (1.0f / 127.0f);
    inv = absmax == 0.0f ? 0.0f : 127.0f * (1.0f / absmax);
  }
  *scale = s;
  for (int64_t i = 0; i < n; ++i) {
    float v = rintf(y[i] * inv);
    if (v < -128.0f) v = -128.0f;
    if (v > 127.0f) v = 127.0f;
    q[i] = (int8_t)v;
  }
}

/* ------------------------------------------------------------------ fused quantizers */
/* Pairwise tree sum over the leaves padded with zeros to a power of two: the order the
 * device kernel's thread/lane/wave reduction produces for any launch shape. */
static double tree_sum(double* v, int64_t n) {
  int64_t p = 1;
  while (p < n) p <<= 1;
  for (int64_t i = n; i < p; ++i) v[i] = 0.0;
  for (int64_t w = 1; w < p; w <<= 1)
    for (int64_t i = 0; i + w < p; i += 2 * w) v[i] = v[i] + v[i + w];
  return v[0];
}

/* int8_linear/fused_quant.py:56-73 (_add_rmsnorm_quant_kernel) and 95-110:
 *   x = f32(x) (+ f32(r)); r_out = cast(x); var = sum(x^2)/H; xn = x*rsqrt(var+eps);
 *   y = cast_x(f32(cast_w(xn)) * f32(w)); quantize.
 * residual == NULL is rmsnorm_quant (fused_quant.py:132-135). */
void or_add_rmsnorm_quant(const void* x, const void* res, const void* w, float eps, int8_t* q,
                          float* scale, void* rout, int64_t M, int64_t H, int act, int wdt,
                          int precise_div) {
  int64_t p = 1;
  while (p < H) p <<= 1;
  float* xs = (float*)malloc(sizeof(float) * H);
  float* y = (float*)malloc(sizeof(float) * H);
  double* sq = (double*)malloc(sizeof(double) * p);
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t i = 0; i < H; ++i) {
      float v = act_load(x, m * H + i, act);
      if (res) {
        v = v + act_load(res, m * H + i, act);
        ((uint16_t*)rout)[m * H + i] = act_bits(v, act);
      }
      xs[i] = v;
      sq[i] = (double)v * (double)v;
    }
    const double tot = tree_sum(sq, H);
    const float var = (float)(tot / (double)H);
    const float rs = or_rsqrtf(var + eps);
    for (int64_t i = 0; i < H; ++i) {
      const float xn = xs[i] * rs;
      y[i] = round_through(round_through(xn, wdt) * act_load(w, i, wdt), act);
    }
    or_quantize_row(y, H, precise_div, q + m * H, scale + m);
  }
  free(xs);
  free(y);
  free(sq);
}

/* int8_linear/fused_quant.py:76-88 (_silu_mul_quant_kernel) and 113-124:
 *   g, u = x[:, :I], x[:, I:]; a = g/(1+exp(-g)); a = f32(cast(a)) if round_silu;
 *   y = f32(cast(a*u)); quantize. */
void or_silu_mul_quant(const void* gu, int8_t* q, float* scale, int64_t M, int64_t I, int act,
                       int round_silu, int precise_div) {
  float* y = (float*)malloc(sizeof(float) * I);
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t i = 0; i < I; ++i) {
      const float g = act_load(gu, m * 2 * I + i, act);
      const float u = act_load(gu, m * 2 * I + I + i, act);
      float a = g / (1.0f + or_expf(-g));
      if (round_silu) a = round_through(a, act);
      y[i] = round_through(a * u, act);
    }
    or_quantize_row(y, I, precise_div, q + m * I, scale + m);
  }
  free(y);
}

/* The quantizer alone on a bf16/fp16 row (vLLM scaled_int8_quant's convention as the
 * reference restates it, tests/test_fused_quant.py:26-31). */
void or_quant_per_token(const void* x, int8_t* q, float* scale, int64_t M, int64_t H, int act,
                        int precise_div) {
  float* y = (float*)malloc(sizeof(float) * H);
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t i = 0; i < H; ++i) y[i] = act_load(x, m * H + i, act);
    or_quantize_row(y, H, precise_div, q + m * H, scale + m);
  }
  free(y);
}

/* bench/bench_linear.py:146-150 (quant_rows): scale = max(absmax, 1e-8)/127;
 * q = clamp(rne(x/scale), -127, 127).  The operand convention of the benchmark configs. */
void or_quant_rows_div(const void* x, int dt, int8_t* q, float* scale, int64_t R, int64_t C) {
  for (int64_t r = 0; r < R; ++r) {
    float am = 0.0f;
    for (int64_t c = 0; c < C; ++c) {
      const float a = fabsf(act_load(x, r * C + c, dt));
      if (a > am) am = a;
    }
    if (am < 1e-8f) am = 1e-8f;
    const float s = am / 127.0f;
    scale[r] = s;
    for (int64_t c = 0; c < C; ++c) {
      float v = rintf(act_load(x, r * C + c, dt) / s);
      if (v < -127.0f) v = -127.0f;
      if (v > 127.0f) v = 127.0f;
      q[r * C + c] = (int8_t)v;
    }
  }
}

/* ------------------------------------------------------------------ GEMM */
/* tests/test_kernel.py:36-38 / int8_linear/kernel.py:94-103: the exact int32 product
 * acc[m,n] = sum_k A[m,k]*B[k,n], A at a + m*sam + k*sak, B at b + k*sbk + n*sbn.
 * Partial sums stay below 2^31 for K < 2^31 / 127^2 * ... (|a*b| <= 16256). */
void or_gemm_i32(const int8_t* a, int64_t sam, int64_t sak, const int8_t* b, int64_t sbk,
                 int64_t sbn, int32_t* acc, int64_t M, int64_t N, int64_t K) {
  const int fast = sak == 1 && sbk == 1;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      const int8_t* ar = a + m * sam;
      const int8_t* br = b + n * sbn;
      int32_t s = 0;
      if (fast) {
        for (int64_t k = 0; k < K; ++k) s += (int32_t)ar[k] * (int32_t)br[k];
      } else {
        for (int64_t k = 0; k < K; ++k) s += (int32_t)ar[k * sak] * (int32_t)br[k * sbk];
      }
      acc[m * N + n] = s;
    }
}

/* int8_linear/kernel.py:105-120: out = f32(acc); out = out*sa[m|0]; out = out*sb[n|0];
 * out = out + f32(bias[n]); one cast to the output dtype (or int32 unchanged when raw). */
void or_epilogue(const int32_t* acc, int64_t M, int64_t N, const float* sa, int64_t sa_len,
                 const float* sb, int64_t sb_len, const void* bias, int bias_dt, void* out,
                 int out_dt) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      const int64_t i = m * N + n;
      if (out_dt == OR_I32) {
        ((int32_t*)out)[i] = acc[i];
        continue;
      }
      float v = (float)acc[i];
      v = v * sa[sa_len == 1 ? 0 : m];
      v = v * sb[sb_len == 1 ? 0 : n];
      if (bias_dt == OR_F32)
        v = v + ((const float*)bias)[n];
      else if (bias_dt == OR_BF16 || bias_dt == OR_F16)
        v = v + act_load(bias, n, bias_dt);
      if (out_dt == OR_F32)
        ((float*)out)[i] = v;
      else
        ((uint16_t*)out)[i] = act_bits(v, out_dt);
    }
}

/* The whole reference CPU path of one linear: exact product, then the epilogue. */
void or_w8a8_mm(const int8_t* a, const int8_t* b_nk, const float* sa, int64_t sa_len,
                const float* sb, int64_t sb_len, const void* bias, int bias_dt, void* out,
                int out_dt, int32_t* acc_scratch, int64_t M, int64_t N, int64_t K) {
  or_gemm_i32(a, K, 1, b_nk, 1, K, acc_scratch, M, N, K);
  or_epilogue(acc_scratch, M, N, sa, sa_len, sb, sb_len, bias, bias_dt, out, out_dt);
}

/* ------------------------------------------------------------------ array helpers */
void or_expf_n(const float* x, float* y, int64_t n) { for (int64_t i = 0; i < n; ++i) y[i] = or_expf(x[i]); }
void or_rsqrtf_n(const float* x, float* y, int64_t n) { for (int64_t i = 0; i < n; ++i) y[i] = or_rsqrtf(x[i]); }
void or_f32_to_bf16_n(const float* x, uint16_t* y, int64_t n) { for (int64_t i = 0; i < n; ++i) y[i] = or_f32_to_bf16(x[i]); }
void or_f32_to_f16_n(const float* x, uint16_t* y, int64_t n) { for (int64_t i = 0; i < n; ++i) y[i] = or_f32_to_f16(x[i]); }
void or_f16_to_f32_n(const uint16_t* x, float* y, int64_t n) { for (int64_t i = 0; i < n; ++i) y[i] = or_f16_to_f32(x[i]); }
