// Fused per-token int8 quantizers for MI355X (gfx950): add+RMSNorm+quantize,
// SiLU-and-mul+quantize and the plain per-token quantizer.
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
//     two, leaf i = x_i^2 (exact in double);  var = f32(sum / H);
//   * rsqrt(v) = f32(1 / sqrt(double(v))) (IEEE double sqrt and divide);
//   * exp is canon_expf (Cody-Waite + degree-7 Taylor with explicit fma).
// Compiled with -ffp-contract=off: every other operation is the single IEEE fp32 op written.
//
// Launch layout.  A token row is owned by NW waves (NW = 1 for rows up to 2048 elements),
// and a workgroup holds RPB rows.  The row is cut into 8-element chunks; lane l of wave w
// owns chunks (w*J + j)*64 + l for j < J, so each load instruction of a wave reads 64
// consecutive chunks (1 KiB of bf16) and each lane's chunk j is an aligned 8-leaf subtree.
// The sum of squares is then evaluated as the perfect binary tree over the padded row:
// the 8 leaves of a chunk in-lane, 64 chunks by a lane butterfly (DPP within 16-lane rows,
// a swizzle across rows, a readlane across the halves) into an aligned 512-element node,
// the J nodes of a wave pairwise, and the NW waves pairwise through LDS.  IEEE addition is
// commutative, so both partners of each butterfly step hold the same node.  Maxima are
// order-free.  A row owned by one wave needs no LDS and no barrier.
#include "i8l_common.h"

namespace i8l {

namespace {

constexpr int kMaxWaves = 16;  // waves per workgroup (1024 threads)

// ------------------------------------------------------------------ cross-lane moves
// (DPP controls, dpp_i and group_tree_sum are in i8l_common.h)
// Sum over the 64 lanes as a perfect binary tree (lane i is leaf i); every lane returns it.
__device__ __forceinline__ double wave_tree_sum(double v) { return group_tree_sum<64>(v); }

__device__ __forceinline__ float fmax_dpp1(float v) {
  return fmaxf(v, __int_as_float(dpp_i<kQuadSwap1>(__float_as_int(v))));
}
// Maximum over the 64 lanes; every lane returns it.
__device__ __forceinline__ float wave_max(float v) {
  v = fmax_dpp1(v);
  v = fmaxf(v, __int_as_float(dpp_i<kQuadSwap2>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_i<kHalfMirror>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_i<kRowMirror>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), kSwizzleXor16)));
  return fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)),
               __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)));
}

// ------------------------------------------------------------------ row chunks
// Row geometry of one wave: which row, which of its NW waves, and the first element of
// each of its J chunks.
struct RowPos {
  int64_t row;
  int rw;     // wave index within the row
  int slot;   // row index within the workgroup
  int lane;
};

// MULTI false: one wave a row (nw == 1), so no division.
template <bool MULTI>
__device__ __forceinline__ RowPos row_pos(int nw, int rpb) {
  RowPos p;
  const int wave = threadIdx.x >> 6;
  p.lane = threadIdx.x & 63;
  p.rw = MULTI ? wave % nw : 0;
  p.slot = MULTI ? wave / nw : wave;
  p.row = (int64_t)blockIdx.x * rpb + p.slot;
  return p;
}

template <int J>
__device__ __forceinline__ int chunk_base(const RowPos& p, int j) {
  return ((p.rw * J + j) * 64 + p.lane) * 8;
}

template <int DT>
__device__ __forceinline__ void unpack8(uint4 v, float* o) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = act_to_f32<DT>(w[i] & 0xffffu);
    o[2 * i + 1] = act_to_f32<DT>(w[i] >> 16);
  }
}

// Elements [e0, e0+8) of a row of length n as floats (zeros past the end).  VEC: n is a
// multiple of 8 and the row is 16-byte aligned, so a chunk is all in or all out.  FULL (with
// VEC): the row fills the launch's chunks exactly, so every chunk is in and nothing is checked.
template <int DT, bool VEC, bool FULL = false>
__device__ __forceinline__ void load8(const uint16_t* p, int e0, int n, float* o) {
  if (VEC) {
    if (FULL || e0 < n) {
      unpack8<DT>(*(const uint4*)(p + e0), o);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = 0.0f;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = e0 + i < n ? act_to_f32<DT>(p[e0 + i]) : 0.0f;
  }
}

// The 16-bit elements [e0, e0+8) of a row packed as they lie in memory (zeros past the end).
template <bool VEC, bool FULL = false>
__device__ __forceinline__ uint4 load_raw8(const uint16_t* p, int e0, int n) {
  if (VEC) return FULL || e0 < n ? *(const uint4*)(p + e0) : make_uint4(0, 0, 0, 0);
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = e0 + 2 * i < n ? p[e0 + 2 * i] : 0u;
    const uint32_t hi = e0 + 2 * i + 1 < n ? p[e0 + 2 * i + 1] : 0u;
    w[i] = lo | (hi << 16);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}
// Elements 2i and 2i+1 of a packed chunk as floats.
template <int DT>
__device__ __forceinline__ void unpack_pair(const uint4& v, int i, float& a, float& b) {
  const uint32_t w = i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
  if (DT == I8L_BF16) {
    a = __uint_as_float(w << 16);
    b = __uint_as_float(w & 0xffff0000u);
  } else {
    a = act_to_f32<DT>(w & 0xffffu);
    b = act_to_f32<DT>(w >> 16);
  }
}

template <int DT, bool VEC, bool FULL = false>
__device__ __forceinline__ void store8(uint16_t* p, int e0, int n, const float* v) {
  if (VEC) {
    if (FULL || e0 < n) {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = f32x2_to_act2<DT>(v[2 * i], v[2 * i + 1]);
      *(uint4*)(p + e0) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (e0 + i < n) p[e0 + i] = f32_to_act<DT>(v[i]);
  }
}

// Max of non-negative values over the NW waves of a row: each wave's maximum goes through
// LDS (sh holds kMaxWaves floats) and comes back as lanes 0..nw-1 of every wave of the row.
// MULTI (nw > 1) is a compile-time choice, so a single-wave row has no branch here.
template <bool MULTI>
__device__ __forceinline__ float row_max(float v, const RowPos& p, int nw, float* sh) {
  v = wave_max(v);
  if constexpr (!MULTI) return v;
  if (p.lane == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  return wave_max(p.lane < nw ? sh[p.slot * nw + p.lane] : 0.0f);
}

// The quantizer of a row whose values y (J chunks of 8 per lane) are final: absmax over the
// row, scale and reciprocal, codes stored as 8-byte pieces, the scale by the row's first lane.
template <int J, bool VEC, bool MULTI, bool FULL = false>
__device__ __forceinline__ void quantize_store(float (&y)[J][8], const RowPos& p, int n, int nw,
                                               int8_t* qrow, float* scale_out, int precise,
                                               float* sh) {
  float am = 0.0f;
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(y[j][i]));
  const float absmax = row_max<MULTI>(am, p, nw, sh);
  // both division conventions, selected (once per row: no branch on the path)
  const float s_div = absmax / 127.0f;
  const float i_div = absmax == 0.0f ? 0.0f : 127.0f / absmax;
  const float s_rcp = absmax * (1.0f / 127.0f);
  const float i_rcp = absmax == 0.0f ? 0.0f : 127.0f * (1.0f / absmax);
  const float scale = precise ? s_div : s_rcp;
  const float inv = precise ? i_div : i_rcp;
  if (p.rw == 0 && p.lane == 0) *scale_out = scale;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e0 = chunk_base<J>(p, j);
    uint32_t c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] = code_rne(y[j][i] * inv);
    if (VEC) {
      if (FULL || e0 < n) {
        const uint32_t lo = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
        const uint32_t hi = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
        *(uint2*)(qrow + e0) = make_uint2(lo, hi);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (e0 + i < n) qrow[e0 + i] = (int8_t)c[i];
    }
  }
}

// ------------------------------------------------------------------ add + RMSNorm + quant
// The sum of squares of a wave's J chunks: leaves in-lane, then lanes, then the chunks.
// x_i^2 is exact in double (24-bit significands), so the first level's x_i^2 + x_{i+1}^2 is
// one fma: RN(x_{i+1}^2 + s) equals RN(RN(x_{i+1}^2) + s) when x_{i+1}^2 is exact.
template <int J>
__device__ __forceinline__ double wave_sumsq(const float (&xv)[J][8]) {
  double node[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    double s[8];
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const double a = (double)xv[j][i], b = (double)xv[j][i + 1];
      s[i] = __builtin_fma(b, b, a * a);
    }
#pragma unroll
    for (int st = 2; st < 8; st <<= 1)
#pragma unroll
      for (int i = 0; i < 8; i += 2 * st) s[i] = s[i] + s[i + st];
    node[j] = wave_tree_sum(s[0]);
  }
#pragma unroll
  for (int st = 1; st < J; st <<= 1)
#pragma unroll
    for (int j = 0; j < J; j += 2 * st) node[j] = node[j] + node[j + st];
  return node[0];
}

// y = cast_x( f32(cast_w(x * rs)) * f32(w) ) for the 8 elements of a chunk.
template <int DT, int WDT>
__device__ __forceinline__ void norm_chunk(float (&xv)[8], float rs, const float (&wv)[8]) {
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    float a = xv[i] * rs, b = xv[i + 1] * rs;
    round_through2<WDT>(a, b);
    a = a * wv[i];
    b = b * wv[i + 1];
    round_through2<DT>(a, b);
    xv[i] = a;
    xv[i + 1] = b;
  }
}

// J and NW are powers of two, so each wave covers an aligned power-of-two span of the row
// and the wave/chunk/lane reductions together evaluate the padded row's pairwise tree.
// FULL (row length exactly NW*J*512): no bounds checks, and every load of the row and of the
// weight vector is issued up front, before any arithmetic (the scheduler would otherwise sink
// the weight loads behind the reduction, where their latency is exposed).
template <int J, int DT, int WDT, bool VEC, bool RES, bool MULTI, bool FULL>
__global__ void __launch_bounds__(1024)
add_rmsnorm_quant_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ res,
                         const uint16_t* __restrict__ w, float eps, int8_t* __restrict__ q,
                         float* __restrict__ scale, uint16_t* __restrict__ rout, int64_t M,
                         int H, int nw, int rpb, int precise) {
  pin_vals(x, res, w, eps, q, scale, rout, M, H, nw, rpb, precise);
  static_assert(!FULL || VEC, "FULL rows are vector rows");
  __shared__ double dsh[kMaxWaves];
  __shared__ float fsh[kMaxWaves];
  const RowPos p = row_pos<MULTI>(nw, rpb);
  if (p.row >= M) return;  // whole single-wave rows only: a row of nw > 1 waves has rpb = 1
  const int64_t ro = p.row * H;
  float xv[J][8];
  uint4 wr[J];
  if constexpr (FULL) {
    uint4 xr[J], rr[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      xr[j] = *(const uint4*)(x + ro + chunk_base<J>(p, j));
      if constexpr (RES) rr[j] = *(const uint4*)(res + ro + chunk_base<J>(p, j));
    }
#pragma unroll
    for (int j = 0; j < J; ++j) wr[j] = *(const uint4*)(w + chunk_base<J>(p, j));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      unpack8<DT>(xr[j], xv[j]);
      if constexpr (RES) {
        float rv[8];
        unpack8<DT>(rr[j], rv);
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[j][i] = xv[j][i] + rv[i];
        store8<DT, true, true>(rout + ro, chunk_base<J>(p, j), H, xv[j]);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < J; ++j) load8<DT, VEC>(x + ro, chunk_base<J>(p, j), H, xv[j]);
    if constexpr (RES) {
      float rv[J][8];
#pragma unroll
      for (int j = 0; j < J; ++j) load8<DT, VEC>(res + ro, chunk_base<J>(p, j), H, rv[j]);
#pragma unroll
      for (int j = 0; j < J; ++j) {
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[j][i] = xv[j][i] + rv[j][i];
        store8<DT, VEC>(rout + ro, chunk_base<J>(p, j), H, xv[j]);
      }
    }
  }
  // sum of squares: the wave's node, then the waves of the row
  double tot = wave_sumsq<J>(xv);
  if constexpr (MULTI) {
    // the nw wave nodes (aligned, a power of two of them) become lanes 0..nw-1 of a tree
    // whose other leaves are +0, which leaves every sum unchanged
    if (p.lane == 0) dsh[threadIdx.x >> 6] = tot;
    __syncthreads();
    tot = wave_tree_sum(p.lane < nw ? dsh[p.slot * nw + p.lane] : 0.0);
  }
  const float var = (float)(tot / (double)H);
  const float rs = canon_rsqrtf(var + eps);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    float wv[8];
    if constexpr (FULL)
      unpack8<WDT>(wr[j], wv);
    else
      load8<WDT, VEC>(w, chunk_base<J>(p, j), H, wv);
    norm_chunk<DT, WDT>(xv[j], rs, wv);
  }
  quantize_store<J, VEC, MULTI, FULL>(xv, p, H, nw, q + ro, scale + p.row, precise, fsh);
}

// ------------------------------------------------------------------ SiLU-and-mul + quant
// FULL (row length exactly NW*J*512): no bounds checks.
template <int J, int DT, bool VEC, bool ROUND, bool MULTI, bool FULL>
__global__ void __launch_bounds__(1024)
silu_mul_quant_kernel(const uint16_t* __restrict__ gu, int8_t* __restrict__ q,
                      float* __restrict__ scale, int64_t M, int I, int nw, int rpb,
                      int precise) {
  pin_vals(gu, q, scale, M, I, nw, rpb, precise);
  __shared__ float fsh[kMaxWaves];
  const RowPos p = row_pos<MULTI>(nw, rpb);
  if (p.row >= M) return;
  const uint16_t* grow = gu + p.row * 2 * I;
  uint4 graw[J], uraw[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    graw[j] = load_raw8<VEC, FULL>(grow, chunk_base<J>(p, j), I);
    uraw[j] = load_raw8<VEC, FULL>(grow + I, chunk_base<J>(p, j), I);
  }
  __builtin_amdgcn_sched_barrier(0);  // every load of the row in flight before the arithmetic
  // d = 1 + exp(-g).  The range selects of canon_expf do not change d: below the normal
  // range exp is < 2^-24 and 1 + e rounds to 1 either way, the clamp already overflows
  // to +inf above 89, and a NaN g makes the quotient NaN whatever d is (checked for every
  // bf16 and fp16 g on gfx950).
  // a = g / d.  For -87 < g < +inf, d is in [1, 7e37], its reciprocal is normal, and one
  // Newton-Markstein correction of g * rcp(d) gives the correctly rounded quotient (checked
  // against IEEE division for every bf16 and fp16 g in that range on gfx950), up to the
  // sign of a zero quotient, which no output of this kernel depends on.  A wave holding any
  // other g recomputes its values with IEEE division.
  float y[J][8];
  float gmin = __builtin_inff(), gmax = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float g[2], u[2], a[2];
      unpack_pair<DT>(graw[j], i, g[0], g[1]);
      unpack_pair<DT>(uraw[j], i, u[0], u[1]);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float d = 1.0f + canon_expf_core(__builtin_amdgcn_fmed3f(-g[h], -87.5f, 89.5f));
        const float r0 = __builtin_amdgcn_rcpf(d);
        const float q0 = g[h] * r0;
        const float e = __builtin_fmaf(-d, q0, g[h]);
        // the quotient's sign is g's except for g = -0, where the correction gives +0 for
        // the IEEE -0; the sign of a zero reaches no output (its code is 0 either way, and
        // absmax takes |y|), so it is not restored here
        a[h] = __builtin_fmaf(e, r0, q0);
        gmin = fminf(gmin, g[h]);
        gmax = fmaxf(gmax, g[h]);
      }
      if (ROUND) round_through2<DT>(a[0], a[1]);
      a[0] = a[0] * u[0];
      a[1] = a[1] * u[1];
      round_through2<DT>(a[0], a[1]);
      y[j][2 * i] = a[0];
      y[j][2 * i + 1] = a[1];
    }
  if (!__all(gmin > -87.0f && gmax < __builtin_inff())) {
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float g[2], u[2], a[2];
        unpack_pair<DT>(graw[j], i, g[0], g[1]);
        unpack_pair<DT>(uraw[j], i, u[0], u[1]);
#pragma unroll
        for (int h = 0; h < 2; ++h)
          a[h] = g[h] / (1.0f + canon_expf_core(__builtin_amdgcn_fmed3f(-g[h], -87.5f, 89.5f)));
        if (ROUND) round_through2<DT>(a[0], a[1]);
        a[0] = a[0] * u[0];
        a[1] = a[1] * u[1];
        round_through2<DT>(a[0], a[1]);
        y[j][2 * i] = a[0];
        y[j][2 * i + 1] = a[1];
      }
  }
  quantize_store<J, VEC, MULTI, FULL>(y, p, I, nw, q + p.row * I, scale + p.row, precise, fsh);
}

// ------------------------------------------------------------------ plain per-token quant
template <int J, int DT, bool VEC, bool MULTI, bool FULL>
__global__ void __launch_bounds__(1024)
quant_kernel(const uint16_t* __restrict__ x, int64_t ldx, int8_t* __restrict__ q,
             float* __restrict__ scale, int64_t M, int H, int nw, int rpb, int precise) {
  pin_vals(x, ldx, q, scale, M, H, nw, rpb, precise);
  __shared__ float fsh[kMaxWaves];
  const RowPos p = row_pos<MULTI>(nw, rpb);
  if (p.row >= M) return;
  float y[J][8];
#pragma unroll
  for (int j = 0; j < J; ++j) load8<DT, VEC, FULL>(x + p.row * ldx, chunk_base<J>(p, j), H, y[j]);
  quantize_store<J, VEC, MULTI, FULL>(y, p, H, nw, q + p.row * H, scale + p.row, precise, fsh);
}

bool a16(const void* p) { return ((uintptr_t)p & 15) == 0; }


int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

bool act_ok(int dt) { return dt == I8L_BF16 || dt == I8L_F16; }

// Launch geometry: J chunks per lane, NW waves per row, RPB rows per workgroup.  A workgroup
// holds several rows only when each row is one wave: such rows never meet at a barrier, so a
// wave whose row is past M may return early.
struct Geom {
  int j, nw, rpb;
};

// Up to this many waves in total, a row is spread over as many waves as possible (one chunk
// a lane): a few rows are latency-bound, and more waves shorten each lane's serial work.
// Beyond it, each wave takes up to 4 chunks a lane, which keeps more bytes in flight per
// wave and reduces cross-wave reductions.  The RMSNorm spreads only up to half as many
// waves: from 1024 rows of 2048 a wave a row (no cross-wave reduction) is the faster.
constexpr int64_t kSpreadWaves = 4096;

// RMSNorm: powers of two throughout (the sum tree needs aligned power-of-two spans).
Geom norm_geom(int64_t M, int h, bool vec) {
  const int p = next_pow2(h);
  Geom g;
  const int64_t spread = (int64_t)M * ((p + 511) / 512);
  if (vec && spread <= kSpreadWaves / 2) {
    g.nw = p / 512 < 1 ? 1 : p / 512;
    g.j = 1;
    while (g.nw > kMaxWaves) g.nw /= 2, g.j *= 2;
  } else {
    g.j = !vec ? 4 : p <= 512 ? 1 : p <= 1024 ? 2 : 4;
    g.nw = p / (512 * g.j) < 1 ? 1 : p / (512 * g.j);
  }
  g.rpb = g.nw == 1 ? 4 : 1;
  return g;
}

// Max-only kernels: any split of the row works.
Geom flat_geom(int64_t M, int n, bool vec) {
  const int chunks = (n + 7) / 8;
  Geom g;
  const int spread_nw = (chunks + 63) / 64;
  if (vec && spread_nw <= kMaxWaves && (int64_t)M * spread_nw <= kSpreadWaves) {
    g.nw = spread_nw;
    g.j = 1;
  } else {
    g.nw = (chunks + 255) / 256;
    g.j = vec ? (chunks + 64 * g.nw - 1) / (64 * g.nw) : 4;
  }
  g.rpb = g.nw == 1 ? 4 : 1;
  return g;
}

// SiLU-and-mul: many operations an element, so rows stay spread over more waves than in the
// max-only kernels: one chunk a lane while the launch has at most kSiluWaves waves, two
// chunks up to twice that, then the max-only kernels' geometry (up to four chunks a lane).
constexpr int64_t kSiluWaves = 8192;
Geom silu_geom(int64_t M, int n, bool vec) {
  const int chunks = (n + 7) / 8;
  if (vec)
    for (int j = 1; j <= 2; j *= 2) {
      const int nw = (chunks + 64 * j - 1) / (64 * j);
      if (nw <= kMaxWaves && (int64_t)M * nw <= kSiluWaves * j) {
        Geom g;
        g.j = j;
        g.nw = nw;
        g.rpb = nw == 1 ? 4 : 1;
        return g;
      }
    }
  return flat_geom(M, n, vec);
}

dim3 grid_of(int64_t M, const Geom& g) { return dim3((unsigned)((M + g.rpb - 1) / g.rpb)); }
dim3 block_of(const Geom& g) { return dim3(64 * g.nw * g.rpb); }

// Kernel selection: the element path (VEC false) is built for J = 4 only.  The residual and
// the multi-wave row are compile-time choices of the kernel, not branches inside it.
template <int DT, int WDT, bool RES, bool MULTI>
void launch_norm_k(const Geom& g, bool vec, dim3 grid, hipStream_t st, const uint16_t* x,
                   const uint16_t* res, const uint16_t* w, float eps, int8_t* q, float* scale,
                   uint16_t* rout, int64_t M, int H, int precise) {
#define I8L_NORM(J_, V_, F_)                                                                \
  hipLaunchKernelGGL((add_rmsnorm_quant_kernel<J_, DT, WDT, V_, RES, MULTI, F_>), grid,      \
                     block_of(g), 0, st, x, res, w, eps, q, scale, rout, M, H, g.nw, g.rpb,   \
                     precise)
  const bool full = vec && H == 512 * g.j * g.nw;
  if (!vec) I8L_NORM(4, false, false);
  else if (g.j == 1 && full) I8L_NORM(1, true, true);
  else if (g.j == 1) I8L_NORM(1, true, false);
  else if (g.j == 2 && full) I8L_NORM(2, true, true);
  else if (g.j == 2) I8L_NORM(2, true, false);
  else if (full) I8L_NORM(4, true, true);
  else I8L_NORM(4, true, false);
#undef I8L_NORM
}

template <int DT, int WDT>
void launch_norm(const Geom& g, bool vec, dim3 grid, hipStream_t st, const uint16_t* x,
                 const uint16_t* res, const uint16_t* w, float eps, int8_t* q, float* scale,
                 uint16_t* rout, int64_t M, int H, int precise) {
  const bool multi = g.nw > 1;
  if (res)
    multi ? launch_norm_k<DT, WDT, true, true>(g, vec, grid, st, x, res, w, eps, q, scale, rout, M, H, precise)
          : launch_norm_k<DT, WDT, true, false>(g, vec, grid, st, x, res, w, eps, q, scale, rout, M, H, precise);
  else
    multi ? launch_norm_k<DT, WDT, false, true>(g, vec, grid, st, x, res, w, eps, q, scale, rout, M, H, precise)
          : launch_norm_k<DT, WDT, false, false>(g, vec, grid, st, x, res, w, eps, q, scale, rout, M, H, precise);
}

template <int DT, bool ROUND, bool MULTI>
void launch_silu_k(const Geom& g, bool vec, dim3 grid, hipStream_t st, const uint16_t* gu,
                   int8_t* q, float* scale, int64_t M, int I, int precise) {
#define I8L_SILU(J_, V_, F_)                                                                \
  hipLaunchKernelGGL((silu_mul_quant_kernel<J_, DT, V_, ROUND, MULTI, F_>), grid, block_of(g), \
                     0, st, gu, q, scale, M, I, g.nw, g.rpb, precise)
  const bool full = vec && I == 512 * g.j * g.nw;
  if (!vec) I8L_SILU(4, false, false);
  else if (g.j == 1 && full) I8L_SILU(1, true, true);
  else if (g.j == 1) I8L_SILU(1, true, false);
  else if (g.j == 2 && full) I8L_SILU(2, true, true);
  else if (g.j == 2) I8L_SILU(2, true, false);
  else if (g.j == 3) I8L_SILU(3, true, false);
  else if (full) I8L_SILU(4, true, true);
  else I8L_SILU(4, true, false);
#undef I8L_SILU
}

template <int DT, bool ROUND>
void launch_silu(const Geom& g, bool vec, dim3 grid, hipStream_t st, const uint16_t* gu,
                 int8_t* q, float* scale, int64_t M, int I, int precise) {
  if (g.nw > 1)
    launch_silu_k<DT, ROUND, true>(g, vec, grid, st, gu, q, scale, M, I, precise);
  else
    launch_silu_k<DT, ROUND, false>(g, vec, grid, st, gu, q, scale, M, I, precise);
}

template <int DT, bool MULTI>
void launch_quant_k(const Geom& g, bool vec, dim3 grid, hipStream_t st, const uint16_t* x,
                    int64_t ldx, int8_t* q, float* scale, int64_t M, int H, int precise) {
#define I8L_QUANT(J_, V_, F_)                                                               \
  hipLaunchKernelGGL((quant_kernel<J_, DT, V_, MULTI, F_>), grid, block_of(g), 0, st, x, ldx, \
                     q, scale, M, H, g.nw, g.rpb, precise)
  const bool full = vec && H == 512 * g.j * g.nw;
  if (!vec) I8L_QUANT(4, false, false);
  else if (g.j == 1) I8L_QUANT(1, true, false);
  else if (g.j == 2) I8L_QUANT(2, true, false);
  else if (g.j == 3) I8L_QUANT(3, true, false);
  else if (full) I8L_QUANT(4, true, true);
  else I8L_QUANT(4, true, false);
#undef I8L_QUANT
}

template <int DT>
void launch_quant(const Geom& g, bool vec, dim3 grid, hipStream_t st, const uint16_t* x,
                  int64_t ldx, int8_t* q, float* scale, int64_t M, int H, int precise) {
  if (g.nw > 1)
    launch_quant_k<DT, true>(g, vec, grid, st, x, ldx, q, scale, M, H, precise);
  else
    launch_quant_k<DT, false>(g, vec, grid, st, x, ldx, q, scale, M, H, precise);
}

}  // namespace
}  // namespace i8l

using namespace i8l;

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
  const int h = (int)H;
  const bool vec = h % 8 == 0 && a16(x) && a16(weight) && a16(q) &&
                   (!residual || (a16(residual) && a16(residual_out)));
  const Geom g = norm_geom(M, h, vec);
  const hipStream_t st = (hipStream_t)stream;
  auto go = [&](auto launch) {
    launch(g, vec, grid_of(M, g), st, (const uint16_t*)x, (const uint16_t*)residual,
           (const uint16_t*)weight, eps, q, scale, (uint16_t*)residual_out, M, h, precise_div);
  };
  if (act_dtype == I8L_BF16)
    w_dtype == I8L_BF16 ? go(launch_norm<I8L_BF16, I8L_BF16>) : go(launch_norm<I8L_BF16, I8L_F16>);
  else
    w_dtype == I8L_BF16 ? go(launch_norm<I8L_F16, I8L_BF16>) : go(launch_norm<I8L_F16, I8L_F16>);
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
  const int i = (int)I;
  const bool vec = i % 8 == 0 && a16(gate_up) && a16(q);
  const hipStream_t st = (hipStream_t)stream;
  const Geom g = silu_geom(M, i, vec);
  auto go = [&](auto launch) {
    launch(g, vec, grid_of(M, g), st, (const uint16_t*)gate_up, q, scale, M, i, precise_div);
  };
  if (act_dtype == I8L_BF16)
    round_silu ? go(launch_silu<I8L_BF16, true>) : go(launch_silu<I8L_BF16, false>);
  else
    round_silu ? go(launch_silu<I8L_F16, true>) : go(launch_silu<I8L_F16, false>);
  return hip_status(hipGetLastError(), "silu_mul_quant launch");
}

extern "C" int i8l_quant_per_token(const void* x, int64_t ldx, int8_t* q, float* scale,
                                   int64_t M, int64_t H, int32_t act_dtype, int32_t precise_div,
                                   void* stream) {
  if (M < 0 || H <= 0 || ldx < H) {
    set_error("quant_per_token: bad sizes M=%lld H=%lld ldx=%lld", (long long)M, (long long)H,
              (long long)ldx);
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
  const int h = (int)H;
  const bool vec = h % 8 == 0 && ldx % 8 == 0 && a16(x) && a16(q);
  const Geom g = flat_geom(M, h, vec);
  const hipStream_t st = (hipStream_t)stream;
  if (act_dtype == I8L_BF16)
    launch_quant<I8L_BF16>(g, vec, grid_of(M, g), st, (const uint16_t*)x, ldx, q, scale, M, h,
                           precise_div);
  else
    launch_quant<I8L_F16>(g, vec, grid_of(M, g), st, (const uint16_t*)x, ldx, q, scale, M, h,
                          precise_div);
  return hip_status(hipGetLastError(), "quant_per_token launch");
}
