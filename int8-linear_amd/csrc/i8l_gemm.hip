// W8A8 scaled matmul for MI355X (gfx950).
//
//   out[m,n] = cast( f32(sum_k A[m,k] * B[k,n]) * sa[m|0] * sb[n|0] (+ f32(bias[n])) )
//
// Semantics follow the reference Triton kernel _w8a8_mm (AshrithaG/int8-linear,
// int8_linear/kernel.py:63-124): exact int32 accumulation (94-103), then the epilogue in
// fp32 in the order acc -> *sa -> *sb -> +bias (109-119) and one cast to the output dtype
// (120); raw mode stores the int32 accumulator (106-107).  This file is built with
// -ffp-contract=off, so the epilogue is exactly that sequence of IEEE operations.
//
// Three schedules:
//  * stream  (decode, M <= 128): weights are streamed from HBM straight into MFMA operand
//    registers (no LDS staging, every weight byte is read once); K is split across the
//    waves of a workgroup and the int32 partials are summed through LDS.
//    v_mfma_i32_16x16x64_i8 with the weight fragment as srcA (16 output columns) and the
//    activation fragment as srcB (16 tokens).
//  * staged  (prefill): BM x BN macro tiles, K in BK-byte steps double-buffered through
//    XOR-swizzled LDS, v_mfma_i32_32x32x32_i8, grouped tile order.
//  * generic: one thread per output, arbitrary strides and alignment (correct, slow);
//    taken only when the operands do not meet the fast schedules' layout requirements.
#include <stdarg.h>
#include <stdio.h>

#include "i8l_common.h"

namespace i8l {

// ------------------------------------------------------------------ epilogue
struct Epi {
  const float* sa;
  const float* sb;
  const void* bias;
  void* out;
  int64_t ldc;  // elements
  int sa_per_row, sb_per_col, bias_dtype, out_dtype;
  int M, N;
};

__device__ __forceinline__ float load_bias(const void* bias, int dt, int64_t n) {
  if (dt == I8L_BF16) return bf16_bits_to_f32(((const uint16_t*)bias)[n]);
  if (dt == I8L_F16) return f16_bits_to_f32(((const uint16_t*)bias)[n]);
  return ((const float*)bias)[n];
}

// Per-column epilogue operands of four consecutive output columns n..n+3.
struct Cols4 {
  float sb[4], bias[4];
};

// Branch-free loads of the epilogue operands of columns n..n+3: every address is chosen
// with a select from pointers that are always valid (a scalar scale is re-read with stride
// 0; an absent bias re-reads scale_b), and every bias dtype is read as 16-bit halves, so
// all loads issue in one basic block and their latency is paid once.
__device__ __forceinline__ Cols4 load_cols4(const Epi& e, int64_t n) {
  Cols4 c;
  if (e.out_dtype == I8L_I32) return c;
  const int64_t sbs = e.sb_per_col ? 1 : 0;
  const bool f32b = e.bias_dtype == I8L_F32;
  const bool hasb = e.bias_dtype != I8L_DTYPE_NONE;
  const uint16_t* bb = hasb ? (const uint16_t*)e.bias : (const uint16_t*)e.sb;
  const int64_t bstep = hasb ? (f32b ? 2 : 1) : 0;
  uint32_t lo[4], hi[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    c.sb[r] = e.sb[(n + r) * sbs];
    const uint16_t* p = bb + (n + r) * bstep;
    lo[r] = p[0];
    hi[r] = p[f32b ? 1 : 0];
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float fb = __uint_as_float(lo[r] | (hi[r] << 16));
    const float bf = bf16_bits_to_f32(lo[r]);
    const float hf = f16_bits_to_f32(lo[r]);
    c.bias[r] = !hasb ? 0.0f : f32b ? fb : e.bias_dtype == I8L_BF16 ? bf : hf;
  }
  return c;
}

// Four consecutive output columns n..n+3 of row m (n a multiple of 4; the fast schedules
// require a 16-byte aligned output with 16-byte aligned rows).
__device__ __forceinline__ float load_sa(const Epi& e, int64_t m) {
  if (e.out_dtype == I8L_I32) return 0.0f;
  return e.sa[m * (e.sa_per_row ? 1 : 0)];
}

__device__ __forceinline__ void store4s(const Epi& e, int64_t m, int64_t n, v4i acc,
                                        const Cols4& c, float sam) {
  if (e.out_dtype == I8L_I32) {
    *(v4i*)((int32_t*)e.out + m * e.ldc + n) = acc;
    return;
  }
  float o[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float v = (float)acc[r];
    v = v * sam;
    v = v * c.sb[r];
    if (e.bias_dtype != I8L_DTYPE_NONE) v = v + c.bias[r];
    o[r] = v;
  }
  if (e.out_dtype == I8L_F32) {
    *(float4*)((float*)e.out + m * e.ldc + n) = make_float4(o[0], o[1], o[2], o[3]);
  } else {
    uint32_t lo, hi;
    if (e.out_dtype == I8L_BF16) {
      lo = f32_to_bf16_bits(o[0]) | ((uint32_t)f32_to_bf16_bits(o[1]) << 16);
      hi = f32_to_bf16_bits(o[2]) | ((uint32_t)f32_to_bf16_bits(o[3]) << 16);
    } else {
      lo = f32_to_f16_bits(o[0]) | ((uint32_t)f32_to_f16_bits(o[1]) << 16);
      hi = f32_to_f16_bits(o[2]) | ((uint32_t)f32_to_f16_bits(o[3]) << 16);
    }
    *(uint2*)((uint16_t*)e.out + m * e.ldc + n) = make_uint2(lo, hi);
  }
}

__device__ __forceinline__ void store4c(const Epi& e, int64_t m, int64_t n, v4i acc,
                                        const Cols4& c) {
  store4s(e, m, n, acc, c, load_sa(e, m));
}

__device__ __forceinline__ void store4(const Epi& e, int64_t m, int64_t n, v4i acc) {
  store4c(e, m, n, acc, load_cols4(e, n));
}

__device__ __forceinline__ void store1(const Epi& e, int64_t m, int64_t n, int32_t acc) {
  if (e.out_dtype == I8L_I32) {
    ((int32_t*)e.out)[m * e.ldc + n] = acc;
    return;
  }
  float v = (float)acc;
  v = v * e.sa[e.sa_per_row ? m : 0];
  v = v * e.sb[e.sb_per_col ? n : 0];
  if (e.bias_dtype != I8L_DTYPE_NONE) v = v + load_bias(e.bias, e.bias_dtype, n);
  if (e.out_dtype == I8L_F32)
    ((float*)e.out)[m * e.ldc + n] = v;
  else if (e.out_dtype == I8L_BF16)
    ((uint16_t*)e.out)[m * e.ldc + n] = f32_to_bf16_bits(v);
  else
    ((uint16_t*)e.out)[m * e.ldc + n] = f32_to_f16_bits(v);
}

__device__ __forceinline__ v4i ld16(const int8_t* p) { return *(const v4i*)p; }
// Weight bytes are read exactly once per call: stream them past the caches.
__device__ __forceinline__ v4i ld16_stream(const int8_t* p) {
  return __builtin_nontemporal_load((const v4i*)p);
}

// ------------------------------------------------------------------ stream schedule
// Workgroup = W waves on the same 16*NT output columns and 16*MT tokens; wave w owns the
// contiguous K slice [w*ks*64, (w+1)*ks*64).  Lane l of a wave loads, per 64-byte K step,
// 16 bytes of weight row (n0 + 16t + l%16) at K offset 16*(l/16), and the same 16 bytes
// of K for token (m0 + 16i + l%16): both MFMA operands then hold the same K positions,
// so the product is the exact dot product whatever order the unit sums them in.
// Accumulator lane l, register r of fragment (i,t) is out[m0+16i+l%16][n0+16t+4*(l/16)+r].
// K steps are loaded U at a time, one group ahead of the MFMAs consuming the previous one.
__host__ __device__ constexpr int stream_unroll(int mt, int nt) { return mt * nt >= 4 ? 2 : 4; }
// Largest workgroup whose waves keep the double-buffered fragments in registers.
__host__ __device__ constexpr int stream_max_threads(int mt, int nt) {
  return 2 * stream_unroll(mt, nt) * (mt + nt) * 4 + mt * nt * 4 <= 80 ? 1024 : 512;
}

// NC (16, 8 or 4) output columns per MFMA tile: with NC < 16, MFMA rows i and i+NC read
// the same weight row (the loads coalesce, so HBM traffic is unchanged) and only rows
// below NC are stored.  Narrow tiles give narrow-N shapes more workgroups.
template <int MT, int NT, int U, int NC>
__global__ void __launch_bounds__(stream_max_threads(MT, NT))
gemm_stream(const int8_t* __restrict__ A, int64_t lda, const int8_t* __restrict__ B,
            int64_t ldb, Epi e, int ks) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int W = blockDim.x >> 6;
  const int r16 = lane & 15, grp = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * (NC * NT);
  const int64_t m0 = (int64_t)blockIdx.y * (16 * MT);
  const int64_t kbeg = (int64_t)wave * ks * 64 + grp * 16;

  const int8_t* bp[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) bp[t] = B + (n0 + NC * t + r16 % NC) * ldb + kbeg;
  const int8_t* ap[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int64_t m = m0 + 16 * i + r16;
    ap[i] = A + (m < e.M ? m : 0) * lda + kbeg;
  }

  v4i acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[i][t] = v4i{0, 0, 0, 0};

  // Two register buffers of U steps each, used in turn (no copies between them, so the
  // wait before each group's MFMAs covers exactly that group's loads).  Padding token
  // rows load row 0's bytes: their output columns are computed but never stored.
  v4i b0[U][NT], a0[U][MT], b1[U][NT], a1[U][MT];
  auto load = [&](v4i (&bb)[U][NT], v4i (&aa)[U][MT], int s) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int t = 0; t < NT; ++t) bb[u][t] = ld16_stream(bp[t] + (s + u) * 64);
#pragma unroll
      for (int i = 0; i < MT; ++i) aa[u][i] = ld16(ap[i] + (s + u) * 64);
    }
    __builtin_amdgcn_sched_barrier(0);  // issue the prefetch before any MFMA waits
  };
  auto mma = [&](const v4i (&bb)[U][NT], const v4i (&aa)[U][MT]) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t)
          acc[i][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bb[u][t], aa[u][i], acc[i][t], 0, 0, 0);
  };
  // Steady state: every load unconditional, so at each wait exactly the group after the
  // one being consumed is still in flight on every path.
  const int G = ks / U;  // groups of U steps
  load(b0, a0, 0);
  // The wave that stores fragment f (f % W == wave) loads its scales and bias now, behind
  // the first weight group, so their latency is hidden by the main loop.
  constexpr int F = MT * NT;
  Cols4 cl0;
  float sa0 = 0.0f;
  if (wave < F && 4 * grp < NC) {
    const int i = wave / NT, t = wave % NT;
    const int64_t m = m0 + 16 * i + r16;
    cl0 = load_cols4(e, n0 + NC * t + 4 * grp);
    sa0 = load_sa(e, m < e.M ? m : 0);
  }
  int g = 0;
  for (; g + 2 < G; g += 2) {
    load(b1, a1, (g + 1) * U);
    mma(b0, a0);
    load(b0, a0, (g + 2) * U);
    mma(b1, a1);
  }
  if (G - g == 2) {
    load(b1, a1, (g + 1) * U);
    mma(b0, a0);
    mma(b1, a1);
  } else {
    mma(b0, a0);
  }

  // Sum the W partial products (int32 addition is exact and order-free), then epilogue.
  extern __shared__ v4i red[];  // [W][MT*NT][64]
  if (W > 1) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int t = 0; t < NT; ++t) red[(wave * F + i * NT + t) * 64 + lane] = acc[i][t];
    __syncthreads();
  }
  for (int f = wave; f < F; f += W) {
    v4i s;
    if (W > 1) {
      s = red[f * 64 + lane];
      for (int w = 1; w < W; ++w) s += red[(w * F + f) * 64 + lane];
    } else {
      // W == 1: the fragment is this wave's own accumulator
      s = v4i{0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t)
          if (i * NT + t == f) s = acc[i][t];
    }
    const int i = f / NT, t = f % NT;
    const int64_t m = m0 + 16 * i + r16;
    if (m < e.M && 4 * grp < NC) {
      if (f == wave)
        store4s(e, m, n0 + NC * t + 4 * grp, s, cl0, sa0);
      else
        store4(e, m, n0 + NC * t + 4 * grp, s);
    }
  }
}

// ------------------------------------------------------------------ staged schedule
// Workgroup = WM x WN waves over a BM (tokens) x BN (columns) tile; K advances BK bytes per
// step through two LDS buffers.  Each LDS tile row (one token or one weight row) holds BK
// bytes as BK/16 chunks of 16 bytes, chunk c stored at slot c ^ swz(row) so that the 16
// lanes of an MFMA fragment read hit distinct banks.
template <int BK>
__device__ __forceinline__ int swz(int row) {
  constexpr int NCH = BK / 16;
  constexpr int SH = (BK == 64) ? 2 : (BK == 128 ? 1 : 0);
  return (row >> SH) & (NCH - 1);
}

template <int BM, int BN, int BK, int WM, int WN>
__global__ void __launch_bounds__(64 * WM * WN)
gemm_staged(const int8_t* __restrict__ A, int64_t lda, const int8_t* __restrict__ B,
            int64_t ldb, Epi e, int K, int group_m) {
  constexpr int T = 64 * WM * WN;
  constexpr int NCH = BK / 16;
  constexpr int CA = BM * NCH / T;  // 16-byte chunks per thread per stage, activations
  constexpr int CB = BN * NCH / T;  // weights
  static_assert(CA * T == BM * NCH && CB * T == BN * NCH, "tile does not split over threads");
  constexpr int TM = BM / WM, TN = BN / WN;  // wave tile (tokens x columns)
  constexpr int FB = TM / 32, FA = TN / 32;  // 32x32 fragments per wave tile
  constexpr int STAGE = (BM + BN) * BK;

  extern __shared__ __attribute__((aligned(16))) int8_t lds[];

  // grouped tile order (GROUP_M rows of tiles walked together for L2 reuse)
  const int pid = blockIdx.x;
  const int num_pid_m = (e.M + BM - 1) / BM;
  const int num_pid_n = e.N / BN;
  const int in_group = group_m * num_pid_n;
  const int first_m = (pid / in_group) * group_m;
  const int gsize = min(num_pid_m - first_m, group_m);
  const int pid_m = first_m + (pid % in_group) % gsize;
  const int pid_n = (pid % in_group) / gsize;
  const int64_t m0 = (int64_t)pid_m * BM, n0 = (int64_t)pid_n * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // global -> register staging: chunk j of this thread is tile row row0 + j*RSTEP, 16-byte
  // column chunk ch.  RSTEP is a multiple of 32 rows, so every chunk of a thread has the
  // same swizzle and its LDS slot is a fixed offset plus j*RSTEP*BK.
  constexpr int RSTEP = T / NCH;
  static_assert(RSTEP % 32 == 0, "row step must keep the swizzle");
  const int row0 = tid / NCH, ch = tid % NCH;
  const int lofs = row0 * BK + ((ch ^ swz<BK>(row0)) * 16);
  const int8_t* ga = A + m0 * lda + (int64_t)row0 * lda + ch * 16;
  const int8_t* gb = B + n0 * ldb + (int64_t)row0 * ldb + ch * 16;
  const int64_t m_left = e.M - m0 - row0;  // chunk j is a real token row iff j*RSTEP < m_left

  v16i acc[FA][FB];
#pragma unroll
  for (int a = 0; a < FA; ++a)
#pragma unroll
    for (int b = 0; b < FB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0;

  v4i ra[CA], rb[CB];
  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int j = 0; j < CA; ++j)
      ra[j] = j * RSTEP < m_left ? ld16(ga + (int64_t)j * RSTEP * lda + k0) : v4i{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < CB; ++j) rb[j] = ld16(gb + (int64_t)j * RSTEP * ldb + k0);
  };
  auto lstore = [&](int buf) {
    int8_t* base = lds + buf * STAGE + lofs;
#pragma unroll
    for (int j = 0; j < CA; ++j) *(v4i*)(base + j * RSTEP * BK) = ra[j];
#pragma unroll
    for (int j = 0; j < CB; ++j) *(v4i*)(base + BM * BK + j * RSTEP * BK) = rb[j];
  };

  // fragment read offsets: lane l reads row (l%32) of a 32-row block, chunk 2*kk + l/32
  const int frow = lane & 31, fhalf = lane >> 5;
  int fofs[BK / 32];
#pragma unroll
  for (int kk = 0; kk < BK / 32; ++kk) fofs[kk] = frow * BK + (((2 * kk + fhalf) ^ swz<BK>(frow)) * 16);

  const int KT = K / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) gload((int64_t)(kt + 1) * BK);
    const int8_t* base = lds + cur * STAGE;
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
      v4i fa[FA], fb[FB];
#pragma unroll
      for (int a = 0; a < FA; ++a)
        fa[a] = *(const v4i*)(base + BM * BK + (wn * TN + a * 32) * BK + fofs[kk]);
#pragma unroll
      for (int b = 0; b < FB; ++b) fb[b] = *(const v4i*)(base + (wm * TM + b * 32) * BK + fofs[kk]);
#pragma unroll
      for (int a = 0; a < FA; ++a)
#pragma unroll
        for (int b = 0; b < FB; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[a], fb[b], acc[a][b], 0, 0, 0);
    }
    if (more) lstore(cur ^ 1);
    __syncthreads();
  }

  // lane l, register r of fragment (a,b) holds
  //   out[m = m0 + wm*TM + 32b + l%32][n = n0 + wn*TN + 32a + 8*(r/4) + 4*(l/32) + r%4]
  // Columns outer (their four scales and biases loaded once), token blocks inner.
#pragma unroll
  for (int a = 0; a < FA; ++a)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t n = n0 + wn * TN + a * 32 + 8 * q + 4 * fhalf;
      Cols4 cl = load_cols4(e, n);
#pragma unroll
      for (int b = 0; b < FB; ++b) {
        const int64_t m = m0 + wm * TM + b * 32 + frow;
        const v4i v = {acc[a][b][4 * q], acc[a][b][4 * q + 1], acc[a][b][4 * q + 2],
                       acc[a][b][4 * q + 3]};
        if (m < e.M) store4c(e, m, n, v, cl);
      }
    }
}

// ------------------------------------------------------------------ generic schedule
__global__ void __launch_bounds__(256)
gemm_generic(const int8_t* __restrict__ A, int64_t sam, int64_t sak, const int8_t* __restrict__ B,
             int64_t sbk, int64_t sbn, Epi e, int64_t K) {
  const int64_t n = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
  const int64_t m = (int64_t)blockIdx.y * 4 + (threadIdx.x >> 6);
  if (m >= e.M || n >= e.N) return;
  int32_t acc = 0;
  const int8_t* a = A + m * sam;
  const int8_t* b = B + n * sbn;
  for (int64_t k = 0; k < K; ++k) acc += (int32_t)a[k * sak] * (int32_t)b[k * sbk];
  store1(e, m, n, acc);
}

// ------------------------------------------------------------------ host side
namespace {

struct StreamTile {
  int mt, nt, nc;
};
struct StagedTile {
  int bm, bn, bk, wm, wn;
};

// The tiles this library is built with.
// (MT, NT, NC): bm = 16*MT tokens, bn = NC*NT columns.  NC < 16 only with NT == 1, so bn
// names the tile unambiguously.
constexpr StreamTile kStream[] = {{1, 1, 16}, {2, 1, 16}, {4, 1, 16}, {8, 1, 16}, {1, 2, 16},
                                  {2, 2, 16}, {4, 2, 16}, {1, 1, 8},  {2, 1, 8},  {1, 1, 4}};
constexpr StagedTile kStaged[] = {{128, 128, 64, 2, 2},  {256, 128, 64, 2, 2},
                                  {128, 256, 64, 2, 2},  {256, 256, 64, 2, 2},
                                  {256, 256, 128, 2, 2}, {128, 128, 128, 2, 2}};

bool stream_ok(const i8l_config& c) {
  if (c.stages != 1 || c.split_k != 1 || c.bm % 16) return false;
  if (c.warps < 1 || c.bk != 64 * c.warps) return false;
  for (auto t : kStream)
    if (t.mt * 16 == c.bm && t.nt * t.nc == c.bn) {
      const int f = t.mt * t.nt;
      return c.warps * 64 <= stream_max_threads(t.mt, t.nt) &&
             (c.warps == 1 || c.warps * f * 1024 <= 96 * 1024);
    }
  return false;
}

int staged_index(const i8l_config& c) {
  if (c.stages != 2 || c.split_k != 1 || c.group_m < 1) return -1;
  for (int i = 0; i < (int)(sizeof(kStaged) / sizeof(kStaged[0])); ++i) {
    const auto& t = kStaged[i];
    if (t.bm == c.bm && t.bn == c.bn && t.bk == c.bk && t.wm * t.wn == c.warps) return i;
  }
  return -1;
}

template <int MT, int NT, int NC>
hipError_t launch_stream_u(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                           const Epi& e, int W, int ks, hipStream_t st) {
  const dim3 grid(e.N / (NC * NT), (e.M + 16 * MT - 1) / (16 * MT));
  const size_t shm = W > 1 ? (size_t)W * MT * NT * 1024 : 0;
  constexpr int UMAX = stream_unroll(MT, NT);
  if (UMAX == 4 && ks % 4 == 0)
    hipLaunchKernelGGL((gemm_stream<MT, NT, UMAX, NC>), grid, dim3(64 * W), shm, st, a, lda, b, ldb, e, ks);
  else if (ks % 2 == 0)
    hipLaunchKernelGGL((gemm_stream<MT, NT, 2, NC>), grid, dim3(64 * W), shm, st, a, lda, b, ldb, e, ks);
  else
    hipLaunchKernelGGL((gemm_stream<MT, NT, 1, NC>), grid, dim3(64 * W), shm, st, a, lda, b, ldb, e, ks);
  return hipGetLastError();
}

hipError_t launch_stream(const i8l_config& c, const int8_t* a, int64_t lda, const int8_t* b,
                         int64_t ldb, const Epi& e, int K, hipStream_t st) {
  const int mt = c.bm / 16, bn = c.bn, W = c.warps, ks = K / (64 * W);
#define I8L_STREAM(MT_, NT_, NC_)                                                          \
  if (mt == MT_ && bn == NT_ * NC_)                                                       \
    return launch_stream_u<MT_, NT_, NC_>(a, lda, b, ldb, e, W, ks, st);
  I8L_STREAM(1, 1, 16) I8L_STREAM(2, 1, 16) I8L_STREAM(4, 1, 16) I8L_STREAM(8, 1, 16)
  I8L_STREAM(1, 2, 16) I8L_STREAM(2, 2, 16) I8L_STREAM(4, 2, 16)
  I8L_STREAM(1, 1, 8) I8L_STREAM(2, 1, 8) I8L_STREAM(1, 1, 4)
#undef I8L_STREAM
  return hipErrorInvalidValue;
}

template <int BM, int BN, int BK, int WM, int WN>
hipError_t launch_staged_t(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                           const Epi& e, int K, int group_m, hipStream_t st) {
  auto kern = gemm_staged<BM, BN, BK, WM, WN>;
  const size_t shm = 2 * (size_t)(BM + BN) * BK;
  static bool attr_set = false;  // opt in to more than 64 KiB of dynamic LDS, once
  if (!attr_set && shm > 64 * 1024) {
    // An unsupported attribute is not fatal: the launch itself reports an LDS overrun.
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)shm);
    (void)hipGetLastError();
    attr_set = true;
  }
  const int tiles = ((e.M + BM - 1) / BM) * (e.N / BN);
  hipLaunchKernelGGL(kern, dim3(tiles), dim3(64 * WM * WN), shm, st, a, lda, b, ldb, e, K, group_m);
  return hipGetLastError();
}

hipError_t launch_staged(int idx, const i8l_config& c, const int8_t* a, int64_t lda,
                         const int8_t* b, int64_t ldb, const Epi& e, int K, hipStream_t st) {
  switch (idx) {
    case 0: return launch_staged_t<128, 128, 64, 2, 2>(a, lda, b, ldb, e, K, c.group_m, st);
    case 1: return launch_staged_t<256, 128, 64, 2, 2>(a, lda, b, ldb, e, K, c.group_m, st);
    case 2: return launch_staged_t<128, 256, 64, 2, 2>(a, lda, b, ldb, e, K, c.group_m, st);
    case 3: return launch_staged_t<256, 256, 64, 2, 2>(a, lda, b, ldb, e, K, c.group_m, st);
    case 4: return launch_staged_t<256, 256, 128, 2, 2>(a, lda, b, ldb, e, K, c.group_m, st);
    case 5: return launch_staged_t<128, 128, 128, 2, 2>(a, lda, b, ldb, e, K, c.group_m, st);
  }
  return hipErrorInvalidValue;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int elt_size(int dt) { return dt == I8L_BF16 || dt == I8L_F16 ? 2 : 4; }

}  // namespace

void default_config(int64_t M, int64_t N, int64_t K, i8l_config* c) {
  *c = i8l_config{0, 0, 0, 0, 0, 1, 1};
  if (M <= 128) {
    const int mt = M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8;
    // enough waves that each owns only a few 64-byte K steps, as many as fit a workgroup
    int W = stream_max_threads(mt, 1) / 64;
    while (W > 1 && (K % (64 * W) != 0 || K / (64 * W) < 4 || W * mt * 1024 > 96 * 1024)) W /= 2;
    c->bm = 16 * mt;
    c->bn = 16;
    c->warps = W;
    c->bk = 64 * W;
    c->stages = 1;
    return;
  }
  c->stages = 2;
  c->warps = 4;
  c->group_m = 8;
  c->bk = 64;
  if (M >= 512 && N % 256 == 0) {
    c->bm = 256;
    c->bn = 256;
  } else if (M >= 512) {
    c->bm = 256;
    c->bn = 128;
  } else {
    c->bm = 128;
    c->bn = 128;
  }
}

}  // namespace i8l

using namespace i8l;

extern "C" int i8l_default_config(int64_t M, int64_t N, int64_t K, i8l_config* cfg_out) {
  if (!cfg_out) {
    set_error("i8l_default_config: cfg_out is NULL");
    return I8L_INVALID_ARG;
  }
  default_config(M, N, K, cfg_out);
  return I8L_OK;
}

extern "C" int i8l_w8a8_mm_supported(int64_t M, int64_t N, int64_t K, const i8l_config* cfg) {
  i8l_config c;
  if (cfg)
    c = *cfg;
  else
    default_config(M, N, K, &c);
  if (c.bn <= 0 || c.bk <= 0 || N % c.bn || K % c.bk) {
    set_error("N=%lld and K=%lld must divide the %dx%dx%d tile", (long long)N, (long long)K,
              c.bm, c.bn, c.bk);
    return I8L_UNSUPPORTED;
  }
  if (!stream_ok(c) && staged_index(c) < 0) {
    set_error("config %dx%dx%d w%d s%d g%d k%d is not built into this library", c.bm, c.bn,
              c.bk, c.warps, c.stages, c.group_m, c.split_k);
    return I8L_UNSUPPORTED;
  }
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) {
    set_error("sizes beyond 2^31 are not supported");
    return I8L_UNSUPPORTED;
  }
  return I8L_OK;
}

extern "C" int i8l_w8a8_mm(const int8_t* a, int64_t stride_am, int64_t stride_ak, const int8_t* b,
                           int64_t stride_bk, int64_t stride_bn, const float* scale_a,
                           int64_t scale_a_len, const float* scale_b, int64_t scale_b_len,
                           const void* bias, int32_t bias_dtype, void* out, int64_t stride_cm,
                           int32_t out_dtype, int64_t M, int64_t N, int64_t K,
                           const i8l_config* cfg, void* stream) {
  if (M < 0 || N < 0 || K < 0) {
    set_error("negative size M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
    return I8L_INVALID_ARG;
  }
  if (out_dtype != I8L_BF16 && out_dtype != I8L_F16 && out_dtype != I8L_F32 &&
      out_dtype != I8L_I32) {
    set_error("unsupported output dtype code %d", out_dtype);
    return I8L_UNSUPPORTED;
  }
  const bool raw = out_dtype == I8L_I32;
  if (!raw) {
    if (scale_a_len != 1 && scale_a_len != M) {
      set_error("scale_a has %lld values for M=%lld", (long long)scale_a_len, (long long)M);
      return I8L_INVALID_ARG;
    }
    if (scale_b_len != 1 && scale_b_len != N) {
      set_error("scale_b has %lld values for N=%lld", (long long)scale_b_len, (long long)N);
      return I8L_INVALID_ARG;
    }
    if (bias_dtype != I8L_DTYPE_NONE && bias_dtype != I8L_BF16 && bias_dtype != I8L_F16 &&
        bias_dtype != I8L_F32) {
      set_error("unsupported bias dtype code %d", bias_dtype);
      return I8L_UNSUPPORTED;
    }
    if ((bias_dtype == I8L_DTYPE_NONE) != (bias == nullptr)) {
      set_error("bias pointer and bias dtype disagree");
      return I8L_INVALID_ARG;
    }
  }
  i8l_config c;
  if (cfg)
    c = *cfg;
  else
    default_config(M, N, K, &c);
  int st = i8l_w8a8_mm_supported(M, N, K, &c);
  if (st != I8L_OK) return st;
  if (M == 0 || N == 0) return I8L_OK;

  Epi e;
  e.sa = scale_a;
  e.sb = scale_b;
  e.bias = raw ? nullptr : bias;
  e.out = out;
  e.ldc = stride_cm;
  e.sa_per_row = !raw && scale_a_len == M && M > 1;
  e.sb_per_col = !raw && scale_b_len == N && N > 1;
  e.bias_dtype = raw ? I8L_DTYPE_NONE : bias_dtype;
  e.out_dtype = out_dtype;
  e.M = (int)M;
  e.N = (int)N;
  hipStream_t hs = (hipStream_t)stream;

  const int osz = elt_size(out_dtype);
  const bool fast = K > 0 && stride_ak == 1 && stride_bk == 1 && aligned16(a) && aligned16(b) &&
                    stride_am % 16 == 0 && stride_bn % 16 == 0 && aligned16(out) &&
                    (stride_cm * osz) % 16 == 0 && stride_cm >= N && N % 4 == 0 &&
                    (e.sb_per_col == 0 || aligned16(scale_b)) &&
                    (e.bias_dtype == I8L_DTYPE_NONE || aligned16(bias));
  hipError_t err;
  if (!fast) {
    const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 3) / 4));
    hipLaunchKernelGGL(gemm_generic, grid, dim3(256), 0, hs, a, stride_am, stride_ak, b,
                       stride_bk, stride_bn, e, K);
    err = hipGetLastError();
  } else if (c.stages == 1) {
    err = launch_stream(c, a, stride_am, b, stride_bn, e, (int)K, hs);
  } else {
    err = launch_staged(staged_index(c), c, a, stride_am, b, stride_bn, e, (int)K, hs);
  }
  return hip_status(err, "i8l_w8a8_mm launch");
}
