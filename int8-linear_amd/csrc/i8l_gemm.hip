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

#include <algorithm>
#include <atomic>

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

// Epilogue kinds.  EK_ANY reads the output dtype, the bias dtype and the scale layout from
// the Epi at run time; the other kinds fix them at compile time (bf16 out, per-column
// scale_b, no bias or a bf16 bias), which leaves the decode kernels' critical path free of
// the dtype branches: every CU starts a short kernel with a cold instruction cache, so each
// taken branch into code not yet fetched waits for a fetch from L2.
enum { EK_ANY = 0, EK_BF16 = 1, EK_BF16_BBF16 = 2 };
template <int EK>
__device__ __forceinline__ int epi_out(const Epi& e) { return EK == EK_ANY ? e.out_dtype : I8L_BF16; }
template <int EK>
__device__ __forceinline__ int epi_bias(const Epi& e) {
  return EK == EK_ANY ? e.bias_dtype : EK == EK_BF16 ? I8L_DTYPE_NONE : I8L_BF16;
}
template <int EK>
__device__ __forceinline__ bool epi_sb_per_col(const Epi& e) { return EK == EK_ANY ? e.sb_per_col != 0 : true; }

// The kind a call can use (host side).
inline int epi_kind(const Epi& e) {
  if (e.out_dtype != I8L_BF16 || !e.sb_per_col) return EK_ANY;
  if (e.bias_dtype == I8L_DTYPE_NONE) return EK_BF16;
  if (e.bias_dtype == I8L_BF16) return EK_BF16_BBF16;
  return EK_ANY;
}

// The epilogue operands of columns n..n+3 (n a multiple of 4): one vector load for the four
// scales and one for the four bias values.  The fast schedules require 16-byte aligned
// per-column scales and bias, so these loads are aligned; the dtype tests are uniform.
template <int EK = EK_ANY>
__device__ __forceinline__ Cols4 load_cols4(const Epi& e, int64_t n) {
  Cols4 c;
  const int od = epi_out<EK>(e), bd = epi_bias<EK>(e);
  if (od == I8L_I32) return c;
  if (epi_sb_per_col<EK>(e)) {
    const float4 v = *(const float4*)(e.sb + n);
    c.sb[0] = v.x, c.sb[1] = v.y, c.sb[2] = v.z, c.sb[3] = v.w;
  } else {
    const float v = e.sb[0];
    c.sb[0] = c.sb[1] = c.sb[2] = c.sb[3] = v;
  }
  if (bd == I8L_F32) {
    const float4 v = *(const float4*)((const float*)e.bias + n);
    c.bias[0] = v.x, c.bias[1] = v.y, c.bias[2] = v.z, c.bias[3] = v.w;
  } else if (bd == I8L_BF16 || bd == I8L_F16) {
    const uint2 h = *(const uint2*)((const uint16_t*)e.bias + n);
    const uint32_t w[4] = {h.x & 0xffffu, h.x >> 16, h.y & 0xffffu, h.y >> 16};
#pragma unroll
    for (int r = 0; r < 4; ++r)
      c.bias[r] = bd == I8L_BF16 ? bf16_bits_to_f32(w[r]) : f16_bits_to_f32(w[r]);
  } else {
    c.bias[0] = c.bias[1] = c.bias[2] = c.bias[3] = 0.0f;
  }
  return c;
}

// Four consecutive output columns n..n+3 of row m (n a multiple of 4; the fast schedules
// require a 16-byte aligned output with 16-byte aligned rows).
template <int EK = EK_ANY>
__device__ __forceinline__ float load_sa(const Epi& e, int64_t m) {
  if (epi_out<EK>(e) == I8L_I32) return 0.0f;
  return e.sa[m * (e.sa_per_row ? 1 : 0)];
}

template <int EK = EK_ANY>
__device__ __forceinline__ void store4s(const Epi& e, int64_t m, int64_t n, v4i acc,
                                        const Cols4& c, float sam) {
  const int od = epi_out<EK>(e), bd = epi_bias<EK>(e);
  if (od == I8L_I32) {
    *(v4i*)((int32_t*)e.out + m * e.ldc + n) = acc;
    return;
  }
  float o[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float v = (float)acc[r];
    v = v * sam;
    v = v * c.sb[r];
    if (bd != I8L_DTYPE_NONE) v = v + c.bias[r];
    o[r] = v;
  }
  if (od == I8L_F32) {
    *(float4*)((float*)e.out + m * e.ldc + n) = make_float4(o[0], o[1], o[2], o[3]);
  } else {
    uint32_t lo, hi;
    if (od == I8L_BF16) {
      lo = f32x2_to_bf16x2_bits(o[0], o[1]);
      hi = f32x2_to_bf16x2_bits(o[2], o[3]);
    } else {
      lo = f32_to_f16_bits(o[0]) | ((uint32_t)f32_to_f16_bits(o[1]) << 16);
      hi = f32_to_f16_bits(o[2]) | ((uint32_t)f32_to_f16_bits(o[3]) << 16);
    }
    *(uint2*)((uint16_t*)e.out + m * e.ldc + n) = make_uint2(lo, hi);
  }
}

template <int EK = EK_ANY>
__device__ __forceinline__ void store4c(const Epi& e, int64_t m, int64_t n, v4i acc,
                                        const Cols4& c) {
  store4s<EK>(e, m, n, acc, c, load_sa<EK>(e, m));
}

template <int EK = EK_ANY>
__device__ __forceinline__ void store4(const Epi& e, int64_t m, int64_t n, v4i acc) {
  store4c<EK>(e, m, n, acc, load_cols4<EK>(e, n));
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

// Column tile of a decode workgroup.  The dispatcher deals workgroups to the 8 XCDs
// round-robin by linear id; with a multiple of 8 column tiles per row, XCD x is given the
// contiguous column range [x, x+1) * gridDim.x/8, so the output lines (and the L2 lines
// they are assembled in) are written from one XCD rather than in pieces from eight.
__device__ __forceinline__ int64_t xcd_col_tile() {
  const int gx = gridDim.x, bx = blockIdx.x;
  return gx % 8 == 0 ? (int64_t)(bx % 8) * (gx / 8) + bx / 8 : (int64_t)bx;
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
  const int64_t n0 = xcd_col_tile() * (NC * NT);
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

// ------------------------------------------------------------------ weights-through-LDS schedule
// Decode tile of 16*MT tokens x NC columns (NC = 16, 8 or 4).  Each wave owns one contiguous
// K slice of `steps` steps of S = 64*KS bytes.  Per step it copies its NC x S weight bytes
// into its own LDS buffer with global_load_lds_dwordx4: one instruction moves 1 KiB, whole
// row segments of S bytes, so HBM sees full cache lines (the MFMA operand layout would read
// 16 rows x 64 bytes per instruction instead).  LDS row r holds 16-byte chunk c at slot
// c ^ (r & SWM), so the MFMA-layout reads (16 rows, one chunk each) spread over the banks.
// The activations of the next step are loaded into registers while the current step
// multiplies.  A wave only reads its own buffers, so its own vmcnt wait is the only
// synchronisation until the cross-wave sum of the int32 partials.
// With NC < 16, MFMA rows i and i+NC read the same weight row and only rows below NC are
// stored.  Token rows past M read row 0 and are never stored.
__host__ __device__ constexpr int wlds_bound(int mt, int ks) { return mt * ks <= 6 ? 1024 : 512; }
// Whether the multi-step kernel's registers fit: two sets of activation fragments, the
// weight fragments of a step and the accumulators, in VGPRs (64 x 4 bytes each).
__host__ __device__ constexpr bool wlds_multi_fits(int mt, int nc, int ks) {
  return 8 * ks * mt + 4 * ks * (nc > 16 ? nc / 16 : 1) + 4 * mt * (nc > 16 ? nc / 16 : 1) <= 176;
}

// s_waitcnt vmcnt(N) (LGKM and EXP counters unconstrained), then a compiler fence so that
// no LDS read of the DMA'd data is scheduled above the wait.
template <int N>
__device__ __forceinline__ void wait_vmcnt_wlds() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}

typedef __attribute__((address_space(3))) int8_t lds_i8_t;

template <int MT, int NC, int KS, int EK>
__global__ void __launch_bounds__(wlds_bound(MT, KS))
gemm_wlds(const int8_t* __restrict__ A, int64_t lda, const int8_t* __restrict__ B, int64_t ldb,
          Epi e, int steps, int nbuf) {
  constexpr int S = 64 * KS;                 // K bytes per row per step
  constexpr int CPR = S / 16;                // 16-byte chunks per row per step
  // The swizzle XORs a slot with (row & SWM); SWM + 1 is a power of two dividing CPR, so
  // every slot maps into the same row's [0, CPR) and no address leaves the row's slice.
  constexpr int CPR_LOW = CPR & -CPR;
  constexpr int SWM = (CPR_LOW < 16 ? CPR_LOW : 16) - 1;
  static_assert(CPR % (SWM + 1) == 0, "the swizzle must permute the row's chunks");
  constexpr int SB = NC * S;                 // weight bytes per wave per step
  constexpr int NI = SB / 1024;              // DMA instructions per wave per step
  static_assert(NI * 1024 == SB, "a step must be whole 1 KiB DMA instructions");
  constexpr int AL = MT * KS;                // activation loads per lane per step
  constexpr int NCF = NC < 16 ? NC : 16;     // output columns of one MFMA fragment
  constexpr int NF = NC / NCF;               // column fragments of the tile (32 columns: 2)
  constexpr int FR = MT * NF;                // output fragments, numbered i * NF + f
  static_assert(NF * NCF == NC, "the tile must be whole column fragments");
  extern __shared__ __attribute__((aligned(16))) int8_t lds[];

  const int lane = threadIdx.x & 63;
  // wave-uniform values live in scalar registers: the per-lane address work before the first
  // load is then a few 32-bit operations
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int r16 = lane & 15, grp = lane >> 4;
  const int64_t n0 = xcd_col_tile() * NC;
  const int64_t m0 = (int64_t)blockIdx.y * (16 * MT);
  const int64_t kw = (int64_t)wave * steps * S;
  int8_t* wbuf = lds + (size_t)wave * nbuf * SB;

  // DMA sources of this lane: instruction t writes LDS bytes [t*1024, t*1024+1024) of the
  // step buffer, lane l the 16 bytes at +16*l, which is row o / S, slot (o % S) / 16.
  // Rows of a tile are < 32 apart, so their offsets fit 32 bits.
  const int8_t* Bw = B + n0 * ldb + kw;
  const int ldb32 = (int)ldb;
  const int8_t* gsrc[NI];
#pragma unroll
  for (int t = 0; t < NI; ++t) {
    const int o = t * 1024 + 16 * lane;
    const int r = o / S, c = ((o % S) / 16) ^ (r & SWM);
    gsrc[t] = Bw + (r * ldb32 + 16 * c);
  }
  // Token rows past M read the tile's first row (always valid); they are never stored.
  const int8_t* Aw = A + m0 * lda + kw + 16 * grp;
  const int lda32 = (int)lda;
  const int8_t* ap[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int ml = 16 * i + r16;
    ap[i] = Aw + (m0 + ml < e.M ? ml * lda32 : 0);
  }
  // MFMA-layout read offsets of one step: fragment f's row br, chunk 4s + grp
  int rofs[KS][NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const int br = NCF * f + r16 % NCF;
#pragma unroll
    for (int s = 0; s < KS; ++s) rofs[s][f] = br * S + 16 * ((4 * s + grp) ^ (br & SWM));
  }

  v4i acc[MT][NF];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int f = 0; f < NF; ++f) acc[i][f] = v4i{0, 0, 0, 0};

  v4i a0[KS][MT], a1[KS][MT];
  // `fenced`: nothing of the previous step's MFMA work moves below the start of the issue,
  // so the LDS reads of the buffer the step may overwrite have completed, and the loads go
  // out before anything after them.  A single-step wave needs neither, and leaving the
  // compiler free to interleave the address arithmetic with the loads issues them sooner.
  auto issue = [&](v4i (&aa)[KS][MT], int step, bool fenced) {
    if (fenced) __builtin_amdgcn_sched_barrier(0);
    lds_i8_t* dst = (lds_i8_t*)(wbuf + (step % nbuf) * SB);
    const int64_t ko = (int64_t)step * S;
#pragma unroll
    for (int t = 0; t < NI; ++t)
      __builtin_amdgcn_global_load_lds((const void*)(gsrc[t] + ko), dst + t * 1024, 16, 0, 0);
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int i = 0; i < MT; ++i) aa[s][i] = ld16(ap[i] + ko + 64 * s);
    if (fenced) __builtin_amdgcn_sched_barrier(0);
  };
  auto compute = [&](const v4i (&aa)[KS][MT], int step) {
    const int8_t* base = wbuf + (step % nbuf) * SB;
    v4i b[KS][NF];
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int f = 0; f < NF; ++f) b[s][f] = *(const v4i*)(base + rofs[s][f]);
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int f = 0; f < NF; ++f)
          acc[i][f] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b[s][f], aa[s][i], acc[i][f], 0, 0, 0);
  };

  issue(a0, 0, steps > 1);
  // The wave that stores fragment fr (fr % W == wave) loads its epilogue operands now,
  // behind the first step, so their latency hides under the main loop.
  Cols4 cl0;
  float sa0 = 0.0f;
  if (wave < FR && 4 * grp < NCF) {
    const int64_t m = m0 + 16 * (wave / NF) + r16;
    cl0 = load_cols4<EK>(e, n0 + NCF * (wave % NF) + 4 * grp);
    sa0 = load_sa<EK>(e, m < e.M ? m : 0);
  }
  // Steady state: every step's loads are issued before the wait for the previous step, and
  // the wait leaves exactly one step's loads outstanding.  The LDS reads of a step complete
  // before its MFMAs, so its buffer is free when the step two later overwrites it.
  int i = 0;
  for (; i + 2 < steps; i += 2) {
    issue(a1, i + 1, true);
    wait_vmcnt_wlds<NI + AL>();
    compute(a0, i);
    issue(a0, i + 2, true);
    wait_vmcnt_wlds<NI + AL>();
    compute(a1, i + 1);
  }
  if (steps - i == 2) {
    issue(a1, i + 1, true);
    wait_vmcnt_wlds<NI + AL>();
    compute(a0, i);
    wait_vmcnt_wlds<0>();
    compute(a1, i + 1);
  } else {
    wait_vmcnt_wlds<0>();
    compute(a0, i);
  }

  // Sum the W partial products (int32 addition is exact and order-free), then epilogue.
  v4i* red = (v4i*)(lds + (size_t)W * nbuf * SB);  // [W][FR][64]
  if (W > 1) {
#pragma unroll
    for (int q = 0; q < MT; ++q)
#pragma unroll
      for (int f = 0; f < NF; ++f) red[(wave * FR + q * NF + f) * 64 + lane] = acc[q][f];
    __syncthreads();
  }
  for (int fr = wave; fr < FR; fr += W) {
    v4i sum;
    if (W > 1) {
      sum = red[fr * 64 + lane];
      for (int w = 1; w < W; ++w) sum += red[(w * FR + fr) * 64 + lane];
    } else {
      sum = acc[0][0];
#pragma unroll
      for (int q = 0; q < MT; ++q)
#pragma unroll
        for (int f = 0; f < NF; ++f)
          if (q * NF + f == fr) sum = acc[q][f];
    }
    const int64_t m = m0 + 16 * (fr / NF) + r16;
    const int64_t n = n0 + NCF * (fr % NF) + 4 * grp;
    if (m < e.M && 4 * grp < NCF) {
      if (fr == wave)
        store4s<EK>(e, m, n, sum, cl0, sa0);
      else
        store4<EK>(e, m, n, sum);
    }
  }
}

// The same tile when every wave's K slice is a single step (K == W * 64 * KS), with the
// wave count and the epilogue kind fixed at compile time: the path from the first load to
// the last store is straight-line code apart from the wave-uniform test of which waves
// store, which matters in a kernel this short (see EK_ANY).
template <int MT, int NC, int KS, int W, int EK>
__global__ void __launch_bounds__(64 * W)
gemm_wlds1(const int8_t* __restrict__ A, int64_t lda, const int8_t* __restrict__ B, int64_t ldb,
           Epi e) {
  constexpr int S = 64 * KS;
  constexpr int CPR = S / 16;
  constexpr int CPR_LOW = CPR & -CPR;
  constexpr int SWM = (CPR_LOW < 16 ? CPR_LOW : 16) - 1;
  static_assert(CPR % (SWM + 1) == 0, "the swizzle must permute the row's chunks");
  constexpr int SB = NC * S;
  constexpr int NI = SB / 1024;
  static_assert(NI * 1024 == SB, "a step must be whole 1 KiB DMA instructions");
  constexpr int NCF = NC < 16 ? NC : 16;     // output columns of one MFMA fragment
  constexpr int NF = NC / NCF;               // column fragments of the tile (32 columns: 2)
  constexpr int FR = MT * NF;                // output fragments of the tile
  static_assert(NF * NCF == NC, "the tile must be whole column fragments");
  static_assert(FR <= W, "every fragment needs a storing wave");
  extern __shared__ __attribute__((aligned(16))) int8_t lds[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, grp = lane >> 4;
  const int64_t n0 = xcd_col_tile() * NC;
  const int64_t m0 = (int64_t)blockIdx.y * (16 * MT);
  const int64_t kw = (int64_t)wave * S;
  int8_t* wbuf = lds + (size_t)wave * SB;

  const int8_t* Bw = B + n0 * ldb + kw;
  const int ldb32 = (int)ldb;
  lds_i8_t* dst = (lds_i8_t*)wbuf;
#pragma unroll
  for (int t = 0; t < NI; ++t) {
    const int o = t * 1024 + 16 * lane;
    const int r = o / S, c = ((o % S) / 16) ^ (r & SWM);
    __builtin_amdgcn_global_load_lds((const void*)(Bw + (r * ldb32 + 16 * c)), dst + t * 1024,
                                     16, 0, 0);
  }
  const int8_t* Aw = A + m0 * lda + kw + 16 * grp;
  const int lda32 = (int)lda;
  v4i a[KS][MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int ml = 16 * i + r16;
    const int8_t* ap = Aw + (m0 + ml < e.M ? ml * lda32 : 0);
#pragma unroll
    for (int s = 0; s < KS; ++s) a[s][i] = ld16(ap + 64 * s);
  }
  // Wave w < FR stores fragment (token block w / NF, column block w % NF) and loads its
  // epilogue operands now, behind the tile; lanes past NCF columns load a valid neighbour
  // and never store.
  Cols4 cl;
  float sam = 0.0f;
  const int64_t mrow = m0 + 16 * (wave / NF) + r16;
  const int64_t ncol = n0 + NCF * (wave % NF) + 4 * (grp & (NCF / 4 - 1));
  if (wave < FR) {
    cl = load_cols4<EK>(e, ncol);
    sam = load_sa<EK>(e, mrow < e.M ? mrow : m0);
  }
  wait_vmcnt_wlds<0>();
  v4i b[KS][NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const int br = NCF * f + r16 % NCF;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      b[s][f] = *(const v4i*)(wbuf + br * S + 16 * ((4 * s + grp) ^ (br & SWM)));
  }
  v4i acc[MT][NF];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int f = 0; f < NF; ++f) acc[i][f] = v4i{0, 0, 0, 0};
#pragma unroll
  for (int s = 0; s < KS; ++s)
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int f = 0; f < NF; ++f)
        acc[i][f] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b[s][f], a[s][i], acc[i][f], 0, 0, 0);

  // cross-wave sum (exact int32), then the storing waves apply the epilogue
  v4i* red = (v4i*)(lds + (size_t)W * SB);  // [W][FR][64]
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int f = 0; f < NF; ++f) red[(wave * FR + i * NF + f) * 64 + lane] = acc[i][f];
  __syncthreads();
  if (wave < FR) {
    v4i sum = red[wave * 64 + lane];
#pragma unroll
    for (int w = 1; w < W; ++w) sum += red[(w * FR + wave) * 64 + lane];
    if (mrow < e.M && 4 * grp < NCF) store4s<EK>(e, mrow, ncol, sum, cl, sam);
  }
}

// Workgroup barrier without a memory fence: LDS accesses are ordered around it by the
// compiler-level fences; waits for outstanding memory are issued explicitly where needed.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ------------------------------------------------------------------ tile epilogue
// Output of a BM x BN macro tile from the accumulators of WM x WN waves.  For 16-bit outputs
// the values are computed in the fragment layout (scales and bias fetched with vector loads),
// written to LDS as a row-major tile with 16 bytes of padding per row (so the 32 rows one
// store instruction touches spread over the banks), and copied out with 16-byte stores,
// 64 lanes covering consecutive columns of consecutive rows.  int32 and fp32 outputs are
// stored straight from the fragments.  `lds` must hold BM * (2*BN + 16) bytes and every wave
// must be done with its previous LDS contents.
template <int BM, int BN, int WM, int WN>
constexpr int tile_epilogue_lds_bytes() { return BM * (2 * BN + 16); }

template <int BM, int BN, int WM, int WN, int FA, int FB>
__device__ __forceinline__ void tile_epilogue(const Epi& e, v16i (&acc)[FA][FB], int8_t* lds,
                                              int64_t m0, int64_t n0, int wm, int wn, int lane,
                                              int tid) {
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int T = 64 * WM * WN;
  const int frow = lane & 31, fhalf = lane >> 5;
  if (e.out_dtype == I8L_I32 || e.out_dtype == I8L_F32) {
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
    return;
  }
  constexpr int PITCH = 2 * BN + 16;  // bytes per LDS row (16-byte aligned)
  float sam[FB];
#pragma unroll
  for (int b = 0; b < FB; ++b) {
    const int64_t m = m0 + wm * TM + b * 32 + frow;
    sam[b] = load_sa(e, m < e.M ? m : 0);
  }
  const bool bf = e.out_dtype == I8L_BF16;
#pragma unroll
  for (int a = 0; a < FA; ++a) {
    Cols4 cl[4];  // one 32-column fragment's scales and bias at a time
#pragma unroll
    for (int q = 0; q < 4; ++q) cl[q] = load_cols4(e, n0 + wn * TN + a * 32 + 8 * q + 4 * fhalf);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = wn * TN + a * 32 + 8 * q + 4 * fhalf;  // column within the tile
#pragma unroll
      for (int b = 0; b < FB; ++b) {
        const int r = wm * TM + b * 32 + frow;             // row within the tile
        uint32_t h[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = (float)acc[a][b][4 * q + i];
          v = v * sam[b];
          v = v * cl[q].sb[i];
          if (e.bias_dtype != I8L_DTYPE_NONE) v = v + cl[q].bias[i];
          h[i] = bf ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
        }
        *(uint2*)(lds + r * PITCH + 2 * c) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
      }
    }
  }
  lds_barrier();
  constexpr int CPR = BN / 8;                  // 16-byte chunks per output row
  static_assert((BM * CPR) % T == 0, "tile rows do not split over the threads");
#pragma unroll
  for (int j = 0; j < BM * CPR / T; ++j) {
    const int i = tid + j * T;
    const int r = i / CPR, c8 = i % CPR;
    const int64_t m = m0 + r;
    const uint4 v = *(const uint4*)(lds + r * PITCH + 16 * c8);
    if (m < e.M) *(uint4*)((uint16_t*)e.out + m * e.ldc + n0 + 8 * c8) = v;
  }
}

// ------------------------------------------------------------------ dynamic-quant decode
// gemm_wlds1 with the per-token activation quantizer folded in, for one 16-token row block.
// A arrives as the bf16/fp16 X [M, K] that quant_per_token would quantize; each wave
// quantizes its own K slice of the block's valid rows, with each row's absmax combined
// across the lanes holding it and then across the waves.  The arithmetic is the quantizer
// kernel's (absmax of |x|, scale = absmax/127, codes = rint(x * 127/absmax) clamped to
// [-128, 127]; reference fused_quant.py:41-53), so the output equals quant_per_token followed
// by w8a8_mm bit for bit, from one kernel instead of two.
//
// Every column tile repeats the row work, so the layout keeps it proportional to the valid
// rows: a wave reads its slice as 16-byte chunks of 8 values, CH = S/8 chunks a row and
// 64/CH rows a pass over the lanes, quantizes them, and writes the codes to an LDS tile of
// 16 rows x S bytes, from which the MFMA fragments are read (rows past M read as zero).
template <int NC, int KS, int W, int P, int EK, int DT>
__global__ void __launch_bounds__(64 * W)
gemm_wlds1_dq(const uint16_t* __restrict__ X, int64_t ldx, const int8_t* __restrict__ B,
              int64_t ldb, Epi e, float* __restrict__ sa_out, int precise) {
  constexpr int S = 64 * KS;
  constexpr int CPR = S / 16;
  constexpr int CPR_LOW = CPR & -CPR;
  constexpr int SWM = (CPR_LOW < 16 ? CPR_LOW : 16) - 1;
  static_assert(CPR % (SWM + 1) == 0, "the swizzle must permute the row's chunks");
  constexpr int SB = NC * S;
  constexpr int NI = SB / 1024;
  static_assert(NI * 1024 == SB, "a step must be whole 1 KiB DMA instructions");
  constexpr int NCF = NC < 16 ? NC : 16;
  constexpr int NF = NC / NCF;
  static_assert(NF * NCF == NC, "the tile must be whole column fragments");
  static_assert(NF <= W, "every fragment needs a storing wave");
  constexpr int CH = S / 8;                  // 8-value chunks of a row in a wave's slice
  constexpr int RPP = 64 / CH;               // rows a pass covers
  static_assert(RPP * CH == 64 && 16 % RPP == 0, "rows must split over the lanes");
  static_assert(P >= 1 && P * RPP <= 16, "P passes of RPP rows cover the block's valid rows");
  extern __shared__ __attribute__((aligned(16))) int8_t lds[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, grp = lane >> 4;
  const int64_t n0 = xcd_col_tile() * NC;
  const int64_t m0 = (int64_t)blockIdx.y * 16;
  // valid rows of the block; the host picks P = ceil(mb / RPP), so every pass is needed and
  // the code has no skipped (taken-branch) passes
  const int mb = (int)min((int64_t)16, (int64_t)e.M - m0);
  const int64_t kw = (int64_t)wave * S;
  int8_t* wbuf = lds + (size_t)wave * SB;
  v4i* red = (v4i*)(lds + (size_t)W * SB);                          // [W][NF][64]
  float* rmax = (float*)(lds + (size_t)W * SB + (size_t)W * NF * 1024);  // [W][16]
  float* scl = rmax + W * 16;               // [W][16]: each wave's copy of the row scales
  int8_t* abuf = lds + (size_t)W * SB + (size_t)W * NF * 1024 + (size_t)W * 128 + wave * 16 * S;

  // The activations are requested first and waited for alone: the quantizer work below
  // then runs while the weights' DMA is still in flight.
  // pass p: lane l holds chunk l % CH of row p*RPP + l/CH (rows past M are not read)
  const int crow = lane / CH, cchunk = lane % CH;
  uint4 xr[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    xr[p] = uint4{0, 0, 0, 0};
    const int r = p * RPP + crow;
    if (r < mb) xr[p] = *(const uint4*)(X + (m0 + r) * ldx + kw + 8 * cchunk);
  }
  __builtin_amdgcn_sched_barrier(0);
  const int8_t* Bw = B + n0 * ldb + kw;
  const int ldb32 = (int)ldb;
  lds_i8_t* dst = (lds_i8_t*)wbuf;
#pragma unroll
  for (int t = 0; t < NI; ++t) {
    const int o = t * 1024 + 16 * lane;
    const int r = o / S, c = ((o % S) / 16) ^ (r & SWM);
    __builtin_amdgcn_global_load_lds((const void*)(Bw + (r * ldb32 + 16 * c)), dst + t * 1024,
                                     16, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  wait_vmcnt_wlds<NI>();  // vector loads complete in issue order: the activations are in

  auto elem = [&](const uint4& v, int k) -> float {
    const uint32_t w32 = k < 4 ? (k < 2 ? v.x : v.y) : (k < 6 ? v.z : v.w);
    return act_to_f32<DT>((k & 1) ? (w32 >> 16) : (w32 & 0xffffu));
  };
  // absmax of each valid row's slice: a lane's chunk, then the CH lanes of the row
#pragma unroll
  for (int p = 0; p < P; ++p) {
    float am = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) am = fmaxf(am, fabsf(elem(xr[p], k)));
    am = group_max<CH>(am);
    if (cchunk == 0) rmax[wave * 16 + p * RPP + crow] = am;
  }
  __syncthreads();
  auto row_scale = [&](int r, float& scale, float& inv) {
    float absmax = rmax[r];
#pragma unroll
    for (int w = 1; w < W; ++w) absmax = fmaxf(absmax, rmax[w * 16 + r]);
    const float s_div = absmax / 127.0f;
    const float i_div = absmax == 0.0f ? 0.0f : 127.0f / absmax;
    const float s_rcp = absmax * (1.0f / 127.0f);
    const float i_rcp = absmax == 0.0f ? 0.0f : 127.0f * (1.0f / absmax);
    scale = precise ? s_div : s_rcp;
    inv = precise ? i_div : i_rcp;
  };
  // codes of each valid chunk into the wave's LDS tile (row pitch S bytes)
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int r = p * RPP + crow;
    if (r < mb) {
      float scale, inv;
      row_scale(r, scale, inv);
      uint32_t word[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        uint32_t packed = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          float v = __builtin_rintf(elem(xr[p], 4 * q + b) * inv);
          v = fminf(fmaxf(v, -128.0f), 127.0f);
          packed |= ((uint32_t)(int)v & 0xffu) << (8 * b);
        }
        word[q] = packed;
      }
      *(uint2*)(abuf + r * S + 8 * cchunk) = make_uint2(word[0], word[1]);
      if (cchunk == 0) {
        scl[wave * 16 + r] = scale;
        if (sa_out != nullptr && blockIdx.x == 0 && wave == 0) sa_out[m0 + r] = scale;
      }
    }
  }
  Cols4 cl;
  const int64_t mrow = m0 + r16;
  const int64_t ncol = n0 + NCF * (wave % NF) + 4 * (grp & (NCF / 4 - 1));
  if (wave < NF) cl = load_cols4<EK>(e, ncol);
  wait_vmcnt_wlds<0>();  // the weights, and the epilogue operands
  // the wave's own LDS writes are complete before its reads below (LDS is in order per wave)
  v4i a[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    a[s] = r16 < mb ? *(const v4i*)(abuf + r16 * S + 64 * s + 16 * grp) : v4i{0, 0, 0, 0};

  v4i b[KS][NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const int br = NCF * f + r16 % NCF;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      b[s][f] = *(const v4i*)(wbuf + br * S + 16 * ((4 * s + grp) ^ (br & SWM)));
  }
  v4i acc[NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) acc[f] = v4i{0, 0, 0, 0};
#pragma unroll
  for (int s = 0; s < KS; ++s)
#pragma unroll
    for (int f = 0; f < NF; ++f)
      acc[f] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b[s][f], a[s], acc[f], 0, 0, 0);

#pragma unroll
  for (int f = 0; f < NF; ++f) red[(wave * NF + f) * 64 + lane] = acc[f];
  __syncthreads();
  if (wave < NF) {
    v4i sum = red[wave * 64 + lane];
#pragma unroll
    for (int w = 1; w < W; ++w) sum += red[(w * NF + wave) * 64 + lane];
    // this wave's own scale of row r16 (written above by this wave: LDS is in order)
    if (r16 < mb && 4 * grp < NCF) store4s<EK>(e, mrow, ncol, sum, cl, scl[wave * 16 + r16]);
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

// Tile order: GROUP_M rows of tiles are walked together so that concurrently running
// workgroups share A rows and B columns in L2, and consecutive positions of that order are
// given to the same XCD (the dispatcher deals workgroups to the 8 XCDs round-robin).
__device__ __forceinline__ void staged_tile(int pid, int npid, int num_pid_m, int num_pid_n,
                                            int group_m, int& pid_m, int& pid_n) {
  if (npid % 8 == 0) pid = (pid % 8) * (npid / 8) + pid / 8;
  const int in_group = group_m * num_pid_n;
  const int first_m = (pid / in_group) * group_m;
  const int gsize = min(num_pid_m - first_m, group_m);
  pid_m = first_m + (pid % in_group) % gsize;
  pid_n = (pid % in_group) / gsize;
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
  constexpr int KK = BK / 32;                // MFMA K substeps per stage
  constexpr int STAGE = (BM + BN) * BK;
  constexpr int RSTEP = T / NCH;             // tile rows between a thread's chunks
  static_assert(RSTEP % 32 == 0, "row step must keep the swizzle");

  extern __shared__ __attribute__((aligned(16))) int8_t lds[];

  const int num_pid_m = (e.M + BM - 1) / BM;
  const int num_pid_n = e.N / BN;
  int pid_m, pid_n;
  staged_tile(blockIdx.x, gridDim.x, num_pid_m, num_pid_n, group_m, pid_m, pid_n);
  const int64_t m0 = (int64_t)pid_m * BM, n0 = (int64_t)pid_n * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // Global -> register staging: chunk j of this thread is tile row row0 + j*RSTEP, 16-byte
  // column chunk ch; all chunks of a thread share one swizzle.  Token rows past M read row
  // M-1 (valid memory; those output rows are never stored).
  const int row0 = tid / NCH, ch = tid % NCH;
  const int lofs = row0 * BK + ((ch ^ swz<BK>(row0)) * 16);
  const int8_t* ga[CA];
#pragma unroll
  for (int j = 0; j < CA; ++j) {
    const int64_t m = min(m0 + row0 + j * RSTEP, (int64_t)e.M - 1);
    ga[j] = A + m * lda + ch * 16;
  }
  const int8_t* gb = B + (n0 + row0) * ldb + ch * 16;

  v16i acc[FA][FB];
#pragma unroll
  for (int a = 0; a < FA; ++a)
#pragma unroll
    for (int b = 0; b < FB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0;

  // Two register sets hold the next two K tiles: the loads of tile t+2 are issued when
  // tile t's MFMAs start and stored to LDS one tile later, so two tiles of MFMA work cover
  // their latency.  Loads past the last tile re-read it (clamped offset): every load is
  // unconditional, so the wait before each LDS store covers exactly the older set.
  v4i ra0[CA], rb0[CB], ra1[CA], rb1[CB];
  const int KT = K / BK;
  auto gload = [&](v4i (&ra)[CA], v4i (&rb)[CB], int t) {
    const int64_t k0 = (int64_t)min(t, KT - 1) * BK;
#pragma unroll
    for (int j = 0; j < CB; ++j) rb[j] = ld16(gb + (int64_t)j * RSTEP * ldb + k0);
#pragma unroll
    for (int j = 0; j < CA; ++j) ra[j] = ld16(ga[j] + k0);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto lstore = [&](const v4i (&ra)[CA], const v4i (&rb)[CB], int buf) {
    int8_t* base = lds + buf * STAGE + lofs;
#pragma unroll
    for (int j = 0; j < CA; ++j) *(v4i*)(base + j * RSTEP * BK) = ra[j];
#pragma unroll
    for (int j = 0; j < CB; ++j) *(v4i*)(base + BM * BK + j * RSTEP * BK) = rb[j];
  };

  // Fragment reads: lane l reads row (l%32) of a 32-row block, 16-byte chunk 2*kk + l/32;
  // the swizzle depends on the row only through l%32 (blocks are 32 rows apart).
  const int frow = lane & 31, fhalf = lane >> 5;
  int fofs[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) fofs[kk] = frow * BK + (((2 * kk + fhalf) ^ swz<BK>(frow)) * 16);
  const int a_row = BM * BK + wn * TN * BK;  // weight rows of this wave
  const int b_row = wm * TM * BK;            // token rows of this wave

  v4i fa[2][FA], fb[2][FB];
  auto fread = [&](const int8_t* base, int kk, int p) {
#pragma unroll
    for (int a = 0; a < FA; ++a) fa[p][a] = *(const v4i*)(base + a_row + a * 32 * BK + fofs[kk]);
#pragma unroll
    for (int b = 0; b < FB; ++b) fb[p][b] = *(const v4i*)(base + b_row + b * 32 * BK + fofs[kk]);
  };
  auto compute = [&](int buf) {
    const int8_t* base = lds + buf * STAGE;
    fread(base, 0, 0);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if (kk + 1 < KK) fread(base, kk + 1, (kk + 1) & 1);
      __builtin_amdgcn_sched_barrier(0);  // next substep's reads go out before these MFMAs
#pragma unroll
      for (int a = 0; a < FA; ++a)
#pragma unroll
        for (int b = 0; b < FB; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[kk & 1][a], fb[kk & 1][b],
                                                            acc[a][b], 0, 0, 0);
    }
  };

  gload(ra0, rb0, 0);
  gload(ra1, rb1, 1);
  lstore(ra0, rb0, 0);
  __syncthreads();
  int t = 0;
  for (; t + 1 < KT; t += 2) {
    gload(ra0, rb0, t + 2);      // set 0 is free: tile t is already in LDS buffer 0
    compute(0);                  // tile t
    lstore(ra1, rb1, 1);         // tile t+1
    __syncthreads();
    gload(ra1, rb1, t + 3);
    compute(1);                  // tile t+1
    lstore(ra0, rb0, 0);         // tile t+2 (a re-read of the last tile past the end)
    __syncthreads();
  }
  if (t < KT) compute(0);        // odd tile count: the last tile sits in buffer 0
  lds_barrier();
  tile_epilogue<BM, BN, WM, WN, FA, FB>(e, acc, lds, m0, n0, wm, wn, lane, tid);
}

// ------------------------------------------------------------------ dma schedule
// The staged schedule's tiles and MFMA work, with K tiles moved from global memory to LDS
// by global_load_lds_dwordx4 (no register staging, no LDS store instructions) through a
// ring of S buffers: tile t+S-1 is requested while tile t is multiplied.  Each wave
// instruction writes 1 KiB of LDS (lane i at +16*i), so 16-byte unit u of a stage lands at
// byte 16*u, which is row u/NCH, slot u%NCH of the swizzled layout; each lane fetches the
// global chunk (slot ^ swz(row)) that belongs in its unit.
//
// Synchronisation is explicit: before tile t is read, each wave waits until only the DMA
// requests of the S-2 later tiles are outstanding (vmcnt), then the workgroup barrier
// makes every wave's requests for tile t complete; the barrier also guarantees that all
// waves have finished reading the buffer that the next request overwrites.  Requests past
// the last tile re-read it (clamped), so every iteration issues the same number and the
// wait count is a constant.
typedef __attribute__((address_space(3))) int8_t lds_i8;


// s_waitcnt with vmcnt = N and the LGKM / EXP counters left unconstrained (gfx9 encoding:
// vmcnt[3:0] in bits 3:0 and vmcnt[5:4] in bits 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int BM, int BN, int BK, int WM, int WN, int S>
__global__ void __launch_bounds__(64 * WM * WN)
gemm_dma(const int8_t* __restrict__ A, int64_t lda, const int8_t* __restrict__ B,
         int64_t ldb, Epi e, int K, int group_m) {
  constexpr int W = WM * WN;
  constexpr int T = 64 * W;
  constexpr int NCH = BK / 16;
  constexpr int UNITS = (BM + BN) * NCH;   // 16-byte units per stage
  constexpr int J = UNITS / T;             // DMA instructions per thread per stage
  static_assert(J * T == UNITS, "stage does not split over the waves");
  static_assert(BM % (64 / NCH) == 0, "one DMA instruction must stay within A or B rows");
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FB = TM / 32, FA = TN / 32;
  constexpr int KK = BK / 32;
  constexpr int STAGE = (BM + BN) * BK;
  static_assert(S >= 3, "the ring needs at least three buffers");

  extern __shared__ __attribute__((aligned(16))) int8_t lds[];

  const int num_pid_m = (e.M + BM - 1) / BM;
  const int num_pid_n = e.N / BN;
  int pid_m, pid_n;
  staged_tile(blockIdx.x, gridDim.x, num_pid_m, num_pid_n, group_m, pid_m, pid_n);
  const int64_t m0 = (int64_t)pid_m * BM, n0 = (int64_t)pid_n * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // Global source of each of this lane's J units (token rows past M read row M-1).
  const int8_t* gp[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int u = (j * W + wave) * 64 + lane;
    const int row = u / NCH, chunk = (u % NCH) ^ swz<BK>(row);
    gp[j] = row < BM ? A + min(m0 + row, (int64_t)e.M - 1) * lda + chunk * 16
                     : B + (n0 + row - BM) * ldb + chunk * 16;
  }
  const int KT = K / BK;
  auto dma = [&](int t) {
    const int64_t k0 = (int64_t)min(t, KT - 1) * BK;
    lds_i8* dst = (lds_i8*)(lds + (t % S) * STAGE + wave * 1024);
#pragma unroll
    for (int j = 0; j < J; ++j)
      __builtin_amdgcn_global_load_lds((const void*)(gp[j] + k0), dst + j * W * 1024, 16, 0, 0);
  };

  v16i acc[FA][FB];
#pragma unroll
  for (int a = 0; a < FA; ++a)
#pragma unroll
    for (int b = 0; b < FB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0;

  const int frow = lane & 31, fhalf = lane >> 5;
  int fofs[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) fofs[kk] = frow * BK + (((2 * kk + fhalf) ^ swz<BK>(frow)) * 16);
  const int a_row = BM * BK + wn * TN * BK;
  const int b_row = wm * TM * BK;
  v4i fa[2][FA], fb[2][FB];
  auto fread = [&](const int8_t* base, int kk, int p) {
#pragma unroll
    for (int a = 0; a < FA; ++a) fa[p][a] = *(const v4i*)(base + a_row + a * 32 * BK + fofs[kk]);
#pragma unroll
    for (int b = 0; b < FB; ++b) fb[p][b] = *(const v4i*)(base + b_row + b * 32 * BK + fofs[kk]);
  };

#pragma unroll
  for (int t = 0; t < S - 1; ++t) dma(t);
  for (int t = 0; t < KT; ++t) {
    wait_vmcnt<J * (S - 2)>();
    lds_barrier();
    dma(t + S - 1);
    const int8_t* base = lds + (t % S) * STAGE;
    fread(base, 0, 0);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if (kk + 1 < KK) fread(base, kk + 1, (kk + 1) & 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int a = 0; a < FA; ++a)
#pragma unroll
        for (int b = 0; b < FB; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[kk & 1][a], fb[kk & 1][b],
                                                            acc[a][b], 0, 0, 0);
    }
  }
  // No DMA may still be writing this workgroup's LDS when it is reused or retires.
  wait_vmcnt<0>();
  lds_barrier();
  tile_epilogue<BM, BN, WM, WN, FA, FB>(e, acc, lds, m0, n0, wm, wn, lane, tid);
}

// ------------------------------------------------------------------ pipelined dma schedule
// The dma schedule with the LDS fragment reads overlapped with the MFMAs.  A K step of BK
// bytes is KK = BK/32 MFMA substeps; substep kk's MFMAs are issued one after another with the
// reads of the next substep's fragments between them (one read after each MFMA), from two
// register sets of one substep each.  Before the last substep of step t, each wave waits for
// its DMA of step t+1 (vmcnt), the workgroup barrier makes step t+1 visible and frees the
// buffer of step t-1 (whose last reads fed MFMAs before the barrier), and step t+S-1 is
// requested into it; the last substep's MFMAs then overlap the reads of step t+1's first
// substep.  The LDS traffic of each substep hides under the matrix work of the one before.
template <int BM, int BN, int BK, int WM, int WN, int S>
__global__ void __launch_bounds__(64 * WM * WN)
gemm_dmap(const int8_t* __restrict__ A, int64_t lda, const int8_t* __restrict__ B,
          int64_t ldb, Epi e, int K, int group_m) {
  constexpr int W = WM * WN;
  constexpr int T = 64 * W;
  constexpr int NCH = BK / 16;
  constexpr int UNITS = (BM + BN) * NCH;
  constexpr int J = UNITS / T;
  static_assert(J * T == UNITS, "stage does not split over the waves");
  static_assert(BM % (64 / NCH) == 0, "one DMA instruction must stay within A or B rows");
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FB = TM / 32, FA = TN / 32;
  constexpr int KK = BK / 32;
  constexpr int STAGE = (BM + BN) * BK;
  constexpr int NM = FA * FB;                // MFMAs per substep
  constexpr int NR = FA + FB;                // fragment reads per substep
  static_assert(S >= 3, "the ring needs at least three buffers");

  extern __shared__ __attribute__((aligned(16))) int8_t lds[];

  const int num_pid_m = (e.M + BM - 1) / BM;
  const int num_pid_n = e.N / BN;
  int pid_m, pid_n;
  staged_tile(blockIdx.x, gridDim.x, num_pid_m, num_pid_n, group_m, pid_m, pid_n);
  const int64_t m0 = (int64_t)pid_m * BM, n0 = (int64_t)pid_n * BN;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;

  const int8_t* gp[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int u = (j * W + wave) * 64 + lane;
    const int row = u / NCH, chunk = (u % NCH) ^ swz<BK>(row);
    gp[j] = row < BM ? A + min(m0 + row, (int64_t)e.M - 1) * lda + chunk * 16
                     : B + (n0 + row - BM) * ldb + chunk * 16;
  }
  const int KT = K / BK;
  auto dma = [&](int t) {
    const int64_t k0 = (int64_t)min(t, KT - 1) * BK;
    lds_i8* dst = (lds_i8*)(lds + (t % S) * STAGE + wave * 1024);
#pragma unroll
    for (int j = 0; j < J; ++j)
      __builtin_amdgcn_global_load_lds((const void*)(gp[j] + k0), dst + j * W * 1024, 16, 0, 0);
  };

  v16i acc[FA][FB];
#pragma unroll
  for (int a = 0; a < FA; ++a)
#pragma unroll
    for (int b = 0; b < FB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0;

  const int frow = lane & 31, fhalf = lane >> 5;
  int fofs[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) fofs[kk] = frow * BK + (((2 * kk + fhalf) ^ swz<BK>(frow)) * 16);
  const int a_row = BM * BK + wn * TN * BK;
  const int b_row = wm * TM * BK;

  v4i f0a[FA], f0b[FB], f1a[FA], f1b[FB];
  auto rd = [&](v4i (&fa)[FA], v4i (&fb)[FB], int t, int kk) {
    const int8_t* base = lds + (t % S) * STAGE;
#pragma unroll
    for (int a = 0; a < FA; ++a) fa[a] = *(const v4i*)(base + a_row + a * 32 * BK + fofs[kk]);
#pragma unroll
    for (int b = 0; b < FB; ++b) fb[b] = *(const v4i*)(base + b_row + b * 32 * BK + fofs[kk]);
  };
  auto mm = [&](const v4i (&fa)[FA], const v4i (&fb)[FB]) {
#pragma unroll
    for (int a = 0; a < FA; ++a)
#pragma unroll
      for (int b = 0; b < FB; ++b)
        acc[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[a], fb[b], acc[a][b], 0, 0, 0);
  };
  // one substep: its MFMAs with the next substep's reads between them
  auto overlap = [&](const v4i (&ca)[FA], const v4i (&cb)[FB], v4i (&na)[FA], v4i (&nb)[FB],
                     int t, int kk) {
    __builtin_amdgcn_sched_barrier(0);
    rd(na, nb, t, kk);
    mm(ca, cb);
    constexpr int P = NR < NM ? NR : NM;
#pragma unroll
    for (int i = 0; i < P; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // one LDS read
    }
    if (NM > P) __builtin_amdgcn_sched_group_barrier(0x008, NM - P, 0);
    if (NR > P) __builtin_amdgcn_sched_group_barrier(0x100, NR - P, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  // Steps requested before the wait in step t: 0 .. t+S-2; step t+1 must be complete.
  auto turn = [&](int t) {
    wait_vmcnt<J * (S - 3)>();
    lds_barrier();
    dma(t + S - 1);
  };
  // One K step from fragment set 0 (holding substep 0); leaves step t+1's substep 0 in set 0
  // when `more`.  KK is even, so the substeps alternate 0,1,0,1,... and end in set 1.
  auto kstep = [&](int t, bool more) {
#pragma unroll
    for (int kk = 0; kk + 1 < KK; ++kk) {
      if (kk % 2 == 0) overlap(f0a, f0b, f1a, f1b, t, kk + 1);
      else overlap(f1a, f1b, f0a, f0b, t, kk + 1);
    }
    if (more) {
      turn(t);
      overlap(f1a, f1b, f0a, f0b, t + 1, 0);
    } else {
      mm(f1a, f1b);
    }
  };
  static_assert(KK % 2 == 0, "substeps alternate between the two fragment sets");

#pragma unroll
  for (int t = 0; t < S - 1; ++t) dma(t);
  wait_vmcnt<J * (S - 2)>();
  lds_barrier();
  rd(f0a, f0b, 0, 0);
  for (int t = 0; t + 1 < KT; ++t) kstep(t, true);
  kstep(KT - 1, false);
  wait_vmcnt<0>();
  lds_barrier();
  tile_epilogue<BM, BN, WM, WN, FA, FB>(e, acc, lds, m0, n0, wm, wn, lane, tid);
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

// Opts a kernel in to `bytes` of dynamic LDS (needed above 64 KiB) on the current device,
// once per device; `done` is the kernel's set of devices already opted in.  An unsupported
// attribute is not fatal: the launch itself then reports the LDS overrun.
void lds_opt_in(const void* kern, size_t bytes, std::atomic<uint64_t>& done) {
  if (bytes <= 64 * 1024) return;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    dev = -1;
  }
  const uint64_t bit = dev >= 0 && dev < 64 ? 1ull << dev : 0;
  if (bit && (done.load(std::memory_order_relaxed) & bit)) return;
  (void)hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  (void)hipGetLastError();
  if (bit) done.fetch_or(bit, std::memory_order_relaxed);
}

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
// (BM, BN, BK, WM, WN); the waves of a workgroup are laid out WM (tokens) x WN (columns).
// (256x256 tiles with 4 waves, or with 128-byte K steps, spill the register file and are
// not built.)
constexpr StagedTile kStaged[] = {{128, 128, 64, 2, 2},  {256, 128, 64, 2, 2},
                                  {128, 256, 64, 2, 2},  {128, 128, 128, 2, 2},
                                  {256, 256, 64, 2, 4},  {256, 128, 64, 2, 4},
                                  {128, 256, 64, 2, 4},  {256, 128, 128, 2, 4},
                                  {128, 256, 128, 2, 4}};

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

struct DmaTile {
  int bm, bn, bk, wm, wn, s;
};
// (BM, BN, BK, WM, WN, ring depth S); the config's `stages` field is S.
constexpr DmaTile kDma[] = {{256, 256, 64, 2, 4, 3}, {256, 256, 64, 2, 4, 4},
                            {256, 128, 64, 2, 4, 4}, {128, 256, 64, 2, 4, 4},
                            {256, 128, 128, 2, 4, 3}, {128, 256, 128, 2, 4, 3},
                            {128, 128, 128, 2, 2, 4}, {128, 128, 64, 2, 2, 4},
                            {256, 256, 64, 2, 4, 5}, {256, 128, 64, 2, 4, 6},
                            {128, 256, 64, 2, 4, 6}, {128, 128, 64, 2, 2, 8}};

// Weights-through-LDS decode tiles (MT, NC, KS): bm = 16*MT, bn = NC, bk = 64*KS bytes of K
// per wave step; the config's `stages` is 3 and K must split into warps x steps x bk.
struct WldsTile {
  int mt, nc, ks;
};
constexpr WldsTile kWlds[] = {{1, 16, 2}, {1, 16, 4}, {1, 16, 6}, {1, 16, 8}, {1, 8, 2},
                              {1, 8, 4},  {1, 8, 6},  {1, 8, 8},  {1, 4, 4},  {1, 4, 8},
                              {2, 16, 2}, {2, 16, 4}, {2, 8, 2},  {2, 8, 4},  {4, 16, 2},
                              {4, 16, 4}, {4, 8, 2},  {4, 8, 4},  {8, 16, 2}, {8, 8, 2},
                              {1, 32, 2}, {1, 32, 4}, {2, 32, 2}, {2, 32, 4}, {4, 32, 2},
                              {4, 32, 4}};
constexpr size_t kMaxLds = 160 * 1024;

size_t wlds_lds_bytes(const i8l_config& c, int64_t K) {
  const int64_t steps = K / ((int64_t)c.bk * c.warps);
  const int nbuf = steps > 1 ? 2 : 1;
  const int nf = c.bn > 16 ? c.bn / 16 : 1;  // 16-column fragments a wave reduces
  return (size_t)c.warps * nbuf * c.bn * c.bk + (size_t)c.warps * (c.bm / 16) * nf * 1024;
}

bool wlds1_built(int mt, int nc, int W, int ks);

bool wlds_ok(const i8l_config& c, int64_t K) {
  if (c.stages != 3 || c.split_k != 1 || c.bn > 32 || c.warps < 1 || c.warps > 16) return false;
  bool built = false;
  for (auto t : kWlds)
    if (16 * t.mt == c.bm && t.nc == c.bn && 64 * t.ks == c.bk &&
        c.warps * 64 <= wlds_bound(t.mt, t.ks))
      built = true;
  if (!built || K <= 0 || K % ((int64_t)c.bk * c.warps)) return false;
  const bool one_step = K == (int64_t)c.bk * c.warps &&
                        wlds1_built(c.bm / 16, c.bn, c.warps, c.bk / 64);
  if (!one_step && !wlds_multi_fits(c.bm / 16, c.bn, c.bk / 64)) return false;
  return wlds_lds_bytes(c, K) <= kMaxLds;
}

// Direct-to-LDS tiles with the fragment reads overlapped with the MFMAs (gemm_dmap): the
// config's `stages` is the ring depth S plus 8.
constexpr DmaTile kDmap[] = {{256, 256, 64, 2, 4, 3}, {256, 256, 64, 2, 4, 4},
                             {256, 256, 64, 2, 4, 5}, {256, 128, 64, 2, 4, 4},
                             {128, 256, 64, 2, 4, 4}, {128, 256, 128, 2, 4, 3},
                             {256, 128, 128, 2, 4, 3}, {128, 128, 64, 2, 2, 4},
                             {128, 128, 128, 2, 2, 4}, {64, 128, 128, 2, 2, 4},
                             {64, 256, 128, 2, 4, 3}, {64, 128, 64, 2, 2, 6},
                             {64, 128, 128, 2, 2, 6}, {64, 64, 128, 2, 2, 4},
                             {128, 64, 128, 2, 2, 4}};
constexpr int kPipelined = 8;

int dmap_index(const i8l_config& c) {
  if (c.stages < 3 + kPipelined || c.split_k != 1 || c.group_m < 1) return -1;
  for (int i = 0; i < (int)(sizeof(kDmap) / sizeof(kDmap[0])); ++i) {
    const auto& t = kDmap[i];
    if (t.bm == c.bm && t.bn == c.bn && t.bk == c.bk && t.wm * t.wn == c.warps &&
        t.s + kPipelined == c.stages)
      return i;
  }
  return -1;
}

int dma_index(const i8l_config& c) {
  if (c.stages < 3 || c.split_k != 1 || c.group_m < 1) return -1;
  for (int i = 0; i < (int)(sizeof(kDma) / sizeof(kDma[0])); ++i) {
    const auto& t = kDma[i];
    if (t.bm == c.bm && t.bn == c.bn && t.bk == c.bk && t.wm * t.wn == c.warps && t.s == c.stages)
      return i;
  }
  return -1;
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

template <int MT, int NC, int KS, int EK>
hipError_t launch_wlds_k(const i8l_config& c, const int8_t* a, int64_t lda, const int8_t* b,
                         int64_t ldb, const Epi& e, int64_t K, hipStream_t st) {
  auto kern = gemm_wlds<MT, NC, KS, EK>;
  const size_t shm = wlds_lds_bytes(c, K);
  static std::atomic<uint64_t> lds_done{0};  // devices this kernel is opted in on
  lds_opt_in((const void*)kern, kMaxLds, lds_done);
  const int steps = (int)(K / ((int64_t)c.bk * c.warps));
  const dim3 grid(e.N / NC, (e.M + 16 * MT - 1) / (16 * MT));
  hipLaunchKernelGGL(kern, grid, dim3(64 * c.warps), shm, st, a, lda, b, ldb, e, steps,
                     steps > 1 ? 2 : 1);
  return hipGetLastError();
}

template <int MT, int NC, int KS, int W, int EK>
hipError_t launch_wlds1_k(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                          const Epi& e, hipStream_t st) {
  auto kern = gemm_wlds1<MT, NC, KS, W, EK>;
  const size_t shm = (size_t)W * NC * 64 * KS + (size_t)W * MT * (NC > 16 ? NC / 16 : 1) * 1024;
  static std::atomic<uint64_t> lds_done{0};  // devices this kernel is opted in on
  lds_opt_in((const void*)kern, shm, lds_done);
  const dim3 grid(e.N / NC, (e.M + 16 * MT - 1) / (16 * MT));
  hipLaunchKernelGGL(kern, grid, dim3(64 * W), shm, st, a, lda, b, ldb, e);
  return hipGetLastError();
}

// Single-step launches for the (waves, step) pairs built: K = 64 * KS * W.
template <int MT, int NC, int KS, int EK>
hipError_t launch_wlds1_w(int W, const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                          const Epi& e, hipStream_t st) {
  constexpr int FR = MT * (NC > 16 ? NC / 16 : 1);  // fragments: one storing wave each
  if constexpr (KS <= 8) {
    if constexpr (FR <= 4)
      if (W == 4 && (KS == 4 || KS == 8)) return launch_wlds1_k<MT, NC, KS, 4, EK>(a, lda, b, ldb, e, st);
    if constexpr (FR <= 8)
      if (W == 8) return launch_wlds1_k<MT, NC, KS, 8, EK>(a, lda, b, ldb, e, st);
    if constexpr (wlds_bound(MT, KS) >= 1024 && KS <= 6)
      if (W == 16) return launch_wlds1_k<MT, NC, KS, 16, EK>(a, lda, b, ldb, e, st);
  }
  return hipErrorInvalidValue;
}

bool wlds1_built(int mt, int nc, int W, int ks) {
  const int fr = mt * (nc > 16 ? nc / 16 : 1);
  return ks <= 8 && ((W == 4 && fr <= 4 && (ks == 4 || ks == 8)) || (W == 8 && fr <= 8) ||
                     (W == 16 && ks <= 6 && wlds_bound(mt, ks) >= 1024));
}

template <int MT, int NC, int KS>
hipError_t launch_wlds_t(const i8l_config& c, const int8_t* a, int64_t lda, const int8_t* b,
                         int64_t ldb, const Epi& e, int64_t K, hipStream_t st) {
  if (K == (int64_t)c.bk * c.warps && wlds1_built(MT, NC, c.warps, KS)) {
    switch (epi_kind(e)) {
      case EK_BF16: return launch_wlds1_w<MT, NC, KS, EK_BF16>(c.warps, a, lda, b, ldb, e, st);
      case EK_BF16_BBF16:
        return launch_wlds1_w<MT, NC, KS, EK_BF16_BBF16>(c.warps, a, lda, b, ldb, e, st);
      default: return launch_wlds1_w<MT, NC, KS, EK_ANY>(c.warps, a, lda, b, ldb, e, st);
    }
  }
  if constexpr (wlds_multi_fits(MT, NC, KS)) {
    switch (epi_kind(e)) {
      case EK_BF16: return launch_wlds_k<MT, NC, KS, EK_BF16>(c, a, lda, b, ldb, e, K, st);
      case EK_BF16_BBF16:
        return launch_wlds_k<MT, NC, KS, EK_BF16_BBF16>(c, a, lda, b, ldb, e, K, st);
      default: return launch_wlds_k<MT, NC, KS, EK_ANY>(c, a, lda, b, ldb, e, K, st);
    }
  }
  return hipErrorInvalidValue;
}

hipError_t launch_wlds(const i8l_config& c, const int8_t* a, int64_t lda, const int8_t* b,
                       int64_t ldb, const Epi& e, int64_t K, hipStream_t st) {
  const int mt = c.bm / 16, nc = c.bn, ks = c.bk / 64;
#define I8L_WLDS(MT_, NC_, KS_)                                                             \
  if (mt == MT_ && nc == NC_ && ks == KS_) return launch_wlds_t<MT_, NC_, KS_>(c, a, lda, b, ldb, e, K, st);
  I8L_WLDS(1, 16, 2) I8L_WLDS(1, 16, 4) I8L_WLDS(1, 16, 6) I8L_WLDS(1, 16, 8)
  I8L_WLDS(1, 8, 2) I8L_WLDS(1, 8, 4) I8L_WLDS(1, 8, 6) I8L_WLDS(1, 8, 8)
  I8L_WLDS(1, 4, 4) I8L_WLDS(1, 4, 8)
  I8L_WLDS(2, 16, 2) I8L_WLDS(2, 16, 4) I8L_WLDS(2, 8, 2) I8L_WLDS(2, 8, 4)
  I8L_WLDS(4, 16, 2) I8L_WLDS(4, 16, 4) I8L_WLDS(4, 8, 2) I8L_WLDS(4, 8, 4)
  I8L_WLDS(8, 16, 2) I8L_WLDS(8, 8, 2)
  I8L_WLDS(1, 32, 2) I8L_WLDS(1, 32, 4) I8L_WLDS(2, 32, 2) I8L_WLDS(2, 32, 4)
  I8L_WLDS(4, 32, 2) I8L_WLDS(4, 32, 4)
#undef I8L_WLDS
  return hipErrorInvalidValue;
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
  const size_t shm = std::max<size_t>(2 * (size_t)(BM + BN) * BK,
                                      tile_epilogue_lds_bytes<BM, BN, WM, WN>());
  static std::atomic<uint64_t> lds_done{0};  // devices this kernel is opted in on
  lds_opt_in((const void*)kern, shm, lds_done);
  const int tiles = ((e.M + BM - 1) / BM) * (e.N / BN);
  hipLaunchKernelGGL(kern, dim3(tiles), dim3(64 * WM * WN), shm, st, a, lda, b, ldb, e, K, group_m);
  return hipGetLastError();
}

template <int BM, int BN, int BK, int WM, int WN, int S>
hipError_t launch_dma_t(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                        const Epi& e, int K, int group_m, hipStream_t st) {
  auto kern = gemm_dma<BM, BN, BK, WM, WN, S>;
  const size_t shm = std::max<size_t>((size_t)S * (BM + BN) * BK,
                                      tile_epilogue_lds_bytes<BM, BN, WM, WN>());
  static std::atomic<uint64_t> lds_done{0};  // devices this kernel is opted in on
  lds_opt_in((const void*)kern, shm, lds_done);
  const int tiles = ((e.M + BM - 1) / BM) * (e.N / BN);
  hipLaunchKernelGGL(kern, dim3(tiles), dim3(64 * WM * WN), shm, st, a, lda, b, ldb, e, K, group_m);
  return hipGetLastError();
}

hipError_t launch_dma(int idx, const i8l_config& c, const int8_t* a, int64_t lda,
                      const int8_t* b, int64_t ldb, const Epi& e, int K, hipStream_t st) {
  switch (idx) {
    case 0: return launch_dma_t<256, 256, 64, 2, 4, 3>(a, lda, b, ldb, e, K, c.group_m, st);
    case 1: return launch_dma_t<256, 256, 64, 2, 4, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 2: return launch_dma_t<256, 128, 64, 2, 4, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 3: return launch_dma_t<128, 256, 64, 2, 4, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 4: return launch_dma_t<256, 128, 128, 2, 4, 3>(a, lda, b, ldb, e, K, c.group_m, st);
    case 5: return launch_dma_t<128, 256, 128, 2, 4, 3>(a, lda, b, ldb, e, K, c.group_m, st);
    case 6: return launch_dma_t<128, 128, 128, 2, 2, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 7: return launch_dma_t<128, 128, 64, 2, 2, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 8: return launch_dma_t<256, 256, 64, 2, 4, 5>(a, lda, b, ldb, e, K, c.group_m, st);
    case 9: return launch_dma_t<256, 128, 64, 2, 4, 6>(a, lda, b, ldb, e, K, c.group_m, st);
    case 10: return launch_dma_t<128, 256, 64, 2, 4, 6>(a, lda, b, ldb, e, K, c.group_m, st);
    case 11: return launch_dma_t<128, 128, 64, 2, 2, 8>(a, lda, b, ldb, e, K, c.group_m, st);
  }
  return hipErrorInvalidValue;
}

template <int BM, int BN, int BK, int WM, int WN, int S>
hipError_t launch_dmap_t(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                         const Epi& e, int K, int group_m, hipStream_t st) {
  auto kern = gemm_dmap<BM, BN, BK, WM, WN, S>;
  const size_t shm = std::max<size_t>((size_t)S * (BM + BN) * BK,
                                      tile_epilogue_lds_bytes<BM, BN, WM, WN>());
  static std::atomic<uint64_t> lds_done{0};  // devices this kernel is opted in on
  lds_opt_in((const void*)kern, shm, lds_done);
  const int tiles = ((e.M + BM - 1) / BM) * (e.N / BN);
  hipLaunchKernelGGL(kern, dim3(tiles), dim3(64 * WM * WN), shm, st, a, lda, b, ldb, e, K, group_m);
  return hipGetLastError();
}

hipError_t launch_dmap(int idx, const i8l_config& c, const int8_t* a, int64_t lda,
                       const int8_t* b, int64_t ldb, const Epi& e, int K, hipStream_t st) {
  switch (idx) {
    case 0: return launch_dmap_t<256, 256, 64, 2, 4, 3>(a, lda, b, ldb, e, K, c.group_m, st);
    case 1: return launch_dmap_t<256, 256, 64, 2, 4, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 2: return launch_dmap_t<256, 256, 64, 2, 4, 5>(a, lda, b, ldb, e, K, c.group_m, st);
    case 3: return launch_dmap_t<256, 128, 64, 2, 4, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 4: return launch_dmap_t<128, 256, 64, 2, 4, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 5: return launch_dmap_t<128, 256, 128, 2, 4, 3>(a, lda, b, ldb, e, K, c.group_m, st);
    case 6: return launch_dmap_t<256, 128, 128, 2, 4, 3>(a, lda, b, ldb, e, K, c.group_m, st);
    case 7: return launch_dmap_t<128, 128, 64, 2, 2, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 8: return launch_dmap_t<128, 128, 128, 2, 2, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 9: return launch_dmap_t<64, 128, 128, 2, 2, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 10: return launch_dmap_t<64, 256, 128, 2, 4, 3>(a, lda, b, ldb, e, K, c.group_m, st);
    case 11: return launch_dmap_t<64, 128, 64, 2, 2, 6>(a, lda, b, ldb, e, K, c.group_m, st);
    case 12: return launch_dmap_t<64, 128, 128, 2, 2, 6>(a, lda, b, ldb, e, K, c.group_m, st);
    case 13: return launch_dmap_t<64, 64, 128, 2, 2, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 14: return launch_dmap_t<128, 64, 128, 2, 2, 4>(a, lda, b, ldb, e, K, c.group_m, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_staged(int idx, const i8l_config& c, const int8_t* a, int64_t lda,
                         const int8_t* b, int64_t ldb, const Epi& e, int K, hipStream_t st) {
  switch (idx) {
    case 0: return launch_staged_t<128, 128, 64, 2, 2>(a, lda, b, ldb, e, K, c.group_m, st);
    case 1: return launch_staged_t<256, 128, 64, 2, 2>(a, lda, b, ldb, e, K, c.group_m, st);
    case 2: return launch_staged_t<128, 256, 64, 2, 2>(a, lda, b, ldb, e, K, c.group_m, st);
    case 3: return launch_staged_t<128, 128, 128, 2, 2>(a, lda, b, ldb, e, K, c.group_m, st);
    case 4: return launch_staged_t<256, 256, 64, 2, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 5: return launch_staged_t<256, 128, 64, 2, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 6: return launch_staged_t<128, 256, 64, 2, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 7: return launch_staged_t<256, 128, 128, 2, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 8: return launch_staged_t<128, 256, 128, 2, 4>(a, lda, b, ldb, e, K, c.group_m, st);
  }
  return hipErrorInvalidValue;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int elt_size(int dt) { return dt == I8L_BF16 || dt == I8L_F16 ? 2 : 4; }

// Dynamic-quant decode tiles (gemm_wlds1_dq, one 16-token row block): (NC, KS, W) with
// K == 64 * KS * W.  The config's bm is 16 and its stages 3, as for gemm_wlds1.
struct DqTile {
  int nc, ks, w;
};
constexpr DqTile kDq[] = {{8, 2, 16}, {16, 2, 16}, {32, 2, 16}, {8, 4, 16}, {16, 4, 16}};

size_t dq_lds_bytes(int nc, int ks, int W) {
  const int nf = nc > 16 ? nc / 16 : 1;
  // weights, the cross-wave sums, the row maxima and scales, the 16-row code tiles
  return (size_t)W * nc * 64 * ks + (size_t)W * nf * 1024 + (size_t)W * 128 +
         (size_t)W * 16 * 64 * ks;
}

bool dq_ok(const i8l_config& c, int64_t K) {
  if (c.stages != 3 || c.split_k != 1 || c.bm != 16) return false;
  for (auto t : kDq)
    if (t.nc == c.bn && 64 * t.ks == c.bk && t.w == c.warps)
      return K == (int64_t)64 * t.ks * t.w && dq_lds_bytes(t.nc, t.ks, t.w) <= kMaxLds;
  return false;
}

// The untuned choice: 16 waves that take K in one step each, 16 columns a workgroup (8 for
// narrow N).
bool default_dq_config(int64_t N, int64_t K, i8l_config* c) {
  const int nc = (N % 16 == 0 && N / 16 >= 256) ? 16 : 8;
  for (int ks : {2, 4}) {
    const i8l_config t{16, nc, 64 * ks, 16, 3, 1, 1};
    if (K == (int64_t)64 * ks * 16 && dq_ok(t, K)) {
      *c = t;
      return true;
    }
  }
  return false;
}

template <int NC, int KS, int W, int P, int EK, int DT>
hipError_t launch_dq_k(const uint16_t* x, int64_t ldx, const int8_t* b, int64_t ldb,
                       const Epi& e, float* sa_out, int precise, hipStream_t st) {
  auto kern = gemm_wlds1_dq<NC, KS, W, P, EK, DT>;
  const size_t shm = dq_lds_bytes(NC, KS, W);
  static std::atomic<uint64_t> lds_done{0};  // devices this kernel is opted in on
  lds_opt_in((const void*)kern, shm, lds_done);
  const dim3 grid(e.N / NC, (e.M + 15) / 16);
  hipLaunchKernelGGL(kern, grid, dim3(64 * W), shm, st, x, ldx, b, ldb, e, sa_out, precise);
  return hipGetLastError();
}

template <int NC, int KS, int W, int P>
hipError_t launch_dq_p(int act_dtype, const uint16_t* x, int64_t ldx, const int8_t* b,
                       int64_t ldb, const Epi& e, float* sa_out, int precise, hipStream_t st) {
  if (act_dtype == I8L_F16)
    return launch_dq_k<NC, KS, W, P, EK_ANY, I8L_F16>(x, ldx, b, ldb, e, sa_out, precise, st);
  switch (epi_kind(e)) {
    case EK_BF16:
      return launch_dq_k<NC, KS, W, P, EK_BF16, I8L_BF16>(x, ldx, b, ldb, e, sa_out, precise,
                                                          st);
    case EK_BF16_BBF16:
      return launch_dq_k<NC, KS, W, P, EK_BF16_BBF16, I8L_BF16>(x, ldx, b, ldb, e, sa_out,
                                                                precise, st);
    default:
      return launch_dq_k<NC, KS, W, P, EK_ANY, I8L_BF16>(x, ldx, b, ldb, e, sa_out, precise,
                                                         st);
  }
}

// Passes of the quantizer prologue: ceil(rows / RPP) for the block's valid rows, taken as
// the next power of two (P in {1, 2, 4, ...}, at most 16 rows).
template <int NC, int KS, int W>
hipError_t launch_dq_t(int act_dtype, const uint16_t* x, int64_t ldx, const int8_t* b,
                       int64_t ldb, const Epi& e, float* sa_out, int precise, hipStream_t st) {
  constexpr int RPP = 64 / (8 * KS);
  const int rows = e.M < 16 ? e.M : 16;
  const int need = (rows + RPP - 1) / RPP;
  if (need <= 1)
    return launch_dq_p<NC, KS, W, 1>(act_dtype, x, ldx, b, ldb, e, sa_out, precise, st);
  if (need <= 2)
    return launch_dq_p<NC, KS, W, 2>(act_dtype, x, ldx, b, ldb, e, sa_out, precise, st);
  if constexpr (16 / RPP >= 4)
    if (need <= 4)
      return launch_dq_p<NC, KS, W, 4>(act_dtype, x, ldx, b, ldb, e, sa_out, precise, st);
  if constexpr (16 / RPP >= 8)
    if (need <= 8)
      return launch_dq_p<NC, KS, W, 8>(act_dtype, x, ldx, b, ldb, e, sa_out, precise, st);
  return hipErrorInvalidValue;
}

hipError_t launch_dq(const i8l_config& c, int act_dtype, const uint16_t* x, int64_t ldx,
                     const int8_t* b, int64_t ldb, const Epi& e, float* sa_out, int precise,
                     hipStream_t st) {
  const int nc = c.bn, ks = c.bk / 64, W = c.warps;
#define I8L_DQ(NC_, KS_, W_)                                                                \
  if (nc == NC_ && ks == KS_ && W == W_)                                                    \
    return launch_dq_t<NC_, KS_, W_>(act_dtype, x, ldx, b, ldb, e, sa_out, precise, st);
  I8L_DQ(8, 2, 16) I8L_DQ(16, 2, 16) I8L_DQ(32, 2, 16) I8L_DQ(8, 4, 16) I8L_DQ(16, 4, 16)
#undef I8L_DQ
  return hipErrorInvalidValue;
}

}  // namespace

void default_config(int64_t M, int64_t N, int64_t K, i8l_config* c) {
  *c = i8l_config{0, 0, 0, 0, 0, 1, 1};
  if (M <= 32 && K % 128 == 0) {
    // weights through LDS: 16 (or, for narrow N, 8) columns a workgroup, the K split over
    // up to 16 waves in one or more steps of up to 512 bytes
    const int mt = M <= 16 ? 1 : 2;
    const int nc = (N % 16 == 0 && N / 16 >= 256) ? 16 : (N % 8 == 0 ? 8 : 4);
    const int64_t k64 = K / 64;
    const int kss[] = {8, 6, 4, 2};
    // first choice: every wave's slice is one step (8, 16 or 4 waves); else 16 waves with
    // the largest step that divides their slices
    for (int W : {8, 16, 4})
      for (int ks : kss) {
        const i8l_config t{16 * mt, nc, 64 * ks, W, 3, 1, 1};
        if (k64 == (int64_t)W * ks && wlds_ok(t, K)) {
          *c = t;
          return;
        }
      }
    for (int ks : kss) {
      const i8l_config t{16 * mt, nc, 64 * ks, 16, 3, 1, 1};
      if (wlds_ok(t, K)) {
        *c = t;
        return;
      }
    }
  }
  // Mid batches on wide or many-token problems: 64-token tiles of 128 columns with the
  // direct-to-LDS ring; the activations are re-read N/128 times instead of N/32.
  // 129 to 1024 tokens, and from 33 tokens on wide N: the largest of the 4-wave overlapped-
  // ring tiles (128x128, 128x64, 64x128, 64x64) that still gives every CU a workgroup, else
  // the smallest.  At these sizes the per-CU latency of the K loop, not the MFMA rate, sets
  // the time, so more workgroups beat fewer re-reads.
  if (M <= 1024 && N % 64 == 0 && K % 128 == 0 && (M > 128 || (M > 32 && N >= 8192))) {
    const int tiles[4][2] = {{128, 128}, {128, 64}, {64, 128}, {64, 64}};
    for (const auto& t : tiles)
      if (N % t[1] == 0 && ((M + t[0] - 1) / t[0]) * (N / t[1]) >= 256) {
        *c = i8l_config{t[0], t[1], 128, 4, 4 + kPipelined, 8, 1};
        return;
      }
    *c = i8l_config{64, 64, 128, 4, 4 + kPipelined, 8, 1};
    return;
  }
  // 17 to 128 tokens: weights through LDS in 32-token x 32-column tiles (several row
  // blocks above 32 tokens), 16 waves of one 128-byte step when K is 2048, else 4 waves
  // stepping through their K slices.
  if (M <= 128 && N % 32 == 0 && K % 128 == 0) {
    const i8l_config one{32, 32, 128, 16, 3, 1, 1};
    const i8l_config steps{32, 32, K % 1024 == 0 ? 256 : 128, 4, 3, 1, 1};
    if (K == 2048 && N < 8192 && wlds_ok(one, K)) {
      *c = one;
      return;
    }
    if (wlds_ok(steps, K)) {
      *c = steps;
      return;
    }
  }
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
  // Prefill: direct-to-LDS macro tiles with the fragment reads overlapped with the MFMAs
  // (the fastest measured family on MI355X): 256x256 tiles once there are enough of them,
  // 128x128 tiles (more workgroups) below.
  c->group_m = 8;
  if (N % 256 == 0 && K % 64 == 0 && M > 1024) {
    *c = i8l_config{256, 256, 64, 8, 12, 4, 1};
  } else if (N % 128 == 0 && K % 128 == 0) {
    *c = i8l_config{128, 128, 128, 4, 12, 8, 1};
  } else if (N % 128 == 0 && K % 64 == 0) {
    *c = i8l_config{128, 128, 64, 4, 12, 8, 1};
  } else {
    // narrow or odd shapes: the weight-streaming tile, one 128-token row block at a time
    int W = stream_max_threads(8, 1) / 64;
    while (W > 1 && K % (64 * W) != 0) W /= 2;
    *c = i8l_config{128, 16, 64 * W, W, 1, 1, 1};
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
  if (!stream_ok(c) && staged_index(c) < 0 && dma_index(c) < 0 && dmap_index(c) < 0 &&
      !wlds_ok(c, K)) {
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
  } else if (c.stages == 3 && c.bn <= 32) {
    // the schedule keeps in-tile row offsets (< 128 token rows, < 32 weight rows) in 32 bits
    if (stride_am > INT32_MAX / 128 || stride_bn > INT32_MAX / 32) {
      const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 3) / 4));
      hipLaunchKernelGGL(gemm_generic, grid, dim3(256), 0, hs, a, stride_am, stride_ak, b,
                         stride_bk, stride_bn, e, K);
      err = hipGetLastError();
    } else {
      err = launch_wlds(c, a, stride_am, b, stride_bn, e, K, hs);
    }
  } else if (c.stages == 2) {
    err = launch_staged(staged_index(c), c, a, stride_am, b, stride_bn, e, (int)K, hs);
  } else if (c.stages >= 3 + kPipelined) {
    err = launch_dmap(dmap_index(c), c, a, stride_am, b, stride_bn, e, (int)K, hs);
  } else {
    err = launch_dma(dma_index(c), c, a, stride_am, b, stride_bn, e, (int)K, hs);
  }
  return hip_status(err, "i8l_w8a8_mm launch");
}

extern "C" int i8l_w8a8_mm_dynq_supported(int64_t M, int64_t N, int64_t K, const i8l_config* cfg) {
  i8l_config c;
  if (cfg) {
    c = *cfg;
  } else if (!default_dq_config(N, K, &c)) {
    set_error("no built dynamic-quant tile takes K=%lld in one step a wave", (long long)K);
    return I8L_UNSUPPORTED;
  }
  if (M < 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) {
    set_error("sizes out of range");
    return I8L_UNSUPPORTED;
  }
  if (c.bn <= 0 || N % c.bn || !dq_ok(c, K)) {
    set_error("config %dx%dx%d w%d s%d is not a built dynamic-quant tile for N=%lld K=%lld",
              c.bm, c.bn, c.bk, c.warps, c.stages, (long long)N, (long long)K);
    return I8L_UNSUPPORTED;
  }
  return I8L_OK;
}

extern "C" int i8l_w8a8_mm_dynq(const void* x, int64_t ldx, int32_t act_dtype,
                                int32_t precise_div, const int8_t* b, int64_t stride_bk,
                                int64_t stride_bn, const float* scale_b, int64_t scale_b_len,
                                const void* bias, int32_t bias_dtype, void* out,
                                int64_t stride_cm, int32_t out_dtype, float* scale_a_out,
                                int64_t M, int64_t N, int64_t K, const i8l_config* cfg,
                                void* stream) {
  if (M < 0 || N < 0 || K < 0) {
    set_error("negative size M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
    return I8L_INVALID_ARG;
  }
  if (act_dtype != I8L_BF16 && act_dtype != I8L_F16) {
    set_error("activations must be bf16 or fp16 (code %d)", act_dtype);
    return I8L_UNSUPPORTED;
  }
  if (out_dtype != I8L_BF16 && out_dtype != I8L_F16 && out_dtype != I8L_F32) {
    set_error("unsupported output dtype code %d", out_dtype);
    return I8L_UNSUPPORTED;
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
  if (ldx < K) {
    set_error("row stride %lld of x is below K=%lld", (long long)ldx, (long long)K);
    return I8L_INVALID_ARG;
  }
  i8l_config c;
  if (cfg) {
    c = *cfg;
  } else if (!default_dq_config(N, K, &c)) {
    set_error("no built dynamic-quant tile takes K=%lld in one step a wave", (long long)K);
    return I8L_UNSUPPORTED;
  }
  const int st = i8l_w8a8_mm_dynq_supported(M, N, K, &c);
  if (st != I8L_OK) return st;
  if (M == 0 || N == 0) return I8L_OK;
  const int osz = elt_size(out_dtype);
  const bool layout = stride_bk == 1 && aligned16(b) && stride_bn % 16 == 0 &&
                      stride_bn <= INT32_MAX / 32 && aligned16(x) && ldx % 8 == 0 &&
                      aligned16(out) && (stride_cm * osz) % 16 == 0 && stride_cm >= N &&
                      N % 4 == 0 && (scale_b_len == 1 || aligned16(scale_b)) &&
                      (bias_dtype == I8L_DTYPE_NONE || aligned16(bias));
  if (!layout) {
    set_error("the dynamic-quant path needs K-contiguous 16-byte aligned operands");
    return I8L_UNSUPPORTED;
  }
  Epi e;
  e.sa = nullptr;
  e.sb = scale_b;
  e.bias = bias;
  e.out = out;
  e.ldc = stride_cm;
  e.sa_per_row = 1;
  e.sb_per_col = scale_b_len == N && N > 1;
  e.bias_dtype = bias_dtype;
  e.out_dtype = out_dtype;
  e.M = (int)M;
  e.N = (int)N;
  const hipError_t err = launch_dq(c, act_dtype, (const uint16_t*)x, ldx, b, stride_bn, e,
                                   scale_a_out, precise_div ? 1 : 0, (hipStream_t)stream);
  return hip_status(err, "i8l_w8a8_mm_dynq launch");
}
