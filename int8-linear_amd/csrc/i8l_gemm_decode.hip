// Decode schedules of the W8A8 GEMM (M <= 128 tokens), their tile tables and launchers:
//  * stream: weights streamed from HBM straight into MFMA operand registers;
//  * wlds / wlds1: weights copied through LDS with direct-to-LDS loads, K split over the
//    waves, one or several steps a wave;
//  * wlds1p: wlds1 walking several column tiles with the activations held in registers;
//  * wlds1_dq: wlds1 with the per-token activation quantizer folded in.
// v_mfma_i32_16x16x64_i8 with the weight fragment as srcA and the activations as srcB.
#include "i8l_gemm.h"

namespace i8l {

// ------------------------------------------------------------------ stream schedule
// Workgroup = W waves on the same 16*NT output columns and 16*MT tokens; wave w owns the
// contiguous K slice [w*ks*64, (w+1)*ks*64).  Lane l of a wave loads, per 64-byte K step,
// 16 bytes of weight row (n0 + 16t + l%16) at K offset 16*(l/16), and the same 16 bytes
// of K for token (m0 + 16i + l%16): both MFMA operands then hold the same K positions,
// so the product is the exact dot product whatever order the unit sums them in.
// Accumulator lane l, register r of fragment (i,t) is out[m0+16i+l%16][n0+16t+4*(l/16)+r].
// K steps are loaded U at a time, one group ahead of the MFMAs consuming the previous one.

// NC (16, 8 or 4) output columns per MFMA tile: with NC < 16, MFMA rows i and i+NC read
// the same weight row (the loads coalesce, so HBM traffic is unchanged) and only rows
// below NC are stored.  Narrow tiles give narrow-N shapes more workgroups.
template <int MT, int NT, int U, int NC>
__global__ void __launch_bounds__(stream_max_threads(MT, NT))
gemm_stream(const int8_t* __restrict__ A, int64_t lda, const int8_t* __restrict__ B,
            int64_t ldb, Epi e, int ks, int nw) {
  pin_args(e, A, lda, B, ldb, ks, nw);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int W = nw;                          // waves (64 * nw threads)
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
// Decode tile of 16*MT tokens x NC columns (NC = 64, 32, 16, 8 or 4).  Each wave owns one
// contiguous K slice of `steps` steps of S = 64*KS bytes.  Per step it copies its NC x S weight bytes
// into its own LDS buffer with global_load_lds_dwordx4: one instruction moves 1 KiB, whole
// row segments of S bytes, so HBM sees full cache lines (the MFMA operand layout would read
// 16 rows x 64 bytes per instruction instead).  LDS row r holds 16-byte chunk c at slot
// c ^ (r & SWM), so the MFMA-layout reads (16 rows, one chunk each) spread over the banks.
// The activations of the next step are loaded into registers while the current step
// multiplies.  A wave only reads its own buffers, so its own vmcnt wait is the only
// synchronisation until the cross-wave sum of the int32 partials.
// With NC < 16, MFMA rows i and i+NC read the same weight row and only rows below NC are
// stored.  Token rows past M read row 0 and are never stored.
// Split of K across workgroups: with gridDim.z = Z > 1, workgroup z takes the z-th of Z equal
// parts of K (W * steps * S bytes each) and stores its exact int32 partial tile into plane z
// of an [Z][M][ldc] int32 buffer (the Epi's output, raw); splitk_sum adds the planes and
// applies the epilogue.


// The end of the multi-step weights-through-LDS tiles: sum the W waves' partial products
// (int32 addition is exact and order-free) through an LDS area that aliases the step ring
// (every wave's last fragment reads of the ring are done at the first barrier, and no DMA
// is outstanding after the last step's wait), then the epilogue; fragment fr = i * NF + f is
// stored by wave fr % W, which loaded the epilogue operands of its first KP fragments (fr =
// wave + j * W, j < KP: clp[j], sap[j]) before its main loop.
template <int MT, int NC, int EK, int KP>
__device__ __forceinline__ void wlds_sum_store(const v4i (&acc)[MT][NC < 16 ? 1 : NC / 16],
                                               int8_t* lds, const Epi& e, int W, int wave,
                                               int lane, int64_t m0, int64_t n0,
                                               const Cols4 (&clp)[KP], const float (&sap)[KP]) {
  constexpr int NCF = NC < 16 ? NC : 16;
  constexpr int NF = NC / NCF;
  constexpr int FR = MT * NF;
  const int r16 = lane & 15, grp = lane >> 4;
  v4i* red = (v4i*)lds;  // [W][FR][64]
  if (W > 1) {
    __syncthreads();
#pragma unroll
    for (int q = 0; q < MT; ++q)
#pragma unroll
      for (int f = 0; f < NF; ++f) red[(wave * FR + q * NF + f) * 64 + lane] = acc[q][f];
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < FR; ++j) {
    const int fr = wave + j * W;
    if (fr >= FR) break;
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
      if (j < KP)
        store4s<EK>(e, m, n, sum, clp[j < KP ? j : 0], sap[j < KP ? j : 0]);
      else
        store4<EK>(e, m, n, sum);
    }
  }
}

template <int MT, int NC, int KS, int EK>
__global__ void __launch_bounds__(wlds_bound(MT, KS, NC))
gemm_wlds(const int8_t* __restrict__ A, int64_t lda, const int8_t* __restrict__ B, int64_t ldb,
          Epi e, int steps, int nbuf, int nw) {
  pin_args(e, A, lda, B, ldb, steps, nbuf, nw);
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
  constexpr int NF = NC / NCF;               // column fragments of the tile (64 columns: 4)
  constexpr int FR = MT * NF;                // output fragments, numbered i * NF + f
  static_assert(NF * NCF == NC, "the tile must be whole column fragments");
  extern __shared__ __attribute__((aligned(16))) int8_t lds[];

  const int lane = threadIdx.x & 63;
  // wave-uniform values live in scalar registers: the per-lane address work before the first
  // load is then a few 32-bit operations
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = nw;                          // waves (64 * nw threads)
  const int r16 = lane & 15, grp = lane >> 4;
  const int64_t n0 = xcd_col_tile() * NC;
  const int64_t m0 = (int64_t)blockIdx.y * (16 * MT);
  const int64_t kw = (int64_t)(blockIdx.z * W + wave) * steps * S;
  if (gridDim.z > 1) e.out = (int32_t*)e.out + (int64_t)blockIdx.z * e.M * e.ldc;
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
      __builtin_amdgcn_global_load_lds((const void*)(gsrc[t] + ko), dst + t * 1024, 16, 0,
                                       kWeightCpol);
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
  // The wave that stores fragment fr (fr % W == wave) loads the epilogue operands of its
  // first KP fragments now, behind the first step, so their latency hides under the main
  // loop (a fragment past them would load its operands after the cross-wave sum: a round
  // trip of ~0.5 us in the 64x32 tile of 4 waves, two fragments a wave).
  constexpr int KP = 1;                      // (more would spill in the register-bound tiles)
  Cols4 clp[KP];
  float sap[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    sap[j] = 0.0f;
    const int fr = wave + j * W;
    if (fr < FR && 4 * grp < NCF) {
      const int64_t m = m0 + 16 * (fr / NF) + r16;
      clp[j] = load_cols4<EK>(e, n0 + NCF * (fr % NF) + 4 * grp);
      sap[j] = load_sa<EK>(e, m < e.M ? m : 0);
    }
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

  wlds_sum_store<MT, NC, EK, KP>(acc, lds, e, W, wave, lane, m0, n0, clp, sap);
}

// gemm_wlds with the activations copied through LDS too: a wave's step buffer holds its NC
// weight rows and then its 16*MT activation rows, S bytes each (same swizzle), all filled by
// global_load_lds_dwordx4 in whole row segments, and both MFMA operands are read from LDS in
// the fragment layout.  gemm_wlds loads the activations straight into the fragment layout
// (16 rows x 64 bytes an instruction: half a cache line a row per request); from 32 tokens
// on, where a CU takes in as many activation bytes as weight bytes, that costs 20-40% of
// the kernel.  Rows past M read the tile's first row (always valid) and are never stored.
template <int MT, int NC, int KS, int EK>
__global__ void __launch_bounds__(wlds_bound(MT, KS, NC))
gemm_wlds_a(const int8_t* __restrict__ A, int64_t lda, const int8_t* __restrict__ B,
            int64_t ldb, Epi e, int steps, int nbuf, int nw) {
  constexpr int S = 64 * KS;
  constexpr int CPR = S / 16;
  constexpr int CPR_LOW = CPR & -CPR;
  constexpr int SWM = (CPR_LOW < 16 ? CPR_LOW : 16) - 1;
  static_assert(CPR % (SWM + 1) == 0, "the swizzle must permute the row's chunks");
  constexpr int ROWS = NC + 16 * MT;         // weight rows, then activation rows
  constexpr int SB = ROWS * S;               // bytes per wave per step
  constexpr int NI = SB / 1024;              // DMA instructions per wave per step
  static_assert(NI * 1024 == SB, "a step must be whole 1 KiB DMA instructions");
  static_assert(NI < 64, "one step's DMA must fit the vmcnt counter");
  constexpr int NCF = NC < 16 ? NC : 16;
  constexpr int NF = NC / NCF;
  constexpr int FR = MT * NF;
  static_assert(NF * NCF == NC, "the tile must be whole column fragments");
  extern __shared__ __attribute__((aligned(16))) int8_t lds[];

  pin_args(e, A, lda, B, ldb, steps, nbuf, nw);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = nw;                          // waves (64 * nw threads)
  const int r16 = lane & 15, grp = lane >> 4;
  const int64_t n0 = xcd_col_tile() * NC;
  const int64_t m0 = (int64_t)blockIdx.y * (16 * MT);
  const int64_t kw = (int64_t)(blockIdx.z * W + wave) * steps * S;
  if (gridDim.z > 1) e.out = (int32_t*)e.out + (int64_t)blockIdx.z * e.M * e.ldc;
  int8_t* wbuf = lds + (size_t)wave * nbuf * SB;

  // DMA sources: instruction t writes buffer bytes [t*1024, t*1024+1024), lane l the 16 bytes
  // at +16*l: row o / S (weight row r < NC, else activation row r - NC), slot (o % S) / 16.
  // In-tile row offsets (< 64 weight rows, < 128 token rows) fit 32 bits.
  const int8_t* Bw = B + n0 * ldb + kw;
  const int8_t* Aw = A + m0 * lda + kw;
  const int ldb32 = (int)ldb, lda32 = (int)lda;
  const int8_t* gsrc[NI];
#pragma unroll
  for (int t = 0; t < NI; ++t) {
    const int o = t * 1024 + 16 * lane;
    const int r = o / S, c = ((o % S) / 16) ^ (r & SWM);
    const int ml = r - NC;
    gsrc[t] = r < NC ? Bw + (r * ldb32 + 16 * c)
                     : Aw + ((m0 + ml < e.M ? ml * lda32 : 0) + 16 * c);
  }
  // fragment read offsets of one step: weight fragment f's row br, activation fragment i's
  // row NC + 16 i + r16, chunk 4s + grp
  int bofs[KS][NF], aofs[KS][MT];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int br = NCF * f + r16 % NCF;
      bofs[s][f] = br * S + 16 * ((4 * s + grp) ^ (br & SWM));
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int ar = NC + 16 * i + r16;
      aofs[s][i] = ar * S + 16 * ((4 * s + grp) ^ (ar & SWM));
    }
  }

  v4i acc[MT][NF];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int f = 0; f < NF; ++f) acc[i][f] = v4i{0, 0, 0, 0};

  // `fenced` as in gemm_wlds: the previous step's fragment reads stay above the issue
  auto issue = [&](int step, bool fenced) {
    if (fenced) __builtin_amdgcn_sched_barrier(0);
    lds_i8_t* dst = (lds_i8_t*)(wbuf + (step % nbuf) * SB);
    const int64_t ko = (int64_t)step * S;
#pragma unroll
    for (int t = 0; t < NI; ++t)
      if (t * 1024 + 1023 < NC * S)   // weight rows only: streamed
        __builtin_amdgcn_global_load_lds((const void*)(gsrc[t] + ko), dst + t * 1024, 16, 0,
                                         kWeightCpol);
      else                            // activation rows, which other workgroups re-read
        __builtin_amdgcn_global_load_lds((const void*)(gsrc[t] + ko), dst + t * 1024, 16, 0, 0);
    if (fenced) __builtin_amdgcn_sched_barrier(0);
  };
  auto compute = [&](int step) {
    const int8_t* base = wbuf + (step % nbuf) * SB;
    v4i b[KS][NF], a[KS][MT];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int f = 0; f < NF; ++f) b[s][f] = *(const v4i*)(base + bofs[s][f]);
#pragma unroll
      for (int i = 0; i < MT; ++i) a[s][i] = *(const v4i*)(base + aofs[s][i]);
    }
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int f = 0; f < NF; ++f)
          acc[i][f] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b[s][f], a[s][i], acc[i][f], 0, 0, 0);
  };

  issue(0, steps > 1);
  constexpr int KP = FR < 4 ? FR : 4;        // fragments a wave stores with operands loaded now
  Cols4 clp[KP];
  float sap[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    sap[j] = 0.0f;
    const int fr = wave + j * W;
    if (fr < FR && 4 * grp < NCF) {
      const int64_t m = m0 + 16 * (fr / NF) + r16;
      clp[j] = load_cols4<EK>(e, n0 + NCF * (fr % NF) + 4 * grp);
      sap[j] = load_sa<EK>(e, m < e.M ? m : 0);
    }
  }
  // each step's copy is requested before the wait for the one before, which leaves exactly
  // one step's DMA outstanding (the epilogue operands were requested between steps 0 and 1,
  // so they have landed too); with three buffers, two steps ahead: the wait for step i
  // leaves steps i+1 and i+2 in flight (a step of a CU's four waves takes ~0.5 us to land,
  // longer than its MFMAs); with four, three steps ahead.  A depth whose outstanding DMA
  // would not fit the vmcnt counter falls back to the next smaller one.
  int i = 0;
  int depth = 1;
  if constexpr (2 * NI < 64)
    if (nbuf >= 3 && steps > 2) depth = 2;
  if constexpr (3 * NI < 64)
    if (nbuf >= 4 && steps > 3) depth = 3;
  if (depth == 3) {
    if constexpr (3 * NI < 64) {
      issue(1, true);
      issue(2, true);
      for (; i + 3 < steps; ++i) {
        issue(i + 3, true);
        wait_vmcnt_wlds<3 * NI>();
        compute(i);
      }
      wait_vmcnt_wlds<2 * NI>();
      compute(i);
      ++i;
      wait_vmcnt_wlds<NI>();
      compute(i);
      ++i;
    }
  } else if (depth == 2) {
    if constexpr (2 * NI < 64) {
      issue(1, true);
      for (; i + 2 < steps; ++i) {
        issue(i + 2, true);
        wait_vmcnt_wlds<2 * NI>();
        compute(i);
      }
      wait_vmcnt_wlds<NI>();
      compute(i);
      ++i;
    }
  } else {
    for (; i + 1 < steps; ++i) {
      issue(i + 1, true);
      wait_vmcnt_wlds<NI>();
      compute(i);
    }
  }
  wait_vmcnt_wlds<0>();
  compute(i);
  wlds_sum_store<MT, NC, EK, KP>(acc, lds, e, W, wave, lane, m0, n0, clp, sap);
}

// The same tile when every wave's K slice is a single step (K == W * 64 * KS), with the
// wave count and the epilogue kind fixed at compile time: the path from the first load to
// the last store is straight-line code apart from the wave-uniform test of which waves
// store, which matters in a kernel this short (see EK_ANY).
template <int MT, int NC, int KS, int W, int EK>
__global__ void __launch_bounds__(64 * W)
gemm_wlds1(const int8_t* __restrict__ A, int64_t lda, const int8_t* __restrict__ B, int64_t ldb,
           Epi e) {
  pin_args(e, A, lda, B, ldb);
  constexpr int S = 64 * KS;
  constexpr int CPR = S / 16;
  constexpr int CPR_LOW = CPR & -CPR;
  constexpr int SWM = (CPR_LOW < 16 ? CPR_LOW : 16) - 1;
  static_assert(CPR % (SWM + 1) == 0, "the swizzle must permute the row's chunks");
  constexpr int SB = NC * S;
  constexpr int NI = SB / 1024;
  static_assert(NI * 1024 == SB, "a step must be whole 1 KiB DMA instructions");
  constexpr int NCF = NC < 16 ? NC : 16;     // output columns of one MFMA fragment
  constexpr int NF = NC / NCF;               // column fragments of the tile (64 columns: 4)
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
                                     16, 0, kWeightCpol);
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

// ------------------------------------------------------------------ persistent single-step decode
// gemm_wlds1 walking several column tiles: a workgroup loads its token rows' activation
// fragments into registers once and then takes the column tiles blockIdx.x, blockIdx.x +
// gridDim.x, ...; each tile's weights are requested into the other of two LDS buffers before
// the current tile's MFMAs, reduction and epilogue.  gemm_wlds1 reads A (its 16*MT rows,
// all of K) once per column tile, as much L2 traffic as the weights themselves at 16 tokens;
// here A is read once per workgroup.  Each wave reads only its own weight slices, so a
// buffer is refilled as soon as the wave's own MFMAs have consumed it; the reduction area
// is shared and is fenced by a barrier on each side.  LOOP false: the straight form for a
// grid with one tile a workgroup (no next tile to request).
//
// ACT kActSilu / kActSiluRound: the gate_up projection with the SiLU-and-mul epilogue.  The
// weight's first N/2 rows are the gate, the last N/2 the up projection; tile t takes gate rows
// [t*H, (t+1)*H) and the same up rows (H = NC/2) into the fragment's first and last H rows,
// and the epilogue writes y = silu(gate) * up, [M, N/2] bf16 (silu_mul_pairs), instead of the
// [M, N] product.
template <int MT, int NC, int KS, int W, int EK, int ACT = kActPlain, bool LOOP = true>
__global__ void __launch_bounds__(64 * W)
gemm_wlds1p(const int8_t* __restrict__ A, int64_t lda, const int8_t* __restrict__ B,
            int64_t ldb, Epi e) {
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
  constexpr int FR = MT * NF;
  static_assert(NF * NCF == NC, "the tile must be whole column fragments");
  static_assert(FR <= W, "every fragment needs a storing wave");
  constexpr bool SILU = ACT != kActPlain;
  static_assert(!SILU || (MT == 1 && NF == 1 && EK != EK_ANY),
                "the SiLU epilogue takes one fragment of bf16 output");
  constexpr int H = NC / 2;                  // SiLU: gate (and up) columns of a tile
  extern __shared__ __attribute__((aligned(16))) int8_t lds[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, grp = lane >> 4;
  const int tiles = e.N / NC;
  const int64_t m0 = (int64_t)blockIdx.y * (16 * MT);
  const int64_t kw = (int64_t)wave * S;
  int8_t* const wb0 = lds + (size_t)wave * SB;
  int8_t* const wb1 = lds + (size_t)(W + wave) * SB;
  v4i* const red = (v4i*)(lds + (size_t)2 * W * SB);  // [W][FR][64]
  const int ldb32 = (int)ldb;

  auto dma = [&](int ct, int8_t* wb) {
    lds_i8_t* dst = (lds_i8_t*)wb;
    if constexpr (SILU) {
      // tile row r: gate row ct*H + r for r < H, else up row N/2 + ct*H + r - H
      const int8_t* Bg = B + (int64_t)ct * H * ldb + kw;
      const int8_t* Bu = Bg + (int64_t)(e.N / 2) * ldb - (int64_t)H * ldb;
#pragma unroll
      for (int t = 0; t < NI; ++t) {
        const int o = t * 1024 + 16 * lane;
        const int r = o / S, c = ((o % S) / 16) ^ (r & SWM);
        __builtin_amdgcn_global_load_lds((const void*)((r < H ? Bg : Bu) + (r * ldb32 + 16 * c)),
                                         dst + t * 1024, 16, 0, kWeightCpol);
      }
    } else {
      const int8_t* Bw = B + (int64_t)ct * NC * ldb + kw;
#pragma unroll
      for (int t = 0; t < NI; ++t) {
        const int o = t * 1024 + 16 * lane;
        const int r = o / S, c = ((o % S) / 16) ^ (r & SWM);
        __builtin_amdgcn_global_load_lds((const void*)(Bw + (r * ldb32 + 16 * c)), dst + t * 1024,
                                         16, 0, kWeightCpol);
      }
    }
  };

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
  const int64_t mrow = m0 + 16 * (wave / NF) + r16;
  float sam = 0.0f;
  if (wave < FR) sam = load_sa<EK>(e, mrow < e.M ? mrow : m0);

  const int cq = 4 * (grp & (NCF / 4 - 1));   // the lane's first column in the fragment
  // SiLU: gate lanes (cq < H) read gate columns ct*H + cq, up lanes up columns N/2 + ...
  auto ncol_of = [&](int ct) -> int64_t {
    return SILU ? (cq < H ? (int64_t)ct * H + cq : (int64_t)(e.N / 2) + ct * H + cq - H)
                : (int64_t)ct * NC + NCF * (wave % NF) + cq;
  };

  // A tile's MFMAs, cross-wave sum and epilogue, from its weights in `cur` and its epilogue
  // operands `cl` (both landed).  ASM: the reduction's LDS stores as inline assembly, for
  // when the next tile's copy is in flight (an LDS store the compiler can see would make it
  // wait for every vector-memory request first: it cannot tell where the copy writes).
  auto body = [&](int ct, const int8_t* cur, const Cols4& cl, auto asm_tag) {
    constexpr bool ASM = decltype(asm_tag)::value;
    const int64_t ncol = ncol_of(ct);
    v4i b[KS][NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int br = NCF * f + r16 % NCF;
#pragma unroll
      for (int s = 0; s < KS; ++s)
        b[s][f] = *(const v4i*)(cur + br * S + 16 * ((4 * s + grp) ^ (br & SWM)));
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
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        v4i* const slot = &red[(wave * FR + i * NF + f) * 64 + lane];
        if constexpr (ASM) lds_store_b128(slot, acc[i][f]);
        else *slot = acc[i][f];
      }
    lds_sync();
    if (wave < FR) {
      v4i sum = red[wave * 64 + lane];
#pragma unroll
      for (int w = 1; w < W; ++w) sum += red[(w * FR + wave) * 64 + lane];
      if constexpr (SILU) {
        float v[4];
        epi_values4<EK>(e, sum, cl, sam, v);
        silu_mul_pairs<ACT, 4 * H>(v, cq < H);
        if (mrow < e.M && cq < H && 4 * grp < NCF) store4_bf16(e.out, e.ldc, mrow, ct * H + cq, v);
      } else {
        if (mrow < e.M && 4 * grp < NCF) store4s<EK>(e, mrow, ncol, sum, cl, sam);
      }
    }
    lds_sync();  // the partials of the next tile overwrite the reduction area
  };

  int ct = blockIdx.x;
  if (ct >= tiles) return;
  if constexpr (!LOOP) {
    // one tile a workgroup (the launcher's choice when the grid covers the tiles): nothing
    // else is requested while it runs
    dma(ct, wb0);
    Cols4 cl;
    if (wave < FR) cl = load_cols4<EK>(e, ncol_of(ct));
    wait_vmcnt_wlds<0>();
    body(ct, wb0, cl, std::false_type{});
    return;
  }
  // Several tiles a workgroup.  A tile's weights and epilogue operands are requested a tile
  // earlier; the explicit vmcnt(0) at the top of each tile is the loop's only wait on vector
  // memory, after which the next tile's are requested, so they are in flight during this
  // tile's MFMAs, reduction and epilogue.  (A use of a loaded register while a direct-to-LDS
  // copy is in flight makes the compiler wait for every request, so the operands live in two
  // register sets that alternate between tiles.)
  auto tile = [&](int ct, const int8_t* cur, int8_t* nxt, const Cols4& cl, Cols4& cln) {
    wait_vmcnt_wlds<0>();
    __builtin_amdgcn_sched_barrier(0);
    const int ctn = ct + (int)gridDim.x;
    if (ctn < tiles) {               // uniform over the workgroup
      dma(ctn, nxt);
      if (wave < FR) cln = load_cols4<EK>(e, ncol_of(ctn));
    }
    __builtin_amdgcn_sched_barrier(0);
    body(ct, cur, cl, std::true_type{});
  };
  Cols4 c0, c1;
  dma(ct, wb0);
  if (wave < FR) c0 = load_cols4<EK>(e, ncol_of(ct));
  for (;;) {
    tile(ct, wb0, wb1, c0, c1);
    ct += gridDim.x;
    if (ct >= tiles) break;
    tile(ct, wb1, wb0, c1, c0);
    ct += gridDim.x;
    if (ct >= tiles) break;
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
//
// ACT selects what is quantized.  kActPlain: X itself.  kActSilu / kActSiluRound: the
// SiLU-and-mul of a gate_up row, X holding the gate values and X + up the up values of the
// same row: y = cast(silu(g) * u), with silu(g) = g / (1 + exp(-g)) from the canonical exp
// and a correctly rounded quotient, rounded to the activation dtype first for kActSiluRound;
// these are the silu_mul_quant kernel's values, so the output equals silu_mul_quant followed
// by w8a8_mm bit for bit (reference fused_quant.py:76-88 then kernel.py:63-124).

template <int NC, int KS, int W, int P, int EK, int DT, int ACT>
__global__ void __launch_bounds__(64 * W)
gemm_wlds1_dq(const uint16_t* __restrict__ X, int64_t ldx, int64_t up,
              const int8_t* __restrict__ B, int64_t ldb, Epi e, float* __restrict__ sa_out,
              int precise) {
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
  // valid rows of the block; the host picks P as ceil(mb / RPP) rounded up to a power of two,
  // so the last pass can find no valid row (e.g. 3 rows at RPP 1 run P = 4): its loads and
  // stores are then skipped by the per-row test
  const int mb = (int)min((int64_t)16, (int64_t)e.M - m0);
  const int64_t kw = (int64_t)wave * S;
  int8_t* wbuf = lds + (size_t)wave * SB;
  v4i* red = (v4i*)(lds + (size_t)W * SB);                          // [W][NF][64]
  float* rmax = (float*)(lds + (size_t)W * SB + (size_t)W * NF * 1024);  // [W][16]
  int8_t* abuf = lds + (size_t)W * SB + (size_t)W * NF * 1024 + (size_t)W * 64 + wave * 16 * S;

  // The activations are requested first and waited for alone: the quantizer work below
  // then runs while the weights' DMA is still in flight.
  // pass p: lane l holds chunk l % CH of row p*RPP + l/CH (rows past M are not read)
  const int crow = lane / CH, cchunk = lane % CH;
  constexpr bool SILU = ACT != kActPlain;
  uint4 xr[P], ur[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    xr[p] = uint4{0, 0, 0, 0};
    ur[p] = uint4{0, 0, 0, 0};
    const int r = p * RPP + crow;
    if (r < mb) {
      const uint16_t* src = X + (m0 + r) * ldx + kw + 8 * cchunk;
      xr[p] = *(const uint4*)src;
      if constexpr (SILU) ur[p] = *(const uint4*)(src + up);
    }
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
                                     16, 0, kWeightCpol);
  }
  __builtin_amdgcn_sched_barrier(0);
  wait_vmcnt_wlds<NI>();  // vector loads complete in issue order: the activations are in
  __builtin_amdgcn_sched_barrier(0);        // no use of the rows above the wait

  auto elem = [&](const uint4& v, int k) -> float {
    const uint32_t w32 = k < 4 ? (k < 2 ? v.x : v.y) : (k < 6 ? v.z : v.w);
    return act_to_f32<DT>((k & 1) ? (w32 >> 16) : (w32 & 0xffffu));
  };
  // the values to quantize, computed once (rows past M hold zeros, silu(0) * 0 = 0)
  float y[P][8];
  // silu(g) = g / d with d = 1 + exp(-g): the quotient as rcp(d) with one Newton-Markstein
  // correction and g's sign, which equals IEEE division for every bf16 and fp16 g in
  // (-87, +inf) (the silu_mul_quant kernel's fast form); a wave holding any other g takes
  // IEEE division for all of its values.
  auto silu = [&](float g, bool ieee) -> float { return silu_canon(g, ieee); };
  auto fill = [&](bool ieee) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
#pragma unroll
      for (int k = 0; k < 8; k += 2) {
        float a0 = elem(xr[p], k), a1 = elem(xr[p], k + 1);
        if constexpr (SILU) {
          a0 = silu(a0, ieee);
          a1 = silu(a1, ieee);
          if constexpr (ACT == kActSiluRound) round_through2<DT>(a0, a1);
          a0 = a0 * elem(ur[p], k);
          a1 = a1 * elem(ur[p], k + 1);
          round_through2<DT>(a0, a1);
        }
        y[p][k] = a0;
        y[p][k + 1] = a1;
      }
    }
  };
  if constexpr (SILU) {
    float gmin = __builtin_inff(), gmax = -__builtin_inff();
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        gmin = fminf(gmin, elem(xr[p], k));
        gmax = fmaxf(gmax, elem(xr[p], k));
      }
    fill(!__all(gmin > -87.0f && gmax < __builtin_inff()));
  } else {
    fill(false);
  }
  // absmax of each valid row's slice: a lane's chunk, then the CH lanes of the row (the
  // passes' cross-lane maxima side by side)
  float am[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    am[p] = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) am[p] = fmaxf(am[p], fabsf(y[p][k]));
  }
  group_max_n<CH, P>(am);
  if (cchunk == 0) {
#pragma unroll
    for (int p = 0; p < P; ++p) rmax[wave * 16 + p * RPP + crow] = am[p];
  }
  lds_sync();
  // each row's scale and inverse once, in lane r of every wave for row r (r = lane % 16,
  // rows past the passes clamped to the last); a pass takes its row's from that lane
  float sc_l, inv_l;
  {
    const int rl = min(r16, P * RPP - 1);
    float absmax = rmax[rl];
#pragma unroll
    for (int w = 1; w < W; ++w) absmax = fmaxf(absmax, rmax[w * 16 + rl]);
    const float s_div = absmax / 127.0f;
    const float i_div = absmax == 0.0f ? 0.0f : 127.0f / absmax;
    const float s_rcp = absmax * (1.0f / 127.0f);
    const float i_rcp = absmax == 0.0f ? 0.0f : 127.0f * (1.0f / absmax);
    sc_l = precise ? s_div : s_rcp;
    inv_l = precise ? i_div : i_rcp;
  }
  if (sa_out != nullptr && blockIdx.x == 0 && wave == 0 && lane < mb) sa_out[m0 + lane] = sc_l;
  // codes of each valid chunk into the wave's LDS tile (row pitch S bytes); the passes'
  // inverses fetched first, together
  float invp[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    if constexpr (RPP == 1) invp[p] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv_l), p));
    else invp[p] = __shfl(inv_l, p * RPP + crow);
  }
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int r = p * RPP + crow;
    const float inv = invp[p];
    if (r < mb) {
      uint32_t word[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        uint32_t packed = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) packed |= code_rne(y[p][4 * q + b] * inv) << (8 * b);
        word[q] = packed;
      }
      lds_store_b64(abuf + r * S + 8 * cchunk, word[0], word[1]);  // the weight copy is in flight
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
    // row r16's scale: this lane computed it above (lane l holds row l % 16)
    if (r16 < mb && 4 * grp < NCF) store4s<EK>(e, mrow, ncol, sum, cl, sc_l);
  }
}

// ------------------------------------------------------------------ host side
struct StreamTile {
  int mt, nt, nc;
};

// The tiles this library is built with.
// (MT, NT, NC): bm = 16*MT tokens, bn = NC*NT columns.  NC < 16 only with NT == 1, so bn
// names the tile unambiguously.
constexpr StreamTile kStream[] = {{1, 1, 16}, {2, 1, 16}, {4, 1, 16}, {8, 1, 16}, {1, 2, 16},
                                  {2, 2, 16}, {4, 2, 16}, {1, 1, 8},  {2, 1, 8},  {1, 1, 4}};

bool stream_ok(const i8l_config& c) {
  if (c.stages != 1 || c.bm % 16) return false;
  if (c.warps < 1 || c.bk != 64 * c.warps) return false;
  for (auto t : kStream)
    if (t.mt * 16 == c.bm && t.nt * t.nc == c.bn) {
      const int f = t.mt * t.nt;
      return c.warps * 64 <= stream_max_threads(t.mt, t.nt) &&
             (c.warps == 1 || c.warps * f * 1024 <= 96 * 1024);
    }
  return false;
}

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
                              {4, 32, 4}, {1, 64, 2}, {2, 64, 2}, {4, 64, 2}, {1, 64, 4},
                              {2, 64, 4}};

// LDS of gemm_wlds: the weight ring, or the reduction area of the partial products, which
// aliases it, whichever is larger.
size_t wlds_lds_bytes(const i8l_config& c, int64_t K) {
  const int64_t steps = K / ((int64_t)c.bk * c.warps);
  const int nbuf = steps > 1 ? 2 : 1;
  const int nf = c.bn > 16 ? c.bn / 16 : 1;  // 16-column fragments a wave reduces
  const size_t ring = (size_t)c.warps * nbuf * c.bn * c.bk;
  const size_t red = (size_t)c.warps * (c.bm / 16) * nf * 1024;
  return std::max(ring, red);
}

// LDS of gemm_wlds_a: the step ring of weight and activation rows, or the reduction area
// that aliases it, whichever is larger.
size_t wlds_a_lds_bytes(const i8l_config& c, int64_t K, int nbuf) {
  const int nf = c.bn > 16 ? c.bn / 16 : 1;
  const size_t ring = (size_t)c.warps * nbuf * (c.bn + c.bm) * c.bk;
  const size_t red = (size_t)c.warps * (c.bm / 16) * nf * 1024;
  return std::max(ring, red);
}

// Buffers of gemm_wlds_a's ring: group_m for a stages-3 config with group_m 3 or 4
// (group_m - 1 steps in flight; wlds_ok takes it only where K has more than that many
// steps a wave and the buffers fit the LDS), else two (one step a wave: one).
int wlds_a_nbuf(const i8l_config& c, int64_t K) {
  const int64_t steps = K / ((int64_t)c.bk * c.warps);
  if (c.stages == 3 && (c.group_m == 3 || c.group_m == 4) && steps > c.group_m - 1)
    return c.group_m;
  return steps > 1 ? 2 : 1;
}

// LDS of gemm_wlds1 (one step a wave): its weight buffers and, after them, the reduction area.
size_t wlds1_lds_bytes(int mt, int nc, int ks, int W) {
  return (size_t)W * nc * 64 * ks + (size_t)W * mt * (nc > 16 ? nc / 16 : 1) * 1024;
}

bool wlds1_built(int mt, int nc, int W, int ks);

bool wlds_ok(const i8l_config& c, int64_t K) {
  if (c.stages != 3 || c.bn > 64 || c.warps < 1 || c.warps > 16) return false;
  bool built = false;
  for (auto t : kWlds)
    if (16 * t.mt == c.bm && t.nc == c.bn && 64 * t.ks == c.bk &&
        c.warps * 64 <= wlds_bound(t.mt, t.ks, t.nc))
      built = true;
  if (!built || K <= 0 || K % ((int64_t)c.bk * c.warps)) return false;
  const bool one_step = K == (int64_t)c.bk * c.warps &&
                        wlds1_built(c.bm / 16, c.bn, c.warps, c.bk / 64);
  if (!one_step && !wlds_multi_fits(c.bm / 16, c.bn, c.bk / 64)) return false;
  if (c.group_m == 3 || c.group_m == 4) {   // gemm_wlds_a's deeper rings
    const int ni = (c.bn + c.bm) * c.bk / 1024;   // DMA instructions a wave a step
    return K > (int64_t)(c.group_m - 1) * c.bk * c.warps && (c.group_m - 1) * ni < 64 &&
           wlds_a_lds_bytes(c, K, c.group_m) <= kMaxLds;
  }
  return (one_step ? wlds1_lds_bytes(c.bm / 16, c.bn, c.bk / 64, c.warps)
                   : wlds_lds_bytes(c, K)) <= kMaxLds;
}

template <int MT, int NT, int NC>
hipError_t launch_stream_u(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                           const Epi& e, int W, int ks, hipStream_t st) {
  const dim3 grid(e.N / (NC * NT), (e.M + 16 * MT - 1) / (16 * MT));
  const size_t shm = W > 1 ? (size_t)W * MT * NT * 1024 : 0;
  constexpr int UMAX = stream_unroll(MT, NT);
  if (UMAX == 4 && ks % 4 == 0)
    hipLaunchKernelGGL((gemm_stream<MT, NT, UMAX, NC>), grid, dim3(64 * W), shm, st, a, lda, b, ldb, e, ks,
                       W);
  else if (ks % 2 == 0)
    hipLaunchKernelGGL((gemm_stream<MT, NT, 2, NC>), grid, dim3(64 * W), shm, st, a, lda, b, ldb, e, ks,
                       W);
  else
    hipLaunchKernelGGL((gemm_stream<MT, NT, 1, NC>), grid, dim3(64 * W), shm, st, a, lda, b, ldb, e, ks,
                       W);
  return hipGetLastError();
}

// The multi-step tile over `parts` equal parts of K (grid z; 1 = no split): with the
// activations copied through LDS when both rings fit (gemm_wlds_a), else loaded into
// registers (gemm_wlds).
template <int MT, int NC, int KS, int EK>
hipError_t launch_wlds_steps(const i8l_config& c, const int8_t* a, int64_t lda,
                             const int8_t* b, int64_t ldb, const Epi& e, int64_t kpart,
                             int parts, hipStream_t st) {
  const int steps = (int)(kpart / ((int64_t)c.bk * c.warps));
  const dim3 grid(e.N / NC, (e.M + 16 * MT - 1) / (16 * MT), parts);
  const int nbuf_a = wlds_a_nbuf(c, kpart);
  const size_t shm_a = wlds_a_lds_bytes(c, kpart, nbuf_a);
  if (shm_a <= kMaxLds) {
    auto kern = gemm_wlds_a<MT, NC, KS, EK>;
    static std::atomic<uint64_t> lds_done{0};  // devices this kernel is opted in on
    lds_opt_in((const void*)kern, kMaxLds, lds_done);
    hipLaunchKernelGGL(kern, grid, dim3(64 * c.warps), shm_a, st, a, lda, b, ldb, e, steps,
                       nbuf_a, c.warps);
  } else {
    auto kern = gemm_wlds<MT, NC, KS, EK>;
    static std::atomic<uint64_t> lds_done{0};
    lds_opt_in((const void*)kern, kMaxLds, lds_done);
    hipLaunchKernelGGL(kern, grid, dim3(64 * c.warps), wlds_lds_bytes(c, kpart), st, a, lda, b,
                       ldb, e, steps, steps > 1 ? 2 : 1, c.warps);
  }
  return hipGetLastError();
}

template <int MT, int NC, int KS, int EK>
hipError_t launch_wlds_k(const i8l_config& c, const int8_t* a, int64_t lda, const int8_t* b,
                         int64_t ldb, const Epi& e, int64_t K, hipStream_t st) {
  return launch_wlds_steps<MT, NC, KS, EK>(c, a, lda, b, ldb, e, K, 1, st);
}

template <int MT, int NC, int KS, int W, int EK>
hipError_t launch_wlds1_k(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                          const Epi& e, hipStream_t st) {
  auto kern = gemm_wlds1<MT, NC, KS, W, EK>;
  const size_t shm = wlds1_lds_bytes(MT, NC, KS, W);
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
  I8L_WLDS(1, 64, 2) I8L_WLDS(2, 64, 2) I8L_WLDS(4, 64, 2) I8L_WLDS(1, 64, 4) I8L_WLDS(2, 64, 4)
#undef I8L_WLDS
  return hipErrorInvalidValue;
}

// ------------------------------------------------------------------ split of K across workgroups
// stages 5: the weights-through-LDS tile (bm, bn, bk, warps as for stages 3) with K cut into
// group_m equal parts, one workgroup each (grid z), so that wide tiles still give every CU
// work.  Pass 1 is gemm_wlds writing exact int32 partial tiles into planes of a workspace;
// pass 2 (splitk_sum) adds the planes, in plane order (int32 addition is exact, so the sum is
// the unsplit accumulator bit for bit), and applies the same epilogue as every other
// schedule.  A tile's L2-to-CU traffic is (bm + bn) bytes per K byte, so at 32-128 tokens a
// 64x64 tile moves half of what 32x32 tiles do; the split restores the workgroup count the
// wide tile gives up.

// One thread per 4 consecutive output columns of one row.  XCD: pass 1 dealt each XCD the
// contiguous columns [x, x+1) * N/8 (xcd_col_tile with N/bn a multiple of 8), so its partial
// planes for those columns sit in that XCD's L2; workgroup b, which the dispatcher gives to
// XCD b % 8, sums columns of that XCD's range and reads them there.  Correct either way.
template <int Z, int EK, bool XCD>
__global__ void __launch_bounds__(256)
splitk_sum(const int32_t* __restrict__ ws, Epi e) {
  pin_args(e, ws);
  int64_t m, n;
  if constexpr (XCD) {
    const int qpr = e.N >> 5;  // quads a row within one XCD's columns
    const int64_t u = (int64_t)(blockIdx.x >> 3) * 256 + threadIdx.x;
    if (u >= (int64_t)e.M * qpr) return;
    m = u / qpr;
    n = (int64_t)(blockIdx.x & 7) * (e.N >> 3) + 4 * (u - m * qpr);
  } else {
    const int nq = e.N >> 2;
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= (int64_t)e.M * nq) return;
    m = q / nq;
    n = (q - m * nq) * 4;
  }
  // the epilogue operands and every partial are requested before any is used: one round trip
  const Cols4 cl = load_cols4<EK>(e, n);
  const float sam = load_sa<EK>(e, m);
  const int64_t plane = (int64_t)e.M * e.N;
  const int32_t* p = ws + m * e.N + n;
  v4i part[Z];
#pragma unroll
  for (int z = 0; z < Z; ++z) part[z] = *(const v4i*)(p + z * plane);
  v4i sum = part[0];
#pragma unroll
  for (int z = 1; z < Z; ++z) sum += part[z];
  store4s<EK>(e, m, n, sum, cl, sam);
}

int64_t wlds_split_workspace(const i8l_config& c, int64_t M, int64_t N) {
  return c.stages == 5 ? (int64_t)c.group_m * M * N * 4 : 0;
}

bool wlds_split_ok(const i8l_config& c, int64_t K) {
  if (c.stages != 5 || (c.group_m != 2 && c.group_m != 4 && c.group_m != 8)) return false;
  if (c.bn > 64 || c.warps < 1 || c.warps > 16 || c.bk <= 0) return false;
  bool built = false;
  for (auto t : kWlds)
    if (16 * t.mt == c.bm && t.nc == c.bn && 64 * t.ks == c.bk &&
        c.warps * 64 <= wlds_bound(t.mt, t.ks, t.nc) && wlds_multi_fits(t.mt, t.nc, t.ks))
      built = true;
  const int64_t part = (int64_t)c.bk * c.warps * c.group_m;
  if (!built || K <= 0 || K % part) return false;
  return wlds_lds_bytes(c, K / c.group_m) <= kMaxLds;
}

template <int Z, bool XCD>
hipError_t launch_splitk_sum_x(const int32_t* ws, const Epi& e, hipStream_t st) {
  const int64_t quads = (int64_t)e.M * (e.N / 4);
  const dim3 grid((unsigned)(XCD ? 8 * ((quads / 8 + 255) / 256) : (quads + 255) / 256));
  switch (epi_kind(e)) {
    case EK_BF16:
      hipLaunchKernelGGL((splitk_sum<Z, EK_BF16, XCD>), grid, dim3(256), 0, st, ws, e);
      break;
    case EK_BF16_BBF16:
      hipLaunchKernelGGL((splitk_sum<Z, EK_BF16_BBF16, XCD>), grid, dim3(256), 0, st, ws, e);
      break;
    default: hipLaunchKernelGGL((splitk_sum<Z, EK_ANY, XCD>), grid, dim3(256), 0, st, ws, e);
  }
  return hipGetLastError();
}

template <int Z>
hipError_t launch_splitk_sum(const int32_t* ws, const Epi& e, int nc, hipStream_t st) {
  const bool xcd = (e.N / nc) % 8 == 0 && e.N % 32 == 0;
  return xcd ? launch_splitk_sum_x<Z, true>(ws, e, st) : launch_splitk_sum_x<Z, false>(ws, e, st);
}

template <int MT, int NC, int KS>
hipError_t launch_wlds_part(const i8l_config& c, const int8_t* a, int64_t lda, const int8_t* b,
                            int64_t ldb, const Epi& e, int64_t K, hipStream_t st) {
  if constexpr (wlds_multi_fits(MT, NC, KS))
    return launch_wlds_steps<MT, NC, KS, EK_ANY>(c, a, lda, b, ldb, e, K / c.group_m,
                                                 c.group_m, st);
  return hipErrorInvalidValue;
}

hipError_t launch_wlds_split(const i8l_config& c, const int8_t* a, int64_t lda,
                             const int8_t* b, int64_t ldb, const Epi& e, int64_t K,
                             int32_t* ws, hipStream_t st) {
  Epi part = e;  // pass 1: raw int32 planes, ldc = N
  part.out = ws;
  part.ldc = e.N;
  part.out_dtype = I8L_I32;
  part.bias = nullptr;
  part.bias_dtype = I8L_DTYPE_NONE;
  part.sa_per_row = part.sb_per_col = 0;
  const int mt = c.bm / 16, nc = c.bn, ks = c.bk / 64;
  hipError_t err = hipErrorInvalidValue;
#define I8L_WLDS(MT_, NC_, KS_)                                                             \
  if (mt == MT_ && nc == NC_ && ks == KS_) err = launch_wlds_part<MT_, NC_, KS_>(c, a, lda, b, ldb, part, K, st); else
  I8L_WLDS(1, 16, 2) I8L_WLDS(1, 16, 4) I8L_WLDS(1, 16, 6) I8L_WLDS(1, 16, 8)
  I8L_WLDS(1, 8, 2) I8L_WLDS(1, 8, 4) I8L_WLDS(1, 8, 6) I8L_WLDS(1, 8, 8)
  I8L_WLDS(1, 4, 4) I8L_WLDS(1, 4, 8)
  I8L_WLDS(2, 16, 2) I8L_WLDS(2, 16, 4) I8L_WLDS(2, 8, 2) I8L_WLDS(2, 8, 4)
  I8L_WLDS(4, 16, 2) I8L_WLDS(4, 16, 4) I8L_WLDS(4, 8, 2) I8L_WLDS(4, 8, 4)
  I8L_WLDS(8, 16, 2) I8L_WLDS(8, 8, 2)
  I8L_WLDS(1, 32, 2) I8L_WLDS(1, 32, 4) I8L_WLDS(2, 32, 2) I8L_WLDS(2, 32, 4)
  I8L_WLDS(4, 32, 2) I8L_WLDS(4, 32, 4)
  I8L_WLDS(1, 64, 2) I8L_WLDS(2, 64, 2) I8L_WLDS(4, 64, 2) I8L_WLDS(1, 64, 4) I8L_WLDS(2, 64, 4)
  {}
#undef I8L_WLDS
  if (err != hipSuccess) return err;
  switch (c.group_m) {
    case 2: return launch_splitk_sum<2>(ws, e, c.bn, st);
    case 4: return launch_splitk_sum<4>(ws, e, c.bn, st);
    case 8: return launch_splitk_sum<8>(ws, e, c.bn, st);
  }
  return hipErrorInvalidValue;
}

// Persistent single-step tiles (stages 4): (MT, NC, KS, W), K = 64 * KS * W.  Two weight
// buffers and the reduction area must fit the LDS, and the activation fragments (4*KS*MT
// VGPRs) with the rest of a wave's state the register file (128 VGPRs at W = 16).
struct WldsPTile {
  int mt, nc, ks, w;
};
constexpr WldsPTile kWldsP[] = {{1, 16, 2, 16}, {2, 16, 2, 16}, {1, 32, 2, 16}, {1, 16, 4, 16},
                                {1, 16, 4, 8},  {2, 16, 4, 8},  {4, 16, 4, 8},  {1, 16, 8, 8},
                                {4, 16, 2, 16}, {8, 16, 4, 8},  {4, 32, 2, 8},  {1, 8, 2, 16},
                                {1, 8, 4, 16},  {1, 8, 8, 8},   {1, 8, 16, 4},  {1, 16, 16, 4},
                                {1, 8, 8, 4},   {1, 16, 8, 4},  {1, 8, 6, 16},  {2, 8, 6, 16},
                                {1, 8, 12, 8},  {1, 8, 4, 8}};

size_t wldsp_lds_bytes(int mt, int nc, int ks, int w) {
  const int nf = nc > 16 ? nc / 16 : 1;
  return (size_t)2 * w * nc * 64 * ks + (size_t)w * mt * nf * 1024;
}

// group_m is the number of workgroups a compute unit runs at once (1, 2 or 4): all of them
// must fit its LDS and its 2048 threads.
bool wldsp_ok(const i8l_config& c, int64_t K) {
  if (c.stages != 4 || c.bn > 32 ||
      (c.group_m != 1 && c.group_m != 2 && c.group_m != 4))
    return false;
  for (auto t : kWldsP)
    if (16 * t.mt == c.bm && t.nc == c.bn && 64 * t.ks == c.bk && t.w == c.warps)
      return K == (int64_t)c.bk * c.warps &&
             (size_t)c.group_m * wldsp_lds_bytes(t.mt, t.nc, t.ks, t.w) <= kMaxLds &&
             c.group_m * 64 * t.w <= 2048;
  return false;
}

// Compute units of the current device (cached per device; 256 if the query fails).
int cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 256;
  }
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      n <= 0) {
    (void)hipGetLastError();
    n = 256;
  }
  cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

template <int MT, int NC, int KS, int W, int EK, int ACT = kActPlain>
hipError_t launch_wldsp_k(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                          const Epi& e, int per_cu, hipStream_t st) {
  const size_t shm = wldsp_lds_bytes(MT, NC, KS, W);
  const int rows = (e.M + 16 * MT - 1) / (16 * MT);
  const int tiles = e.N / NC;
  const int per_row = std::max(1, per_cu * cu_count() / rows);  // per_cu workgroups a CU
  const dim3 grid((unsigned)std::min(tiles, per_row), (unsigned)rows);
  // the straight single-tile form where every workgroup has one tile, else the tile loop
  const bool loop = tiles > (int)grid.x;
  auto kern = loop ? gemm_wlds1p<MT, NC, KS, W, EK, ACT, true> : gemm_wlds1p<MT, NC, KS, W, EK, ACT, false>;
  static std::atomic<uint64_t> lds_done_loop{0}, lds_done_one{0};  // devices opted in on
  lds_opt_in((const void*)kern, shm, loop ? lds_done_loop : lds_done_one);
  hipLaunchKernelGGL(kern, grid, dim3(64 * W), shm, st, a, lda, b, ldb, e);
  return hipGetLastError();
}

template <int MT, int NC, int KS, int W>
hipError_t launch_wldsp_t(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                          const Epi& e, int per_cu, hipStream_t st) {
  switch (epi_kind(e)) {
    case EK_BF16: return launch_wldsp_k<MT, NC, KS, W, EK_BF16>(a, lda, b, ldb, e, per_cu, st);
    case EK_BF16_BBF16:
      return launch_wldsp_k<MT, NC, KS, W, EK_BF16_BBF16>(a, lda, b, ldb, e, per_cu, st);
    default: return launch_wldsp_k<MT, NC, KS, W, EK_ANY>(a, lda, b, ldb, e, per_cu, st);
  }
}

hipError_t launch_wldsp(const i8l_config& c, const int8_t* a, int64_t lda, const int8_t* b,
                        int64_t ldb, const Epi& e, hipStream_t st) {
  const int mt = c.bm / 16, nc = c.bn, ks = c.bk / 64, w = c.warps;
#define I8L_WLDSP(MT_, NC_, KS_, W_)                                                        \
  if (mt == MT_ && nc == NC_ && ks == KS_ && w == W_)                                        \
    return launch_wldsp_t<MT_, NC_, KS_, W_>(a, lda, b, ldb, e, c.group_m, st);
  I8L_WLDSP(1, 16, 2, 16) I8L_WLDSP(2, 16, 2, 16) I8L_WLDSP(1, 32, 2, 16) I8L_WLDSP(1, 16, 4, 16)
  I8L_WLDSP(1, 16, 4, 8) I8L_WLDSP(2, 16, 4, 8) I8L_WLDSP(4, 16, 4, 8) I8L_WLDSP(1, 16, 8, 8)
  I8L_WLDSP(4, 16, 2, 16) I8L_WLDSP(8, 16, 4, 8) I8L_WLDSP(4, 32, 2, 8) I8L_WLDSP(1, 8, 2, 16)
  I8L_WLDSP(1, 8, 4, 16) I8L_WLDSP(1, 8, 8, 8) I8L_WLDSP(1, 8, 16, 4) I8L_WLDSP(1, 16, 16, 4)
  I8L_WLDSP(1, 8, 8, 4) I8L_WLDSP(1, 16, 8, 4) I8L_WLDSP(1, 8, 6, 16) I8L_WLDSP(2, 8, 6, 16)
  I8L_WLDSP(1, 8, 12, 8) I8L_WLDSP(1, 8, 4, 8)
#undef I8L_WLDSP
  return hipErrorInvalidValue;
}

// The persistent single-step tiles with the SiLU-and-mul epilogue (one 16-row block, 8 or 16
// columns a tile, bf16 output with no bias or a bf16 bias).
// Every kWldsP tile of one 16-row block and 8 or 16 columns has its SiLU-epilogue instances
// in launch_wldsp_silu below (the GPU test of the epilogue walks the same list).
bool wldsp_silu_ok(const i8l_config& c, int64_t K) {
  return wldsp_ok(c, K) && c.bm == 16 && (c.bn == 8 || c.bn == 16);
}

template <int NC, int KS, int W, int ACT>
hipError_t launch_wldsp_silu_t(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                               const Epi& e, int per_cu, hipStream_t st) {
  switch (epi_kind(e)) {
    case EK_BF16: return launch_wldsp_k<1, NC, KS, W, EK_BF16, ACT>(a, lda, b, ldb, e, per_cu, st);
    case EK_BF16_BBF16:
      return launch_wldsp_k<1, NC, KS, W, EK_BF16_BBF16, ACT>(a, lda, b, ldb, e, per_cu, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_wldsp_silu(const i8l_config& c, const int8_t* a, int64_t lda, const int8_t* b,
                             int64_t ldb, const Epi& e, int round_silu, hipStream_t st) {
  const int nc = c.bn, ks = c.bk / 64, w = c.warps;
  if (c.bm != 16) return hipErrorInvalidValue;
#define I8L_WLDSP_SILU(NC_, KS_, W_)                                                        \
  if (nc == NC_ && ks == KS_ && w == W_)                                                     \
    return round_silu                                                                        \
        ? launch_wldsp_silu_t<NC_, KS_, W_, kActSiluRound>(a, lda, b, ldb, e, c.group_m, st) \
        : launch_wldsp_silu_t<NC_, KS_, W_, kActSilu>(a, lda, b, ldb, e, c.group_m, st);
  I8L_WLDSP_SILU(16, 2, 16) I8L_WLDSP_SILU(16, 4, 16) I8L_WLDSP_SILU(16, 4, 8)
  I8L_WLDSP_SILU(16, 8, 8) I8L_WLDSP_SILU(8, 2, 16) I8L_WLDSP_SILU(8, 4, 16)
  I8L_WLDSP_SILU(8, 8, 8) I8L_WLDSP_SILU(8, 16, 4) I8L_WLDSP_SILU(16, 16, 4)
  I8L_WLDSP_SILU(8, 8, 4) I8L_WLDSP_SILU(16, 8, 4) I8L_WLDSP_SILU(8, 6, 16)
  I8L_WLDSP_SILU(8, 12, 8) I8L_WLDSP_SILU(8, 4, 8)
#undef I8L_WLDSP_SILU
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

// Dynamic-quant decode tiles (gemm_wlds1_dq, one 16-token row block): (NC, KS, W) with
// K == 64 * KS * W.  The config's bm is 16 and its stages 3, as for gemm_wlds1.
struct DqTile {
  int nc, ks, w;
};
// {8, 8, 12}: 12 waves of 512-byte slices for K = 6144 (the down projection fed by the
// gate_up GEMM's SiLU-and-mul epilogue).
constexpr DqTile kDq[] = {{8, 2, 16}, {16, 2, 16}, {32, 2, 16}, {8, 4, 16}, {16, 4, 16},
                          {8, 8, 12}};
// The SiLU-and-mul form's tiles (gate_up rows of 2K values feeding K = 64 * KS * W): 12 waves
// of 512-byte slices take Qwen3-1.7B's K = 6144 (a slice of 384 bytes would not split the
// 8-value chunks of a row over the lanes).  One 16-token row block with at most 8 valid
// rows: the row values stay in registers.
constexpr DqTile kDqSilu[] = {{8, 8, 12}};
constexpr int kDqSiluMaxRows = 8;

size_t dq_lds_bytes(int nc, int ks, int W) {
  const int nf = nc > 16 ? nc / 16 : 1;
  // weights, the cross-wave sums, the row maxima, the 16-row code tiles
  return (size_t)W * nc * 64 * ks + (size_t)W * nf * 1024 + (size_t)W * 64 +
         (size_t)W * 16 * 64 * ks;
}

// Token rows a dynamic-quant tile takes: a 16-row block, built with up to 8 passes of
// 64 / (S/8) rows (so 8 rows for 512-byte slices).
int dq_max_rows(const i8l_config& c) { return std::min(16, 8 * (512 / c.bk)); }

bool dq_ok(const i8l_config& c, int64_t K) {
  if (c.stages != 3 || c.bm != 16) return false;
  for (auto t : kDq)
    if (t.nc == c.bn && 64 * t.ks == c.bk && t.w == c.warps)
      return K == (int64_t)64 * t.ks * t.w && dq_lds_bytes(t.nc, t.ks, t.w) <= kMaxLds;
  return false;
}

// The untuned choice: 16 waves that take K in one step each, 16 columns a workgroup (8 for
// narrow N); K = 6144 takes 12 waves of 512 bytes and 8 columns.
bool default_dq_config(int64_t N, int64_t K, i8l_config* c) {
  const int nc = (N % 16 == 0 && N / 16 >= 256) ? 16 : 8;
  for (int ks : {2, 4}) {
    const i8l_config t{16, nc, 64 * ks, 16, 3, 1};
    if (K == (int64_t)64 * ks * 16 && dq_ok(t, K)) {
      *c = t;
      return true;
    }
  }
  const i8l_config t{16, 8, 512, 12, 3, 1};
  if (N % 8 == 0 && dq_ok(t, K)) {
    *c = t;
    return true;
  }
  return false;
}

bool dq_silu_ok(const i8l_config& c, int64_t K) {
  if (c.stages != 3 || c.bm != 16) return false;
  for (auto t : kDqSilu)
    if (t.nc == c.bn && 64 * t.ks == c.bk && t.w == c.warps)
      return K == (int64_t)64 * t.ks * t.w && dq_lds_bytes(t.nc, t.ks, t.w) <= kMaxLds;
  return false;
}

bool default_dq_silu_config(int64_t N, int64_t K, i8l_config* c) {
  for (auto t : kDqSilu) {
    const i8l_config cand{16, t.nc, 64 * t.ks, t.w, 3, 1};
    if (N % t.nc == 0 && dq_silu_ok(cand, K)) {
      *c = cand;
      return true;
    }
  }
  return false;
}

int dq_silu_max_rows() { return kDqSiluMaxRows; }

template <int NC, int KS, int W, int P, int EK, int DT, int ACT>
hipError_t launch_dq_k(const uint16_t* x, int64_t ldx, int64_t up, const int8_t* b,
                       int64_t ldb, const Epi& e, float* sa_out, int precise, hipStream_t st) {
  auto kern = gemm_wlds1_dq<NC, KS, W, P, EK, DT, ACT>;
  const size_t shm = dq_lds_bytes(NC, KS, W);
  static std::atomic<uint64_t> lds_done{0};  // devices this kernel is opted in on
  lds_opt_in((const void*)kern, shm, lds_done);
  const dim3 grid(e.N / NC, (e.M + 15) / 16);
  hipLaunchKernelGGL(kern, grid, dim3(64 * W), shm, st, x, ldx, up, b, ldb, e, sa_out, precise);
  return hipGetLastError();
}

template <int NC, int KS, int W, int P, int ACT>
hipError_t launch_dq_p(int act_dtype, const uint16_t* x, int64_t ldx, int64_t up,
                       const int8_t* b, int64_t ldb, const Epi& e, float* sa_out, int precise,
                       hipStream_t st) {
  if (act_dtype == I8L_F16)
    return launch_dq_k<NC, KS, W, P, EK_ANY, I8L_F16, ACT>(x, ldx, up, b, ldb, e, sa_out,
                                                           precise, st);
  switch (epi_kind(e)) {
    case EK_BF16:
      return launch_dq_k<NC, KS, W, P, EK_BF16, I8L_BF16, ACT>(x, ldx, up, b, ldb, e, sa_out,
                                                               precise, st);
    case EK_BF16_BBF16:
      return launch_dq_k<NC, KS, W, P, EK_BF16_BBF16, I8L_BF16, ACT>(x, ldx, up, b, ldb, e,
                                                                     sa_out, precise, st);
    default:
      return launch_dq_k<NC, KS, W, P, EK_ANY, I8L_BF16, ACT>(x, ldx, up, b, ldb, e, sa_out,
                                                              precise, st);
  }
}

// Passes of the quantizer prologue: ceil(rows / RPP) for the block's valid rows, taken as
// the next power of two (P in {1, 2, 4, ...}, at most 16 rows, or MAXR for the SiLU form).
template <int NC, int KS, int W, int ACT, int MAXR>
hipError_t launch_dq_t(int act_dtype, const uint16_t* x, int64_t ldx, int64_t up,
                       const int8_t* b, int64_t ldb, const Epi& e, float* sa_out, int precise,
                       hipStream_t st) {
  constexpr int RPP = 64 / (8 * KS);
  const int rows = e.M < 16 ? e.M : 16;
  const int need = (rows + RPP - 1) / RPP;
  if (need <= 1)
    return launch_dq_p<NC, KS, W, 1, ACT>(act_dtype, x, ldx, up, b, ldb, e, sa_out, precise,
                                          st);
  if (need <= 2)
    return launch_dq_p<NC, KS, W, 2, ACT>(act_dtype, x, ldx, up, b, ldb, e, sa_out, precise,
                                          st);
  if constexpr (MAXR / RPP >= 4)
    if (need <= 4)
      return launch_dq_p<NC, KS, W, 4, ACT>(act_dtype, x, ldx, up, b, ldb, e, sa_out, precise,
                                            st);
  if constexpr (MAXR / RPP >= 8)
    if (need <= 8)
      return launch_dq_p<NC, KS, W, 8, ACT>(act_dtype, x, ldx, up, b, ldb, e, sa_out, precise,
                                            st);
  return hipErrorInvalidValue;
}

hipError_t launch_dq(const i8l_config& c, int act_dtype, const uint16_t* x, int64_t ldx,
                     const int8_t* b, int64_t ldb, const Epi& e, float* sa_out, int precise,
                     hipStream_t st) {
  const int nc = c.bn, ks = c.bk / 64, W = c.warps;
#define I8L_DQ(NC_, KS_, W_)                                                                \
  if (nc == NC_ && ks == KS_ && W == W_)                                                    \
    return launch_dq_t<NC_, KS_, W_, kActPlain, 16>(act_dtype, x, ldx, 0, b, ldb, e, sa_out, \
                                                    precise, st);
  I8L_DQ(8, 2, 16) I8L_DQ(16, 2, 16) I8L_DQ(32, 2, 16) I8L_DQ(8, 4, 16) I8L_DQ(16, 4, 16)
  I8L_DQ(8, 8, 12)
#undef I8L_DQ
  return hipErrorInvalidValue;
}

hipError_t launch_dq_silu(const i8l_config& c, int act_dtype, int round_silu,
                          const uint16_t* gate_up, int64_t ldgu, int64_t up, const int8_t* b,
                          int64_t ldb, const Epi& e, float* sa_out, int precise,
                          hipStream_t st) {
  if (e.M > kDqSiluMaxRows) return hipErrorInvalidValue;
  const int nc = c.bn, ks = c.bk / 64, W = c.warps;
#define I8L_DQS(NC_, KS_, W_)                                                               \
  if (nc == NC_ && ks == KS_ && W == W_)                                                    \
    return round_silu                                                                       \
        ? launch_dq_t<NC_, KS_, W_, kActSiluRound, kDqSiluMaxRows>(                         \
              act_dtype, gate_up, ldgu, up, b, ldb, e, sa_out, precise, st)                 \
        : launch_dq_t<NC_, KS_, W_, kActSilu, kDqSiluMaxRows>(act_dtype, gate_up, ldgu, up, \
                                                              b, ldb, e, sa_out, precise,   \
                                                              st);
  I8L_DQS(8, 8, 12)
#undef I8L_DQS
  return hipErrorInvalidValue;
}

}  // namespace i8l
