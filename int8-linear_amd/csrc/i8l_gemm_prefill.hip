// Prefill schedules of the W8A8 GEMM (BM x BN macro tiles of 64 to 256, v_mfma_i32_32x32x32_i8),
// their tile tables and launchers: staged (LDS double buffer through registers), dma (a
// ring of direct-to-LDS buffers) and dmap (the ring with the LDS fragment reads overlapped
// with the MFMAs).
#include "i8l_gemm.h"

namespace i8l {

// ------------------------------------------------------------------ tile epilogue
// Output of a BM x BN macro tile from the accumulators of WM x WN waves.  For 16-bit outputs
// the values are computed in the fragment layout (scales and bias fetched with vector loads),
// written to LDS as a row-major tile with 16 bytes of padding per row (so the 32 rows one
// store instruction touches spread over the banks), and copied out with 16-byte stores,
// 64 lanes covering consecutive columns of consecutive rows.  int32 and fp32 outputs take the
// same staging half of the tile's rows at a time (BM/2 rows of 4*BN bytes fit the area).  The
// copies out are non-temporal stores.  `lds` must hold BM * (2*BN + 16) bytes and every wave
// must be done with its previous LDS contents.
template <int BM, int BN, int WM, int WN>
constexpr int tile_epilogue_lds_bytes() { return BM * (2 * BN + 16); }

// The scales and bias of a wave's FA x 4 column quads (column n = nb + 32a + 8q), every load
// issued before any is used: one memory round trip.  BD (the bias dtype) and SBC (per-column
// scale_b) are fixed per specialization, so no branch separates the loads.
template <int FA, int BD, bool SBC>
__device__ __forceinline__ void load_tile_cols_k(const Epi& e, int64_t nb, Cols4 (&cl)[FA][4]) {
  float4 sbv[FA][4];
  float sb0 = 0.0f;
  uint2 bh[FA][4];
  float4 bf[FA][4];
#pragma unroll
  for (int a = 0; a < FA; ++a)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t n = nb + 32 * a + 8 * q;
      if constexpr (SBC) sbv[a][q] = *(const float4*)(e.sb + n);
      if constexpr (BD == I8L_F32) bf[a][q] = *(const float4*)((const float*)e.bias + n);
      if constexpr (BD == I8L_BF16 || BD == I8L_F16)
        bh[a][q] = *(const uint2*)((const uint16_t*)e.bias + n);
    }
  if constexpr (!SBC) sb0 = e.sb[0];
#pragma unroll
  for (int a = 0; a < FA; ++a)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      Cols4& c = cl[a][q];
      if constexpr (SBC) {
        c.sb[0] = sbv[a][q].x, c.sb[1] = sbv[a][q].y, c.sb[2] = sbv[a][q].z, c.sb[3] = sbv[a][q].w;
      } else {
        c.sb[0] = c.sb[1] = c.sb[2] = c.sb[3] = sb0;
      }
      if constexpr (BD == I8L_F32) {
        c.bias[0] = bf[a][q].x, c.bias[1] = bf[a][q].y, c.bias[2] = bf[a][q].z,
        c.bias[3] = bf[a][q].w;
      } else if constexpr (BD == I8L_BF16 || BD == I8L_F16) {
        const uint32_t w[4] = {bh[a][q].x & 0xffffu, bh[a][q].x >> 16, bh[a][q].y & 0xffffu,
                               bh[a][q].y >> 16};
#pragma unroll
        for (int r = 0; r < 4; ++r)
          c.bias[r] = BD == I8L_BF16 ? bf16_bits_to_f32(w[r]) : f16_bits_to_f32(w[r]);
      } else {
        // no bias: -0, the identity of IEEE addition (x + -0 == x for every x, -0 and NaN
        // included), so the epilogue adds the bias without a test
        c.bias[0] = c.bias[1] = c.bias[2] = c.bias[3] = -0.0f;
      }
    }
}

template <int FA, bool SBC>
__device__ __forceinline__ void load_tile_cols_s(const Epi& e, int64_t nb, Cols4 (&cl)[FA][4]) {
  switch (e.bias_dtype) {
    case I8L_DTYPE_NONE: load_tile_cols_k<FA, I8L_DTYPE_NONE, SBC>(e, nb, cl); break;
    case I8L_BF16: load_tile_cols_k<FA, I8L_BF16, SBC>(e, nb, cl); break;
    case I8L_F16: load_tile_cols_k<FA, I8L_F16, SBC>(e, nb, cl); break;
    default: load_tile_cols_k<FA, I8L_F32, SBC>(e, nb, cl); break;
  }
}

template <int BM, int BN, int WM, int WN, int FA, int FB>
__device__ __forceinline__ void tile_epilogue(const Epi& e, v16i (&acc)[FA][FB], int8_t* lds,
                                              int64_t m0, int64_t n0, int wm, int wn, int lane,
                                              int tid) {
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int T = 64 * WM * WN;
  const int frow = lane & 31, fhalf = lane >> 5;
  const bool out4 = e.out_dtype == I8L_I32 || e.out_dtype == I8L_F32;
  float sam[FB];
  Cols4 cls[FA][4];
  if (e.out_dtype != I8L_I32) {
#pragma unroll
    for (int b = 0; b < FB; ++b) {
      const int64_t m = m0 + wm * TM + b * 32 + frow;
      sam[b] = load_sa(e, m < e.M ? m : 0);
    }
    if (e.sb_per_col)
      load_tile_cols_s<FA, true>(e, n0 + wn * TN + 4 * fhalf, cls);
    else
      load_tile_cols_s<FA, false>(e, n0 + wn * TN + 4 * fhalf, cls);
  }
  // The value of element (a, b, q, i) before its cast: acc * scale_a * scale_b + bias in
  // fp32, left to right (a missing bias is -0, the identity of the addition).
  auto value = [&](int a, int b, int q, int i) {
    float v = (float)acc[a][b][4 * q + i];
    v = v * sam[b];
    v = v * cls[a][q].sb[i];
    return v + cls[a][q].bias[i];
  };
  if (out4) {
    // 4-byte outputs (int32 raw, fp32): staged through LDS half the tile's rows at a time
    // (BM/2 rows of 4*BN bytes fit the area of the 16-bit staging) and written in whole
    // 16-byte chunks by consecutive lanes, as the 16-bit outputs are.  A wave's TM rows lie
    // in one half (WM is even).
    static_assert(WM % 2 == 0, "a wave's rows must lie in one half of the tile");
    constexpr int HR = BM / 2;
    constexpr int PITCH4 = 4 * BN + 16;
    constexpr int CPR4 = BN / 4;                 // 16-byte chunks per output row
    static_assert((HR * CPR4) % T == 0, "half-tile rows do not split over the threads");
    const bool raw = e.out_dtype == I8L_I32;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if ((wm * TM) / HR == h) {
#pragma unroll
        for (int a = 0; a < FA; ++a)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int c = wn * TN + a * 32 + 8 * q + 4 * fhalf;
#pragma unroll
            for (int b = 0; b < FB; ++b) {
              const int r = wm * TM + b * 32 + frow - h * HR;
              v4i v;
              if (raw) {
                v = v4i{acc[a][b][4 * q], acc[a][b][4 * q + 1], acc[a][b][4 * q + 2],
                        acc[a][b][4 * q + 3]};
              } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = __float_as_int(value(a, b, q, i));
              }
              *(v4i*)(lds + r * PITCH4 + 4 * c) = v;
            }
          }
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < HR * CPR4 / T; ++j) {
        const int i = tid + j * T;
        const int r = i / CPR4, c4 = i % CPR4;
        const int64_t m = m0 + h * HR + r;
        const v4i v = *(const v4i*)(lds + r * PITCH4 + 16 * c4);
        if (m < e.M) __builtin_nontemporal_store(v, (v4i*)((int32_t*)e.out + m * e.ldc + n0 + 4 * c4));
      }
      if (h == 0) __syncthreads();   // the second half reuses the area
    }
    return;
  }
  constexpr int PITCH = 2 * BN + 16;  // bytes per LDS row (16-byte aligned)
  // the output dtype is uniform: one copy of the conversion loop per dtype, no per-value select
  auto stage = [&](auto pack2) {
#pragma unroll
    for (int a = 0; a < FA; ++a) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c = wn * TN + a * 32 + 8 * q + 4 * fhalf;  // column within the tile
#pragma unroll
        for (int b = 0; b < FB; ++b) {
          const int r = wm * TM + b * 32 + frow;             // row within the tile
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = value(a, b, q, i);
          *(uint2*)(lds + r * PITCH + 2 * c) = make_uint2(pack2(v[0], v[1]), pack2(v[2], v[3]));
        }
      }
    }
  };
  if (e.out_dtype == I8L_BF16)
    stage([](float x, float y) { return f32x2_to_bf16x2_bits(x, y); });
  else
    stage([](float x, float y) {
      return (uint32_t)f32_to_f16_bits(x) | ((uint32_t)f32_to_f16_bits(y) << 16);
    });
  // Other waves read these stores: the barrier must also wait for them to complete
  // (s_barrier alone does not, and with two workgroups a CU sharing the LDS they do lag).
  __syncthreads();
  constexpr int CPR = BN / 8;                  // 16-byte chunks per output row
  static_assert((BM * CPR) % T == 0, "tile rows do not split over the threads");
#pragma unroll
  for (int j = 0; j < BM * CPR / T; ++j) {
    const int i = tid + j * T;
    const int r = i / CPR, c8 = i % CPR;
    const int64_t m = m0 + r;
    const v4i v = *(const v4i*)(lds + r * PITCH + 16 * c8);
    // the output is written once and read by the next operation, not by this one: stream it
    // past the caches, which keep the operand panels the other tiles still read
    if (m < e.M) __builtin_nontemporal_store(v, (v4i*)((uint16_t*)e.out + m * e.ldc + n0 + 8 * c8));
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
  pin_args(e, A, lda, B, ldb, K, group_m);
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

// The same with lgkmcnt = 0 as well: this wave's LDS reads (and scalar loads) have returned.
template <int N>
__device__ __forceinline__ void wait_vmcnt_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

template <int BM, int BN, int BK, int WM, int WN, int S>
__global__ void __launch_bounds__(64 * WM * WN)
gemm_dma(const int8_t* __restrict__ A, int64_t lda, const int8_t* __restrict__ B,
         int64_t ldb, Epi e, int K, int group_m) {
  pin_args(e, A, lda, B, ldb, K, group_m);
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
// its own fragment reads of step t (lgkmcnt 0: the last substep's fragments are in registers,
// so it is done with step t's buffer) and for its DMA of step t+1 (vmcnt); the workgroup
// barrier then makes step t+1 visible and frees step t's buffer, and step t+S is requested
// into it.  So all S buffers of the ring hold requested steps: step t+1 was requested S-1
// steps of work before it is needed, and S = 2 is a double buffer.  The last substep's MFMAs
// then overlap the reads of step t+1's first substep.  The LDS traffic of each substep hides
// under the matrix work of the one before.
template <int BM, int BN, int BK, int WM, int WN, int S>
__global__ void __launch_bounds__(64 * WM * WN)
gemm_dmap(const int8_t* __restrict__ A, int64_t lda, const int8_t* __restrict__ B,
          int64_t ldb, Epi e, int K, int group_m) {
  pin_args(e, A, lda, B, ldb, K, group_m);
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
  static_assert(S >= 2, "the ring needs at least two buffers");

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
  // Steps requested before the wait in step t: 0 .. t+S-1; step t+1 must be complete, and
  // this wave's reads of step t's buffer done before the barrier lets it be refilled.
  auto turn = [&](int t) {
    wait_vmcnt_lgkm0<J * (S - 2)>();
    lds_barrier();
    dma(t + S);
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
  for (int t = 0; t < S; ++t) dma(t);
  wait_vmcnt<J * (S - 1)>();
  lds_barrier();
  rd(f0a, f0b, 0, 0);
  for (int t = 0; t + 1 < KT; ++t) kstep(t, true);
  kstep(KT - 1, false);
  wait_vmcnt<0>();
  lds_barrier();
  tile_epilogue<BM, BN, WM, WN, FA, FB>(e, acc, lds, m0, n0, wm, wn, lane, tid);
}

// ------------------------------------------------------------------ host side
struct StagedTile {
  int bm, bn, bk, wm, wn;
};

// (BM, BN, BK, WM, WN); the waves of a workgroup are laid out WM (tokens) x WN (columns).
// (256x256 tiles with 4 waves, or with 128-byte K steps, spill the register file and are
// not built.)
constexpr StagedTile kStaged[] = {{128, 128, 64, 2, 2},  {256, 128, 64, 2, 2},
                                  {128, 256, 64, 2, 2},  {128, 128, 128, 2, 2},
                                  {256, 256, 64, 2, 4},  {256, 128, 64, 2, 4},
                                  {128, 256, 64, 2, 4},  {256, 128, 128, 2, 4},
                                  {128, 256, 128, 2, 4}};

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

// Direct-to-LDS tiles with the fragment reads overlapped with the MFMAs (gemm_dmap): the
// config's `stages` is the ring depth S plus 8.
constexpr DmaTile kDmap[] = {{256, 256, 64, 2, 4, 3}, {256, 256, 64, 2, 4, 4},
                             {256, 256, 64, 2, 4, 5}, {256, 128, 64, 2, 4, 4},
                             {128, 256, 64, 2, 4, 4}, {128, 256, 128, 2, 4, 3},
                             {256, 128, 128, 2, 4, 3}, {128, 128, 64, 2, 2, 4},
                             {128, 128, 128, 2, 2, 4}, {64, 128, 128, 2, 2, 4},
                             {64, 256, 128, 2, 4, 3}, {64, 128, 64, 2, 2, 6},
                             {64, 128, 128, 2, 2, 6}, {64, 64, 128, 2, 2, 4},
                             {128, 64, 128, 2, 2, 4}, {128, 384, 64, 2, 4, 3},
                             {128, 384, 64, 2, 4, 4}, {128, 192, 64, 2, 2, 4},
                             {256, 192, 64, 2, 2, 4}, {64, 192, 64, 2, 2, 4},
                             {64, 192, 128, 2, 2, 4}, {256, 256, 128, 2, 4, 2},
                             {256, 128, 128, 2, 4, 2}, {128, 256, 128, 2, 4, 2},
                             {256, 192, 128, 4, 2, 2}};

int dmap_index(const i8l_config& c) {
  if (c.stages < 2 + kPipelined || c.group_m < 1) return -1;
  for (int i = 0; i < (int)(sizeof(kDmap) / sizeof(kDmap[0])); ++i) {
    const auto& t = kDmap[i];
    if (t.bm == c.bm && t.bn == c.bn && t.bk == c.bk && t.wm * t.wn == c.warps &&
        t.s + kPipelined == c.stages)
      return i;
  }
  return -1;
}

int dma_index(const i8l_config& c) {
  if (c.stages < 3 || c.group_m < 1) return -1;
  for (int i = 0; i < (int)(sizeof(kDma) / sizeof(kDma[0])); ++i) {
    const auto& t = kDma[i];
    if (t.bm == c.bm && t.bn == c.bn && t.bk == c.bk && t.wm * t.wn == c.warps && t.s == c.stages)
      return i;
  }
  return -1;
}

int staged_index(const i8l_config& c) {
  if (c.stages != 2 || c.group_m < 1) return -1;
  for (int i = 0; i < (int)(sizeof(kStaged) / sizeof(kStaged[0])); ++i) {
    const auto& t = kStaged[i];
    if (t.bm == c.bm && t.bn == c.bn && t.bk == c.bk && t.wm * t.wn == c.warps) return i;
  }
  return -1;
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
    case 15: return launch_dmap_t<128, 384, 64, 2, 4, 3>(a, lda, b, ldb, e, K, c.group_m, st);
    case 16: return launch_dmap_t<128, 384, 64, 2, 4, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 17: return launch_dmap_t<128, 192, 64, 2, 2, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 18: return launch_dmap_t<256, 192, 64, 2, 2, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 19: return launch_dmap_t<64, 192, 64, 2, 2, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 20: return launch_dmap_t<64, 192, 128, 2, 2, 4>(a, lda, b, ldb, e, K, c.group_m, st);
    case 21: return launch_dmap_t<256, 256, 128, 2, 4, 2>(a, lda, b, ldb, e, K, c.group_m, st);
    case 22: return launch_dmap_t<256, 128, 128, 2, 4, 2>(a, lda, b, ldb, e, K, c.group_m, st);
    case 23: return launch_dmap_t<128, 256, 128, 2, 4, 2>(a, lda, b, ldb, e, K, c.group_m, st);
    case 24: return launch_dmap_t<256, 192, 128, 4, 2, 2>(a, lda, b, ldb, e, K, c.group_m, st);
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

}  // namespace i8l
