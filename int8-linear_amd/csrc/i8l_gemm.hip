// W8A8 scaled matmul for MI355X (gfx950): the C entry points, the schedule dispatch and the
// library's default configuration.  The schedules live in i8l_gemm_decode.hip (decode,
// weights streamed or copied through LDS) and i8l_gemm_prefill.hip (macro tiles); the
// generic kernel below takes any strides and alignment and runs only when the operands do
// not meet the fast schedules' layout requirements (an N-contiguous weight, a transposed or
// unaligned activation, strides past 32 bits).
#include "i8l_gemm.h"

namespace i8l {

// ------------------------------------------------------------------ generic schedule
// Any strides, any alignment, any M, N, K (K = 0 included).  A workgroup of 4 waves computes
// a 64 x 64 output tile in 64-byte K steps: the A and B tiles are gathered byte by byte into
// LDS as [row][k] and [column][k] (zeros past M, N, K), with the lanes walking whichever index
// of each operand has unit stride so the global reads coalesce, then each wave multiplies
// its 16 token rows by the 4 column blocks with v_mfma_i32_16x16x64_i8, the fragment layout
// of the decode schedules.  Outputs go through the scalar epilogue (any output stride).
__global__ void __launch_bounds__(256)
gemm_generic(const int8_t* __restrict__ A, int64_t sam, int64_t sak, const int8_t* __restrict__ B,
             int64_t sbk, int64_t sbn, Epi e, int64_t K) {
  __shared__ __attribute__((aligned(16))) int8_t As[64 * 64];
  __shared__ __attribute__((aligned(16))) int8_t Bs[64 * 64];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r16 = lane & 15, grp = lane >> 4;
  const int64_t ntn = (e.N + 63) / 64;  // column tiles; the grid is tiles of N x tiles of M
  const int64_t m0 = (int64_t)(blockIdx.x / ntn) * 64, n0 = (int64_t)(blockIdx.x % ntn) * 64;
  const bool a_k = sak == 1, b_k = sbk == 1 || sbn != 1;
  v4i acc[4] = {};
  for (int64_t k0 = 0; k0 < K; k0 += 64) {
#pragma unroll 4
    for (int i = 0; i < 16; ++i) {
      const int idx = i * 256 + t;  // 0..4095: (row, k) of the 64 x 64 tile
      const int hi = idx >> 6, lo = idx & 63;
      const int ra = a_k ? hi : lo, ka = a_k ? lo : hi;
      const int64_t m = m0 + ra, ka_g = k0 + ka;
      As[ra * 64 + ka] = (m < e.M && ka_g < K) ? A[m * sam + ka_g * sak] : (int8_t)0;
      const int cb = b_k ? hi : lo, kb = b_k ? lo : hi;
      const int64_t n = n0 + cb, kb_g = k0 + kb;
      Bs[cb * 64 + kb] = (n < e.N && kb_g < K) ? B[kb_g * sbk + n * sbn] : (int8_t)0;
    }
    __syncthreads();
    const v4i a = *(const v4i*)(As + (16 * wave + r16) * 64 + 16 * grp);
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      const v4i b = *(const v4i*)(Bs + (16 * f + r16) * 64 + 16 * grp);
      acc[f] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b, a, acc[f], 0, 0, 0);
    }
    __syncthreads();
  }
  const int64_t m = m0 + 16 * wave + r16;
  if (m >= e.M) return;
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t n = n0 + 16 * f + 4 * grp + r;
      if (n < e.N) store1(e, m, n, acc[f][r]);
    }
}

void default_config(int64_t M, int64_t N, int64_t K, i8l_config* c) {
  *c = i8l_config{0, 0, 0, 0, 0, 1};
  if (M <= 32 && K % 128 == 0) {
    const int mt = M <= 16 ? 1 : 2;
    // Many column tiles (N/16 >= 512) from 9 tokens: the persistent single-step tile with two
    // workgroups a CU, which loads the activations once a workgroup instead of once a tile.
    if (M > 8 && N % 16 == 0 && N / 16 >= 512) {
      const i8l_config p = K == 4096 ? i8l_config{16 * mt, 8, 512, 8, 4, 2}
                                     : i8l_config{16 * mt, 16, 256, 8, 4, 2};
      if (wldsp_ok(p, K)) {
        *c = p;
        return;
      }
    }
    // weights through LDS: 16 (or, for narrow N, 8) columns a workgroup, the K split over
    // up to 16 waves in one or more steps of up to 512 bytes
    const int nc = (N % 16 == 0 && N / 16 >= 256) ? 16 : (N % 8 == 0 ? 8 : 4);
    const int64_t k64 = K / 64;
    const int kss[] = {8, 6, 4, 2};
    // first choice: every wave's slice is one step (8, 16 or 4 waves); else 16 waves with
    // the largest step that divides their slices
    for (int W : {8, 16, 4})
      for (int ks : kss) {
        const i8l_config t{16 * mt, nc, 64 * ks, W, 3, 1};
        if (k64 == (int64_t)W * ks && wlds_ok(t, K)) {
          *c = t;
          return;
        }
      }
    for (int ks : kss) {
      const i8l_config t{16 * mt, nc, 64 * ks, 16, 3, 1};
      if (wlds_ok(t, K)) {
        *c = t;
        return;
      }
    }
  }
  // 129 tokens and more, and from 33 tokens on wide N (K a multiple of 128): the overlapped-
  // ring tile with the least (waves of workgroups, one a CU) x (one wave's time).  kRing holds
  // each tile's time for one wave, relative to the 64x64 tile's 2.08 ns per K byte, the
  // median over 15 weight shapes (K 2048-28672, N 2048-57344) at 48-4096 tokens on MI355X.
  // Small tiles win while there are few tokens (more workgroups), large ones once every tile
  // size fills the CUs (fewer operand re-reads); a last wave of a few workgroups costs as much
  // as a full one, and of two tiles within 1% of each other the one with fewer waves wins
  // (each wave boundary drains the ring).  Over those shapes the pick was within 9% of the
  // fastest of these tiles, 0.2% on the geometric mean (the costs fitted on half the shapes
  // picked within 1.2% on the other half).
  struct RingTile {
    int bm, bn, warps, stages, group_m, cost;
  };
  static constexpr RingTile kRing[] = {
      {64, 64, 4, 4 + kPipelined, 8, 100},   {128, 64, 4, 4 + kPipelined, 8, 165},
      {64, 128, 4, 4 + kPipelined, 8, 178},  {128, 128, 4, 4 + kPipelined, 8, 249},
      {64, 256, 8, 3 + kPipelined, 8, 285},  {256, 128, 8, 3 + kPipelined, 8, 369},
      {128, 256, 8, 3 + kPipelined, 8, 384}, {256, 192, 8, 2 + kPipelined, 4, 555},
      {256, 256, 8, 2 + kPipelined, 4, 570}};
  if (K % 128 == 0 && N % 64 == 0 && (M > 128 || (M > 32 && N >= 8192))) {
    const int64_t cus = cu_count();
    int64_t best = -1, best_waves = 0;
    for (const auto& t : kRing) {
      if (N % t.bn != 0) continue;
      const int64_t waves = (((M + t.bm - 1) / t.bm) * (N / t.bn) + cus - 1) / cus;
      const int64_t cost = t.cost * waves;
      if (best < 0 || cost * 100 < best * 99 || (cost * 100 <= best * 101 && waves < best_waves)) {
        best = cost;
        best_waves = waves;
        *c = i8l_config{t.bm, t.bn, 128, t.warps, t.stages, t.group_m};
      }
    }
    return;
  }
  // 17 to 128 tokens: weights through LDS in 32-token x 32-column tiles (several row
  // blocks above 32 tokens), 16 waves of one 128-byte step when K is 2048, else 4 waves
  // stepping through their K slices.
  if (M <= 128 && N % 32 == 0 && K % 128 == 0) {
    const i8l_config one{32, 32, 128, 16, 3, 1};
    const i8l_config steps{32, 32, K % 1024 == 0 ? 256 : 128, 4, 3, 1};
    if (K == 2048 && N < 8192 && wlds_ok(one, K)) {
      *c = one;
      return;
    }
    if (wlds_ok(steps, K)) {
      *c = steps;
      return;
    }
  }
  // N not a multiple of 16: the 8-column (at most 32-token) or 4-column (16-token) streaming
  // tiles, several row blocks if M needs them.
  const int sbn = N % 16 == 0 ? 16 : N % 8 == 0 ? 8 : 4;
  const int smt_max = sbn == 16 ? 8 : sbn == 8 ? 2 : 1;
  if (M <= 128) {
    const int mt = std::min(M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8, smt_max);
    // enough waves that each owns only a few 64-byte K steps, as many as fit a workgroup
    int W = stream_max_threads(mt, 1) / 64;
    while (W > 1 && (K % (64 * W) != 0 || K / (64 * W) < 4 || W * mt * 1024 > 96 * 1024)) W /= 2;
    c->bm = 16 * mt;
    c->bn = sbn;
    c->warps = W;
    c->bk = 64 * W;
    c->stages = 1;
    return;
  }
  // Prefill with K not a multiple of 128 (or N not of 64): direct-to-LDS macro tiles with the
  // fragment reads overlapped with the MFMAs, 256x256 in 64-byte K steps when N allows,
  // 128x128 tiles below.
  c->group_m = 8;
  if (N % 256 == 0 && K % 64 == 0 && M > 1024) {
    *c = i8l_config{256, 256, 64, 8, 12, 4};
  } else if (N % 128 == 0 && K % 64 == 0) {
    *c = i8l_config{128, 128, 64, 4, 12, 8};
  } else {
    // narrow or odd shapes: the weight-streaming tile, one 128-token row block at a time
    // (32 or 16 tokens for N not a multiple of 16)
    int W = stream_max_threads(smt_max, 1) / 64;
    while (W > 1 && K % (64 * W) != 0) W /= 2;
    *c = i8l_config{16 * smt_max, sbn, 64 * W, W, 1, 1};
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
      !wlds_ok(c, K) && !wldsp_ok(c, K) && !wlds_split_ok(c, K)) {
    set_error("config %dx%dx%d w%d s%d g%d is not built into this library", c.bm, c.bn,
              c.bk, c.warps, c.stages, c.group_m);
    return I8L_UNSUPPORTED;
  }
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) {
    set_error("sizes beyond 2^31 are not supported");
    return I8L_UNSUPPORTED;
  }
  return I8L_OK;
}

extern "C" int64_t i8l_w8a8_mm_workspace_bytes(int64_t M, int64_t N, int64_t K,
                                               const i8l_config* cfg) {
  if (!cfg || M <= 0 || N <= 0 || !wlds_split_ok(*cfg, K)) return 0;
  return wlds_split_workspace(*cfg, M, N);
}

namespace i8l {

// The GEMM behind every entry point: validation, then the schedule of the config.  `ws` is
// the split of K's workspace (NULL, 0 when the caller has none).
int w8a8_mm(const int8_t* a, int64_t stride_am, int64_t stride_ak, const int8_t* b,
            int64_t stride_bk, int64_t stride_bn, const float* scale_a, int64_t scale_a_len,
            const float* scale_b, int64_t scale_b_len, const void* bias, int32_t bias_dtype,
            void* out, int64_t stride_cm, int32_t out_dtype, int64_t M, int64_t N, int64_t K,
            void* ws, int64_t ws_bytes, const i8l_config* cfg, void* stream,
            const char* who) {
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
  // the weights-through-LDS schedules keep in-tile row offsets (< 128 token rows, < 64
  // weight rows) in 32 bits; larger strides take the generic kernel
  const bool wlds = c.stages >= 3 && c.stages <= 5 && c.bn <= 64;
  const bool small_strides = stride_am <= INT32_MAX / 128 && stride_bn <= INT32_MAX / 64;
  if (fast && wlds && small_strides && c.stages == 5) {
    const int64_t need = wlds_split_workspace(c, M, N);
    if (!ws) {
      set_error("%s: config %dx%dx%d w%d s%d g%d splits K and needs a %lld-byte workspace "
                "(i8l_w8a8_mm_ws)", who, c.bm, c.bn, c.bk, c.warps, c.stages, c.group_m,
                (long long)need);
      return I8L_UNSUPPORTED;
    }
    if (ws_bytes < need || !aligned16(ws)) {
      set_error("%s: the workspace must be 16-byte aligned and hold %lld bytes (got %lld)",
                who, (long long)need, (long long)ws_bytes);
      return I8L_INVALID_ARG;
    }
  }
  hipError_t err;
  if (!fast || (wlds && !small_strides)) {
    const int64_t tiles = ((N + 63) / 64) * ((M + 63) / 64);
    if (tiles > INT32_MAX) {
      set_error("%s: %lld x %lld is too large for the generic kernel", who, (long long)M,
                (long long)N);
      return I8L_UNSUPPORTED;
    }
    const dim3 grid((unsigned)tiles);
    hipLaunchKernelGGL(gemm_generic, grid, dim3(256), 0, hs, a, stride_am, stride_ak, b,
                       stride_bk, stride_bn, e, K);
    err = hipGetLastError();
  } else if (c.stages == 1) {
    err = launch_stream(c, a, stride_am, b, stride_bn, e, (int)K, hs);
  } else if (wlds && c.stages == 5) {
    err = launch_wlds_split(c, a, stride_am, b, stride_bn, e, K, (int32_t*)ws, hs);
  } else if (wlds && c.stages == 4) {
    err = launch_wldsp(c, a, stride_am, b, stride_bn, e, hs);
  } else if (wlds && c.stages == 3) {
    err = launch_wlds(c, a, stride_am, b, stride_bn, e, K, hs);
  } else if (c.stages == 2) {
    err = launch_staged(staged_index(c), c, a, stride_am, b, stride_bn, e, (int)K, hs);
  } else if (c.stages >= 2 + kPipelined) {
    err = launch_dmap(dmap_index(c), c, a, stride_am, b, stride_bn, e, (int)K, hs);
  } else {
    err = launch_dma(dma_index(c), c, a, stride_am, b, stride_bn, e, (int)K, hs);
  }
  return hip_status(err, who);
}

}  // namespace i8l

extern "C" int i8l_w8a8_mm(const int8_t* a, int64_t stride_am, int64_t stride_ak, const int8_t* b,
                           int64_t stride_bk, int64_t stride_bn, const float* scale_a,
                           int64_t scale_a_len, const float* scale_b, int64_t scale_b_len,
                           const void* bias, int32_t bias_dtype, void* out, int64_t stride_cm,
                           int32_t out_dtype, int64_t M, int64_t N, int64_t K,
                           const i8l_config* cfg, void* stream) {
  return w8a8_mm(a, stride_am, stride_ak, b, stride_bk, stride_bn, scale_a, scale_a_len,
                 scale_b, scale_b_len, bias, bias_dtype, out, stride_cm, out_dtype, M, N, K,
                 nullptr, 0, cfg, stream, "i8l_w8a8_mm");
}

extern "C" int i8l_w8a8_mm_ws(const int8_t* a, int64_t stride_am, int64_t stride_ak,
                              const int8_t* b, int64_t stride_bk, int64_t stride_bn,
                              const float* scale_a, int64_t scale_a_len, const float* scale_b,
                              int64_t scale_b_len, const void* bias, int32_t bias_dtype,
                              void* out, int64_t stride_cm, int32_t out_dtype, int64_t M,
                              int64_t N, int64_t K, void* workspace, int64_t workspace_bytes,
                              const i8l_config* cfg, void* stream) {
  return w8a8_mm(a, stride_am, stride_ak, b, stride_bk, stride_bn, scale_a, scale_a_len,
                 scale_b, scale_b_len, bias, bias_dtype, out, stride_cm, out_dtype, M, N, K,
                 workspace, workspace_bytes, cfg, stream, "i8l_w8a8_mm_ws");
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
  // a tile built for fewer than 16 rows a block takes one block of that many
  if (dq_max_rows(c) < 16 && M > dq_max_rows(c)) {
    set_error("the dynamic-quant tile %dx%dx%d w%d takes up to %d tokens, got %lld", c.bm, c.bn,
              c.bk, c.warps, dq_max_rows(c), (long long)M);
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

extern "C" int i8l_silu_mul_quant_mm_supported(int64_t M, int64_t N, int64_t K,
                                               const i8l_config* cfg) {
  i8l_config c;
  if (cfg) {
    c = *cfg;
  } else if (!default_dq_silu_config(N, K, &c)) {
    set_error("no built SiLU-and-mul quant tile takes K=%lld, N=%lld", (long long)K,
              (long long)N);
    return I8L_UNSUPPORTED;
  }
  if (M < 0 || M > dq_silu_max_rows() || N > INT32_MAX || K > INT32_MAX) {
    set_error("the SiLU-and-mul quant matmul takes up to %d tokens, got %lld",
              dq_silu_max_rows(), (long long)M);
    return I8L_UNSUPPORTED;
  }
  if (c.bn <= 0 || N % c.bn || !dq_silu_ok(c, K)) {
    set_error("config %dx%dx%d w%d s%d is not a built SiLU-and-mul quant tile for N=%lld K=%lld",
              c.bm, c.bn, c.bk, c.warps, c.stages, (long long)N, (long long)K);
    return I8L_UNSUPPORTED;
  }
  return I8L_OK;
}

extern "C" int i8l_silu_mul_quant_mm(const void* gate_up, int64_t ldgu, int32_t act_dtype,
                                     int32_t round_silu, int32_t precise_div, const int8_t* b,
                                     int64_t stride_bk, int64_t stride_bn, const float* scale_b,
                                     int64_t scale_b_len, const void* bias, int32_t bias_dtype,
                                     void* out, int64_t stride_cm, int32_t out_dtype,
                                     float* scale_a_out, int64_t M, int64_t N, int64_t K,
                                     const i8l_config* cfg, void* stream) {
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
  if (ldgu < 2 * K) {
    set_error("row stride %lld of gate_up is below 2K=%lld", (long long)ldgu, (long long)(2 * K));
    return I8L_INVALID_ARG;
  }
  i8l_config c;
  if (cfg) {
    c = *cfg;
  } else if (!default_dq_silu_config(N, K, &c)) {
    set_error("no built SiLU-and-mul quant tile takes K=%lld, N=%lld", (long long)K,
              (long long)N);
    return I8L_UNSUPPORTED;
  }
  const int st = i8l_silu_mul_quant_mm_supported(M, N, K, &c);
  if (st != I8L_OK) return st;
  if (M == 0 || N == 0) return I8L_OK;
  const int osz = elt_size(out_dtype);
  const bool layout = stride_bk == 1 && aligned16(b) && stride_bn % 16 == 0 &&
                      stride_bn <= INT32_MAX / 32 && aligned16(gate_up) && ldgu % 8 == 0 &&
                      K % 8 == 0 && aligned16(out) && (stride_cm * osz) % 16 == 0 &&
                      stride_cm >= N && N % 4 == 0 && (scale_b_len == 1 || aligned16(scale_b)) &&
                      (bias_dtype == I8L_DTYPE_NONE || aligned16(bias));
  if (!layout) {
    set_error("the SiLU-and-mul quant path needs K-contiguous 16-byte aligned operands");
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
  const hipError_t err = launch_dq_silu(c, act_dtype, round_silu ? 1 : 0,
                                        (const uint16_t*)gate_up, ldgu, K, b, stride_bn, e,
                                        scale_a_out, precise_div ? 1 : 0, (hipStream_t)stream);
  return hip_status(err, "i8l_silu_mul_quant_mm launch");
}

// ------------------------------------------------------------------ add + RMSNorm + quant + GEMM
extern "C" int i8l_add_rmsnorm_quant_mm_supported(int64_t M, int64_t N, int64_t K,
                                                  const i8l_config* cfg) {
  i8l_config c;
  if (cfg) {
    c = *cfg;
  } else if (!default_nq_config(M, N, K, &c)) {
    set_error("no built norm-quant tile takes K=%lld, N=%lld", (long long)K, (long long)N);
    return I8L_UNSUPPORTED;
  }
  if (M < 0 || M > nq_max_rows() || N > INT32_MAX || K > INT32_MAX) {
    set_error("the add+RMSNorm+quant matmul takes up to %d tokens, got %lld", nq_max_rows(),
              (long long)M);
    return I8L_UNSUPPORTED;
  }
  if (c.bn <= 0 || N % c.bn || !nq_ok(c, K)) {
    set_error("config %dx%dx%d w%d s%d g%d is not a built norm-quant tile for N=%lld K=%lld",
              c.bm, c.bn, c.bk, c.warps, c.stages, c.group_m, (long long)N, (long long)K);
    return I8L_UNSUPPORTED;
  }
  return I8L_OK;
}

extern "C" int i8l_add_rmsnorm_quant_mm(const void* x, const void* residual, const void* weight,
                                        float eps, int32_t act_dtype, int32_t precise_div,
                                        int32_t epilogue_act,
                                        void* residual_out, const int8_t* b, int64_t stride_bk,
                                        int64_t stride_bn, const float* scale_b,
                                        int64_t scale_b_len, const void* bias,
                                        int32_t bias_dtype, void* out, int64_t stride_cm,
                                        int32_t out_dtype, float* scale_a_out, int64_t M,
                                        int64_t N, int64_t K, const i8l_config* cfg,
                                        void* stream) {
  if (M < 0 || N < 0 || K < 0) {
    set_error("negative size M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
    return I8L_INVALID_ARG;
  }
  if (act_dtype != I8L_BF16 && act_dtype != I8L_F16) {
    set_error("activations and norm weight must be bf16 or fp16 (code %d)", act_dtype);
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
  if ((residual == nullptr) != (residual_out == nullptr)) {
    set_error("residual and residual_out must both be given or both be NULL");
    return I8L_INVALID_ARG;
  }
  if (x == nullptr || weight == nullptr) {
    set_error("x and the norm weight are required");
    return I8L_INVALID_ARG;
  }
  if (epilogue_act < 0 || epilogue_act > 2) {
    set_error("epilogue_act must be 0 (none), 1 (SiLU-and-mul) or 2 (rounded SiLU)");
    return I8L_INVALID_ARG;
  }
  if (epilogue_act != 0 && (act_dtype != I8L_BF16 || out_dtype != I8L_BF16 ||
                            bias_dtype != I8L_DTYPE_NONE || residual == nullptr ||
                            scale_b_len != N || N % 2)) {
    set_error("the SiLU-and-mul epilogue takes bf16 activations and output, a residual, "
              "per-channel scale_b, no bias and an even N");
    return I8L_UNSUPPORTED;
  }
  i8l_config c;
  if (cfg) {
    c = *cfg;
  } else if (!default_nq_config(M, N, K, &c)) {
    set_error("no built norm-quant tile takes K=%lld, N=%lld", (long long)K, (long long)N);
    return I8L_UNSUPPORTED;
  }
  const int st = i8l_add_rmsnorm_quant_mm_supported(M, N, K, &c);
  if (st != I8L_OK) return st;
  if (M == 0 || N == 0) return I8L_OK;
  const int osz = elt_size(out_dtype);
  const int64_t ncols = epilogue_act ? N / 2 : N;   // the output's columns
  const bool layout = stride_bk == 1 && aligned16(b) && stride_bn % 16 == 0 &&
                      stride_bn <= INT32_MAX / 32 && aligned16(x) && aligned16(weight) &&
                      (residual == nullptr || (aligned16(residual) && aligned16(residual_out))) &&
                      aligned16(out) && (stride_cm * osz) % 16 == 0 && stride_cm >= ncols &&
                      N % 4 == 0 && (scale_b_len == 1 || aligned16(scale_b)) &&
                      (bias_dtype == I8L_DTYPE_NONE || aligned16(bias));
  if (!layout) {
    set_error("the norm-quant path needs K-contiguous 16-byte aligned operands");
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
  const hipError_t err = launch_nq(c, act_dtype, (const uint16_t*)x, (const uint16_t*)residual,
                                   (const uint16_t*)weight, eps, (uint16_t*)residual_out, b,
                                   stride_bn, e, scale_a_out, precise_div ? 1 : 0, epilogue_act,
                                   (hipStream_t)stream);
  return hip_status(err, "i8l_add_rmsnorm_quant_mm launch");
}

// ------------------------------------------------------------------ GEMM + SiLU-and-mul
// The untuned choice: the persistent single-step tile (one 16-row block) with 16 columns a
// tile (8 gate and 8 up), 4 waves of 512-byte slices for K = 2048 and two workgroups a
// compute unit, else the first of these built forms that takes K (K = 6144: 8 columns, 16
// waves of 384 bytes, as the plain GEMM's tuned entries at that K).
static bool default_silu_config(int64_t N, int64_t K, i8l_config* c) {
  static const int pref[][4] = {{16, 512, 4, 2}, {16, 256, 8, 2}, {16, 128, 16, 1},
                                {16, 512, 8, 1}, {16, 256, 16, 1}, {16, 1024, 4, 1},
                                {8, 512, 4, 2},  {8, 256, 8, 2},   {8, 128, 16, 1},
                                {8, 384, 16, 1}, {8, 768, 8, 1}};
  for (const auto& p : pref) {
    const i8l_config t{16, p[0], p[1], p[2], 4, p[3]};
    if (N % t.bn == 0 && wldsp_silu_ok(t, K)) {
      *c = t;
      return true;
    }
  }
  return false;
}

extern "C" int i8l_w8a8_mm_silu_mul_supported(int64_t M, int64_t N, int64_t K,
                                              const i8l_config* cfg) {
  i8l_config c;
  if (cfg) {
    c = *cfg;
  } else if (!default_silu_config(N, K, &c)) {
    set_error("no built SiLU-epilogue tile takes K=%lld, N=%lld", (long long)K, (long long)N);
    return I8L_UNSUPPORTED;
  }
  if (M < 0 || M > 16 || N > INT32_MAX || K > INT32_MAX) {
    set_error("the SiLU-and-mul epilogue takes up to 16 tokens, got %lld", (long long)M);
    return I8L_UNSUPPORTED;
  }
  if (c.bn <= 0 || N % c.bn || !wldsp_silu_ok(c, K)) {
    set_error("config %dx%dx%d w%d s%d g%d is not a built SiLU-epilogue tile for N=%lld K=%lld",
              c.bm, c.bn, c.bk, c.warps, c.stages, c.group_m, (long long)N, (long long)K);
    return I8L_UNSUPPORTED;
  }
  return I8L_OK;
}

extern "C" int i8l_w8a8_mm_silu_mul(const int8_t* a, int64_t stride_am, const int8_t* b,
                                    int64_t stride_bk, int64_t stride_bn, const float* scale_a,
                                    int64_t scale_a_len, const float* scale_b,
                                    int64_t scale_b_len, const void* bias, int32_t bias_dtype,
                                    void* out, int64_t stride_cm, int32_t round_silu,
                                    int64_t M, int64_t N, int64_t K, const i8l_config* cfg,
                                    void* stream) {
  if (M < 0 || N < 0 || K < 0) {
    set_error("negative size M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
    return I8L_INVALID_ARG;
  }
  if (scale_a_len != 1 && scale_a_len != M) {
    set_error("scale_a has %lld values for M=%lld", (long long)scale_a_len, (long long)M);
    return I8L_INVALID_ARG;
  }
  if (scale_b_len != N || N % 2) {
    set_error("the SiLU-and-mul epilogue needs N even and N per-channel scales (got %lld "
              "for N=%lld)", (long long)scale_b_len, (long long)N);
    return I8L_INVALID_ARG;
  }
  if (bias_dtype != I8L_DTYPE_NONE && bias_dtype != I8L_BF16) {
    set_error("the SiLU-and-mul epilogue takes no bias or a bf16 bias (code %d)", bias_dtype);
    return I8L_UNSUPPORTED;
  }
  if ((bias_dtype == I8L_DTYPE_NONE) != (bias == nullptr)) {
    set_error("bias pointer and bias dtype disagree");
    return I8L_INVALID_ARG;
  }
  i8l_config c;
  if (cfg) {
    c = *cfg;
  } else if (!default_silu_config(N, K, &c)) {
    set_error("no built SiLU-epilogue tile takes K=%lld, N=%lld", (long long)K, (long long)N);
    return I8L_UNSUPPORTED;
  }
  const int st = i8l_w8a8_mm_silu_mul_supported(M, N, K, &c);
  if (st != I8L_OK) return st;
  if (M == 0 || N == 0) return I8L_OK;
  const bool layout = stride_bk == 1 && aligned16(b) && stride_bn % 16 == 0 &&
                      stride_bn <= INT32_MAX / 64 && aligned16(a) && stride_am % 16 == 0 &&
                      stride_am <= INT32_MAX / 128 && aligned16(out) && (stride_cm * 2) % 16 == 0 &&
                      stride_cm >= N / 2 && aligned16(scale_b) &&
                      (bias_dtype == I8L_DTYPE_NONE || aligned16(bias));
  if (!layout) {
    set_error("the SiLU-epilogue path needs K-contiguous 16-byte aligned operands");
    return I8L_UNSUPPORTED;
  }
  Epi e;
  e.sa = scale_a;
  e.sb = scale_b;
  e.bias = bias;
  e.out = out;
  e.ldc = stride_cm;
  e.sa_per_row = scale_a_len == M && M > 1;
  e.sb_per_col = 1;
  e.bias_dtype = bias_dtype;
  e.out_dtype = I8L_BF16;
  e.M = (int)M;
  e.N = (int)N;
  const hipError_t err = launch_wldsp_silu(c, a, stride_am, b, stride_bn, e, round_silu ? 1 : 0,
                                           (hipStream_t)stream);
  return hip_status(err, "i8l_w8a8_mm_silu_mul launch");
}

// ------------------------------------------------------------------ allocation-free entry
// i8l_w8a8_mm_noalloc: i8l_w8a8_mm for callers that cannot allocate (code under HIP graph
// capture, serving loops that forbid allocation), with the split of K's partial planes in
// `scratch`, a device array of this library (kScratchBytes on every GPU the library runs on,
// held until the process ends).  Every call on a GPU shares that GPU's array: calls that
// overlap in time on one GPU race.  Nothing in it has to start at zero (the first kernel of
// a split writes every partial the second reads), so it is never cleared.
namespace i8l {

constexpr int64_t kScratchBytes = 16ll << 20;
static __device__ __align__(256) int32_t scratch[kScratchBytes / 4];

constexpr int kScratchDevices = 64;
static std::atomic<void*> g_scratch[kScratchDevices];

// The device address of `scratch` on device `dev`, looked up once per device with that device
// current (in host code the array's name stands for the symbol, not for device memory); the
// calling thread's current device is restored.
static int scratch_setup(int dev, void** out, const char* where) {
  if (dev < 0 || dev >= kScratchDevices) {
    set_error("%s: device %d is beyond the %d this library serves", where, dev,
              kScratchDevices);
    return I8L_UNSUPPORTED;
  }
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) return hip_status(e, where);
    if (!p) {
      set_error("%s: no device address for the scratch array", where);
      return I8L_HIP_ERROR;
    }
    g_scratch[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return I8L_OK;
}

// The scratch address on the GPU that runs `stream` (set up by i8l_init, else here).
static int scratch_address(hipStream_t stream, void** out) {
  int dev = 0;
  const hipError_t e = hipStreamGetDevice(stream, &dev);
  if (e != hipSuccess) return hip_status(e, "i8l_w8a8_mm_noalloc: hipStreamGetDevice");
  return scratch_setup(dev, out, "i8l_w8a8_mm_noalloc");
}

}  // namespace i8l

extern "C" int i8l_init(int32_t device) {
  int dev = device;
  if (dev < 0) {
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "i8l_init: hipGetDevice");
  } else {
    int count = 0;
    const hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return hip_status(e, "i8l_init: hipGetDeviceCount");
    if (dev >= count) {
      set_error("i8l_init: device %d of %d", dev, count);
      return I8L_INVALID_ARG;
    }
  }
  void* p = nullptr;
  return scratch_setup(dev, &p, "i8l_init");
}

extern "C" int i8l_w8a8_mm_noalloc(const int8_t* a, int64_t stride_am, int64_t stride_ak,
                                   const int8_t* b, int64_t stride_bk, int64_t stride_bn,
                                   const float* scale_a, int64_t scale_a_len,
                                   const float* scale_b, int64_t scale_b_len, const void* bias,
                                   int32_t bias_dtype, void* out, int64_t stride_cm,
                                   int32_t out_dtype, int64_t M, int64_t N, int64_t K,
                                   const i8l_config* cfg, void* stream) {
  const int64_t need = i8l_w8a8_mm_workspace_bytes(M, N, K, cfg);
  if (need > kScratchBytes) {
    set_error("i8l_w8a8_mm_noalloc: M=%lld N=%lld with %d parts of K needs %lld bytes of "
              "workspace, beyond the %lld-byte scratch (use i8l_w8a8_mm_ws)", (long long)M,
              (long long)N, cfg ? cfg->group_m : 1, (long long)need, (long long)kScratchBytes);
    return I8L_UNSUPPORTED;
  }
  void* ws = nullptr;
  if (need > 0) {
    const int st = scratch_address((hipStream_t)stream, &ws);
    if (st != I8L_OK) return st;
  }
  return w8a8_mm(a, stride_am, stride_ak, b, stride_bk, stride_bn, scale_a, scale_a_len,
                 scale_b, scale_b_len, bias, bias_dtype, out, stride_cm, out_dtype, M, N, K,
                 ws, need > 0 ? kScratchBytes : 0, cfg, stream, "i8l_w8a8_mm_noalloc");
}
