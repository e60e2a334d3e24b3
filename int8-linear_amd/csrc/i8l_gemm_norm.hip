// add + RMSNorm + per-token int8 quantize folded into the persistent decode GEMM, for few
// tokens (up to 8):
//
//   (q, s, residual_out) = add_rmsnorm_quant(x, residual, gamma, eps)
//   out = w8a8_mm(q, B, scale_a = s, scale_b, bias)
//
// bit for bit as the two launches give them, from one launch.  The reference runs these two
// kernels back to back before its qkv and gate_up projections (bench/fuse_quant.py:226-240
// of AshrithaG/int8-linear; int8_linear/fused_quant.py:56-73 and kernel.py:63-124).  At a
// few tokens each launch costs more than its work (an empty kernel in a HIP graph takes
// 1.6 us), so the norm is computed where its codes are consumed.
//
// Schedule (gemm_wlds1p_nq): the persistent single-step tile of the decode GEMM (each of the
// W waves owns one K slice of S = 64*KS bytes, and a workgroup walks the column tiles
// blockIdx.x, blockIdx.x + gridDim.x, ...).  Before its first tile the workgroup normalizes
// and quantizes the token rows itself, while that tile's weight copy is in flight:
//   * the activation rows and the norm weight are requested first, then the first tile's
//     weights (direct-to-LDS), and the wave waits for the activations alone;
//   * wave w holds its K slice of each row as 8-value chunks, CH = S/8 lanes a row and
//     RPP = 64/CH rows a pass (P passes);
//   * x + residual, and residual_out from the first workgroup only;
//   * the sum of squares as the canonical tree of the quantizer kernel: 8 leaves in a lane
//     (x_i^2 exact in double), the CH lanes of the row by a butterfly, then the W waves'
//     nodes pairwise through LDS (K = W*S is a power of two, the waves' slices are aligned
//     nodes);
//   * rsqrt, the two roundings of the norm, the row's absmax across lanes and waves, scale
//     and codes exactly as add_rmsnorm_quant_kernel computes them (a row's rsqrt and scale
//     once, in the lane of that row, not in every pass);
//   * the codes go to an LDS tile of the wave's own, which aliases the wave's second weight
//     buffer (not yet in use), and come back as the wave's MFMA activation fragments, held in
//     registers for every column tile the workgroup takes.
// Every workgroup repeats the row work, which is why this pays only for a few tokens.
#include "i8l_gemm.h"

namespace i8l {

template <int DT>
__device__ __forceinline__ void unpack8_act(const uint4& v, float* o) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = act_to_f32<DT>(w[i] & 0xffffu);
    o[2 * i + 1] = act_to_f32<DT>(w[i] >> 16);
  }
}

// NC columns a tile, K slices of S = 64*KS bytes over W waves (K = W*S), P passes of RPP
// rows over the token rows (at most 8), DT the activation dtype (the norm weight's too),
// RES whether a residual is added (else the first layer's plain RMSNorm).  ACT kActSilu /
// kActSiluRound: the gate_up projection with the SiLU-and-mul epilogue of gemm_wlds1p
// (tile t: gate rows [t*H, (t+1)*H) and the same up rows, H = NC/2; y = silu(gate) * up,
// [M, N/2] bf16).
template <int NC, int KS, int W, int P, int EK, int DT, bool RES, int ACT = kActPlain>
__global__ void __launch_bounds__(64 * W)
gemm_wlds1p_nq(const uint16_t* __restrict__ X, const uint16_t* __restrict__ R,
               const uint16_t* __restrict__ G, float eps, uint16_t* __restrict__ rout,
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
  static_assert(NF * NCF == NC && NF <= W, "every column fragment needs a storing wave");
  constexpr int K = W * S;
  constexpr int CH = S / 8;                 // 8-value chunks of a row in a wave's slice
  constexpr int RPP = 64 / CH;              // rows a pass covers
  static_assert(CH == 16 || CH == 32 || CH == 64, "a row's slice spans 16, 32 or 64 lanes");
  static_assert((W & (W - 1)) == 0, "the waves' slices must be nodes of the row's tree");
  static_assert(P >= 1 && P * RPP <= 16, "the passes cover at most one 16-row block");
  static_assert(NC >= 8, "the code tile of up to 8 rows lives in a weight buffer");
  constexpr bool SILU = ACT != kActPlain;
  static_assert(!SILU || (NF == 1 && EK != EK_ANY), "the SiLU epilogue takes bf16 output");
  constexpr int H = NC / 2;                 // SiLU: gate (and up) columns of a tile
  extern __shared__ __attribute__((aligned(16))) int8_t lds[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, grp = lane >> 4;
  const int tiles = e.N / NC;
  const int mb = e.M;                       // the host takes at most 8 token rows
  const int kw = wave * S;
  int8_t* const wb0 = lds + (size_t)wave * SB;
  int8_t* const wb1 = lds + (size_t)(W + wave) * SB;   // also the wave's code tile
  v4i* const red = (v4i*)(lds + (size_t)2 * W * SB);   // [W][NF][64]
  double* const dsum = (double*)(lds + (size_t)2 * W * SB + (size_t)W * NF * 1024);  // [W][16]
  float* const rmax = (float*)(dsum + W * 16);          // [W][16]
  const int ldb32 = (int)ldb;

  auto dma = [&](int ct, int8_t* wb) {
    lds_i8_t* dst = (lds_i8_t*)wb;
    // tile row r: weight row ct*NC + r; SiLU: gate row ct*H + r for r < H, else up row
    // N/2 + ct*H + r - H
    const int8_t* Bw = B + (int64_t)ct * (SILU ? H : NC) * ldb + kw;
    const int8_t* Bu = SILU ? Bw + (int64_t)(e.N / 2) * ldb - (int64_t)H * ldb : Bw;
#pragma unroll
    for (int t = 0; t < NI; ++t) {
      const int o = t * 1024 + 16 * lane;
      const int r = o / S, c = ((o % S) / 16) ^ (r & SWM);
      __builtin_amdgcn_global_load_lds((const void*)((SILU && r >= H ? Bu : Bw) +
                                                     (r * ldb32 + 16 * c)),
                                       dst + t * 1024, 16, 0, kWeightCpol);
    }
  };

  // pass p: lane l holds chunk l % CH of the wave's slice of row p*RPP + l/CH
  const int crow = lane / CH, cchunk = lane % CH;
  const int c0 = kw + 8 * cchunk;
  uint4 xr[P], rr[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int r = p * RPP + crow;
    xr[p] = rr[p] = uint4{0, 0, 0, 0};
    if (r < mb) {
      xr[p] = *(const uint4*)(X + (int64_t)r * K + c0);
      if constexpr (RES) rr[p] = *(const uint4*)(R + (int64_t)r * K + c0);
    }
  }
  const uint4 gr = *(const uint4*)(G + c0);
  __builtin_amdgcn_sched_barrier(0);
  dma(blockIdx.x, wb0);                     // the first tile's weights, while the rows work
  __builtin_amdgcn_sched_barrier(0);
  wait_vmcnt_wlds<NI>();                    // loads land in issue order: the rows are in
  __builtin_amdgcn_sched_barrier(0);        // no use of the rows above the wait

  // x (+ residual) and each row's node of the sum of squares, the passes' cross-lane trees
  // side by side; then residual_out (first workgroup only)
  float xv[P][8];
  double node[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    unpack8_act<DT>(xr[p], xv[p]);
    if constexpr (RES) {
      float rv[8];
      unpack8_act<DT>(rr[p], rv);
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[p][i] = xv[p][i] + rv[i];
    }
    // leaves x_i^2 are exact in double, so x_i^2 + x_{i+1}^2 is one fma
    double s[8];
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const double a = (double)xv[p][i], b = (double)xv[p][i + 1];
      s[i] = __builtin_fma(b, b, a * a);
    }
#pragma unroll
    for (int st = 2; st < 8; st <<= 1)
#pragma unroll
      for (int i = 0; i < 8; i += 2 * st) s[i] = s[i] + s[i + st];
    node[p] = s[0];
  }
  group_tree_sum_n<CH, P>(node);
  if (cchunk == 0) {
#pragma unroll
    for (int p = 0; p < P; ++p) dsum[wave * 16 + p * RPP + crow] = node[p];
  }
  if constexpr (RES) {
    if (blockIdx.x == 0) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const int r = p * RPP + crow;
        if (r < mb) {
          uint32_t w[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) w[i] = f32x2_to_act2<DT>(xv[p][2 * i], xv[p][2 * i + 1]);
          *(uint4*)(rout + (int64_t)r * K + c0) = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
    }
  }
  lds_sync();

  // Each row's scalar work is done once, in lane r of every wave for row r (r = lane % 16,
  // rows past the passes clamped to the last): the sum over the waves' nodes and the rsqrt
  // here, the absmax over the waves and the scale below.  A pass takes its row's values from
  // that lane, so the per-row division and square-root chains are not repeated P times.
  const int rl = min(r16, P * RPP - 1);
  float rs_l;
  {
    double nd[W];
#pragma unroll
    for (int w = 0; w < W; ++w) nd[w] = dsum[w * 16 + rl];
#pragma unroll
    for (int st = 1; st < W; st <<= 1)
#pragma unroll
      for (int w = 0; w < W; w += 2 * st) nd[w] = nd[w] + nd[w + st];
    const float var = (float)(nd[0] / (double)K);
    rs_l = canon_rsqrtf(var + eps);
  }
  // pass p's row value from lane r: a readlane when the pass is one row, else a permute
  auto row_val = [&](float v, int p) {
    if constexpr (RPP == 1) return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), p));
    else return __shfl(v, p * RPP + crow);
  };

  // y = cast(f32(cast(x * rs)) * gamma), and the row's absmax (the passes' cross-lane
  // maxima side by side)
  float gv[8];
  unpack8_act<DT>(gr, gv);
  float am[P], rsp[P];
#pragma unroll
  for (int p = 0; p < P; ++p) rsp[p] = row_val(rs_l, p);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const float rs = rsp[p];
    am[p] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      float a = xv[p][i] * rs, b = xv[p][i + 1] * rs;
      round_through2<DT>(a, b);
      a = a * gv[i];
      b = b * gv[i + 1];
      round_through2<DT>(a, b);
      xv[p][i] = a;
      xv[p][i + 1] = b;
      am[p] = fmaxf(fmaxf(am[p], fabsf(a)), fabsf(b));   // one max3 with |.| operands
    }
  }
  group_max_n<CH, P>(am);
  if (cchunk == 0) {
#pragma unroll
    for (int p = 0; p < P; ++p) rmax[wave * 16 + p * RPP + crow] = am[p];
  }
  lds_sync();

  // scale and inverse of row rl (the quantizer of add_rmsnorm_quant_kernel)
  float sc_l, inv_l;
  {
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
  if (sa_out != nullptr && blockIdx.x == 0 && wave == 0 && lane < mb) sa_out[lane] = sc_l;

  // codes into the code tile (the passes' inverses fetched first, together)
  float invp[P];
#pragma unroll
  for (int p = 0; p < P; ++p) invp[p] = row_val(inv_l, p);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int r = p * RPP + crow;
    const float inv = invp[p];
    if (r < mb) {
      uint32_t word[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t packed = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) packed |= code_rne(xv[p][4 * h + b] * inv) << (8 * b);
        word[h] = packed;
      }
      lds_store_b64(wb1 + r * S + 8 * cchunk, word[0], word[1]);   // the first tile's copy is in flight
    }
  }
  // the wave's activation fragments from its own code tile (LDS is in order within a wave;
  // rows past M are zero), and its row scale for the epilogue
  v4i a[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    a[s] = r16 < mb ? *(const v4i*)(wb1 + r16 * S + 64 * s + 16 * grp) : v4i{0, 0, 0, 0};
  const float sam = wave < NF && r16 < mb ? sc_l : 0.0f;   // lane l computed row l % 16
  wait_lgkmcnt0();                          // the code tile is read before wb1 is refilled

  const int cq = 4 * (grp & (NCF / 4 - 1));   // the lane's first column in the fragment
  auto ncol_of = [&](int ct) -> int64_t {
    return SILU ? (cq < H ? (int64_t)ct * H + cq : (int64_t)(e.N / 2) + ct * H + cq - H)
                : (int64_t)ct * NC + NCF * (wave % NF) + cq;
  };
  // One column tile, as in gemm_wlds1p: the explicit vmcnt(0) at the top is the only wait on
  // vector memory (this tile's weights and epilogue operands, requested a tile earlier), then
  // the next tile's are requested; operands in two alternating register sets, the
  // reduction's LDS stores in inline assembly (a use of a loaded register, or an LDS store,
  // while a direct-to-LDS copy is in flight makes the compiler wait for every request).
  auto tile = [&](int ct, int8_t* cur, int8_t* nxt, const Cols4& cl, Cols4& cln) {
    wait_vmcnt_wlds<0>();
    __builtin_amdgcn_sched_barrier(0);
    const int ctn = ct + (int)gridDim.x;
    if (ctn < tiles) {               // uniform over the workgroup
      dma(ctn, nxt);
      if (wave < NF) cln = load_cols4<EK>(e, ncol_of(ctn));
    }
    __builtin_amdgcn_sched_barrier(0);
    const int64_t ncol = ncol_of(ct);
    v4i b[KS][NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int br = NCF * f + r16 % NCF;
#pragma unroll
      for (int s = 0; s < KS; ++s)
        b[s][f] = *(const v4i*)(cur + br * S + 16 * ((4 * s + grp) ^ (br & SWM)));
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
    for (int f = 0; f < NF; ++f) lds_store_b128(&red[(wave * NF + f) * 64 + lane], acc[f]);
    lds_sync();
    if (wave < NF) {
      v4i sum = red[wave * 64 + lane];
#pragma unroll
      for (int w = 1; w < W; ++w) sum += red[(w * NF + wave) * 64 + lane];
      if constexpr (SILU) {
        float v[4];
        epi_values4<EK>(e, sum, cl, sam, v);
        silu_mul_pairs<ACT, 4 * H>(v, cq < H);
        if (r16 < mb && cq < H && 4 * grp < NCF) store4_bf16(e.out, e.ldc, r16, ct * H + cq, v);
      } else {
        if (r16 < mb && 4 * grp < NCF) store4s<EK>(e, r16, ncol, sum, cl, sam);
      }
    }
    lds_sync();  // the partials of the next tile overwrite the reduction area
  };

  // the first tile's weights were requested before the row work
  int ct = blockIdx.x;
  Cols4 cla, clb;
  if (ct < tiles && wave < NF) cla = load_cols4<EK>(e, ncol_of(ct));
  for (;;) {
    if (ct >= tiles) break;
    tile(ct, wb0, wb1, cla, clb);
    ct += gridDim.x;
    if (ct >= tiles) break;
    tile(ct, wb1, wb0, clb, cla);
    ct += gridDim.x;
  }
}

// ------------------------------------------------------------------ host side
// Tiles (NC, KS, W): K = 64 * KS * W, a row's slice 16, 32 or 64 lanes (KS = 2, 4 or 8).
struct NqTile {
  int nc, ks, w;
};
constexpr NqTile kNq[] = {{16, 8, 4}, {16, 4, 8}, {8, 8, 4}, {8, 4, 8}, {16, 8, 8}, {8, 8, 8}};
constexpr int kNqMaxRows = 8;

int nq_max_rows() { return kNqMaxRows; }

static size_t nq_lds_bytes(int nc, int ks, int w) {
  const int nf = nc > 16 ? nc / 16 : 1;
  // two weight buffers a wave, the cross-wave sums, the row nodes and maxima
  return (size_t)2 * w * nc * 64 * ks + (size_t)w * nf * 1024 + (size_t)w * 16 * (8 + 4);
}

// stages 4 (persistent), bm 16; group_m workgroups a compute unit (1, 2 or 4).
bool nq_ok(const i8l_config& c, int64_t K) {
  if (c.stages != 4 || c.bm != 16 || (c.group_m != 1 && c.group_m != 2 && c.group_m != 4))
    return false;
  for (auto t : kNq)
    if (t.nc == c.bn && 64 * t.ks == c.bk && t.w == c.warps)
      return K == (int64_t)64 * t.ks * t.w &&
             (size_t)c.group_m * nq_lds_bytes(t.nc, t.ks, t.w) <= kMaxLds &&
             c.group_m * 64 * t.w <= 2048;
  return false;
}

// The untuned choice, from a sweep of the built tiles on MI355X (K = 2048, N = 4096 and
// 12288, 1-8 tokens, HIP graph, cold weights): 4 waves of 512-byte slices wherever every
// workgroup has one tile (N = 4096: 3.63 / 4.72 / 4.90 / 6.57 us at 1 / 3 / 4 / 8 tokens
// against 4.81 / 5.03 / 5.15 / 6.71 with 8 waves) and up to 4 tokens otherwise, two
// workgroups a compute unit (N = 12288 at 4 tokens: 7.51 us against 7.59 with 8 waves); from
// 5 tokens with several tiles a workgroup, 8 waves of 256-byte slices, the row work spread
// over twice the lanes, one workgroup a compute unit (N = 12288 at 5 / 8 tokens: 8.92 / 9.18
// us against 9.52 / 10.24 with 4 waves, 9.20 / 9.93 with two workgroups); 16 columns a tile
// (8 when N does not give 256 tiles of 16).  Two workgroups a compute unit only where a
// workgroup would otherwise walk more than one tile and the LDS holds two.  K = 4096 takes
// 8 waves of 512 bytes.
bool default_nq_config(int64_t M, int64_t N, int64_t K, i8l_config* c) {
  const int nc = N % 16 == 0 && N / 16 >= 256 ? 16 : 8;
  static const int one[3][2] = {{512, 4}, {256, 8}, {512, 8}};    // (bk, waves) by preference
  static const int more[3][2] = {{256, 8}, {512, 4}, {512, 8}};
  const bool few = N / nc <= cu_count() || M <= 4;
  const int (&pref)[3][2] = few ? one : more;
  static const int g_few[2] = {2, 1}, g_more[2] = {1, 2};
  const int* gs = few ? g_few : g_more;
  for (const auto& bw : pref)
    for (int gi = 0; gi < 2; ++gi) {
      const int g = gs[gi];
      if (g == 2 && N / nc <= 256) continue;
      const i8l_config t{16, nc, bw[0], bw[1], 4, g};
      if (N % nc == 0 && nq_ok(t, K)) {
        *c = t;
        return true;
      }
    }
  return false;
}

template <int NC, int KS, int W, int P, int EK, int DT, bool RES, int ACT = kActPlain>
hipError_t launch_nq_k(const uint16_t* x, const uint16_t* res, const uint16_t* gamma, float eps,
                       uint16_t* rout, const int8_t* b, int64_t ldb, const Epi& e,
                       float* sa_out, int precise, int per_cu, hipStream_t st) {
  auto kern = gemm_wlds1p_nq<NC, KS, W, P, EK, DT, RES, ACT>;
  const size_t shm = nq_lds_bytes(NC, KS, W);
  static std::atomic<uint64_t> lds_done{0};  // devices this kernel is opted in on
  lds_opt_in((const void*)kern, shm, lds_done);
  const int tiles = e.N / NC;
  const dim3 grid((unsigned)std::min(tiles, std::max(1, per_cu * cu_count())));
  hipLaunchKernelGGL(kern, grid, dim3(64 * W), shm, st, x, res, gamma, eps, rout, b, ldb, e,
                     sa_out, precise);
  return hipGetLastError();
}

template <int NC, int KS, int W, int P, int DT, bool RES>
hipError_t launch_nq_e(const uint16_t* x, const uint16_t* res, const uint16_t* gamma, float eps,
                       uint16_t* rout, const int8_t* b, int64_t ldb, const Epi& e,
                       float* sa_out, int precise, int per_cu, int act, hipStream_t st) {
  // the SiLU epilogue: bf16 activations and output, a residual, no bias (the MLP's gate_up)
  if constexpr (DT == I8L_BF16 && RES) {
    if (act != kActPlain) {
      if (epi_kind(e) != EK_BF16) return hipErrorInvalidValue;
      return act == kActSiluRound
          ? launch_nq_k<NC, KS, W, P, EK_BF16, DT, RES, kActSiluRound>(
                x, res, gamma, eps, rout, b, ldb, e, sa_out, precise, per_cu, st)
          : launch_nq_k<NC, KS, W, P, EK_BF16, DT, RES, kActSilu>(
                x, res, gamma, eps, rout, b, ldb, e, sa_out, precise, per_cu, st);
    }
  }
  if (act != kActPlain) return hipErrorInvalidValue;
  if constexpr (DT == I8L_BF16) {
    switch (epi_kind(e)) {
      case EK_BF16:
        return launch_nq_k<NC, KS, W, P, EK_BF16, DT, RES>(x, res, gamma, eps, rout, b, ldb, e,
                                                          sa_out, precise, per_cu, st);
      case EK_BF16_BBF16:
        return launch_nq_k<NC, KS, W, P, EK_BF16_BBF16, DT, RES>(x, res, gamma, eps, rout, b,
                                                                ldb, e, sa_out, precise,
                                                                per_cu, st);
      default: break;
    }
  }
  return launch_nq_k<NC, KS, W, P, EK_ANY, DT, RES>(x, res, gamma, eps, rout, b, ldb, e, sa_out,
                                                   precise, per_cu, st);
}

// Passes: ceil(rows / RPP) rounded up to a power of two, for at most kNqMaxRows rows.
template <int NC, int KS, int W, int P>
hipError_t launch_nq_p(int act_dtype, const uint16_t* x, const uint16_t* res,
                       const uint16_t* gamma, float eps, uint16_t* rout, const int8_t* b,
                       int64_t ldb, const Epi& e, float* sa_out, int precise, int per_cu,
                       int act, hipStream_t st) {
  if (act_dtype == I8L_F16)
    return res ? launch_nq_e<NC, KS, W, P, I8L_F16, true>(x, res, gamma, eps, rout, b, ldb, e,
                                                          sa_out, precise, per_cu, act, st)
               : launch_nq_e<NC, KS, W, P, I8L_F16, false>(x, res, gamma, eps, rout, b, ldb, e,
                                                           sa_out, precise, per_cu, act, st);
  return res ? launch_nq_e<NC, KS, W, P, I8L_BF16, true>(x, res, gamma, eps, rout, b, ldb, e,
                                                         sa_out, precise, per_cu, act, st)
             : launch_nq_e<NC, KS, W, P, I8L_BF16, false>(x, res, gamma, eps, rout, b, ldb, e,
                                                          sa_out, precise, per_cu, act, st);
}

template <int NC, int KS, int W>
hipError_t launch_nq_t(int act_dtype, const uint16_t* x, const uint16_t* res,
                       const uint16_t* gamma, float eps, uint16_t* rout, const int8_t* b,
                       int64_t ldb, const Epi& e, float* sa_out, int precise, int per_cu,
                       int act, hipStream_t st) {
  constexpr int RPP = 64 / (8 * KS);
  const int need = (e.M + RPP - 1) / RPP;
  // P = 1, 2, 4, 8 where P passes are the fewest that cover some row count up to the maximum
#define I8L_NQ_P(P_)                                                                         \
  if constexpr (P_ == 1 || (P_ / 2) * RPP < kNqMaxRows)                                      \
    if (need <= P_)                                                                          \
      return launch_nq_p<NC, KS, W, P_>(act_dtype, x, res, gamma, eps, rout, b, ldb, e,      \
                                        sa_out, precise, per_cu, act, st);
  I8L_NQ_P(1) I8L_NQ_P(2) I8L_NQ_P(4) I8L_NQ_P(8)
#undef I8L_NQ_P
  return hipErrorInvalidValue;
}

hipError_t launch_nq(const i8l_config& c, int act_dtype, const uint16_t* x,
                     const uint16_t* residual, const uint16_t* gamma, float eps,
                     uint16_t* residual_out, const int8_t* b, int64_t ldb, const Epi& e,
                     float* sa_out, int precise, int act, hipStream_t st) {
  const int nc = c.bn, ks = c.bk / 64, w = c.warps;
#define I8L_NQ(NC_, KS_, W_)                                                                 \
  if (nc == NC_ && ks == KS_ && w == W_)                                                     \
    return launch_nq_t<NC_, KS_, W_>(act_dtype, x, residual, gamma, eps, residual_out, b,    \
                                     ldb, e, sa_out, precise, c.group_m, act, st);
  I8L_NQ(16, 8, 4) I8L_NQ(16, 4, 8) I8L_NQ(8, 8, 4) I8L_NQ(8, 4, 8) I8L_NQ(16, 8, 8)
  I8L_NQ(8, 8, 8)
#undef I8L_NQ
  return hipErrorInvalidValue;
}

}  // namespace i8l
