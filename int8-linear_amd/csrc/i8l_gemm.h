// Internal interface of the W8A8 GEMM: the epilogue and memory helpers shared by the decode
// schedules (i8l_gemm_decode.hip), the prefill schedules (i8l_gemm_prefill.hip) and the
// dispatch and C entry points (i8l_gemm.hip), and the host functions each exports.
//
//   out[m,n] = cast( f32(sum_k A[m,k] * B[k,n]) * sa[m|0] * sb[n|0] (+ f32(bias[n])) )
//
// Semantics follow the reference Triton kernel _w8a8_mm (AshrithaG/int8-linear,
// int8_linear/kernel.py:63-124): exact int32 accumulation (94-103), then the epilogue in
// fp32 in the order acc -> *sa -> *sb -> +bias (109-119) and one cast to the output dtype
// (120); raw mode stores the int32 accumulator (106-107).  Every GEMM source is built with
// -ffp-contract=off, so the epilogue is exactly that sequence of IEEE operations.
#pragma once

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

// Per-column epilogue operands of four consecutive output columns n..n+3.  A 16-bit bias is
// kept as loaded (hb: four bf16/fp16 values) and widened where the epilogue adds it: widening
// at the load would make the compiler wait for that load (and for every memory request
// issued before it, such as the current weight copy) before the next copy is requested.
struct Cols4 {
  float sb[4], bias[4];
  uint2 hb;
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
    c.sb[0] = e.sb[0];   // one scale for every column: store4s reads sb[0] (no copies here)
  }
  if (bd == I8L_F32) {
    const float4 v = *(const float4*)((const float*)e.bias + n);
    c.bias[0] = v.x, c.bias[1] = v.y, c.bias[2] = v.z, c.bias[3] = v.w;
  } else if (bd == I8L_BF16 || bd == I8L_F16) {
    c.hb = *(const uint2*)((const uint16_t*)e.bias + n);   // widened in store4s
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

// The four epilogue values acc * sa * sb (+ bias) in fp32, before the cast (not for raw).
template <int EK = EK_ANY>
__device__ __forceinline__ void epi_values4(const Epi& e, v4i acc, const Cols4& c, float sam,
                                            float (&o)[4]) {
  const int bd = epi_bias<EK>(e);
  float bias[4];
  if (bd == I8L_BF16 || bd == I8L_F16) {
    const uint32_t w[4] = {c.hb.x & 0xffffu, c.hb.x >> 16, c.hb.y & 0xffffu, c.hb.y >> 16};
#pragma unroll
    for (int r = 0; r < 4; ++r)
      bias[r] = bd == I8L_BF16 ? bf16_bits_to_f32(w[r]) : f16_bits_to_f32(w[r]);
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) bias[r] = c.bias[r];
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float v = (float)acc[r];
    v = v * sam;
    v = v * (epi_sb_per_col<EK>(e) ? c.sb[r] : c.sb[0]);
    if (bd != I8L_DTYPE_NONE) v = v + bias[r];
    o[r] = v;
  }
}

template <int EK = EK_ANY>
__device__ __forceinline__ void store4s(const Epi& e, int64_t m, int64_t n, v4i acc,
                                        const Cols4& c, float sam) {
  const int od = epi_out<EK>(e);
  if (od == I8L_I32) {
    *(v4i*)((int32_t*)e.out + m * e.ldc + n) = acc;
    return;
  }
  float o[4];
  epi_values4<EK>(e, acc, c, sam, o);
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

// ------------------------------------------------------------------ SiLU-and-mul
// What a fused kernel applies to its values: kActPlain nothing; kActSilu the SiLU-and-mul of
// gate and up values, y = cast(silu(g) * u); kActSiluRound the same with silu(g) rounded to
// the activation dtype first (reference fused_quant.py:76-88, ROUND_SILU).
enum { kActPlain = 0, kActSilu = 1, kActSiluRound = 2 };

// silu(g) = g / d with d = 1 + exp(-g) from the canonical exp.  The quotient as rcp(d) with
// one Newton-Markstein correction and g's sign equals IEEE division for every bf16 and fp16
// g in (-87, +inf) (the silu_mul_quant kernel's fast form); ieee takes the IEEE division,
// which a wave holding any other g uses for all of its values.
__device__ __forceinline__ float silu_canon(float g, bool ieee) {
  const float d = 1.0f + canon_expf_core(__builtin_amdgcn_fmed3f(-g, -87.5f, 89.5f));
  if (ieee) return g / d;
  const float r0 = __builtin_amdgcn_rcpf(d);
  const float q0 = g * r0;
  const float q1 = __builtin_fmaf(__builtin_fmaf(-d, q0, g), r0, q0);
  return __uint_as_float((__float_as_uint(q1) & 0x7fffffffu) | (__float_as_uint(g) & 0x80000000u));
}

// The SiLU-and-mul epilogue of a decode tile whose MFMA fragment holds the gate columns of a
// column range in its first rows and the up columns of the same range after them: lane l
// holds four consecutive columns of one half, and lane l ^ PO the same four columns of the
// other.  v: the lane's four epilogue values; they are rounded to bf16 (the gate_up output
// the unfused path would store), swapped with the partner lane, and on the gate lanes turned
// into y = bf16(silu(g) (rounded for kActSiluRound) * u), the silu_mul_quant kernel's values.
// Every lane of the wave must call it (cross-lane moves, and the wave-wide IEEE choice).
template <int ACT, int PO>
__device__ __forceinline__ void silu_mul_pairs(float (&v)[4], bool gate_lane) {
  static_assert(ACT == kActSilu || ACT == kActSiluRound, "a SiLU epilogue");
  float p[4];
#pragma unroll
  for (int r = 0; r < 4; r += 2) round_through2<I8L_BF16>(v[r], v[r + 1]);
#pragma unroll
  for (int r = 0; r < 4; ++r) p[r] = __shfl_xor(v[r], PO);
  float gmin = __builtin_inff(), gmax = -__builtin_inff();
  if (gate_lane)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      gmin = fminf(gmin, v[r]);
      gmax = fmaxf(gmax, v[r]);
    }
  const bool ieee = !__all(gmin > -87.0f && gmax < __builtin_inff());
  float a[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) a[r] = silu_canon(v[r], ieee);
  if constexpr (ACT == kActSiluRound) {
    round_through2<I8L_BF16>(a[0], a[1]);
    round_through2<I8L_BF16>(a[2], a[3]);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) v[r] = a[r] * p[r];
}

// Four bf16 values at (m, n) of a row-major bf16 output with row pitch ldc.
__device__ __forceinline__ void store4_bf16(void* out, int64_t ldc, int64_t m, int64_t n,
                                            const float (&v)[4]) {
  *(uint2*)((uint16_t*)out + m * ldc + n) =
      make_uint2(f32x2_to_bf16x2_bits(v[0], v[1]), f32x2_to_bf16x2_bits(v[2], v[3]));
}

// Cache policy of the decode schedules' weight copies (global_load_lds): NT, non-temporal.
// Each weight byte is read once per call, and loaded with the default policy the stream
// (8-117 MB a call) displaces from L2 what the next launches do reuse: the kernels'
// instructions, the activations and the epilogue operands.  Measured over the decode sweep
// (72 linears of four shapes in one graph, cold weights): 5.75 -> 5.44 us per linear.
constexpr int kWeightCpol = 2;

__device__ __forceinline__ v4i ld16(const int8_t* p) { return *(const v4i*)p; }
// Weight bytes are read exactly once per call: stream them past the caches.
__device__ __forceinline__ v4i ld16_stream(const int8_t* p) {
  return __builtin_nontemporal_load((const v4i*)p);
}

// The Epi fields (pin_vals: one round trip for every kernel argument), the grid size and up
// to 10 more arguments.  blockDim is not read by these kernels: it costs two dependent round
// trips (the grid size, then a 16-bit load that picks the last workgroup's remainder), so a
// kernel that needs its wave count takes it as an argument.
template <typename... T>
__device__ __forceinline__ void pin_args(const Epi& e, T... more) {
  static_assert(sizeof...(T) <= 10, "at most 10 more arguments");
  const int64_t x[10] = {pin_value(more)...};
  asm volatile("" ::"s"(e.sa), "s"(e.sb), "s"(e.bias), "s"(e.out), "s"(e.ldc), "s"(e.sa_per_row),
               "s"(e.sb_per_col), "s"(e.bias_dtype), "s"(e.out_dtype), "s"(e.M), "s"(e.N),
               "s"((int)gridDim.x), "s"((int)gridDim.y), "s"((int)gridDim.z), "s"(x[0]),
               "s"(x[1]), "s"(x[2]), "s"(x[3]), "s"(x[4]), "s"(x[5]), "s"(x[6]), "s"(x[7]),
               "s"(x[8]), "s"(x[9]));
}

// Column tile of a decode workgroup.  The dispatcher deals workgroups to the 8 XCDs
// round-robin by linear id; with a multiple of 8 column tiles per row, XCD x is given the
// contiguous column range [x, x+1) * gridDim.x/8, so the output lines (and the L2 lines
// they are assembled in) are written from one XCD rather than in pieces from eight.
__device__ __forceinline__ int64_t xcd_col_tile() {
  const int gx = gridDim.x, bx = blockIdx.x;
  return gx % 8 == 0 ? (int64_t)(bx % 8) * (gx / 8) + bx / 8 : (int64_t)bx;
}

// ------------------------------------------------------------------ shared limits
// Decode register-streaming tiles: K steps loaded U at a time (U = stream_unroll).
__host__ __device__ constexpr int stream_unroll(int mt, int nt) { return mt * nt >= 4 ? 2 : 4; }
// Largest workgroup whose waves keep the double-buffered fragments in registers.
__host__ __device__ constexpr int stream_max_threads(int mt, int nt) {
  return 2 * stream_unroll(mt, nt) * (mt + nt) * 4 + mt * nt * 4 <= 80 ? 1024 : 512;
}

// Weights-through-LDS decode tiles: the largest workgroup (threads) of a tile.
// 64-column tiles hold twice the weight fragments and accumulators, so they count double.
__host__ __device__ constexpr int wlds_bound(int mt, int ks, int nc = 16) {
  return mt * ks * (nc > 32 ? 2 : 1) <= 6 ? 1024 : 512;
}
// Whether the multi-step kernel's registers fit: two sets of activation fragments, the
// weight fragments of a step and the accumulators, in VGPRs (64 x 4 bytes each).
__host__ __device__ constexpr bool wlds_multi_fits(int mt, int nc, int ks) {
  return 8 * ks * mt + 4 * ks * (nc > 16 ? nc / 16 : 1) + 4 * mt * (nc > 16 ? nc / 16 : 1) <= 176;
}

constexpr size_t kMaxLds = 160 * 1024;  // LDS per CU, bytes
constexpr int kPipelined = 8;           // the overlapped-ring configs' stages: ring depth + 8

// Workgroup barrier without a memory fence or wait: the compiler keeps LDS accesses on their
// side of it, but outstanding LDS stores and reads are not waited for (gfx950's s_barrier does
// not wait, and the compiler adds no wait before it).  It suits the ring turns, where the
// buffers are written by direct-to-LDS loads that each wave waits for (vmcnt) before the
// barrier; LDS stores that other waves read after a barrier need __syncthreads().
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(N) (LGKM and EXP counters unconstrained), then a compiler fence so that
// no LDS read of the DMA'd data is scheduled above the wait.  Vector memory loads (the
// direct-to-LDS copies among them) complete in issue order, so vmcnt(N) means that all but
// the N most recent loads have landed.
template <int N>
__device__ __forceinline__ void wait_vmcnt_wlds() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}

// s_waitcnt lgkmcnt(0) (vector memory and EXP counters unconstrained): the wave's LDS reads
// have returned their data.
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
  asm volatile("" ::: "memory");
}

typedef __attribute__((address_space(3))) int8_t lds_i8_t;

// A 16-byte LDS store written as inline assembly, so that the compiler does not see an LDS
// store: with a direct-to-LDS copy in flight it would first wait for every vector-memory
// request (it cannot tell that the copy writes elsewhere).  The caller must not store where
// a copy in flight writes, and waits for the store itself (lgkmcnt, as lds_sync does) before
// other waves read it.  The s_nops give 21 wait states (s_nop N waits N + 1): an MFMA result
// needs up to 18 before a DS instruction may read it (16-pass XDL operations).
__device__ __forceinline__ void lds_store_b128(void* p, v4i v) {
  const uint32_t a = (uint32_t)(uintptr_t)(lds_i8_t*)p;
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 4\n\tds_write_b128 %0, %1" ::"v"(a), "v"(v) : "memory");
}
// The same for 8 bytes written by ordinary VALU code (no MFMA wait states needed).
__device__ __forceinline__ void lds_store_b64(void* p, uint32_t lo, uint32_t hi) {
  const uint32_t a = (uint32_t)(uintptr_t)(lds_i8_t*)p;
  const uint64_t v = (uint64_t)lo | ((uint64_t)hi << 32);
  asm volatile("ds_write_b64 %0, %1" ::"v"(a), "v"(v) : "memory");
}

// Workgroup barrier for data the waves exchange through LDS stores (ds_write): each wave's
// LDS operations have completed (lgkmcnt 0), then s_barrier.  Unlike __syncthreads() it does
// not wait for the wave's outstanding global loads and direct-to-LDS copies (vmcnt), so a
// weight copy requested before it stays in flight across it; it does not publish
// direct-to-LDS data to other waves (each wave waits for its own copies).
__device__ __forceinline__ void lds_sync() {
  wait_lgkmcnt0();
  lds_barrier();
}

// ------------------------------------------------------------------ host helpers
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

inline int elt_size(int dt) { return dt == I8L_BF16 || dt == I8L_F16 ? 2 : 4; }

// Opts a kernel in to `bytes` of dynamic LDS (needed above 64 KiB) on the current device,
// once per device; `done` is the kernel's set of devices already opted in.  An unsupported
// attribute is not fatal: the launch itself then reports the LDS overrun.
inline void lds_opt_in(const void* kern, size_t bytes, std::atomic<uint64_t>& done) {
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

// ------------------------------------------------------------------ schedules (host side)
// Decode (i8l_gemm_decode.hip).
int cu_count();   // compute units of the current device, 256 without one
bool stream_ok(const i8l_config& c);
bool wlds_ok(const i8l_config& c, int64_t K);
bool wlds_split_ok(const i8l_config& c, int64_t K);
int64_t wlds_split_workspace(const i8l_config& c, int64_t M, int64_t N);
hipError_t launch_wlds_split(const i8l_config& c, const int8_t* a, int64_t lda,
                             const int8_t* b, int64_t ldb, const Epi& e, int64_t K,
                             int32_t* ws, hipStream_t st);
hipError_t launch_stream(const i8l_config& c, const int8_t* a, int64_t lda, const int8_t* b,
                         int64_t ldb, const Epi& e, int K, hipStream_t st);
hipError_t launch_wlds(const i8l_config& c, const int8_t* a, int64_t lda, const int8_t* b,
                       int64_t ldb, const Epi& e, int64_t K, hipStream_t st);
bool wldsp_ok(const i8l_config& c, int64_t K);
bool wldsp_silu_ok(const i8l_config& c, int64_t K);
hipError_t launch_wldsp_silu(const i8l_config& c, const int8_t* a, int64_t lda, const int8_t* b,
                             int64_t ldb, const Epi& e, int round_silu, hipStream_t st);
hipError_t launch_wldsp(const i8l_config& c, const int8_t* a, int64_t lda, const int8_t* b,
                        int64_t ldb, const Epi& e, hipStream_t st);
bool dq_ok(const i8l_config& c, int64_t K);
int dq_max_rows(const i8l_config& c);
bool default_dq_config(int64_t N, int64_t K, i8l_config* c);
bool dq_silu_ok(const i8l_config& c, int64_t K);
bool default_dq_silu_config(int64_t N, int64_t K, i8l_config* c);
int dq_silu_max_rows();
// add + RMSNorm + quantize folded into the persistent decode GEMM (i8l_gemm_norm.hip).
bool nq_ok(const i8l_config& c, int64_t K);
bool default_nq_config(int64_t M, int64_t N, int64_t K, i8l_config* c);
int nq_max_rows();
hipError_t launch_nq(const i8l_config& c, int act_dtype, const uint16_t* x,
                     const uint16_t* residual, const uint16_t* gamma, float eps,
                     uint16_t* residual_out, const int8_t* b, int64_t ldb, const Epi& e,
                     float* sa_out, int precise, int act, hipStream_t st);
hipError_t launch_dq(const i8l_config& c, int act_dtype, const uint16_t* x, int64_t ldx,
                     const int8_t* b, int64_t ldb, const Epi& e, float* sa_out, int precise,
                     hipStream_t st);
hipError_t launch_dq_silu(const i8l_config& c, int act_dtype, int round_silu,
                          const uint16_t* gate_up, int64_t ldgu, int64_t up, const int8_t* b,
                          int64_t ldb, const Epi& e, float* sa_out, int precise,
                          hipStream_t st);
// Prefill (i8l_gemm_prefill.hip): the index of a config among the built tiles, or -1.
int staged_index(const i8l_config& c);
int dma_index(const i8l_config& c);
int dmap_index(const i8l_config& c);
hipError_t launch_staged(int idx, const i8l_config& c, const int8_t* a, int64_t lda,
                         const int8_t* b, int64_t ldb, const Epi& e, int K, hipStream_t st);
hipError_t launch_dma(int idx, const i8l_config& c, const int8_t* a, int64_t lda,
                      const int8_t* b, int64_t ldb, const Epi& e, int K, hipStream_t st);
hipError_t launch_dmap(int idx, const i8l_config& c, const int8_t* a, int64_t lda,
                       const int8_t* b, int64_t ldb, const Epi& e, int K, hipStream_t st);

}  // namespace i8l
