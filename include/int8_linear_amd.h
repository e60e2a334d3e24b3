/*
 * int8_linear_amd.h -- C ABI of the MI355X (gfx950) W8A8 linear path.
 *
 * Every entry point takes raw device pointers, element strides, sizes, dtype codes and the
 * caller's hipStream_t (passed as void* so that this header needs no HIP include).  The
 * library never allocates, frees or synchronises, and never touches host memory on the hot
 * path: it validates, launches on `stream`, and returns.  Launches are therefore legal
 * inside hipGraph stream capture.  Outputs are allocated by the caller, as in the
 * reference's Python wrappers (int8_linear/kernel.py:242, int8_linear/fused_quant.py:100-102,
 * 118-119 of AshrithaG/int8-linear).
 *
 * Return value of every entry point is an i8l_status.  On a non-zero status,
 * i8l_last_error() returns a thread-local, NUL-terminated description of the last failure.
 * The Python host layer maps I8L_UNSUPPORTED to int8_linear.NotSupported, I8L_INVALID_ARG to
 * ValueError and I8L_HIP_ERROR to RuntimeError, which is the reference's error convention
 * (int8_linear/kernel.py:45-46, 221-238).
 */
#ifndef INT8_LINEAR_AMD_H
#define INT8_LINEAR_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
enum {
  I8L_OK = 0,
  I8L_UNSUPPORTED = 1, /* the kernels do not take this shape/dtype/config: caller falls back */
  I8L_INVALID_ARG = 2, /* inconsistent shapes or sizes */
  I8L_HIP_ERROR = 3    /* a HIP runtime call failed (launch error, no device, ...) */
};

/* Element type codes for bias, outputs and bf16/fp16 activations. */
enum {
  I8L_DTYPE_NONE = 0, /* "no tensor" (bias absent) */
  I8L_BF16 = 1,
  I8L_F16 = 2,
  I8L_F32 = 3,
  I8L_I32 = 4         /* GEMM output only: the raw int32 product (reference raw=True) */
};

/*
 * Tile configuration of one GEMM launch; mirrors int8_linear.kernel.Config
 * (reference int8_linear/kernel.py:49-60) with the MI355X meaning of each field:
 *   bm, bn, bk : output rows (tokens) x output columns x K bytes per workgroup step
 *   warps      : wavefronts (64 lanes) per workgroup
 *   stages     : the schedule: 1 weights streamed into registers (decode); 3 with bm <= 128
 *                and bn <= 64 weights through LDS (decode); 4 with bn <= 32 the same in one
 *                K step a wave, each workgroup walking several column tiles with the
 *                activations held in registers (decode, K == bk * warps); 5 the stages-3
 *                tile with K split over group_m workgroups and their int32 partials summed
 *                by a second kernel (decode; needs a workspace, see i8l_w8a8_mm_ws); 2 LDS
 *                staged through registers, 3..8 a ring of that many direct-to-LDS buffers,
 *                >= 10 a ring of stages - 8 buffers (2: a double buffer) with fragment reads
 *                overlapped with the MFMAs (prefill)
 *   group_m    : rows of tiles walked together for L2 reuse (1 = row-major order); stages 3
 *                with bn <= 64: 3 keeps two K steps in flight (three step buffers a
 *                wave), 4 three (four buffers), else one; with stages 4, the workgroups a compute unit runs at once (1, 2 or 4); with
 *                stages 5, the parts K is split into (2, 4 or 8)
 * A config the library was not built for returns I8L_UNSUPPORTED.
 */
typedef struct i8l_config {
  int32_t bm, bn, bk, warps, stages, group_m;
} i8l_config;

/*
 * W8A8 scaled matmul:  out[m,n] = cast( f32(sum_k A[m,k]*B[k,n]) * sa[m|0] * sb[n|0] + f32(bias[n]) )
 * with the int32 sum exact and the epilogue evaluated left to right in fp32 with no fused
 * multiply-add, then one round-to-nearest-even cast.  out_dtype I8L_I32 writes the raw int32
 * product and ignores scales and bias.
 *
 * A is int8 [M,K] at a + m*stride_am + k*stride_ak.  B is int8 [K,N] at b + k*stride_bk +
 * n*stride_bn; the fast schedules want stride_bk == 1 (the transposed view of an [N,K]
 * nn.Linear weight, as vLLM passes it).  Other strides and unaligned pointers run a
 * correct generic kernel.  scale_a has scale_a_len 1 or M fp32 values, scale_b has 1 or N.
 * bias is NULL (bias_dtype I8L_DTYPE_NONE) or N values of bf16/f16/f32.  out is [M,N] with
 * row stride stride_cm and unit column stride, of out_dtype bf16/f16/f32/i32.
 * cfg NULL picks the library default for (M,N,K).
 *
 * A config that splits K (stages 5) needs a workspace: this entry declines it with
 * I8L_UNSUPPORTED; i8l_w8a8_mm_ws takes it.
 *
 * Replaces the reference's launch of the Triton kernel _w8a8_mm from
 * w8a8_mm (int8_linear/kernel.py:202-257; kernel body 63-124).
 */
int i8l_w8a8_mm(const int8_t* a, int64_t stride_am, int64_t stride_ak,
                const int8_t* b, int64_t stride_bk, int64_t stride_bn,
                const float* scale_a, int64_t scale_a_len,
                const float* scale_b, int64_t scale_b_len,
                const void* bias, int32_t bias_dtype,
                void* out, int64_t stride_cm, int32_t out_dtype,
                int64_t M, int64_t N, int64_t K,
                const i8l_config* cfg, void* stream);

/*
 * Bytes of device workspace that i8l_w8a8_mm_ws needs for (M,N,K,cfg): group_m * M * N * 4
 * for a split of K (stages 5: one int32 partial plane per part), 0 for every other
 * schedule and for cfg NULL (the default config never splits).  Host-only; always >= 0.
 * Replaces nothing in the reference (its Triton kernel keeps the whole K loop in one
 * program, int8_linear/kernel.py:94-103); it sizes the buffer the caller allocates.
 */
int64_t i8l_w8a8_mm_workspace_bytes(int64_t M, int64_t N, int64_t K, const i8l_config* cfg);

/*
 * i8l_w8a8_mm with a caller-allocated device workspace of workspace_bytes bytes, 16-byte
 * aligned (NULL and 0 when i8l_w8a8_mm_workspace_bytes is 0).  Only a split of K uses it:
 * the first kernel writes every byte it later reads, so the contents on entry do not
 * matter, and on return they are undefined.  Calls in flight at the same time must not
 * share a workspace.  A workspace smaller than needed returns I8L_INVALID_ARG.
 * Replaces the same reference launch as i8l_w8a8_mm (int8_linear/kernel.py:202-257), with
 * the kernel's K loop (kernel.py:94-103) split across workgroups for stages 5.
 */
int i8l_w8a8_mm_ws(const int8_t* a, int64_t stride_am, int64_t stride_ak,
                   const int8_t* b, int64_t stride_bk, int64_t stride_bn,
                   const float* scale_a, int64_t scale_a_len,
                   const float* scale_b, int64_t scale_b_len,
                   const void* bias, int32_t bias_dtype,
                   void* out, int64_t stride_cm, int32_t out_dtype,
                   int64_t M, int64_t N, int64_t K,
                   void* workspace, int64_t workspace_bytes,
                   const i8l_config* cfg, void* stream);

/*
 * The gate_up projection with the SiLU-and-mul in its epilogue, for few tokens (M <= 16):
 *   y = cast(silu(g) * u)  [M, N/2] bf16,  g | u = i8l_w8a8_mm(a, b, scale_a, scale_b, bias)
 * where g is the product's first N/2 columns and u its last N/2, each rounded to bf16 first
 * (the gate_up output); round_silu rounds silu(g) to bf16 before the product.  These are the
 * values i8l_silu_mul_quant quantizes, bit for bit, so i8l_quant_per_token(y) (or the
 * quantizer folded into the next GEMM, i8l_w8a8_mm_dynq) gives silu_mul_quant's codes and
 * scales.  Each workgroup's tile pairs gate and up columns, so every value is computed once.
 * a int8 [M,K] K-contiguous, b the K-contiguous [K,N] view, scale_b per channel [N], bias
 * none or bf16 [N]; out bf16 with row pitch stride_cm >= N/2, 16-byte aligned.  cfg is a
 * persistent single-step tile (bm 16, bn 8 or 16, stages 4, K == warps * bk) or NULL.
 *
 * Replaces the reference's gate_up_proj _w8a8_mm and the SiLU-and-mul half of
 * silu_mul_quant (bench/fuse_quant.py:236-240; kernel.py:63-124, fused_quant.py:76-88).
 */
int i8l_w8a8_mm_silu_mul(const int8_t* a, int64_t stride_am, const int8_t* b, int64_t stride_bk,
                         int64_t stride_bn, const float* scale_a, int64_t scale_a_len,
                         const float* scale_b, int64_t scale_b_len, const void* bias,
                         int32_t bias_dtype, void* out, int64_t stride_cm, int32_t round_silu,
                         int64_t M, int64_t N, int64_t K, const i8l_config* cfg, void* stream);

/* Whether i8l_w8a8_mm_silu_mul takes (M,N,K,cfg) (cfg NULL: the library's choice); host-only. */
int i8l_w8a8_mm_silu_mul_supported(int64_t M, int64_t N, int64_t K, const i8l_config* cfg);

/*
 * i8l_w8a8_mm for callers that cannot allocate: code under HIP graph capture, serving loops
 * and harnesses that forbid allocation.  No counterpart in the reference (its Triton kernel
 * needs no workspace).  Same arguments, validation and results as i8l_w8a8_mm_ws, but a
 * split of K (stages 5) keeps its partial planes in a device array of the library itself,
 * 16 MiB on each GPU it runs on (held until the process ends); a config that needs more
 * (group_m * M * N * 4 bytes > 16 MiB) returns I8L_UNSUPPORTED.  No call allocates or frees
 * memory.  All calls on one GPU share that array: calls that overlap in time on one GPU race.
 */
int i8l_w8a8_mm_noalloc(const int8_t* a, int64_t stride_am, int64_t stride_ak,
                        const int8_t* b, int64_t stride_bk, int64_t stride_bn,
                        const float* scale_a, int64_t scale_a_len,
                        const float* scale_b, int64_t scale_b_len,
                        const void* bias, int32_t bias_dtype,
                        void* out, int64_t stride_cm, int32_t out_dtype,
                        int64_t M, int64_t N, int64_t K,
                        const i8l_config* cfg, void* stream);

/*
 * Library set-up on one GPU (device -1: the calling thread's current device): looks up the
 * device address of i8l_w8a8_mm_noalloc's scratch array there, with that device made
 * current and the thread's previous current device restored before returning.  Optional:
 * i8l_w8a8_mm_noalloc does the same on its first call on a device otherwise.  Call it once
 * per GPU at set-up, before any HIP graph capture, so that no later call switches devices
 * or looks up a symbol.  Allocates nothing beyond the array the library holds on every GPU
 * it runs on.  No counterpart in the reference; host-only, safe to call more than once.
 */
int i8l_init(int32_t device);

/*
 * Whether i8l_w8a8_mm takes this (M,N,K,cfg) on a fast schedule: returns I8L_OK or
 * I8L_UNSUPPORTED without launching anything (host-only; no GPU needed).  The decline
 * rule is the reference's: N % bn or K % bk non-zero (int8_linear/kernel.py:228-229),
 * or a tile the library was not built for.
 */
int i8l_w8a8_mm_supported(int64_t M, int64_t N, int64_t K, const i8l_config* cfg);

/* The default config the library uses for (M,N,K) (reference default_config,
 * int8_linear/kernel.py:127-134, re-derived for MI355X). Host-only. */
int i8l_default_config(int64_t M, int64_t N, int64_t K, i8l_config* cfg_out);

/*
 * Fused add + RMSNorm + per-token int8 quantize, one row per token:
 *   x = f32(x) (+ f32(residual));  residual_out = cast(x)          (when residual != NULL)
 *   var = sum(x^2)/H;  xn = x * rsqrt(var + eps)
 *   y = cast_x( f32(cast_w(xn)) * f32(weight) )
 *   scale = absmax(y)/127;  q = clamp(rne(y * 127/absmax), -128, 127)   (0 for a zero row)
 * x, residual, residual_out: [M,H] contiguous of act_dtype (bf16/f16); weight [H] of
 * w_dtype (bf16/f16); q int8 [M,H]; scale fp32 [M].  residual and residual_out are both
 * NULL or both non-NULL.  precise_div 1 = IEEE divisions; 0 = multiply by the IEEE
 * reciprocal.  M == 0 launches nothing.
 * Replaces add_rmsnorm_quant / _add_rmsnorm_quant_kernel (int8_linear/fused_quant.py:56-73,
 * 95-110); residual == NULL is rmsnorm_quant (fused_quant.py:132-135).
 */
int i8l_add_rmsnorm_quant(const void* x, const void* residual, const void* weight, float eps,
                          int8_t* q, float* scale, void* residual_out,
                          int64_t M, int64_t H, int32_t act_dtype, int32_t w_dtype,
                          int32_t precise_div, void* stream);

/*
 * Fused SiLU-and-mul + per-token int8 quantize:
 *   g = f32(gate_up[m, :I]), u = f32(gate_up[m, I:]);  a = g / (1 + exp(-g))
 *   a = f32(cast(a)) if round_silu;  y = f32(cast(a*u));  then the quantizer above.
 * gate_up [M, 2I] contiguous bf16/f16; q int8 [M,I]; scale fp32 [M].
 * Replaces silu_mul_quant / _silu_mul_quant_kernel (int8_linear/fused_quant.py:76-88, 113-124).
 */
int i8l_silu_mul_quant(const void* gate_up, int8_t* q, float* scale,
                       int64_t M, int64_t I, int32_t act_dtype,
                       int32_t round_silu, int32_t precise_div, void* stream);

/*
 * Plain per-token int8 quantize of a bf16/f16 [M,H] tensor whose rows lie ldx elements apart
 * (ldx >= H; ldx == H is a contiguous tensor): the quantizer of
 * int8_linear/fused_quant.py:41-53 on its own.  Stands in for vLLM's scaled_int8_quant, which
 * the reference's decoder stand-in calls on the o_proj input (bench/fuse_quant.py:234,
 * bench/situ_tune.py:110).  With ldx > H it quantizes a column slice in place, e.g. the
 * q columns of a qkv output, which the reference first copies with .contiguous()
 * (bench/fuse_quant.py:233).
 */
int i8l_quant_per_token(const void* x, int64_t ldx, int8_t* q, float* scale,
                        int64_t M, int64_t H, int32_t act_dtype,
                        int32_t precise_div, void* stream);

/*
 * The per-token quantizer and the W8A8 matmul in one launch, for few tokens:
 *   out = i8l_w8a8_mm(quant(x), b, scale_a = the quantizer's scales, scale_b, bias)
 * bit for bit, where quant is i8l_quant_per_token.  x is bf16/f16 [M,K] with row stride ldx
 * (a multiple of 8 elements, >= K; a column slice such as the q columns of a qkv output is
 * read in place) and a 16-byte aligned base.  Every column tile quantizes its token rows
 * itself, so the work grows with M times the number of column tiles: the host layer takes
 * this path for M <= 8 (the library takes any M and gives the same bits).  scale_a_out, if not NULL, receives the M per-token scales.
 * b must be K-contiguous (stride_bk == 1) and 16-byte aligned, out 16-byte aligned with
 * 16-byte row pitch; anything else returns I8L_UNSUPPORTED (use the two calls).  cfg is a
 * single-step weights-through-LDS tile with 16 waves (bm 16, bn 8/16/32, bk 128 or 256,
 * stages 3, K == 16 * bk) or NULL for the library's choice.
 *
 * Replaces the pair the reference's stand-in issues per o_proj, vLLM's scaled_int8_quant
 * then _w8a8_mm (bench/fuse_quant.py:233-235 of AshrithaG/int8-linear; kernel.py:202-257).
 */
int i8l_w8a8_mm_dynq(const void* x, int64_t ldx, int32_t act_dtype, int32_t precise_div,
                     const int8_t* b, int64_t stride_bk, int64_t stride_bn,
                     const float* scale_b, int64_t scale_b_len,
                     const void* bias, int32_t bias_dtype,
                     void* out, int64_t stride_cm, int32_t out_dtype, float* scale_a_out,
                     int64_t M, int64_t N, int64_t K,
                     const i8l_config* cfg, void* stream);

/* Whether i8l_w8a8_mm_dynq takes (M,N,K,cfg) (cfg NULL: the library's choice); host-only. */
int i8l_w8a8_mm_dynq_supported(int64_t M, int64_t N, int64_t K, const i8l_config* cfg);

/*
 * The SiLU-and-mul quantizer and the W8A8 matmul in one launch, for few tokens:
 *   out = i8l_w8a8_mm(q, b, scale_a = s, scale_b, bias)  with  (q, s) = silu_mul_quant(gate_up)
 * bit for bit (i8l_silu_mul_quant with the same round_silu and precise_div).  gate_up is
 * bf16/f16 [M, 2K] with row stride ldgu (a multiple of 8 elements, >= 2K) and a 16-byte aligned
 * base: the gate values in columns [0, K), the up values in [K, 2K); K is the matmul's K (the
 * MLP's intermediate size) and a multiple of 8.  Every column tile computes the SiLU-and-mul
 * and the row scales of its token rows itself, so the work grows with M times the number of
 * column tiles: M is at most 8 (larger M returns I8L_UNSUPPORTED; use the two calls).
 * scale_a_out, if not NULL, receives the M per-token scales.  b must be K-contiguous
 * (stride_bk == 1) and 16-byte aligned, out 16-byte aligned with 16-byte row pitch.  cfg is a
 * single-step weights-through-LDS tile of the SiLU form (bm 16, bn 8, bk 512, 12 waves,
 * stages 3, K == 12 * 512) or NULL for the library's choice.
 *
 * Replaces the pair the reference's stand-in issues per down_proj, silu_mul_quant then
 * _w8a8_mm (bench/fuse_quant.py:238-240 of AshrithaG/int8-linear; fused_quant.py:113-124 and
 * kernel.py:202-257).
 */
int i8l_silu_mul_quant_mm(const void* gate_up, int64_t ldgu, int32_t act_dtype,
                          int32_t round_silu, int32_t precise_div,
                          const int8_t* b, int64_t stride_bk, int64_t stride_bn,
                          const float* scale_b, int64_t scale_b_len,
                          const void* bias, int32_t bias_dtype,
                          void* out, int64_t stride_cm, int32_t out_dtype, float* scale_a_out,
                          int64_t M, int64_t N, int64_t K,
                          const i8l_config* cfg, void* stream);

/* Whether i8l_silu_mul_quant_mm takes (M,N,K,cfg) (cfg NULL: the library's choice);
 * host-only. */
int i8l_silu_mul_quant_mm_supported(int64_t M, int64_t N, int64_t K, const i8l_config* cfg);

/*
 * add + RMSNorm + per-token int8 quantize and the W8A8 matmul in one launch, for few tokens:
 *   (q, s, residual_out) = i8l_add_rmsnorm_quant(x, residual, weight, eps)
 *   out = i8l_w8a8_mm(q, b, scale_a = s, scale_b, bias)
 * bit for bit (same precise_div).  x, residual and residual_out are [M,K] contiguous of
 * act_dtype (bf16/f16), weight [K] of act_dtype; residual and residual_out are both NULL
 * (plain RMSNorm, rmsnorm_quant) or both given.  residual_out is written once (by one
 * workgroup).  Every workgroup normalizes the token rows itself, so M is at most 8 (larger
 * M returns I8L_UNSUPPORTED; use the two calls).  scale_a_out, if not NULL, receives the M
 * per-token scales.  b must be K-contiguous (stride_bk == 1) and 16-byte aligned, every
 * activation pointer and out 16-byte aligned with 16-byte row pitch.  cfg is a persistent
 * single-step tile of this form (bm 16, bn 8 or 16, bk 256 or 512, 4 or 8 waves, stages 4,
 * K == warps * bk a power of two, group_m workgroups a compute unit) or NULL for the
 * library's choice.  epilogue_act 0 writes the product out [M,N]; 1 and 2 treat b as a
 * gate_up weight (gate rows [0, N/2), up rows [N/2, N)) and write
 *   y = cast(silu(g) * u)  [M, N/2] bf16   (2: silu(g) rounded to bf16 first),
 * the values i8l_silu_mul_quant quantizes, from the bf16 products g, u (bf16 activations and
 * output, per-channel scale_b, no bias, a residual; else I8L_UNSUPPORTED).
 *
 * Replaces the pair the reference's stand-in issues before its qkv and gate_up projections,
 * add_rmsnorm_quant then _w8a8_mm (bench/fuse_quant.py:226-240 of AshrithaG/int8-linear;
 * int8_linear/fused_quant.py:56-73, 95-110 and kernel.py:202-257).
 */
int i8l_add_rmsnorm_quant_mm(const void* x, const void* residual, const void* weight, float eps,
                             int32_t act_dtype, int32_t precise_div, int32_t epilogue_act,
                             void* residual_out,
                             const int8_t* b, int64_t stride_bk, int64_t stride_bn,
                             const float* scale_b, int64_t scale_b_len,
                             const void* bias, int32_t bias_dtype,
                             void* out, int64_t stride_cm, int32_t out_dtype, float* scale_a_out,
                             int64_t M, int64_t N, int64_t K,
                             const i8l_config* cfg, void* stream);

/* Whether i8l_add_rmsnorm_quant_mm takes (M,N,K,cfg) (cfg NULL: the library's choice);
 * host-only. */
int i8l_add_rmsnorm_quant_mm_supported(int64_t M, int64_t N, int64_t K, const i8l_config* cfg);

/* Thread-local description of the last failure ("" if none). */
const char* i8l_last_error(void);

/* Library version string, e.g. "int8_linear_amd 0.1.0 gfx950". */
const char* i8l_version(void);

#ifdef __cplusplus
}
#endif

#endif /* INT8_LINEAR_AMD_H */
