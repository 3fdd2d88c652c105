/*
 * sage_attn.h — C ABI of the MI355X (gfx950) SageAttention hot path.
 *
 * The library replaces the two device stages of TriBench's
 * kernels/sage_attn/triton_impl.py:
 *
 *   sage_prepass()  <- per_block_int8()              triton_impl.py:35-82
 *                      quant_per_block_int8_kernel() triton_impl.py:7-33
 *                      (+ the K channel-mean hook     triton_impl.py:39-40,
 *                         + FP8 V, which the reference does not have)
 *   sage_vtiles()   <- v.to(torch.float16)            triton_impl.py:189
 *                      (fused with the attention's V tile layout)
 *   sage_prepass_vt() <- both of the above in the pre-pass's launches
 *   sage_attn_fwd() <- _attn_fwd[grid](...) launch    triton_impl.py:186-199
 *                      _attn_fwd / _attn_fwd_inner    triton_impl.py:86-160
 *
 * and, with the same attention kernel on unquantized fp16/bf16 Q and K,
 * the flash_attn pack's forward:
 *
 *   sage_flash_fwd() <- run_flash_attn / _flash_attn_fwd_kernel
 *                       kernels/flash_attn/triton_impl.py:12-121
 *
 * The Python entry point that strings them together (the counterpart of
 * run_sage_attn, triton_impl.py:162-200) lives in
 * tribench_amd/kernels/sage_attn/hip_impl.py and binds this header with ctypes.
 *
 * Conventions
 *  - Every tensor is described by a base pointer, its logical sizes and the
 *    element strides of its batch, head and sequence dimensions (3 values,
 *    in that order).  The head-dim stride must be 1.  Row starts must be
 *    16-byte aligned.  This covers both of the reference's layouts
 *    ("HND" and "NHD", triton_impl.py:42-55).
 *  - The caller owns every device buffer.  The library never allocates or
 *    frees device memory and keeps no pointer after a call returns.
 *  - Every call is asynchronous on `stream` (a hipStream_t; NULL means the
 *    default stream) and returns 0 on success.  A non-zero status leaves a
 *    message in sage_last_error(); argument errors contain the words
 *    "invalid argument".
 *  - Head dims 64 and 128 are supported.
 */
#ifndef SAGE_ATTN_H
#define SAGE_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SAGE_ABI_VERSION 6

/* element types (dtype codes used by every entry point) */
#define SAGE_DTYPE_F32 0
#define SAGE_DTYPE_F16 1
#define SAGE_DTYPE_BF16 2
#define SAGE_DTYPE_FP8E4M3 3 /* OCP e4m3 ("e4m3fn"), bias 7, max 448 */
#define SAGE_DTYPE_VTILES 4  /* V in the tile layout of sage_vtiles() (type set by pv_mode) */

/* v_mode of sage_prepass */
#define SAGE_V_NONE 0      /* V is not touched by the pre-pass */
#define SAGE_V_FP8 1       /* per-channel FP8 e4m3 V: v_scale[c] = max|v[:,c]| / 448 and
                              v8 = RNE_sat(v / v_scale[c]), row-major like v */
#define SAGE_V_FP8_SCALE 2 /* v_scale only (for sage_vtiles with SAGE_PV_FP8) */

/* pv_mode of sage_attn_fwd: the operand type of the P.V product */
#define SAGE_PV_F16 0  /* P and V rounded to fp16 (the reference's choice, triton_impl.py:112-113,189) */
#define SAGE_PV_BF16 1 /* P and V in bf16 */
#define SAGE_PV_FP8 2  /* P and V in FP8 e4m3 with per-channel V scales */

/* Library version; bumped whenever a signature below changes. */
int sage_abi_version(void);

/* Message of the last failed call on the calling thread ("" if none). */
const char* sage_last_error(void);

/* Bytes of the V tile buffer of sage_vtiles() for the given problem and pv_mode. */
size_t sage_vtile_bytes(int64_t B, int64_t Hkv, int64_t Nkv, int64_t D, int pv_mode);

/* Bytes of scratch that sage_prepass needs for the given problem
 * (the per-chunk K channel sums and V channel maxima). */
size_t sage_prepass_workspace_bytes(int64_t B, int64_t Hkv, int64_t Nkv, int64_t D, int smooth_k,
                                    int v_mode);

/*
 * Pre-pass: INT8 per-block quantization of Q and K with fp32 scales.
 * Replaces per_block_int8() (triton_impl.py:35-82).
 *
 *  q [B,Hq,Nq,D], k [B,Hkv,Nkv,D], v [B,Hkv,Nkv,D]   in_dtype (F32/F16/BF16)
 *  q_mul     fp32 multiplier folded into Q before quantization; the
 *            reference passes fp32(sm_scale * 1.44269504) (triton_impl.py:69)
 *  blkq/blkk rows per scale block (reference: 128 / 64); 16 <= blk <= 256,
 *            multiples of 16
 *  q_sub     rows per Q scale: blkq (one scale per block, the reference), a
 *            divisor of blkq that is a multiple of 16 (per-wave scales), or 1
 *            (one scale per row: the rows one lane of the attention kernel's
 *            MFMA operand holds)
 *  smooth_k  1: km[c] = mean over tokens of k[..,c] (fp32, fixed reduction
 *            order), K is quantized as fp32(k) - km[c]
 *  outputs   q8 [B,Hq,Nq,D] int8 + q_scale [B,Hq,ceil(Nq/blkq)*(blkq/q_sub)]
 *            k8 [B,Hkv,Nkv,D] int8 + k_scale [B,Hkv,ceil(Nkv/blkk)]
 *            km [B,Hkv,D] fp32 (written when smooth_k; may be NULL otherwise)
 *            v8 [B,Hkv,Nkv,D] e4m3 bytes + v_scale [B,Hkv,D] (v_mode FP8)
 *            v_scale only (v_mode FP8_SCALE; v8 may be NULL)
 *  q8/k8/v8 strides are given like the input strides; scales, km and
 *  v_scale are dense.
 *  q, q_strides, q8, q8_strides and q_scale may all be NULL: K (and V) only,
 *  for sage_attn_fwd_q, which quantizes Q itself.
 */
int sage_prepass(const void* q, const void* k, const void* v, int in_dtype, int64_t B, int64_t Hq,
                 int64_t Hkv, int64_t Nq, int64_t Nkv, int64_t D, const int64_t* q_strides,
                 const int64_t* k_strides, const int64_t* v_strides, float q_mul, int blkq,
                 int blkk, int q_sub, int smooth_k, int v_mode, int8_t* q8,
                 const int64_t* q8_strides, float* q_scale, int8_t* k8, const int64_t* k8_strides,
                 float* k_scale, float* km, uint8_t* v8, const int64_t* v8_strides, float* v_scale,
                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * V converted to the P.V operand type and laid out in tiles of 64 keys for
 * sage_attn_fwd.  Replaces the reference's `v.to(torch.float16)` before the
 * attention launch (triton_impl.py:189).
 *
 *  v        [B,Hkv,Nkv,D] in in_dtype (F32/F16/BF16), strides as above
 *  pv_mode  SAGE_PV_F16 / SAGE_PV_BF16: round to that type (RNE);
 *           SAGE_PV_FP8: e4m3 codes RNE_sat(v / v_scale[b,h,d]) (0 where the
 *           scale is 0), v_scale [B,Hkv,D] from sage_prepass
 *  out      sage_vtile_bytes() bytes.  Element (b, h, key n, channel d) sits
 *           at element index (((b*Hkv + h)*T + n/64)*D + d)*64 + pos(n%64),
 *           T = ceil(Nkv/64), pos(32t + 8i + 4j + r) = 32j + 16t + 4i + r;
 *           keys past Nkv hold 0.
 */
int sage_vtiles(const void* v, int in_dtype, int64_t B, int64_t Hkv, int64_t Nkv, int64_t D,
                const int64_t* v_strides, int pv_mode, const float* v_scale, void* out,
                size_t out_bytes, void* stream);

/*
 * sage_prepass and sage_vtiles in one call (per_block_int8 and the
 * v.to(torch.float16) before the attention launch, triton_impl.py:35-82, 189):
 * the V tiles are written by the pre-pass's own launches — beside the K
 * statistics for fp16/bf16 P.V, beside the K quantization for FP8 P.V (whose
 * codes need v_scale, so v_mode must then be FP8 or FP8_SCALE).  The
 * outputs equal those of sage_prepass followed by sage_vtiles(v, in_dtype,
 * B, Hkv, Nkv, D, v_strides, pv_mode, v_scale, vtiles, vtile_bytes).
 *
 *  every argument of sage_prepass, then
 *  pv_mode      SAGE_PV_F16 / SAGE_PV_BF16 / SAGE_PV_FP8, as sage_vtiles
 *  vtiles       sage_vtile_bytes(B, Hkv, Nkv, D, pv_mode) bytes (vtile_bytes);
 *               v and v_strides are required
 */
int sage_prepass_vt(const void* q, const void* k, const void* v, int in_dtype, int64_t B, int64_t Hq,
                    int64_t Hkv, int64_t Nq, int64_t Nkv, int64_t D, const int64_t* q_strides,
                    const int64_t* k_strides, const int64_t* v_strides, float q_mul, int blkq,
                    int blkk, int q_sub, int smooth_k, int v_mode, int8_t* q8,
                    const int64_t* q8_strides, float* q_scale, int8_t* k8, const int64_t* k8_strides,
                    float* k_scale, float* km, uint8_t* v8, const int64_t* v8_strides, float* v_scale,
                    void* workspace, size_t workspace_bytes, int pv_mode, void* vtiles,
                    size_t vtile_bytes, void* stream);

/* Bytes of the fixed scratch array that sage_prepass_vt_noalloc uses on each GPU. */
#define SAGE_SCRATCH_BYTES (4u << 20)

/*
 * sage_prepass_vt without a workspace argument.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * per-chunk K channel sums and V channel maxima live in a scratch array of
 * SAGE_SCRATCH_BYTES inside the library, one copy per GPU, held until the
 * process ends; the call allocates nothing.  Problems whose
 * sage_prepass_workspace_bytes() exceeds SAGE_SCRATCH_BYTES fail with
 * "invalid argument" (every BASELINE configuration needs at most 1 MiB).
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (other streams, other host threads) race and must be serialized by the
 * caller.  Outputs equal those of sage_prepass_vt.
 *
 *  every argument of sage_prepass_vt except workspace and workspace_bytes
 */
int sage_prepass_vt_noalloc(const void* q, const void* k, const void* v, int in_dtype, int64_t B,
                            int64_t Hq, int64_t Hkv, int64_t Nq, int64_t Nkv, int64_t D,
                            const int64_t* q_strides, const int64_t* k_strides,
                            const int64_t* v_strides, float q_mul, int blkq, int blkk, int q_sub,
                            int smooth_k, int v_mode, int8_t* q8, const int64_t* q8_strides,
                            float* q_scale, int8_t* k8, const int64_t* k8_strides, float* k_scale,
                            float* km, uint8_t* v8, const int64_t* v8_strides, float* v_scale,
                            int pv_mode, void* vtiles, size_t vtile_bytes, void* stream);

/*
 * Fused attention: O = softmax2(dequant(Q8 K8^T)) V with an online,
 * base-2 softmax (the log2(e) factor is already folded into q_scale).
 * Replaces the _attn_fwd launch (triton_impl.py:186-199).
 *
 *  q8/q_scale/k8/k_scale  as written by sage_prepass (same blkq, q_sub, blkk)
 *  v      the V tiles of sage_vtiles() for the same pv_mode (v_dtype must be
 *         SAGE_DTYPE_VTILES; v_strides is not read and may be NULL);
 *         v_scale [B,Hkv,D] with SAGE_PV_FP8
 *  o      [B,Hq,Nq,D] in o_dtype (F32/F16/BF16)
 *  causal 1: key j is visible to query i iff j <= i (top-left aligned, the
 *         torch.tril mask of reference.py:19-22)
 *  GQA    query head h reads KV head h / (Hq/Hkv) (triton_impl.py:137,145,147)
 *  blkk must be 64, 128 or 256; q_sub 1 or a multiple of 32 that divides blkq.
 */
int sage_attn_fwd(const int8_t* q8, const int64_t* q8_strides, const float* q_scale,
                  const int8_t* k8, const int64_t* k8_strides, const float* k_scale,
                  const void* v, int v_dtype, const int64_t* v_strides, const float* v_scale,
                  void* o, int o_dtype, const int64_t* o_strides, int64_t B, int64_t Hq,
                  int64_t Hkv, int64_t Nq, int64_t Nkv, int64_t D, int causal, int blkq, int blkk,
                  int q_sub, int pv_mode, void* stream);

/*
 * sage_attn_fwd with the Q quantization of sage_prepass done in the kernel's
 * prologue (fused, so Q is read once and Q8 never reaches memory): the
 * per-block INT8 quantization of per_block_int8 (triton_impl.py:25-33, 63-71)
 * with the same arithmetic, hence the same Q8 and q_scale bit for bit.
 *
 *  q [B,Hq,Nq,D] in q_dtype (F32/F16/BF16); o has q's type, o_strides its own
 *  q_mul     fp32(sm_scale * 1.44269504), as for sage_prepass
 *  blkq      must be 128 (four 32-row waves); q_sub 1, 32, 64 or 128
 *  q8_out, q_scale_out  optional (NULL: not written): Q8 with q's element
 *            strides and q_scale [B,Hq,ceil(Nq/128)*(128/q_sub)]
 *  everything else as sage_attn_fwd.
 */
int sage_attn_fwd_q(const void* q, const int64_t* q_strides, int q_dtype, float q_mul, int8_t* q8_out,
                    float* q_scale_out, const int8_t* k8, const int64_t* k8_strides, const float* k_scale,
                    const void* v, int v_dtype, const int64_t* v_strides, const float* v_scale, void* o,
                    const int64_t* o_strides, int64_t B, int64_t Hq, int64_t Hkv, int64_t Nq, int64_t Nkv,
                    int64_t D, int causal, int blkq, int blkk, int q_sub, int pv_mode, void* stream);

/*
 * Unquantized attention: S = Q K^T from fp16/bf16 MFMAs (fp32 accumulate),
 * the online base-2 softmax of sage_attn_fwd, P rounded to the input type
 * (the reference casts p to V's dtype, kernels/flash_attn/triton_impl.py:87-88),
 * O += P V in fp32.  Replaces run_flash_attn (kernels/flash_attn/triton_impl.py:103-121).
 *
 *  q [B,Hq,Nq,D], k [B,Hkv,Nkv,D]  in_dtype (F16 or BF16), strides as above
 *  v       the V tiles of sage_vtiles() with pv_mode SAGE_PV_F16 for fp16
 *          inputs, SAGE_PV_BF16 for bf16 (v_dtype SAGE_DTYPE_VTILES;
 *          v_strides is not read and may be NULL)
 *  o       [B,Hq,Nq,D] in in_dtype
 *  qk_mul  fp32(sm_scale * 1.44269504): the scores in log2 units
 *  causal and GQA as in sage_attn_fwd.
 */
int sage_flash_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                   const void* v, int v_dtype, const int64_t* v_strides, void* o, const int64_t* o_strides,
                   int in_dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t Nq, int64_t Nkv, int64_t D,
                   float qk_mul, int causal, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SAGE_ATTN_H */
