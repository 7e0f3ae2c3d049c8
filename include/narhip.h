/*
 * narhip -- MI355X (gfx950) kernels for NAR's online rotate-and-quantize path.
 *
 * C ABI: plain pointers (device memory unless stated), sizes in elements,
 * the HIP stream to launch on.  Every entry point validates its arguments on
 * the host, launches asynchronously on `stream`, and returns NARHIP_OK or a
 * negative code; narhip_last_error_string() then describes the failure (per
 * calling thread).  No entry point allocates device memory: scratch space is
 * passed in through `workspace` (size from the matching *_workspace query).
 *
 * Layouts (row-major, identical to the reference's):
 *   x        bf16 [tokens, ld_x]                     (ld_x >= n, ld_x % 8 == 0)
 *   v        fp32 [n, k]      Y'  (u = x V)
 *   w_t      fp32 [k, n]      W''^T (x' = H x - u W''^T, i.e. U = -W'')
 *   partial  fp32 [tokens, splits*k], partial[t, s*k + r] = sum over split s
 *   codes    uint8 [rows, n/2], byte j = q[2j] | q[2j+1] << 4
 *   scales, zeros  fp16 [rows, n/group]
 * with rows = tokens, or the destination rows named by dest_rows[t].
 */
#ifndef NARHIP_H
#define NARHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NARHIP_ABI_VERSION 1

enum {
    NARHIP_OK = 0,
    NARHIP_EINVAL = -1,        /* invalid argument (maps to ValueError)   */
    NARHIP_EUNSUPPORTED = -2,  /* shape/mode not built (ValueError)       */
    NARHIP_EHIP = -3,          /* HIP runtime error (RuntimeError)        */
    NARHIP_EWORKSPACE = -4     /* workspace missing or too small          */
};

/* Rank-k arithmetic selection for narhip_rotate_quant / narhip_group_quant. */
enum {
    NARHIP_RANK_AUTO = 0,      /* MFMA for k >= 16 over a full row, else exact */
    NARHIP_RANK_EXACT = 1,     /* fp64 accumulation, one rounding (VALU)       */
    NARHIP_RANK_MFMA = 2       /* bf16 MFMA with split-precision factor terms  */
};

/* ABI version of the loaded library (NARHIP_ABI_VERSION at build time). */
int narhip_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char *narhip_last_error_string(void);

/* Host memory: the +-1 Paley Hadamard factor of order m (12, 20, 28, 68, 76
 * or 200) that the kernels use, row-major int8 [m, m].  Replaces the
 * constructions _paley_hadamard_12 (nar/extended_experiment.py:459-472),
 * paley_hadamard_28 (nar/activation_experiments.py:114-128) and
 * paley_hadamard (nar/activation_experiments.py:141-185), unnormalised. */
int narhip_paley(int32_t m, int8_t *out_host);

/* Fused rotate -> rank-k -> INT4 quantize (one call per batch of tokens).
 *
 * Replaces, for one call: full_hadamard_rows(x, signs)
 * (nar/activation_experiments.py:188-217) or the block FWHT of
 * nar/kernels/r4_fused_v2.py:43-52, the rank-k term of
 * quarot-llama3/nar_r4_kernel.py:190-202, and dynamic_asym_int4
 * (nar/experiment.py:158-184) with the packed layout of
 * nar/kernels/r4_fused_v2.py:67-92 -- i.e. the Python launchers
 * launch_nar_fused / launch_hadamard (nar/kernels/r4_fused_v2.py:327-350).
 *
 *   had_m, had_q : Hadamard blocks of had_m*had_q channels get H_m (x) H_q;
 *                  had_m in {1, 12, 20, 28}, had_q a power of two in [128, 1024]
 *                  (H_20: 128 or 256), or had_m = 1, had_q = n in {2048, 4096,
 *                  8192} (one FWHT over the row, k = 0).
 *                  had_m = 1 with had_q < n is the block Hadamard of nar/kernels;
 *                  had_m > 1 requires had_m*had_q = n (one Kronecker row).
 *   signs        : fp32 [n] or NULL, applied to the Hadamard input only.
 *   k            : rank (0 = Hadamard only), <= 64.
 *   rank_block   : n (one projection over the row) or had_q (independent
 *                  per-block factors, e.g. per KV head; needs k <= 8).
 *   v, w_t       : fp32 factors (see layouts above).
 *   prepared     : optional output of narhip_prepare_rank_factors for (v, w_t);
 *                  NULL = prepared in the workspace on every call.
 *   partial      : optional precomputed projection partials (splits >= 1);
 *                  NULL = computed here.
 *   group        : 32, 64 or 128, dividing had_q.
 *   rotated      : optional fp32 [tokens, n] copy of x' before quantization.
 *   dest_rows    : optional int64 [tokens]: token t writes output row dest_rows[t]
 *                  (a KV-cache slot); NULL = row t.  Values must be valid rows.
 *   rank_mode    : NARHIP_RANK_*.
 */
int narhip_rotate_quant(const void *x_bf16, int64_t tokens, int64_t n, int64_t ld_x,
                        int32_t had_m, int32_t had_q, const float *signs,
                        int32_t k, int64_t rank_block, const float *v, const float *w_t,
                        const void *prepared, const float *partial, int32_t splits,
                        int32_t group, uint8_t *codes, void *scales_f16, void *zeros_f16,
                        float *rotated, const int64_t *dest_rows, int32_t rank_mode,
                        void *workspace, size_t workspace_bytes, void *stream);

/* Allocation-free narhip_rotate_quant.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments and
 * results as narhip_rotate_quant without the workspace: the scratch the call
 * needs comes from a per-device array of NARHIP_NOALLOC_SCRATCH_BYTES that the
 * library holds from its load until the process ends; the MFMA rank path
 * processes the tokens in chunks (>= 256 tokens) that fit in it.  Arguments
 * whose scratch still exceeds it (e.g. RANK_EXACT with a Kronecker factor over
 * more than ~1000 rows of 14336) fail with NARHIP_EWORKSPACE.  The call
 * allocates nothing and leaves the scratch holding its own data; every byte it
 * reads there it has written first.  Calls that overlap on one GPU (concurrent
 * streams, or host threads) share that GPU's scratch and race: serialize them.
 */
#define NARHIP_NOALLOC_SCRATCH_BYTES (64ll << 20)

int narhip_rotate_quant_noalloc(const void *x_bf16, int64_t tokens, int64_t n, int64_t ld_x,
                                int32_t had_m, int32_t had_q, const float *signs,
                                int32_t k, int64_t rank_block, const float *v, const float *w_t,
                                const void *prepared, const float *partial, int32_t splits,
                                int32_t group, uint8_t *codes, void *scales_f16, void *zeros_f16,
                                float *rotated, const int64_t *dest_rows, int32_t rank_mode, void *stream);

/* Workspace bytes narhip_rotate_quant needs for these arguments (0 when none;
 * have_partial / have_prepared = 1 when the caller passes them). */
size_t narhip_rotate_quant_workspace(int64_t tokens, int64_t n, int32_t had_m, int32_t had_q,
                                     int32_t k, int64_t rank_block, int32_t have_partial,
                                     int32_t splits, int32_t have_prepared, int32_t rank_mode);

/* Bytes of the prepared rank factors for (n, k): V and W''^T as three exact
 * bf16 terms each in the MFMA layouts.  Replaces the term preparation of
 * FoldedR4.from_factor (nar/fold_signed_permutation.py:80-95) and fp16_terms /
 * w_terms (quarot-llama3/nar_r4_kernel.py:151-187). */
size_t narhip_rank_factors_bytes(int64_t n, int32_t k);

/* Fill `prepared` from fp32 v [n, k] and/or w_t [k, n] (either may be NULL to
 * refresh only the other half). */
int narhip_prepare_rank_factors(const float *v, const float *w_t, int64_t n, int32_t k,
                                void *prepared, size_t prepared_bytes, void *stream);

/* Kernel A: rank-k projection partials.
 * Replaces projection_triton_fp32 / rank_projection_kernel
 * (nar/kernels/r4_fused_v2.py:122-152, 292-303) and launch_projection_dot
 * (nar/kernels/r4_fused_v3.py:83-135, 187-201): partial[t, s*k + r] holds the
 * sum over the s-th of `splits` equal channel chunks.  The MFMA form (rank_mode
 * MFMA, or AUTO with k >= 16, `prepared` given and n % (128*splits) == 0)
 * reads `prepared`; the exact form reads `v`. */
int narhip_rank_projection(const void *x_bf16, int64_t tokens, int64_t n, int64_t ld_x,
                           const float *v, const void *prepared, int32_t k, int32_t splits,
                           float *partial, int32_t rank_mode, void *stream);

/* Kernel B: rotate, fold the split partials into u, subtract u W''^T, quantize.
 * Replaces nar_group_quant_kernel / launch_nar (nar/kernels/r4_fused_v2.py:
 * 155-178, 306-324; nar/kernels/r4_fused_v3.py:206-234, 251-261). */
int narhip_group_quant(const void *x_bf16, int64_t tokens, int64_t n, int64_t ld_x,
                       int32_t had_m, int32_t had_q, const float *partial, int32_t splits,
                       int32_t k, const float *w_t, const void *prepared, int32_t group,
                       uint8_t *codes, void *scales_f16, void *zeros_f16, int32_t rank_mode,
                       void *workspace, size_t workspace_bytes, void *stream);

/* Dequantize packed codes: out[r, i] = q * s + z (fp32 multiply then add).
 * Replaces dequantize (nar/kernels/r4_fused_v2.py:364-369). */
int narhip_dequantize(const uint8_t *codes, const void *scales_f16, const void *zeros_f16,
                      int64_t rows, int64_t n, int32_t group, float *out, void *stream);

/* The hooks' quantizer on the GPU: dynamic_asym_int4 over rows x n elements of
 * x (dtype 0 fp32, 1 bf16, 2 fp16), groups of `group` consecutive elements
 * (a power of two in [8, 512] dividing n).  Outputs in the reference's tuple
 * layout: codes uint8 [rows, n] (one code per byte), scales and zeros fp16
 * [rows, n/group], deq [rows, n] in the input dtype.  Replaces
 * dynamic_asym_int4 (nar/experiment.py:158-184) for device tensors. */
int narhip_dynamic_asym_int4(const void *x, int32_t dtype, int64_t rows, int64_t n, int32_t group,
                             uint8_t *codes, void *scales_f16, void *zeros_f16, void *deq, void *stream);

/* Rotate, then the hooks' quantizer, in one call: dynamic_asym_int4's tuple
 * (codes uint8 [tokens, n] one per byte, scales and zeros fp16
 * [tokens, n/group], deq fp32 [tokens, n]) of x' = H_s x - (x V) W''^T, with the
 * transform arguments of narhip_rotate_quant (no prepared factors, partials,
 * destination rows or rotated copy) and any group a power of two in [8, 512]
 * dividing n.  Replaces the hook sequence full_hadamard_rows or
 * RotationFactor.apply followed by dynamic_asym_int4
 * (nar/activation_experiments.py:295-299,603-606; nar/experiment.py:904-906;
 * nar/e14_w4a4kv4.py:725).  One kernel, reading x once, for groups of 32, 64
 * or 128 dividing had_q on: block / per-head Hadamards with no rank term or a
 * per-block rank (rank_block = had_q, k <= 8), the full-row FWHT of
 * n in {2048, 4096, 8192}, and H_m (x) H_q without a rank term (rank_mode
 * AUTO or MFMA); otherwise x' is staged in the workspace and quantized by a
 * second kernel.  had_m in {68, 76, 200} (the Qwen3 widths, n = m q <= 32768)
 * runs the whole-row Paley kernel, with no rank term or an exact full-row one
 * (rank_block = n, k <= 64), then the quantizer. */
size_t narhip_rotate_dynamic_asym_int4_workspace(int64_t tokens, int64_t n, int32_t had_m, int32_t had_q,
                                                 int32_t k, int64_t rank_block, int32_t group, int32_t rank_mode);
int narhip_rotate_dynamic_asym_int4(const void *x_bf16, int64_t tokens, int64_t n, int64_t ld_x, int32_t had_m,
                                    int32_t had_q, const float *signs, int32_t k, int64_t rank_block,
                                    const float *v, const float *w_t, int32_t group, uint8_t *codes,
                                    void *scales_f16, void *zeros_f16, float *deq, int32_t rank_mode,
                                    void *workspace, size_t workspace_bytes, void *stream);

/* The Kronecker Hadamard of each row alone, fp32 out [rows, n]:
 * (H_m (x) H_q) diag(signs) x with m in {1, 12, 20, 28} (m = 1: every aligned
 * block of q channels), q in {128, ..., 1024} (H_20: q in {128, 256}), or
 * m = 1 with q = n in {2048, 4096, 8192} (one FWHT over the row), or
 * m in {68, 76, 200} with n = m q <= 32768, q a power of two <= 1024 (the
 * Qwen3 widths 68 * 256, 76 * 128, 200 * 128; the fp64 product of the
 * reference for 68 and 200); signs fp32 [n] or NULL.  Replaces
 * full_hadamard_rows (nar/activation_experiments.py:188-217) for the widths
 * 12 * 2^j, 20 * 2^j, 28 * 2^j, 68 * 2^j, 76 * 2^j, 200 * 2^j and
 * 2^j <= 8192, and block Hadamards. */
int narhip_hadamard_rows(const void *x_bf16, int64_t rows, int64_t n, int64_t ld_x, int32_t had_m, int32_t had_q,
                         const float *signs, float *out, void *stream);

/* E28's down_proj transform, fp16 in and fp16 out, no quantization:
 * out = fp16( H_q-blocks(x) / fp32(sqrt q) - RN32(u W^T) ) per row of x fp16
 * [tokens, ld_x], q in {128, ..., 1024} (E28: 128), w_t fp32 [k, n], k <= 64.
 * u comes from `partial` fp32 [tokens, splits*k] (the split partials of
 * narhip_rank_projection_f16, folded in split order; Kernel B alone) or, with
 * partial NULL, is computed here from v fp32 [n, k] (u = RN32(x V), fp64
 * sums).  Scratch: a workspace of narhip_transform_f16_workspace() bytes
 * (enough for either form).  k = 0: Hadamard blocks only.  Replaces NARDownTransform.forward
 * (quarot-llama3/nar_r4_kernel.py:256-275) and launch_kernel_b with its
 * kernels nar_group_transform_kernel / nar_group_transform_tc_kernel
 * (quarot-llama3/nar_r4_kernel.py:56-120, :155-175). */
int narhip_transform_f16(const void *x_f16, int64_t tokens, int64_t n, int64_t ld_x, int32_t had_q,
                         const float *v, const float *partial, int32_t splits, const float *w_t, int32_t k,
                         void *out_f16, void *workspace, size_t workspace_bytes, void *stream);
size_t narhip_transform_f16_workspace(int64_t tokens, int64_t n, int32_t k);

/* Kernel A of the E28 transform on fp16 rows: partial[t, s*k + r] =
 * RN32(sum over channel split s of x[t, i] v[i, r]) with fp64 sums, v fp32
 * [n, k], 1 <= k <= 64, n / splits even.  Replaces launch_projection_dot on fp16
 * input with TERMS = 2 fp16 factor terms (quarot-llama3/nar_r4_kernel.py:272,
 * nar/kernels/r4_fused_v3.py:187-201). */
int narhip_rank_projection_f16(const void *x_f16, int64_t tokens, int64_t n, int64_t ld_x, const float *v,
                               int32_t k, int32_t splits, float *partial, void *stream);

/* Group-asymmetric W4A4 GEMM, the consumer of the packed INT4 format:
 * out[t, o] = sum_i (qA[t,i] sA[t,i/128] + zA[t,i/128]) (qW[o,i] sW[o,i/128] + zW[o,i/128])
 * for activations (codes uint8 [tokens, n/2], low nibble = even channel; fp16
 * scales / zeros [tokens, n/128]: the output of narhip_rotate_quant) and
 * weights in the same format [out_features, ...]; out fp32 [tokens, ld_out].
 * Per group: the code products sum qA qW exactly on the fp8 matrix cores
 * (a code byte c read as e4m3 is c * 2^-9), then
 * sA sW sum qA qW + sA SA zW + zA (sW SW + 128 zW) in fp32 (SA, SW the code
 * sums).  group must be 128.  With few output tiles (decode) the groups are
 * split over workgroups and the partials summed in split order.  The reference documents this form and runs no
 * such GEMM (quarot-llama3/e28_v2/docs/quantizer_contract.md:134-140); it is
 * the consumer named by the packed layout of nar/kernels/r4_fused_v2.py:80-92. */
int narhip_w4a4_gemm(const uint8_t *a_codes, const void *a_scales, const void *a_zeros, int64_t tokens,
                     const uint8_t *w_codes, const void *w_scales, const void *w_zeros, int64_t out_features,
                     int64_t n, int32_t group, float *out, int64_t ld_out, void *workspace, size_t workspace_bytes,
                     void *stream);
/* Scratch bytes narhip_w4a4_gemm needs (0 when the reduction is not split:
 * split partials [splits][tokens][out_features] fp32 for few output tiles). */
size_t narhip_w4a4_workspace(int64_t tokens, int64_t out_features, int64_t n);

/* Device self-test of the MFMA operand mapping the kernels rely on (no
 * counterpart in the reference): one v_mfma_f32_16x16x32_bf16 with
 * a_bf16[64*8], b_bf16[64*8] per lane, d[64*4] per lane (device memory). */
int narhip_mfma_probe(const void *a_bf16, const void *b_bf16, float *d, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* NARHIP_H */
