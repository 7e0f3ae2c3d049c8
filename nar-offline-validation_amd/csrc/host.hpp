// Host-side declarations shared by the translation units of libnarhip: error
// reporting, sizing helpers of the planner, and the kernel launchers.  Each
// launcher is defined in exactly one launch_*.hip unit (that unit instantiates
// the kernels it launches); abi.hip holds the planner and the extern "C"
// entry points.  Every kernel header is visible everywhere (structs, layouts),
// but a kernel is only compiled where it is launched.
#pragma once

#include "../../include/narhip.h"
#include "corr_quant.hip"
#include "dequant.hip"
#include "fwht_rows.hip"
#include "hooks.hip"
#include "kron_mfma.hip"
#include "mfma.hpp"
#include "narhip_device.hpp"
#include "paley_rows.hip"
#include "rank_exact.hip"
#include "rank_mfma.hip"
#include "rq_row.hip"
#include "rq_seg.hip"
#include "transform_f16.hip"
#include "w4a4.hip"

#include <cmath>

namespace narhip {
namespace host {

// ------------------------------------------------------------ errors (abi.hip)

// Sets the calling thread's error message and returns `code`.
int fail(int code, const char *fmt, ...);
// NARHIP_EHIP with the runtime's message if the last launch failed, else OK.
int check_launch(const char *what);
// The calling thread's last message / clear it (entry points clear on entry).
const char *last_error();
void clear_error();

// ------------------------------------------------------------------ helpers

inline bool pow2(int64_t v) { return v > 0 && !(v & (v - 1)); }
inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }
inline int round_up(int v, int m) { return (v + m - 1) / m * m; }
inline float f32_sqrt(int v) { return (float)std::sqrt((double)v); }

// Paley factor of order m (1, 12, 20, 28, 68, 76 or 200) as +-1 int8 [m][m];
// 0 on success, -1 for an unsupported order, -2 if the result fails H H^T = m I.
int build_paley(int m, int8_t *out);
// The prime and kind (1: Paley I over Z_p, 2: Paley II) of the Z_p
// constructions (orders 12, 20, 68, 76, 200); false for the others.
bool paley_zp(int m, int &p, int &kind);
PaleyTable paley_table(int m);

// Raise a kernel's dynamic LDS limit for blocks of 48 KB and more (the kernels
// also hold a few KB of static LDS on top of the dynamic block).
template <typename K>
int set_lds(K kernel, size_t lds)
{
    if (lds < 48 * 1024) return NARHIP_OK;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return fail(NARHIP_EHIP, "hipFuncSetAttribute: %s", hipGetErrorString(e));
    return NARHIP_OK;
}

// Workgroups of `kernel` resident on the current device at once (occupancy at
// this block size and dynamic LDS times the CU count), cached per kernel,
// block size, LDS size and device.
int64_t resident_blocks(const void *kernel, int threads, size_t lds);

// Grid of a persistent kernel: as many workgroups as fit at once, at most `work`.
template <typename K>
int64_t persistent_grid(K kernel, int threads, size_t lds, int64_t work)
{
    const int64_t r = resident_blocks(reinterpret_cast<const void *>(kernel), threads, lds);
    return r < work ? r : work;
}

// --------------------------------------------------------- planner sizing

// Prepared factor layout: vt [3][kp16][n] bf16, then wtt [3][n][kp32] bf16.
inline int kp16(int k) { return round_up(k < 1 ? 1 : k, 16); }
inline int kp32(int k) { return round_up(k < 1 ? 1 : k, 32); }
inline size_t vt_bytes(int64_t n, int k) { return align256(sizeof(uint16_t) * 3 * (size_t)kp16(k) * (size_t)n); }
inline size_t wtt_bytes(int64_t n, int k) { return align256(sizeof(uint16_t) * 3 * (size_t)kp32(k) * (size_t)n); }
inline size_t prepared_bytes(int64_t n, int k) { return vt_bytes(n, k) + wtt_bytes(n, k); }

// Splits of the fp64 VALU projection (16-token tiles): about 1024 workgroups,
// each split a whole number of 128-channel blocks.
inline int f64_splits(int64_t T, int64_t n)
{
    const int64_t tiles = (T + 15) / 16;
    int s = 1;
    while (s < 64 && tiles * s * 2 <= 1024 && n % (128 * 2 * (int64_t)s) == 0) s *= 2;
    return s;
}
// rank stride of the fp64 partials: 8, else k rounded up to slices of 16
inline int f64_kmax(int k) { return k <= 8 ? 8 : round_up(k, 16); }

// Channel splits for the MFMA projection: enough workgroups for two per CU
// (128-token tiles, splits of a multiple of 128 channels).
inline int mfma_splits(int64_t T, int64_t n)
{
    const int64_t tiles = (T + 127) / 128;
    int s = 1;
    while (s < 64 && tiles * s < 512 && n % (128 * 2 * (int64_t)s) == 0) s *= 2;
    return s;
}
inline bool mfma_projection_ok(int64_t n, int splits) { return n % (128 * (int64_t)splits) == 0; }

// u terms [T][3][kp32] bf16 (the MFMA correction's B operand), then the
// correction kernel's scratch area for the stores of lanes with nothing to store
inline size_t u3_bytes(int64_t T, int k) { return sizeof(uint16_t) * 3 * (size_t)kp32(k) * (size_t)T; }
inline size_t corr_scratch_bytes(int64_t T, int64_t n, int k)
{
    (void)n;
    return align256(u3_bytes(T, k)) + CQ_DUMMY_BYTES;
}

// fp16 transform at q = 128, k <= 8: proj_tok (unless the caller brings
// partials) + xform128, which folds the chunk sums itself.
inline bool xf_fast(int32_t had_q, int32_t k) { return had_q == 128 && k >= 1 && k <= XF_K; }

// Channel chunks per projection block (proj_tok, blocks of 64 PT_TL tokens):
// the smallest divisor S of n/128 that gives >= 256 blocks with chunks of at
// most 8192 channels (all 128-channel blocks when none does).  Measured at
// 2048 x 14336: 256 blocks (S = 16) 73.7 us per call against 77.4 us for 448
// and 82-84 us for 896; at 32768 x 14336 two chunks (512 blocks) 790 us
// against 806 us for one.
inline int xf_splits(int64_t T, int64_t n)
{
    const int64_t nb = n / 128, tiles = (T + 64 * PT_TL - 1) / (64 * PT_TL);
    for (int64_t d = 1; d <= nb; d++)
        if (nb % d == 0 && tiles * d >= 256 && n / d <= 8192) return (int)d;
    return (int)nb;
}
inline size_t xf_pd_bytes(int64_t T, int S) { return align256(sizeof(double) * XF_K * (size_t)T * (size_t)S); }

// ------------------------------------------------------------- launchers

// launch_seg.hip
int launch_seg(const SegArgs &a, int q, int b, int mode, hipStream_t s);
// full-row FWHT of n = q in {2048, 4096, 8192} channels (fwht_rows.hip)
inline bool fwht_rows_width(int64_t q) { return q == 2048 || q == 4096 || q == 8192; }
int launch_fwht(const FwhtArgs &a, int q, int b, hipStream_t s);
int launch_seg_f16(const SegArgs &a, int q, int k, hipStream_t s);

// launch_kron.hip: exact rq_row (RowArgs) when ra, else kron_mfma (KronArgs)
int launch_kron(const RowArgs *ra, const KronArgs *ka, bool quant, int m, int q, int b, hipStream_t s);

// launch_rank.hip
int launch_proj_exact(const uint16_t *x, int64_t T, int64_t n, int64_t ldx, const float *v, int k, int splits,
                      float *partial, hipStream_t s);
int launch_corr_exact(const float *partial, int splits, int k, const float *wt, int64_t T, int64_t n, float *corr,
                      hipStream_t s);
int launch_prepare(const float *v, const float *wt, int64_t n, int k, void *prep, hipStream_t s);
int launch_proj_f64(const uint16_t *x, int64_t T, int64_t n, int64_t ldx, const float *v, int k, int splits,
                    double *pd, hipStream_t s, bool f16 = false, float *pf = nullptr);
int launch_fold_f64(const double *pd, int splits, int kmax, int k, int64_t T, float *u, hipStream_t s);
int launch_fold_f32(const float *partial, int splits, int k, int64_t T, float *u, hipStream_t s);
int launch_proj_mfma(const uint16_t *x, int64_t T, int64_t n, int64_t ldx, const void *prep, int k, int splits,
                     float *partial, hipStream_t s);
int launch_fold_u(const float *partial, int splits, int k, int kp, int64_t T, __bf16 *u3, hipStream_t s);
int launch_corr_quant(CorrQuantArgs a, int b, hipStream_t s);
int launch_mfma_probe(const __bf16 *a, const __bf16 *b, float *d, hipStream_t s);

// launch_f16.hip
int launch_proj_tok(const uint16_t *x, int64_t T, int64_t n, int64_t ldx, const float *v, int k, int S,
                    double *pd, float *pf, hipStream_t s, bool f16 = true);
// u from proj_tok's chunk sums pd [T][S][XF_K], or from the caller's fp32
// partials pf [T][S*k].  quant != null: bf16 rows, INT4 group-128 outputs
// (codes, scales, zeros, dest and signs from *quant); else fp16 rows to fp16 `out`.
int launch_xform128(const uint16_t *x, int64_t T, int64_t n, int64_t ldx, const float *w_t, const double *pd,
                    const float *pf, int S, int k, uint16_t *out, hipStream_t s, const XformArgs *quant = nullptr);

// launch_misc.hip
int launch_dequant(const uint8_t *codes, const uint16_t *scales, const uint16_t *zeros, int64_t rows, int64_t n,
                   int group, float *out, hipStream_t s);
int launch_quant_tuple(int dtype, const void *x, int64_t elems, int group, uint8_t *codes, uint16_t *scales,
                       uint16_t *zeros, void *deq, hipStream_t s);
int launch_w4a4(const W4A4Args &a, int64_t gx, int64_t gy, float *out, hipStream_t s);
// rows of H_m (x) H_q for the Paley orders without a Kronecker kernel (paley_rows.hip)
int launch_paley_rows(const PaleyRowsArgs &a, hipStream_t s);

}  // namespace host
}  // namespace narhip
