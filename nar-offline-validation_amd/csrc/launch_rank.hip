// Launchers of the rank-k kernels: the exact fp64 forms (rank_exact.hip) and
// the bf16-MFMA projection, fold and correction-quantizer (rank_mfma.hip).
#include "host.hpp"

namespace narhip {
namespace host {

int launch_proj_exact(const uint16_t *x, int64_t T, int64_t n, int64_t ldx, const float *v,
                      int k, int splits, float *partial, hipStream_t s)
{
    if (T == 0) return NARHIP_OK;
    ProjArgs a{x, ldx, T, n, v, partial, k, splits};
    hipLaunchKernelGGL(proj_exact_kernel<>, dim3((unsigned)((T + 31) / 32), (unsigned)splits), dim3(256), 0, s, a);
    return check_launch("proj_exact_kernel");
}

int launch_corr_exact(const float *partial, int splits, int k, const float *wt, int64_t T, int64_t n,
                      float *corr, hipStream_t s)
{
    if (T == 0) return NARHIP_OK;
    CorrArgs a{partial, splits, k, wt, T, n, corr};
    hipLaunchKernelGGL(corr_exact_kernel<>, dim3((unsigned)((T + 31) / 32), (unsigned)(n / 64)), dim3(256), 0, s, a);
    return check_launch("corr_exact_kernel");
}


int launch_prepare(const float *v, const float *wt, int64_t n, int k, void *prep, hipStream_t s)
{
    __bf16 *vt = static_cast<__bf16 *>(prep);
    __bf16 *wtt = reinterpret_cast<__bf16 *>(static_cast<char *>(prep) + vt_bytes(n, k));
    if (v) {
        const int64_t nv = n * kp16(k);
        hipLaunchKernelGGL(prep_v_kernel<>, dim3((unsigned)((nv + 255) / 256)), dim3(256), 0, s, v, n, k, kp16(k), vt);
        if (int rc = check_launch("prep_v_kernel")) return rc;
    }
    if (wt) {
        const int64_t nw = n * kp32(k);
        hipLaunchKernelGGL(prep_w_kernel<>, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0, s, wt, n, k, kp32(k), wtt);
        if (int rc = check_launch("prep_w_kernel")) return rc;
    }
    return NARHIP_OK;
}

int launch_proj_f64(const uint16_t *x, int64_t T, int64_t n, int64_t ldx, const float *v, int k, int splits,
                    double *pd, hipStream_t s, bool f16, float *pf)
{
    if (T == 0) return NARHIP_OK;
    ProjF64Args a{x, ldx, T, n, v, pd, k, splits, pf, 0, f64_kmax(k)};
    dim3 grid((unsigned)((T + 15) / 16), (unsigned)splits);
    // k > 16: one launch per slice of 16 ranks (each an fp64 sum per rank, so
    // the slicing does not change any partial)
    for (a.r0 = 0; a.r0 < k; a.r0 += 16) {
        if (f16) {
            if (k <= 8) hipLaunchKernelGGL((proj_f64_kernel<8, true>), grid, dim3(256), 0, s, a);
            else hipLaunchKernelGGL((proj_f64_kernel<16, true>), grid, dim3(256), 0, s, a);
        } else {
            if (k <= 8) hipLaunchKernelGGL((proj_f64_kernel<8>), grid, dim3(256), 0, s, a);
            else hipLaunchKernelGGL((proj_f64_kernel<16>), grid, dim3(256), 0, s, a);
        }
        if (int rc = check_launch("proj_f64_kernel")) return rc;
    }
    return NARHIP_OK;
}

int launch_fold_f64(const double *pd, int splits, int kmax, int k, int64_t T, float *u, hipStream_t s)
{
    const int64_t n = T * k;
    hipLaunchKernelGGL(fold_f64_kernel<>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, pd, splits, kmax, k, T, u);
    return check_launch("fold_f64_kernel");
}

int launch_fold_f32(const float *partial, int splits, int k, int64_t T, float *u, hipStream_t s)
{
    const int64_t n = T * k;
    hipLaunchKernelGGL(fold_f32_kernel<>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, partial, splits, k, T, u);
    return check_launch("fold_f32_kernel");
}

int launch_proj_mfma(const uint16_t *x, int64_t T, int64_t n, int64_t ldx, const void *prep, int k, int splits,
                     float *partial, hipStream_t s)
{
    if (T == 0) return NARHIP_OK;
    if (!mfma_projection_ok(n, splits))
        return fail(NARHIP_EUNSUPPORTED, "MFMA projection needs n %% (128*splits) == 0 (n=%lld, splits=%d)",
                    (long long)n, splits);
    ProjMfmaArgs a{x, ldx, T, n, static_cast<const __bf16 *>(prep), kp16(k), k, splits, n / splits, partial};
    dim3 grid((unsigned)((T + 127) / 128), (unsigned)splits);
    switch (kp16(k) / 16) {
    case 1: hipLaunchKernelGGL((proj_mfma_kernel<1>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((proj_mfma_kernel<2>), grid, dim3(256), 0, s, a); break;
    case 3: hipLaunchKernelGGL((proj_mfma_kernel<3>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((proj_mfma_kernel<4>), grid, dim3(256), 0, s, a); break;
    default: return fail(NARHIP_EUNSUPPORTED, "rank %d", k);
    }
    return check_launch("proj_mfma_kernel");
}

int launch_fold_u(const float *partial, int splits, int k, int kp, int64_t T, __bf16 *u3, hipStream_t s)
{
    const int64_t n = T * kp;
    hipLaunchKernelGGL(fold_u_kernel<>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, partial, splits, k, kp, T, u3);
    return check_launch("fold_u_kernel");
}

namespace {

template <int B, int KS, int TPW>
int launch_cq(const CorrQuantArgs &a, dim3 grid, hipStream_t s)
{
    if (a.rotated) hipLaunchKernelGGL((corr_quant_kernel<B, KS, true, TPW>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((corr_quant_kernel<B, KS, false, TPW>), grid, dim3(256), 0, s, a);
    return check_launch("corr_quant_kernel");
}

template <int B, int KS>
int launch_cq_t(const CorrQuantArgs &a, dim3 grid, hipStream_t s)
{
    if constexpr (KS == 2) {
        if (a.tpg == 32) return launch_cq<B, KS, 8>(a, grid, s);
    }
    return a.tpg == 16 ? launch_cq<B, KS, 4>(a, grid, s) : launch_cq<B, KS, 1>(a, grid, s);
}

}  // namespace

// A workgroup owns one 128-channel block and tpg 16-token tiles (tpg / 4 per
// wave): 16 tiles where that still leaves about 2048 workgroups or more, else 4
// (32 at k > 32 on the largest shapes).
int launch_corr_quant(CorrQuantArgs a, int b, hipStream_t s)
{
    if (a.T == 0) return NARHIP_OK;
    if (a.n % CQ_CB) return fail(NARHIP_EUNSUPPORTED, "rank correction needs n %% 128 == 0");
    const int ks = a.kp / 32;
    if (ks < 1 || ks > 2) return fail(NARHIP_EUNSUPPORTED, "rank correction supports k <= 64");
    a.ncb = a.n / CQ_CB;
    const int64_t tiles = (a.T + 15) / 16;
    a.tpg = tiles * a.ncb >= 16 * 2048 ? 16 : 4;
    // k > 32: the W'' terms staged per workgroup are 48 KB; twice the tiles per
    // workgroup where that still leaves 2048 workgroups or more (down_proj 70B,
    // 16384 x 28672: 1463 -> 1413 us per call; 64 tiles, code unrolled 16 times
    // per wave, runs twice as slow)
    if (ks == 2 && tiles * a.ncb >= 32 * 2048) a.tpg = 32;
    const int64_t groups = (tiles + a.tpg - 1) / a.tpg;
    const int64_t blocks = 8 * a.ncb * ((groups + 7) / 8);
    if (blocks > 0x7fffffff) return fail(NARHIP_EUNSUPPORTED, "too many tokens");
    const dim3 grid((unsigned)blocks);
    switch (b * 4 + ks) {
    case 32 * 4 + 1: return launch_cq_t<32, 1>(a, grid, s);
    case 32 * 4 + 2: return launch_cq_t<32, 2>(a, grid, s);
    case 64 * 4 + 1: return launch_cq_t<64, 1>(a, grid, s);
    case 64 * 4 + 2: return launch_cq_t<64, 2>(a, grid, s);
    case 128 * 4 + 1: return launch_cq_t<128, 1>(a, grid, s);
    case 128 * 4 + 2: return launch_cq_t<128, 2>(a, grid, s);
    }
    return fail(NARHIP_EUNSUPPORTED, "group %d not built", b);
}

int launch_mfma_probe(const __bf16 *a, const __bf16 *b, float *d, hipStream_t s)
{
    hipLaunchKernelGGL(mfma_probe_kernel<>, dim3(1), dim3(64), 0, s, a, b, d);
    return check_launch("mfma_probe_kernel");
}

}  // namespace host
}  // namespace narhip
