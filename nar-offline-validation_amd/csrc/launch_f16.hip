// Launchers of the block-H_128 transform kernels (transform_f16.hip).
#include "host.hpp"

namespace narhip {
namespace host {

int launch_proj_tok(const uint16_t *x, int64_t T, int64_t n, int64_t ldx, const float *v, int k, int S,
                    double *pd, float *pf, hipStream_t s, bool f16)
{
    ProjTokArgs a{x, ldx, T, n, v, pd, pf, k, S, k % 4 == 0 && aligned16(v)};
    const dim3 grid((unsigned)((T + 64 * PT_TL - 1) / (64 * PT_TL)), (unsigned)S);
    if (f16) hipLaunchKernelGGL((proj_tok_kernel<true, PT_TL>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((proj_tok_kernel<false, PT_TL>), grid, dim3(256), 0, s, a);
    return check_launch("proj_tok_kernel");
}

// u from proj_tok's chunk sums pd [T][S][XF_K], or from the caller's fp32
// partials pf [T][S*k].  quant != null: bf16 rows, INT4 group-128 outputs
// (codes, scales, zeros, dest and signs from *quant); else fp16 rows to fp16 `out`.
int launch_xform128(const uint16_t *x, int64_t T, int64_t n, int64_t ldx, const float *w_t, const double *pd,
                    const float *pf, int S, int k, uint16_t *out, hipStream_t s, const XformArgs *quant)
{
    // ~2048 workgroups, but at least 32 tokens each (each loads 64 KB of W^T
    // before its first token) while that still leaves >= 512 workgroups
    const int64_t gx = (n / 128 + 15) / 16;
    int64_t gy = (2048 + gx - 1) / gx;
    if (T < 32 * gy) {
        const int64_t lo = (512 + gx - 1) / gx;
        gy = (T + 31) / 32 > lo ? (T + 31) / 32 : lo;
    }
    if (gy > T) gy = T;
    const int64_t tpb = (T + gy - 1) / gy;
    gy = (T + tpb - 1) / tpb;
    XformArgs a = quant ? *quant : XformArgs{};
    a.x = x; a.ldx = ldx; a.T = T; a.n = n; a.wt = w_t; a.pd = pd; a.pf = pf; a.S = S; a.out = out; a.k = k; a.tpb = (int)tpb;
    a.sq = f32_sqrt(128);
    a.rsq = 1.0f / a.sq;
    const dim3 grid((unsigned)gx, (unsigned)gy);
    if (quant) hipLaunchKernelGGL(xform128_kernel<true>, grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL(xform128_kernel<false>, grid, dim3(256), 0, s, a);
    return check_launch("xform128_kernel");
}
}  // namespace host
}  // namespace narhip
