// Launchers of the segment kernels (rq_seg.hip): one 16-lane row per Hadamard
// block, the quantizer or an fp32 / fp16 store.
#include "host.hpp"

namespace narhip {
namespace host {

namespace {

template <int Q, int B>
int launch_seg_qb(const SegArgs &a, int mode, hipStream_t s)
{
    const int64_t segs = a.T * (a.n / Q);
    dim3 grid((unsigned)((segs + 15) / 16));
    if (grid.x == 0) return NARHIP_OK;
    if (mode == RANK_LOCAL && Q == 128) {
        // per-head form: grid (token tiles, heads); with few segments (decode)
        // one wave per workgroup, so they spread over four times as many CUs
        // (decode V-cache 64 x 8 heads: 5.0 -> 4.1 us per kernel)
        const int64_t heads = a.n / 128;
        if (heads > 65535) return fail(NARHIP_EUNSUPPORTED, "too many 128-channel blocks per token");
        const int rows = segs <= 4096 ? 4 : 16;
        const dim3 g2((unsigned)((a.T + rows - 1) / rows), (unsigned)heads), blk((unsigned)(16 * rows));
        if (a.k <= 2) hipLaunchKernelGGL((rq_seg_kernel<Q, B, RANK_LOCAL, 2>), g2, blk, 0, s, a);
        else if (a.k <= 4) hipLaunchKernelGGL((rq_seg_kernel<Q, B, RANK_LOCAL, 4>), g2, blk, 0, s, a);
        else hipLaunchKernelGGL((rq_seg_kernel<Q, B, RANK_LOCAL, 8>), g2, blk, 0, s, a);
        return check_launch("rq_seg_kernel");
    }
    switch (mode) {
    case RANK_NONE: hipLaunchKernelGGL((rq_seg_kernel<Q, B, RANK_NONE, 0>), grid, dim3(256), 0, s, a); break;
    case RANK_LOCAL:
        // per-block rank at Q > 128, compiled for the rank
        if (a.k <= 2) hipLaunchKernelGGL((rq_seg_kernel<Q, B, RANK_LOCAL, 2>), grid, dim3(256), 0, s, a);
        else if (a.k <= 4) hipLaunchKernelGGL((rq_seg_kernel<Q, B, RANK_LOCAL, 4>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((rq_seg_kernel<Q, B, RANK_LOCAL, 8>), grid, dim3(256), 0, s, a);
        break;
    default:
        if (a.k <= 16) hipLaunchKernelGGL((rq_seg_kernel<Q, B, RANK_PARTIAL, 16>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((rq_seg_kernel<Q, B, RANK_PARTIAL, 64>), grid, dim3(256), 0, s, a);
        break;
    }
    return check_launch("rq_seg_kernel");
}

template <int Q>
int launch_seg_q(const SegArgs &a, int b, int mode, hipStream_t s)
{
    switch (b) {
    case 32: return launch_seg_qb<Q, 32>(a, mode, s);
    case 64: return launch_seg_qb<Q, 64>(a, mode, s);
    case 128: return launch_seg_qb<Q, 128>(a, mode, s);
    }
    return fail(NARHIP_EUNSUPPORTED, "group %d not built", b);
}


}  // namespace

int launch_seg(const SegArgs &a, int q, int b, int mode, hipStream_t s)
{
    switch (q) {
    case 128: return launch_seg_q<128>(a, b, mode, s);
    case 256: return launch_seg_q<256>(a, b, mode, s);
    case 512: return launch_seg_q<512>(a, b, mode, s);
    case 1024: return launch_seg_q<1024>(a, b, mode, s);
    }
    return fail(NARHIP_EUNSUPPORTED, "segment width %d not built", q);
}

namespace {

template <int L>
int launch_fwht_l(const FwhtArgs &a, int b, hipStream_t s)
{
    const dim3 grid((unsigned)a.T);
    switch (b) {
    case 32: hipLaunchKernelGGL((fwht_rows_kernel<L, 32>), grid, dim3(256), 0, s, a); break;
    case 64: hipLaunchKernelGGL((fwht_rows_kernel<L, 64>), grid, dim3(256), 0, s, a); break;
    case 128: hipLaunchKernelGGL((fwht_rows_kernel<L, 128>), grid, dim3(256), 0, s, a); break;
    default: return fail(NARHIP_EUNSUPPORTED, "group %d not built", b);
    }
    return check_launch("fwht_rows_kernel");
}

}  // namespace

int launch_fwht(const FwhtArgs &a, int q, int b, hipStream_t s)
{
    if (a.T == 0) return NARHIP_OK;
    if (a.T > 0x7fffffff) return fail(NARHIP_EUNSUPPORTED, "too many rows");
    switch (q) {
    case 2048: return launch_fwht_l<11>(a, b, s);
    case 4096: return launch_fwht_l<12>(a, b, s);
    case 8192: return launch_fwht_l<13>(a, b, s);
    }
    return fail(NARHIP_EUNSUPPORTED, "FWHT row width %d not built", q);
}

// fp16 rows in and out (E28's transform for block widths other than the fast
// q = 128 path): the rank term from fp32 partials or folded u (a.partial).
int launch_seg_f16(const SegArgs &a, int q, int k, hipStream_t s)
{
    const int64_t segs = a.T * (a.n / q);
    dim3 grid((unsigned)((segs + 15) / 16));
    if (grid.x == 0) return NARHIP_OK;
#define NARHIP_F16_SEG(QQ)                                                                                      \
    if (k > 16) hipLaunchKernelGGL((rq_seg_kernel<QQ, 128, RANK_PARTIAL, 64, true>), grid, dim3(256), 0, s, a); \
    else if (k > 0) hipLaunchKernelGGL((rq_seg_kernel<QQ, 128, RANK_PARTIAL, 16, true>), grid, dim3(256), 0, s, a); \
    else hipLaunchKernelGGL((rq_seg_kernel<QQ, 128, RANK_NONE, 0, true>), grid, dim3(256), 0, s, a);
    switch (q) {
    case 128: NARHIP_F16_SEG(128) break;
    case 256: NARHIP_F16_SEG(256) break;
    case 512: NARHIP_F16_SEG(512) break;
    case 1024: NARHIP_F16_SEG(1024) break;
    default: return fail(NARHIP_EUNSUPPORTED, "segment width %d not built", q);
    }
#undef NARHIP_F16_SEG
    return check_launch("rq_seg_kernel (fp16)");
}

}  // namespace host
}  // namespace narhip
