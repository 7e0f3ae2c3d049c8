// Launchers of the stand-alone kernels: dequantization, the hooks' quantizer
// (hooks.hip), the W4A4 GEMM (w4a4.hip) and the large-order Paley rows
// (paley_rows.hip).
#include "host.hpp"

namespace narhip {
namespace host {

namespace {

template <int CPL, bool FP64P>
int launch_paley_rows_t(const PaleyRowsArgs &a, size_t lds, hipStream_t s)
{
    if (int rc = set_lds(paley_rows_kernel<CPL, FP64P>, lds)) return rc;
    hipLaunchKernelGGL((paley_rows_kernel<CPL, FP64P>), dim3((unsigned)a.T), dim3(PR_THREADS), lds, s, a);
    return check_launch("paley_rows_kernel");
}

template <bool FP64P>
int launch_paley_rows_p(const PaleyRowsArgs &a, size_t lds, hipStream_t s)
{
    switch (a.q <= 64 ? 1 : a.q / 64) {
    case 1: return launch_paley_rows_t<1, FP64P>(a, lds, s);
    case 2: return launch_paley_rows_t<2, FP64P>(a, lds, s);
    case 4: return launch_paley_rows_t<4, FP64P>(a, lds, s);
    default:   // m >= 68 and m q <= 32768 leave q <= 256
        return fail(NARHIP_EUNSUPPORTED, "Paley rows need q <= 256 (q=%d)", a.q);
    }
}

}  // namespace

int launch_paley_rows(const PaleyRowsArgs &a, hipStream_t s)
{
    const size_t lds = sizeof(float) * (size_t)a.m * (size_t)a.q + sizeof(uint32_t) * (size_t)a.m * paley_sign_words(a.m);
    return a.fp64_product ? launch_paley_rows_p<true>(a, lds, s) : launch_paley_rows_p<false>(a, lds, s);
}

int launch_dequant(const uint8_t *codes, const uint16_t *scales, const uint16_t *zeros, int64_t rows, int64_t n,
                   int group, float *out, hipStream_t s)
{
    const int64_t words = rows * n / 8;
    hipLaunchKernelGGL(dequant_kernel<>, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, s, codes, scales, zeros,
                       rows, n, group, out);
    return check_launch("dequant_kernel");
}

int launch_quant_tuple(int dtype, const void *x, int64_t elems, int group, uint8_t *codes, uint16_t *scales,
                       uint16_t *zeros, void *deq, hipStream_t s)
{
    dim3 grid((unsigned)((elems / 8 + 255) / 256));
    switch (dtype) {
    case DT_F32: hipLaunchKernelGGL(quant_tuple_kernel<DT_F32>, grid, dim3(256), 0, s, x, elems, group, codes, scales, zeros, deq); break;
    case DT_BF16: hipLaunchKernelGGL(quant_tuple_kernel<DT_BF16>, grid, dim3(256), 0, s, x, elems, group, codes, scales, zeros, deq); break;
    default: hipLaunchKernelGGL(quant_tuple_kernel<DT_F16>, grid, dim3(256), 0, s, x, elems, group, codes, scales, zeros, deq); break;
    }
    return check_launch("quant_tuple_kernel");
}

// a.out is the output itself (one split) or the fp32 partials [splits][T][O]
// that the reduction sums in split order into `out`.
int launch_w4a4(const W4A4Args &a, int64_t gx, int64_t gy, float *out, hipStream_t s)
{
    hipLaunchKernelGGL(w4a4_kernel<>, dim3((unsigned)gx, (unsigned)gy, (unsigned)a.splits), dim3(256), 0, s, a);
    int rc = check_launch("w4a4_kernel");
    if (rc || a.splits == 1) return rc;
    const int64_t cnt = a.T * a.O;
    hipLaunchKernelGGL(w4a4_reduce_kernel<>, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, s, a.out, a.splits,
                       a.T, a.O, out, a.ldo);
    return check_launch("w4a4_reduce_kernel");
}

}  // namespace host
}  // namespace narhip
