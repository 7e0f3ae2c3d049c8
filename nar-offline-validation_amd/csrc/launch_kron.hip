// Launchers of the Kronecker row kernels: kron_mfma (Paley factor on MFMA)
// and rq_row (exact fp64 Paley sums).
#include "host.hpp"

namespace narhip {
namespace host {

namespace {

template <int M, int Q, int B>
int launch_row_mqb(const RowArgs &a, hipStream_t s)
{
    const size_t lds = sizeof(float) * M * Q;
    if (int rc = set_lds(&rq_row_kernel<M, Q, B>, lds)) return rc;
    hipLaunchKernelGGL((rq_row_kernel<M, Q, B>), dim3((unsigned)a.T), dim3(256), lds, s, a);
    return check_launch("rq_row_kernel");
}


template <int M, int Q, int B>
int launch_kron_mqb(const KronArgs &a, bool quant, hipStream_t s)
{
    const size_t lds = sizeof(float) * kron_rows<M>() * (Q + KPAD);
    // persistent (as many workgroups as are resident, each walking tokens with
    // the next token's x requested ahead) from Q = 512 on: H28 x H512, 8192
    // tokens, 343 -> 335 us per rotate_quant call; at Q = 256 (H12 x H256) it
    // was slower (49.5 -> 51.7 us)
    constexpr bool persist = Q >= 512;
    if (quant) {
        auto k = &kron_mfma_kernel<M, Q, B, true, persist>;
        if (int rc = set_lds(k, lds)) return rc;
        const int64_t grid = persist ? persistent_grid(k, 16 * M, lds, a.T) : a.T;
        hipLaunchKernelGGL((kron_mfma_kernel<M, Q, B, true, persist>), dim3((unsigned)grid), dim3(16 * M), lds, s, a);
    } else {
        auto k = &kron_mfma_kernel<M, Q, 128, false, persist>;
        if (int rc = set_lds(k, lds)) return rc;
        const int64_t grid = persist ? persistent_grid(k, 16 * M, lds, a.T) : a.T;
        hipLaunchKernelGGL((kron_mfma_kernel<M, Q, 128, false, persist>), dim3((unsigned)grid), dim3(16 * M), lds, s, a);
    }
    return check_launch("kron_mfma_kernel");
}

// exact: rq_row (fp64 Paley) with RowArgs; otherwise kron_mfma with KronArgs
template <int M, int Q>
int launch_kron_mq(const RowArgs *ra, const KronArgs *ka, bool quant, int b, hipStream_t s)
{
    switch (b) {
    case 32: return ra ? launch_row_mqb<M, Q, 32>(*ra, s) : launch_kron_mqb<M, Q, 32>(*ka, quant, s);
    case 64: return ra ? launch_row_mqb<M, Q, 64>(*ra, s) : launch_kron_mqb<M, Q, 64>(*ka, quant, s);
    case 128: return ra ? launch_row_mqb<M, Q, 128>(*ra, s) : launch_kron_mqb<M, Q, 128>(*ka, quant, s);
    }
    return fail(NARHIP_EUNSUPPORTED, "group %d not built", b);
}

template <int M>
int launch_kron_m(const RowArgs *ra, const KronArgs *ka, bool quant, int q, int b, hipStream_t s)
{
    switch (q) {
    case 256: return launch_kron_mq<M, 256>(ra, ka, quant, b, s);
    case 512: return launch_kron_mq<M, 512>(ra, ka, quant, b, s);
    case 1024: return launch_kron_mq<M, 1024>(ra, ka, quant, b, s);
    }
    return fail(NARHIP_EUNSUPPORTED, "Kronecker H_%d x H_%d not built", M, q);
}

// H_20 (x) H_q: the Qwen3 widths 2560 = 20 x 128 and 5120 = 20 x 256
int launch_kron_20(const RowArgs *ra, const KronArgs *ka, bool quant, int q, int b, hipStream_t s)
{
    switch (q) {
    case 128: return launch_kron_mq<20, 128>(ra, ka, quant, b, s);
    case 256: return launch_kron_mq<20, 256>(ra, ka, quant, b, s);
    }
    return fail(NARHIP_EUNSUPPORTED, "Kronecker H_20 x H_%d not built", q);
}

}  // namespace

int launch_kron(const RowArgs *ra, const KronArgs *ka, bool quant, int m, int q, int b, hipStream_t s)
{
    if (m == 12) return launch_kron_m<12>(ra, ka, quant, q, b, s);
    if (m == 20) return launch_kron_20(ra, ka, quant, q, b, s);
    if (m == 28) return launch_kron_m<28>(ra, ka, quant, q, b, s);
    return fail(NARHIP_EUNSUPPORTED, "Paley order %d not built", m);
}
}  // namespace host
}  // namespace narhip
