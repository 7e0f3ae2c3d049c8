// Row kernel: one workgroup per token for the Kronecker factors H_M (x) H_Q
// (M = 12 or 28, Q <= 1024) over the whole row, as in full_hadamard_rows
// (nar/activation_experiments.py:188-217):
//   F[a, :] = FWHT_Q(x[a*Q : (a+1)*Q]) / fp32(sqrt(Q))      per segment a
//   P[a, c] = sum_a' Hm[a, a'] F[a', c]                       Hm = +-1/fp32(sqrt(M))
//   x'      = P - C                                          C = u W^T (precomputed)
// then the group-B INT4 quantizer.
//
// The FWHT of each segment runs in one 16-lane row (as in rq_seg.hip), F is
// staged in LDS, the Paley product reads one column of F per thread.  The
// Paley sum is accumulated in fp64 in index order and rounded once -- the
// definition the oracle uses for the reference's BLAS product.
#pragma once
#include "narhip_device.hpp"

namespace narhip {

struct RowArgs {
    const uint16_t *x;      // bf16 [T, ldx]
    int64_t ldx;
    int64_t T, n;           // n = M * Q
    const float *signs;     // [n] or null
    const float *corr;      // [T, n] fp32 rank-k term C, or null
    uint8_t *codes;
    uint16_t *scales;
    uint16_t *zeros;
    const int64_t *dest;
    float *rotated;
    PaleyTable paley;
    float sq, rsq;          // fp32(sqrt(Q)), RN(1/sq)
    float hm;               // fp32(1) / fp32(sqrt(M))
};

template <int M, int Q, int B>
__global__ void __launch_bounds__(256)
rq_row_kernel(RowArgs a)
{
    constexpr int NH = Q / 128;
    constexpr int NV = 8 * NH;
    constexpr int N = M * Q;
    extern __shared__ float F[];               // [N]
    const int tid = threadIdx.x;
    const int l16 = tid & 15;
    const int row = tid >> 4;
    const int chunk = lane_chunk(l16);
    const int64_t t = blockIdx.x;
    const uint16_t *xt = a.x + t * a.ldx;

    // ---- phase 1: FWHT_Q of each segment, normalised, into LDS
    for (int s = row; s < M; s += 16) {
        float v[NV];
#pragma unroll
        for (int h = 0; h < NH; h++) {
            uint4 w = *reinterpret_cast<const uint4 *>(xt + s * Q + h * 128 + chunk * 8);
            v[h * 8 + 0] = bf16lo(w.x); v[h * 8 + 1] = bf16hi(w.x);
            v[h * 8 + 2] = bf16lo(w.y); v[h * 8 + 3] = bf16hi(w.y);
            v[h * 8 + 4] = bf16lo(w.z); v[h * 8 + 5] = bf16hi(w.z);
            v[h * 8 + 6] = bf16lo(w.w); v[h * 8 + 7] = bf16hi(w.w);
        }
        if (a.signs) {
#pragma unroll
            for (int h = 0; h < NH; h++)
#pragma unroll
                for (int e = 0; e < 8; e++) v[h * 8 + e] *= a.signs[s * Q + h * 128 + chunk * 8 + e];
        }
#pragma unroll
        for (int w = 1; w < 8; w <<= 1)
#pragma unroll
            for (int h = 0; h < NH; h++)
#pragma unroll
                for (int e = 0; e < 8; e++)
                    if (!(e & w)) {
                        float x0 = v[h * 8 + e], x1 = v[h * 8 + e + w];
                        v[h * 8 + e] = x0 + x1;
                        v[h * 8 + e + w] = x0 - x1;
                    }
        {
            const float s0 = (chunk & 1) ? -1.0f : 1.0f;
            const float s1 = (chunk & 2) ? -1.0f : 1.0f;
            const float s2 = (chunk & 4) ? -1.0f : 1.0f;
            const float s3 = (chunk & 8) ? -1.0f : 1.0f;
#pragma unroll
            for (int i = 0; i < NV; i++) v[i] = __builtin_fmaf(s0, v[i], xchg<0>(v[i]));
#pragma unroll
            for (int i = 0; i < NV; i++) v[i] = __builtin_fmaf(s1, v[i], xchg<1>(v[i]));
#pragma unroll
            for (int i = 0; i < NV; i++) v[i] = __builtin_fmaf(s2, v[i], xchg<2>(v[i]));
#pragma unroll
            for (int i = 0; i < NV; i++) v[i] = __builtin_fmaf(s3, v[i], xchg<3>(v[i]));
        }
#pragma unroll
        for (int wh = 1; wh < NH; wh <<= 1)
#pragma unroll
            for (int h = 0; h < NH; h++)
                if (!(h & wh))
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        float x0 = v[h * 8 + e], x1 = v[(h + wh) * 8 + e];
                        v[h * 8 + e] = x0 + x1;
                        v[(h + wh) * 8 + e] = x0 - x1;
                    }
        div_sqrt_q<Q>(v, a.sq, a.rsq);
#pragma unroll
        for (int h = 0; h < NH; h++) {
            float4 *d = reinterpret_cast<float4 *>(F + s * Q + h * 128 + chunk * 8);
            d[0] = make_float4(v[h * 8 + 0], v[h * 8 + 1], v[h * 8 + 2], v[h * 8 + 3]);
            d[1] = make_float4(v[h * 8 + 4], v[h * 8 + 5], v[h * 8 + 6], v[h * 8 + 7]);
        }
    }
    __syncthreads();

    // ---- phase 2: Paley product per column (fp64 accumulate, one rounding),
    //      minus the rank-k term, written back in place
    {
        const float hm = a.hm;
        for (int c = tid; c < Q; c += 256) {
            float f[M];
#pragma unroll
            for (int j = 0; j < M; j++) f[j] = F[j * Q + c];
#pragma unroll
            for (int i = 0; i < M; i++) {
                const uint32_t neg = a.paley.neg[i];
                double acc = 0.0;
#pragma unroll
                for (int j = 0; j < M; j++) {
                    const double h = (neg >> j) & 1u ? -(double)hm : (double)hm;
                    acc = fma((double)f[j], h, acc);
                }
                float p = (float)acc;
                if (a.corr) p = p - a.corr[t * N + i * Q + c];
                F[i * Q + c] = p;
            }
        }
    }
    __syncthreads();

    if (a.rotated) {
        for (int i = tid; i < N / 4; i += 256)
            reinterpret_cast<float4 *>(a.rotated + t * N)[i] = reinterpret_cast<const float4 *>(F)[i];
    }

    // ---- phase 3: quantize groups of B (B/8 consecutive lanes per group)
    constexpr int G8 = B / 8;
    constexpr int CHUNKS = N / 8;
    const int64_t orow = a.dest ? a.dest[t] : t;
    for (int c0 = 0; c0 < CHUNKS; c0 += 256) {
        const int ch = c0 + tid;
        const bool ok = ch < CHUNKS;
        const int chs = ok ? ch : 0;
        float v[8];
        {
            const float4 *s = reinterpret_cast<const float4 *>(F + chs * 8);
            float4 p0 = s[0], p1 = s[1];
            v[0] = p0.x; v[1] = p0.y; v[2] = p0.z; v[3] = p0.w;
            v[4] = p1.x; v[5] = p1.y; v[6] = p1.z; v[7] = p1.w;
        }
        GroupParams g;
        const uint32_t word = quant_group8<G8>(v, g);
        if (ok) {
            *reinterpret_cast<uint32_t *>(a.codes + orow * (N / 2) + ch * 4) = word;
            if ((ch % G8) == 0) {
                const int64_t gi = orow * (N / B) + (ch * 8) / B;
                a.scales[gi] = g.s16;
                a.zeros[gi] = g.z16;
            }
        }
    }
}

}  // namespace narhip
