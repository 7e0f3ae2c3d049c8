// Rank-k kernels, exact form (fp64 accumulation, one rounding to fp32).
//
//   u[t, s*k + r] = RN32( sum_{i in split s} x[t, i] * V[i, r] )    projection
//   C[t, i]       = RN32( sum_r u[t, r] * Wt[r, i] )                correction
//
// These are the reference's two BLAS products (quarot-llama3/nar_r4_kernel.py:
// 201-202; nar/kernels/r4_fused_v2.py:122-152 for the split partial layout
// partial[t, s*k + r]) computed as the exact sums: every product of a bf16 or
// fp32 value with an fp32 factor is exact in fp64, each thread adds its
// channels in index order.  Tiles of 32 tokens share every factor read.
#include "narhip_device.hpp"

namespace narhip {

struct ProjArgs {
    const uint16_t *x;      // bf16 [T, ldx]
    int64_t ldx;
    int64_t T, n;
    const float *v;         // [n, k]
    float *partial;         // [T, splits*k]
    int k, splits;
};

// grid: (ceil(T/32), splits); block 256.  Thread (tt, r) pairs are strided.
__global__ void __launch_bounds__(256)
proj_exact_kernel(ProjArgs a)
{
    constexpr int TT = 32, CW = 64;
    __shared__ float xs[TT][CW + 1];
    __shared__ float vs[CW][65];
    const int tid = threadIdx.x;
    const int64_t t0 = (int64_t)blockIdx.x * TT;
    const int split = blockIdx.y;
    const int64_t chunk = a.n / a.splits;
    const int64_t c_begin = split * chunk, c_end = c_begin + chunk;
    const int pairs = TT * a.k;
    double acc[8];
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] = 0.0;

    for (int64_t c0 = c_begin; c0 < c_end; c0 += CW) {
        const int cw = (int)((c_end - c0) < CW ? (c_end - c0) : CW);
        __syncthreads();
        for (int i = tid; i < TT * CW; i += 256) {
            const int tt = i / CW, cc = i % CW;
            const int64_t t = t0 + tt;
            float val = 0.0f;
            if (t < a.T && cc < cw) val = bf16lo(a.x[t * a.ldx + c0 + cc]);
            xs[tt][cc] = val;
        }
        for (int i = tid; i < CW * a.k; i += 256) {
            const int cc = i / a.k, r = i % a.k;
            vs[cc][r] = cc < cw ? a.v[(c0 + cc) * a.k + r] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int p = tid + j * 256;
            if (p < pairs) {
                const int tt = p / a.k, r = p % a.k;
                double s = acc[j];
                for (int cc = 0; cc < cw; cc++) s = fma((double)xs[tt][cc], (double)vs[cc][r], s);
                acc[j] = s;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int p = tid + j * 256;
        if (p < pairs) {
            const int tt = p / a.k, r = p % a.k;
            const int64_t t = t0 + tt;
            if (t < a.T) a.partial[t * (int64_t)a.splits * a.k + split * a.k + r] = (float)acc[j];
        }
    }
}

struct CorrArgs {
    const float *partial;   // [T, splits*k]
    int splits, k;
    const float *wt;        // [k, n]
    int64_t T, n;
    float *corr;            // [T, n]
};

// grid: (ceil(T/32), n/64); block 256: thread = (token tt = tid/8, 8 columns).
__global__ void __launch_bounds__(256)
corr_exact_kernel(CorrArgs a)
{
    constexpr int TT = 32, CW = 64;
    __shared__ float us[TT][65];
    __shared__ float ws[64][CW];
    const int tid = threadIdx.x;
    const int64_t t0 = (int64_t)blockIdx.x * TT;
    const int64_t c0 = (int64_t)blockIdx.y * CW;
    for (int i = tid; i < TT * a.k; i += 256) {
        const int tt = i / a.k, r = i % a.k;
        const int64_t t = t0 + tt;
        double s = 0.0;
        if (t < a.T)
            for (int sp = 0; sp < a.splits; sp++) s += (double)a.partial[t * (int64_t)a.splits * a.k + sp * a.k + r];
        us[tt][r] = (float)s;
    }
    for (int i = tid; i < a.k * CW; i += 256) {
        const int r = i / CW, cc = i % CW;
        ws[r][cc] = a.wt[(int64_t)r * a.n + c0 + cc];
    }
    __syncthreads();
    const int tt = tid >> 3;
    const int cb = (tid & 7) * 8;
    const int64_t t = t0 + tt;
    double acc[8];
#pragma unroll
    for (int e = 0; e < 8; e++) acc[e] = 0.0;
    for (int r = 0; r < a.k; r++) {
        const double ur = (double)us[tt][r];
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] = fma(ur, (double)ws[r][cb + e], acc[e]);
    }
    if (t < a.T) {
        float4 *d = reinterpret_cast<float4 *>(a.corr + t * a.n + c0 + cb);
        d[0] = make_float4((float)acc[0], (float)acc[1], (float)acc[2], (float)acc[3]);
        d[1] = make_float4((float)acc[4], (float)acc[5], (float)acc[6], (float)acc[7]);
    }
}

}  // namespace narhip
