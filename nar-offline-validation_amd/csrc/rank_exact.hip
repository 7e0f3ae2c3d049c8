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
#pragma once
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
template <int = 0>
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

// Projection on fp64 VALU for small ranks (k <= KMAX <= 16): fp64 partial sums
// per channel split, pd[t][s][KMAX] (internal workspace layout), folded by
// fold_f64_kernel into u = RN32(total).  Exact products, fp64 sums (the order
// of the fp64 additions differs from a sequential sum only by fp64 rounding).
//
// grid (ceil(T/16), splits), block 256: wave w owns tokens 4w..4w+3 of the
// 16-token tile, lane l the channel pairs c_begin + 2l + 128j of the split.  A
// lane keeps V of its two channels in fp64 registers and the 4 x KMAX running
// sums; x arrives as one 4-byte load per token (256 bytes per wave).  The lane
// sums are combined across the wave once per split (DPP within rows, then
// across rows).
struct ProjF64Args {
    const uint16_t *x;      // bf16 or (F16) fp16 rows
    int64_t ldx, T, n;
    const float *v;         // [n, k]
    double *pd;             // [T][splits][kstride], or null when pf is set
    int k, splits;
    float *pf;              // null, or fp32 partials [T, splits*k] (each split rounded once)
    int r0;                 // first rank of this launch's slice of KMAX ranks
    int kstride;            // rank stride of pd (>= k, a multiple of KMAX)
};

__device__ __forceinline__ double wave_sum64(double v)
{
    v += xchg64<0>(v);
    v += xchg64<1>(v);
    v += xchg64<2>(v);
    v += xchg64<3>(v);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

template <int KMAX, bool F16 = false>
__global__ void __launch_bounds__(256)
proj_f64_kernel(ProjF64Args a)
{
    constexpr int TT = 4;
    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int64_t t0 = (int64_t)blockIdx.x * 16 + TT * w;
    const int split = blockIdx.y;
    const int64_t chunk = a.n / a.splits;
    const int64_t c_begin = split * chunk, c_end = c_begin + chunk;
    const uint16_t *xr[TT];
#pragma unroll
    for (int tt = 0; tt < TT; tt++) {
        const int64_t t = t0 + tt < a.T ? t0 + tt : a.T - 1;
        xr[tt] = a.x + t * a.ldx;
    }
    double acc[TT][KMAX];
#pragma unroll
    for (int tt = 0; tt < TT; tt++)
#pragma unroll
        for (int r = 0; r < KMAX; r++) acc[tt][r] = 0.0;
    for (int64_t c = c_begin + 2 * lane; c < c_end; c += 128) {
        double v0[KMAX], v1[KMAX];
        if (a.k == KMAX && a.r0 == 0) {
            // rows c and c+1 of V: 2 KMAX contiguous floats, 32-byte aligned
            const float4 *vr = reinterpret_cast<const float4 *>(a.v + c * KMAX);
#pragma unroll
            for (int q = 0; q < KMAX / 4; q++) {
                const float4 f0 = vr[q], f1 = vr[KMAX / 4 + q];
                v0[4 * q] = f0.x; v0[4 * q + 1] = f0.y; v0[4 * q + 2] = f0.z; v0[4 * q + 3] = f0.w;
                v1[4 * q] = f1.x; v1[4 * q + 1] = f1.y; v1[4 * q + 2] = f1.z; v1[4 * q + 3] = f1.w;
            }
        } else {
#pragma unroll
            for (int r = 0; r < KMAX; r++) {
                const int rr = a.r0 + r;
                v0[r] = rr < a.k ? (double)a.v[c * a.k + rr] : 0.0;
                v1[r] = rr < a.k ? (double)a.v[(c + 1) * a.k + rr] : 0.0;
            }
        }
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            const uint32_t xw = *reinterpret_cast<const uint32_t *>(xr[tt] + c);
            const double x0 = F16 ? (double)f16_bits_to_f32((uint16_t)(xw & 0xffffu)) : (double)bf16lo(xw);
            const double x1 = F16 ? (double)f16_bits_to_f32((uint16_t)(xw >> 16)) : (double)bf16hi(xw);
#pragma unroll
            for (int r = 0; r < KMAX; r++) acc[tt][r] = fma(x1, v1[r], fma(x0, v0[r], acc[tt][r]));
        }
    }
#pragma unroll
    for (int tt = 0; tt < TT; tt++) {
        const int64_t t = t0 + tt;
#pragma unroll
        for (int r = 0; r < KMAX; r++) {
            const double sum = wave_sum64(acc[tt][r]);
            if (lane == 0 && t < a.T) {
                if (a.pf) {
                    if (a.r0 + r < a.k) a.pf[(t * a.splits + split) * a.k + a.r0 + r] = (float)sum;
                } else {
                    a.pd[(t * a.splits + split) * a.kstride + a.r0 + r] = sum;
                }
            }
        }
    }
}

// u[t, r] = RN32( sum_s pd[t][s][r] ), fp64 partials folded in split order.
template <int = 0>
__global__ void __launch_bounds__(256)
fold_f64_kernel(const double *pd, int splits, int kmax, int k, int64_t T, float *u)
{
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= T * k) return;
    const int64_t t = idx / k;
    const int r = (int)(idx % k);
    const double *p = pd + t * (int64_t)splits * kmax + r;
    double s = 0.0;
    for (int sp = 0; sp < splits; sp++) s += p[(int64_t)sp * kmax];
    u[idx] = (float)s;
}

// u[t, r] = RN32( sum_s partial[t, s*k + r] ), the split partials folded in
// fp64 in split order (one thread per (t, r)).
template <int = 0>
__global__ void __launch_bounds__(256)
fold_f32_kernel(const float *partial, int splits, int k, int64_t T, float *u)
{
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= T * k) return;
    const int64_t t = idx / k;
    const int r = (int)(idx % k);
    const float *p = partial + t * (int64_t)splits * k + r;
    double s = 0.0;
    for (int sp = 0; sp < splits; sp++) s += (double)p[(int64_t)sp * k];
    u[idx] = (float)s;
}

struct CorrArgs {
    const float *partial;   // [T, splits*k]
    int splits, k;
    const float *wt;        // [k, n]
    int64_t T, n;
    float *corr;            // [T, n]
};

// grid: (ceil(T/32), n/64); block 256: thread = (token tt = tid/8, 8 columns).
template <int = 0>
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
