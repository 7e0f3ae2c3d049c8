// Full-row Hadamard rows for the large Paley orders of the Qwen3 widths
// (nar/activation_experiments.py:188-217): 68 x 256 (14B), 76 x 128 (8B),
// 200 x 128 (32B), i.e. y = (H_m (x) H_q) diag(signs) x per row, fp32 out.
//
// One workgroup per row.  The row goes into LDS as fp32 (times the signs),
// every q-point segment gets the reference's FWHT stages (widths 1, 2, ..,
// q/2, in that order) and the fp32 division by fp32(sqrt q); then each output
// y[a][c] = RN32(sum_{a'} F[a'][c] * h[a][a']) is accumulated in fp64 over a'
// in increasing order, with h = +-|entry|:
//   orders 68 and 200: |entry| = fp64(1/sqrt(m)); each product is rounded in
//     fp64 before the add (the reference forms this product in fp64);
//   other orders: |entry| = fp32(1/sqrt(m)); the product is exact in fp64 and
//     one fma adds it.
// The +-1 pattern is built once per workgroup as sign bits in LDS from the
// quadratic-residue table of the construction's prime, and read as one word
// per 32 terms (rows by waves, so the row and the word are wave-uniform and
// each term's sign is a scalar bit test): Paley I (order p + 1, p a
// prime = 3 mod 4: ones bordering Q - I, Q[r][c] = chi(r - c)) or Paley II
// (order 2(p + 1), p = 1 mod 4: [[C + I, C - I], [C - I, -C - I]] with the
// conference matrix C bordered by ones around Q), the constructions of
// nar/activation_experiments.py:141-185.
//
// A full-row rank term arrives as C = RN32(u W^T) (corr_exact_kernel) and is
// subtracted in fp32 at the store, x' = P - C as the reference's
// reference_transform.  Not a bandwidth kernel: m fp64 terms per output
// element (m = 200: 5.1 M per row of 25600).  It serves the hooks'
// full_hadamard_rows and rotate-then-quantize for these widths.
#pragma once
#include "narhip_device.hpp"

namespace narhip {

constexpr int PR_MAX_ELEMS = 32768;       // m q <= 32768: the row fits 128 KB of LDS
constexpr int PR_THREADS = 1024;

struct PaleyRowsArgs {
    const uint16_t *x;      // bf16 [T, ldx]
    int64_t ldx, T;
    const float *signs;     // [m q] or null
    float *out;             // fp32 [T, m q]
    const float *corr;      // fp32 [T, m q] rank-k term C (out = P - C), or null
    int m, q;               // Paley order, power-of-two factor
    int p;                  // the construction's prime
    int kind;               // 1: Paley I, 2: Paley II
    int fp64_product;       // 1: products rounded in fp64 (orders 68, 200)
    float sq;               // fp32(sqrt q)
    double hm;              // |entry| of H_m / sqrt(m) as the products use it
    uint32_t residue[8];    // bit d set <=> d is a nonzero square mod p (p < 256)
};

// Entry (r, c) of the +-1 Paley matrix is -1 (r, c < m); res = the quadratic
// residue bits of the construction's prime.
__device__ __forceinline__ bool paley_neg(const PaleyRowsArgs &a, const uint32_t *res, int r, int c)
{
    auto chi_neg = [&](int i, int j) {       // chi(i - j mod p) = -1, i != j, i, j in [1, p]
        int d = i - j;
        if (d < 0) d += a.p;
        return ((res[d >> 5] >> (d & 31)) & 1u) == 0;
    };
    if (a.kind == 1) {
        if (r == 0 || c == 0) return false;
        if (r == c) return true;             // Q[r][r] - 1 = -1
        return chi_neg(r, c);
    }
    const int h = a.p + 1;
    const bool br = r >= h, bc = c >= h;
    const int rr = br ? r - h : r, cc = bc ? c - h : c;
    int cv;                                  // conference entry C[rr][cc]
    if (rr == cc) cv = 0;
    else if (rr == 0 || cc == 0) cv = 1;
    else cv = chi_neg(rr, cc) ? -1 : 1;
    const int e = rr == cc ? 1 : 0;
    const int v = (!br && !bc) ? cv + e : (br != bc) ? cv - e : -cv - e;
    return v < 0;
}

// Words of sign bits per row of H_m.
__host__ __device__ constexpr int paley_sign_words(int m) { return (m + 31) / 32; }

// CPL output columns per lane (q = 64 CPL, or q < 64 with CPL = 1); FP64P:
// products rounded in fp64 (a.fp64_product), as a template argument so that
// the term loop has no branch.
template <int CPL, bool FP64P>
__global__ void __launch_bounds__(PR_THREADS)
paley_rows_kernel(PaleyRowsArgs a)
{
    extern __shared__ __align__(16) float F[];          // [m][q], then the sign bits [m][W]
    __shared__ uint32_t res[8];
    const int n = a.m * a.q;
    const int W = paley_sign_words(a.m);
    uint32_t *sgn = reinterpret_cast<uint32_t *>(F + n);
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < 8; j++)
        if (tid == j) res[j] = a.residue[j];
    __syncthreads();
    // the sign bits of H_m, once per workgroup: bit b of word (r, w) is entry (r, 32 w + b) < 0
    for (int i = tid; i < a.m * W; i += PR_THREADS) {
        const int r = i / W, w = i - r * W;
        uint32_t bits = 0;
        for (int b = 0; b < 32; b++) {
            const int c = 32 * w + b;
            if (c < a.m && paley_neg(a, res, r, c)) bits |= 1u << b;
        }
        sgn[i] = bits;
    }
    const uint16_t *xr = a.x + (int64_t)blockIdx.x * a.ldx;
    for (int i = tid; i < n; i += PR_THREADS) {
        float v = __uint_as_float((uint32_t)xr[i] << 16);
        if (a.signs) v *= a.signs[i];
        F[i] = v;
    }
    __syncthreads();
    // FWHT_q of each segment: at width w, pair (i, i + w) in blocks of 2w
    const int half = a.q >> 1;
    for (int w = 1; w < a.q; w <<= 1) {
        for (int b = tid; b < n / 2; b += PR_THREADS) {
            const int s = b / half, j = b - s * half;
            const int i0 = s * a.q + (j / w) * 2 * w + j % w, i1 = i0 + w;
            const float x0 = F[i0], x1 = F[i1];
            F[i0] = x0 + x1;
            F[i1] = x0 - x1;
        }
        __syncthreads();
    }
    for (int i = tid; i < n; i += PR_THREADS) F[i] = F[i] / a.sq;
    __syncthreads();

    // rows of H_m by waves, columns by lanes
    const int lane = tid & 63, wave = tid >> 6;
    float *o = a.out + (int64_t)blockIdx.x * n;
    for (int r = wave; r < a.m; r += PR_THREADS / 64) {
        const int ru = __builtin_amdgcn_readfirstlane(r);
        double acc[CPL];
#pragma unroll
        for (int j = 0; j < CPL; j++) acc[j] = 0.0;
        for (int w = 0; w < W; w++) {
            const uint32_t bits = __builtin_amdgcn_readfirstlane(sgn[ru * W + w]);
            const int cend = a.m - 32 * w < 32 ? a.m - 32 * w : 32;
#pragma unroll 4
            for (int b = 0; b < cend; b++) {
                const double h = (bits >> b) & 1u ? -a.hm : a.hm;
                const float *fr = F + (32 * w + b) * a.q;
#pragma unroll
                for (int j = 0; j < CPL; j++) {
                    const int c = lane + 64 * j;
                    const double f = (double)fr[c < a.q ? c : 0];
                    if constexpr (FP64P) {
                        const double pr = f * h;
                        acc[j] = acc[j] + pr;
                    } else {
                        acc[j] = fma(f, h, acc[j]);
                    }
                }
            }
        }
        const float *cr = a.corr ? a.corr + (int64_t)blockIdx.x * n : nullptr;
#pragma unroll
        for (int j = 0; j < CPL; j++) {
            const int c = lane + 64 * j;
            if (c < a.q) {
                const float pv = (float)acc[j];
                o[ru * a.q + c] = cr ? pv - cr[ru * a.q + c] : pv;
            }
        }
    }
}

}  // namespace narhip
