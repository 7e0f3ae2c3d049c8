// Rank-k stages on bf16 MFMA (k >= 16 over a full row).
//
//   prep_v / prep_w : fp32 factors -> three exact bf16 terms in MFMA-friendly
//                     layouts (done once per factor set, like the reference's
//                     fp16_terms / FoldedR4 term padding, nar_r4_kernel.py:151-187)
//   proj_mfma       : Kernel A, u partials = x V over channel splits
//                     (nar/kernels/r4_fused_v3.py:83-135): x is bf16 (exact),
//                     V enters as hi/mid/lo terms with separate accumulators,
//                     several short accumulation chains per wave reduced in fp64
//   corr_quant      : x' = P - u W^T with u and W^T both as three bf16 terms
//                     (six significant term products), then the INT4 quantizer
#include "mfma.hpp"
#include "narhip_device.hpp"

namespace narhip {

// v [n, k] fp32 -> vt [3][kp16][n] bf16 (rank-major, zero rows for r >= k)
__global__ void __launch_bounds__(256)
prep_v_kernel(const float *v, int64_t n, int k, int kp, __bf16 *vt)
{
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= n * kp) return;
    const int64_t r = idx / n, i = idx % n;
    const float val = r < k ? v[i * k + r] : 0.0f;
    __bf16 h, m, l;
    split3(val, h, m, l);
    const int64_t plane = (int64_t)kp * n;
    vt[r * n + i] = h;
    vt[plane + r * n + i] = m;
    vt[2 * plane + r * n + i] = l;
}

// w_t [k, n] fp32 -> wtt [3][n][kp32] bf16 (channel-major, zero ranks for r >= k)
__global__ void __launch_bounds__(256)
prep_w_kernel(const float *wt, int64_t n, int k, int kp, __bf16 *wtt)
{
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= n * kp) return;
    const int64_t i = idx / kp, r = idx % kp;
    const float val = r < k ? wt[r * n + i] : 0.0f;
    __bf16 h, m, l;
    split3(val, h, m, l);
    const int64_t plane = (int64_t)kp * n;
    wtt[i * kp + r] = h;
    wtt[plane + i * kp + r] = m;
    wtt[2 * plane + i * kp + r] = l;
}

struct ProjMfmaArgs {
    const uint16_t *x;     // bf16 [T, ldx]
    int64_t ldx, T, n;
    const __bf16 *vt;      // [3][kp][n]
    int kp, k, splits;
    int64_t cs;            // channels per split (multiple of 32)
    float *partial;        // [T, splits*k]
};

// grid (ceil(T/64), splits), block 256: wave w owns tokens 16w..16w+15 of the tile,
// all MT rank tiles of 16.  NCH independent accumulation chains per tile.
template <int MT, int NCH>
__global__ void __launch_bounds__(256)
proj_mfma_kernel(ProjMfmaArgs a)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int64_t t = (int64_t)blockIdx.x * 64 + w * 16 + c16;
    const int64_t tc = t < a.T ? t : a.T - 1;
    const int s = blockIdx.y;
    const int64_t c_begin = (int64_t)s * a.cs;
    const int steps = (int)(a.cs / 32);
    const uint16_t *xrow = a.x + tc * a.ldx + c_begin + 8 * g;
    const int64_t plane = (int64_t)a.kp * a.n;

    floatx4 acc_h[MT][NCH], acc_l[MT][NCH];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int c = 0; c < NCH; c++) { acc_h[mt][c] = zero4(); acc_l[mt][c] = zero4(); }

    for (int j0 = 0; j0 < steps; j0 += NCH) {
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            const int j = j0 + c;
            if (j < steps) {
                const bf16x8 b = *reinterpret_cast<const bf16x8 *>(xrow + 32 * j);
                const int64_t col = c_begin + 32 * j + 8 * g;
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const __bf16 *vp = a.vt + (int64_t)(16 * mt + c16) * a.n + col;
                    acc_h[mt][c] = mfma_bf16(load_bf16x8(vp), b, acc_h[mt][c]);
                    acc_l[mt][c] = mfma_bf16(load_bf16x8(vp + plane), b, acc_l[mt][c]);
                    acc_l[mt][c] = mfma_bf16(load_bf16x8(vp + 2 * plane), b, acc_l[mt][c]);
                }
            }
        }
    }
    if (t >= a.T) return;
    float *out = a.partial + t * (int64_t)a.splits * a.k + (int64_t)s * a.k;
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 16 * mt + 4 * g + i;
            double sum = 0.0;
#pragma unroll
            for (int c = 0; c < NCH; c++) sum += (double)acc_h[mt][c][i] + (double)acc_l[mt][c][i];
            if (r < a.k) out[r] = (float)sum;
        }
}

struct CorrQuantArgs {
    const float *P;        // [T, n] rotated rows before the rank term
    int64_t T, n;
    const float *partial;  // [T, splits*k]
    int splits, k;
    const __bf16 *wtt;     // [3][n][kp]
    int kp;
    uint8_t *codes;
    uint16_t *scales;
    uint16_t *zeros;
    const int64_t *dest;
    float *rotated;        // optional x' [T, n]
    int64_t cw;            // channels per workgroup (multiple of 128)
};

// grid (ceil(T/64), n/cw), block 256.  Tile: 64 tokens (wave w: tokens 16w..) x
// cw channels in sub-tiles of 128.  MFMA: M = tokens, N = channels, K = ranks.
template <int B, int KS>
__global__ void __launch_bounds__(256)
corr_quant_kernel(CorrQuantArgs a)
{
    constexpr int KP = 32 * KS;
    __shared__ __bf16 us[3][64][KP + 8];
    __shared__ uint8_t cstage[64][128 + 4];
    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int64_t t0 = (int64_t)blockIdx.x * 64;
    const int64_t cbase = (int64_t)blockIdx.y * a.cw;

    // u for the 64 tokens: fp64 fold of the split partials, rounded once, split in 3
    for (int p = tid; p < 64 * KP; p += 256) {
        const int tl = p / KP, r = p % KP;
        const int64_t t = t0 + tl;
        double sum = 0.0;
        if (t < a.T && r < a.k) {
            const float *pp = a.partial + t * (int64_t)a.splits * a.k + r;
            for (int s = 0; s < a.splits; s++) sum += (double)pp[(int64_t)s * a.k];
        }
        __bf16 h, m, l;
        split3((float)sum, h, m, l);
        us[0][tl][r] = h; us[1][tl][r] = m; us[2][tl][r] = l;
    }
    __syncthreads();
    bf16x8 ua[3][KS];
#pragma unroll
    for (int term = 0; term < 3; term++)
#pragma unroll
        for (int ks = 0; ks < KS; ks++)
            ua[term][ks] = *reinterpret_cast<const bf16x8 *>(&us[term][16 * w + c16][32 * ks + 8 * g]);

    const int64_t plane = (int64_t)a.kp * a.n;
    const int tl4 = 16 * w + 4 * g;            // first of this lane's 4 token rows
    for (int64_t c0 = cbase; c0 < cbase + a.cw; c0 += 128) {
        float xv[8][4];
#pragma unroll
        for (int nt = 0; nt < 8; nt++) {
            const int64_t ch = c0 + 16 * nt + c16;
            floatx4 main = zero4(), small = zero4();
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const __bf16 *wp = a.wtt + ch * a.kp + 32 * ks + 8 * g;
                const bf16x8 wh = load_bf16x8(wp), wm = load_bf16x8(wp + plane), wl = load_bf16x8(wp + 2 * plane);
                main = mfma_bf16(ua[0][ks], wh, main);
                small = mfma_bf16(ua[0][ks], wm, small);
                small = mfma_bf16(ua[1][ks], wh, small);
                small = mfma_bf16(ua[0][ks], wl, small);
                small = mfma_bf16(ua[2][ks], wh, small);
                small = mfma_bf16(ua[1][ks], wm, small);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                int64_t t = t0 + tl4 + i;
                if (t >= a.T) t = a.T - 1;
                const float corr = main[i] + small[i];
                xv[nt][i] = a.P[t * a.n + ch] - corr;
            }
        }
        if (a.rotated) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int64_t t = t0 + tl4 + i;
                if (t < a.T)
#pragma unroll
                    for (int nt = 0; nt < 8; nt++) a.rotated[t * a.n + c0 + 16 * nt + c16] = xv[nt][i];
            }
        }
        // quantize: group = B/16 consecutive N-tiles x the 16 lanes of this row group
        constexpr int NTG = B / 16;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int64_t t = t0 + tl4 + i;
            const int64_t orow = t < a.T ? (a.dest ? a.dest[t] : t) : 0;
#pragma unroll
            for (int gq = 0; gq < 8 / NTG; gq++) {
                float lo = xv[gq * NTG][i], hi = lo;
#pragma unroll
                for (int j = 1; j < NTG; j++) { lo = fminf(lo, xv[gq * NTG + j][i]); hi = fmaxf(hi, xv[gq * NTG + j][i]); }
                group_minmax<16>(lo, hi);
                const GroupParams gp = group_params(lo, hi);
#pragma unroll
                for (int j = 0; j < NTG; j++)
                    cstage[tl4 + i][16 * (gq * NTG + j) + c16] = (uint8_t)quant_code(xv[gq * NTG + j][i], gp);
                if (c16 == 0 && t < a.T) {
                    const int64_t gi = orow * (a.n / B) + (c0 + gq * B) / B;
                    a.scales[gi] = gp.s16;
                    a.zeros[gi] = gp.z16;
                }
            }
        }
        __syncthreads();
        // pack: 64 tokens x 16 words (8 codes each) = 1024 words, 4 per thread
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int idx = tid + 256 * p;
            const int tl = idx >> 4, wd = idx & 15;
            const int64_t t = t0 + tl;
            uint32_t word = 0;
#pragma unroll
            for (int e = 0; e < 8; e++) word |= (uint32_t)cstage[tl][wd * 8 + e] << (4 * e);
            if (t < a.T) {
                const int64_t orow = a.dest ? a.dest[t] : t;
                *reinterpret_cast<uint32_t *>(a.codes + orow * (a.n / 2) + (c0 + wd * 8) / 2) = word;
            }
        }
        __syncthreads();
    }
}

// Device self-test of the operand mapping: one MFMA on per-lane inputs.
__global__ void mfma_probe_kernel(const __bf16 *a, const __bf16 *b, float *d)
{
    const int l = threadIdx.x;
    const floatx4 r = mfma_bf16(load_bf16x8(a + 8 * l), load_bf16x8(b + 8 * l), zero4());
#pragma unroll
    for (int i = 0; i < 4; i++) d[4 * l + i] = r[i];
}

}  // namespace narhip
