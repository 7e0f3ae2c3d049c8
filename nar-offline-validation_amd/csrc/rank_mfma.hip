// Rank-k stages on bf16 MFMA (k >= 16 over a full row).
//
//   prep_v / prep_w : fp32 factors -> three exact bf16 terms in MFMA-friendly
//                     layouts (done once per factor set, like the reference's
//                     fp16_terms / FoldedR4 term padding, nar_r4_kernel.py:151-187)
//   proj_mfma       : Kernel A, u partials = x V over channel splits
//                     (nar/kernels/r4_fused_v3.py:83-135): x is bf16 (exact),
//                     V enters as hi/mid/lo terms, hi and mid+lo in separate
//                     accumulators, folded in fp64 at the end of the split
//   corr_quant      : x' = P - u W^T with u and W^T both as three bf16 terms
//                     (the six term products of weight >= 2^-16), then the
//                     INT4 quantizer of nar/experiment.py:158-184
// Factor tiles are staged in LDS once per workgroup and shared by its waves.
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
    int64_t cs;            // channels per split (multiple of 128)
    float *partial;        // [T, splits*k]
};

// grid (ceil(T/256), splits), block 256.  Wave w owns tokens 64w..64w+63 of the
// 256-token tile as four 16-token N tiles; all MT rank tiles of 16 rows.  The V
// terms of each 128-channel block are staged in LDS and read by all waves.
template <int MT>
__global__ void __launch_bounds__(256)
proj_mfma_kernel(ProjMfmaArgs a)
{
    constexpr int KB = 128;                 // channels per LDS block
    constexpr int ROWS = 16 * MT;
    __shared__ __bf16 vs[3][ROWS][KB + 8];
    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int64_t tbase = (int64_t)blockIdx.x * 256 + w * 64 + c16;
    const int s = blockIdx.y;
    const int64_t c_begin = (int64_t)s * a.cs;
    const int64_t plane = (int64_t)a.kp * a.n;
    const uint16_t *xrow[4];
#pragma unroll
    for (int nt = 0; nt < 4; nt++) {
        int64_t t = tbase + 16 * nt;
        if (t >= a.T) t = a.T - 1;
        xrow[nt] = a.x + t * a.ldx + c_begin + 8 * g;
    }
    floatx4 acc_h[MT][4], acc_l[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < 4; nt++) { acc_h[mt][nt] = zero4(); acc_l[mt][nt] = zero4(); }

    for (int64_t cb = 0; cb < a.cs; cb += KB) {
        __syncthreads();
        // stage 3 x ROWS x 128 bf16 (16-byte pieces)
        for (int p = tid; p < 3 * ROWS * (KB / 8); p += 256) {
            const int term = p / (ROWS * (KB / 8));
            const int rem = p % (ROWS * (KB / 8));
            const int r = rem / (KB / 8), c8 = rem % (KB / 8);
            *reinterpret_cast<bf16x8 *>(&vs[term][r][c8 * 8]) =
                load_bf16x8(a.vt + term * plane + (int64_t)r * a.n + c_begin + cb + c8 * 8);
        }
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < KB / 32; ks++) {
            bf16x8 b[4];
#pragma unroll
            for (int nt = 0; nt < 4; nt++)
                b[nt] = *reinterpret_cast<const bf16x8 *>(xrow[nt] + cb + 32 * ks);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const bf16x8 ah = *reinterpret_cast<const bf16x8 *>(&vs[0][16 * mt + c16][32 * ks + 8 * g]);
                const bf16x8 am = *reinterpret_cast<const bf16x8 *>(&vs[1][16 * mt + c16][32 * ks + 8 * g]);
                const bf16x8 al = *reinterpret_cast<const bf16x8 *>(&vs[2][16 * mt + c16][32 * ks + 8 * g]);
#pragma unroll
                for (int nt = 0; nt < 4; nt++) {
                    acc_h[mt][nt] = mfma_bf16(ah, b[nt], acc_h[mt][nt]);
                    acc_l[mt][nt] = mfma_bf16(am, b[nt], acc_l[mt][nt]);
                    acc_l[mt][nt] = mfma_bf16(al, b[nt], acc_l[mt][nt]);
                }
            }
        }
    }
#pragma unroll
    for (int nt = 0; nt < 4; nt++) {
        const int64_t t = tbase + 16 * nt;
        if (t >= a.T) continue;
        float *out = a.partial + t * (int64_t)a.splits * a.k + (int64_t)s * a.k;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = 16 * mt + 4 * g + i;
                if (r < a.k) out[r] = (float)((double)acc_h[mt][nt][i] + (double)acc_l[mt][nt][i]);
            }
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

// grid (ceil(T/64), n/cw), block 256.  Tile: 64 tokens (wave w: tokens 16w..16w+15,
// the MFMA N dimension) x 128-channel sub-tiles (8 M tiles of 16 channels).
// Lane l holds x' for token 16w + l%16 and channels 16 mt + 4g .. +3 (g = l/16).
template <int B, int KS>
__global__ void __launch_bounds__(256)
corr_quant_kernel(CorrQuantArgs a)
{
    constexpr int KP = 32 * KS;
    __shared__ __bf16 us[3][64][KP + 8];
    __shared__ __bf16 ws[3][128][KP + 8];
    __shared__ uint8_t cstage[64][128 + 16];
    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int64_t t0 = (int64_t)blockIdx.x * 64;
    const int64_t cbase = (int64_t)blockIdx.y * a.cw;
    const int tl = 16 * w + c16;                 // this lane's token within the tile
    const int64_t t = t0 + tl;
    const int64_t tc = t < a.T ? t : a.T - 1;
    const bool tok_ok = t < a.T;

    // u for the 64 tokens: fp64 fold of the split partials, rounded once, split in 3
    for (int p = tid; p < 64 * KP; p += 256) {
        const int tt = p / KP, r = p % KP;
        const int64_t tg = t0 + tt;
        double sum = 0.0;
        if (tg < a.T && r < a.k) {
            const float *pp = a.partial + tg * (int64_t)a.splits * a.k + r;
            for (int s = 0; s < a.splits; s++) sum += (double)pp[(int64_t)s * a.k];
        }
        __bf16 h, m, l;
        split3((float)sum, h, m, l);
        us[0][tt][r] = h; us[1][tt][r] = m; us[2][tt][r] = l;
    }
    __syncthreads();
    bf16x8 ub[3][KS];
#pragma unroll
    for (int term = 0; term < 3; term++)
#pragma unroll
        for (int ks = 0; ks < KS; ks++)
            ub[term][ks] = *reinterpret_cast<const bf16x8 *>(&us[term][tl][32 * ks + 8 * g]);

    const int64_t plane = (int64_t)a.kp * a.n;
    const int64_t orow = tok_ok ? (a.dest ? a.dest[t] : t) : 0;
    for (int64_t c0 = cbase; c0 < cbase + a.cw; c0 += 128) {
        // stage W^T terms of these 128 channels
        for (int p = tid; p < 3 * 128 * (KP / 8); p += 256) {
            const int term = p / (128 * (KP / 8));
            const int rem = p % (128 * (KP / 8));
            const int ch = rem / (KP / 8), r8 = rem % (KP / 8);
            *reinterpret_cast<bf16x8 *>(&ws[term][ch][r8 * 8]) =
                load_bf16x8(a.wtt + term * plane + (c0 + ch) * a.kp + r8 * 8);
        }
        __syncthreads();
        float xv[8][4];
        const float *prow = a.P + tc * a.n + c0 + 4 * g;
#pragma unroll
        for (int mt = 0; mt < 8; mt++) {
            const float4 pv = *reinterpret_cast<const float4 *>(prow + 16 * mt);
            floatx4 main = zero4(), small = zero4();
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const bf16x8 wh = *reinterpret_cast<const bf16x8 *>(&ws[0][16 * mt + c16][32 * ks + 8 * g]);
                const bf16x8 wm = *reinterpret_cast<const bf16x8 *>(&ws[1][16 * mt + c16][32 * ks + 8 * g]);
                const bf16x8 wl = *reinterpret_cast<const bf16x8 *>(&ws[2][16 * mt + c16][32 * ks + 8 * g]);
                main = mfma_bf16(wh, ub[0][ks], main);
                small = mfma_bf16(wm, ub[0][ks], small);
                small = mfma_bf16(wh, ub[1][ks], small);
                small = mfma_bf16(wl, ub[0][ks], small);
                small = mfma_bf16(wh, ub[2][ks], small);
                small = mfma_bf16(wm, ub[1][ks], small);
            }
            xv[mt][0] = pv.x - (main[0] + small[0]);
            xv[mt][1] = pv.y - (main[1] + small[1]);
            xv[mt][2] = pv.z - (main[2] + small[2]);
            xv[mt][3] = pv.w - (main[3] + small[3]);
        }
        if (a.rotated && tok_ok) {
#pragma unroll
            for (int mt = 0; mt < 8; mt++)
                *reinterpret_cast<float4 *>(a.rotated + t * a.n + c0 + 16 * mt + 4 * g) =
                    make_float4(xv[mt][0], xv[mt][1], xv[mt][2], xv[mt][3]);
        }
        // quantize: a group of B channels = B/16 M tiles x the four lane groups g
        // (lanes c16, c16+16, c16+32, c16+48 hold the same token)
        constexpr int MTG = B / 16;
#pragma unroll
        for (int gq = 0; gq < 8 / MTG; gq++) {
            float lo = xv[gq * MTG][0], hi = lo;
#pragma unroll
            for (int j = 0; j < MTG; j++)
#pragma unroll
                for (int i = 0; i < 4; i++) { lo = fminf(lo, xv[gq * MTG + j][i]); hi = fmaxf(hi, xv[gq * MTG + j][i]); }
            lo = fminf(lo, __shfl_xor(lo, 16)); hi = fmaxf(hi, __shfl_xor(hi, 16));
            lo = fminf(lo, __shfl_xor(lo, 32)); hi = fmaxf(hi, __shfl_xor(hi, 32));
            const GroupParams gp = group_params(lo, hi);
            const float rs = 1.0f / gp.s;
            bool tie = false;
            uint32_t q4[MTG];
#pragma unroll
            for (int j = 0; j < MTG; j++) {
                q4[j] = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) q4[j] |= quant_code_fast(xv[gq * MTG + j][i], gp.z, rs, tie) << (8 * i);
            }
            if (__builtin_expect(__any(tie), 0)) {
#pragma unroll
                for (int j = 0; j < MTG; j++) {
                    q4[j] = 0;
#pragma unroll
                    for (int i = 0; i < 4; i++) q4[j] |= quant_code(xv[gq * MTG + j][i], gp) << (8 * i);
                }
            }
#pragma unroll
            for (int j = 0; j < MTG; j++)
                *reinterpret_cast<uint32_t *>(&cstage[tl][16 * (gq * MTG + j) + 4 * g]) = q4[j];
            if (g == 0 && tok_ok) {
                const int64_t gi = orow * (a.n / B) + (c0 + gq * B) / B;
                a.scales[gi] = gp.s16;
                a.zeros[gi] = gp.z16;
            }
        }
        __syncthreads();
        // pack: 64 tokens x 16 words (8 codes each), 4 per thread
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int idx = tid + 256 * p;
            const int tt = idx >> 4, wd = idx & 15;
            const int64_t tg = t0 + tt;
            const uint8_t *src = &cstage[tt][wd * 8];
            uint32_t word = 0;
#pragma unroll
            for (int e = 0; e < 8; e++) word |= (uint32_t)src[e] << (4 * e);
            if (tg < a.T) {
                const int64_t orw = a.dest ? a.dest[tg] : tg;
                *reinterpret_cast<uint32_t *>(a.codes + orw * (a.n / 2) + (c0 + wd * 8) / 2) = word;
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
