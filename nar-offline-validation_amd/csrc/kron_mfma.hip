// Kronecker row transform with the Paley factor on bf16 MFMA.
//
// Persistent workgroups over tokens, one 16-lane row per segment (16 M threads):
//   phase 1  F[a, :] = FWHT_Q(x[a*Q:(a+1)*Q]) / fp32(sqrt(Q))   (DPP, as rq_row.hip)
//   phase 2  P[a, c] = hm * S[a, c],  S = Hm(+-1) F                  (MFMA)
//            F enters as three exact bf16 terms; S1 = Hm F_hi and S23 = Hm (F_mid + F_lo)
//            are sums of bf16 values with +-1 weights, and P = fma(hm, S1, hm*S23)
//            is the fp32 rounding of hm*S -- the oracle's fp64 definition of the
//            reference's BLAS product -- whenever the two sums are exact in fp32.
//   phase 3  either the group quantizer (no rank term) or a coalesced copy of P
//            to global memory for the rank-k correction kernel.
#pragma once
#include "mfma.hpp"
#include "narhip_device.hpp"

namespace narhip {

struct KronArgs {
    const uint16_t *x;
    int64_t ldx, T, n;
    const float *signs;
    float *P;              // [T, n] output when not quantizing
    uint8_t *codes;
    uint16_t *scales;
    uint16_t *zeros;
    const int64_t *dest;
    float *rotated;
    PaleyTable paley;
    float sq, rsq, hm;     // fp32(sqrt(Q)), RN(1/sq), RN(1/fp32(sqrt(M)))
    float *deq;            // fp32 [rows, n]: the hooks' tuple (codes unpacked [rows, n]), or null
};

// F in LDS: row a of the token's M x Q block at a * Q, column c stored at
// c ^ fsw(a).  Phase 2 reads a column from rows 8g + j and writes rows
// 16 mt + 4g + i (g = lane / 16); flipping column bit 4 by bit 3 ^ bit 2 of the
// row puts lanes with g = 0 and g = 1 in different halves of the 32 banks in
// both, and moves only whole 16-float blocks, so the row-wise float4 accesses of
// phases 1 and 3 stay aligned.
constexpr int KPAD = 0;
__device__ __forceinline__ int fsw(int a) { return (((a >> 3) ^ (a >> 2)) & 1) << 4; }

// Rows of F in LDS.  For M > 16 the block is padded to the MFMA's 32 rows:
// rows M..31 are zeroed once per workgroup, and phase 2 then reads and writes
// all 32 rows without row guards (the Paley operand's columns >= M are zero,
// and the padded rows are always rewritten with +0).
template <int M> constexpr int kron_rows() { return M > 16 ? 32 : M; }

// PERSIST: a grid of at most one wave of workgroups walks all tokens,
// prefetching the next token's x (the launcher uses it from Q = 512 on);
// otherwise one workgroup per token.
template <int M, int Q, int B, bool QUANT, bool PERSIST>
__global__ void __launch_bounds__(16 * M)
kron_mfma_kernel(KronArgs a)
{
    constexpr int NH = Q / 128;
    constexpr int NV = 8 * NH;
    constexpr int N = M * Q;
    constexpr int QS = Q + KPAD;            // LDS row stride (floats, no padding)
    constexpr int NMT = (M + 15) / 16;
    constexpr int NT = 16 * M;              // threads: one 16-lane row per segment
    constexpr int NW = NT / 64;             // waves
    extern __shared__ __align__(16) float F[];
    const int tid = threadIdx.x;
    const int l16 = tid & 15;
    const int row = tid >> 4;
    const int chunk = lane_chunk(l16);
    float sj[4];
#pragma unroll
    for (int j = 0; j < 4; j++) sj[j] = ((chunk >> j) & 1) ? -1.0f : 1.0f;
    const float sigma = sj[0] * sj[1] * sj[2] * sj[3];

    // Paley rows as the MFMA A operand, lane l's fragment at hat[mt][l]: built
    // by wave 0 only (the lane-indexed table lookup is a select chain) and read
    // by every wave after the first barrier
    const int lane = tid & 63, wv = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    __shared__ __align__(16) bf16x8 hat[NMT][64];
    if (wv == 0) {
#pragma unroll
        for (int mt = 0; mt < NMT; mt++) {
            const int r = 16 * mt + c16;
            const uint32_t negbits = r < M ? a.paley.neg[r] : 0u;
            bf16x8 h;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int c = 8 * g + j;
                float e = 0.0f;
                if (r < M && c < M) e = ((negbits >> c) & 1u) ? -1.0f : 1.0f;
                h[j] = (__bf16)e;
            }
            hat[mt][lane] = h;
        }
    }

    constexpr bool PAD = kron_rows<M>() > M;
    if constexpr (PAD) {
        for (int i = tid; i < (kron_rows<M>() - M) * (Q / 4); i += NT)
            reinterpret_cast<float4 *>(F + M * QS)[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }

    // Persistent over tokens t = blockIdx.x, + gridDim.x, ...; the next token's
    // x segment is requested before the current one is transformed.
    int64_t t = blockIdx.x;
    if (t >= a.T) return;
    const int s = row;
    uint4 xw[NH];
#pragma unroll
    for (int h = 0; h < NH; h++)
        xw[h] = *reinterpret_cast<const uint4 *>(a.x + t * a.ldx + s * Q + h * 128 + chunk * 8);
    for (; t < a.T; t += gridDim.x) {
    // ---- phase 1 (the arithmetic of rq_row_kernel): row `row` transforms segment `row`
    {
        float v[NV];
        unpack_x<NH>(v, xw);
        if constexpr (PERSIST) {
            const int64_t tn = t + gridDim.x < a.T ? t + gridDim.x : a.T - 1;
#pragma unroll
            for (int h = 0; h < NH; h++)
                xw[h] = *reinterpret_cast<const uint4 *>(a.x + tn * a.ldx + s * Q + h * 128 + chunk * 8);
        }
        if (a.signs) apply_signs<NH>(v, a.signs + s * Q + chunk * 8);
        fwht_lane_stages<NH>(v);
        if constexpr (NH == 1) {
            // Q = 128: one 8-value block per cross-lane stage, too few for the
            // fused DPP form below; plain butterflies and the checked division
            fwht_xlane_plain(v, sj);
            div_sqrt_q<Q>(v, a.sq, a.rsq);
        } else {
        // cross-lane stages as one v_fmac with a DPP source: v + s_j * partner.
        // The lower lane of each pair holds the sum, the upper lane the negated
        // difference, so after the four stages the lane holds sigma * (true
        // value) with sigma = s_0 s_1 s_2 s_3; fma with a +-1 multiplier rounds
        // exactly like the add or subtract, and RN is odd-symmetric, so every
        // nonzero value is bit-exact; sigma is folded into the division below.
        fwht_xlane_signed(v, sj);
        fwht_h_stages<NH>(v);
        // Only a zero (or a value below div_sqrt_q_min, where the division
        // shortcut is not exact) can differ: a zero's sign follows sigma instead of IEEE
        // x + (-x) = +0.  A wave holding one recomputes its rows with the plain
        // butterflies and the IEEE division (x is re-read).
        float amin = __builtin_fabsf(v[0]);
#pragma unroll
        for (int i = 1; i < NV; i++) amin = fminf(amin, __builtin_fabsf(v[i]));
        if (__builtin_expect(__any(amin < div_sqrt_q_min<Q>()), 0)) {
            uint4 xr[NH];
#pragma unroll
            for (int h = 0; h < NH; h++)
                xr[h] = *reinterpret_cast<const uint4 *>(a.x + t * a.ldx + s * Q + h * 128 + chunk * 8);
            unpack_x<NH>(v, xr);
            if (a.signs) apply_signs<NH>(v, a.signs + s * Q + chunk * 8);
            fwht_lane_stages<NH>(v);
            fwht_xlane_plain(v, sj);
            fwht_h_stages<NH>(v);
#pragma unroll
            for (int i = 0; i < NV; i++) v[i] = v[i] / a.sq;
        } else {
            div_sqrt_q_fast<Q>(v, sigma * a.sq, sigma * a.rsq);
        }
        }
#pragma unroll
        for (int h = 0; h < NH; h++) {
            float4 *d = reinterpret_cast<float4 *>(F + s * QS + ((h * 128 + chunk * 8) ^ fsw(s)));
            d[0] = make_float4(v[h * 8 + 0], v[h * 8 + 1], v[h * 8 + 2], v[h * 8 + 3]);
            d[1] = make_float4(v[h * 8 + 4], v[h * 8 + 5], v[h * 8 + 6], v[h * 8 + 7]);
        }
    }
    __syncthreads();

    // ---- phase 2: Paley product on MFMA, one 16-column block at a time, in place
    {
        bf16x8 ha[NMT];
#pragma unroll
        for (int mt = 0; mt < NMT; mt++) ha[mt] = hat[mt][lane];
        const float hm = a.hm;
        constexpr int CB = Q / 16;
        // one 16-column block: ridx(j) is the LDS index of row 8g + j of the
        // lane's column, widx(mt, i) that of row 16 mt + 4g + i
        auto paley_block = [&](auto ridx, auto widx) {
            float f[8];
#pragma unroll
            for (int j = 0; j < 8; j++) f[j] = (PAD || 8 * g + j < M) ? F[ridx(j)] : 0.0f;
            bf16x8 bh, bm, bl;
            split3x8_trunc(f, bh, bm, bl);
#pragma unroll
            for (int mt = 0; mt < NMT; mt++) {
                const floatx4 s1 = mfma_bf16(ha[mt], bh, zero4());
                floatx4 s2 = mfma_bf16(ha[mt], bm, zero4());
                s2 = mfma_bf16(ha[mt], bl, s2);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int ar = 16 * mt + 4 * g + i;
                    // padded rows get an exact +0, whatever the column held: an
                    // Inf or NaN of this token must not reach the next token's
                    // Paley stage through 0 * NaN
                    // An infinite F value splits into (Inf, NaN, NaN): s1 then
                    // carries the IEEE sum (+-Inf, or NaN for Inf - Inf) and s2 is
                    // NaN.  The median with +-FLT_MAX returns a NaN operand's
                    // minimum (-FLT_MAX), so a NaN s2 leaves hm * s1 alone;
                    // finite products pass unchanged.
                    const float s2c = __builtin_amdgcn_fmed3f(hm * s2[i], -0x1.fffffep+127f, 0x1.fffffep+127f);
                    const float p = __builtin_fmaf(hm, s1[i], s2c);
                    if (PAD) F[widx(mt, i)] = ar < M ? p : 0.0f;
                    else if (ar < M) F[widx(mt, i)] = p;
                }
            }
        };
        if constexpr (PAD) {
            // Column block cb of row r sits at r * QS + 16 (cb ^ (fsw(r) >> 4)) + c16.
            // The flip (fsw(r) >> 4) is (g ^ (j >> 2)) & 1 for the rows 8g + j
            // read and ((g >> 1) ^ g) & 1 for the rows 16 mt + 4g + i written, and
            // cb ^ f = cb + dlt(cb & 1, f) with dlt = 16 ((q ^ f) - q).  cb = wv +
            // NW it alternates parity with it, so per lane and parity of it the
            // offsets are fixed and every access is a base plus an immediate
            // (C3: 80 -> 69 VALU instructions per block and wave).  Unrolled only
            // for the padded blocks: at M = 12 the row guards made it slower.
            constexpr int ITER = (CB + NW - 1) / NW;
            static_assert(NW % 2 == 1, "block parity alternates with the iteration");
            auto dlt = [](int q, int f) { return 16 * ((q ^ f) - q); };
            const int wq = wv & 1;
            const int fr0 = g & 1, fr1 = fr0 ^ 1, fw = ((g >> 1) ^ g) & 1;
            const int rb = 8 * g * QS + 16 * wv + c16, wb = 4 * g * QS + 16 * wv + c16;
            const int rd0[2] = {rb + dlt(wq, fr0), rb + dlt(wq ^ 1, fr0)};   // rows 8g + 0..3
            const int rd1[2] = {rb + dlt(wq, fr1), rb + dlt(wq ^ 1, fr1)};   // rows 8g + 4..7
            const int wr[2] = {wb + dlt(wq, fw), wb + dlt(wq ^ 1, fw)};
#pragma unroll
            for (int it = 0; it < ITER; it++) {
                if (wv + NW * it >= CB) break;
                const int co = 16 * NW * it;
                paley_block([&](int j) { return (j < 4 ? rd0[it & 1] : rd1[it & 1]) + j * QS + co; },
                            [&](int mt, int i) { return wr[it & 1] + (16 * mt + i) * QS + co; });
            }
        } else {
            for (int cb = wv; cb < CB; cb += NW) {
                const int c = 16 * cb + c16;
                paley_block([&](int j) { return (8 * g + j) * QS + (c ^ fsw(8 * g + j)); },
                            [&](int mt, int i) {
                                const int ar = 16 * mt + 4 * g + i;
                                return ar * QS + (c ^ fsw(ar));
                            });
            }
        }
    }
    __syncthreads();

    // row-major float4 index i of the token's N floats -> its float4 in F
    const float4 *F4 = reinterpret_cast<const float4 *>(F);
    auto f4 = [](int i) {
        const int a = i / (Q / 4);
        return a * (QS / 4) + ((i % (Q / 4)) ^ (fsw(a) >> 2));
    };
    // row `row` copies segment row `row`: lane l16 moves float4 l16 + 16 j
    // (256 contiguous bytes per 16 lanes and instruction; the swizzle only flips
    // bit 2 of the float4 index, so every offset is a constant).  The rows are
    // written once and read once by the next kernel: non-temporal stores keep
    // them from evicting x (read by the projection just before) from the
    // Infinity Cache (C3 8192 x 14336: 367 -> 343 us per call).
    auto copy_row = [&](float *dst_row) {
        const float4 *src = F4 + row * (QS / 4) + (l16 ^ (fsw(row) >> 2));
        floatx4 *dst = reinterpret_cast<floatx4 *>(dst_row + row * Q) + l16;
#pragma unroll
        for (int j = 0; j < Q / 64; j++) {
            const float4 v = src[16 * j];
            __builtin_nontemporal_store(floatx4{v.x, v.y, v.z, v.w}, dst + 16 * j);
        }
    };
    if constexpr (!QUANT) {
        copy_row(a.P + t * N);
    } else {
        if (a.rotated) copy_row(a.rotated + t * N);
        constexpr int G8 = B / 8;
        constexpr int CHUNKS = N / 8;
        const int64_t orow = a.dest ? a.dest[t] : t;
        for (int c0 = 0; c0 < CHUNKS; c0 += NT) {
            const int ch = c0 + tid;
            const bool ok = ch < CHUNKS;
            const int chs = ok ? ch : 0;
            float v[8];
            {
                const float4 p0 = F4[f4(2 * chs)], p1 = F4[f4(2 * chs) + 1];
                v[0] = p0.x; v[1] = p0.y; v[2] = p0.z; v[3] = p0.w;
                v[4] = p1.x; v[5] = p1.y; v[6] = p1.z; v[7] = p1.w;
            }
                GroupParams gp;
            const uint32_t word = quant_group8<G8>(v, gp);
            if (ok) {
                if (a.deq)
                    store_tuple8(v, gp, word, a.codes + orow * N + ch * 8, a.deq + orow * N + ch * 8);
                else
                    *reinterpret_cast<uint32_t *>(a.codes + orow * (N / 2) + ch * 4) = word;
                if ((ch % G8) == 0) {
                    const int64_t gi = orow * (N / B) + (ch * 8) / B;
                    a.scales[gi] = gp.s16;
                    a.zeros[gi] = gp.z16;
                }
            }
        }
    }
    if constexpr (!PERSIST) break;
    __syncthreads();   // F is rewritten by the next token
    }
}

}  // namespace narhip
