// Segment kernel: Hadamard blocks of Q <= 1024 channels, each handled by one
// 16-lane row, fused with the rank-k term and the INT4 group quantizer.
//
// Covers the per-head paths (K/V cache: H_128 per head, per-head rank-k factors,
// groups of 32) and the block-Hadamard paths of nar/kernels (block-H_128,
// groups of 128, rank-k from a full-row projection given as split partials).
//
// Data layout in registers: segment position p = hi*128 + chunk(lane)*8 + e,
// e in [0,8) the element inside one 16-byte bf16 load, hi in [0, Q/128).
// Stages w = 1,2,4 are in-register, w = 8..64 are DPP exchanges inside the row,
// w = 128.. are in-register again -- the reference's stage order
// (nar/extended_experiment.py:443-456) is preserved exactly.
#pragma once
#include "narhip_device.hpp"

namespace narhip {

enum RankMode : int { RANK_NONE = 0, RANK_LOCAL = 1, RANK_PARTIAL = 2 };

struct SegArgs {
    const uint16_t *x;      // bf16 [T, ldx]
    int64_t ldx;
    int64_t T, n;           // tokens, channels per token
    const float *signs;     // [n] or null
    const float *v;         // [n, k] (RANK_LOCAL)
    const float *wt;        // [k, n]
    const float *partial;   // [T, splits*k] (RANK_PARTIAL)
    int splits;
    int k;
    uint8_t *codes;         // [rows_out, n/2], or unpacked [rows_out, n] when deq is set
    uint16_t *scales;       // [rows_out, n/B]
    uint16_t *zeros;
    const int64_t *dest;    // [T] output row per token, or null
    float *rotated;         // [T, n] or null
    float sq, rsq;          // fp32(sqrt(Q)) and RN(1/sq), computed on the host
    float *deq;             // fp32 [rows_out, n]: the hooks' tuple output (unpacked codes), or null
};

// F16IO: fp16 rows in, fp16 rows out (the E28 transform epilogue: no
// quantization; `rotated` then points to fp16 [T, n]), else bf16 in and INT4 out.
template <int Q, int B, int MODE, int KMAX, bool F16IO = false>
__global__ void __launch_bounds__(256)
rq_seg_kernel(SegArgs a)
{
    constexpr int NH = Q / 128;          // 128-position chunks per segment
    constexpr int NV = 8 * NH;           // values per lane
    constexpr int G8 = B / 8;            // lanes per quant group (4, 8, 16)
    const int lane = threadIdx.x & 63;
    const int l16 = lane & 15;
    const int row = threadIdx.x >> 4;    // one 16-lane row per segment
    const int rows = blockDim.x >> 4;
    // per-head rank: grid (token tiles, heads), so the rows of a wave are
    // consecutive tokens of one head and share its V and W rows (one set of
    // addresses per wave), and no 64-bit division is needed to place a row;
    // otherwise a 1-D grid over the token-major segments
    constexpr bool HEAD = MODE == RANK_LOCAL && NH == 1;
    int64_t t, base;                     // token; channel offset in the token
    bool active;
    if constexpr (HEAD) {
        const int64_t tr = (int64_t)blockIdx.x * rows + row;
        active = tr < a.T;
        t = active ? tr : 0;
        base = (int64_t)blockIdx.y * Q;
    } else {
        const int64_t segs_per_token = a.n / Q;
        const int64_t seg = (int64_t)blockIdx.x * rows + row;
        active = seg < a.T * segs_per_token;
        const int64_t sg = active ? seg : 0;
        t = sg / segs_per_token;
        base = (sg % segs_per_token) * Q;
    }
    const int chunk = lane_chunk(l16);

    // ---- load: NH x 16-byte bf16 loads per lane
    float v[NV];
    uint32_t raw[NV / 2];
    const uint16_t *xr = a.x + t * a.ldx + base;
#pragma unroll
    for (int h = 0; h < NH; h++) {
        uint4 w = *reinterpret_cast<const uint4 *>(xr + h * 128 + chunk * 8);
        raw[h * 4 + 0] = w.x; raw[h * 4 + 1] = w.y; raw[h * 4 + 2] = w.z; raw[h * 4 + 3] = w.w;
    }
#pragma unroll
    for (int i = 0; i < NV / 2; i++) {
        if constexpr (F16IO) {
            v[2 * i] = f16_bits_to_f32((uint16_t)(raw[i] & 0xffffu));
            v[2 * i + 1] = f16_bits_to_f32((uint16_t)(raw[i] >> 16));
        } else {
            v[2 * i] = bf16lo(raw[i]);
            v[2 * i + 1] = bf16hi(raw[i]);
        }
    }

    // ---- per-head rank (one 128-channel block per row): the V rows of the
    // lane's 8 channels, the W rows over them and the destination row are
    // requested together with x, so the row waits on memory once (the decode
    // and KV-cache shapes are latency-bound)
    float vh[HEAD ? 8 * KMAX : 1], wh[HEAD ? 8 * KMAX : 1];
    if constexpr (HEAD) {
        const int64_t c0 = base + chunk * 8;
        if (a.k == KMAX && (reinterpret_cast<uintptr_t>(a.v) & 15u) == 0) {
            const float4 *vr = reinterpret_cast<const float4 *>(a.v + c0 * KMAX);
#pragma unroll
            for (int q4 = 0; q4 < 2 * KMAX; q4++) {
                const float4 f = vr[q4];
                vh[4 * q4] = f.x; vh[4 * q4 + 1] = f.y; vh[4 * q4 + 2] = f.z; vh[4 * q4 + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++)
#pragma unroll
                for (int r = 0; r < KMAX; r++) vh[e * KMAX + r] = r < a.k ? a.v[(c0 + e) * a.k + r] : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < KMAX; r++) {
            const int rr = r < a.k ? r : 0;   // rows r >= k are loaded but never used
            const float4 *wr = reinterpret_cast<const float4 *>(a.wt + (int64_t)rr * a.n + c0);
            const float4 w0 = wr[0], w1 = wr[1];
            wh[r * 8 + 0] = w0.x; wh[r * 8 + 1] = w0.y; wh[r * 8 + 2] = w0.z; wh[r * 8 + 3] = w0.w;
            wh[r * 8 + 4] = w1.x; wh[r * 8 + 5] = w1.y; wh[r * 8 + 6] = w1.z; wh[r * 8 + 7] = w1.w;
        }
    }
    const int64_t orow = a.dest ? a.dest[t] : t;

    // ---- rank-k projection of the raw input (fp64, rounded once to fp32)
    float u[KMAX > 0 ? KMAX : 1];
    if constexpr (HEAD) {
        double acc[KMAX];
#pragma unroll
        for (int r = 0; r < KMAX; r++) acc[r] = 0.0;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const double xv = (double)v[e];
#pragma unroll
            for (int r = 0; r < KMAX; r++)
                if (r < a.k) acc[r] = fma(xv, (double)vh[e * KMAX + r], acc[r]);
        }
#pragma unroll
        for (int r = 0; r < KMAX; r++) u[r] = (float)row_sum64(acc[r]);
    } else if constexpr (MODE == RANK_LOCAL) {
        double acc[KMAX];
#pragma unroll
        for (int r = 0; r < KMAX; r++) acc[r] = 0.0;
#pragma unroll
        for (int h = 0; h < NH; h++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int64_t ch = base + h * 128 + chunk * 8 + e;
                const double xv = (double)v[h * 8 + e];
#pragma unroll
                for (int r = 0; r < KMAX; r++)
                    if (r < a.k) acc[r] = fma(xv, (double)a.v[ch * a.k + r], acc[r]);
            }
#pragma unroll
        for (int r = 0; r < KMAX; r++) u[r] = (float)row_sum64(acc[r]);
    } else if constexpr (MODE == RANK_PARTIAL) {
        const float *p = a.partial + t * (int64_t)a.splits * a.k;
#pragma unroll
        for (int r = 0; r < KMAX; r++) {
            double s = 0.0;
            if (r < a.k)
                for (int sp = 0; sp < a.splits; sp++) s += (double)p[sp * a.k + r];
            u[r] = (float)s;
        }
    }

    // ---- signs (Hadamard input only)
    if (a.signs) {
#pragma unroll
        for (int h = 0; h < NH; h++)
#pragma unroll
            for (int e = 0; e < 8; e++) v[h * 8 + e] *= a.signs[base + h * 128 + chunk * 8 + e];
    }

    // ---- FWHT_Q, then the normalisation: fp32 division by fp32(sqrt(Q))
    if constexpr (NH == 1) {
        fwht128_div(v, chunk, a.sq, a.rsq);
    } else {
        fwht_row<NH>(v, chunk);
        div_sqrt_q<Q>(v, a.sq, a.rsq);
    }

    // ---- rank-k correction: x' = Hx - RN32(sum_r u_r W[r, i])
    if constexpr (HEAD) {
        double acc[8];
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] = 0.0;
#pragma unroll
        for (int r = 0; r < KMAX; r++) {
            if (r < a.k) {
                const double ur = (double)u[r];
#pragma unroll
                for (int e = 0; e < 8; e++) acc[e] = fma(ur, (double)wh[r * 8 + e], acc[e]);
            }
        }
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = v[e] - (float)acc[e];
    } else if constexpr (MODE != RANK_NONE) {
        // per channel: fp64 sum over r in order, rounded once; W rows read as float4
#pragma unroll
        for (int h = 0; h < NH; h++) {
            double acc[8];
#pragma unroll
            for (int e = 0; e < 8; e++) acc[e] = 0.0;
#pragma unroll
            for (int r = 0; r < KMAX; r++) {
                if (r < a.k) {
                    const float4 *wr =
                        reinterpret_cast<const float4 *>(a.wt + (int64_t)r * a.n + base + h * 128 + chunk * 8);
                    const float4 w0 = wr[0], w1 = wr[1];
                    const double ur = (double)u[r];
                    acc[0] = fma(ur, (double)w0.x, acc[0]); acc[1] = fma(ur, (double)w0.y, acc[1]);
                    acc[2] = fma(ur, (double)w0.z, acc[2]); acc[3] = fma(ur, (double)w0.w, acc[3]);
                    acc[4] = fma(ur, (double)w1.x, acc[4]); acc[5] = fma(ur, (double)w1.y, acc[5]);
                    acc[6] = fma(ur, (double)w1.z, acc[6]); acc[7] = fma(ur, (double)w1.w, acc[7]);
                }
            }
#pragma unroll
            for (int e = 0; e < 8; e++) v[h * 8 + e] = v[h * 8 + e] - (float)acc[e];
        }
    }

    if constexpr (F16IO) {
        if (active) {
            uint16_t *o = reinterpret_cast<uint16_t *>(a.rotated) + t * a.n + base;
#pragma unroll
            for (int h = 0; h < NH; h++) {
                uint32_t w[4];
#pragma unroll
                for (int j = 0; j < 4; j++)
                    w[j] = (uint32_t)f32_to_f16_bits(v[h * 8 + 2 * j]) |
                           ((uint32_t)f32_to_f16_bits(v[h * 8 + 2 * j + 1]) << 16);
                *reinterpret_cast<uint4 *>(o + h * 128 + chunk * 8) = make_uint4(w[0], w[1], w[2], w[3]);
            }
        }
        return;
    }
    if (a.rotated && active) {
        float *o = a.rotated + t * a.n + base;
#pragma unroll
        for (int h = 0; h < NH; h++) {
            float4 *d = reinterpret_cast<float4 *>(o + h * 128 + chunk * 8);
            d[0] = make_float4(v[h * 8 + 0], v[h * 8 + 1], v[h * 8 + 2], v[h * 8 + 3]);
            d[1] = make_float4(v[h * 8 + 4], v[h * 8 + 5], v[h * 8 + 6], v[h * 8 + 7]);
        }
    }

    // ---- quantize groups of B and store (codes == null: rotation only, into
    // `rotated`; deq set: the hooks' tuple, codes unpacked)
    if (!a.codes) return;
    const int64_t gpt = a.n / B;   // groups per token
#pragma unroll
    for (int h = 0; h < NH; h++) {
        GroupParams g;
        const uint32_t word = quant_group8<G8>(v + h * 8, g);
        if (active) {
            const int64_t pos = base + h * 128 + chunk * 8;
            if (a.deq)
                store_tuple8(v + h * 8, g, word, a.codes + orow * a.n + pos, a.deq + orow * a.n + pos);
            else
                *reinterpret_cast<uint32_t *>(a.codes + orow * (a.n / 2) + pos / 2) = word;
            if ((chunk & (G8 - 1)) == 0) {
                const int64_t gi = orow * gpt + pos / B;
                a.scales[gi] = g.s16;
                a.zeros[gi] = g.z16;
            }
        }
    }
}

}  // namespace narhip
