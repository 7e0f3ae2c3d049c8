// Block-H_128 rows with a full-row rank term of k <= 8:
//   E28's fp16 down_proj transform (quarot-llama3/nar_r4_kernel.py
//   NARDownTransform): out = fp16( H_128 blocks(x) / fp32(sqrt 128) - RN32(u W^T) ),
//   u = RN32(x V), from fp16 rows;
//   E17's block-H_128 rotate-and-quantize (nar/kernels/r4_fused_v3.py launch_nar
//   at k = 8): the same x' from bf16 rows, then the group-128 INT4 quantizer
//   (each 128-channel segment is one group).
//
// Two streaming passes over x, each organised so that the factor it needs
// stays on chip for many tokens instead of being re-read per token:
//
//   proj_tok_kernel   two tokens per lane (128 tokens per block), the
//                     block's channel chunk streamed through LDS in 64-channel
//                     tiles of x and of V (converted to fp64 as it is staged;
//                     double-buffered, one barrier per tile); each V row is
//                     read by a whole wave at one address (LDS broadcast) and
//                     used for both tokens of every lane.  fp64 FMAs; fp64
//                     sums per channel chunk, or, with one chunk, u = RN32(sum)
//                     itself.
//   xform128_kernel   one 16-lane row per 128-channel segment, 16 segments per
//                     block; each lane keeps W^T for its 8 channels in
//                     registers as fp64 and loops over a range of tokens (x
//                     prefetched XF_PF tokens ahead).  u comes by scalar loads:
//                     as stored, or RN32 of the chunk sums (or of the caller's
//                     fp32 partials) added in chunk order.  The
//                     butterflies (fwht128_div), the division and the fp64
//                     correction sum are those of the segment kernel, so the
//                     fp32 values equal its; then fp16 out, or (QUANT) the
//                     group-128 INT4 quantizer.
#pragma once
#include "narhip_device.hpp"

namespace narhip {

constexpr int XF_K = 8;             // rank slots held by the kernels below

struct ProjTokArgs {
    const uint16_t *x;        // fp16 (or bf16) rows [T, ldx]
    int64_t ldx, T, n;
    const float *v;           // V [n, k]
    double *pd;               // [T][S][XF_K] fp64 chunk sums (S == 1: RN32 of the sum), or null
    float *pf;                // [T][S*k] fp32 chunk sums (each rounded once), or null
    int k, S;                 // chunk = n / S channels, a multiple of 128
    bool v4;                  // k % 4 == 0 and v 16-byte aligned: V rows by float4 loads
};

// proj_tok tiles: TL tokens per lane (64 TL tokens per block), TC channels per
// LDS tile, TC / 4 per wave.  Each V row read from LDS (one broadcast address
// per wave) feeds 8 TL fp64 FMAs.  The launcher uses TL = PT_TL = 2 (the LDS
// return of the broadcast V rows bounded TL = 1: E17 8B k = 8, 2048 tokens,
// 79.3 -> 73.7 us per call; E28 8B, 32768 tokens, 855 -> 790 us).
constexpr int PT_TL = 2;
template <int TL> struct PtShape {
    static constexpr int TC = TL == 1 ? 128 : 64;      // channels per tile
    static constexpr int ROWB = TC * 2 + 16;           // padded x row: conflict-free b128 column reads
    static constexpr int XB = 64 * TL * ROWB;          // x tile bytes
    static constexpr int VB = TC * XF_K * 8;           // V tile bytes (fp64)
    static constexpr int BUF = XB + VB;
    static constexpr int PR = TC / 8;                  // 16-byte pieces per x row
    static constexpr int XPT = 64 * TL * PR / 256;     // x pieces per thread per tile
    static constexpr int VPT = TC * XF_K / 256;        // V elements per thread per tile
    static constexpr int CW = TC / 4;                  // channels per wave per tile
    static_assert(XPT == 4 && VPT * 256 == TC * XF_K && (VPT == 2 || VPT == 4), "tile split");
    static_assert(2 * BUF >= 4 * 64 * TL * XF_K * 8, "the cross-wave sums reuse the tile buffers");
};

template <bool F16, int TL>
__global__ void __launch_bounds__(256, 3)
proj_tok_kernel(ProjTokArgs a)
{
    using S = PtShape<TL>;
    __shared__ __align__(16) uint8_t lds[2 * S::BUF];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = tid >> 6;
    const int64_t t0 = (int64_t)blockIdx.x * 64 * TL;
    const int64_t chunk = a.n / a.S;
    const int64_t c0 = (int64_t)blockIdx.y * chunk;
    const int ntiles = (int)(chunk / S::TC);

    // loader: x -- piece i of the thread is linear piece i * 256 + tid of the
    //         tile (PR 16-byte pieces per row): every load instruction covers
    //         whole rows of the tile;
    //         V -- thread -> tile elements VPT tid .. of [TC channels][XF_K ranks]
    //         (rank slots >= k are 0), stored as fp64
    // (piece i of the thread is row tid / PR + i * 256 / PR, the same column)
    const int xr0 = tid / S::PR, xpc = tid % S::PR;
    constexpr int XRS = 256 / S::PR;               // rows between the thread's pieces
    auto xrow = [&](int i) __attribute__((always_inline)) {
        const int64_t r = t0 + xr0 + i * XRS;
        return reinterpret_cast<const uint4 *>(a.x + (r < a.T ? r : a.T - 1) * a.ldx + c0) + xpc;
    };
    const uint4 *xs0 = xrow(0), *xs1 = xrow(1), *xs2 = xrow(2), *xs3 = xrow(3);
    const int xoff = xr0 * S::ROWB + xpc * 16;
    const int vc = (S::VPT * tid) / XF_K, vr = (S::VPT * tid) % XF_K;    // channel in the tile, first rank slot
    const float *vsrc = a.v + (c0 + vc) * a.k;
    const int voff = S::XB + 8 * S::VPT * tid;
    float vf[S::VPT];
    uint4 x0, x1, x2, x3;
    // branch-free: out-of-rank slots load a valid element and are replaced by 0
    auto load_tile = [&](int tile) __attribute__((always_inline)) {
        const int xo = tile * (S::TC / 8);
        x0 = xs0[xo]; x1 = xs1[xo]; x2 = xs2[xo]; x3 = xs3[xo];
        const float *vt = vsrc + (int64_t)tile * S::TC * a.k;
        bool done = false;
        if constexpr (S::VPT == 4) {
            if (a.v4) {
                const float4 f = *reinterpret_cast<const float4 *>(vt + (vr < a.k ? vr : 0));
                const bool ok = vr < a.k;
                vf[0] = ok ? f.x : 0.0f; vf[1] = ok ? f.y : 0.0f; vf[2] = ok ? f.z : 0.0f; vf[3] = ok ? f.w : 0.0f;
                done = true;
            }
        }
        if (!done) {
#pragma unroll
            for (int j = 0; j < S::VPT; j++) {
                const float f = vt[vr + j < a.k ? vr + j : 0];
                vf[j] = vr + j < a.k ? f : 0.0f;
            }
        }
    };
    auto store_tile = [&](uint8_t *buf) __attribute__((always_inline)) {
        *reinterpret_cast<uint4 *>(buf + xoff) = x0;
        *reinterpret_cast<uint4 *>(buf + xoff + XRS * S::ROWB) = x1;
        *reinterpret_cast<uint4 *>(buf + xoff + 2 * XRS * S::ROWB) = x2;
        *reinterpret_cast<uint4 *>(buf + xoff + 3 * XRS * S::ROWB) = x3;
        double2 *dv = reinterpret_cast<double2 *>(buf + voff);
#pragma unroll
        for (int j = 0; j < S::VPT / 2; j++) dv[j] = make_double2((double)vf[2 * j], (double)vf[2 * j + 1]);
    };
    load_tile(0);
    store_tile(lds);
    __syncthreads();

    double acc[TL][XF_K];
#pragma unroll
    for (int i = 0; i < TL; i++)
#pragma unroll
        for (int r = 0; r < XF_K; r++) acc[i][r] = 0.0;
    // the wave's CW channels of each tile: x by lane = token (TL rows), V rows broadcast
    const int xme = lane * S::ROWB + w * S::CW * 2;
    const int vme = S::XB + w * S::CW * XF_K * 8;
    constexpr int WPR = S::CW / 2;                 // x words (two channels) per row

    for (int tile = 0; tile < ntiles; tile++) {
        const uint8_t *buf = lds + (tile & 1) * S::BUF;
        // next tile's x and V into registers (the last tile reloads itself), then
        // into the other buffer after this tile's FMAs: no branches, so the
        // loads, the FMAs and the stores stay in one schedule region
        load_tile(tile + 1 < ntiles ? tile + 1 : tile);
        uint32_t wd[TL][WPR];
#pragma unroll
        for (int i = 0; i < TL; i++) {
            const uint4 *row = reinterpret_cast<const uint4 *>(buf + xme + i * 64 * S::ROWB);
#pragma unroll
            for (int q = 0; q < WPR / 4; q++) {
                const uint4 p = row[q];
                wd[i][4 * q] = p.x; wd[i][4 * q + 1] = p.y; wd[i][4 * q + 2] = p.z; wd[i][4 * q + 3] = p.w;
            }
        }
        const double2 *vt = reinterpret_cast<const double2 *>(buf + vme);
        // V rows two channels ahead of the FMAs; the fences keep the compiler
        // from hoisting all the row reads of the tile into registers
        double2 va[XF_K / 2], vb[XF_K / 2];
#pragma unroll
        for (int r2 = 0; r2 < XF_K / 2; r2++) {
            va[r2] = vt[r2];
            vb[r2] = vt[XF_K / 2 + r2];
        }
#pragma unroll
        for (int c = 0; c < S::CW; c++) {
            double2 vc[XF_K / 2];
#pragma unroll
            for (int r2 = 0; r2 < XF_K / 2; r2++) {
                vc[r2] = va[r2];
                va[r2] = vb[r2];
            }
            if (c + 2 < S::CW) {
#pragma unroll
                for (int r2 = 0; r2 < XF_K / 2; r2++) vb[r2] = vt[(c + 2) * (XF_K / 2) + r2];
            }
#pragma unroll
            for (int i = 0; i < TL; i++) {
                double xv;
                const uint32_t h = (c & 1) ? (wd[i][c >> 1] >> 16) : (wd[i][c >> 1] & 0xffffu);
                if constexpr (F16) xv = (double)f16_bits_to_f32((uint16_t)h);
                else xv = (double)__uint_as_float(h << 16);
#pragma unroll
                for (int r2 = 0; r2 < XF_K / 2; r2++) {
                    acc[i][2 * r2] = fma(xv, vc[r2].x, acc[i][2 * r2]);
                    acc[i][2 * r2 + 1] = fma(xv, vc[r2].y, acc[i][2 * r2 + 1]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        store_tile(lds + ((tile + 1) & 1) * S::BUF);
        __syncthreads();
    }

    // combine the four waves' channel quarters in wave order
    double *red = reinterpret_cast<double *>(lds);     // [4][64 TL][XF_K]
#pragma unroll
    for (int i = 0; i < TL; i++)
#pragma unroll
        for (int r = 0; r < XF_K; r++) red[(w * 64 * TL + i * 64 + lane) * XF_K + r] = acc[i][r];
    __syncthreads();
    if (tid < 64 * TL) {
        const int64_t t = t0 + tid;
        if (t < a.T) {
#pragma unroll
            for (int r = 0; r < XF_K; r++) {
                double s = red[tid * XF_K + r];
                s += red[(64 * TL + tid) * XF_K + r];
                s += red[(2 * 64 * TL + tid) * XF_K + r];
                s += red[(3 * 64 * TL + tid) * XF_K + r];
                if (a.pd) a.pd[(t * a.S + blockIdx.y) * XF_K + r] = a.S == 1 ? (double)(float)s : s;
                else if (r < a.k) a.pf[(t * a.S + blockIdx.y) * a.k + r] = (float)s;
            }
        }
    }
}

struct XformArgs {
    const uint16_t *x;        // fp16 rows [T, ldx] (QUANT: bf16)
    int64_t ldx, T, n;
    const float *wt;          // [k, n]
    const double *pd;         // u: proj_tok's [T][S][XF_K] (S == 1: already RN32), or null
    const float *pf;          // u: caller's fp32 partials [T][S*k] (used when pd is null)
    int S;
    uint16_t *out;            // fp16 [T, n] (transform form)
    int k;
    int tpb;                  // tokens per block (blockIdx.y-th range)
    float sq, rsq;            // fp32(sqrt 128), RN(1/sq)
    // QUANT form: groups of 128 = one segment
    const float *signs;       // [n] or null (applied to x before the transform)
    uint8_t *codes;           // [rows, n/2]
    uint16_t *scales, *zeros; // [rows, n/128]
    const int64_t *dest;      // [T] output row per token, or null
};

__device__ __forceinline__ void f16x8_to_f32(const uint4 p, float (&v)[8])
{
    const uint32_t wd[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        v[2 * j] = f16_bits_to_f32((uint16_t)(wd[j] & 0xffffu));
        v[2 * j + 1] = f16_bits_to_f32((uint16_t)(wd[j] >> 16));
    }
}

constexpr int XF_PF = 8;            // x prefetch depth of xform128 (tokens)

constexpr int XF_UW = 32;           // tokens per u window (one fold pass of the block)
static_assert(XF_UW * XF_K == 256 && XF_UW % XF_PF == 0, "u window: one (token, rank) per thread");

// u[t][r] as the fp64 value of an fp32 number: RN32 of the chunk sums added in
// chunk order (proj_tok's fp64 sums, already rounded when there is one chunk,
// or the caller's fp32 partials).  Ranks >= k: 0.
__device__ __forceinline__ double fold_u(const XformArgs &a, int64_t t, int r)
{
    if (r >= a.k) return 0.0;
    double s = 0.0;
    if (a.pd) {
        const double *p = a.pd + t * a.S * XF_K + r;
        if (a.S == 1) return p[0];
        int c = 0;
        for (; c + 16 <= a.S; c += 16) {      // sixteen loads in flight, added in order
            double v[16];
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = p[(c + j) * XF_K];
#pragma unroll
            for (int j = 0; j < 16; j++) s += v[j];
        }
        for (; c < a.S; c++) s += p[c * XF_K];
    } else {
        const float *p = a.pf + t * a.S * a.k + r;
        for (int c = 0; c < a.S; c++) s += (double)p[c * a.k];
    }
    return (double)(float)s;
}

template <bool QUANT>
__device__ __forceinline__ void xform_token(const XformArgs &a, const double (&W)[XF_K][8], const float (&sg)[8],
                                            const double *ut, uint4 x, int64_t t, int64_t ch, int chunk,
                                            bool active)
{
    float v[8];
    if constexpr (QUANT) {
        v[0] = bf16lo(x.x); v[1] = bf16hi(x.x); v[2] = bf16lo(x.y); v[3] = bf16hi(x.y);
        v[4] = bf16lo(x.z); v[5] = bf16hi(x.z); v[6] = bf16lo(x.w); v[7] = bf16hi(x.w);
        if (a.signs) {
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] *= sg[e];
        }
    } else {
        f16x8_to_f32(x, v);
    }
    fwht128_div(v, chunk, a.sq, a.rsq);
    double u[XF_K];
    {
        const double2 *u2 = reinterpret_cast<const double2 *>(ut);     // one LDS address per wave
#pragma unroll
        for (int r = 0; r < XF_K / 2; r++) {
            const double2 d = u2[r];
            u[2 * r] = d.x; u[2 * r + 1] = d.y;
        }
    }
    double acc[8];
#pragma unroll
    for (int e = 0; e < 8; e++) acc[e] = 0.0;
#pragma unroll
    for (int r = 0; r < XF_K; r++) {
        if (r < a.k) {
            const double ur = u[r];
#pragma unroll
            for (int e = 0; e < 8; e++) acc[e] = fma(ur, W[r][e], acc[e]);
        }
    }
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = v[e] - (float)acc[e];
    if constexpr (QUANT) {
        // the segment is one group of 128: min/max over the row, then the codes
        GroupParams g;
        const uint32_t word = quant_group8<16>(v, g);
        if (active) {
            const int64_t orow = a.dest ? a.dest[t] : t;
            *reinterpret_cast<uint32_t *>(a.codes + orow * (a.n / 2) + ch / 2) = word;
            if (chunk == 0) {
                a.scales[orow * (a.n / 128) + ch / 128] = g.s16;
                a.zeros[orow * (a.n / 128) + ch / 128] = g.z16;
            }
        }
    } else {
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; j++)
            o[j] = (uint32_t)f32_to_f16_bits(v[2 * j]) | ((uint32_t)f32_to_f16_bits(v[2 * j + 1]) << 16);
        if (active) *reinterpret_cast<uint4 *>(a.out + t * a.n + ch) = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

template <bool QUANT>
__global__ void __launch_bounds__(256)
xform128_kernel(XformArgs a)
{
    const int lane = threadIdx.x & 63;
    const int l16 = lane & 15;
    const int row = threadIdx.x >> 4;
    const int64_t nseg = a.n / 128;
    const int64_t seg = (int64_t)blockIdx.x * 16 + row;
    const bool active = seg < nseg;
    const int chunk = lane_chunk(l16);
    const int64_t ch = (active ? seg : 0) * 128 + chunk * 8;

    // W^T for the lane's 8 channels, fp64
    double W[XF_K][8];
#pragma unroll
    for (int r = 0; r < XF_K; r++) {
        if (r < a.k) {
            const float4 *wr = reinterpret_cast<const float4 *>(a.wt + (int64_t)r * a.n + ch);
            const float4 w0 = wr[0], w1 = wr[1];
            W[r][0] = w0.x; W[r][1] = w0.y; W[r][2] = w0.z; W[r][3] = w0.w;
            W[r][4] = w1.x; W[r][5] = w1.y; W[r][6] = w1.z; W[r][7] = w1.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) W[r][e] = 0.0;
        }
    }

    float sg[8];
#pragma unroll
    for (int e = 0; e < 8; e++) sg[e] = 1.0f;
    if (QUANT && a.signs) {
        const float4 *sp = reinterpret_cast<const float4 *>(a.signs + ch);
        const float4 s0 = sp[0], s1 = sp[1];
        sg[0] = s0.x; sg[1] = s0.y; sg[2] = s0.z; sg[3] = s0.w;
        sg[4] = s1.x; sg[5] = s1.y; sg[6] = s1.z; sg[7] = s1.w;
    }

    __shared__ double ubuf[2][XF_UW][XF_K];
    const int64_t tb = (int64_t)blockIdx.y * a.tpb;
    const int64_t te = tb + a.tpb < a.T ? tb + a.tpb : a.T;
    if (tb >= te) return;
    const uint16_t *xc = a.x + ch;
    // x rows XF_PF tokens ahead of the arithmetic (loads past te repeat row te-1)
    uint4 ring[XF_PF];
#pragma unroll
    for (int i = 0; i < XF_PF; i++) {
        const int64_t tl = tb + i < te ? tb + i : te - 1;
        ring[i] = *reinterpret_cast<const uint4 *>(xc + tl * a.ldx);
    }
    // windows of XF_UW tokens: the block folds their u into LDS (thread ->
    // token, rank), then every row reads them; two buffers, one barrier each
    for (int64_t w0 = tb, wi = 0; w0 < te; w0 += XF_UW, wi++) {
        double (*ub)[XF_K] = ubuf[wi & 1];
        {
            const int i = threadIdx.x / XF_K, r = threadIdx.x % XF_K;
            ub[i][r] = w0 + i < te ? fold_u(a, w0 + i, r) : 0.0;
        }
        __syncthreads();
        const int64_t we = w0 + XF_UW < te ? w0 + XF_UW : te;
        for (int64_t t0 = w0; t0 < we; t0 += XF_PF) {
#pragma unroll
            for (int i = 0; i < XF_PF; i++) {
                const int64_t t = t0 + i;
                const uint4 cur = ring[i];
                const int64_t tl = t + XF_PF < te ? t + XF_PF : te - 1;
                ring[i] = *reinterpret_cast<const uint4 *>(xc + tl * a.ldx);
                if (t < we) xform_token<QUANT>(a, W, sg, ub[t - w0], cur, t, ch, chunk, active);
            }
        }
    }
}

}  // namespace narhip
