// Rank-k correction and INT4 quantizer on bf16 MFMA: x' = P - u W''^T, then
// dynamic asymmetric INT4 over groups of B channels (nar/experiment.py:158-184;
// the correction of nar/kernels/r4_fused_v3.py:224-230 in the row form
// x' = H x - (x Y') W''^T of quarot-llama3/nar_r4_kernel.py:190-202).
//
// A workgroup (4 waves) owns one block of 128 channels and a range of 16-token
// tiles; every wave walks its own tiles with the next tile's P and u requested
// before the current tile is computed (two register buffers), so each wave
// keeps 8 KB of P in flight while its MFMAs and quantizer run.
//
// MFMA mapping (v_mfma_f32_16x16x32_bf16, M = channels, N = tokens, K = ranks):
// M tile mt is channels 16 mt .. 16 mt + 15 of the block, so lane l (token
// l % 16, g = l / 16) holds channels 16 mt + 4g .. +3 of every M tile: each P
// load instruction reads 64 contiguous bytes per token (16 cache-line halves
// per instruction, the L1 tag rate the kernel is bound by otherwise).  A
// quantization group of B channels is B/16 M tiles of the four lanes of a
// token.  The lanes' packed codes are transposed across the four row groups
// (v_permlane32_swap, v_permlane16_swap) so that each lane stores 16
// contiguous bytes.
//
// C = u W''^T with u and W''^T as three exact bf16 terms each (hi, mid, lo):
// the five cross products of weight >= 2^-16 accumulate first, then the hi*hi
// products are added on top by the last MFMA of each K step, and
// x' = P - C is one fp32 subtraction.
#pragma once
#include "mfma.hpp"
#include "narhip_device.hpp"

namespace narhip {

struct CorrQuantArgs {
    const float *P;        // [T, n] rotated rows before the rank term
    int64_t T, n;
    const __bf16 *u3;      // [T][3][kp] terms of u
    const __bf16 *wtt;     // [3][n][kp] terms of W''^T
    int kp;                // 32 KS
    uint8_t *codes;        // [rows, n/2]
    uint16_t *scales;      // [rows, n/B]
    uint16_t *zeros;
    const int64_t *dest;   // token -> output row (null: identity)
    float *rotated;        // x' [T, n] (kernel variant ROT only)
    uint8_t *dummy;        // >= CQ_DUMMY_BYTES scratch: stores of lanes that have nothing to store
    int64_t ncb;           // n / 128 channel blocks
    int64_t tpg;           // 16-token tiles per workgroup (4 TPW)
};

constexpr int CQ_CB = 128;         // channels per workgroup block
constexpr int CQ_MT = CQ_CB / 16;  // M tiles per block
constexpr int CQ_DUMMY_BYTES = 1024;

// One tile's operands in registers: P for the lane's 32 channels, u terms and
// the output row of the lane's token.
template <int KS>
struct CqTile {
    float4 p[CQ_MT];
    bf16x8 u[3][KS];
    int64_t row;
};

// Every load is unconditional (tokens past the end re-read the last row; the
// dest load reads u3 when there is no dest table) so that the compiler's wait
// counts stay exact and a wait for this tile never waits for the next one.
template <int KS>
__device__ __forceinline__ void cq_load(CqTile<KS> &d, const CorrQuantArgs &a, int64_t t0, int64_t cbeg, int c16,
                                        int g)
{
    int64_t t = t0 + c16;
    if (t >= a.T) t = a.T - 1;
    const float4 *prow = reinterpret_cast<const float4 *>(a.P + t * a.n + cbeg + 4 * g);
#pragma unroll
    for (int mt = 0; mt < CQ_MT; mt++) d.p[mt] = prow[4 * mt];
    const __bf16 *urow = a.u3 + t * 3 * (int64_t)(32 * KS) + 8 * g;
#pragma unroll
    for (int term = 0; term < 3; term++)
#pragma unroll
        for (int ks = 0; ks < KS; ks++) d.u[term][ks] = load_bf16x8(urow + term * 32 * KS + 32 * ks);
    const int64_t *dp = a.dest ? a.dest + t : reinterpret_cast<const int64_t *>(a.u3);
    const int64_t r = *dp;
    d.row = a.dest ? r : t;
}

// The value of lane l ^ 16 / l ^ 32 through the gfx950 row swaps (no LDS
// round trip): permlane16_swap(v, v) puts row r ^ 1's value in row r of one
// of its two results, permlane32_swap(v, v) row r ^ 2's.
__device__ __forceinline__ float xor16(float v, int g)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((g & 1) ? r[0] : r[1]);
}
__device__ __forceinline__ float xor32(float v, int g)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((g & 2) ? r[0] : r[1]);
}

// Min/max over the four lanes of a token (rows g = 0..3 of the wave).
template <bool NAN_PROP>
__device__ __forceinline__ void cq_lanes_reduce(float &lo, float &hi, int g)
{
    float lo2 = xor16(lo, g), hi2 = xor16(hi, g);
    lo = NAN_PROP ? min_nan(lo, lo2) : fminf(lo, lo2);
    hi = NAN_PROP ? max_nan(hi, hi2) : fmaxf(hi, hi2);
    lo2 = xor32(lo, g); hi2 = xor32(hi, g);
    lo = NAN_PROP ? min_nan(lo, lo2) : fminf(lo, lo2);
    hi = NAN_PROP ? max_nan(hi, hi2) : fmaxf(hi, hi2);
}

// w[q] of the lane in row group g -> word q' of the lane in row group q' is
// the old w[q'] of row group ... : out[r] at row group q = in[q] at row group r
// (a 4 x 4 transpose between the row-group index and the register index).
__device__ __forceinline__ void cq_transpose4(uint32_t (&w)[4])
{
    auto s02 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
    auto s13 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
    auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
    auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
    w[0] = s01[0]; w[1] = s01[1]; w[2] = s23[0]; w[3] = s23[1];
}

// Eight codes c0..c7 (integral floats in [0, 15]) -> one word, nibble e = code e.
__device__ __forceinline__ uint32_t pack8(const float (&c)[8])
{
    uint32_t ev = 0, od = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        ev = __builtin_amdgcn_cvt_pk_u8_f32(c[2 * j], j, ev);
        od = __builtin_amdgcn_cvt_pk_u8_f32(c[2 * j + 1], j, od);
    }
    return ev | (od << 4);
}

// grid: 8 * ncb * ceil(token groups / 8) workgroups of 256 threads.  Workgroup
// b takes token group 8 (b / (8 ncb)) + b % 8 and channel block (b / 8) % ncb:
// the dispatcher places workgroup b on XCD b % 8, so all channel blocks of a
// token group share one XCD (its L2 merges their 2-byte scale and zero stores
// and holds the group's u terms).
// TPW tiles per wave, unrolled: the whole walk is straight-line code, so the
// compiler's wait counts are exact and the wait for tile j never waits for the
// request of tile j + 1.  Register use (gfx950 build): TPW = 1 118-128 VGPRs
// at k <= 32 and 162-174 at k <= 64, TPW = 4 and 8 234-256 (two waves per
// SIMD; measured faster on the large shapes than more waves with shorter
// walks).
template <int B, int KS, bool ROT, int TPW>
__global__ void __launch_bounds__(256, 2)
corr_quant_kernel(CorrQuantArgs a)
{
    constexpr int NG = CQ_CB / B;                  // quantization groups per block
    constexpr int MPG = B / 16;                    // M tiles per group
    __shared__ __align__(16) bf16x8 wl[3][KS][CQ_MT][64];   // W''^T fragments, lane order
    const int tid = threadIdx.x;
    const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, c16 = lane & 15;
    const int64_t cb = ((int64_t)blockIdx.x / 8) % a.ncb;
    const int64_t tg = ((int64_t)blockIdx.x / (8 * a.ncb)) * 8 + blockIdx.x % 8;
    const int64_t tile0 = tg * a.tpg;
    if (tile0 * 16 >= a.T) return;
    const int64_t cbeg = cb * CQ_CB;

    // stage the block's W''^T terms in fragment order: piece (term, ks, mt, l)
    // is channel 16 mt + l % 16 of the block, ranks 32 ks + 8 (l/16) ..
    {
        const int64_t plane = (int64_t)a.kp * a.n;
        constexpr int PIECES = 3 * KS * CQ_MT * 64;
        for (int p = tid; p < PIECES; p += 256) {
            const int l = p & 63, mt = (p >> 6) % CQ_MT, ks = (p >> 6) / CQ_MT % KS, term = (p >> 6) / CQ_MT / KS;
            const int64_t ch = cbeg + 16 * mt + (l & 15);
            wl[term][ks][mt][l] = load_bf16x8(a.wtt + term * plane + ch * a.kp + 32 * ks + 8 * (l >> 4));
        }
    }
    __syncthreads();

    // this wave's tiles: tile0 + w + 4 j (j < TPW); past the last tile of the
    // workgroup a wave repeats the last one (identical values, written again)
    const int64_t tiles = (a.T + 15) / 16;
    const int64_t tile_end = tile0 + 4 * TPW < tiles ? tile0 + 4 * TPW : tiles;
    const int64_t my0 = tile0 + w;
    const int64_t mylast = my0 < tile_end ? my0 + 4 * ((tile_end - 1 - my0) / 4) : tile_end - 1;
    auto tile_of = [&](int j) {
        const int64_t t = my0 + 4 * (int64_t)j;
        return (t < mylast ? t : mylast) * 16;
    };
    // stage A of a tile: x' = P - u W''^T (MFMA) into xv
    auto stage_a = [&](const CqTile<KS> &cur, float (&xv)[CQ_MT][4]) {
        // x' = P - u W''^T.  The fragment base is laundered per tile so that
        // the W''^T reads are not shared between tiles (shared, they would pin
        // 12 KS x 8 VGPRs for the whole walk).
        // (Only the integer offset is laundered: the reads keep their LDS
        // address space, so they stay ds_read and need no vector-memory wait.)
        uint32_t fo = lane;
        asm volatile("" : "+v"(fo));
        auto frag = [&](int term, int ks, int mt) { return (&wl[term][ks][mt][0])[fo]; };
        // term-major: the 8 M tiles' accumulators are independent chains, so
        // consecutive MFMAs never wait on each other; the five cross products
        // first, the hi*hi products last
        floatx4 acc[CQ_MT];
#pragma unroll
        for (int mt = 0; mt < CQ_MT; mt++) acc[mt] = zero4();
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
#pragma unroll
            for (int mt = 0; mt < CQ_MT; mt++) {
                const bf16x8 wm = frag(1, ks, mt);
                acc[mt] = mfma_bf16(wm, cur.u[0][ks], acc[mt]);
                acc[mt] = mfma_bf16(wm, cur.u[1][ks], acc[mt]);
            }
#pragma unroll
            for (int mt = 0; mt < CQ_MT; mt++) acc[mt] = mfma_bf16(frag(2, ks, mt), cur.u[0][ks], acc[mt]);
#pragma unroll
            for (int mt = 0; mt < CQ_MT; mt++) {
                const bf16x8 wh = frag(0, ks, mt);
                acc[mt] = mfma_bf16(wh, cur.u[1][ks], acc[mt]);
                acc[mt] = mfma_bf16(wh, cur.u[2][ks], acc[mt]);
            }
        }
#pragma unroll
        for (int ks = 0; ks < KS; ks++)
#pragma unroll
            for (int mt = 0; mt < CQ_MT; mt++) acc[mt] = mfma_bf16(frag(0, ks, mt), cur.u[0][ks], acc[mt]);
#pragma unroll
        for (int mt = 0; mt < CQ_MT; mt++) {
            xv[mt][0] = cur.p[mt].x - acc[mt][0];
            xv[mt][1] = cur.p[mt].y - acc[mt][1];
            xv[mt][2] = cur.p[mt].z - acc[mt][2];
            xv[mt][3] = cur.p[mt].w - acc[mt][3];
        }
    };

    // stage B of a tile: rotated store, group parameters, codes, stores
    auto stage_b = [&](const float (&xv)[CQ_MT][4], int64_t row, int64_t t0) {
        const bool live = t0 + c16 < a.T;
        if constexpr (ROT) {
            float4 *r = live ? reinterpret_cast<float4 *>(a.rotated + (t0 + c16) * a.n + cbeg + 4 * g)
                             : reinterpret_cast<float4 *>(a.dummy + 128) + 8 * g;
            const int rs = live ? 4 : 1;
#pragma unroll
            for (int mt = 0; mt < CQ_MT; mt++) r[rs * mt] = make_float4(xv[mt][0], xv[mt][1], xv[mt][2], xv[mt][3]);
        }
        // group parameters (NaN-dropping reduction on the common path)
        GroupParams gp[NG];
#pragma unroll
        for (int gi = 0; gi < NG; gi++) {
            float lo = xv[gi * MPG][0], hi = lo;
#pragma unroll
            for (int mt = gi * MPG; mt < (gi + 1) * MPG; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) { lo = fminf(lo, xv[mt][i]); hi = fmaxf(hi, xv[mt][i]); }
            cq_lanes_reduce<false>(lo, hi, g);
            gp[gi] = group_params(lo, hi);
        }
        // codes of two M tiles at a time, packed as they are made: word q holds
        // the lane's codes of M tiles 2q (low 16 bits) and 2q + 1
        float rs[NG];
#pragma unroll
        for (int gi = 0; gi < NG; gi++) rs[gi] = recip_scale(gp[gi].s);
        bool flag = false;
        uint32_t word[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            float e[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int gi = (2 * q + j / 4) / MPG;
                const float y = (xv[2 * q + j / 4][j % 4] - gp[gi].z) * rs[gi];
                const float r = __builtin_rintf(y);
                flag |= !(__builtin_fabsf(y - r) < 0.5f - 0x1p-18f);
                e[j] = __builtin_amdgcn_fmed3f(r, 0.0f, 15.0f);
            }
            word[q] = pack8(e);
        }
        if (__builtin_expect(__any(flag), 0)) {
            // a near-tie or a NaN element in the wave: NaN-propagating
            // parameters and the correctly rounded division for every code
#pragma unroll
            for (int gi = 0; gi < NG; gi++) {
                float lo, hi;
                lane_minmax_nan<4 * MPG>(&xv[gi * MPG][0], lo, hi);
                cq_lanes_reduce<true>(lo, hi, g);
                gp[gi] = group_params(lo, hi);
            }
#pragma unroll
            for (int q = 0; q < 4; q++) {
                float e[8];
#pragma unroll
                for (int j = 0; j < 8; j++) e[j] = (float)quant_code(xv[2 * q + j / 4][j % 4], gp[(2 * q + j / 4) / MPG]);
                word[q] = pack8(e);
            }
        }
        // lane (token, g) now holds word q' of lane (token, q') for q' = 0..3
        // in word[q']; its 16 bytes at 16 g of the block's code row are M tiles
        // 2g (bytes 0-7: two bytes per source lane) and 2g + 1 (bytes 8-15)
        cq_transpose4(word);
        const uint4 out = make_uint4(__builtin_amdgcn_perm(word[1], word[0], 0x05040100u),
                                     __builtin_amdgcn_perm(word[3], word[2], 0x05040100u),
                                     __builtin_amdgcn_perm(word[1], word[0], 0x07060302u),
                                     __builtin_amdgcn_perm(word[3], word[2], 0x07060302u));
        // stores: lanes of tokens past the end, and the lanes that do not
        // hold a group's parameters, write to the scratch area
        uint8_t *cdst = live ? a.codes + row * (a.n / 2) + cbeg / 2 + 16 * g : a.dummy;
        *reinterpret_cast<uint4 *>(cdst) = out;
        // lane g < NG stores the parameters of group g (selected, not indexed:
        // a lane-dependent index would move gp to scratch memory)
        uint16_t s16 = gp[0].s16, z16 = gp[0].z16;
#pragma unroll
        for (int gi = 1; gi < NG; gi++) {
            s16 = g == gi ? gp[gi].s16 : s16;
            z16 = g == gi ? gp[gi].z16 : z16;
        }
        const bool owner = live && g < NG;
        const int64_t go = row * (a.n / B) + cbeg / B + g;
        uint16_t *sdst = owner ? a.scales + go : reinterpret_cast<uint16_t *>(a.dummy + 64);
        uint16_t *zdst = owner ? a.zeros + go : reinterpret_cast<uint16_t *>(a.dummy + 66);
        *sdst = s16;
        *zdst = z16;
    };

    // Software pipeline over the wave's tiles: the MFMA stage of tile j + 1
    // and the quantizer stage of tile j share one scheduling region (the MFMA
    // pipe and the VALU work side by side); tile j + 2 is requested into the
    // buffer tile j has released.  Scheduling barriers between iterations keep
    // every tile's requests in program order (exact wait counts).
    CqTile<KS> buf[2];
    float xv[2][CQ_MT][4];
    int64_t row[2];
    cq_load<KS>(buf[0], a, tile_of(0), cbeg, c16, g);
    __builtin_amdgcn_sched_barrier(0);
    if (TPW > 1) cq_load<KS>(buf[1], a, tile_of(1), cbeg, c16, g);
    __builtin_amdgcn_sched_barrier(0);
    stage_a(buf[0], xv[0]);
    row[0] = buf[0].row;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < TPW; j++) {
        if (j + 1 < TPW) {
            stage_a(buf[(j + 1) & 1], xv[(j + 1) & 1]);
            row[(j + 1) & 1] = buf[(j + 1) & 1].row;
        }
        if (j + 2 < TPW) cq_load<KS>(buf[j & 1], a, tile_of(j + 2), cbeg, c16, g);
        stage_b(xv[j & 1], row[j & 1], tile_of(j));
        __builtin_amdgcn_sched_barrier(0);
    }
}

}  // namespace narhip
