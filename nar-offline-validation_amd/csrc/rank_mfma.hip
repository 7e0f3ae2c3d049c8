// Rank-k stages on bf16 MFMA (k >= 16 over a full row).
//
//   prep_v / prep_w : fp32 factors -> three exact bf16 terms in MFMA-friendly
//                     layouts (done once per factor set, like the reference's
//                     fp16_terms / FoldedR4 term padding, nar_r4_kernel.py:151-187)
//   proj_mfma       : Kernel A, u partials = x V over channel splits
//                     (nar/kernels/r4_fused_v3.py:83-135): x is bf16 (exact),
//                     V enters as hi/mid/lo terms, hi and mid+lo in separate
//                     accumulators, folded in fp64 at the end of the split
//   fold_u          : u = fp64 fold of the split partials, rounded once, as
//                     three bf16 terms per token
//   corr_quant      : x' = P - u W^T with u and W^T both as three bf16 terms
//                     (the six term products of weight >= 2^-16), then the
//                     INT4 quantizer of nar/experiment.py:158-184
#pragma once
#include "mfma.hpp"
#include "narhip_device.hpp"

namespace narhip {

// v [n, k] fp32 -> vt [3][kp16][n] bf16 (rank-major, zero rows for r >= k)
template <int = 0>
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
template <int = 0>
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

// grid (ceil(T/128), splits), block 256.  Wave w owns tokens 32w..32w+31 of
// the 128-token tile as two 16-token N tiles; all MT rank tiles of 16 rows.
// The split's channels are walked in blocks of 64: the V terms of a block are
// staged in LDS (two buffers, one barrier per block); x runs three blocks
// ahead in a register ring and V two blocks ahead (down_proj 70B, 16384 x
// 28672, k = 64: 315 -> 258 us; one block ahead of both left a single block of
// x in flight per wave).
template <int MT>
__global__ void __launch_bounds__(256, 2)
proj_mfma_kernel(ProjMfmaArgs a)
{
    constexpr int KB = 64;                  // channels per block (two LDS buffers, 28 KB at k = 32:
                                            // leaves room for a concurrent transform workgroup)
    constexpr int ROWS = 16 * MT;
    constexpr int VSTR = KB + 8;            // padded LDS row (bf16)
    constexpr int VPIECES = 3 * ROWS * (KB / 8);              // 16-byte pieces per block
    constexpr int VPT = (VPIECES + 255) / 256;                // pieces per thread
    constexpr bool VFULL = VPIECES % 256 == 0;                // no guard: loads outside branches
    constexpr int XD = 3;                   // x blocks in flight per wave (12 KB; at 512 workgroups
                                            // two waves per SIMD must cover HBM latency)
    __shared__ __align__(16) __bf16 vs[2][3][ROWS][VSTR];
    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int s = blockIdx.y;
    const int64_t c_begin = (int64_t)s * a.cs;
    const int64_t plane = (int64_t)a.kp * a.n;
    const int nblk = (int)(a.cs / KB);
    const uint16_t *xrow[2];
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        int64_t t = (int64_t)blockIdx.x * 128 + w * 32 + 16 * nt + c16;
        if (t >= a.T) t = a.T - 1;
        xrow[nt] = a.x + t * a.ldx + c_begin + 8 * g;
    }
    auto v_src = [&](int p, int blk) -> const __bf16 * {
        const int term = p / (ROWS * (KB / 8)), rem = p % (ROWS * (KB / 8));
        const int r = rem / (KB / 8), c8 = rem % (KB / 8);
        return a.vt + term * plane + (int64_t)r * a.n + c_begin + (int64_t)blk * KB + c8 * 8;
    };
    auto v_dst = [&](int p, int buf) -> __bf16 * {
        const int term = p / (ROWS * (KB / 8)), rem = p % (ROWS * (KB / 8));
        const int r = rem / (KB / 8), c8 = rem % (KB / 8);
        return &vs[buf][term][r][c8 * 8];
    };
    floatx4 acc_h[MT][2], acc_l[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++) { acc_h[mt][nt] = zero4(); acc_l[mt][nt] = zero4(); }

    // Loads run ahead of use: x of block b + XD is requested after block b's
    // MFMAs (slot b % XD of a register ring), V of block b + 2 before them
    // (slot b % 2); V of block b + 1, requested one block earlier, goes to LDS
    // at the end of block b.  Memory operations complete in order, so waiting
    // for that V load waits only for the x of block b + 1 as well.  The loop is
    // unrolled by 2 XD so every slot is a fixed register range.  Requests past
    // the split's last block re-request that block (L2 hits).
    bf16x8 xq[XD][KB / 32][2], vr[2][VPT];
    auto load_v = [&](bf16x8 (&dst)[VPT], int blk) {
#pragma unroll
        for (int i = 0; i < VPT; i++) {
            const int p = tid + 256 * i;
            if (VFULL || p < VPIECES) dst[i] = load_bf16x8(v_src(p, blk));
        }
    };
    auto store_v = [&](const bf16x8 (&src)[VPT], int buf) {
#pragma unroll
        for (int i = 0; i < VPT; i++) {
            const int p = tid + 256 * i;
            if (VFULL || p < VPIECES) *reinterpret_cast<bf16x8 *>(v_dst(p, buf)) = src[i];
        }
    };
    auto load_x = [&](bf16x8 (&dst)[KB / 32][2], int blk) {
        const int64_t bo = (int64_t)(blk < nblk ? blk : nblk - 1) * KB;
#pragma unroll
        for (int ks = 0; ks < KB / 32; ks++)
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
                dst[ks][nt] = *reinterpret_cast<const bf16x8 *>(xrow[nt] + bo + 32 * ks);
    };
    load_v(vr[0], 0);
#pragma unroll
    for (int d = 0; d < XD; d++) load_x(xq[d], d);
    load_v(vr[1], nblk > 1 ? 1 : 0);
    store_v(vr[0], 0);
    __syncthreads();
    for (int b0 = 0; b0 < nblk; b0 += 2 * XD) {
#pragma unroll
        for (int d = 0; d < 2 * XD; d++) {
            const int b = b0 + d;
            if (b >= nblk) break;
            load_v(vr[d % 2], b + 2 < nblk ? b + 2 : nblk - 1);
            __builtin_amdgcn_sched_barrier(0);
            const int cur = b & 1;
#pragma unroll
            for (int ks = 0; ks < KB / 32; ks++) {
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const bf16x8 ah = *reinterpret_cast<const bf16x8 *>(&vs[cur][0][16 * mt + c16][32 * ks + 8 * g]);
                    const bf16x8 am = *reinterpret_cast<const bf16x8 *>(&vs[cur][1][16 * mt + c16][32 * ks + 8 * g]);
                    const bf16x8 al = *reinterpret_cast<const bf16x8 *>(&vs[cur][2][16 * mt + c16][32 * ks + 8 * g]);
#pragma unroll
                    for (int nt = 0; nt < 2; nt++) {
                        acc_h[mt][nt] = mfma_bf16(ah, xq[d % XD][ks][nt], acc_h[mt][nt]);
                        acc_l[mt][nt] = mfma_bf16(am, xq[d % XD][ks][nt], acc_l[mt][nt]);
                        acc_l[mt][nt] = mfma_bf16(al, xq[d % XD][ks][nt], acc_l[mt][nt]);
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            load_x(xq[d % XD], b + XD);
            store_v(vr[(d + 1) % 2], cur ^ 1);
            __syncthreads();
        }
    }
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        const int64_t t = (int64_t)blockIdx.x * 128 + w * 32 + 16 * nt + c16;
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

// u for each token from the split partials: fp64 fold in split order, rounded
// once to fp32, then split in three bf16 terms.  u3 [T][3][kp] (zero for r >= k).
template <int = 0>
__global__ void __launch_bounds__(256)
fold_u_kernel(const float *partial, int splits, int k, int kp, int64_t T, __bf16 *u3)
{
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= T * kp) return;
    const int64_t t = idx / kp;
    const int r = (int)(idx % kp);
    double sum = 0.0;
    if (r < k) {
        const float *pp = partial + t * (int64_t)splits * k + r;
        for (int s = 0; s < splits; s++) sum += (double)pp[(int64_t)s * k];
    }
    __bf16 h, m, l;
    split3((float)sum, h, m, l);
    __bf16 *o = u3 + t * 3 * kp + r;
    o[0] = h; o[kp] = m; o[2 * kp] = l;
}

struct CorrQuantArgs {
    const float *P;        // [T, n] rotated rows before the rank term
    int64_t T, n;
    const __bf16 *u3;      // [T][3][kp] terms of u
    const __bf16 *wtt;     // [3][n][kp] terms of W^T
    int kp;
    uint8_t *codes;
    uint16_t *scales;
    uint16_t *zeros;
    const int64_t *dest;
    float *rotated;        // x' [T, n] (kernel variant ROT only)
    uint8_t *dummy;        // scratch row (>= n/2 bytes) that takes the stores of tokens >= T
    int64_t ncb;           // n / CW channel blocks
    int tpw;               // 128-token tiles per workgroup
};

// One unit of corr_quant work: 16 tokens (one MFMA N tile) x one quantization
// group of B channels (B/16 M tiles).  Lane l holds P / x' for token l%16 of
// the tile and channels 16 mt + 4g .. +3 (g = l/16): B/16 float4 per lane.
template <int B>
struct CqUnit {
    float v[B / 16][4];
};

template <int B>
__device__ __forceinline__ void cq_load(CqUnit<B> &p, const float *prow)
{
#pragma unroll
    for (int mt = 0; mt < B / 16; mt++) {
        const float4 pv = *reinterpret_cast<const float4 *>(prow + 16 * mt);
        p.v[mt][0] = pv.x; p.v[mt][1] = pv.y; p.v[mt][2] = pv.z; p.v[mt][3] = pv.w;
    }
}

// x' = P - u W^T for one group of B channels and both 16-token halves (W^T
// terms of the group at wl in LDS: rows of WROW bf16, planes of WPLANE; each
// fragment read once and used for both halves), then codes, scales and zeros
// staged in LDS: codes of token 16h + c16 at crow[(16h + c16) * CSTRIDE + ...]
// (uint16 = four codes), scale and zero at sz[2 (16h + c16)], sz[... + 1].
// Only x' (variant ROT) goes to memory here.
template <int B, int KS, int WROW, int WPLANE, int CSTRIDE, bool ROT>
__device__ __forceinline__ void cq_group(CqUnit<B> (&xt)[2], const CorrQuantArgs &a,
                                         const bf16x8 (&ub)[2][3][KS], float *const (&rrow)[2],
                                         const __bf16 *wl, uint16_t *crow, uint16_t *sz, int lane)
{
    constexpr int MTG = B / 16;
    const int g = lane >> 4, c16 = lane & 15;
#pragma unroll
    for (int mt = 0; mt < MTG; mt++) {
        const __bf16 *wrow = wl + (16 * mt + c16) * WROW + 8 * g;
        bf16x8 wh[KS], wm[KS], wo[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            wh[ks] = *reinterpret_cast<const bf16x8 *>(wrow + 32 * ks);
            wm[ks] = *reinterpret_cast<const bf16x8 *>(wrow + WPLANE + 32 * ks);
            wo[ks] = *reinterpret_cast<const bf16x8 *>(wrow + 2 * WPLANE + 32 * ks);
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            floatx4 main = zero4(), small = zero4();
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                main = mfma_bf16(wh[ks], ub[h][0][ks], main);
                small = mfma_bf16(wm[ks], ub[h][0][ks], small);
                small = mfma_bf16(wh[ks], ub[h][1][ks], small);
                small = mfma_bf16(wo[ks], ub[h][0][ks], small);
                small = mfma_bf16(wh[ks], ub[h][2][ks], small);
                small = mfma_bf16(wm[ks], ub[h][1][ks], small);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) xt[h].v[mt][i] = xt[h].v[mt][i] - (main[i] + small[i]);
        }
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
        auto &xv = xt[h].v;
        if constexpr (ROT) {
#pragma unroll
            for (int mt = 0; mt < MTG; mt++)
                *reinterpret_cast<float4 *>(rrow[h] + 16 * mt) = make_float4(xv[mt][0], xv[mt][1], xv[mt][2], xv[mt][3]);
        }
        // the group of token c16 is spread over lanes c16 + 16g
        float lo = xv[0][0], hi = lo;
#pragma unroll
        for (int mt = 0; mt < MTG; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) { lo = fminf(lo, xv[mt][i]); hi = fmaxf(hi, xv[mt][i]); }
        lo = fminf(lo, __shfl_xor(lo, 16)); hi = fmaxf(hi, __shfl_xor(hi, 16));
        lo = fminf(lo, __shfl_xor(lo, 32)); hi = fmaxf(hi, __shfl_xor(hi, 32));
        GroupParams gp = group_params(lo, hi);
        const float rs = 1.0f / gp.s;
        bool flag = false;
        uint32_t q16[MTG];
#pragma unroll
        for (int mt = 0; mt < MTG; mt++) {
            q16[mt] = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) q16[mt] |= quant_code_fast(xv[mt][i], gp.z, rs, flag) << (4 * i);
        }
        if (__builtin_expect(__any(flag), 0)) {
            // a near-tie or a NaN element: NaN-propagating parameters, exact codes
            lane_minmax_nan<4 * MTG>(&xv[0][0], lo, hi);
            lo = min_nan(lo, __shfl_xor(lo, 16)); hi = max_nan(hi, __shfl_xor(hi, 16));
            lo = min_nan(lo, __shfl_xor(lo, 32)); hi = max_nan(hi, __shfl_xor(hi, 32));
            gp = group_params(lo, hi);
#pragma unroll
            for (int mt = 0; mt < MTG; mt++) {
                q16[mt] = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) q16[mt] |= quant_code(xv[mt][i], gp) << (4 * i);
            }
        }
#pragma unroll
        for (int mt = 0; mt < MTG; mt++) crow[(16 * h + c16) * CSTRIDE + 4 * mt + g] = (uint16_t)q16[mt];
        if (g == 0) {
            sz[2 * (16 * h + c16)] = gp.s16;
            sz[2 * (16 * h + c16) + 1] = gp.z16;
        }
    }
}

// grid (8 * ncb * ceil(token groups / 8)), block 256.  A workgroup owns CW
// channels: it stages their W^T terms in LDS once ([3][CW][KP], 48 KB) and
// then runs a.tpw tiles of 128 tokens over them.  Within a tile every wave
// works alone (no further workgroup barriers) on 32 tokens x CW channels:
// all of its P (128 VGPRs at CW = 256) is requested at once, then the groups
// are processed in load order, each waiting only for its own loads.  Codes, scales and zeros are staged in LDS and stored
// after the last unit; tokens >= T store into a scratch row, so that no
// memory operation sits under a branch and the wait counts stay exact.
// Workgroups are dispatched to the 8 XCDs round-robin by block id, so the
// token group is chosen from (id % 8) and the channel block from the quotient:
// all channel blocks of a token group run on one XCD, and the 2-byte scale and
// zero stores of those tokens merge into whole lines in that XCD's L2.
template <int B, int KS, int CW, bool ROT>
__global__ void __launch_bounds__(256, 2)
corr_quant_kernel(CorrQuantArgs a)
{
    constexpr int KP = 32 * KS;
    constexpr int WROW = KP + 8;             // padded channel row: fragment reads hit distinct banks
    constexpr int WPLANE = CW * WROW;
    constexpr int NG = CW / B;               // groups per channel block
    constexpr int CSTRIDE = CW / 4 + 8;      // uint16 per token row of staged codes (16-byte rows, padded
                                             // so the 16 tokens of a store land in different banks)
    __shared__ __align__(16) __bf16 ws[3 * WPLANE];
    __shared__ __align__(16) uint16_t cst[4][32 * CSTRIDE];
    __shared__ __align__(16) uint16_t szs[4][NG][64];   // [2 t + 0] scale, [2 t + 1] zero of token t
    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int64_t j = (int64_t)blockIdx.x / 8;
    const int64_t cb = j % a.ncb;
    const int64_t tg = (j / a.ncb) * 8 + blockIdx.x % 8;
    if (tg * a.tpw * 128 >= a.T) return;
    const int64_t cbeg = cb * CW;
    const int64_t plane = (int64_t)KP * a.n;

    for (int p = tid; p < 3 * CW * (KP / 8); p += 256) {
        const int term = p / (CW * (KP / 8)), rem = p % (CW * (KP / 8));
        const int ch = rem / (KP / 8), k8 = rem % (KP / 8);
        *reinterpret_cast<bf16x8 *>(&ws[term * WPLANE + ch * WROW + k8 * 8]) =
            load_bf16x8(a.wtt + term * plane + (cbeg + ch) * KP + k8 * 8);
    }
    __syncthreads();

    for (int tt = 0; tt < a.tpw; tt++) {
        const int64_t t0 = (tg * a.tpw + tt) * 128 + w * 32;
        if (t0 >= a.T) return;
        // output rows: code stores (token lane/2), scale stores (token lane, lanes < 32)
        const int64_t tc = t0 + (lane >> 1), ts = t0 + (lane & 31);
        int64_t crow_out = tc < a.T ? tc : -1, srow_out = ts < a.T ? ts : -1;
        if (a.dest) {
            if (crow_out >= 0) crow_out = a.dest[crow_out];
            if (srow_out >= 0) srow_out = a.dest[srow_out];
        }
        const float *prow[2];
        float *rrow[2];
        bf16x8 ub[2][3][KS];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int64_t t = t0 + 16 * h + c16;
            const int64_t tk = t < a.T ? t : a.T - 1;
            prow[h] = a.P + tk * a.n + cbeg + 4 * g;
            rrow[h] = ROT ? (t < a.T ? a.rotated + tk * a.n + cbeg + 4 * g
                                     : reinterpret_cast<float *>(a.dummy) + 4 * g) : nullptr;
#pragma unroll
            for (int term = 0; term < 3; term++)
#pragma unroll
                for (int ks = 0; ks < KS; ks++)
                    ub[h][term][ks] = load_bf16x8(a.u3 + (tk * 3 + term) * KP + 32 * ks + 8 * g);
        }
        CqUnit<B> U[NG][2];
#pragma unroll
        for (int gi = 0; gi < NG; gi++)
#pragma unroll
            for (int h = 0; h < 2; h++) cq_load<B>(U[gi][h], prow[h] + gi * B);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int gi = 0; gi < NG; gi++) {
            float *const rr[2] = {ROT ? rrow[0] + gi * B : nullptr, ROT ? rrow[1] + gi * B : nullptr};
            cq_group<B, KS, WROW, WPLANE, CSTRIDE, ROT>(U[gi], a, ub, rr, ws + gi * B * WROW,
                                                        &cst[w][gi * B / 4], &szs[w][gi][0], lane);
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // codes: two lanes per token, CW/4 bytes each (16-byte pieces)
        {
            const int half = lane & 1;
            uint8_t *base = crow_out >= 0 ? a.codes + crow_out * (a.n / 2) + cbeg / 2 : a.dummy;
            uint4 *dst = reinterpret_cast<uint4 *>(base + half * (CW / 4));
            const uint4 *src = reinterpret_cast<const uint4 *>(&cst[w][(lane >> 1) * CSTRIDE + half * (CW / 8)]);
#pragma unroll
            for (int q = 0; q < CW / 64; q++) dst[q] = src[q];
        }
        // scales and zeros: lanes 0..31 write token lane's NG groups (lanes 32..63 repeat them)
        {
            uint16_t *sd = srow_out >= 0 ? a.scales + srow_out * (a.n / B) + cbeg / B
                                         : reinterpret_cast<uint16_t *>(a.dummy);
            uint16_t *zd = srow_out >= 0 ? a.zeros + srow_out * (a.n / B) + cbeg / B
                                         : reinterpret_cast<uint16_t *>(a.dummy);
            const int tl = lane & 31;
#pragma unroll
            for (int q = 0; q < NG; q++) {
                sd[q] = szs[w][q][2 * tl];
                zd[q] = szs[w][q][2 * tl + 1];
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// Device self-test of the operand mapping: one MFMA on per-lane inputs.
template <int = 0>
__global__ void mfma_probe_kernel(const __bf16 *a, const __bf16 *b, float *d)
{
    const int l = threadIdx.x;
    const floatx4 r = mfma_bf16(load_bf16x8(a + 8 * l), load_bf16x8(b + 8 * l), zero4());
#pragma unroll
    for (int i = 0; i < 4; i++) d[4 * l + i] = r[i];
}

}  // namespace narhip
