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
//   (the correction and quantizer that consume u are in corr_quant.hip)
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
        // eight partials in flight, added in split order
        const float *pp = partial + t * (int64_t)splits * k + r;
        int sp = 0;
        for (; sp + 8 <= splits; sp += 8) {
            float f[8];
#pragma unroll
            for (int j = 0; j < 8; j++) f[j] = pp[(int64_t)(sp + j) * k];
#pragma unroll
            for (int j = 0; j < 8; j++) sum += (double)f[j];
        }
        for (; sp < splits; sp++) sum += (double)pp[(int64_t)sp * k];
    }
    __bf16 h, m, l;
    split3((float)sum, h, m, l);
    __bf16 *o = u3 + t * 3 * kp + r;
    o[0] = h; o[kp] = m; o[2 * kp] = l;
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
