// Group-asymmetric W4A4 GEMM: the consumer of the packed INT4 format.
//
// Activations and weights both come as the rotate-quant output format: codes
// uint8 [rows, n/2] (low nibble = even channel), fp16 scale s and zero z per
// group of 128 channels along the reduction axis, dequantized value q s + z.
// For one group g of output y[t, o]:
//
//   sum_j (qA sA + zA)(qW sW + zW)
//     = sA sW sum_j qA qW  +  (sA SA) zW  +  zA (sW SW + 128 zW)
//
// with SA, SW the group's code sums (the four-term form of
// quarot-llama3/e28_v2/docs/quantizer_contract.md:134-140, the last two terms
// regrouped per side).  The integer code products run on
// v_mfma_i32_16x16x64_i8 (codes 0..15 as int8, two K steps per group); the two
// rank-2 terms on v_mfma_f32_16x16x4_f32, accumulated straight into the fp32
// output tile; the first term's scale product costs three VALU operations per
// (token, output, group).
//
// Block: 128 tokens x 128 outputs, four waves of 64 x 64 (4 x 4 MFMA tiles).
// Per group the block unpacks its A and W codes once into LDS as int8 (the
// low-nibble bytes, then the high-nibble bytes, of each packed word: the same
// channel order on both sides, so the contraction pairs equal channels), sums
// the codes of each row with v_dot4, and stages the per-row scalars; the next
// group's packed codes are loaded during the current group's MFMAs (two LDS
// buffers, one barrier per group).  Dispatch is round-robin over the 8 XCDs by
// linear block id, so when gridDim.x (weight tiles) is a multiple of 8 all
// blocks of one weight tile run on one XCD and share its L2.
#pragma once
#include "narhip_device.hpp"

namespace narhip {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct W4A4Args {
    const uint8_t *ac;        // A codes [T, n/2]
    const uint16_t *as, *az;  // A fp16 scales / zeros [T, G]
    int64_t T;
    const uint8_t *wc;        // W codes [O, n/2]
    const uint16_t *ws, *wz;  // W fp16 scales / zeros [O, G]
    int64_t O;
    int64_t n;                // reduction length, multiple of 128
    float *out;               // [T, ldo] fp32, or split partials [splits][T][O] (blockIdx.z)
    int64_t ldo;
    int splits;               // groups divided over gridDim.z
};

constexpr int WQ_TM = 128, WQ_TN = 128;           // block tile (tokens, outputs)
constexpr int WQ_ROWB = 144;                      // unpacked row: 128 int8 codes + 16 pad (conflict-free b128 reads)
constexpr int WQ_AB = WQ_TM * WQ_ROWB;            // A codes per buffer
constexpr int WQ_WB = WQ_TN * WQ_ROWB;            // W codes per buffer
constexpr int WQ_SB = (WQ_TM + WQ_TN) * 3 * 4;    // row scalars: A {sA, sA*SA, zA}, W {sW, zW, sW*SW + 128 zW}
constexpr int WQ_BUF = WQ_AB + WQ_WB + WQ_SB;

// One thread's share of a group: 32 packed bytes (64 codes) of one row.
struct WqStage {
    uint4 p0, p1;
    uint16_t s, z;
};

__device__ __forceinline__ void wq_load(WqStage &st, const uint8_t *row, const uint16_t *sc, const uint16_t *zr,
                                        int g)
{
    const uint4 *p = reinterpret_cast<const uint4 *>(row + g * 64);
    st.p0 = p[0];
    st.p1 = p[1];
    st.s = sc[g];
    st.z = zr[g];
}

// Unpack to LDS (row r, half h of the group), return the code sum of this half.
__device__ __forceinline__ uint32_t wq_unpack(const WqStage &st, uint8_t *dst)
{
    const uint32_t w[8] = {st.p0.x, st.p0.y, st.p0.z, st.p0.w, st.p1.x, st.p1.y, st.p1.z, st.p1.w};
    uint32_t o[16];
    uint32_t sum = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t lo = w[j] & 0x0F0F0F0Fu, hi = (w[j] >> 4) & 0x0F0F0F0Fu;
        o[2 * j] = lo;
        o[2 * j + 1] = hi;
        sum = __builtin_amdgcn_udot4(lo, 0x01010101u, sum, false);
        sum = __builtin_amdgcn_udot4(hi, 0x01010101u, sum, false);
    }
    uint4 *d = reinterpret_cast<uint4 *>(dst);
#pragma unroll
    for (int q = 0; q < 4; q++) d[q] = make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
    return sum;
}

template <int = 0>
__global__ void __launch_bounds__(256, 2)
w4a4_kernel(W4A4Args a)
{
    __shared__ __align__(16) uint8_t lds[2 * WQ_BUF];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wm = w & 1, wn = w >> 1;               // wave tile: tokens 64 wm.., outputs 64 wn..
    const int l16 = lane & 15, lg = lane >> 4;
    const int64_t o0 = (int64_t)blockIdx.x * WQ_TN, t0 = (int64_t)blockIdx.y * WQ_TM;
    const int G = (int)(a.n / 128);
    const int gb = (int)((int64_t)blockIdx.z * G / a.splits), ge = (int)((int64_t)(blockIdx.z + 1) * G / a.splits);
    const int64_t rowbytes = a.n / 2;

    // loader: row lr (0..127) of both tiles, 64-code half lh of the group
    const int lr = tid >> 1, lh = tid & 1;
    const int64_t ta = t0 + lr < a.T ? t0 + lr : a.T - 1;
    const int64_t ow = o0 + lr < a.O ? o0 + lr : a.O - 1;
    const uint8_t *arow = a.ac + ta * rowbytes + lh * 32;
    const uint8_t *wrow = a.wc + ow * rowbytes + lh * 32;
    const uint16_t *asr = a.as + ta * G, *azr = a.az + ta * G;
    const uint16_t *wsr = a.ws + ow * G, *wzr = a.wz + ow * G;

    auto stage = [&](const WqStage &sa, const WqStage &sw, uint8_t *buf) {
        uint32_t ca = wq_unpack(sa, buf + lr * WQ_ROWB + lh * 64);
        uint32_t cw = wq_unpack(sw, buf + WQ_AB + lr * WQ_ROWB + lh * 64);
        ca += __shfl_xor(ca, 1);
        cw += __shfl_xor(cw, 1);
        if (lh == 0) {
            float *sc = reinterpret_cast<float *>(buf + WQ_AB + WQ_WB);
            const float sA = f16_bits_to_f32(sa.s), zA = f16_bits_to_f32(sa.z);
            const float sW = f16_bits_to_f32(sw.s), zW = f16_bits_to_f32(sw.z);
            sc[lr] = sA;
            sc[WQ_TM + lr] = sA * (float)ca;
            sc[2 * WQ_TM + lr] = zA;
            sc[3 * WQ_TM + lr] = sW;
            sc[3 * WQ_TM + WQ_TN + lr] = zW;
            sc[3 * WQ_TM + 2 * WQ_TN + lr] = __builtin_fmaf(sW, (float)cw, 128.0f * zW);
        }
    };

    WqStage sa, sw;
    wq_load(sa, arow, asr, azr, gb);
    wq_load(sw, wrow, wsr, wzr, gb);
    stage(sa, sw, lds);
    __syncthreads();

    f32x4 acc[4][4];
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int nt = 0; nt < 4; nt++) acc[mt][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    for (int g = gb; g < ge; g++) {
        const uint8_t *buf = lds + ((g - gb) & 1) * WQ_BUF;
        // next group's packed codes and scalars (the last group reloads itself)
        const int gn = g + 1 < ge ? g + 1 : g;
        wq_load(sa, arow, asr, azr, gn);
        wq_load(sw, wrow, wsr, wzr, gn);

        i32x4 d[4][4];
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            i32x4 fa[4], fb[4];
#pragma unroll
            for (int mt = 0; mt < 4; mt++)
                fa[mt] = *reinterpret_cast<const i32x4 *>(buf + (wm * 64 + mt * 16 + l16) * WQ_ROWB + kk * 64 + lg * 16);
#pragma unroll
            for (int nt = 0; nt < 4; nt++)
                fb[nt] = *reinterpret_cast<const i32x4 *>(buf + WQ_AB + (wn * 64 + nt * 16 + l16) * WQ_ROWB + kk * 64 +
                                                          lg * 16);
#pragma unroll
            for (int mt = 0; mt < 4; mt++)
#pragma unroll
                for (int nt = 0; nt < 4; nt++)
                    d[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                        fa[mt], fb[nt], kk ? d[mt][nt] : i32x4{0, 0, 0, 0}, 0, 0, 0);
        }

        // epilogue of the group
        const float *sc = reinterpret_cast<const float *>(buf + WQ_AB + WQ_WB);
        f32x4 sA4[4];
        float pA[4], sWv[4], qB[4];
#pragma unroll
        for (int mt = 0; mt < 4; mt++) {
            const int r = wm * 64 + mt * 16;
            sA4[mt] = *reinterpret_cast<const f32x4 *>(sc + r + 4 * lg);
            // f32 MFMA A operand: row l16, K slot lg: (sA SA, zA, 0, 0)
            pA[mt] = lg < 2 ? sc[(1 + lg) * WQ_TM + r + l16] : 0.0f;
        }
#pragma unroll
        for (int nt = 0; nt < 4; nt++) {
            const int c = wn * 64 + nt * 16 + l16;
            sWv[nt] = sc[3 * WQ_TM + c];
            // B operand: column l16, K slot lg: (zW, sW SW + 128 zW, 0, 0)
            qB[nt] = lg < 2 ? sc[3 * WQ_TM + (1 + lg) * WQ_TN + c] : 0.0f;
        }
#pragma unroll
        for (int mt = 0; mt < 4; mt++)
#pragma unroll
            for (int nt = 0; nt < 4; nt++) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[mt][nt][i] = __builtin_fmaf(sA4[mt][i] * sWv[nt], (float)d[mt][nt][i], acc[mt][nt][i]);
                acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(pA[mt], qB[nt], acc[mt][nt], 0, 0, 0);
            }

        stage(sa, sw, lds + ((g + 1 - gb) & 1) * WQ_BUF);
        __syncthreads();
    }

    // one split: the output; several: partial [blockIdx.z][T][O], summed in split order by w4a4_reduce
    float *dst = a.splits == 1 ? a.out : a.out + (int64_t)blockIdx.z * a.T * a.O;
    const int64_t ld = a.splits == 1 ? a.ldo : a.O;

#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int nt = 0; nt < 4; nt++) {
            const int64_t o = o0 + wn * 64 + nt * 16 + l16;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int64_t t = t0 + wm * 64 + mt * 16 + 4 * lg + i;
                if (t < a.T && o < a.O) dst[t * ld + o] = acc[mt][nt][i];
            }
        }
}

// out[t, o] = sum over splits s, in order, of part[s][t][o].
template <int = 0>
__global__ void __launch_bounds__(256)
w4a4_reduce_kernel(const float *part, int splits, int64_t T, int64_t O, float *out, int64_t ldo)
{
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= T * O) return;
    const int64_t t = i / O, o = i % O;
    float s = part[i];
    for (int z = 1; z < splits; z++) s += part[(int64_t)z * T * O + i];
    out[t * ldo + o] = s;
}

}  // namespace narhip
