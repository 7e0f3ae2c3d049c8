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
// regrouped per side).
//
// The code products run on the fp8 matrix cores: a code byte c (0..15) read as
// OCP e4m3 is exactly c * 2^-9 (c < 8 are the subnormals m * 2^-9, 8..15 have
// exponent field 1 and mantissa c - 8), so one v_mfma_scale_f32_16x16x128_f8f6f4
// on the unpacked code bytes gives sum_j qA qW * 2^-18 for a whole group,
// exactly (integers below 2^15 times a power of two), already in fp32.  The
// 2^18 goes into the staged weight scale, so the first term costs one multiply
// and one FMA per (token, output, group).  The two offset terms run as a rank-4
// product on v_mfma_f32_16x16x4_f32, two groups per instruction.
//
// Block: 128 tokens x 128 outputs, four waves of 64 x 64 (4 x 4 MFMA tiles).
// Per group the block unpacks its A and W codes once into LDS as bytes (the
// low-nibble bytes, then the high-nibble bytes, of each packed word: the same
// channel order on both sides, so the contraction pairs equal channels), sums
// the codes of each row with v_dot8 and stages the per-row scalars: the scales
// beside the codes (two buffers, one barrier per group), the offset-term
// scalars in a three-slot ring, so that a pair of groups can be read after the
// first group's code buffer is reused.  Packed codes travel in two register
// sets, loaded two groups ahead.  Within a group each code MFMA is issued
// ahead of four VALU operations (scale terms of the tile before it, unpack of
// the next group).  Dispatch is round-robin over the 8 XCDs by linear block
// id, so when gridDim.x (weight tiles) is a multiple of 8 all blocks of one
// weight tile run on one XCD and share its L2.
#pragma once
#include "narhip_device.hpp"

namespace narhip {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
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
constexpr int WQ_ROWB = 144;                      // unpacked row: 128 code bytes + 16 pad (conflict-free b128 reads)
constexpr int WQ_AB = WQ_TM * WQ_ROWB;            // A codes per buffer
constexpr int WQ_WB = WQ_TN * WQ_ROWB;            // W codes per buffer
constexpr int WQ_SB = (WQ_TM + WQ_TN) * 4;        // scale scalars: A sA, W sW 2^18
constexpr int WQ_BUF = WQ_AB + WQ_WB + WQ_SB;     // one group's codes and scales (two buffers)
constexpr int WQ_RB = (WQ_TM + WQ_TN) * 2 * 4;    // one group's offset-term scalars (three-slot ring):
                                                  // A {sA SA, zA}, W {zW, sW SW + 128 zW}
constexpr int WQ_LDS = 2 * WQ_BUF + 3 * WQ_RB;
static_assert(WQ_LDS <= 81920, "two workgroups per CU share 160 KiB of LDS");
constexpr float WQ_E4M3_UNIT2 = 262144.0f;        // 2^18 = 1 / (2^-9 * 2^-9)
constexpr int WQ_E8M0_ONE = 127;                  // MFMA block scale 2^0

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
        o[2 * j] = w[j] & 0x0F0F0F0Fu;
        o[2 * j + 1] = (w[j] >> 4) & 0x0F0F0F0Fu;
        sum = __builtin_amdgcn_udot8(w[j], 0x11111111u, sum, false);
    }
    uint4 *d = reinterpret_cast<uint4 *>(dst);
#pragma unroll
    for (int q = 0; q < 4; q++) d[q] = make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
    return sum;
}

__device__ __forceinline__ i32x8 wq_frag(const uint8_t *p)
{
    const i32x4 lo = *reinterpret_cast<const i32x4 *>(p), hi = *reinterpret_cast<const i32x4 *>(p + 16);
    return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

template <int = 0>
__global__ void __launch_bounds__(256, 2)
w4a4_kernel(W4A4Args a)
{
    __shared__ __align__(16) uint8_t lds[WQ_LDS];
    float *const ring = reinterpret_cast<float *>(lds + 2 * WQ_BUF);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wm = w & 1, wn = w >> 1;               // wave tile: tokens 64 wm.., outputs 64 wn..
    const int l16 = lane & 15, lg = lane >> 4;
    const int64_t o0 = (int64_t)blockIdx.x * WQ_TN, t0 = (int64_t)blockIdx.y * WQ_TM;
    const int G = (int)(a.n / 128);
    const int gb = (int)((int64_t)blockIdx.z * G / a.splits), ge = (int)((int64_t)(blockIdx.z + 1) * G / a.splits);
    const int cnt = ge - gb;
    const int64_t rowbytes = a.n / 2;

    // loader: row lr (0..127) of both tiles, 64-code half lh of the group
    const int lr = tid >> 1, lh = tid & 1;
    const int64_t ta = t0 + lr < a.T ? t0 + lr : a.T - 1;
    const int64_t ow = o0 + lr < a.O ? o0 + lr : a.O - 1;
    const uint8_t *arow = a.ac + ta * rowbytes + lh * 32;
    const uint8_t *wrow = a.wc + ow * rowbytes + lh * 32;
    const uint16_t *asr = a.as + ta * G, *azr = a.az + ta * G;
    const uint16_t *wsr = a.ws + ow * G, *wzr = a.wz + ow * G;
    auto load = [&](WqStage &sa, WqStage &sw, int j) {
        const int g = gb + (j < cnt ? j : cnt - 1);   // past the end: reload the last group
        wq_load(sa, arow, asr, azr, g);
        wq_load(sw, wrow, wsr, wzr, g);
    };

    // Unpack group j into its code buffer and scalar slots; branch-free (the
    // even thread of a row pair writes the A scalars, the odd one the W
    // scalars) so that a group step stays one scheduling region.
    static_assert(WQ_TM == WQ_TN, "scalar rows are addressed with one stride");
    auto stage = [&](const WqStage &sa, const WqStage &sw, int j) {
        uint8_t *buf = lds + (j & 1) * WQ_BUF;
        uint32_t ca = wq_unpack(sa, buf + lr * WQ_ROWB + lh * 64);
        uint32_t cw = wq_unpack(sw, buf + WQ_AB + lr * WQ_ROWB + lh * 64);
        ca += __shfl_xor(ca, 1);
        cw += __shfl_xor(cw, 1);
        const bool isA = lh == 0;
        const float sv = f16_bits_to_f32(isA ? sa.s : sw.s), zv = f16_bits_to_f32(isA ? sa.z : sw.z);
        const float cs = (float)(isA ? ca : cw);
        float *rs = ring + (j % 3) * (WQ_RB / 4) + lh * 2 * WQ_TM;
        rs[lr] = isA ? sv * cs : zv;                                      // sA SA | zW
        rs[WQ_TM + lr] = isA ? zv : __builtin_fmaf(sv, cs, 128.0f * zv);  // zA   | sW SW + 128 zW
        reinterpret_cast<float *>(buf + WQ_AB + WQ_WB)[lh * WQ_TM + lr] = isA ? sv : sv * WQ_E4M3_UNIT2;
    };

    // two register sets of packed codes in flight: group j + 1 is loaded
    // during group j - 1, so its latency spans two group steps
    WqStage st[2][2];
    load(st[0][0], st[0][1], 0);
    load(st[1][0], st[1][1], 1);
    stage(st[0][0], st[0][1], 0);
    __syncthreads();

    f32x4 acc[4][4];
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int nt = 0; nt < 4; nt++) acc[mt][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // rank-4 offset terms of the pair of groups (j - 1, j) (slots 0, 1 from
    // the first, 2, 3 from the second), or of group j alone (slots 2, 3 zero)
    auto offsets = [&](int j, bool pair) {
        const int slot = lg < 2 ? (pair ? (j + 2) % 3 : j % 3) : j % 3;
        const float *rs = ring + slot * (WQ_RB / 4);
        const bool live = pair || lg < 2;
        float pA[4], qB[4];
#pragma unroll
        for (int mt = 0; mt < 4; mt++) {
            const float v = rs[(lg & 1) * WQ_TM + wm * 64 + mt * 16 + l16];                  // (sA SA, zA)
            pA[mt] = live ? v : 0.0f;
        }
#pragma unroll
        for (int nt = 0; nt < 4; nt++) {
            const float v = rs[2 * WQ_TM + (lg & 1) * WQ_TN + wn * 64 + nt * 16 + l16];   // (zW, sW SW + 128 zW)
            qB[nt] = live ? v : 0.0f;
        }
#pragma unroll
        for (int mt = 0; mt < 4; mt++)
#pragma unroll
            for (int nt = 0; nt < 4; nt++)
                acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(pA[mt], qB[nt], acc[mt][nt], 0, 0, 0);
    };

    // One group: load group j + 2 into the register set group j came in;
    // the 16 code MFMAs with their scale terms; at the second group of a pair
    // (PAR = 1) the pair's offset terms; unpack group j + 1; barrier.
    auto step = [&](auto par, int j) {
        constexpr int PAR = decltype(par)::value;
        load(st[PAR][0], st[PAR][1], j + 2);
        const uint8_t *buf = lds + PAR * WQ_BUF;
        const float *sc = reinterpret_cast<const float *>(buf + WQ_AB + WQ_WB);
        f32x4 sA4[4];
        float sWv[4];
#pragma unroll
        for (int mt = 0; mt < 4; mt++) sA4[mt] = *reinterpret_cast<const f32x4 *>(sc + wm * 64 + mt * 16 + 4 * lg);
#pragma unroll
        for (int nt = 0; nt < 4; nt++) sWv[nt] = sc[WQ_TM + wn * 64 + nt * 16 + l16];

        i32x8 fb[4];
#pragma unroll
        for (int nt = 0; nt < 4; nt++) fb[nt] = wq_frag(buf + WQ_AB + (wn * 64 + nt * 16 + l16) * WQ_ROWB + lg * 32);
        f32x4 d[4][4];
#pragma unroll
        for (int mt = 0; mt < 4; mt++) {
            const i32x8 fa = wq_frag(buf + (wm * 64 + mt * 16 + l16) * WQ_ROWB + lg * 32);
#pragma unroll
            for (int nt = 0; nt < 4; nt++)
                d[mt][nt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                    fa, fb[nt], f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0, WQ_E8M0_ONE, 0, WQ_E8M0_ONE);
        }
#pragma unroll
        for (int mt = 0; mt < 4; mt++)
#pragma unroll
            for (int nt = 0; nt < 4; nt++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[mt][nt][i] = __builtin_fmaf(sA4[mt][i] * sWv[nt], d[mt][nt][i], acc[mt][nt][i]);
        if constexpr (PAR == 1) offsets(j, true);
        // unconditional: after the last group this rewrites the other buffer
        // and a free ring slot with a reloaded group that nothing reads
        stage(st[1 - PAR][0], st[1 - PAR][1], j + 1);
        // issue order: each code MFMA followed by 4 VALU operations (the
        // scale terms of the tile before it, the unpack), so that the matrix
        // cores and the VALU of the wave work at the same time
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
#pragma unroll
        for (int i = 0; i < 15; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        __syncthreads();
    };

    int j = 0;
    for (; j + 1 < cnt; j += 2) {
        step(std::integral_constant<int, 0>{}, j);
        step(std::integral_constant<int, 1>{}, j + 1);
    }
    if (j < cnt) {
        step(std::integral_constant<int, 0>{}, j);
        offsets(j, false);      // an unpaired last group
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
