// Device-side building blocks shared by the NAR rotate-and-quantize kernels.
//
// gfx950 (CDNA4), wave64.  Every fp32 operation that the reference pins is
// written so that it compiles to exactly one IEEE round-to-nearest-even
// operation: butterflies are plain add/sub (or fma with a +-1 multiplier,
// which is exact), divisions use the correctly rounded fp32 divide, rounding
// to integers uses v_rndne.  The library is built without fast-math and
// without fp32 denormal flushing.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace narhip {

// ------------------------------------------------------------ conversions --

__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> fp16 bits, round to nearest even (hardware v_cvt_f16_f32, default
// rounding mode), subnormals and overflow to infinity as IEEE.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f)
{
    return __half_as_ushort(__float2half_rn(f));
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h)
{
    return __half2float(__ushort_as_half(h));
}

// ----------------------------------------------------- row-local exchange --
//
// A "row" is 16 consecutive lanes.  The kernels map the 4 lane bits of a row
// to 4 bits of a segment position through
//     chunk(L) = (l0^l2) | (l1^l2)<<1 | (l2^l3)<<2 | l3<<3
// so that flipping chunk bit j is a lane exchange with xor mask 1, 2, 7, 15 --
// exactly the DPP patterns quad_perm[1,0,3,2], quad_perm[2,3,0,1],
// row_half_mirror and row_mirror.  Every butterfly stage that crosses lanes is
// therefore one DPP move within the row, with no LDS traffic.

enum : int {
    DPP_XOR1 = 0xB1,         // quad_perm [1,0,3,2]
    DPP_XOR2 = 0x4E,         // quad_perm [2,3,0,1]
    DPP_XOR7 = 0x141,        // row_half_mirror
    DPP_XOR15 = 0x140,       // row_mirror
};

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v)
{
    int lo = __builtin_amdgcn_mov_dpp(__double2loint(v), CTRL, 0xF, 0xF, false);
    int hi = __builtin_amdgcn_mov_dpp(__double2hiint(v), CTRL, 0xF, 0xF, false);
    return __hiloint2double(hi, lo);
}

// Lane exchange for cross-lane butterfly stage j (0..3) within a row.
template <int J>
__device__ __forceinline__ float xchg(float v)
{
    if constexpr (J == 0) return dpp_f32<DPP_XOR1>(v);
    else if constexpr (J == 1) return dpp_f32<DPP_XOR2>(v);
    else if constexpr (J == 2) return dpp_f32<DPP_XOR7>(v);
    else return dpp_f32<DPP_XOR15>(v);
}

template <int J>
__device__ __forceinline__ double xchg64(double v)
{
    if constexpr (J == 0) return dpp_f64<DPP_XOR1>(v);
    else if constexpr (J == 1) return dpp_f64<DPP_XOR2>(v);
    else if constexpr (J == 2) return dpp_f64<DPP_XOR7>(v);
    else return dpp_f64<DPP_XOR15>(v);
}

__device__ __forceinline__ int lane_chunk(int l16)
{
    int l0 = l16 & 1, l1 = (l16 >> 1) & 1, l2 = (l16 >> 2) & 1, l3 = (l16 >> 3) & 1;
    return (l0 ^ l2) | ((l1 ^ l2) << 1) | ((l2 ^ l3) << 2) | (l3 << 3);
}

// FWHT_Q of one segment held by a 16-lane row, NH = Q/128 chunks of 8 values
// per lane (segment position p = h*128 + chunk*8 + e).  Stages w = 1, 2, 4 are
// in-register, w = 8..64 one DPP exchange each (lower lane x + p, upper p - x),
// w >= 128 in-register across h: the stage order of the reference's FWHT
// (nar/extended_experiment.py:443-456), every stage one fp32 add or subtract.
template <int NH>
__device__ __forceinline__ void fwht_row(float (&v)[8 * NH], int chunk)
{
#pragma unroll
    for (int w = 1; w < 8; w <<= 1)
#pragma unroll
        for (int h = 0; h < NH; h++)
#pragma unroll
            for (int e = 0; e < 8; e++)
                if (!(e & w)) {
                    float x0 = v[h * 8 + e], x1 = v[h * 8 + e + w];
                    v[h * 8 + e] = x0 + x1;
                    v[h * 8 + e + w] = x0 - x1;
                }
    const float s0 = (chunk & 1) ? -1.0f : 1.0f;
    const float s1 = (chunk & 2) ? -1.0f : 1.0f;
    const float s2 = (chunk & 4) ? -1.0f : 1.0f;
    const float s3 = (chunk & 8) ? -1.0f : 1.0f;
#pragma unroll
    for (int i = 0; i < 8 * NH; i++) v[i] = __builtin_fmaf(s0, v[i], dpp_f32<DPP_XOR1>(v[i]));
#pragma unroll
    for (int i = 0; i < 8 * NH; i++) v[i] = __builtin_fmaf(s1, v[i], dpp_f32<DPP_XOR2>(v[i]));
#pragma unroll
    for (int i = 0; i < 8 * NH; i++) v[i] = __builtin_fmaf(s2, v[i], dpp_f32<DPP_XOR7>(v[i]));
#pragma unroll
    for (int i = 0; i < 8 * NH; i++) v[i] = __builtin_fmaf(s3, v[i], dpp_f32<DPP_XOR15>(v[i]));
#pragma unroll
    for (int wh = 1; wh < NH; wh <<= 1)
#pragma unroll
        for (int h = 0; h < NH; h++)
            if (!(h & wh))
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    float x0 = v[h * 8 + e], x1 = v[(h + wh) * 8 + e];
                    v[h * 8 + e] = x0 + x1;
                    v[(h + wh) * 8 + e] = x0 - x1;
                }
}

// The stages of fwht_row as separate steps, for kernels that interleave other
// work or take the cross-lane stages in the signed form below.  x arrives as
// NH uint4 words of 8 bf16 (element h*8 + e at offset h*128 + e of the lane's
// chunk).
template <int NH>
__device__ __forceinline__ void unpack_x(float (&v)[8 * NH], const uint4 (&xw)[NH])
{
#pragma unroll
    for (int h = 0; h < NH; h++) {
        v[h * 8 + 0] = bf16lo(xw[h].x); v[h * 8 + 1] = bf16hi(xw[h].x);
        v[h * 8 + 2] = bf16lo(xw[h].y); v[h * 8 + 3] = bf16hi(xw[h].y);
        v[h * 8 + 4] = bf16lo(xw[h].z); v[h * 8 + 5] = bf16hi(xw[h].z);
        v[h * 8 + 6] = bf16lo(xw[h].w); v[h * 8 + 7] = bf16hi(xw[h].w);
    }
}

// v *= signs (the lane's chunk of the segment starts at sg)
template <int NH>
__device__ __forceinline__ void apply_signs(float (&v)[8 * NH], const float *sg)
{
#pragma unroll
    for (int h = 0; h < NH; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) v[h * 8 + e] *= sg[h * 128 + e];
}

// stages of width 1, 2, 4 (within the lane's 8 consecutive positions)
template <int NH>
__device__ __forceinline__ void fwht_lane_stages(float (&v)[8 * NH])
{
#pragma unroll
    for (int w = 1; w < 8; w <<= 1)
#pragma unroll
        for (int h = 0; h < NH; h++)
#pragma unroll
            for (int e = 0; e < 8; e++)
                if (!(e & w)) {
                    float x0 = v[h * 8 + e], x1 = v[h * 8 + e + w];
                    v[h * 8 + e] = x0 + x1;
                    v[h * 8 + e + w] = x0 - x1;
                }
}

// stages of width 8 .. 64 across the 16 lanes of the row, IEEE form: the lower
// lane of a pair computes own + partner, the upper lane partner - own
// (sj[j] = -1 on lanes whose chunk bit j is set)
template <int NV>
__device__ __forceinline__ void fwht_xlane_plain(float (&v)[NV], const float (&sj)[4])
{
#pragma unroll
    for (int i = 0; i < NV; i++) v[i] = __builtin_fmaf(sj[0], v[i], dpp_f32<DPP_XOR1>(v[i]));
#pragma unroll
    for (int i = 0; i < NV; i++) v[i] = __builtin_fmaf(sj[1], v[i], dpp_f32<DPP_XOR2>(v[i]));
#pragma unroll
    for (int i = 0; i < NV; i++) v[i] = __builtin_fmaf(sj[2], v[i], dpp_f32<DPP_XOR7>(v[i]));
#pragma unroll
    for (int i = 0; i < NV; i++) v[i] = __builtin_fmaf(sj[3], v[i], dpp_f32<DPP_XOR15>(v[i]));
}

// The same stages as one v_fmac_f32 with a DPP source each: v + sj * partner.
// Every lane of a pair holds the same sign factor before a stage, so the lower
// lane gets sign * (a + b) and the upper lane -sign * (b - a): after the four
// stages v = sigma * (IEEE result), sigma = sj[0] sj[1] sj[2] sj[3], for every
// nonzero result (fma with a +-1 multiplier is one rounding of the same exact
// value, and RN is odd-symmetric).  A zero result can carry the wrong sign.
//
// Written as v_fmac_f32_dpp directly (the compiler keeps a separate DPP move).
// A DPP read of a VGPR needs 2 wait states after a VALU write of it: each block
// of 8 starts with s_nop 1, and within a stage every register is written once
// and read by DPP only in the next stage, 8 or more instructions later.
#define NARHIP_FMAC_DPP8(CTRL)                                                              \
    asm volatile("s_nop 1\n\t"                                                              \
                 "v_fmac_f32_dpp %0, %0, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"        \
                 "v_fmac_f32_dpp %1, %1, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"        \
                 "v_fmac_f32_dpp %2, %2, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"        \
                 "v_fmac_f32_dpp %3, %3, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"        \
                 "v_fmac_f32_dpp %4, %4, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"        \
                 "v_fmac_f32_dpp %5, %5, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"        \
                 "v_fmac_f32_dpp %6, %6, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"        \
                 "v_fmac_f32_dpp %7, %7, %8 " CTRL " row_mask:0xf bank_mask:0xf"            \
                 : "+v"(p[0]), "+v"(p[1]), "+v"(p[2]), "+v"(p[3]), "+v"(p[4]), "+v"(p[5]),   \
                   "+v"(p[6]), "+v"(p[7])                                                    \
                 : "v"(m))

template <int J>
__device__ __forceinline__ void fmac_dpp8(float *p, float m)
{
    if constexpr (J == 0) NARHIP_FMAC_DPP8("quad_perm:[1,0,3,2]");
    else if constexpr (J == 1) NARHIP_FMAC_DPP8("quad_perm:[2,3,0,1]");
    else if constexpr (J == 2) NARHIP_FMAC_DPP8("row_half_mirror");
    else NARHIP_FMAC_DPP8("row_mirror");
}
#undef NARHIP_FMAC_DPP8

template <int NV>
__device__ __forceinline__ void fwht_xlane_signed(float (&v)[NV], const float (&sj)[4])
{
    static_assert(NV % 8 == 0, "blocks of 8");
#pragma unroll
    for (int b = 0; b < NV; b += 8) fmac_dpp8<0>(v + b, sj[0]);
#pragma unroll
    for (int b = 0; b < NV; b += 8) fmac_dpp8<1>(v + b, sj[1]);
#pragma unroll
    for (int b = 0; b < NV; b += 8) fmac_dpp8<2>(v + b, sj[2]);
#pragma unroll
    for (int b = 0; b < NV; b += 8) fmac_dpp8<3>(v + b, sj[3]);
}

// stages of width 128 .. 64 NH (across the lane's NH chunks)
template <int NH>
__device__ __forceinline__ void fwht_h_stages(float (&v)[8 * NH])
{
#pragma unroll
    for (int wh = 1; wh < NH; wh <<= 1)
#pragma unroll
        for (int h = 0; h < NH; h++)
            if (!(h & wh))
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    float x0 = v[h * 8 + e], x1 = v[(h + wh) * 8 + e];
                    v[h * 8 + e] = x0 + x1;
                    v[(h + wh) * 8 + e] = x0 - x1;
                }
}

// Sum over the 16 lanes of a row in fp64; every lane receives the identical value.
__device__ __forceinline__ double row_sum64(double v)
{
    v += xchg64<0>(v);
    v += xchg64<1>(v);
    v += xchg64<2>(v);
    v += xchg64<3>(v);
    return v;
}

// Min/max over the lanes of a group of G8 chunks (G8 = 4, 8 or 16 lanes, the
// lanes whose chunk indices share chunk >> log2(G8)).  Exact in any order.
// fminf/fmaxf drop a NaN operand: the quantizers below use this form on the
// common path and detect NaN elements from their codes.
template <int G8>
__device__ __forceinline__ void group_minmax(float &lo, float &hi)
{
    lo = fminf(lo, xchg<0>(lo)); hi = fmaxf(hi, xchg<0>(hi));
    lo = fminf(lo, xchg<1>(lo)); hi = fmaxf(hi, xchg<1>(hi));
    if constexpr (G8 >= 8) { lo = fminf(lo, xchg<2>(lo)); hi = fmaxf(hi, xchg<2>(hi)); }
    if constexpr (G8 >= 16) { lo = fminf(lo, xchg<3>(lo)); hi = fmaxf(hi, xchg<3>(hi)); }
}

// NaN-propagating min/max, the semantics of torch.amin / torch.amax that the
// reference's quantizer reduces with (nar/experiment.py:166-167): a NaN
// operand wins.
__device__ __forceinline__ float min_nan(float a, float b) { return (b < a || b != b) ? b : a; }
__device__ __forceinline__ float max_nan(float a, float b) { return (b > a || b != b) ? b : a; }

template <int NV>
__device__ __forceinline__ void lane_minmax_nan(const float *v, float &lo, float &hi)
{
    lo = v[0]; hi = v[0];
#pragma unroll
    for (int e = 1; e < NV; e++) { lo = min_nan(lo, v[e]); hi = max_nan(hi, v[e]); }
}

template <int G8>
__device__ __forceinline__ void group_minmax_nan(float &lo, float &hi)
{
    lo = min_nan(lo, xchg<0>(lo)); hi = max_nan(hi, xchg<0>(hi));
    lo = min_nan(lo, xchg<1>(lo)); hi = max_nan(hi, xchg<1>(hi));
    if constexpr (G8 >= 8) { lo = min_nan(lo, xchg<2>(lo)); hi = max_nan(hi, xchg<2>(hi)); }
    if constexpr (G8 >= 16) { lo = min_nan(lo, xchg<3>(lo)); hi = max_nan(hi, xchg<3>(hi)); }
}

// ------------------------------------------------------------- quantizer --
//
// dynamic_asym_int4 group parameters (nar/experiment.py:166-181):
//   raw = (hi - lo) / 15 (fp32 division); s16 = fp16(raw > 0 ? raw : 1);
//   s16 <= 0 -> 1; z16 = fp16(lo).
// A NaN lo (a group holding a NaN) gives raw = NaN -> s16 = 1 and the
// canonical quiet NaN 0x7E00 as zero-point, whatever the NaN's sign or payload
// (torch's min reduction and fp16 conversion return that for +NaN and -NaN).
struct GroupParams {
    float s, z;
    uint16_t s16, z16;
};

// RN(d / 15) for d = hi - lo >= 0 (and +Inf, NaN) without a divide:
// q0 = d * RN(1/15), one Markstein correction q1 = fma(fma(-q0, 15, d), RN(1/15), q0)
// (Markstein, "Computation of elementary functions on the IBM RISC System/6000
// processor", IBM J. Res. Dev. 34(1), 1990), +Inf passed through.  Checked
// against the correctly rounded quotient for every non-negative fp32 pattern
// (tests/native/group_params_check.c): equal, or both below 2^-25 (fp16 zero).
__device__ __forceinline__ float div15(float d)
{
    constexpr float c = 0x1.111112p-4f;            // RN(1/15)
    const float q0 = d * c;
    const float r = __builtin_fmaf(-q0, 15.0f, d);
    const float q1 = __builtin_fmaf(r, c, q0);
    return d == __builtin_inff() ? d : q1;
}

// RN(1/s) for a positive fp16 scale s: one Newton step from the hardware
// reciprocal (within one ulp), equal to RN(1/s) for every fp16 s
// (tests/native/group_params_check.c).  s = +Inf gives NaN, which sends every
// code of its group to the exact path.
__device__ __forceinline__ float recip_scale(float s)
{
    const float r0 = __builtin_amdgcn_rcpf(s);
    const float e = __builtin_fmaf(-s, r0, 1.0f);
    return __builtin_fmaf(e, r0, r0);
}

__device__ __forceinline__ GroupParams group_params(float lo, float hi)
{
    GroupParams g;
    float raw = div15(hi - lo);
    float sr = raw > 0.0f ? raw : 1.0f;
    uint16_t sh = f32_to_f16_bits(sr);
    if (!(f16_bits_to_f32(sh) > 0.0f)) sh = 0x3c00u;
    uint16_t zh = lo != lo ? (uint16_t)0x7e00u : f32_to_f16_bits(lo);
    g.s16 = sh; g.z16 = zh;
    g.s = f16_bits_to_f32(sh);
    g.z = f16_bits_to_f32(zh);
    return g;
}

// q = clamp(round_half_even((x - z) / s), 0, 15) with the fp32 subtraction and
// the correctly rounded fp32 division of the reference.  A NaN quotient
// (NaN input or zero-point, Inf - Inf, Inf / Inf) gives code 0, the uint8
// conversion of the reference's NaN.
__device__ __forceinline__ uint32_t quant_code(float x, const GroupParams &g)
{
    float d = x - g.z;
    float q = __builtin_rintf(d / g.s);
    q = fminf(fmaxf(q, 0.0f), 15.0f);
    return (uint32_t)q;
}

// The same code from y = (x - z) * RN(1/s).  y is within 2^-23 |d/s| of the
// exact quotient and RN(d/s) within 2^-24 |d/s|, so below 16 both round to the
// same integer unless y lies within 2^-18 of a half-integer; such lanes set
// `flag` and the caller recomputes with quant_code.  (Half-integers at or above
// 15.5 and below 0.5 clamp to the same code either way.)  The comparison is
// written so that a NaN y also sets `flag`: a group holding a NaN element
// passed the NaN-dropping min/max of the common path, and the caller's slow
// path recomputes its parameters with the NaN-propagating reduction.
__device__ __forceinline__ uint32_t quant_code_fast(float x, float z, float rs, bool &flag)
{
    const float y = (x - z) * rs;
    const float r = __builtin_rintf(y);
    flag |= !(__builtin_fabsf(y - r) < 0.5f - 0x1p-18f);
    return (uint32_t)fminf(fmaxf(r, 0.0f), 15.0f);
}

// Eight codes of one lane packed into a 32-bit word (nibble e = element e).
__device__ __forceinline__ uint32_t quant_word8_exact(const float *v, const GroupParams &g)
{
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) word |= quant_code(v[e], g) << (4 * e);
    return word;
}

__device__ __forceinline__ uint32_t quant_word8_fast(const float *v, const GroupParams &g, bool &flag)
{
    const float rs = recip_scale(g.s);
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) word |= quant_code_fast(v[e], g.z, rs, flag) << (4 * e);
    return word;
}

// One lane's 8 values of a group that spans G8 lanes of a row (group_minmax):
// the group parameters in g and the lane's packed codes.  Bit-identical to the
// reference quantizer: the common path reduces with fminf/fmaxf and takes the
// codes from the reciprocal; a wave holding a near-tie or a NaN element redoes
// the reduction with NaN propagation, the parameters and the exact codes.
// Every lane of the wave must call it (cross-lane moves, wave-uniform branch).
template <int G8>
__device__ __forceinline__ uint32_t quant_group8(const float *v, GroupParams &g)
{
    float lo = v[0], hi = v[0];
#pragma unroll
    for (int e = 1; e < 8; e++) { lo = fminf(lo, v[e]); hi = fmaxf(hi, v[e]); }
    group_minmax<G8>(lo, hi);
    g = group_params(lo, hi);
    bool flag = false;
    uint32_t word = quant_word8_fast(v, g, flag);
    if (__builtin_expect(__any(flag), 0)) {
        lane_minmax_nan<8>(v, lo, hi);
        group_minmax_nan<G8>(lo, hi);
        g = group_params(lo, hi);
        word = quant_word8_exact(v, g);
    }
    return word;
}

// The hooks' tuple for one lane's 8 consecutive elements of a group
// (dynamic_asym_int4, nar/experiment.py:158-184): the codes of `word` unpacked
// one per byte, and deq = RN(RN(q s) + z) in fp32 -- NaN where the reference's
// quotient (x - z) / s is NaN (NaN x or zero-point, Inf - Inf, Inf / Inf with an
// infinite scale), whose code is 0.  codes 8-byte and deq 16-byte aligned.
__device__ __forceinline__ void store_tuple8(const float *v, const GroupParams &g, uint32_t word, uint8_t *codes,
                                             float *deq)
{
    float d[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float r = v[e] - g.z;
        const bool nanq = r != r || (__builtin_isinf(r) && __builtin_isinf(g.s));
        const float q = (float)((word >> (4 * e)) & 15u);
        d[e] = nanq ? __builtin_nanf("") : __fadd_rn(__fmul_rn(q, g.s), g.z);
    }
    // nibble pairs -> one byte each: 0x0000000H -> byte lanes
    const uint32_t lo = (word & 0xfu) | ((word & 0xf0u) << 4) | ((word & 0xf00u) << 8) | ((word & 0xf000u) << 12);
    const uint32_t w2 = word >> 16;
    const uint32_t hi = (w2 & 0xfu) | ((w2 & 0xf0u) << 4) | ((w2 & 0xf00u) << 8) | ((w2 & 0xf000u) << 12);
    *reinterpret_cast<uint2 *>(codes) = make_uint2(lo, hi);
    float4 *o = reinterpret_cast<float4 *>(deq);
    o[0] = make_float4(d[0], d[1], d[2], d[3]);
    o[1] = make_float4(d[4], d[5], d[6], d[7]);
}

// ------------------------------------------------- division by fp32(sqrt Q) --
//
// v[i] <- RN(v[i] / c) with c = fp32(sqrt(Q)), rc = RN(1/c).
// Q a power of 4: c is a power of two and RN(v * rc) is the quotient.
// Q = 128 and 512: RN(v / c) = fma(v, H, RN(v * L)) with 1/c split as H =
// RN(1/c), L = RN(1/c - H) (multiplication by a constant in two pieces,
// Brisebarre and Muller, "Correctly rounded multiplication by arbitrary
// precision constants", IEEE Trans. Computers 57(2), 2008), checked against
// the correctly rounded fp32 quotient for every finite fp32 v of both signs:
// equal for all |v| >= 2^-90 (below, v * L is subnormal).  Two operations.
// Otherwise q0 = v*rc, r = fma(q0, c, -v), q1 = fma(-r, rc, q0), checked the
// same way for Q in {2, 8, 12, 28, 32, 128, 512, 2048}: equal for all
// |v| >= 2^-100.  A wave holding any |v| below the bound (zeros included)
// takes the division instead.
template <int Q> struct RecipSqrtQ { static constexpr bool split = false; static constexpr float hi = 0, lo = 0; };
template <> struct RecipSqrtQ<128> {
    static constexpr bool split = true;
    static constexpr float hi = 0x1.6a09e6p-4f, lo = 0x1.9fcef4p-29f;
};
template <> struct RecipSqrtQ<512> {
    static constexpr bool split = true;
    static constexpr float hi = 0x1.6a09e6p-5f, lo = 0x1.9fcef4p-30f;
};
// smallest |v| for which the shortcut of div_sqrt_q_fast<Q> is exact
template <int Q> constexpr float div_sqrt_q_min() { return RecipSqrtQ<Q>::split ? 0x1p-90f : 0x1p-100f; }

template <int Q, int NV>
__device__ __forceinline__ void div_sqrt_q(float (&v)[NV], float c, float rc)
{
    constexpr bool pow4 = (Q & (Q - 1)) == 0 && (Q & 0x55555555) == Q;
    if constexpr (pow4) {
#pragma unroll
        for (int i = 0; i < NV; i++) v[i] *= rc;
    } else {
        bool tiny = false;
#pragma unroll
        for (int i = 0; i < NV; i++) tiny |= __builtin_fabsf(v[i]) < div_sqrt_q_min<Q>();
        if (__builtin_expect(__any(tiny), 0)) {
#pragma unroll
            for (int i = 0; i < NV; i++) v[i] = v[i] / c;
        } else if constexpr (RecipSqrtQ<Q>::split) {
#pragma unroll
            for (int i = 0; i < NV; i++) v[i] = __builtin_fmaf(v[i], RecipSqrtQ<Q>::hi, v[i] * RecipSqrtQ<Q>::lo);
        } else {
#pragma unroll
            for (int i = 0; i < NV; i++) {
                const float q0 = v[i] * rc;
                const float r = __builtin_fmaf(q0, c, -v[i]);
                v[i] = __builtin_fmaf(-r, rc, q0);
            }
        }
    }
}

// RN(v / c) without the range check of div_sqrt_q: every |v| must be >=
// div_sqrt_q_min<Q>() (or Q a power of 4).  c and rc may carry a common sign
// (c = sigma fp32(sqrt Q), rc = sigma RN(1/fp32(sqrt Q))): then the result is
// RN((sigma v) / fp32(sqrt Q)) (RN is odd-symmetric, so the split constants
// take the sign of rc).
template <int Q, int NV>
__device__ __forceinline__ void div_sqrt_q_fast(float (&v)[NV], float c, float rc)
{
    constexpr bool pow4 = (Q & (Q - 1)) == 0 && (Q & 0x55555555) == Q;
    if constexpr (pow4) {
#pragma unroll
        for (int i = 0; i < NV; i++) v[i] *= rc;
    } else if constexpr (RecipSqrtQ<Q>::split) {
        const float hi = __builtin_copysignf(RecipSqrtQ<Q>::hi, rc);
        const float lo = __builtin_copysignf(RecipSqrtQ<Q>::lo, rc);
#pragma unroll
        for (int i = 0; i < NV; i++) v[i] = __builtin_fmaf(v[i], hi, v[i] * lo);
    } else {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const float q0 = v[i] * rc;
            const float r = __builtin_fmaf(q0, c, -v[i]);
            v[i] = __builtin_fmaf(-r, rc, q0);
        }
    }
}

// FWHT_128 of a 16-lane row (8 values per lane) and RN(v / fp32(sqrt 128)),
// bit-identical to fwht_row<1> followed by div_sqrt_q<128>: the cross-lane
// stages in the signed form (one v_fmac_f32_dpp per value instead of a DPP move
// and an fma) with sigma folded into the split-constant division.  A wave in
// which any result is below div_sqrt_q_min (zeros, whose sign can differ in
// the signed form) or NaN redoes its rows from the input with the plain stages
// and the checked division.
__device__ __forceinline__ void fwht128_div(float (&v)[8], int chunk, float sq, float rsq)
{
    float in[8];
#pragma unroll
    for (int i = 0; i < 8; i++) in[i] = v[i];
    const float sj[4] = {(chunk & 1) ? -1.0f : 1.0f, (chunk & 2) ? -1.0f : 1.0f, (chunk & 4) ? -1.0f : 1.0f,
                         (chunk & 8) ? -1.0f : 1.0f};
    fwht_lane_stages<1>(v);
    fwht_xlane_signed(v, sj);
    bool odd = false;
#pragma unroll
    for (int i = 0; i < 8; i++) odd |= !(__builtin_fabsf(v[i]) >= div_sqrt_q_min<128>());
    if (__builtin_expect(__any(odd), 0)) {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = in[i];
        fwht_row<1>(v, chunk);
        div_sqrt_q<128>(v, sq, rsq);
    } else {
        const float sigma = sj[0] * sj[1] * sj[2] * sj[3];
        div_sqrt_q_fast<128>(v, sigma * sq, sigma * rsq);
    }
}

// ----------------------------------------------------------------- Paley --

// Rows of the +-1 Paley matrices as bit masks: bit a' of row a set <=> entry -1.
// Filled from the construction of the reference (Paley I over Z_11 for 12,
// over GF(27) for 28) by the host at library load.
struct PaleyTable {
    uint32_t neg[28];
};

}  // namespace narhip
