// The hooks' quantizer as a standalone GPU operator: dynamic_asym_int4
// (nar/experiment.py:158-184) on any [rows, n] input of fp32, bf16 or fp16,
// returning its tuple layout -- dequantized values in the input dtype, fp16
// scale and zero per group, and the codes unpacked, one byte per element.
//
// Arithmetic as the reference: the input converted to fp32 (exact), group
// min/max, raw = (hi - lo) / 15, both degenerate-group guards, fp16 RNE of scale
// and zero, q = clamp(round_half_even(RN(x - z) / s), 0, 15), deq = RN(q * s) + z
// rounded once to the input dtype.
#pragma once
#include "narhip_device.hpp"

namespace narhip {

enum : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

template <int DT>
__device__ __forceinline__ void load8(const void *p, int64_t i, float (&v)[8])
{
    if constexpr (DT == DT_F32) {
        const float4 *q = reinterpret_cast<const float4 *>(static_cast<const float *>(p) + i);
        const float4 a = q[0], b = q[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const uint4 w = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(p) + i);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if constexpr (DT == DT_BF16) {
                v[2 * j] = bf16lo(ws[j]);
                v[2 * j + 1] = bf16hi(ws[j]);
            } else {
                v[2 * j] = f16_bits_to_f32((uint16_t)(ws[j] & 0xffffu));
                v[2 * j + 1] = f16_bits_to_f32((uint16_t)(ws[j] >> 16));
            }
        }
    }
}

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet)
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f)
{
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

template <int DT>
__device__ __forceinline__ void store8(void *p, int64_t i, const float (&v)[8])
{
    if constexpr (DT == DT_F32) {
        float4 *q = reinterpret_cast<float4 *>(static_cast<float *>(p) + i);
        q[0] = make_float4(v[0], v[1], v[2], v[3]);
        q[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
        uint32_t ws[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if constexpr (DT == DT_BF16)
                ws[j] = f32_to_bf16_bits(v[2 * j]) | (f32_to_bf16_bits(v[2 * j + 1]) << 16);
            else
                ws[j] = (uint32_t)f32_to_f16_bits(v[2 * j]) | ((uint32_t)f32_to_f16_bits(v[2 * j + 1]) << 16);
        }
        *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(p) + i) = make_uint4(ws[0], ws[1], ws[2], ws[3]);
    }
}

// One lane per 8 consecutive elements; a group of B elements is B/8 adjacent
// lanes (B/8 <= 64), reduced with butterflies over those lanes.
template <int DT>
__global__ void __launch_bounds__(256)
quant_tuple_kernel(const void *x, int64_t elems, int group, uint8_t *codes, uint16_t *scales, uint16_t *zeros,
                   void *deq)
{
    const int64_t chunk = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t nchunks = elems / 8;
    const bool ok = chunk < nchunks;
    const int64_t c = ok ? chunk : nchunks - 1;
    float v[8];
    load8<DT>(x, c * 8, v);
    // torch.amin / torch.amax semantics: a NaN anywhere in the group wins
    float lo, hi;
    lane_minmax_nan<8>(v, lo, hi);
    const int lanes = group / 8;
    for (int off = 1; off < lanes; off <<= 1) {
        lo = min_nan(lo, __shfl_xor(lo, off));
        hi = max_nan(hi, __shfl_xor(hi, off));
    }
    const GroupParams g = group_params(lo, hi);
    uint32_t q[8];
    float d[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        q[e] = quant_code(v[e], g);
        // the reference dequantizes the clamped float quotient, which stays NaN
        // where (x - z) / s is NaN (Inf - Inf, Inf / Inf); its uint8 code is 0
        const float quo = __builtin_rintf((v[e] - g.z) / g.s);
        d[e] = quo != quo ? quo : __fadd_rn(__fmul_rn((float)q[e], g.s), g.z);
    }
    if (!ok) return;
    const uint32_t lo4 = q[0] | (q[1] << 8) | (q[2] << 16) | (q[3] << 24);
    const uint32_t hi4 = q[4] | (q[5] << 8) | (q[6] << 16) | (q[7] << 24);
    *reinterpret_cast<uint2 *>(codes + c * 8) = make_uint2(lo4, hi4);
    store8<DT>(deq, c * 8, d);
    if ((c % lanes) == 0) {
        const int64_t gi = c / lanes;
        scales[gi] = g.s16;
        zeros[gi] = g.z16;
    }
}

}  // namespace narhip
