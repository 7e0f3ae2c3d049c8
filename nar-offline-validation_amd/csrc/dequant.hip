// Dequantization of the packed INT4 layout: out = q * s + z, computed as an
// fp32 multiply followed by an fp32 add (no fused multiply-add), as
// nar/kernels/r4_fused_v2.py:364-369 and nar/experiment.py:183 do.
#pragma once
#include "narhip_device.hpp"

namespace narhip {

// One thread per 8 channels (one 32-bit word of codes).
template <int = 0>
__global__ void __launch_bounds__(256)
dequant_kernel(const uint8_t *codes, const uint16_t *scales, const uint16_t *zeros,
               int64_t rows, int64_t n, int group, float *out)
{
    const int64_t w = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (w >= rows * n / 8) return;
    const int64_t r = (w * 8) / n;
    const int64_t c = (w * 8) % n;
    const uint32_t word = reinterpret_cast<const uint32_t *>(codes)[w];
    const int64_t gi = r * (n / group) + c / group;
    const float s = f16_bits_to_f32(scales[gi]);
    const float z = f16_bits_to_f32(zeros[gi]);
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float q = (float)((word >> (4 * e)) & 15u);
        const float prod = __fmul_rn(q, s);
        o[e] = __fadd_rn(prod, z);
    }
    float4 *d = reinterpret_cast<float4 *>(out + r * n + c);
    d[0] = make_float4(o[0], o[1], o[2], o[3]);
    d[1] = make_float4(o[4], o[5], o[6], o[7]);
}

}  // namespace narhip
