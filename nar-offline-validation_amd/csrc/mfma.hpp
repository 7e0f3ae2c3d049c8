// bf16 MFMA building blocks (gfx950 v_mfma_f32_16x16x32_bf16).
//
// Operand mapping used by every kernel (lane l of a wave64, g = l / 16):
//   A (16 x 32, M x K):  lane l supplies row m = l % 16, K slots 8g .. 8g+7
//   B (32 x 16, K x N):  lane l supplies column n = l % 16, K slots 8g .. 8g+7
//   D (16 x 16):         lane l holds D[4g + i][l % 16], i = 0..3
// A and B use the same K-slot numbering, so the contraction is over matching
// slots whatever order the hardware sums them in.  narhip_mfma_probe() checks
// the mapping on the device.
//
// fp32 values enter the bf16 MFMA as three bf16 terms hi + mid + lo whose sum
// is the fp32 value exactly (8 + 8 + 8 significant bits, each split step
// exact), so every product of a term with a bf16 (or +-1) operand is exact.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace narhip {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma_bf16(bf16x8 a, bf16x8 b, floatx4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ floatx4 zero4()
{
    floatx4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    return z;
}

// x = h + m + l exactly (bf16 conversions round to nearest even).
__device__ __forceinline__ void split3(float x, __bf16 &h, __bf16 &m, __bf16 &l)
{
    h = (__bf16)x;
    const float r1 = x - (float)h;
    m = (__bf16)r1;
    const float r2 = r1 - (float)m;
    l = (__bf16)r2;
}

__device__ __forceinline__ void split3x8(const float (&x)[8], bf16x8 &h, bf16x8 &m, bf16x8 &l)
{
#pragma unroll
    for (int j = 0; j < 8; j++) {
        __bf16 a, b, c;
        split3(x[j], a, b, c);
        h[j] = a; m[j] = b; l[j] = c;
    }
}

__device__ __forceinline__ bf16x8 load_bf16x8(const __bf16 *p)
{
    return *reinterpret_cast<const bf16x8 *>(p);
}

}  // namespace narhip
