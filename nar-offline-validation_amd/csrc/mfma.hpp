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

// The same decomposition by truncation, for eight values at once: h is x with
// the low 16 bits cleared (a bf16 value), r = x - h is exact, m is r with its
// low 16 bits cleared, l = r - m is exact and has at most 8 significant bits,
// so the upper halves of h, m and l are the three bf16 terms.  Packing takes
// the upper halves of two fp32 words per v_perm_b32.
__device__ __forceinline__ void split3x8_trunc(const float (&x)[8], bf16x8 &h, bf16x8 &m, bf16x8 &l)
{
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 hw, mw, lw;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const uint32_t ua = __float_as_uint(x[2 * d]), ub = __float_as_uint(x[2 * d + 1]);
        const float ra = x[2 * d] - __uint_as_float(ua & 0xffff0000u);
        const float rb = x[2 * d + 1] - __uint_as_float(ub & 0xffff0000u);
        const uint32_t ura = __float_as_uint(ra), urb = __float_as_uint(rb);
        const float la = ra - __uint_as_float(ura & 0xffff0000u);
        const float lb = rb - __uint_as_float(urb & 0xffff0000u);
        hw[d] = __builtin_amdgcn_perm(ub, ua, 0x07060302u);
        mw[d] = __builtin_amdgcn_perm(urb, ura, 0x07060302u);
        lw[d] = __builtin_amdgcn_perm(__float_as_uint(lb), __float_as_uint(la), 0x07060302u);
    }
    h = __builtin_bit_cast(bf16x8, hw);
    m = __builtin_bit_cast(bf16x8, mw);
    l = __builtin_bit_cast(bf16x8, lw);
}

__device__ __forceinline__ bf16x8 load_bf16x8(const __bf16 *p)
{
    return *reinterpret_cast<const bf16x8 *>(p);
}

}  // namespace narhip
