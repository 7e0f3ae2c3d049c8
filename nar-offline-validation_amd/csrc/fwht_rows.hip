// Full-row Walsh-Hadamard transform of power-of-two rows wider than one
// segment kernel row (n = 2^L, 2048 <= n <= 8192): the branch of
// _full_hadamard_rows for power-of-two widths (nar/extended_experiment.py:
// 443-456,475-478), the widths of the Llama-3.1-8B hidden state (4096) and
// the Llama-3.2-3B down_proj input (8192).
//
// One workgroup of 256 threads per row; each thread holds E = n/256 values.
// The index bits are taken in passes of log2(E) bits from the lowest up: in
// pass [b0, b0+r) a thread holds the values whose index differs only in those
// bits (and in bits its other registers cover), and applies the butterfly
// stages of widths 2^b0, ..., 2^(b0+r-1) in increasing order; between passes
// the row goes through LDS.  Every butterfly (a + b, a - b) of the reference's
// stage order is applied exactly once and in order, so the result is the
// reference's fp32 FWHT bit for bit; then RN(v / fp32(sqrt n)).
//
// Outputs (any combination): the rotated fp32 row, and either the packed INT4
// row of the fused quantizer (codes [rows, n/2], fp16 scales / zeros) or the
// hooks' tuple (codes unpacked [rows, n], fp32 dequantized row).
#pragma once
#include "narhip_device.hpp"

namespace narhip {

struct FwhtArgs {
    const uint16_t *x;      // bf16 [T, ldx]
    int64_t ldx, T;
    const float *signs;     // [n] or null
    float *rotated;         // fp32 [T, n] or null
    uint8_t *codes;         // packed [rows, n/2], or unpacked [rows, n] when deq is set; null: no quantizer
    uint16_t *scales;       // fp16 [rows, n/B]
    uint16_t *zeros;
    float *deq;             // fp32 [rows, n] (tuple output) or null
    const int64_t *dest;    // [T] output row per token, or null
    float sq, rsq;          // fp32(sqrt(n)), RN(1/sq)
};

// LDS position of row index i: bits 0-4 flipped by bits 5-9, so that the
// strided accesses of every pass and the 8-element chunk reads of the output
// stage spread over the 32 banks.
__device__ __forceinline__ int fw_swz(int i) { return i ^ ((i >> 5) & 31); }

// Index held in register j of thread t during the pass over bits [B0, B0+R)
// (E = 2^(L-8) registers): the low R bits of j select bits [B0, B0+R); the
// other bits of j and the 8 bits of t fill the remaining index bits in order.
template <int L, int B0, int R>
__device__ __forceinline__ int fw_index(int t, int j)
{
    const int jl = j & ((1 << R) - 1);
    const int o = t + 256 * (j >> R);
    return (o & ((1 << B0) - 1)) | (jl << B0) | ((o >> B0) << (B0 + R));
}

template <int E, int R>
__device__ __forceinline__ void fw_stages(float (&v)[E])
{
#pragma unroll
    for (int w = 1; w < (1 << R); w <<= 1)
#pragma unroll
        for (int j = 0; j < E; j++)
            if (!(j & w)) {
                const float a = v[j], b = v[j + w];
                v[j] = a + b;
                v[j + w] = a - b;
            }
}

// Passes over bits [B0, L) after the first: store under the previous pass's
// mapping, reload under this one, apply its stages.
template <int L, int PB0, int PR, int B0>
__device__ __forceinline__ void fw_passes(float (&v)[1 << (L - 8)], float *lds, int t)
{
    constexpr int E = 1 << (L - 8);
    constexpr int e = L - 8;
    if constexpr (B0 < L) {
        constexpr int R = (L - B0) < e ? (L - B0) : e;
#pragma unroll
        for (int j = 0; j < E; j++) lds[fw_swz(fw_index<L, PB0, PR>(t, j))] = v[j];
        __syncthreads();
#pragma unroll
        for (int j = 0; j < E; j++) v[j] = lds[fw_swz(fw_index<L, B0, R>(t, j))];
        __syncthreads();
        fw_stages<E, R>(v);
        fw_passes<L, B0, R, B0 + R>(v, lds, t);
    } else {
        // final: the row back to LDS in natural order for the output stage
#pragma unroll
        for (int j = 0; j < E; j++) lds[fw_swz(fw_index<L, PB0, PR>(t, j))] = v[j];
        __syncthreads();
    }
}

template <int L, int B>
__global__ void __launch_bounds__(256)
fwht_rows_kernel(FwhtArgs a)
{
    constexpr int N = 1 << L;
    constexpr int E = N / 256;
    constexpr int e = L - 8;
    constexpr int G8 = B / 8;
    static_assert(L >= 11 && L <= 13, "2048 <= n <= 8192");
    __shared__ float lds[N];
    const int t = threadIdx.x;
    const int64_t row = blockIdx.x;

    // ---- pass 0: E consecutive values per thread (16-byte bf16 loads)
    float v[E];
    const uint16_t *xr = a.x + row * a.ldx + t * E;
#pragma unroll
    for (int h = 0; h < E / 8; h++) {
        const uint4 w = *reinterpret_cast<const uint4 *>(xr + 8 * h);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[8 * h + 2 * i] = bf16lo(ws[i]);
            v[8 * h + 2 * i + 1] = bf16hi(ws[i]);
        }
    }
    if (a.signs) {
#pragma unroll
        for (int j = 0; j < E; j++) v[j] *= a.signs[t * E + j];
    }
    fw_stages<E, e>(v);
    fw_passes<L, 0, e, e>(v, lds, t);

    // ---- output stage: chunk c * 256 + t of 8 consecutive values
    const int64_t orow = a.dest ? a.dest[row] : row;
#pragma unroll
    for (int c = 0; c < E / 8; c++) {
        const int pos = (c * 256 + t) * 8;
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; i++) y[i] = lds[fw_swz(pos + i)];
        div_sqrt_q<N>(y, a.sq, a.rsq);
        if (a.rotated) {
            float4 *o = reinterpret_cast<float4 *>(a.rotated + row * N + pos);
            o[0] = make_float4(y[0], y[1], y[2], y[3]);
            o[1] = make_float4(y[4], y[5], y[6], y[7]);
        }
        if (a.codes) {
            GroupParams g;
            const uint32_t word = quant_group8<G8>(y, g);
            if (a.deq)
                store_tuple8(y, g, word, a.codes + orow * N + pos, a.deq + orow * N + pos);
            else
                *reinterpret_cast<uint32_t *>(a.codes + orow * (N / 2) + pos / 2) = word;
            if ((t & (G8 - 1)) == 0) {
                const int64_t gi = orow * (N / B) + pos / B;
                a.scales[gi] = g.s16;
                a.zeros[gi] = g.z16;
            }
        }
    }
}

}  // namespace narhip
