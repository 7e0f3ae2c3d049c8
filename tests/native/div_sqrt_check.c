/* Scan of the constant division used by the FWHT normalisation kernels.
 *
 * For c = fp32(sqrt(Q)) and rc = RN(1/c) the kernels compute
 *     q0 = v * rc;  r = fma(q0, c, -v);  q1 = fma(-r, rc, q0)
 * and fall back to the IEEE division when |v| < 2^-100.  This program compares
 * that against the correctly rounded quotient v / c, bit for bit, for every
 * finite fp32 bit pattern congruent to `phase` modulo `stride` (stride 1 scans
 * all 2^32 patterns, about ten seconds per Q).
 *
 * usage: div_sqrt_check STRIDE PHASE Q...   prints "Q mismatches checked" lines
 *
 * Split-constant form (Q = 128, 512): the kernels compute fma(v, HI, v * LO)
 * with 1/c = HI + LO split in two fp32 pieces, and fall back to the IEEE
 * division when |v| < 2^-90:
 *        div_sqrt_check split STRIDE PHASE Q HI LO   (HI, LO as C float literals)
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static int split_scan(int argc, char **argv)
{
    if (argc != 7) return 2;
    const uint64_t stride = strtoull(argv[2], 0, 10), phase = strtoull(argv[3], 0, 10);
    const int q = atoi(argv[4]);
    const float c = (float)sqrt((double)q), hi = strtof(argv[5], 0), lo = strtof(argv[6], 0);
    uint64_t bad = 0, checked = 0;
    for (uint64_t u = phase; u <= 0xffffffffull; u += stride) {
        if (((uint32_t)u & 0x7f800000u) == 0x7f800000u) continue;
        const float v = from_bits((uint32_t)u);
        const float got = fabsf(v) < 0x1p-90f ? v / c : fmaf(v, hi, v * lo);
        checked++;
        if (to_bits(got) != to_bits(v / c)) bad++;
    }
    printf("%d %llu %llu\n", q, (unsigned long long)bad, (unsigned long long)checked);
    return 0;
}

int main(int argc, char **argv)
{
    if (argc > 1 && strcmp(argv[1], "split") == 0) return split_scan(argc, argv);
    if (argc < 4) return 2;
    const uint64_t stride = strtoull(argv[1], 0, 10), phase = strtoull(argv[2], 0, 10);
    for (int a = 3; a < argc; a++) {
        const int q = atoi(argv[a]);
        const float c = (float)sqrt((double)q), rc = 1.0f / c;
        uint64_t bad = 0, checked = 0;
        for (uint64_t u = phase; u <= 0xffffffffull; u += stride) {
            if (((uint32_t)u & 0x7f800000u) == 0x7f800000u) continue;
            const float v = from_bits((uint32_t)u);
            float got;
            if (fabsf(v) < 0x1p-100f) {
                got = v / c;
            } else {
                const float q0 = v * rc;
                const float r = fmaf(q0, c, -v);
                got = fmaf(-r, rc, q0);
            }
            checked++;
            if (to_bits(got) != to_bits(v / c)) bad++;
        }
        printf("%d %llu %llu\n", q, (unsigned long long)bad, (unsigned long long)checked);
    }
    return 0;
}
