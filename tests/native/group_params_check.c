/* Scans of the two divisions of the quantizer's group parameters as the
 * kernels compute them (narhip_device.hpp: div15, recip_scale).
 *
 * div15: raw = RN(d / 15) for the group range d = hi - lo >= 0 by
 *     q0 = d * c;  r = fma(-q0, 15, d);  q1 = fma(r, c, q0),   c = RN(1/15)
 * (Markstein's correction step), with d = +Inf passed through.  Compared bit
 * for bit with the correctly rounded quotient d / 15.0f for every
 * non-negative fp32 pattern (finite, subnormal, +Inf, NaN) congruent to
 * PHASE modulo STRIDE; a difference is allowed only where both round to the
 * same fp16 value below 2^-24 (the kernels only use fp16(raw), and a raw
 * that small gives fp16 zero either way).
 *
 * recip: rs = fma(fma(-s, r0, 1), r0, r0), one Newton step from a
 * reciprocal r0 within one ulp of 1/s (the hardware v_rcp_f32), for every
 * positive finite fp16 scale s, with r0 = RN(1/s) and its two neighbours:
 * rs must equal RN(1/s) in every case.
 *
 * usage: group_params_check STRIDE PHASE [naive]   prints "div15 mismatches
 *        checked" and "recip mismatches checked"; `naive` drops the correction
 *        steps (q0 and r0 alone), the planted mistake a test must see fail.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static int naive = 0;

static float div15(float d)
{
    const float c = (float)(1.0 / 15.0);
    const float q0 = d * c;
    const float r = fmaf(-q0, 15.0f, d);
    const float q1 = fmaf(r, c, q0);
    return naive ? q0 : (d == INFINITY ? d : q1);
}

static float f16_to_f32(uint16_t h)
{
    const uint32_t e = (h >> 10) & 31, m = h & 1023;
    float v = e == 0 ? ldexpf((float)m, -24) : e == 31 ? (m ? NAN : INFINITY) : ldexpf((float)(m | 1024), (int)e - 25);
    return (h & 0x8000) ? -v : v;
}

int main(int argc, char **argv)
{
    if (argc != 3 && argc != 4) return 2;
    naive = argc == 4;
    const uint64_t stride = strtoull(argv[1], 0, 10), phase = strtoull(argv[2], 0, 10);
    uint64_t bad = 0, checked = 0;
    for (uint64_t u = phase; u <= 0x7fffffffull; u += stride) {
        const float d = from_bits((uint32_t)u);
        const float want = d / 15.0f, got = div15(d);
        checked++;
        if (isnan(want) && isnan(got)) continue;
        if (to_bits(want) == to_bits(got)) continue;
        if (fabsf(want) < 0x1p-25f && fabsf(got) < 0x1p-25f) continue;   /* both fp16 zero */
        if (bad < 5) fprintf(stderr, "div15 d=%a want %a got %a\n", d, want, got);
        bad++;
    }
    printf("div15 %llu %llu\n", (unsigned long long)bad, (unsigned long long)checked);
    uint64_t rbad = 0, rchecked = 0;
    for (uint32_t h = 1; h < 0x7c00; h++) {
        const float s = f16_to_f32((uint16_t)h);
        const float want = 1.0f / s;
        const float cand[3] = {nextafterf(want, 0.0f), want, nextafterf(want, INFINITY)};
        for (int i = 0; i < 3; i++) {
            const float r0 = cand[i];
            const float e = fmaf(-s, r0, 1.0f);
            const float rs = naive ? r0 : fmaf(e, r0, r0);
            rchecked++;
            if (to_bits(rs) != to_bits(want)) {
                if (rbad < 5) fprintf(stderr, "recip s=%a r0=%a got %a want %a\n", s, r0, rs, want);
                rbad++;
            }
        }
    }
    printf("recip %llu %llu\n", (unsigned long long)rbad, (unsigned long long)rchecked);
    return 0;
}
