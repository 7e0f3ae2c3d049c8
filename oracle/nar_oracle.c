/*
 * CPU oracle for the NAR online rotate-and-quantize path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the restatement that the HIP kernels
 * are compared against; it is never linked into, loaded by or called from the
 * product library.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may use it.
 *
 * It restates, in plain C, the reference's PyTorch arithmetic for the path:
 *
 *   x'  = H_s x - (x Y') W''^T           (reference row form; U = -W'', V = Y')
 *   H_s = (H_m (x) H_q) diag(s)           Kronecker Walsh-Hadamard, optional signs
 *   INT4 = dynamic_asym_int4(x', b)       per-token groups of b channels
 *
 * Every arithmetic step the reference pins is reproduced operation for
 * operation in fp32:
 *   - FWHT stage order and butterfly (a+b, a-b) at widths 1, 2, 4, ..., q/2:
 *       nar/extended_experiment.py:443-456 (_fast_walsh_hadamard),
 *       nar/kernels/r4_fused_v2.py:33-52 (_fwht_stage), quarot-llama3/nar_r4_kernel.py:195-199
 *   - normalisation as a fp32 DIVISION by fp32(sqrt(q)):
 *       nar/extended_experiment.py:456 (`y / math.sqrt(n)` on a fp32 tensor)
 *   - Paley entries fp32(+-1) / fp32(sqrt(m)):
 *       nar/extended_experiment.py:459-472, nar/activation_experiments.py:114-128
 *   - Kronecker layout y[a*q + c] = sum_a' Hm[a, a'] F[a', c] and the 28-then-12
 *     dispatch order: nar/activation_experiments.py:188-217
 *   - subtraction of the rank-k term: quarot-llama3/nar_r4_kernel.py:190-202,
 *     nar/fold_signed_permutation.py:121-129
 *   - quantizer: nar/experiment.py:158-184 (dynamic_asym_int4): fp32 min/max,
 *     raw = (hi-lo)/15 as a division, fp16 RNE of scale and zero, the two
 *     degenerate-group guards, q = round_half_even((x - z)/s) clamped to
 *     [0, 15], dequant q*s + z as a multiply then an add
 *   - packing: nar/kernels/r4_fused_v2.py:80-92 (low nibble = even channel)
 *
 * The reference computes three stages with BLAS matrix products whose
 * summation order it does not pin (torch `@`): the Paley factor product
 * (activation_experiments.py:200-201), u = x @ Y' and u @ W''^T
 * (nar_r4_kernel.py:201-202).  The oracle defines each of them as the exact
 * sum accumulated in fp64 in index order and rounded once to fp32 -- the value
 * an ideal fp32 BLAS returns.  Tests pin these definitions against torch's own
 * sgemm to within a few fp32 ulp.
 *
 * Build: oracle/build.py (gcc -O2 -ffp-contract=off, no fast-math).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define NAR_QMAX 15

/* ------------------------------------------------------------------ fp16 --- */

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary32 -> binary16, round to nearest even, with subnormals,
 * overflow to infinity and NaN propagation (what torch `.to(float16)` does). */
uint16_t nar_oracle_f32_to_f16(float f)
{
    uint32_t x = f32_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t a = x & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (a == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    if (a <= 0x33000000u) return sign;                 /* |f| <= 2^-25 -> 0 */
    int e = (int)(a >> 23) - 127;
    uint32_t m = (a & 0x7fffffu) | 0x800000u;
    if (e < -14) {                                      /* fp16 subnormal */
        uint32_t s = (uint32_t)(-(e + 1));              /* 14..24 */
        uint32_t q = m >> s;
        uint32_t rem = m & ((1u << s) - 1u);
        uint32_t half = 1u << (s - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = m >> 13;
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    int eh = e + 15;
    if (q == 0x800u) { q = 0x400u; eh++; }
    if (eh >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)eh << 10) | (q & 0x3ffu));
}

float nar_oracle_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t m = (uint32_t)h & 0x3ffu;
    if (e == 0x1fu) return bits_f32(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return bits_f32(sign);
        /* subnormal: m * 2^-24 is exact in fp32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* ---------------------------------------------------------------- Paley ---- */

static int gf27_mul(int a, int b)
{
    /* GF(3^3) with modulus x^3 + 2x + 1, element c0 + 3 c1 + 9 c2
     * (nar/activation_experiments.py:90-105). */
    int ac[3], bc[3], prod[5] = {0, 0, 0, 0, 0};
    for (int i = 0; i < 3; i++) { ac[i] = a % 3; a /= 3; bc[i] = b % 3; b /= 3; }
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++) prod[i + j] = (prod[i + j] + ac[i] * bc[j]) % 3;
    /* x^3 = x + 2 (i.e. -2x - 1), x^4 = x^2 + 2x */
    for (int d = 4; d >= 3; d--) {
        int c = prod[d] % 3;
        if (!c) continue;
        prod[d] = 0;
        prod[d - 3] = (prod[d - 3] + 2 * c) % 3;
        prod[d - 2] = (prod[d - 2] + c) % 3;
    }
    return prod[0] + 3 * prod[1] + 9 * prod[2];
}

static int gf27_sub(int a, int b)
{
    int r = 0, p = 1;
    for (int i = 0; i < 3; i++) {
        int d = ((a % 3) - (b % 3) + 3) % 3;
        r += d * p; p *= 3; a /= 3; b /= 3;
    }
    return r;
}

static int is_prime(int q)
{
    if (q < 2) return 0;
    for (int d = 2; d * d <= q; d++) if (q % d == 0) return 0;
    return 1;
}

/* chi(d) over Z_q: 0 for d = 0, +1 for a quadratic residue, -1 otherwise. */
static int chi_mod(int d, int q)
{
    d = ((d % q) + q) % q;
    if (d == 0) return 0;
    for (int v = 1; v < q; v++) if ((v * v) % q == d) return 1;
    return -1;
}

/* Paley's constructions over Z_q for the Qwen3 orders
 * (nar/activation_experiments.py:141-185): Paley I for a prime q = order - 1
 * = 3 (mod 4) (ones bordering Q - I, Q[r][c] = chi(r - c)); Paley II for a
 * prime q = order/2 - 1 = 1 (mod 4) (C the conference matrix bordering Q with
 * ones and a zero corner, H = [[C + I, C - I], [C - I, -C - I]]). */
static int paley_zq(int m, int8_t *out)
{
    int q = m - 1;
    if (is_prime(q) && q % 4 == 3) {
        for (int r = 0; r < m; r++)
            for (int c = 0; c < m; c++)
                out[r * m + c] = (int8_t)((r == 0 || c == 0) ? 1 : chi_mod(r - c, q) - (r == c));
        return 0;
    }
    q = m / 2 - 1;
    if (m % 2 || !is_prime(q) || q % 4 != 1) return -1;
    const int h = q + 1;
    for (int r = 0; r < m; r++)
        for (int c = 0; c < m; c++) {
            const int rr = r % h, cc = c % h;
            const int conf = (rr == 0 && cc == 0) ? 0 : (rr == 0 || cc == 0) ? 1 : chi_mod(rr - cc, q);
            const int eye = rr == cc;
            int val;
            if (r < h && c < h) val = conf + eye;
            else if (r < h || c < h) val = conf - eye;
            else val = -conf - eye;
            out[r * m + c] = (int8_t)val;
        }
    return 0;
}

/* Fill out[m*m] with the +-1 Paley Hadamard matrix of order m (row-major,
 * row = output index).  Supports m = 1 (trivial), 12 (Paley I over Z_11,
 * nar/extended_experiment.py:459-472), 28 (Paley I over GF(27),
 * nar/activation_experiments.py:114-128) and the Qwen3 orders 20, 68, 76 and
 * 200 (paley_zq).  Returns 0 or -1. */
int nar_oracle_paley(int m, int8_t *out)
{
    if (m == 1) { out[0] = 1; return 0; }
    if (m == 20 || m == 68 || m == 76 || m == 200) return paley_zq(m, out);
    if (m != 12 && m != 28) return -1;
    int q = m - 1;
    int residue[27];
    memset(residue, 0, sizeof residue);
    for (int v = 1; v < q; v++) {
        int sq = (m == 12) ? (v * v) % q : gf27_mul(v, v);
        residue[sq] = 1;
    }
    for (int r = 0; r < m; r++)
        for (int c = 0; c < m; c++) {
            int val;
            if (r == 0 || c == 0) {
                val = 1;
            } else {
                int d = (m == 12) ? ((r - 1) - (c - 1) + q) % q : gf27_sub(r - 1, c - 1);
                int core = d == 0 ? 0 : (residue[d] ? 1 : -1);
                val = core - (r == c ? 1 : 0);
            }
            out[r * m + c] = (int8_t)val;
        }
    return 0;
}

/* ----------------------------------------------------------------- FWHT ---- */

/* In-place natural-order FWHT, stage widths 1..q/2, (a+b, a-b) in fp32. */
static void fwht_f32(float *y, int q)
{
    for (int w = 1; w < q; w <<= 1)
        for (int i0 = 0; i0 < q; i0 += 2 * w)
            for (int c = 0; c < w; c++) {
                float a = y[i0 + c], b = y[i0 + w + c];
                y[i0 + c] = a + b;
                y[i0 + w + c] = a - b;
            }
}

static int is_pow2(int64_t v) { return v > 0 && !(v & (v - 1)); }

/* x (fp32 [T, ldx]) -> out (fp32 [T, ldo]) = H_s x - u W^T, u = x V.
 *   m, q       : Hadamard factors; blocks of m*q channels each get H_m (x) H_q
 *   signs      : optional fp32 [n] applied to the Hadamard input only
 *   k, nb      : rank and rank-block width (nb = n: one projection over the
 *                whole row; nb = 128: independent per-head factors)
 *   v          : fp32 [n, k]  (Y', row i of block j belongs to block j)
 *   wt         : fp32 [k, n]  (W''^T)
 * Returns 0, or -1 on an invalid shape. */
int nar_oracle_rotate(const float *x, int64_t T, int64_t n, int64_t ldx,
                      int m, int q, const float *signs,
                      int k, int64_t nb, const float *v, const float *wt,
                      float *out, int64_t ldo)
{
    if (T < 0 || n <= 0 || ldx < n || ldo < n || !is_pow2(q)) return -1;
    int64_t blk = (int64_t)m * q;
    if (m < 1 || m > 200 || n % blk) return -1;
    if (k < 0 || (k > 0 && (nb <= 0 || n % nb || !v || !wt))) return -1;

    int8_t *pal = (int8_t *)malloc((size_t)m * (size_t)m);
    if (!pal) return -1;
    if (nar_oracle_paley(m, pal)) { free(pal); return -1; }
    const float sq = (float)sqrt((double)q);
    /* |entry| of H_m / sqrt(m): fp32(1) / fp32(sqrt(m)) as the reference's fp32
     * factors (12, 28; for 20 and 76 equal to RN32 of the fp64 1/sqrt(m) that
     * paley_hadamard casts); the fp64 value for 68 and 200, whose product the
     * reference forms in fp64 (nar/activation_experiments.py:205-215) */
    const double hm = (m == 68 || m == 200) ? 1.0 / sqrt((double)m) : (double)(1.0f / (float)sqrt((double)m));

    float *row = (float *)malloc(sizeof(float) * (size_t)n);
    float *pr = (float *)malloc(sizeof(float) * (size_t)n);
    float *u = (float *)malloc(sizeof(float) * (size_t)(k > 0 ? (n / nb) * k : 1));
    if (!row || !pr || !u) { free(row); free(pr); free(u); free(pal); return -1; }

    for (int64_t t = 0; t < T; t++) {
        const float *xt = x + t * ldx;
        for (int64_t i = 0; i < n; i++) row[i] = signs ? xt[i] * signs[i] : xt[i];
        for (int64_t b0 = 0; b0 < n; b0 += blk)
            for (int a = 0; a < m; a++) {
                float *seg = row + b0 + (int64_t)a * q;
                fwht_f32(seg, q);
                for (int c = 0; c < q; c++) seg[c] = seg[c] / sq;
            }
        if (m > 1) {
            for (int64_t b0 = 0; b0 < n; b0 += blk)
                for (int a = 0; a < m; a++)
                    for (int c = 0; c < q; c++) {
                        double acc = 0.0;
                        for (int a2 = 0; a2 < m; a2++) {
                            double h = pal[a * m + a2] > 0 ? hm : -hm;
                            acc += (double)row[b0 + (int64_t)a2 * q + c] * (double)h;
                        }
                        pr[b0 + (int64_t)a * q + c] = (float)acc;
                    }
        } else {
            memcpy(pr, row, sizeof(float) * (size_t)n);
        }
        if (k > 0) {
            int64_t nblocks = n / nb;
            for (int64_t j = 0; j < nblocks; j++)
                for (int r = 0; r < k; r++) {
                    double acc = 0.0;
                    for (int64_t i = j * nb; i < (j + 1) * nb; i++)
                        acc += (double)xt[i] * (double)v[i * k + r];
                    u[j * k + r] = (float)acc;
                }
            for (int64_t i = 0; i < n; i++) {
                const float *uj = u + (i / nb) * k;
                double acc = 0.0;
                for (int r = 0; r < k; r++) acc += (double)uj[r] * (double)wt[(int64_t)r * n + i];
                float corr = (float)acc;
                out[t * ldo + i] = pr[i] - corr;
            }
        } else {
            memcpy(out + t * ldo, pr, sizeof(float) * (size_t)n);
        }
    }
    free(row); free(pr); free(u); free(pal);
    return 0;
}

/* The rank-k projection u = x V alone (fp32 [T, nblocks*k]), as defined above. */
int nar_oracle_projection(const float *x, int64_t T, int64_t n, int64_t ldx,
                          int k, int64_t nb, const float *v, float *u)
{
    if (k <= 0 || nb <= 0 || n % nb) return -1;
    int64_t nblocks = n / nb;
    for (int64_t t = 0; t < T; t++)
        for (int64_t j = 0; j < nblocks; j++)
            for (int r = 0; r < k; r++) {
                double acc = 0.0;
                for (int64_t i = j * nb; i < (j + 1) * nb; i++)
                    acc += (double)x[t * ldx + i] * (double)v[i * k + r];
                u[(t * nblocks + j) * k + r] = (float)acc;
            }
    return 0;
}

/* -------------------------------------------------------------- quantize --- */

/* dynamic_asym_int4 on fp32 rows (nar/experiment.py:158-184).
 * codes : uint8 [T, n] unpacked (one code per channel), may be NULL
 * packed: uint8 [T, n/2] (byte j = q[2j] | q[2j+1] << 4), may be NULL
 * scales, zeros: fp16 bits [T, n/b]
 * deq   : fp32 [T, n] = q*s + z, may be NULL */
int nar_oracle_quant(const float *xr, int64_t T, int64_t n, int64_t ldx, int b,
                     uint8_t *codes, uint8_t *packed, uint16_t *scales, uint16_t *zeros,
                     float *deq)
{
    if (b <= 0 || n % b || (packed && (n & 1))) return -1;
    int64_t groups = n / b;
    for (int64_t t = 0; t < T; t++) {
        const float *row = xr + t * ldx;
        for (int64_t g = 0; g < groups; g++) {
            const float *xv = row + g * b;
            float lo = xv[0], hi = xv[0];
            int nan = isnan(xv[0]);
            for (int i = 1; i < b; i++) {
                float val = xv[i];
                if (isnan(val)) nan = 1;
                if (val < lo) lo = val;
                if (val > hi) hi = val;
            }
            if (nan) { lo = NAN; hi = NAN; }
            float raw = (hi - lo) / (float)NAR_QMAX;
            float sr = raw > 0.0f ? raw : 1.0f;
            uint16_t sh = nar_oracle_f32_to_f16(sr);
            if (!(nar_oracle_f16_to_f32(sh) > 0.0f)) sh = 0x3c00u;   /* second guard */
            uint16_t zh = nar_oracle_f32_to_f16(lo);
            float s = nar_oracle_f16_to_f32(sh), z = nar_oracle_f16_to_f32(zh);
            scales[t * groups + g] = sh;
            zeros[t * groups + g] = zh;
            for (int i = 0; i < b; i++) {
                float d = xv[i] - z;
                float qf = rintf(d / s);
                if (qf < 0.0f) qf = 0.0f;
                if (qf > (float)NAR_QMAX) qf = (float)NAR_QMAX;
                uint8_t c = isnan(qf) ? 0 : (uint8_t)qf;
                int64_t idx = t * n + g * b + i;
                if (codes) codes[idx] = c;
                if (packed) {
                    uint8_t *dst = packed + t * (n / 2) + (g * b + i) / 2;
                    if (((g * b + i) & 1) == 0) *dst = c;
                    else *dst = (uint8_t)(*dst | (c << 4));
                }
                if (deq) {
                    /* the reference dequantizes the clamped float quotient: a NaN
                     * quotient (x - z = Inf - Inf, or Inf / Inf) stays NaN */
                    float prod = (float)c * s;
                    deq[idx] = isnan(qf) ? qf : prod + z;
                }
            }
        }
    }
    return 0;
}
