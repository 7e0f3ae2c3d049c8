// extern "C" boundary of libnarhip: argument validation, kernel selection and
// launch.  See include/narhip.h for the contract of every entry point.
#include "../../include/narhip.h"
#include "narhip_device.hpp"
#include "rank_exact.hip"
#include "rq_row.hip"
#include "rq_seg.hip"
#include "dequant.hip"

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

using namespace narhip;

namespace {

thread_local std::string g_error;

int fail(int code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

int check_launch(const char *what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(NARHIP_EHIP, "%s: %s", what, hipGetErrorString(e));
    return NARHIP_OK;
}

bool pow2(int64_t v) { return v > 0 && !(v & (v - 1)); }
bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ----------------------------------------------------------- Paley factors
// Paley I construction: order m = p + 1 from the quadratic residues of a
// field of p elements; first row and column +1, lower-right block Q - I with
// Q[r][c] = chi(r - c).  p = 11 uses Z_11; p = 27 uses GF(3^3) with modulus
// x^3 + 2x + 1 and elements c0 + 3 c1 + 9 c2 (the encoding the reference's
// construction uses, so the +-1 pattern is the same matrix).

int gf3_digit(int a, int i) { for (; i > 0; i--) a /= 3; return a % 3; }

int gf27_mul(int a, int b)
{
    int c[5] = {0, 0, 0, 0, 0};
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++) c[i + j] += gf3_digit(a, i) * gf3_digit(b, j);
    for (int i = 0; i < 5; i++) c[i] %= 3;
    // reduce with x^3 = x + 2 (mod 3): x^4 -> x^2 + 2x, x^3 -> x + 2
    for (int d = 4; d >= 3; d--) {
        if (!c[d]) continue;
        c[d - 2] = (c[d - 2] + c[d]) % 3;
        c[d - 3] = (c[d - 3] + 2 * c[d]) % 3;
        c[d] = 0;
    }
    return c[0] + 3 * c[1] + 9 * c[2];
}

int gf27_sub(int a, int b)
{
    int r = 0, p = 1;
    for (int i = 0; i < 3; i++, p *= 3) r += ((gf3_digit(a, i) - gf3_digit(b, i) + 3) % 3) * p;
    return r;
}

int build_paley(int m, int8_t *out)
{
    if (m == 1) { out[0] = 1; return 0; }
    if (m != 12 && m != 28) return -1;
    const int p = m - 1;
    bool residue[27] = {};
    for (int v = 1; v < p; v++) residue[m == 12 ? (v * v) % p : gf27_mul(v, v)] = true;
    for (int r = 0; r < m; r++)
        for (int c = 0; c < m; c++) {
            int val = 1;
            if (r > 0 && c > 0) {
                int d = m == 12 ? ((r - c) % p + p) % p : gf27_sub(r - 1, c - 1);
                val = (d == 0 ? 0 : (residue[d] ? 1 : -1)) - (r == c ? 1 : 0);
            }
            out[r * m + c] = (int8_t)val;
        }
    // H H^T = m I
    for (int r = 0; r < m; r++)
        for (int s = 0; s < m; s++) {
            int dot = 0;
            for (int c = 0; c < m; c++) dot += out[r * m + c] * out[s * m + c];
            if (dot != (r == s ? m : 0)) return -2;
        }
    return 0;
}

PaleyTable paley_table(int m)
{
    PaleyTable t{};
    int8_t h[28 * 28];
    build_paley(m, h);
    for (int r = 0; r < m; r++) {
        uint32_t bits = 0;
        for (int c = 0; c < m; c++) if (h[r * m + c] < 0) bits |= 1u << c;
        t.neg[r] = bits;
    }
    return t;
}

float f32_sqrt(int v) { return (float)std::sqrt((double)v); }

// ------------------------------------------------------------ dispatchers

template <int Q, int B>
int launch_seg_qb(const SegArgs &a, int mode, hipStream_t s)
{
    const int64_t segs = a.T * (a.n / Q);
    dim3 grid((unsigned)((segs + 15) / 16));
    if (grid.x == 0) return NARHIP_OK;
    switch (mode) {
    case RANK_NONE: hipLaunchKernelGGL((rq_seg_kernel<Q, B, RANK_NONE, 0>), grid, dim3(256), 0, s, a); break;
    case RANK_LOCAL: hipLaunchKernelGGL((rq_seg_kernel<Q, B, RANK_LOCAL, 8>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((rq_seg_kernel<Q, B, RANK_PARTIAL, 64>), grid, dim3(256), 0, s, a); break;
    }
    return check_launch("rq_seg_kernel");
}

template <int Q>
int launch_seg_q(const SegArgs &a, int b, int mode, hipStream_t s)
{
    switch (b) {
    case 32: return launch_seg_qb<Q, 32>(a, mode, s);
    case 64: return launch_seg_qb<Q, 64>(a, mode, s);
    case 128: return launch_seg_qb<Q, 128>(a, mode, s);
    }
    return fail(NARHIP_EUNSUPPORTED, "group %d not built", b);
}

int launch_seg(const SegArgs &a, int q, int b, int mode, hipStream_t s)
{
    switch (q) {
    case 128: return launch_seg_q<128>(a, b, mode, s);
    case 256: return launch_seg_q<256>(a, b, mode, s);
    case 512: return launch_seg_q<512>(a, b, mode, s);
    case 1024: return launch_seg_q<1024>(a, b, mode, s);
    }
    return fail(NARHIP_EUNSUPPORTED, "segment width %d not built", q);
}

template <int M, int Q, int B>
int launch_row_mqb(const RowArgs &a, hipStream_t s)
{
    if (a.T == 0) return NARHIP_OK;
    const size_t lds = sizeof(float) * M * Q;
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&rq_row_kernel<M, Q, B>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return fail(NARHIP_EHIP, "hipFuncSetAttribute: %s", hipGetErrorString(e));
        attr = true;
    }
    hipLaunchKernelGGL((rq_row_kernel<M, Q, B>), dim3((unsigned)a.T), dim3(256), lds, s, a);
    return check_launch("rq_row_kernel");
}

template <int M, int Q>
int launch_row_mq(const RowArgs &a, int b, hipStream_t s)
{
    switch (b) {
    case 32: return launch_row_mqb<M, Q, 32>(a, s);
    case 64: return launch_row_mqb<M, Q, 64>(a, s);
    case 128: return launch_row_mqb<M, Q, 128>(a, s);
    }
    return fail(NARHIP_EUNSUPPORTED, "group %d not built", b);
}

template <int M>
int launch_row_m(const RowArgs &a, int q, int b, hipStream_t s)
{
    switch (q) {
    case 256: return launch_row_mq<M, 256>(a, b, s);
    case 512: return launch_row_mq<M, 512>(a, b, s);
    case 1024: return launch_row_mq<M, 1024>(a, b, s);
    }
    return fail(NARHIP_EUNSUPPORTED, "Kronecker H_%d x H_%d not built", M, q);
}

int launch_row(const RowArgs &a, int m, int q, int b, hipStream_t s)
{
    if (m == 12) return launch_row_m<12>(a, q, b, s);
    if (m == 28) return launch_row_m<28>(a, q, b, s);
    return fail(NARHIP_EUNSUPPORTED, "Paley order %d not built", m);
}

int launch_proj_exact(const uint16_t *x, int64_t T, int64_t n, int64_t ldx, const float *v,
                      int k, int splits, float *partial, hipStream_t s)
{
    if (T == 0) return NARHIP_OK;
    ProjArgs a{x, ldx, T, n, v, partial, k, splits};
    hipLaunchKernelGGL(proj_exact_kernel, dim3((unsigned)((T + 31) / 32), (unsigned)splits), dim3(256), 0, s, a);
    return check_launch("proj_exact_kernel");
}

int launch_corr_exact(const float *partial, int splits, int k, const float *wt, int64_t T, int64_t n,
                      float *corr, hipStream_t s)
{
    if (T == 0) return NARHIP_OK;
    CorrArgs a{partial, splits, k, wt, T, n, corr};
    hipLaunchKernelGGL(corr_exact_kernel, dim3((unsigned)((T + 31) / 32), (unsigned)(n / 64)), dim3(256), 0, s, a);
    return check_launch("corr_exact_kernel");
}

struct Plan {
    bool kron;          // row kernel (H_m (x) H_q over the row)
    int seg_mode;       // rq_seg rank mode
    bool need_proj;     // projection computed into the workspace
    bool need_corr;     // correction materialised into the workspace
    size_t proj_bytes, corr_bytes;
};

int make_plan(int64_t T, int64_t n, int m, int q, int k, int64_t nb, bool have_partial, int splits,
              int rank_mode, Plan &p)
{
    if (T < 0 || n <= 0) return fail(NARHIP_EINVAL, "tokens %lld / n %lld invalid", (long long)T, (long long)n);
    if (!pow2(q) || q < 128 || q > 1024)
        return fail(NARHIP_EUNSUPPORTED, "Hadamard block width %d: need a power of two in [128, 1024]", q);
    if (m != 1 && m != 12 && m != 28) return fail(NARHIP_EUNSUPPORTED, "no Paley factor of order %d", m);
    if (n % ((int64_t)m * q)) return fail(NARHIP_EINVAL, "n=%lld is not a multiple of %d*%d", (long long)n, m, q);
    if (m > 1 && (int64_t)m * q != n)
        return fail(NARHIP_EUNSUPPORTED, "Kronecker factor must span the row (m*q = n)");
    if (k < 0 || k > 64) return fail(NARHIP_EUNSUPPORTED, "rank k=%d outside [0, 64]", k);
    if (rank_mode < 0 || rank_mode > 2) return fail(NARHIP_EINVAL, "rank_mode %d", rank_mode);
    p = Plan{};
    p.kron = m > 1;
    if (k == 0) { p.seg_mode = RANK_NONE; return NARHIP_OK; }
    if (nb != n && !(nb == q && m == 1))
        return fail(NARHIP_EUNSUPPORTED, "rank_block %lld: need n or the Hadamard block width", (long long)nb);
    if (nb == q && m == 1 && nb != n) {
        if (k > 8) return fail(NARHIP_EUNSUPPORTED, "per-block rank k=%d > 8", k);
        if (have_partial) return fail(NARHIP_EINVAL, "partials are only defined for a full-row rank block");
        p.seg_mode = RANK_LOCAL;
        return NARHIP_OK;
    }
    if (have_partial) {
        if (splits < 1 || n % splits) return fail(NARHIP_EINVAL, "splits=%d must divide n=%lld", splits, (long long)n);
    }
    p.seg_mode = RANK_PARTIAL;
    p.need_proj = !have_partial;
    p.proj_bytes = p.need_proj ? sizeof(float) * (size_t)T * (size_t)k : 0;
    p.need_corr = p.kron;
    p.corr_bytes = p.need_corr ? sizeof(float) * (size_t)T * (size_t)n : 0;
    if (n % 64) return fail(NARHIP_EUNSUPPORTED, "full-row rank needs n %% 64 == 0");
    return NARHIP_OK;
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

int run_rotate_quant(const void *x_bf16, int64_t T, int64_t n, int64_t ldx, int m, int q, const float *signs,
                     int k, int64_t nb, const float *v, const float *wt, const float *partial, int splits,
                     int group, uint8_t *codes, void *scales, void *zeros, float *rotated,
                     const int64_t *dest, int rank_mode, void *ws, size_t ws_bytes, hipStream_t s)
{
    Plan p;
    int rc = make_plan(T, n, m, q, k, nb, partial != nullptr, splits, rank_mode, p);
    if (rc) return rc;
    if (group != 32 && group != 64 && group != 128) return fail(NARHIP_EUNSUPPORTED, "group %d", group);
    if (q % group) return fail(NARHIP_EINVAL, "group %d must divide the Hadamard block %d", group, q);
    if (ldx < n || ldx % 8) return fail(NARHIP_EINVAL, "ld_x=%lld must be >= n and a multiple of 8", (long long)ldx);
    if (T > 0 && (!x_bf16 || !codes || !scales || !zeros)) return fail(NARHIP_EINVAL, "null tensor argument");
    if (!aligned16(x_bf16) || !aligned16(codes) || (rotated && !aligned16(rotated)))
        return fail(NARHIP_EINVAL, "x, codes and rotated must be 16-byte aligned");
    if (k > 0 && (!wt || (p.need_proj && !v))) return fail(NARHIP_EINVAL, "rank factors missing");
    const size_t need = align256(p.proj_bytes) + align256(p.corr_bytes);
    if (need > 0 && (!ws || ws_bytes < need))
        return fail(NARHIP_EWORKSPACE, "workspace of %zu bytes required, %zu given", need, ws_bytes);
    if (T == 0) return NARHIP_OK;

    char *wsp = static_cast<char *>(ws);
    float *proj = p.need_proj ? reinterpret_cast<float *>(wsp) : nullptr;
    float *corr = p.need_corr ? reinterpret_cast<float *>(wsp + align256(p.proj_bytes)) : nullptr;
    const float *part = partial;
    int sp = splits;
    if (p.need_proj) {
        rc = launch_proj_exact(static_cast<const uint16_t *>(x_bf16), T, n, ldx, v, k, 1, proj, s);
        if (rc) return rc;
        part = proj;
        sp = 1;
    }
    if (p.kron) {
        if (k > 0) {
            rc = launch_corr_exact(part, sp, k, wt, T, n, corr, s);
            if (rc) return rc;
        }
        RowArgs a{};
        a.x = static_cast<const uint16_t *>(x_bf16); a.ldx = ldx; a.T = T; a.n = n;
        a.signs = signs; a.corr = k > 0 ? corr : nullptr;
        a.codes = codes; a.scales = static_cast<uint16_t *>(scales); a.zeros = static_cast<uint16_t *>(zeros);
        a.dest = dest; a.rotated = rotated; a.paley = paley_table(m);
        a.sq = f32_sqrt(q); a.hm = 1.0f / f32_sqrt(m);
        return launch_row(a, m, q, group, s);
    }
    SegArgs a{};
    a.x = static_cast<const uint16_t *>(x_bf16); a.ldx = ldx; a.T = T; a.n = n;
    a.signs = signs; a.v = v; a.wt = wt; a.partial = part; a.splits = sp; a.k = k;
    a.codes = codes; a.scales = static_cast<uint16_t *>(scales); a.zeros = static_cast<uint16_t *>(zeros);
    a.dest = dest; a.rotated = rotated; a.sq = f32_sqrt(q);
    return launch_seg(a, q, group, p.seg_mode, s);
}

}  // namespace

extern "C" {

int narhip_abi_version(void) { return NARHIP_ABI_VERSION; }

const char *narhip_last_error_string(void) { return g_error.c_str(); }

int narhip_paley(int32_t m, int8_t *out_host)
{
    if (!out_host) return fail(NARHIP_EINVAL, "null output");
    int rc = build_paley(m, out_host);
    if (rc == -1) return fail(NARHIP_EUNSUPPORTED, "no Paley factor of order %d", m);
    if (rc) return fail(NARHIP_EINVAL, "Paley construction of order %d failed H H^T = mI", m);
    return NARHIP_OK;
}

size_t narhip_rotate_quant_workspace(int64_t tokens, int64_t n, int32_t had_m, int32_t had_q, int32_t k,
                                     int64_t rank_block, int32_t have_partial, int32_t splits, int32_t rank_mode)
{
    Plan p;
    if (make_plan(tokens, n, had_m, had_q, k, rank_block, have_partial != 0, splits, rank_mode, p)) return 0;
    return align256(p.proj_bytes) + align256(p.corr_bytes);
}

int narhip_rotate_quant(const void *x_bf16, int64_t tokens, int64_t n, int64_t ld_x,
                        int32_t had_m, int32_t had_q, const float *signs,
                        int32_t k, int64_t rank_block, const float *v, const float *w_t,
                        const float *partial, int32_t splits,
                        int32_t group, uint8_t *codes, void *scales_f16, void *zeros_f16,
                        float *rotated, const int64_t *dest_rows, int32_t rank_mode,
                        void *workspace, size_t workspace_bytes, void *stream)
{
    g_error.clear();
    return run_rotate_quant(x_bf16, tokens, n, ld_x, had_m, had_q, signs, k, rank_block, v, w_t, partial,
                            splits, group, codes, scales_f16, zeros_f16, rotated, dest_rows, rank_mode,
                            workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int narhip_rank_projection(const void *x_bf16, int64_t tokens, int64_t n, int64_t ld_x,
                           const float *v, int32_t k, int32_t splits, float *partial,
                           int32_t rank_mode, void *stream)
{
    g_error.clear();
    if (tokens < 0 || n <= 0 || ld_x < n) return fail(NARHIP_EINVAL, "bad shape");
    if (k < 1 || k > 64) return fail(NARHIP_EUNSUPPORTED, "rank k=%d outside [1, 64]", k);
    if (splits < 1 || n % splits) return fail(NARHIP_EINVAL, "%lld channels do not divide into %d splits",
                                              (long long)n, splits);
    if (rank_mode < 0 || rank_mode > 2) return fail(NARHIP_EINVAL, "rank_mode %d", rank_mode);
    if (tokens > 0 && (!x_bf16 || !v || !partial)) return fail(NARHIP_EINVAL, "null tensor argument");
    return launch_proj_exact(static_cast<const uint16_t *>(x_bf16), tokens, n, ld_x, v, k, splits, partial,
                             static_cast<hipStream_t>(stream));
}

int narhip_group_quant(const void *x_bf16, int64_t tokens, int64_t n, int64_t ld_x,
                       int32_t had_m, int32_t had_q, const float *partial, int32_t splits,
                       int32_t k, const float *w_t, int32_t group,
                       uint8_t *codes, void *scales_f16, void *zeros_f16,
                       void *workspace, size_t workspace_bytes, void *stream)
{
    g_error.clear();
    if (k > 0 && !partial) return fail(NARHIP_EINVAL, "partials required");
    return run_rotate_quant(x_bf16, tokens, n, ld_x, had_m, had_q, nullptr, k, n, nullptr, w_t, partial, splits,
                            group, codes, scales_f16, zeros_f16, nullptr, nullptr, NARHIP_RANK_EXACT,
                            workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int narhip_dequantize(const uint8_t *codes, const void *scales_f16, const void *zeros_f16,
                      int64_t rows, int64_t n, int32_t group, float *out, void *stream)
{
    g_error.clear();
    if (rows < 0 || n <= 0 || group <= 0 || n % group || group % 8)
        return fail(NARHIP_EINVAL, "bad shape rows=%lld n=%lld group=%d", (long long)rows, (long long)n, group);
    if (rows == 0) return NARHIP_OK;
    if (!codes || !scales_f16 || !zeros_f16 || !out) return fail(NARHIP_EINVAL, "null tensor argument");
    if (!aligned16(out) || (reinterpret_cast<uintptr_t>(codes) & 3u))
        return fail(NARHIP_EINVAL, "codes must be 4-byte and out 16-byte aligned");
    const int64_t words = rows * n / 8;
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), codes, static_cast<const uint16_t *>(scales_f16),
                       static_cast<const uint16_t *>(zeros_f16), rows, n, group, out);
    return check_launch("dequant_kernel");
}

}  // extern "C"
