// extern "C" boundary of libnarhip: argument validation, planning and the
// entry points of include/narhip.h.  The kernels are launched through the
// launchers of host.hpp (launch_*.hip); this unit compiles no kernel.  Its only
// device object is the scratch array of the allocation-free entry point.
#include "host.hpp"

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>

using namespace narhip;
using namespace narhip::host;

namespace narhip {
namespace host {

namespace {
thread_local std::string g_error;
}  // namespace

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

const char *last_error() { return g_error.c_str(); }
void clear_error() { g_error.clear(); }

int64_t resident_blocks(const void *kernel, int threads, size_t lds)
{
    static std::mutex mu;
    static std::map<std::tuple<const void *, int, size_t, int>, int64_t> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    const auto key = std::make_tuple(kernel, threads, lds, dev);
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int cus = 0, per = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, lds) != hipSuccess || per < 1) per = 1;
    const int64_t r = (int64_t)cus * per;
    cache.emplace(key, r);
    return r;
}

// ----------------------------------------------------------- Paley factors
// Paley I construction: order m = p + 1 from the quadratic residues of a
// field of p elements; first row and column +1, lower-right block Q - I with
// Q[r][c] = chi(r - c).  p = 11 and 19 use Z_p; p = 27 uses GF(3^3) with modulus
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

static bool small_prime(int v)
{
    if (v < 2) return false;
    for (int d = 2; d * d <= v; d++)
        if (v % d == 0) return false;
    return true;
}

bool paley_zp(int m, int &p, int &kind)
{
    if (m != 12 && m != 20 && m != 68 && m != 76 && m != 200) return false;
    if (small_prime(m - 1) && (m - 1) % 4 == 3) { p = m - 1; kind = 1; return true; }
    if (m % 2 == 0 && small_prime(m / 2 - 1) && (m / 2 - 1) % 4 == 1) { p = m / 2 - 1; kind = 2; return true; }
    return false;
}

int build_paley(int m, int8_t *out)
{
    if (m == 1) { out[0] = 1; return 0; }
    // Paley I (order p + 1, p = 3 mod 4): core entry chi(row - col) over Z_p
    // (over GF(27) for 28), bordered by ones, minus I.  Paley II (order
    // 2(p + 1), p = 1 mod 4): the conference matrix C (core bordered by ones,
    // zero corner) in [[C + I, C - I], [C - I, -C - I]].
    int p = 27, kind = 1;
    const bool field = m == 28;
    if (!field && !paley_zp(m, p, kind)) return -1;
    bool residue[256] = {};
    for (int v = 1; v < p; v++) residue[field ? gf27_mul(v, v) : (v * v) % p] = true;
    auto chi = [&](int r, int c) {               // r != c, both in [1, p]
        const int d = field ? gf27_sub(r - 1, c - 1) : ((r - c) % p + p) % p;
        return residue[d] ? 1 : -1;
    };
    for (int r = 0; r < m; r++)
        for (int c = 0; c < m; c++) {
            int val;
            if (kind == 1) {
                val = (r == 0 || c == 0) ? 1 : (r == c ? -1 : chi(r, c));
            } else {
                const int h = p + 1;
                const bool br = r >= h, bc = c >= h;
                const int rr = br ? r - h : r, cc = bc ? c - h : c;
                const int cv = rr == cc ? 0 : (rr == 0 || cc == 0) ? 1 : chi(rr, cc);
                const int e = rr == cc ? 1 : 0;
                val = (!br && !bc) ? cv + e : (br != bc) ? cv - e : -cv - e;
            }
            out[r * m + c] = (int8_t)val;
        }
    // H H^T = m I
    for (int r = 0; r < m; r++)
        for (int q = 0; q < m; q++) {
            int dot = 0;
            for (int c = 0; c < m; c++) dot += out[r * m + c] * out[q * m + c];
            if (dot != (r == q ? m : 0)) return -2;
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

}  // namespace host
}  // namespace narhip

namespace {

// --------------------------------------------------------------- planning

enum Path { PATH_SEG, PATH_SEG_PARTIAL_EXACT, PATH_KRON_EXACT, PATH_KRON_MFMA_QUANT, PATH_MFMA_RANK, PATH_FWHT };

// The MFMA rank path stages the rotated rows P through memory between the
// transform and the correction kernels; tokens are processed in chunks so that
// the P workspace stays bounded (4 GB by default).  Chunks small enough to stay
// resident in the 256 MB Infinity Cache were measured slower on MI355X (the
// per-chunk launches under-fill the GPU), so the default covers every
// benchmark shape in one chunk.
#ifndef NARHIP_CHUNK_BYTES
#define NARHIP_CHUNK_BYTES (4096ll << 20)
#endif

int64_t chunk_tokens(int64_t T, int64_t n)
{
    int64_t tc = NARHIP_CHUNK_BYTES / (n * (int64_t)sizeof(float));
    tc = tc / 256 * 256;
    if (tc < 256) tc = 256;
    return tc < T ? tc : T;
}



struct Plan {
    Path path;
    bool kron;
    int seg_mode;
    bool need_prep, need_proj, need_P, need_corr, vproj;
    bool xf;          // block-H_128, k <= 8: proj_tok + xform128 (group 128, no rotated output)
    int splits;
    int64_t chunk;
    size_t prep_b, proj_b, P_b, corr_b, u_b, xf_b;
    size_t total() const
    {
        const size_t sum = align256(prep_b) + align256(proj_b) + align256(P_b) + align256(corr_b) + align256(u_b);
        return xf_b > sum ? xf_b : sum;
    }
};

// budget > 0: the MFMA rank path halves its token chunk (down to 256 tokens)
// until the workspace fits in `budget` bytes; the other paths are not chunked.
int make_plan(int64_t T, int64_t n, int m, int q, int k, int64_t nb, bool have_partial, int splits,
              bool have_prepared, int rank_mode, Plan &p, size_t budget = 0)
{
    if (T < 0 || n <= 0) return fail(NARHIP_EINVAL, "tokens %lld / n %lld invalid", (long long)T, (long long)n);
    if (m == 1 && q == n && fwht_rows_width(q)) {
        // one FWHT over the whole power-of-two row, no rank term
        if (k != 0) return fail(NARHIP_EUNSUPPORTED, "rank term over a %d-wide FWHT row not built", q);
        if (rank_mode < 0 || rank_mode > 2) return fail(NARHIP_EINVAL, "rank_mode %d", rank_mode);
        p = Plan{};
        p.path = PATH_FWHT;
        return NARHIP_OK;
    }
    if (!pow2(q) || q < 128 || q > 1024)
        return fail(NARHIP_EUNSUPPORTED,
                    "Hadamard block width %d: need a power of two in [128, 1024] (or q = n in [2048, 8192])", q);
    if (m != 1 && m != 12 && m != 20 && m != 28)
        return fail(NARHIP_EUNSUPPORTED, "no Paley factor of order %d", m);
    if (n % ((int64_t)m * q)) return fail(NARHIP_EINVAL, "n=%lld is not a multiple of %d*%d", (long long)n, m, q);
    if (m > 1 && (int64_t)m * q != n)
        return fail(NARHIP_EUNSUPPORTED, "Kronecker factor must span the row (m*q = n)");
    if (k < 0 || k > 64) return fail(NARHIP_EUNSUPPORTED, "rank k=%d outside [0, 64]", k);
    if (rank_mode < 0 || rank_mode > 2) return fail(NARHIP_EINVAL, "rank_mode %d", rank_mode);
    p = Plan{};
    p.kron = m > 1;
    const bool exact = rank_mode == NARHIP_RANK_EXACT;
    if (k == 0) {
        p.path = p.kron ? (exact ? PATH_KRON_EXACT : PATH_KRON_MFMA_QUANT) : PATH_SEG;
        p.seg_mode = RANK_NONE;
        return NARHIP_OK;
    }
    if (nb != n && !(nb == q && m == 1))
        return fail(NARHIP_EUNSUPPORTED, "rank_block %lld: need n or the Hadamard block width", (long long)nb);
    if (nb == q && m == 1 && nb != n) {
        if (k > 8) return fail(NARHIP_EUNSUPPORTED, "per-block rank k=%d > 8", k);
        if (have_partial) return fail(NARHIP_EINVAL, "partials are only defined for a full-row rank block");
        p.path = PATH_SEG;
        p.seg_mode = RANK_LOCAL;
        return NARHIP_OK;
    }
    if (have_partial && (splits < 1 || n % splits))
        return fail(NARHIP_EINVAL, "splits=%d must divide n=%lld", splits, (long long)n);
    if (n % 128) return fail(NARHIP_EUNSUPPORTED, "full-row rank needs n %% 128 == 0");
    const bool mfma = !exact && (rank_mode == NARHIP_RANK_MFMA || k >= 16);
    if (mfma) {
        p.path = PATH_MFMA_RANK;
        p.need_prep = !have_prepared;
        p.prep_b = p.need_prep ? prepared_bytes(n, k) : 0;
        p.need_proj = !have_partial;
        p.need_P = true;
        // the channel splits of the projection follow the unbounded chunk, so a
        // token's partials, u and output do not depend on the budget
        p.splits = have_partial ? splits : mfma_splits(chunk_tokens(T, n), n);
        auto size_chunk = [&](int64_t chunk) {
            p.chunk = chunk;
            p.proj_b = p.need_proj ? sizeof(float) * (size_t)chunk * (size_t)p.splits * (size_t)k : 0;
            p.P_b = sizeof(float) * (size_t)chunk * (size_t)n;
            p.u_b = corr_scratch_bytes(chunk, n, k);
        };
        size_chunk(chunk_tokens(T, n));
        while (budget && p.total() > budget && p.chunk > 256) {
            const int64_t half = (p.chunk / 2 + 255) / 256 * 256;
            size_chunk(half > 256 ? half : 256);
        }
        return NARHIP_OK;
    }
    p.need_proj = !have_partial;
    // exact mode: the fp64 projection in one split, u one fp64 sum rounded once
    // (bit-exact); otherwise the fp64 VALU projection over channel splits with
    // fp64 partials, folded once
    p.vproj = p.need_proj && !exact && k <= 16;
    p.splits = have_partial ? splits : (p.vproj ? f64_splits(T, n) : 1);
    p.proj_b = !p.need_proj ? 0
               : p.vproj ? sizeof(double) * (size_t)T * (size_t)p.splits * (size_t)f64_kmax(k)
                         : sizeof(float) * (size_t)T * (size_t)k;
    if (p.vproj || p.splits > 1) p.u_b = sizeof(float) * (size_t)T * (size_t)k;   // folded u
    if (p.kron) {
        p.path = PATH_KRON_EXACT;
        p.need_corr = true;
        p.corr_b = sizeof(float) * (size_t)T * (size_t)n;
    } else {
        p.path = PATH_SEG_PARTIAL_EXACT;
        p.seg_mode = RANK_PARTIAL;
        if (!exact && q == 128 && xf_fast(q, k)) {
            p.xf = true;
            p.xf_b = have_partial ? 0 : xf_pd_bytes(T, xf_splits(T, n));
        }
    }
    return NARHIP_OK;
}

int run_rotate_quant(const void *x_bf16, int64_t T, int64_t n, int64_t ldx, int m, int q, const float *signs,
                     int k, int64_t nb, const float *v, const float *wt, const void *prepared,
                     const float *partial, int splits, int group, uint8_t *codes, void *scales, void *zeros,
                     float *rotated, const int64_t *dest, int rank_mode, void *ws, size_t ws_bytes, hipStream_t s,
                     size_t budget = 0)
{
    Plan p;
    int rc = make_plan(T, n, m, q, k, nb, partial != nullptr, splits, prepared != nullptr, rank_mode, p, budget);
    if (rc) return rc;
    if (group != 32 && group != 64 && group != 128) return fail(NARHIP_EUNSUPPORTED, "group %d", group);
    if (q % group) return fail(NARHIP_EINVAL, "group %d must divide the Hadamard block %d", group, q);
    if (ldx < n || ldx % 8) return fail(NARHIP_EINVAL, "ld_x=%lld must be >= n and a multiple of 8", (long long)ldx);
    if (T > 0 && (!x_bf16 || !codes || !scales || !zeros)) return fail(NARHIP_EINVAL, "null tensor argument");
    if (!aligned16(x_bf16) || !aligned16(codes) || (rotated && !aligned16(rotated)) || !aligned16(prepared) ||
        !aligned16(wt))
        return fail(NARHIP_EINVAL, "x, codes, rotated, prepared and w_t must be 16-byte aligned");
    // only the MFMA rank path reads the prepared W^T terms; every other path
    // with a rank term reads w_t itself
    if (k > 0 && p.path != PATH_SEG && !wt && !(p.path == PATH_MFMA_RANK && prepared))
        return fail(NARHIP_EINVAL, "rank factor w_t missing");
    if (k > 0 && (p.need_proj || p.seg_mode == RANK_LOCAL) && !v && !(p.path == PATH_MFMA_RANK && prepared))
        return fail(NARHIP_EINVAL, "rank factor v missing");
    if (p.seg_mode == RANK_LOCAL && (!v || !wt)) return fail(NARHIP_EINVAL, "rank factors missing");
    const size_t need = p.total();
    if (need > 0 && (!ws || ws_bytes < need))
        return fail(NARHIP_EWORKSPACE, "workspace of %zu bytes required, %zu given", need, ws_bytes);
    if (T == 0) return NARHIP_OK;
    if (p.path == PATH_FWHT) {
        FwhtArgs fa{};
        fa.x = static_cast<const uint16_t *>(x_bf16); fa.ldx = ldx; fa.T = T; fa.signs = signs;
        fa.rotated = rotated; fa.codes = codes; fa.scales = static_cast<uint16_t *>(scales);
        fa.zeros = static_cast<uint16_t *>(zeros); fa.dest = dest;
        fa.sq = f32_sqrt(q); fa.rsq = 1.0f / fa.sq;
        return launch_fwht(fa, q, group, s);
    }

    char *wsp = static_cast<char *>(ws);
    void *prep = p.need_prep ? wsp : const_cast<void *>(prepared);
    wsp += align256(p.prep_b);
    float *proj = p.need_proj ? reinterpret_cast<float *>(wsp) : nullptr;
    wsp += align256(p.proj_b);
    float *Pbuf = p.need_P ? reinterpret_cast<float *>(wsp) : nullptr;
    wsp += align256(p.P_b);
    float *corr = p.need_corr ? reinterpret_cast<float *>(wsp) : nullptr;
    wsp += align256(p.corr_b);
    __bf16 *u3 = p.u_b ? reinterpret_cast<__bf16 *>(wsp) : nullptr;
    const uint16_t *x = static_cast<const uint16_t *>(x_bf16);

    if (p.path == PATH_MFMA_RANK) {
        if (p.need_prep && (rc = launch_prepare(v, wt, n, k, prep, s))) return rc;
        for (int64_t t0 = 0; t0 < T; t0 += p.chunk) {
            const int64_t tn = T - t0 < p.chunk ? T - t0 : p.chunk;
            const uint16_t *xc = x + t0 * ldx;
            const float *part = partial ? partial + t0 * (int64_t)splits * k : nullptr;
            // projection and fold first, on the caller's stream: x then sits in
            // the Infinity Cache for the transform (measured faster than running
            // them on a second stream under the transform)
            if (p.need_proj) {
                if ((rc = launch_proj_mfma(xc, tn, n, ldx, prep, k, p.splits, proj, s))) return rc;
                if ((rc = launch_fold_u(proj, p.splits, k, kp32(k), tn, u3, s))) return rc;
            } else {
                if ((rc = launch_fold_u(part, splits, k, kp32(k), tn, u3, s))) return rc;
            }
            if (p.kron) {
                KronArgs ka{};
                ka.x = xc; ka.ldx = ldx; ka.T = tn; ka.n = n; ka.signs = signs; ka.P = Pbuf;
                ka.paley = paley_table(m); ka.sq = f32_sqrt(q); ka.rsq = 1.0f / ka.sq; ka.hm = 1.0f / f32_sqrt(m);
                if ((rc = launch_kron(nullptr, &ka, false, m, q, group, s))) return rc;
            } else {
                SegArgs sa{};
                sa.x = xc; sa.ldx = ldx; sa.T = tn; sa.n = n; sa.signs = signs; sa.k = 0;
                sa.codes = nullptr; sa.rotated = Pbuf; sa.sq = f32_sqrt(q); sa.rsq = 1.0f / sa.sq;
                if ((rc = launch_seg(sa, q, group, RANK_NONE, s))) return rc;
            }
            CorrQuantArgs ca{};
            ca.P = Pbuf; ca.T = tn; ca.n = n; ca.u3 = u3;
            ca.wtt = reinterpret_cast<const __bf16 *>(static_cast<const char *>(prep) + vt_bytes(n, k));
            ca.kp = kp32(k);
            ca.dest = dest ? dest + t0 : nullptr;
            ca.dummy = reinterpret_cast<uint8_t *>(u3) + align256(u3_bytes(tn, k));
            const int64_t row0 = dest ? 0 : t0;
            ca.codes = codes + row0 * (n / 2);
            ca.scales = static_cast<uint16_t *>(scales) + row0 * (n / group);
            ca.zeros = static_cast<uint16_t *>(zeros) + row0 * (n / group);
            ca.rotated = rotated ? rotated + t0 * n : nullptr;
            if ((rc = launch_corr_quant(ca, group, s))) return rc;
        }
        return NARHIP_OK;
    }

    if (p.xf && group == 128 && !rotated && aligned16(signs)) {
        // u as fp64 of RN32(sum), W^T for the lane's channels held in registers
        double *pd = nullptr;
        int S = splits;
        if (!partial) {
            S = xf_splits(T, n);
            pd = static_cast<double *>(ws);
            if ((rc = launch_proj_tok(x, T, n, ldx, v, k, S, pd, nullptr, s, false))) return rc;
        }
        XformArgs qa{};
        qa.signs = signs;
        qa.codes = codes;
        qa.scales = static_cast<uint16_t *>(scales);
        qa.zeros = static_cast<uint16_t *>(zeros);
        qa.dest = dest;
        return launch_xform128(x, T, n, ldx, wt, pd, partial, S, k, nullptr, s, &qa);
    }
    const float *part = partial;
    int sp = splits;
    float *uf = reinterpret_cast<float *>(u3);
    if (p.vproj) {
        double *pd = reinterpret_cast<double *>(proj);
        if ((rc = launch_proj_f64(x, T, n, ldx, v, k, p.splits, pd, s))) return rc;
        if ((rc = launch_fold_f64(pd, p.splits, f64_kmax(k), k, T, uf, s))) return rc;
        part = uf;
        sp = 1;
    } else if (p.need_proj) {
        if ((rc = launch_proj_exact(x, T, n, ldx, v, k, 1, proj, s))) return rc;
        part = proj;
        sp = 1;
    } else if (sp > 1 && uf) {
        if ((rc = launch_fold_f32(part, sp, k, T, uf, s))) return rc;
        part = uf;
        sp = 1;
    }
    if (p.kron) {
        if (k > 0 && (rc = launch_corr_exact(part, sp, k, wt, T, n, corr, s))) return rc;
        if (p.path == PATH_KRON_MFMA_QUANT) {
            KronArgs ka{};
            ka.x = x; ka.ldx = ldx; ka.T = T; ka.n = n; ka.signs = signs;
            ka.codes = codes; ka.scales = static_cast<uint16_t *>(scales); ka.zeros = static_cast<uint16_t *>(zeros);
            ka.dest = dest; ka.rotated = rotated;
            ka.paley = paley_table(m); ka.sq = f32_sqrt(q); ka.rsq = 1.0f / ka.sq; ka.hm = 1.0f / f32_sqrt(m);
            return launch_kron(nullptr, &ka, true, m, q, group, s);
        }
        RowArgs a{};
        a.x = x; a.ldx = ldx; a.T = T; a.n = n;
        a.signs = signs; a.corr = k > 0 ? corr : nullptr;
        a.codes = codes; a.scales = static_cast<uint16_t *>(scales); a.zeros = static_cast<uint16_t *>(zeros);
        a.dest = dest; a.rotated = rotated; a.paley = paley_table(m);
        a.sq = f32_sqrt(q); a.rsq = 1.0f / a.sq; a.hm = 1.0f / f32_sqrt(m);
        return launch_kron(&a, nullptr, true, m, q, group, s);
    }
    SegArgs a{};
    a.x = x; a.ldx = ldx; a.T = T; a.n = n;
    a.signs = signs; a.v = v; a.wt = wt; a.partial = part; a.splits = sp; a.k = k;
    a.codes = codes; a.scales = static_cast<uint16_t *>(scales); a.zeros = static_cast<uint16_t *>(zeros);
    a.dest = dest; a.rotated = rotated; a.sq = f32_sqrt(q); a.rsq = 1.0f / a.sq;
    return launch_seg(a, q, group, p.seg_mode, s);
}

// ------------------------------------------- allocation-free entry point

// Scratch of narhip_rotate_quant_noalloc: one copy per device, held from the
// library's load until the process ends.  Host code never passes `scratch`
// itself to a kernel (on the host it is a stand-in, not a device address):
// noalloc_scratch looks up each device's address once and every call uses that.
static __device__ __align__(256) unsigned char scratch[NARHIP_NOALLOC_SCRATCH_BYTES];

constexpr int SCRATCH_MAX_DEVICES = 64;

// The device address of `scratch` on the device that owns stream s (the
// current device for the null stream), looked up with that device current.
int noalloc_scratch(hipStream_t s, void **out)
{
    static std::mutex mu;
    static void *addr[SCRATCH_MAX_DEVICES] = {};
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return fail(NARHIP_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
    int dev = cur;
    if (s && (e = hipStreamGetDevice(s, &dev)) != hipSuccess)
        return fail(NARHIP_EHIP, "hipStreamGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= SCRATCH_MAX_DEVICES) return fail(NARHIP_EUNSUPPORTED, "device %d", dev);
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess)
            return fail(NARHIP_EHIP, "hipSetDevice(%d): %s", dev, hipGetErrorString(e));
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (dev != cur) (void)hipSetDevice(cur);
        if (e != hipSuccess) return fail(NARHIP_EHIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        if (!ptr) return fail(NARHIP_EHIP, "hipGetSymbolAddress(scratch) returned null");
        addr[dev] = ptr;
    }
    *out = addr[dev];
    return NARHIP_OK;
}

}  // namespace

extern "C" {

int narhip_abi_version(void) { return NARHIP_ABI_VERSION; }

const char *narhip_last_error_string(void) { return last_error(); }

int narhip_paley(int32_t m, int8_t *out_host)
{
    if (!out_host) return fail(NARHIP_EINVAL, "null output");
    int rc = build_paley(m, out_host);
    if (rc == -1) return fail(NARHIP_EUNSUPPORTED, "no Paley factor of order %d", m);
    if (rc) return fail(NARHIP_EINVAL, "Paley construction of order %d failed H H^T = mI", m);
    return NARHIP_OK;
}

size_t narhip_rank_factors_bytes(int64_t n, int32_t k)
{
    if (n <= 0 || k < 1 || k > 64) return 0;
    return prepared_bytes(n, k);
}

int narhip_prepare_rank_factors(const float *v, const float *w_t, int64_t n, int32_t k, void *prepared,
                                size_t prepared_bytes_given, void *stream)
{
    clear_error();
    if (n <= 0 || k < 1 || k > 64) return fail(NARHIP_EINVAL, "bad shape n=%lld k=%d", (long long)n, k);
    if (!prepared || !aligned16(prepared)) return fail(NARHIP_EINVAL, "prepared buffer missing or misaligned");
    if (prepared_bytes_given < prepared_bytes(n, k))
        return fail(NARHIP_EWORKSPACE, "prepared buffer of %zu bytes required", prepared_bytes(n, k));
    if (!v && !w_t) return fail(NARHIP_EINVAL, "no factor given");
    return launch_prepare(v, w_t, n, k, prepared, static_cast<hipStream_t>(stream));
}

size_t narhip_rotate_quant_workspace(int64_t tokens, int64_t n, int32_t had_m, int32_t had_q, int32_t k,
                                     int64_t rank_block, int32_t have_partial, int32_t splits,
                                     int32_t have_prepared, int32_t rank_mode)
{
    Plan p;
    if (make_plan(tokens, n, had_m, had_q, k, rank_block, have_partial != 0, splits, have_prepared != 0,
                  rank_mode, p))
        return 0;
    return p.total();
}

int narhip_rotate_quant(const void *x_bf16, int64_t tokens, int64_t n, int64_t ld_x,
                        int32_t had_m, int32_t had_q, const float *signs,
                        int32_t k, int64_t rank_block, const float *v, const float *w_t, const void *prepared,
                        const float *partial, int32_t splits,
                        int32_t group, uint8_t *codes, void *scales_f16, void *zeros_f16,
                        float *rotated, const int64_t *dest_rows, int32_t rank_mode,
                        void *workspace, size_t workspace_bytes, void *stream)
{
    clear_error();
    return run_rotate_quant(x_bf16, tokens, n, ld_x, had_m, had_q, signs, k, rank_block, v, w_t, prepared,
                            partial, splits, group, codes, scales_f16, zeros_f16, rotated, dest_rows, rank_mode,
                            workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int narhip_rotate_quant_noalloc(const void *x_bf16, int64_t tokens, int64_t n, int64_t ld_x,
                                int32_t had_m, int32_t had_q, const float *signs,
                                int32_t k, int64_t rank_block, const float *v, const float *w_t,
                                const void *prepared, const float *partial, int32_t splits,
                                int32_t group, uint8_t *codes, void *scales_f16, void *zeros_f16,
                                float *rotated, const int64_t *dest_rows, int32_t rank_mode, void *stream)
{
    clear_error();
    const size_t cap = (size_t)NARHIP_NOALLOC_SCRATCH_BYTES;
    Plan p;
    if (int rc = make_plan(tokens, n, had_m, had_q, k, rank_block, partial != nullptr, splits,
                           prepared != nullptr, rank_mode, p, cap))
        return rc;
    if (p.total() > cap)
        return fail(NARHIP_EWORKSPACE,
                    "these arguments need %zu bytes of scratch; the allocation-free entry point holds %zu "
                    "(call narhip_rotate_quant with a workspace)", p.total(), cap);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    void *ws = nullptr;
    if (p.total() > 0)
        if (int rc = noalloc_scratch(s, &ws)) return rc;
    return run_rotate_quant(x_bf16, tokens, n, ld_x, had_m, had_q, signs, k, rank_block, v, w_t, prepared,
                            partial, splits, group, codes, scales_f16, zeros_f16, rotated, dest_rows, rank_mode,
                            ws, cap, s, cap);
}

int narhip_rank_projection(const void *x_bf16, int64_t tokens, int64_t n, int64_t ld_x,
                           const float *v, const void *prepared, int32_t k, int32_t splits, float *partial,
                           int32_t rank_mode, void *stream)
{
    clear_error();
    if (tokens < 0 || n <= 0 || ld_x < n || ld_x % 8) return fail(NARHIP_EINVAL, "bad shape");
    if (k < 1 || k > 64) return fail(NARHIP_EUNSUPPORTED, "rank k=%d outside [1, 64]", k);
    if (splits < 1 || n % splits) return fail(NARHIP_EINVAL, "%lld channels do not divide into %d splits",
                                              (long long)n, splits);
    if (rank_mode < 0 || rank_mode > 2) return fail(NARHIP_EINVAL, "rank_mode %d", rank_mode);
    const bool mfma = rank_mode == NARHIP_RANK_MFMA ||
                      (rank_mode == NARHIP_RANK_AUTO && k >= 16 && prepared && mfma_projection_ok(n, splits));
    if (tokens > 0 && (!x_bf16 || !partial || (mfma ? !prepared : !v)))
        return fail(NARHIP_EINVAL, "null tensor argument");
    if (!aligned16(x_bf16) || !aligned16(prepared)) return fail(NARHIP_EINVAL, "x and prepared must be 16-byte aligned");
    if (mfma)
        return launch_proj_mfma(static_cast<const uint16_t *>(x_bf16), tokens, n, ld_x, prepared, k, splits, partial,
                                static_cast<hipStream_t>(stream));
    return launch_proj_exact(static_cast<const uint16_t *>(x_bf16), tokens, n, ld_x, v, k, splits, partial,
                             static_cast<hipStream_t>(stream));
}

int narhip_group_quant(const void *x_bf16, int64_t tokens, int64_t n, int64_t ld_x,
                       int32_t had_m, int32_t had_q, const float *partial, int32_t splits,
                       int32_t k, const float *w_t, const void *prepared, int32_t group,
                       uint8_t *codes, void *scales_f16, void *zeros_f16, int32_t rank_mode,
                       void *workspace, size_t workspace_bytes, void *stream)
{
    clear_error();
    if (k > 0 && !partial) return fail(NARHIP_EINVAL, "partials required");
    return run_rotate_quant(x_bf16, tokens, n, ld_x, had_m, had_q, nullptr, k, n, nullptr, w_t, prepared, partial,
                            splits, group, codes, scales_f16, zeros_f16, nullptr, nullptr, rank_mode,
                            workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int narhip_dequantize(const uint8_t *codes, const void *scales_f16, const void *zeros_f16,
                      int64_t rows, int64_t n, int32_t group, float *out, void *stream)
{
    clear_error();
    if (rows < 0 || n <= 0 || group <= 0 || n % group || group % 8)
        return fail(NARHIP_EINVAL, "bad shape rows=%lld n=%lld group=%d", (long long)rows, (long long)n, group);
    if (rows == 0) return NARHIP_OK;
    if (!codes || !scales_f16 || !zeros_f16 || !out) return fail(NARHIP_EINVAL, "null tensor argument");
    if (!aligned16(out) || (reinterpret_cast<uintptr_t>(codes) & 3u))
        return fail(NARHIP_EINVAL, "codes must be 4-byte and out 16-byte aligned");
    return launch_dequant(codes, static_cast<const uint16_t *>(scales_f16), static_cast<const uint16_t *>(zeros_f16),
                          rows, n, group, out, static_cast<hipStream_t>(stream));
}

// The hooks' fused form: one kernel where the transform kernel has the tuple
// epilogue (block or per-head segments with no rank term or per-block rank,
// the full-row FWHT, the Kronecker MFMA transform without a rank term);
// otherwise x' goes through the workspace and the standalone quantizer.
static bool tuple_one_pass(const Plan &p, int group, int q)
{
    if (group != 32 && group != 64 && group != 128) return false;
    if (q % group) return false;
    return p.path == PATH_FWHT || p.path == PATH_KRON_MFMA_QUANT || (p.path == PATH_SEG && !p.kron);
}

static bool tuple_group_ok(int64_t n, int group)
{
    return group > 0 && n % group == 0 && group % 8 == 0 && group <= 512 && !(group & (group - 1));
}

// The large Paley orders of the Qwen3 widths (paley_rows.hip): no Kronecker
// kernel, one exact kernel per row of H_m (x) H_q, fp32 out.
static bool large_paley(int m) { return m == 68 || m == 76 || m == 200; }

static int check_paley_rows(int64_t rows, int64_t n, int64_t ld_x, int32_t m, int32_t q)
{
    if (!pow2(q) || q > 1024 || (int64_t)m * q != n || n > PR_MAX_ELEMS)
        return fail(NARHIP_EUNSUPPORTED, "H_%d x H_%d: need n = m q, q a power of two <= 1024, n <= %d", m, q,
                    PR_MAX_ELEMS);
    if (ld_x < n || ld_x % 8) return fail(NARHIP_EINVAL, "ld_x=%lld must be >= n and a multiple of 8", (long long)ld_x);
    if (rows > 0x7fffffff) return fail(NARHIP_EUNSUPPORTED, "too many rows");
    return NARHIP_OK;
}

static int run_paley_rows(const void *x_bf16, int64_t rows, int64_t n, int64_t ld_x, int32_t m, int32_t q,
                          const float *signs, float *out, void *stream, const float *corr = nullptr)
{
    if (int rc = check_paley_rows(rows, n, ld_x, m, q)) return rc;
    if (rows == 0) return NARHIP_OK;
    if (!x_bf16 || !out) return fail(NARHIP_EINVAL, "null tensor argument");
    if (!aligned16(x_bf16) || !aligned16(out)) return fail(NARHIP_EINVAL, "x and out must be 16-byte aligned");
    PaleyRowsArgs pa{};
    pa.x = static_cast<const uint16_t *>(x_bf16); pa.ldx = ld_x; pa.T = rows; pa.signs = signs; pa.out = out;
    pa.corr = corr; pa.m = m; pa.q = q;
    if (!paley_zp(m, pa.p, pa.kind)) return fail(NARHIP_EUNSUPPORTED, "no Z_p construction of order %d", m);
    for (int v = 1; v < pa.p; v++) {
        const int d = (v * v) % pa.p;
        pa.residue[d >> 5] |= 1u << (d & 31);
    }
    // |entry|: the fp64 1/sqrt(m) for 68 and 200, whose product the reference
    // forms in fp64; otherwise fp32(1) / fp32(sqrt m)
    pa.fp64_product = m == 68 || m == 200;
    pa.sq = f32_sqrt(q);
    pa.hm = pa.fp64_product ? 1.0 / std::sqrt((double)m) : (double)(1.0f / f32_sqrt(m));
    return launch_paley_rows(pa, static_cast<hipStream_t>(stream));
}

// Workspace of the large-Paley tuple path: x' fp32, and with a full-row rank
// term (k <= 64, exact) the projection u and the correction C before it.
static size_t paley_tuple_bytes(int64_t tokens, int64_t n, int32_t k)
{
    const size_t T = (size_t)tokens, N = (size_t)n;
    return align256(4 * T * N) + (k > 0 ? align256(4 * T * (size_t)k) + align256(4 * T * N) : 0);
}
static bool paley_rank_ok(int64_t n, int32_t k, int64_t rank_block)
{
    return k == 0 || (k >= 1 && k <= 64 && rank_block == n && n % 64 == 0);
}

size_t narhip_rotate_dynamic_asym_int4_workspace(int64_t tokens, int64_t n, int32_t had_m, int32_t had_q, int32_t k,
                                                 int64_t rank_block, int32_t group, int32_t rank_mode)
{
    if (large_paley(had_m)) {
        if (tokens <= 0 || !tuple_group_ok(n, group) || !paley_rank_ok(n, k, rank_block) ||
            check_paley_rows(tokens, n, n, had_m, had_q))
            return 0;
        return paley_tuple_bytes(tokens, n, k);
    }
    Plan p;
    if (tokens < 0 || !tuple_group_ok(n, group) ||
        make_plan(tokens, n, had_m, had_q, k, rank_block, false, 0, false, rank_mode, p))
        return 0;
    if (tuple_one_pass(p, group, had_q)) return 0;
    const size_t T = (size_t)tokens, N = (size_t)n;
    return align256(p.total()) + align256(4 * T * N) + align256(T * N / 2) + 2 * align256(2 * T * (N / 128));
}

int narhip_rotate_dynamic_asym_int4(const void *x_bf16, int64_t tokens, int64_t n, int64_t ld_x, int32_t had_m,
                                    int32_t had_q, const float *signs, int32_t k, int64_t rank_block, const float *v,
                                    const float *w_t, int32_t group, uint8_t *codes, void *scales_f16,
                                    void *zeros_f16, float *deq, int32_t rank_mode, void *workspace,
                                    size_t workspace_bytes, void *stream)
{
    clear_error();
    if (large_paley(had_m)) {
        // x' of the Paley rows staged in the workspace (with a full-row rank
        // term: exact projection and correction first), then the hooks' quantizer
        if (!paley_rank_ok(n, k, rank_block))
            return fail(NARHIP_EUNSUPPORTED, "H_%d rows: rank term needs k <= 64 over the whole row, n %% 64 == 0",
                        had_m);
        if (k > 0 && (!v || !w_t)) return fail(NARHIP_EINVAL, "rank factors missing");
        if (!tuple_group_ok(n, group))
            return fail(NARHIP_EINVAL, "group size %d: need a power of two in [8, 512] dividing %lld", group,
                        (long long)n);
        if (tokens < 0) return fail(NARHIP_EINVAL, "bad token count %lld", (long long)tokens);
        if (int rc = check_paley_rows(tokens, n, ld_x, had_m, had_q)) return rc;
        if (tokens == 0) return NARHIP_OK;
        if (!x_bf16 || !codes || !scales_f16 || !zeros_f16 || !deq) return fail(NARHIP_EINVAL, "null tensor argument");
        if (!aligned16(x_bf16) || !aligned16(deq) || (reinterpret_cast<uintptr_t>(codes) & 7u))
            return fail(NARHIP_EINVAL, "x and deq must be 16-byte aligned, codes 8-byte aligned");
        const size_t need = paley_tuple_bytes(tokens, n, k);
        if (!workspace || workspace_bytes < need)
            return fail(NARHIP_EWORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
        if (!aligned16(workspace)) return fail(NARHIP_EINVAL, "workspace must be 16-byte aligned");
        // every argument is checked before the first launch
        float *rot = static_cast<float *>(workspace);
        float *corr = nullptr;
        if (k > 0) {
            hipStream_t hs = static_cast<hipStream_t>(stream);
            float *u = reinterpret_cast<float *>(static_cast<char *>(workspace) + align256(4 * (size_t)tokens * (size_t)n));
            corr = reinterpret_cast<float *>(reinterpret_cast<char *>(u) + align256(4 * (size_t)tokens * (size_t)k));
            if (int rc = launch_proj_exact(static_cast<const uint16_t *>(x_bf16), tokens, n, ld_x, v, k, 1, u, hs))
                return rc;
            if (int rc = launch_corr_exact(u, 1, k, w_t, tokens, n, corr, hs)) return rc;
        }
        if (int rc = run_paley_rows(x_bf16, tokens, n, ld_x, had_m, had_q, signs, rot, stream, corr)) return rc;
        return launch_quant_tuple(DT_F32, rot, tokens * n, group, codes, static_cast<uint16_t *>(scales_f16),
                                  static_cast<uint16_t *>(zeros_f16), deq, static_cast<hipStream_t>(stream));
    }
    Plan p;
    if (int rc = make_plan(tokens, n, had_m, had_q, k, rank_block, false, 0, false, rank_mode, p)) return rc;
    if (!tuple_group_ok(n, group))
        return fail(NARHIP_EINVAL, "group size %d: need a power of two in [8, 512] dividing %lld", group,
                    (long long)n);
    if (ld_x < n || ld_x % 8) return fail(NARHIP_EINVAL, "ld_x=%lld must be >= n and a multiple of 8", (long long)ld_x);
    if (tokens == 0) return NARHIP_OK;
    if (!x_bf16 || !codes || !scales_f16 || !zeros_f16 || !deq) return fail(NARHIP_EINVAL, "null tensor argument");
    if (!aligned16(x_bf16) || !aligned16(deq) || (reinterpret_cast<uintptr_t>(codes) & 7u))
        return fail(NARHIP_EINVAL, "x and deq must be 16-byte aligned, codes 8-byte aligned");
    if (k > 0 && (!v || !w_t)) return fail(NARHIP_EINVAL, "rank factors missing");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint16_t *x = static_cast<const uint16_t *>(x_bf16);
    uint16_t *sc = static_cast<uint16_t *>(scales_f16), *zc = static_cast<uint16_t *>(zeros_f16);
    if (tuple_one_pass(p, group, had_q)) {
        if (p.path == PATH_FWHT) {
            FwhtArgs fa{};
            fa.x = x; fa.ldx = ld_x; fa.T = tokens; fa.signs = signs;
            fa.codes = codes; fa.scales = sc; fa.zeros = zc; fa.deq = deq;
            fa.sq = f32_sqrt(had_q); fa.rsq = 1.0f / fa.sq;
            return launch_fwht(fa, had_q, group, s);
        }
        if (p.path == PATH_KRON_MFMA_QUANT) {
            KronArgs ka{};
            ka.x = x; ka.ldx = ld_x; ka.T = tokens; ka.n = n; ka.signs = signs;
            ka.codes = codes; ka.scales = sc; ka.zeros = zc; ka.deq = deq;
            ka.paley = paley_table(had_m); ka.sq = f32_sqrt(had_q); ka.rsq = 1.0f / ka.sq;
            ka.hm = 1.0f / f32_sqrt(had_m);
            return launch_kron(nullptr, &ka, true, had_m, had_q, group, s);
        }
        SegArgs sa{};
        sa.x = x; sa.ldx = ld_x; sa.T = tokens; sa.n = n; sa.signs = signs; sa.v = v; sa.wt = w_t; sa.k = k;
        sa.codes = codes; sa.scales = sc; sa.zeros = zc; sa.deq = deq;
        sa.sq = f32_sqrt(had_q); sa.rsq = 1.0f / sa.sq;
        return launch_seg(sa, had_q, group, p.seg_mode, s);
    }
    // two passes: the fused operator into the workspace (x' in fp32; its own
    // group-128 codes are scratch), then the hooks' quantizer on x'
    const size_t T = (size_t)tokens, N = (size_t)n;
    const size_t need = narhip_rotate_dynamic_asym_int4_workspace(tokens, n, had_m, had_q, k, rank_block, group,
                                                                  rank_mode);
    if (!workspace || workspace_bytes < need)
        return fail(NARHIP_EWORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
    char *w = static_cast<char *>(workspace);
    const size_t rq = p.total();
    float *rot = reinterpret_cast<float *>(w + align256(rq));
    uint8_t *pc = reinterpret_cast<uint8_t *>(rot) + align256(4 * T * N);
    uint16_t *ps = reinterpret_cast<uint16_t *>(pc + align256(T * N / 2));
    uint16_t *pz = reinterpret_cast<uint16_t *>(reinterpret_cast<char *>(ps) + align256(2 * T * (N / 128)));
    if (int rc = run_rotate_quant(x_bf16, tokens, n, ld_x, had_m, had_q, signs, k, rank_block, v, w_t, nullptr,
                                  nullptr, 0, 128, pc, ps, pz, rot, nullptr, rank_mode, rq ? w : nullptr, rq, s))
        return rc;
    return launch_quant_tuple(DT_F32, rot, tokens * n, group, codes, sc, zc, deq, s);
}

int narhip_dynamic_asym_int4(const void *x, int32_t dtype, int64_t rows, int64_t n, int32_t group,
                             uint8_t *codes, void *scales_f16, void *zeros_f16, void *deq, void *stream)
{
    clear_error();
    if (rows < 0 || n <= 0) return fail(NARHIP_EINVAL, "bad shape rows=%lld n=%lld", (long long)rows, (long long)n);
    if (group <= 0 || n % group)
        return fail(NARHIP_EINVAL, "last dimension %lld is not divisible by group size %d", (long long)n, group);
    if (group % 8 || group > 512 || (group & (group - 1)))
        return fail(NARHIP_EUNSUPPORTED, "group size %d: need a power of two in [8, 512]", group);
    if (dtype < DT_F32 || dtype > DT_F16) return fail(NARHIP_EINVAL, "dtype code %d", dtype);
    if (rows == 0) return NARHIP_OK;
    if (!x || !codes || !scales_f16 || !zeros_f16 || !deq) return fail(NARHIP_EINVAL, "null tensor argument");
    if (!aligned16(x) || !aligned16(deq) || (reinterpret_cast<uintptr_t>(codes) & 7u))
        return fail(NARHIP_EINVAL, "x and deq must be 16-byte aligned, codes 8-byte aligned");
    return launch_quant_tuple(dtype, x, rows * n, group, codes, static_cast<uint16_t *>(scales_f16),
                              static_cast<uint16_t *>(zeros_f16), deq, static_cast<hipStream_t>(stream));
}

int narhip_hadamard_rows(const void *x_bf16, int64_t rows, int64_t n, int64_t ld_x, int32_t had_m, int32_t had_q,
                         const float *signs, float *out, void *stream)
{
    clear_error();
    if (rows < 0 || n <= 0) return fail(NARHIP_EINVAL, "bad shape rows=%lld n=%lld", (long long)rows, (long long)n);
    if (large_paley(had_m)) return run_paley_rows(x_bf16, rows, n, ld_x, had_m, had_q, signs, out, stream);
    const bool full = had_m == 1 && had_q == n && fwht_rows_width(n);
    if (!full && (!pow2(had_q) || had_q < 128 || had_q > 1024))
        return fail(NARHIP_EUNSUPPORTED,
                    "Hadamard block width %d: need a power of two in [128, 1024] (or q = n in [2048, 8192])", had_q);
    if (had_m != 1 && had_m != 12 && had_m != 20 && had_m != 28)
        return fail(NARHIP_EUNSUPPORTED, "no Paley factor of order %d", had_m);
    if ((int64_t)had_m * had_q != n && !(had_m == 1 && n % had_q == 0))
        return fail(NARHIP_EUNSUPPORTED, "H_%d x H_%d does not tile a row of %lld", had_m, had_q, (long long)n);
    if (ld_x < n || ld_x % 8) return fail(NARHIP_EINVAL, "ld_x=%lld must be >= n and a multiple of 8", (long long)ld_x);
    if (rows == 0) return NARHIP_OK;
    if (!x_bf16 || !out) return fail(NARHIP_EINVAL, "null tensor argument");
    if (!aligned16(x_bf16) || !aligned16(out)) return fail(NARHIP_EINVAL, "x and out must be 16-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint16_t *x = static_cast<const uint16_t *>(x_bf16);
    if (full) {
        FwhtArgs fa{};
        fa.x = x; fa.ldx = ld_x; fa.T = rows; fa.signs = signs; fa.rotated = out;
        fa.sq = f32_sqrt(had_q); fa.rsq = 1.0f / fa.sq;
        return launch_fwht(fa, had_q, 128, s);
    }
    if (had_m > 1) {
        KronArgs ka{};
        ka.x = x; ka.ldx = ld_x; ka.T = rows; ka.n = n; ka.signs = signs; ka.P = out;
        ka.paley = paley_table(had_m); ka.sq = f32_sqrt(had_q); ka.rsq = 1.0f / ka.sq;
        ka.hm = 1.0f / f32_sqrt(had_m);
        return launch_kron(nullptr, &ka, false, had_m, had_q, 128, s);
    }
    SegArgs sa{};
    sa.x = x; sa.ldx = ld_x; sa.T = rows; sa.n = n; sa.signs = signs; sa.k = 0;
    sa.codes = nullptr; sa.rotated = out; sa.sq = f32_sqrt(had_q); sa.rsq = 1.0f / sa.sq;
    return launch_seg(sa, had_q, 128, RANK_NONE, s);
}


size_t narhip_transform_f16_workspace(int64_t tokens, int64_t n, int32_t k)
{
    if (tokens <= 0 || n <= 0 || k <= 0 || k > 64) return 0;
    size_t fast = 0;
    if (k <= XF_K && n % 128 == 0)
        fast = xf_pd_bytes(tokens, xf_splits(tokens, n));
    const int sp = f64_splits(tokens, n);
    const size_t seg = align256(sizeof(double) * (size_t)tokens * (size_t)sp * (size_t)f64_kmax(k)) +
                       align256(sizeof(float) * (size_t)tokens * (size_t)k);
    return fast > seg ? fast : seg;
}

int narhip_rank_projection_f16(const void *x_f16, int64_t tokens, int64_t n, int64_t ld_x, const float *v,
                               int32_t k, int32_t splits, float *partial, void *stream)
{
    clear_error();
    if (tokens < 0 || n <= 0 || ld_x < n || ld_x % 8) return fail(NARHIP_EINVAL, "bad shape");
    if (k < 1 || k > 64) return fail(NARHIP_EUNSUPPORTED, "fp16 projection supports rank k in [1, 64] (got %d)", k);
    if (splits < 1 || n % splits || (n / splits) % 2)
        return fail(NARHIP_EINVAL, "%lld channels do not divide into %d even splits", (long long)n, splits);
    if (tokens == 0) return NARHIP_OK;
    if (!x_f16 || !v || !partial) return fail(NARHIP_EINVAL, "null tensor argument");
    if (!aligned16(x_f16) || !aligned16(v)) return fail(NARHIP_EINVAL, "x and v must be 16-byte aligned");
    return launch_proj_f64(static_cast<const uint16_t *>(x_f16), tokens, n, ld_x, v, k, splits, nullptr,
                           static_cast<hipStream_t>(stream), true, partial);
}

int narhip_transform_f16(const void *x_f16, int64_t tokens, int64_t n, int64_t ld_x, int32_t had_q,
                         const float *v, const float *partial, int32_t splits, const float *w_t, int32_t k,
                         void *out_f16, void *workspace, size_t workspace_bytes, void *stream)
{
    clear_error();
    if (tokens < 0 || n <= 0) return fail(NARHIP_EINVAL, "bad shape tokens=%lld n=%lld", (long long)tokens, (long long)n);
    if (!pow2(had_q) || had_q < 128 || had_q > 1024 || n % had_q)
        return fail(NARHIP_EUNSUPPORTED, "block Hadamard width %d must be a power of two in [128, 1024] dividing n",
                    had_q);
    if (k < 0 || k > 64) return fail(NARHIP_EUNSUPPORTED, "fp16 transform supports rank k <= 64 (got %d)", k);
    if (ld_x < n || ld_x % 8) return fail(NARHIP_EINVAL, "ld_x=%lld must be >= n and a multiple of 8", (long long)ld_x);
    if (partial && (splits < 1 || k < 1)) return fail(NARHIP_EINVAL, "partials need splits >= 1 and k >= 1");
    if (tokens == 0) return NARHIP_OK;
    if (!x_f16 || !out_f16 || (k > 0 && (!w_t || (!partial && !v)))) return fail(NARHIP_EINVAL, "null tensor argument");
    const bool fast = xf_fast(had_q, k);
    const size_t need = partial ? 0 : narhip_transform_f16_workspace(tokens, n, k);
    if (need > 0 && (!workspace || workspace_bytes < need))
        return fail(NARHIP_EWORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
    if (!aligned16(x_f16) || !aligned16(out_f16) || !aligned16(w_t) || !aligned16(v))
        return fail(NARHIP_EINVAL, "x, out, v and w_t must be 16-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint16_t *x = static_cast<const uint16_t *>(x_f16);
    int rc;
    if (fast) {
        double *pd = nullptr;
        int S = splits;
        if (!partial) {
            S = xf_splits(tokens, n);
            pd = static_cast<double *>(workspace);
            if ((rc = launch_proj_tok(x, tokens, n, ld_x, v, k, S, pd, nullptr, s))) return rc;
        }
        return launch_xform128(x, tokens, n, ld_x, w_t, pd, partial, S, k, static_cast<uint16_t *>(out_f16), s);
    }
    SegArgs a{};
    a.splits = 1;
    if (partial) {
        a.partial = partial;
        a.splits = splits;
    } else if (k > 0) {
        const int sp = f64_splits(tokens, n);
        double *pd = static_cast<double *>(workspace);
        float *u = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                             align256(sizeof(double) * (size_t)tokens * (size_t)sp * (size_t)f64_kmax(k)));
        if ((rc = launch_proj_f64(x, tokens, n, ld_x, v, k, sp, pd, s, true))) return rc;
        if ((rc = launch_fold_f64(pd, sp, f64_kmax(k), k, tokens, u, s))) return rc;
        a.partial = u;
    }
    a.x = x; a.ldx = ld_x; a.T = tokens; a.n = n; a.signs = nullptr;
    a.wt = w_t; a.k = k;
    a.codes = nullptr; a.rotated = static_cast<float *>(out_f16);
    a.sq = f32_sqrt(had_q); a.rsq = 1.0f / a.sq;
    return launch_seg_f16(a, had_q, k, s);
}

namespace {
// Reduction splits of the W4A4 GEMM: enough workgroups for the 256 CUs when
// the output tiles alone are few (decode), at least two groups per split.
int w4a4_splits(int64_t tokens, int64_t out_features, int64_t n)
{
    const int64_t tiles = ((out_features + WQ_TN - 1) / WQ_TN) * ((tokens + WQ_TM - 1) / WQ_TM);
    const int64_t G = n / 128;
    int64_t s = 1;
    while (tiles * s * 2 <= 512 && G / (s * 2) >= 2) s *= 2;
    return (int)s;
}
}  // namespace

size_t narhip_w4a4_workspace(int64_t tokens, int64_t out_features, int64_t n)
{
    if (tokens <= 0 || out_features <= 0 || n <= 0 || n % 128) return 0;
    const int s = w4a4_splits(tokens, out_features, n);
    return s == 1 ? 0 : sizeof(float) * (size_t)s * (size_t)tokens * (size_t)out_features;
}

int narhip_w4a4_gemm(const uint8_t *a_codes, const void *a_scales, const void *a_zeros, int64_t tokens,
                     const uint8_t *w_codes, const void *w_scales, const void *w_zeros, int64_t out_features,
                     int64_t n, int32_t group, float *out, int64_t ld_out, void *workspace, size_t workspace_bytes,
                     void *stream)
{
    clear_error();
    if (tokens < 0 || out_features < 0 || n <= 0)
        return fail(NARHIP_EINVAL, "bad shape tokens=%lld out_features=%lld n=%lld", (long long)tokens,
                    (long long)out_features, (long long)n);
    if (group != 128) return fail(NARHIP_EUNSUPPORTED, "W4A4 GEMM is built for groups of 128 (got %d)", group);
    if (n % 128) return fail(NARHIP_EINVAL, "n=%lld is not a multiple of the group size", (long long)n);
    if (ld_out < out_features) return fail(NARHIP_EINVAL, "ld_out=%lld < out_features", (long long)ld_out);
    if (tokens == 0 || out_features == 0) return NARHIP_OK;
    if (!a_codes || !a_scales || !a_zeros || !w_codes || !w_scales || !w_zeros || !out)
        return fail(NARHIP_EINVAL, "null tensor argument");
    if (!aligned16(a_codes) || !aligned16(w_codes) || (reinterpret_cast<uintptr_t>(a_scales) |
        reinterpret_cast<uintptr_t>(a_zeros) | reinterpret_cast<uintptr_t>(w_scales) |
        reinterpret_cast<uintptr_t>(w_zeros) | reinterpret_cast<uintptr_t>(out)) & 3u)
        return fail(NARHIP_EINVAL, "codes must be 16-byte aligned, scales, zeros and out 4-byte aligned");
    const int64_t gx = (out_features + WQ_TN - 1) / WQ_TN, gy = (tokens + WQ_TM - 1) / WQ_TM;
    if (gy > 65535) return fail(NARHIP_EUNSUPPORTED, "too many tokens for one launch");
    const int splits = w4a4_splits(tokens, out_features, n);
    const size_t need = narhip_w4a4_workspace(tokens, out_features, n);
    if (need && (!workspace || workspace_bytes < need || !aligned16(workspace)))
        return fail(NARHIP_EWORKSPACE, "workspace of %zu bytes (16-byte aligned) required, %zu given", need,
                    workspace_bytes);
    hipStream_t s = static_cast<hipStream_t>(stream);
    float *part = splits == 1 ? out : static_cast<float *>(workspace);
    W4A4Args a{a_codes, static_cast<const uint16_t *>(a_scales), static_cast<const uint16_t *>(a_zeros), tokens,
               w_codes, static_cast<const uint16_t *>(w_scales), static_cast<const uint16_t *>(w_zeros),
               out_features, n, part, ld_out, splits};
    return launch_w4a4(a, gx, gy, out, s);
}

int narhip_mfma_probe(const void *a_bf16, const void *b_bf16, float *d, void *stream)
{
    clear_error();
    if (!a_bf16 || !b_bf16 || !d) return fail(NARHIP_EINVAL, "null argument");
    return launch_mfma_probe(static_cast<const __bf16 *>(a_bf16), static_cast<const __bf16 *>(b_bf16), d,
                             static_cast<hipStream_t>(stream));
}

}  // extern "C"
