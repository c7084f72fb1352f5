/*
 * mxfp8_oracle.c - CPU restatement of the reference's MXFP8 FMHA forward.
 *
 * TEST INFRASTRUCTURE ONLY (see mxfp8_oracle.h): used by tests/, the smoke
 * check and bench.py's cpu_baseline leg; never by the product path.
 *
 * Parity pins (what checks each function; tests/test_oracle.py):
 *   e4m3 decode/encode     all 256 / brute force against the decode table
 *   cvt_bf16_fp8, pknorm   the gfx950 hardware on all 65536 bf16 inputs
 *                          (tests/golden/isa_conversions.json, measured)
 *   generate               reference-published statistics + independent
 *                          numpy restatement of ref_host.cpp:208-263
 *   select_path            the reference's tabulated choices (docs/perf-matrix.md)
 *   check_fp64             a numpy float64 softmax on small shapes
 *   emulate                closed-form invariants (uniform scores, one-hot V,
 *                          split == full when splits cover one range) and the
 *                          lazy-vs-naive recurrence known answers of
 *                          crates/amdgpu-codegen/tests/functional_proofs.rs:37-69
 */
#include "mxfp8_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#define D 128

/* V element scale: 2^(E8M0 - 127) of its 32-key block and column under per-32 V scales (extension), else 1 */
static inline double v_block_scale(const mxo_problem* p, int b, int key, int kvh, int d) {
    if (!p->vs32) return 1.0;
    const size_t nb = ((size_t)p->SK + 31) / 32;
    return ldexp(1.0, (int)p->vs32[(((size_t)b * nb + (size_t)key / 32) * p->HK + kvh) * D + d] - 127);
}
/* the per-tensor V descale the output is multiplied by (1 under per-32 V scales) */
static inline float v_tensor_descale(const mxo_problem* p) { return p->vs32 ? 1.0f : p->vdescale; }

/* The in-kernel softmax scale (extension, qk_scale > 0): c = f32(qk_scale * log2 e) = 2^e m with m in [1, 2). The
 * kernel adds e to the Q scale exponents (exact) and multiplies S by m; the seed of S is b / m, so that
 * m (S + b / m) carries the bias. Without the extension c = 1 (e = 0, m = 1). */
typedef struct { float c, m, rm; int e; } qk_scaling;
static qk_scaling qk_scaling_of(const mxo_problem* p) {
    qk_scaling r = {1.0f, 1.0f, 1.0f, 0};
    if (!(p->qk_scale > 0.0f)) return r;
    r.c = p->qk_scale * 1.44269504088896340736f;
    uint32_t u;
    memcpy(&u, &r.c, 4);
    r.e = (int)((u >> 23) & 0xffu) - 127;
    u = (u & 0x007fffffu) | (127u << 23);
    memcpy(&r.m, &u, 4);
    r.rm = 1.0f / r.m;
    return r;
}
/* natural-log score multiplier of the fp64 check: ln 2 per base-2 unit, times c */
static double score_mul(const mxo_problem* p) { return 0.6931471805599453 * (double)qk_scaling_of(p).c; }

/* ------------------------------------------------------------------ scalars */

double mxo_e4m3_decode(uint8_t b) {
    /* ref_host.cpp:26-33 */
    const int s = (b >> 7) & 1, e = (b >> 3) & 0xF, m = b & 0x7;
    double v;
    if (e == 0xF && m == 0x7) v = 0.0;
    else if (e == 0) v = (m / 8.0) * ldexp(1.0, -6);
    else v = (1.0 + m / 8.0) * ldexp(1.0, e - 7);
    return s ? -v : v;
}

static float g_e4m3_pos[127];
static pthread_once_t g_once = PTHREAD_ONCE_INIT;
static double g_e4m3_val[256];
static void init_tables(void) {
    for (int b = 0; b < 127; ++b) g_e4m3_pos[b] = (float)mxo_e4m3_decode((uint8_t)b);
    for (int b = 0; b < 256; ++b) g_e4m3_val[b] = mxo_e4m3_decode((uint8_t)b);
}

uint8_t mxo_e4m3_encode_sat(float x) {
    /* ref_host.cpp:216-228: RNE, ties to the even byte, saturating at 448 */
    pthread_once(&g_once, init_tables);
    const uint8_t sgn = x < 0 ? 0x80 : 0;
    const float a = fabsf(x);
    if (!(a < 448.0f)) return sgn | 126;
    /* upper_bound(pos, a) - 1 */
    int lo = 0, hi_i = 127;
    while (lo < hi_i) {
        int mid = (lo + hi_i) / 2;
        if (g_e4m3_pos[mid] <= a) lo = mid + 1; else hi_i = mid;
    }
    lo = lo - 1;
    if (lo < 0) lo = 0;
    const int hi = lo + 1 < 127 ? lo + 1 : lo;
    const float dl = a - g_e4m3_pos[lo], dh = g_e4m3_pos[hi] - a;
    const int pick = dh < dl ? hi : dl < dh ? lo : (lo % 2 == 0 ? lo : hi);
    return sgn | (uint8_t)pick;
}

float mxo_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t mxo_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float mxo_f16_to_f32(uint16_t h) {
    const int s = (h >> 15) & 1, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 0x400), e - 25);
    return s ? -v : v;
}

uint16_t mxo_f32_to_f16(float f) {
    /* round to nearest even, IEEE binary16 */
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t au = u & 0x7fffffffu;
    if (au > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (au >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    float a;
    memcpy(&a, &au, 4);
    if (au < 0x38800000u) { /* below 2^-14: subnormal, quantum 2^-24 */
        const float q = a * 16777216.0f; /* exact scaling */
        const float r = nearbyintf(q);   /* default rounding mode: RNE */
        return (uint16_t)(sign | (uint32_t)r);
    }
    const int e = (int)(au >> 23) - 127;            /* -14..15 */
    const uint32_t mant = au & 0x7fffffu;
    uint32_t h = (uint32_t)(e + 15) << 10 | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1;
    return (uint16_t)(sign | h);
}

uint16_t mxo_pknorm_u16(float x) {
    const double c = x < 0.0f ? 0.0 : (x > 1.0f ? 1.0 : (double)x);
    if (x != x) return 0;
    return (uint16_t)nearbyint(c * 65535.0);
}

uint8_t mxo_cvt_bf16_fp8(uint16_t bf16, float scale) {
    const float f = mxo_bf16_to_f32(bf16);
    if (f != f) return 0xff;   /* gfx950 returns the negative NaN byte for any NaN input */
    const double x = (double)f / (double)scale;
    const uint8_t sgn = (signbit(x) ? 0x80 : 0);
    const double a = fabs(x);
    if (a > 464.0) return sgn | 0x7f;
    if (a >= 448.0) return sgn | 126;
    pthread_once(&g_once, init_tables);
    int lo = 0, hi_i = 127;
    while (lo < hi_i) {
        int mid = (lo + hi_i) / 2;
        if ((double)g_e4m3_pos[mid] <= a) lo = mid + 1; else hi_i = mid;
    }
    lo -= 1;
    if (lo < 0) lo = 0;
    const int hi = lo + 1 < 127 ? lo + 1 : lo;
    const double dl = a - g_e4m3_pos[lo], dh = g_e4m3_pos[hi] - a;
    const int pick = dh < dl ? hi : dl < dh ? lo : (lo % 2 == 0 ? lo : hi);
    return sgn | (uint8_t)pick;
}

/* --------------------------------------------------------------- generator */

size_t mxo_qs_bytes(int B, int H, int S) { return (size_t)B * S * H * 4 + (size_t)(256 + 256) * H * 4; }
size_t mxo_ks_bytes(int B, int H, int HK, int SK) { return (size_t)B * SK * HK * 4 + (size_t)(512 + 128) * H * 4; }

typedef struct { uint64_t st; } xs64;
static uint64_t xs_next(xs64* r) { r->st ^= r->st << 13; r->st ^= r->st >> 7; r->st ^= r->st << 17; return r->st; }
static double xs_unif(xs64* r) { return (double)(xs_next(r) >> 11) * (1.0 / 9007199254740992.0); }
static double xs_gauss(xs64* r) {
    double u1 = xs_unif(r);
    double u2 = xs_unif(r);
    if (u1 < 1e-300) u1 = 1e-300;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

static void quant_rows(xs64* r, uint8_t* dst, uint8_t* sc, long nrows, int heads, double mul) {
    /* ref_host.cpp:239-251: E8M0 = clamp(floor(log2 amax) - 8 + 127, 0, 254), e4m3 RNE saturating */
    double blk[32];
    for (long row = 0; row < nrows; ++row)
        for (int h = 0; h < heads; ++h)
            for (int bk = 0; bk < 4; ++bk) {
                double amax = 0;
                for (int i = 0; i < 32; ++i) {
                    blk[i] = xs_gauss(r) * mul;
                    amax = fmax(amax, fabs(blk[i]));
                }
                const int e = amax > 0 ? (int)floor(log2(amax)) - 8 : -127;
                int eb = e + 127;
                if (eb < 0) eb = 0;
                if (eb > 254) eb = 254;
                sc[((size_t)row * heads + h) * 4 + bk] = (uint8_t)eb;
                const double inv = ldexp(1.0, -(eb - 127));
                for (int i = 0; i < 32; ++i) dst[((size_t)row * heads + h) * D + 32 * bk + i] = mxo_e4m3_encode_sat((float)(blk[i] * inv));
            }
}

float mxo_generate(int mode, int B, int H, int HK, int S, int SK, uint64_t seed_mix,
                   uint8_t* q, uint8_t* k, uint8_t* v, uint8_t* qs, uint8_t* ks) {
    /* ref_host.cpp:183-263 */
    static const uint8_t palette[11] = {0x00, 0x20, 0x28, 0x30, 0x38, 0x3C, 0x40, 0xA0, 0xA8, 0xB0, 0xB8};
    uint32_t seed = 20260101u ^ (uint32_t)seed_mix;
#define RND() (seed = seed * 1664525u + 1013904223u, (seed >> 16) & 0xFFu)
    const size_t nq = (size_t)B * S * H * D, nk = (size_t)B * SK * HK * D;
    for (size_t i = 0; i < nq; ++i) q[i] = palette[RND() % 11];
    for (size_t i = 0; i < nk; ++i) k[i] = palette[RND() % 11];
    for (size_t i = 0; i < nk; ++i) v[i] = palette[RND() % 11];
    memset(qs, 0, mxo_qs_bytes(B, H, S));
    memset(ks, 0, mxo_ks_bytes(B, H, HK, SK));
    for (int b = 0; b < B; ++b)
        for (int s = 0; s < S; ++s)
            for (int h = 0; h < H; ++h)
                for (int blk = 0; blk < 4; ++blk) qs[(((size_t)b * S + s) * H + h) * 4 + blk] = (uint8_t)(126 + RND() % 3);
    for (int b = 0; b < B; ++b)
        for (int s = 0; s < SK; ++s)
            for (int h = 0; h < HK; ++h)
                for (int blk = 0; blk < 4; ++blk) ks[(((size_t)b * SK + s) * HK + h) * 4 + blk] = (uint8_t)(126 + RND() % 3);
#undef RND
    float vdescale = 1.0f;
    if (mode == 0) return vdescale;
    xs64 r = {0x9E3779B97F4A7C15ull ^ seed_mix};
    if (mode == 1) {
        for (size_t i = 0; i < nq; ++i) { uint8_t x; do { x = (uint8_t)(xs_next(&r) >> 56); } while ((x & 0x7F) == 0x7F); q[i] = x; }
        for (size_t i = 0; i < nk; ++i) { uint8_t x; do { x = (uint8_t)(xs_next(&r) >> 56); } while ((x & 0x7F) == 0x7F); k[i] = x; }
        for (size_t i = 0; i < nk; ++i) { uint8_t x; do { x = (uint8_t)(xs_next(&r) >> 56); } while ((x & 0x7F) == 0x7F); v[i] = x; }
        return vdescale;
    }
    const double qmul = 1.4426950408889634 / sqrt((double)D);
    quant_rows(&r, q, qs, (long)B * S, H, qmul);
    quant_rows(&r, k, ks, (long)B * SK, HK, 1.0);
    double* vv = (double*)malloc(nk * sizeof(double));
    double vmax = 0;
    for (size_t i = 0; i < nk; ++i) { vv[i] = xs_gauss(&r); vmax = fmax(vmax, fabs(vv[i])); }
    vdescale = (float)(vmax / 448.0);
    for (size_t i = 0; i < nk; ++i) v[i] = mxo_e4m3_encode_sat((float)(vv[i] / vdescale));
    free(vv);
    return vdescale;
}

/* ---------------------------------------------------------------- dispatch */

int mxo_select_path(long B, long H, long S, long SK, int* splits) {
    /* dispatch.rs:494-511 */
    const long blocks256 = (S + 255) / 256 * H * B;
    const long ntiles = (SK + 127) / 128;
    long sp = 0;
    if (ntiles >= 16 && blocks256 <= 64) sp = 4;
    else if (ntiles >= 32 && blocks256 <= 128) sp = 2;
    if (sp > 0) {
        const long tps = (ntiles + sp - 1) / sp;
        if ((sp - 1) * tps < ntiles) { *splits = (int)sp; return 2; }
    }
    *splits = 0;
    return blocks256 <= 64 ? 1 : 0;
}

void mxo_split_range(int SK, int splits, int s, int* key_lo, int* kv_eff) {
    /* components.rs:58-74 */
    const int ntiles = (SK + 127) / 128;
    const int tps = (ntiles + splits - 1) / splits;
    const int tile_lo = s * tps;
    int tile_hi = tile_lo + tps;
    if (tile_hi > ntiles) tile_hi = ntiles;
    int key_hi = tile_hi * 128;
    if (key_hi > SK) key_hi = SK;
    *key_lo = tile_lo * 128;
    *kv_eff = key_hi - tile_lo * 128;
}

/* ----------------------------------------------------------------- threads */

typedef struct {
    const void* ctx;
    void (*fn)(const void* ctx, long item);
    long n;
    long next;
    pthread_mutex_t mu;
} pool_t;

static void* pool_worker(void* arg) {
    pool_t* p = (pool_t*)arg;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        const long it = p->next++;
        pthread_mutex_unlock(&p->mu);
        if (it >= p->n) break;
        p->fn(p->ctx, it);
    }
    return NULL;
}

static void run_parallel(int threads, long n, const void* ctx, void (*fn)(const void*, long)) {
    if (threads <= 0) threads = (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pool_t p = {ctx, fn, n, 0, PTHREAD_MUTEX_INITIALIZER};
    if (threads == 1 || n <= 1) { pool_worker(&p); return; }
    pthread_t tid[256];
    int started = 0;
    for (int i = 0; i < threads; ++i)
        if (pthread_create(&tid[i], NULL, pool_worker, &p) == 0) ++started;
    if (started == 0) pool_worker(&p);
    for (int i = 0; i < started; ++i) pthread_join(tid[i], NULL);
}

/* Keys visible to query row i: [0, lim) */
static int visible_keys(const mxo_problem* p, int i) {
    if (!p->causal) return p->SK;
    long lim = (long)i + p->SK - p->S + 1;
    if (lim < 0) lim = 0;
    if (lim > p->SK) lim = p->SK;
    return (int)lim;
}

/* ------------------------------------------------------------- fp64 check */

typedef struct {
    const mxo_problem* p;
    const uint16_t* o;
    int rows;
    const int* list; /* the checked rows: list[0 .. rows) (NULL: rows 0 .. rows - 1) */
    double* worst;   /* per (b,h) */
    double* sum_abs;
    double* max_ref;
    uint64_t* bad;
    uint64_t* cnt;
} check_ctx;

static void check_item(const void* vctx, long item) {
    const check_ctx* c = (const check_ctx*)vctx;
    const mxo_problem* p = c->p;
    const int b = (int)(item / p->H), h = (int)(item % p->H);
    const int gqa = p->H / p->HK, kvh = h / gqa;
    const double cpu_scale = score_mul(p);
    double* sc = (double*)malloc(sizeof(double) * (size_t)p->SK);
    double qd[D];
    double worst = 0, sum_abs = 0, max_ref = 0;
    uint64_t bad = 0, cnt = 0;
    for (int ii = 0; ii < c->rows && (c->list || ii < p->S); ++ii) {
        const int i = c->list ? c->list[ii] : ii;
        for (int kk = 0; kk < D; ++kk)
            qd[kk] = mxo_e4m3_decode(p->q[(((size_t)b * p->S + i) * p->H + h) * D + kk]) *
                     ldexp(1.0, (int)p->qs[(((size_t)b * p->S + i) * p->H + h) * 4 + kk / 32] - 127);
        const int nvis = visible_keys(p, i);
        double mx = -1e300;
        for (int t = 0; t < nvis; ++t) {
            double acc = 0.0;
            const uint8_t* kr = p->k + (((size_t)b * p->SK + t) * p->HK + kvh) * D;
            const uint8_t* ksr = p->ks + (((size_t)b * p->SK + t) * p->HK + kvh) * 4;
            for (int kk = 0; kk < D; ++kk) acc += qd[kk] * mxo_e4m3_decode(kr[kk]) * ldexp(1.0, (int)ksr[kk / 32] - 127);
            sc[t] = acc * cpu_scale;
            if (sc[t] > mx) mx = sc[t];
        }
        double den = 0.0;
        for (int t = 0; t < nvis; ++t) { sc[t] = exp(sc[t] - mx); den += sc[t]; }
        for (int d = 0; d < D; ++d) {
            double acc = 0.0;
            for (int t = 0; t < nvis; ++t)
                acc += sc[t] / den * mxo_e4m3_decode(p->v[(((size_t)b * p->SK + t) * p->HK + kvh) * D + d]) * v_block_scale(p, b, t, kvh, d);
            acc *= v_tensor_descale(p);
            const double got = mxo_bf16_to_f32(c->o[(((size_t)b * p->S + i) * p->H + h) * D + d]);
            const double err = fabs(got - acc);
            if (err != err) worst = INFINITY; else worst = fmax(worst, err);
            sum_abs += err;
            max_ref = fmax(max_ref, fabs(acc));
            ++cnt;
            if (!(err <= 0.05 + 0.05 * fabs(acc))) ++bad;
        }
    }
    free(sc);
    c->worst[item] = worst; c->sum_abs[item] = sum_abs; c->max_ref[item] = max_ref; c->bad[item] = bad; c->cnt[item] = cnt;
}

mxo_check_result mxo_check_fp64(const mxo_problem* p, const uint16_t* out_bf16, int rows, int threads) {
    return mxo_check_fp64_rows(p, out_bf16, NULL, rows, threads);
}

mxo_check_result mxo_check_fp64_rows(const mxo_problem* p, const uint16_t* out_bf16, const int* row_list, int rows, int threads) {
    const long n = (long)p->B * p->H;
    check_ctx c = {p, out_bf16, rows, row_list, calloc(n, 8), calloc(n, 8), calloc(n, 8), calloc(n, 8), calloc(n, 8)};
    run_parallel(threads, n, &c, check_item);
    mxo_check_result r = {0, 0, 0, 0, 0};
    double sum_abs = 0;
    for (long i = 0; i < n; ++i) {   /* the same accumulation as one sequential pass, in (b,h) order */
        r.checked += c.cnt[i];
        r.bad += c.bad[i];
        r.worst_err = (c.worst[i] != c.worst[i] || r.worst_err == INFINITY) ? INFINITY : fmax(r.worst_err, c.worst[i]);
        sum_abs += c.sum_abs[i];
        r.max_ref = fmax(r.max_ref, c.max_ref[i]);
    }
    r.mean_err = r.checked ? sum_abs / (double)r.checked : 0.0;
    free(c.worst); free(c.sum_abs); free(c.max_ref); free(c.bad); free(c.cnt);
    return r;
}

/* -------------------------------------------------------- fp32 attention */

typedef struct {
    const mxo_problem* p;
    const float* qf;   /* dequantised Q [B,S,H,128] (log2 units) */
    const float* kf;   /* dequantised K [B,SK,HK,128] */
    const float* vf;   /* dequantised V [B,SK,HK,128] (x vdescale) */
    float* out;
    int rows;
    int rows_per_item;
    long items_per_bh;
    float c;           /* base-2 score multiplier (1, or the in-kernel scale's c) */
} attn_ctx;

static void attn_item(const void* vctx, long item) {
    const attn_ctx* c = (const attn_ctx*)vctx;
    const mxo_problem* p = c->p;
    const long bh = item / c->items_per_bh, blk = item % c->items_per_bh;
    const int b = (int)(bh / p->H), h = (int)(bh % p->H);
    const int kvh = h / (p->H / p->HK);
    const int r0 = (int)blk * c->rows_per_item;
    int r1 = r0 + c->rows_per_item;
    if (r1 > c->rows) r1 = c->rows;
    float* sc = (float*)malloc(sizeof(float) * (size_t)p->SK);
    float acc[D];
    const size_t kstride = (size_t)p->HK * D;
    const float* kbase = c->kf + ((size_t)b * p->SK * p->HK + kvh) * D;
    const float* vbase = c->vf + ((size_t)b * p->SK * p->HK + kvh) * D;
    for (int i = r0; i < r1; ++i) {
        const float* qr = c->qf + (((size_t)b * p->S + i) * p->H + h) * D;
        const int nvis = visible_keys(p, i);
        float mx = -INFINITY;
        for (int t = 0; t < nvis; ++t) {
            const float* kr = kbase + (size_t)t * kstride;
            float s = 0.0f;
            for (int d = 0; d < D; ++d) s += qr[d] * kr[d];
            sc[t] = s * c->c;
            mx = s > mx ? s : mx;
        }
        float den = 0.0f;
        for (int t = 0; t < nvis; ++t) { sc[t] = exp2f(sc[t] - mx); den += sc[t]; }
        for (int d = 0; d < D; ++d) acc[d] = 0.0f;
        for (int t = 0; t < nvis; ++t) {
            const float w = sc[t];
            const float* vr = vbase + (size_t)t * kstride;
            for (int d = 0; d < D; ++d) acc[d] += w * vr[d];
        }
        const float inv = 1.0f / den;
        if (c->out) {
            float* orow = c->out + (((size_t)b * p->S + i) * p->H + h) * D;
            for (int d = 0; d < D; ++d) orow[d] = acc[d] * inv;
        }
    }
    free(sc);
}

double mxo_attention_fp32(const mxo_problem* p, int rows, float* out_f32, int threads) {
    if (rows <= 0 || rows > p->S) rows = p->S;
    const size_t nq = (size_t)p->B * p->S * p->H * D, nk = (size_t)p->B * p->SK * p->HK * D;
    float* qf = (float*)malloc(nq * 4);
    float* kf = (float*)malloc(nk * 4);
    float* vf = (float*)malloc(nk * 4);
    for (size_t i = 0; i < nq; ++i) qf[i] = (float)(mxo_e4m3_decode(p->q[i]) * ldexp(1.0, (int)p->qs[i / 32] - 127));
    for (size_t i = 0; i < nk; ++i) kf[i] = (float)(mxo_e4m3_decode(p->k[i]) * ldexp(1.0, (int)p->ks[i / 32] - 127));
    for (size_t i = 0; i < nk; ++i) {
        const int d = (int)(i % D), kvh = (int)(i / D % p->HK), key = (int)(i / D / p->HK % p->SK), b = (int)(i / D / p->HK / p->SK);
        vf[i] = (float)(mxo_e4m3_decode(p->v[i]) * v_block_scale(p, b, key, kvh, d)) * v_tensor_descale(p);
    }
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    attn_ctx c = {p, qf, kf, vf, out_f32, rows, 16, 0, qk_scaling_of(p).c};
    c.items_per_bh = (rows + c.rows_per_item - 1) / c.rows_per_item;
    run_parallel(threads, (long)p->B * p->H * c.items_per_bh, &c, attn_item);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    free(qf); free(kf); free(vf);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

/* -------------------------------------------------------------- emulator */

typedef struct {
    float thr, b131, conv;
    int lazy, lut;
} recipe_t;

static float f32_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static recipe_t recipe_for(int SK) {
    /* state.rs:75-77: fewer than 4 tiles of the WHOLE sequence keep the exact LUT copy (Recipe::vsx(true), softmax.rs:24-27);
     * otherwise the lazy copy of set_vendor_ref (softmax.rs:76-89) with decide_lazy. */
    recipe_t r;
    if ((SK + 127) / 128 < 4) { r.thr = 120.0f / 512.0f; r.b131 = 131.0f / 512.0f; r.conv = 1.0f; r.lazy = 0; r.lut = 1; }
    else { r.thr = f32_from_bits(0x3e85d086u); r.b131 = f32_from_bits(0x3e7df17eu); r.conv = 0.25f; r.lazy = 1; r.lut = 0; }
    return r;
}

/* LUT correction of the pknorm exponent rounding (reduce.rs:84-91, 94-110): u -= LUT[(u >> 4) & 7],
 * LUT = {0, 6, 9, 11, 11, 10, 7, 3}, 16-bit wrap (v_pk_sub_u16). */
static uint16_t lut_correct(uint16_t u) {
    static const uint16_t lut[8] = {0, 6, 9, 11, 11, 10, 7, 3};
    return (uint16_t)(u - lut[(u >> 4) & 7]);
}

typedef struct {
    uint32_t w;       /* two f16 words: hi = low half, lo = high half; reference b = 4 (hi + lo) */
    float l;          /* row sum of the quantised P (the smfmac accumulator) */
    float o[D];       /* unscaled P.V accumulator */
} row_state;

static float bias_value(uint32_t w) {
    const float hi = mxo_f16_to_f32((uint16_t)(w & 0xffff));
    const float lo = mxo_f16_to_f32((uint16_t)(w >> 16));
    return (hi + lo) * 4.0f;
}

/* One query row over keys [klo, khi) (tiles of 128 from klo; keys >= kvis are masked, the
 * key range of this call ends at khi). qd: dequantised-by-MFMA operand (e4m3 values), sq: the
 * two-byte-selected Q scale exponents (qs - 9), per 32-block. Only keys [jlo, jhi) of every tile take part
 * (0, 128 for the reference's order; a 64-key half for one stream of the library's split-tile order, below). */
static void emulate_row(const mxo_problem* p, const recipe_t* rc, int b, int kvh, const double* qv, const int* sq,
                        int klo, int khi, int kvis, int jlo, int jhi, row_state* st) {
    pthread_once(&g_once, init_tables);
    st->w = 0x48004800u;
    st->l = 0.0f;
    for (int d = 0; d < D; ++d) st->o[d] = 0.0f;
    float s[128];
    uint8_t pb[128];
    const qk_scaling qc = qk_scaling_of(p);
    for (int t0 = klo; t0 < khi; t0 += 128) {
        const float bb = bias_value(st->w) * qc.rm;   /* the seed (b / m; b when unscaled) */
        /* S' = b + S * 2^-9: the scaled QK MFMA of d 0..63 then d 64..127 accumulating onto the reference */
        double qsd[D];
        for (int d = 0; d < D; ++d) qsd[d] = qv[d] * ldexp(1.0, (sq[d / 32] & 0xff) - 127);
        for (int j = 0; j < 128; ++j) {
            int key = t0 + j;
            const int kr = key < p->SK ? key : p->SK - 1;
            const uint8_t* krow = p->k + (((size_t)b * p->SK + kr) * p->HK + kvh) * D;
            const uint8_t* ksr = p->ks + (((size_t)b * p->SK + kr) * p->HK + kvh) * 4;
            float acc = bb;
            for (int c = 0; c < 2; ++c) {
                double dot = 0.0;
                for (int blk = 2 * c; blk < 2 * c + 2; ++blk) {
                    double part = 0.0;   /* exact: 32 products of 4-bit mantissas */
                    for (int d = 32 * blk; d < 32 * blk + 32; ++d) part += qsd[d] * g_e4m3_val[krow[d]];
                    dot += part * ldexp(1.0, (int)ksr[blk] - 127);
                }
                acc = (float)((double)acc + dot);
            }
            s[j] = acc * qc.m;
        }
        const int vlim = khi < kvis ? khi : kvis;
        /* row max over the valid keys (reduce.rs:52-64; masked keys -1e30, reduce.rs:13-49) */
        float m = -1.0e30f;
        for (int j = 0; j < 128; ++j) {
            const float x = (t0 + j < vlim && j >= jlo && j < jhi) ? s[j] : -1.0e30f;
            m = fmaxf(m, x);
        }
        const int grow = rc->lazy ? !(rc->thr >= m) : (rc->thr < m);
        if (grow) {
            /* softmax.rs:125-160 / 200-241 */
            const uint32_t w_old = st->w;
            const float hi_o = mxo_f16_to_f32((uint16_t)(w_old & 0xffff));
            const float lo_o = mxo_f16_to_f32((uint16_t)(w_old >> 16));
            const float b_old = (hi_o + lo_o) * 4.0f;
            const float tt = rc->b131 - m;
            const float b_new = b_old + tt;
            const float qq = b_new * 0.25f;
            const uint16_t h_raw = mxo_f32_to_f16(qq);
            const float hq = mxo_f16_to_f32(h_raw);
            const float r = qq - hq;
            const uint16_t l_raw = mxo_f32_to_f16(r);
            const float lq = mxo_f16_to_f32(l_raw);
            const float b_q = (hq + lq) * 4.0f;
            const float delta = b_q - b_old;
            st->w = (uint32_t)h_raw + ((uint32_t)l_raw << 16);
            for (int j = 0; j < 128; ++j) s[j] += delta;
            const float corr = exp2f(delta * 512.0f);
            for (int d = 0; d < D; ++d) st->o[d] *= corr;
            st->l *= corr;
        }
        /* P = fp8(pknorm(S') [- LUT]) / conv  (reduce.rs:94-113); masked keys 0 */
        double psum = 0.0;
        for (int j = 0; j < 128; ++j) {
            const float x = (t0 + j < vlim) ? s[j] : 0.0f;
            uint16_t u = mxo_pknorm_u16(x);
            if (rc->lut) u = lut_correct(u);
            pb[j] = (j >= jlo && j < jhi) ? mxo_cvt_bf16_fp8(u, rc->conv) : 0;
            psum += g_e4m3_val[pb[j]];
        }
        st->l = (float)((double)st->l + psum);
        /* O += P.V over two 64-key halves (unscaled fp8 MFMA) */
        for (int half = 0; half < 2; ++half)
            for (int d = 0; d < D; ++d) {
                double a = 0.0;
                for (int jj = 0; jj < 64; ++jj) {
                    const int j = 64 * half + jj;
                    if (!pb[j]) continue;
                    const int key = t0 + j;
                    const int kr = key < p->SK ? key : p->SK - 1;
                    a += g_e4m3_val[pb[j]] * g_e4m3_val[p->v[(((size_t)b * p->SK + kr) * p->HK + kvh) * D + d]] *
                         v_block_scale(p, b, kr, kvh, d);
                }
                st->o[d] = (float)((double)st->o[d] + a);
            }
    }
}

/* The library's split-tile order (extension, no reference counterpart): a KV-split block with at most 128 query rows
 * (S - 256 floor(i / 256) <= 128), and every row of the full-sequence split-tile kernel (the t128 path), with the
 * non-LUT recipe, run two streams per row, keys 0..63 and 64..127 of every tile, and merge them: with b the stream's bias (O and l carry 2^(512 b)), the smaller b is kept and the other
 * stream scaled by 2^(512 (b_min - b)), O = fma(O_b, s_b, O_a s_a) in the order of the kernel's merge. */
static int split_tile_order(const mxo_problem* p, const recipe_t* rc, int i) {
    return !rc->lut && p->S - 256 * (i / 256) <= 128;
}
static void merge_streams(row_state* a, const row_state* bst) {
    const float ba = bias_value(a->w), bb = bias_value(bst->w);
    const int keep_a = ba <= bb;
    const float sc = exp2f(512.0f * (keep_a ? ba - bb : bb - ba));
    const float sa = keep_a ? 1.0f : sc, sb = keep_a ? sc : 1.0f;
    for (int d = 0; d < D; ++d) a->o[d] = fmaf(bst->o[d], sb, a->o[d] * sa);
    a->l = fmaf(bst->l, sb, a->l * sa);
    if (!keep_a) a->w = bst->w;
}

typedef struct {
    const mxo_problem* p;
    int splits, rows;
    uint16_t* out;
    void* ohat;          /* fp16 rows, or f32 rows when f32_partials */
    float* lse;
    int f32_partials;
    int split_tiles;     /* 1: the library's split-tile order where it applies (KV split only) */
    const int* list;     /* the emulated rows: list[0 .. rows) (NULL: rows 0 .. rows - 1) */
} emu_ctx;

static void emu_item(const void* vctx, long item) {
    const emu_ctx* c = (const emu_ctx*)vctx;
    const mxo_problem* p = c->p;
    const int rows = c->rows;
    const long bh = item / rows;
    const int i = c->list ? c->list[item % rows] : (int)(item % rows);
    const int b = (int)(bh / p->H), h = (int)(bh % p->H);
    const int kvh = h / (p->H / p->HK);
    const recipe_t rc = recipe_for(p->SK);
    double qv[D];
    int sq[4];
    for (int d = 0; d < D; ++d) qv[d] = mxo_e4m3_decode(p->q[(((size_t)b * p->S + i) * p->H + h) * D + d]);
    const int qe = qk_scaling_of(p).e;
    for (int blk = 0; blk < 4; ++blk) sq[blk] = ((int)p->qs[(((size_t)b * p->S + i) * p->H + h) * 4 + blk] - 9 + qe) & 0xff;
    const int kvis = visible_keys(p, i);
    const float vd = v_tensor_descale(p);
    row_state st;
    uint16_t* orow = c->out + (((size_t)b * p->S + i) * p->H + h) * D;
    if (c->splits <= 0) {
        if (c->split_tiles && !rc.lut) {
            /* the full-sequence split-tile kernel (t128's shapes): every row in the two-stream order */
            row_state st_b;
            emulate_row(p, &rc, b, kvh, qv, sq, 0, p->SK, kvis, 0, 64, &st);
            emulate_row(p, &rc, b, kvh, qv, sq, 0, p->SK, kvis, 64, 128, &st_b);
            merge_streams(&st, &st_b);
        } else {
            emulate_row(p, &rc, b, kvh, qv, sq, 0, p->SK, kvis, 0, 128, &st);
        }
        /* state.rs:79-83 (v_rcp_f32, then x v_descale); a row with no visible key (causal extension, S > SK) is 0 */
        const float fin = st.l > 0.0f ? (1.0f / st.l) * vd : 0.0f;
        for (int d = 0; d < D; ++d) orow[d] = mxo_f32_to_bf16(st.o[d] * fin);
        return;
    }
    const long rows_total = (long)p->B * p->S * p->H;
    const long prow = ((long)b * p->S + i) * p->H + h;
    float lse_s[MXO_MAX_SPLITS];
    float oh[MXO_MAX_SPLITS][D];      /* the partial row as stored (fp16-rounded unless f32_partials) */
    for (int s = 0; s < c->splits; ++s) {
        int key_lo, kv_eff;
        mxo_split_range(p->SK, c->splits, s, &key_lo, &kv_eff);
        if (c->split_tiles && split_tile_order(p, &rc, i)) {
            row_state st_b;
            emulate_row(p, &rc, b, kvh, qv, sq, key_lo, key_lo + kv_eff, kvis, 0, 64, &st);
            emulate_row(p, &rc, b, kvh, qv, sq, key_lo, key_lo + kv_eff, kvis, 64, 128, &st_b);
            merge_streams(&st, &st_b);
        } else {
            emulate_row(p, &rc, b, kvh, qv, sq, key_lo, key_lo + kv_eff, kvis, 0, 128, &st);
        }
        /* block3.rs:291-356 (Ohat = O * v_descale / l, fp16) and softmax.rs:308-322 (lse = log2(l_total) - 2048 (hi + lo)),
         * with l_total = l / 16 (softmax.rs:277-305): the scaled PV form accumulates O / 16 */
        const float l_total = st.l * 0.0625f;
        const float fin = st.l > 0.0f ? (1.0f / l_total) * vd : 0.0f;
        for (int d = 0; d < D; ++d) {
            const float x = (st.o[d] * 0.0625f) * fin;
            /* extension: f32 partial rows keep x; the reference's fp16 rows round it (block3.rs:334-336) */
            oh[s][d] = c->f32_partials ? x : mxo_f16_to_f32(mxo_f32_to_f16(x));
        }
        const float hl = mxo_f16_to_f32((uint16_t)(st.w & 0xffff)) + mxo_f16_to_f32((uint16_t)(st.w >> 16));
        /* a split without keys gets lse -1e30: weight 0 in the combine */
        lse_s[s] = st.l > 0.0f ? log2f(l_total) + (hl * 2048.0f) * -1.0f : -1.0e30f;
        if (c->ohat) {
            if (c->f32_partials) {
                memcpy((float*)c->ohat + ((size_t)s * rows_total + prow) * D, oh[s], 4 * D);
            } else {
                uint16_t* dst = (uint16_t*)c->ohat + ((size_t)s * rows_total + prow) * D;
                for (int d = 0; d < D; ++d) dst[d] = mxo_f32_to_f16(oh[s][d]);
            }
        }
        if (c->lse) c->lse[(size_t)s * rows_total + prow] = lse_s[s];
    }
    /* combine (epilogue.rs:89-167) */
    float m = -1.0e30f, den = 0.0f, acc[D];
    for (int d = 0; d < D; ++d) acc[d] = 0.0f;
    for (int s = 0; s < c->splits; ++s) {
        const float l = lse_s[s];
        const float m_new = fmaxf(m, l);
        const float dm = m_new * -1.0f;
        const float a = exp2f(m + dm), w = exp2f(l + dm);
        den = den * a + w;
        for (int d = 0; d < D; ++d) acc[d] = acc[d] * a + w * oh[s][d];
        m = m_new;
    }
    const float rd = 1.0f / den;
    for (int d = 0; d < D; ++d) orow[d] = mxo_f32_to_bf16(acc[d] * rd);
}

void mxo_emulate_ex(const mxo_problem* p, int splits, int rows, uint16_t* out_bf16, void* ohat, float* lse_f32,
                    int f32_partials, int split_tiles, int threads) {
    if (splits > MXO_MAX_SPLITS) return;   /* refused (the Python wrapper checks first) */
    if (rows <= 0 || rows > p->S) rows = p->S;
    emu_ctx c = {p, splits, rows, out_bf16, ohat, lse_f32, f32_partials, split_tiles, NULL};
    run_parallel(threads, (long)p->B * p->H * rows, &c, emu_item);
}

void mxo_emulate_rows(const mxo_problem* p, int splits, const int* row_list, int rows, uint16_t* out_bf16, int f32_partials,
                      int split_tiles, int threads) {
    if (splits > MXO_MAX_SPLITS) return;   /* refused (the Python wrapper checks first) */
    emu_ctx c = {p, splits, rows, out_bf16, NULL, NULL, f32_partials, split_tiles, row_list};
    run_parallel(threads, (long)p->B * p->H * rows, &c, emu_item);
}

void mxo_emulate(const mxo_problem* p, int splits, int rows, uint16_t* out_bf16,
                 uint16_t* ohat_f16, float* lse_f32, int threads) {
    mxo_emulate_ex(p, splits, rows, out_bf16, ohat_f16, lse_f32, 0, 0, threads);
}

/* The combine on f32 partial rows (the FMHA_KVS_F32_PARTIALS extension): the same arithmetic, no fp16 decode. */
void mxo_combine_f32(const float* ohat_f32, const float* lse, uint16_t* out_bf16, long rows_total, int splits) {
    for (long r = 0; r < rows_total; ++r) {
        float m = -1.0e30f, den = 0.0f, acc[D];
        for (int d = 0; d < D; ++d) acc[d] = 0.0f;
        for (int s = 0; s < splits; ++s) {
            const float l = lse[(size_t)s * rows_total + r];
            const float m_new = fmaxf(m, l);
            const float dm = m_new * -1.0f;
            const float a = exp2f(m + dm), w = exp2f(l + dm);
            den = den * a + w;
            const float* o = ohat_f32 + ((size_t)s * rows_total + r) * D;
            for (int d = 0; d < D; ++d) acc[d] = acc[d] * a + w * o[d];
            m = m_new;
        }
        const float rd = 1.0f / den;
        for (int d = 0; d < D; ++d) out_bf16[(size_t)r * D + d] = mxo_f32_to_bf16(acc[d] * rd);
    }
}

void mxo_combine(const uint16_t* ohat_f16, const float* lse, uint16_t* out_bf16, long rows_total, int splits) {
    for (long r = 0; r < rows_total; ++r) {
        float m = -1.0e30f, den = 0.0f, acc[D];
        for (int d = 0; d < D; ++d) acc[d] = 0.0f;
        for (int s = 0; s < splits; ++s) {
            const float l = lse[(size_t)s * rows_total + r];
            const float m_new = fmaxf(m, l);
            const float dm = m_new * -1.0f;
            const float a = exp2f(m + dm), w = exp2f(l + dm);
            den = den * a + w;
            const uint16_t* o = ohat_f16 + ((size_t)s * rows_total + r) * D;
            for (int d = 0; d < D; ++d) acc[d] = acc[d] * a + w * mxo_f16_to_f32(o[d]);
            m = m_new;
        }
        const float rd = 1.0f / den;
        for (int d = 0; d < D; ++d) out_bf16[(size_t)r * D + d] = mxo_f32_to_bf16(acc[d] * rd);
    }
}

/* ---- quantisers of bf16 inputs (the generator's rule, ref_host.cpp:239-251, applied to given values) ---- */

static int e8m0_rule(double amax) {
    /* ref_host.cpp:243-244. +-Inf maxima are outside the generator's domain (its int cast of floor(log2(inf)) is
     * undefined); the library defines them as exponent field 255 - 8 = 247, and so does this restatement. */
    if (isinf(amax)) return 247;
    const int e = amax > 0 ? (int)floor(log2(amax)) - 8 : -127;
    int eb = e + 127;
    if (eb < 0) eb = 0;
    if (eb > 254) eb = 254;
    return eb;
}

static double running_max(double amax, double a) { return amax < a ? a : amax; }   /* std::max(amax, a) */

void mxo_quant_rows_bf16(const uint16_t* x, long rows, float mul, uint8_t* q, uint8_t* sc) {
    for (long r = 0; r < rows; ++r)
        for (int bk = 0; bk < 4; ++bk) {
            float y[32];
            double amax = 0;
            for (int i = 0; i < 32; ++i) {
                y[i] = mxo_bf16_to_f32(x[(size_t)r * D + 32 * bk + i]) * mul;
                amax = running_max(amax, fabs((double)y[i]));
            }
            const int eb = e8m0_rule(amax);
            sc[(size_t)r * 4 + bk] = (uint8_t)eb;
            const double inv = ldexp(1.0, -(eb - 127));
            for (int i = 0; i < 32; ++i) q[(size_t)r * D + 32 * bk + i] = mxo_e4m3_encode_sat((float)(y[i] * inv));
        }
}

float mxo_quant_tensor_bf16(const uint16_t* x, long n, uint8_t* q) {
    /* ref_host.cpp:248-251: vdescale = (float)(vmax / 448), v = e4m3((float)(x / vdescale)) */
    double vmax = 0;
    for (long i = 0; i < n; ++i) vmax = running_max(vmax, fabs((double)mxo_bf16_to_f32(x[i])));
    const float d = (float)(vmax / 448.0);
    for (long i = 0; i < n; ++i) q[i] = mxo_e4m3_encode_sat((float)((double)mxo_bf16_to_f32(x[i]) / d));
    return d;
}

void mxo_quant_seq32_bf16(const uint16_t* x, int B, int SK, int HK, uint8_t* q, uint8_t* sc) {
    const int nblk = (SK + 31) / 32;
    for (int b = 0; b < B; ++b)
        for (int blk = 0; blk < nblk; ++blk)
            for (int h = 0; h < HK; ++h)
                for (int d = 0; d < D; ++d) {
                    const int k0 = 32 * blk, nk = SK - k0 < 32 ? SK - k0 : 32;
                    double amax = 0;
                    for (int k = 0; k < nk; ++k)
                        amax = running_max(amax, fabs((double)mxo_bf16_to_f32(x[(((size_t)b * SK + k0 + k) * HK + h) * D + d])));
                    const int eb = e8m0_rule(amax);
                    sc[(((size_t)b * nblk + blk) * HK + h) * D + d] = (uint8_t)eb;
                    const double inv = ldexp(1.0, -(eb - 127));
                    for (int k = 0; k < nk; ++k) {
                        const size_t i = (((size_t)b * SK + k0 + k) * HK + h) * D + d;
                        q[i] = mxo_e4m3_encode_sat((float)(mxo_bf16_to_f32(x[i]) * inv));
                    }
                }
}
