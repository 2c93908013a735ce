/*  p2_blas.c – the reference's GEMM API (csrc/blas.h) over the MI355X kernels (include/p2_blas.h).
 *
 *  Host code in C: operand staging, the device weight cache, the mode latch and the reference's argument
 *  conventions. Every product is computed by libp2hip.so on the GPU; this file does no arithmetic on operands.
 */
#include "p2_blas.h"
#include "p2hip.h"

#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ── failure ───────────────────────────────────────────────────────────────────────────────────────────────── */

static void die(const char *who, const char *what)
{
    fprintf(stderr, "%s: %s\n", who, what);
    abort();
}

static void check(int rc, const char *who)
{
    if (rc != 0) die(who, p2h_last_error());
}

/* blas.c:989-995 */
static void require_panel_aligned(int N, const char *who)
{
    if (N % 16 != 0) {
        fprintf(stderr, "%s: N = %d is not a multiple of %d\n", who, N, 16);
        abort();
    }
}

/* ── the mode latch (blas.c:1027-1066) ─────────────────────────────────────────────────────────────────────── */

static int gemm_mode = -1;
static pthread_once_t gemm_mode_once = PTHREAD_ONCE_INIT;

/* P2_GEMM = int8 | int8w | exact, P2_EXACT non-"0" forces exact. The GPU always has int8 dot products, so the
 * reference's "no dot-product extension → exact" clause (blas.c:1043-1045) never applies. */
static void gemm_mode_init(void)
{
    const char *e = getenv("P2_EXACT");
    const char *g = getenv("P2_GEMM");
    int mode = P2H_INT8W;
    if (g && strcmp(g, "exact") == 0) mode = P2H_EXACT;
    else if (g && strcmp(g, "int8") == 0) mode = P2H_INT8;
    else if (g && strcmp(g, "int8w") == 0) mode = P2H_INT8W;
    if (e && e[0] && e[0] != '0') mode = P2H_EXACT;
    gemm_mode = mode;
}

static int current_mode(void)
{
    pthread_once(&gemm_mode_once, gemm_mode_init);
    return gemm_mode;
}

int p2_gemm_exact(void) { return current_mode() == P2H_EXACT; }

const char *p2_gemm_mode(void)
{
    switch (current_mode()) {
    case P2H_INT8:  return "int8 dot products, exact weights";
    case P2H_INT8W: return "int8 dot products, int8 weights";
    default:        return "fp32 expansion (exact)";
    }
}

/* ── call accounting (p2_gpu_stats_take) ───────────────────────────────────────────────────────────────────── */

/* Nanoseconds inside each family of entries (summed over calling threads), the part of them spent uploading
 * weights on first touch, and the operand bytes moved each way over PCIe. */
enum { ST_FVB_CALLS, ST_FVB_NS, ST_Q8B_CALLS, ST_Q8B_NS, ST_SG_CALLS, ST_SG_NS, ST_UPLOAD_NS, ST_H2D, ST_D2H, ST_N };
static _Atomic long long stats[ST_N];

static long long now_ns(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (long long)ts.tv_sec * 1000000000ll + ts.tv_nsec;
}

static void stat_add(int k, long long v) { atomic_fetch_add_explicit(&stats[k], v, memory_order_relaxed); }

static void stat_call(int calls, int ns, long long t0)
{
    stat_add(calls, 1);
    stat_add(ns, now_ns() - t0);
}

void p2_gpu_stats_take(double out[P2_GPU_STATS_N])
{
    long long v[ST_N];
    for (int k = 0; k < ST_N; k++) v[k] = atomic_exchange_explicit(&stats[k], 0, memory_order_relaxed);
    out[0] = (double)v[ST_FVB_CALLS]; out[1] = v[ST_FVB_NS] * 1e-6;
    out[2] = (double)v[ST_Q8B_CALLS]; out[3] = v[ST_Q8B_NS] * 1e-6;
    out[4] = (double)v[ST_SG_CALLS];  out[5] = v[ST_SG_NS] * 1e-6;
    out[6] = v[ST_UPLOAD_NS] * 1e-6;
    out[7] = v[ST_H2D] * 1e-6;        out[8] = v[ST_D2H] * 1e-6;
}

/* ── device start-up ───────────────────────────────────────────────────────────────────────────────────────── */

static pthread_once_t dev_once = PTHREAD_ONCE_INIT;

static void dev_init(void) { check(p2h_init(), "phonon2 GPU GEMM"); }

/* ── per-thread staging ────────────────────────────────────────────────────────────────────────────────────── */

typedef struct {
    void *stream;
    void *dA;  size_t capA;     /* activations (fp32) */
    void *dB;  size_t capB;     /* fp32 B of p2_sgemm */
    void *dC;  size_t capC;     /* output */
    void *dW;  size_t capW;     /* quantisation workspace */
    float *hq; size_t capq;     /* pinned host rows of the QuantA handed out by p2_quant_prepare */
    float *hs; size_t caps;     /* its scales array (never read: the GPU quantises) */
    void *hp;  size_t capp;     /* pinned host rows: strided operands packed or unpacked on the way */
} Ctx;

static pthread_key_t ctx_key;
static pthread_once_t ctx_once = PTHREAD_ONCE_INIT;

static void ctx_free(void *p)
{
    Ctx *c = (Ctx *)p;
    if (!c) return;
    p2h_free(c->dA); p2h_free(c->dB); p2h_free(c->dC); p2h_free(c->dW);
    p2h_host_free(c->hq);
    p2h_host_free(c->hp);
    free(c->hs);
    p2h_stream_destroy(c->stream);
    free(c);
}

static void ctx_key_init(void) { pthread_key_create(&ctx_key, ctx_free); }

static Ctx *ctx(void)
{
    pthread_once(&dev_once, dev_init);
    pthread_once(&ctx_once, ctx_key_init);
    Ctx *c = (Ctx *)pthread_getspecific(ctx_key);
    if (!c) {
        c = (Ctx *)calloc(1, sizeof *c);
        if (!c) die("phonon2 GPU GEMM", "out of memory");
        c->stream = p2h_stream_create();
        if (!c->stream) die("phonon2 GPU GEMM", p2h_last_error());
        pthread_setspecific(ctx_key, c);
    }
    return c;
}

static void *dgrow(void **p, size_t *cap, size_t need, const char *who)
{
    if (need > *cap || !*p) {
        p2h_free(*p);
        size_t n = need < 4096 ? 4096 : need + need / 4;
        *p = p2h_malloc(n);
        if (!*p) die(who, p2h_last_error());
        *cap = n;
    }
    return *p;
}

static void *hgrow(Ctx *c, size_t need, const char *who)
{
    if (need > c->capp || !c->hp) {
        p2h_host_free(c->hp);
        size_t n = need < 4096 ? 4096 : need + need / 4;
        c->hp = p2h_host_malloc(n);
        if (!c->hp) die(who, p2h_last_error());
        c->capp = n;
    }
    return c->hp;
}

/* rows of `width` bytes at host pitch `pitch` to a packed device buffer: one linear copy when the rows are packed,
 * else packed into pinned host memory first (a 2-D copy from the host goes row by row, milliseconds for a few
 * hundred rows) */
static void h2d_rows(Ctx *c, void *d, const void *h, size_t width, size_t pitch, size_t rows, const char *who)
{
    stat_add(ST_H2D, (long long)(rows * width));
    if (pitch == width) {
        check(p2h_memcpy_h2d(d, h, rows * width, c->stream), who);
        return;
    }
    check(p2h_stream_sync(c->stream), who);   /* a copy from the pinned rows may still be in flight */
    char *hp = (char *)hgrow(c, rows * width, who);
    for (size_t r = 0; r < rows; r++) memcpy(hp + r * width, (const char *)h + r * pitch, width);
    check(p2h_memcpy_h2d(d, hp, rows * width, c->stream), who);
}

/* ── the device weight cache ───────────────────────────────────────────────────────────────────────────────── */

/* One device copy per host weight, keyed on its plane pointers, shape and a content fingerprint. A call holds a
 * reference for as long as its kernels may read the copy: an entry that is dropped (p2_gpu_weight_cache_clear, or new
 * contents at the same address) while a call holds it is only unlinked, and the last holder frees it. */
typedef struct Entry {
    const void *a, *b, *c, *d;   /* signs, flags, lo, hi  /  q8, scales */
    int K, N, ld, kind;
    uint64_t fp;
    P2hWeight *w;                /* five-value */
    void *dq8; float *dsc;       /* int8 table: [K][N] int8, [N] scales */
    int refs;                    /* calls using the copy now */
    int dead;                    /* unlinked from the cache: freed when refs drops to 0 */
    int ready;                   /* the device copy is complete (0 while its first caller uploads it) */
    struct Entry *next;
    struct Entry *free_next;     /* on a list of entries to free once cache_mu is released */
} Entry;

#define CACHE_BUCKETS 1024
static Entry *cache[CACHE_BUCKETS];
/* cache_mu guards the table and the entries' refs / dead / ready; uploads and frees run outside it, so one thread's
 * first-touch upload or a cache clear does not stall other threads' calls on weights already on the device. A
 * caller that finds an entry still being uploaded waits on cache_cv for it. */
static pthread_mutex_t cache_mu = PTHREAD_MUTEX_INITIALIZER;
static pthread_cond_t cache_cv = PTHREAD_COND_INITIALIZER;

/* P2_GPU_WEIGHT_CACHE=0: every call uploads its weight and frees the copy afterwards (for callers that change
 * weights in place, which the fingerprint does not fully cover) */
static int cache_on = 1;
static pthread_once_t cache_env_once = PTHREAD_ONCE_INIT;
static void cache_env_init(void)
{
    const char *v = getenv("P2_GPU_WEIGHT_CACHE");
    cache_on = !(v && v[0] == '0' && v[1] == 0);
}

static uint64_t fnv(uint64_t h, const void *p, size_t n)
{
    const unsigned char *s = (const unsigned char *)p;
    for (size_t i = 0; i < n; i++) { h ^= s[i]; h *= 0x100000001B3ull; }
    return h;
}

/* lo/hi (or scales) in full, and the first and last 64 bytes of each plane */
static uint64_t fingerprint(const void *p1, size_t n1, const void *p2, size_t n2, const void *v1, const void *v2,
                            size_t nv)
{
    uint64_t h = 0xCBF29CE484222325ull;
    size_t e1 = n1 < 64 ? n1 : 64, e2 = n2 < 64 ? n2 : 64;
    h = fnv(h, p1, e1); h = fnv(h, (const char *)p1 + n1 - e1, e1);
    if (p2) { h = fnv(h, p2, e2); h = fnv(h, (const char *)p2 + n2 - e2, e2); }
    h = fnv(h, v1, nv);
    if (v2) h = fnv(h, v2, nv);
    return h;
}

static size_t bucket(const void *a, int K, int N)
{
    uint64_t x = (uint64_t)(uintptr_t)a ^ ((uint64_t)K << 32) ^ (uint64_t)N;
    x ^= x >> 29; x *= 0xBF58476D1CE4E5B9ull; x ^= x >> 32;
    return (size_t)(x % CACHE_BUCKETS);
}

static void entry_free(Entry *e)
{
    p2h_weight_free(e->w);
    p2h_free(e->dq8);
    p2h_free(e->dsc);
    free(e);
}

/* frees a list made under cache_mu, after it is released (hipFree synchronises the device) */
static void free_list(Entry *list)
{
    while (list) {
        Entry *n = list->free_next;
        entry_free(list);
        list = n;
    }
}

/* cache_mu held: take e out of the cache; put it on *to_free if no call holds it, else its last holder frees it */
static void entry_drop_locked(Entry *e, Entry **to_free)
{
    e->dead = 1;
    if (e->refs == 0) {
        e->free_next = *to_free;
        *to_free = e;
    }
}

/* a call is done with e (its kernels have finished) */
static void entry_put(Entry *e)
{
    pthread_mutex_lock(&cache_mu);
    const int last = --e->refs == 0 && e->dead;
    pthread_mutex_unlock(&cache_mu);
    if (last) entry_free(e);
}

/* cache_mu held: e was found in the cache; wait until its first caller has finished uploading it */
static void entry_wait_ready_locked(Entry *e)
{
    while (!e->ready) pthread_cond_wait(&cache_cv, &cache_mu);
}

/* the uploader's device copy is complete: wake the callers waiting for it */
static void entry_publish(Entry *e)
{
    pthread_mutex_lock(&cache_mu);
    e->ready = 1;
    pthread_cond_broadcast(&cache_cv);
    pthread_mutex_unlock(&cache_mu);
}

/* cache_mu held: the live entry for this key with this fingerprint, taken (refs + 1); a stale entry at the same key
 * is dropped (onto *to_free when nothing holds it); NULL when there is none */
static Entry *entry_find_locked(size_t h, int kind, const void *a, const void *b, const void *c, const void *d, int K,
                                int N, int ld, uint64_t fp, Entry **to_free)
{
    for (Entry **pe = &cache[h]; *pe; pe = &(*pe)->next) {
        Entry *e = *pe;
        if (e->kind == kind && e->a == a && e->b == b && e->c == c && e->d == d && e->K == K && e->N == N &&
            e->ld == ld) {
            if (e->fp == fp) {
                e->refs++;
                return e;
            }
            *pe = e->next;   /* same addresses, new contents: drop the stale copy */
            entry_drop_locked(e, to_free);
            return NULL;
        }
    }
    return NULL;
}

/* cache_mu held: a new entry holding one reference, in the cache unless caching is off */
static Entry *entry_new_locked(size_t h, int kind, const void *a, const void *b, const void *c, const void *d, int K,
                               int N, int ld, uint64_t fp, const char *who)
{
    Entry *e = (Entry *)calloc(1, sizeof *e);
    if (!e) die(who, "out of memory");
    e->a = a; e->b = b; e->c = c; e->d = d;
    e->K = K; e->N = N; e->ld = ld; e->kind = kind; e->fp = fp;
    e->refs = 1;
    if (cache_on) {
        e->next = cache[h];
        cache[h] = e;
    } else {
        e->dead = 1;
    }
    return e;
}

/* The cache entry of a five-value weight, taken (refs + 1): found, waiting for its upload if another thread is
 * making it, or made here: a placeholder goes into the cache under cache_mu, the upload runs outside it. */
static Entry *fv_weight(const FiveValueB *B, int K, int N)
{
    pthread_once(&cache_env_once, cache_env_init);
    size_t kn = (size_t)K * N;
    uint64_t fp = fingerprint(B->signs, kn / 4 ? kn / 4 : 1, B->flags, kn / 8 ? kn / 8 : 1, B->lo, B->hi,
                              (size_t)N * sizeof(float));
    size_t h = bucket(B->signs, K, N);
    Entry *to_free = NULL;
    pthread_mutex_lock(&cache_mu);
    Entry *e = cache_on ? entry_find_locked(h, 0, B->signs, B->flags, B->lo, B->hi, K, N, 0, fp, &to_free) : NULL;
    if (e) {
        entry_wait_ready_locked(e);
        pthread_mutex_unlock(&cache_mu);
        free_list(to_free);
        return e;
    }
    e = entry_new_locked(h, 0, B->signs, B->flags, B->lo, B->hi, K, N, 0, fp, "p2_sgemm_fvb");
    pthread_mutex_unlock(&cache_mu);
    free_list(to_free);
    const long long t0 = now_ns();
    e->w = p2h_fv_weight_upload(B->signs, B->flags, B->lo, B->hi, K, N);
    if (!e->w) die("p2_sgemm_fvb: weight upload", p2h_last_error());
    stat_add(ST_UPLOAD_NS, now_ns() - t0);
    entry_publish(e);
    return e;
}

static Entry *q8_weight(const signed char *B, const float *scales, int ldb, int K, int N, void *stream)
{
    pthread_once(&cache_env_once, cache_env_init);
    size_t rows_bytes = K > 0 ? (size_t)(K - 1) * ldb + N : 1;
    uint64_t fp = fingerprint(B, rows_bytes, NULL, 0, scales, NULL, (size_t)N * sizeof(float));
    size_t h = bucket(B, K, N);
    Entry *to_free = NULL;
    pthread_mutex_lock(&cache_mu);
    Entry *e = cache_on ? entry_find_locked(h, 1, B, NULL, scales, NULL, K, N, ldb, fp, &to_free) : NULL;
    if (e) {
        entry_wait_ready_locked(e);
        pthread_mutex_unlock(&cache_mu);
        free_list(to_free);
        return e;
    }
    e = entry_new_locked(h, 1, B, NULL, scales, NULL, K, N, ldb, fp, "p2_sgemm_q8b");
    pthread_mutex_unlock(&cache_mu);
    free_list(to_free);
    const long long t0 = now_ns();
    e->dq8 = p2h_malloc((size_t)K * N + 16);
    e->dsc = (float *)p2h_malloc((size_t)N * sizeof(float));
    if (!e->dq8 || !e->dsc) die("p2_sgemm_q8b: weight upload", p2h_last_error());
    check(p2h_memcpy2d_h2d(e->dq8, (size_t)N, B, (size_t)ldb, (size_t)N, (size_t)K, stream), "p2_sgemm_q8b");
    check(p2h_memcpy_h2d(e->dsc, scales, (size_t)N * sizeof(float), stream), "p2_sgemm_q8b");
    check(p2h_stream_sync(stream), "p2_sgemm_q8b");
    stat_add(ST_UPLOAD_NS, now_ns() - t0);
    entry_publish(e);
    return e;
}

void p2_gpu_weight_cache_clear(void)
{
    Entry *to_free = NULL;
    pthread_mutex_lock(&cache_mu);
    for (int i = 0; i < CACHE_BUCKETS; i++) {
        Entry *e = cache[i];
        while (e) {
            Entry *n = e->next;
            entry_drop_locked(e, &to_free);
            e = n;
        }
        cache[i] = NULL;
    }
    pthread_mutex_unlock(&cache_mu);
    free_list(to_free);
}

/* ── operand staging ───────────────────────────────────────────────────────────────────────────────────────── */

/* rows × cols fp32 from host (pitch ld) into the thread's buffer *slot, packed (pitch cols). */
static float *upload_f32(Ctx *c, void **slot, size_t *cap, const float *h, int rows, int cols, int ld,
                         const char *who)
{
    size_t bytes = (size_t)rows * cols * sizeof(float);
    float *d = (float *)dgrow(slot, cap, bytes ? bytes : 4, who);
    if (bytes) h2d_rows(c, d, h, (size_t)cols * 4, (size_t)ld * 4, (size_t)rows, who);
    return d;
}

static float *stage_c(Ctx *c, const float *C, int M, int N, int ldc, int need_old, const char *who)
{
    float *d = (float *)dgrow(&c->dC, &c->capC, (size_t)M * N * sizeof(float) + 16, who);
    if (need_old) h2d_rows(c, d, C, (size_t)N * 4, (size_t)ldc * 4, (size_t)M, who);
    return d;
}

/* the packed device result into the caller's rows (pitch ldc), through pinned host memory when they are strided */
static void finish_c(Ctx *c, float *C, const float *dC, int M, int N, int ldc, const char *who)
{
    const size_t width = (size_t)N * 4, rows = (size_t)M;
    stat_add(ST_D2H, (long long)(rows * width));
    if (ldc == N) {
        check(p2h_memcpy_d2h(C, dC, rows * width, c->stream), who);
        check(p2h_stream_sync(c->stream), who);
        return;
    }
    check(p2h_stream_sync(c->stream), who);   /* a copy from the pinned rows may still be in flight */
    char *hp = (char *)hgrow(c, rows * width, who);
    check(p2h_memcpy_d2h(hp, dC, rows * width, c->stream), who);
    check(p2h_stream_sync(c->stream), who);
    for (size_t r = 0; r < rows; r++) memcpy((char *)C + r * (size_t)ldc * 4, hp + r * width, width);
}

static void *workspace_of(Ctx *c, size_t need, size_t *bytes, const char *who)
{
    *bytes = need;
    if (need == 0) return NULL;
    dgrow(&c->dW, &c->capW, need, who);
    *bytes = c->capW;
    return c->dW;
}

/* the five-value entries' workspace (quantised rows, split partials) */
static void *workspace(Ctx *c, int mode, int M, int N, int K, size_t *bytes, const char *who)
{
    return workspace_of(c, p2h_fvb_workspace_bytes(mode, M, N, K), bytes, who);
}

/* the int8-table entries' workspace (quantised rows, and room to split K) */
static void *workspace_q8b(Ctx *c, int mode, int M, int N, int K, size_t *bytes, const char *who)
{
    return workspace_of(c, p2h_q8b_workspace_bytes(mode, M, N, K), bytes, who);
}

/* C = beta · C for alpha == 0 (blas.c:1434-1435, 1488 and 748-749). */
static void scale_only(Ctx *c, float *C, int M, int N, int ldc, float beta, const char *who)
{
    if (beta == 1.0f || M <= 0 || N <= 0) return;
    float *dC = stage_c(c, C, M, N, ldc, beta != 0.0f, who);
    check(p2h_scale_c(M, N, beta, dC, N, c->stream), who);
    finish_c(c, C, dC, M, N, ldc, who);
}

/* The int8 routes with K == 0: beta outside {0, 1} pre-scales C and no K block runs, so C is otherwise left as it
 * is – with beta == 0 too (blas.c:1436 and 1339, sgemm_i8_worker's block loop is empty). */
static void int8_empty_k(Ctx *c, float *C, int M, int N, int ldc, float beta, const char *who)
{
    if (beta != 0.0f && beta != 1.0f) scale_only(c, C, M, N, ldc, beta, who);
}

/* ── the five-value GEMMs ──────────────────────────────────────────────────────────────────────────────────── */

static void p2_sgemm_fvb_body(int M, int N, int K, float alpha, const float *A, int lda, const FiveValueB *B, float beta,
                  float *C, int ldc)
{
    static const char who[] = "p2_sgemm_fvb";
    require_panel_aligned(N, who);
    Ctx *c = ctx();
    if (M <= 0 || N <= 0) return;
    if (alpha == 0.0f) { scale_only(c, C, M, N, ldc, beta, who); return; }
    int mode = current_mode();
    if (mode != P2H_EXACT && K == 0) { int8_empty_k(c, C, M, N, ldc, beta, who); return; }
    Entry *e = fv_weight(B, K, N);
    float *dA = upload_f32(c, &c->dA, &c->capA, A, M, K, lda, who);
    float *dC = stage_c(c, C, M, N, ldc, beta != 0.0f, who);
    size_t wsb = 0;
    void *ws = (mode != P2H_EXACT && K % 4 == 0) ? workspace(c, mode, M, N, K, &wsb, who) : NULL;
    check(p2h_fvb_gemm(mode, M, N, K, alpha, dA, K, e->w, beta, dC, N, ws, wsb, c->stream), who);
    finish_c(c, C, dC, M, N, ldc, who);
    entry_put(e);
}

void p2_sgemm_fvb(int M, int N, int K, float alpha, const float *A, int lda, const FiveValueB *B, float beta,
                  float *C, int ldc)
{
    const long long t0 = now_ns();
    p2_sgemm_fvb_body(M, N, K, alpha, A, lda, B, beta, C, ldc);
    stat_call(ST_FVB_CALLS, ST_FVB_NS, t0);
}

int p2_quant_prepare(QuantA *qa, int M, int K)
{
    if (current_mode() == P2H_EXACT || K % 4 != 0 || M < 0) return -1;   /* blas.c:1175 */
    Ctx *c = ctx();
    size_t need = (size_t)(M > 0 ? M : 1) * (K > 0 ? K : 1) * sizeof(float);
    if (need > c->capq || !c->hq) {
        p2h_host_free(c->hq);
        c->hq = (float *)p2h_host_malloc(need);
        if (!c->hq) { c->capq = 0; return -1; }
        c->capq = need;
    }
    size_t sneed = (size_t)(M > 0 ? M : 1) * sizeof(float);
    if (sneed > c->caps || !c->hs) {
        free(c->hs);
        c->hs = (float *)calloc(1, sneed);
        if (!c->hs) { c->caps = 0; return -1; }
        c->caps = sneed;
    }
    qa->q = (signed char *)c->hq;
    qa->scales = c->hs;
    qa->M = M;
    qa->K = K;
    return 0;
}

void p2_quant_row(const QuantA *qa, int m, const float *row)
{
    memcpy((float *)(void *)qa->q + (size_t)m * qa->K, row, (size_t)qa->K * sizeof(float));
}

static void p2_sgemm_fvb_q8a_body(int M, int N, int K, float alpha, const QuantA *A, const FiveValueB *B, float beta, float *C,
                      int ldc)
{
    static const char who[] = "p2_sgemm_fvb_q8a";
    require_panel_aligned(N, who);
    Ctx *c = ctx();
    if (M <= 0 || N <= 0) return;
    if (alpha == 0.0f) { scale_only(c, C, M, N, ldc, beta, who); return; }
    if (K % 4 != 0) die(who, "K is not a multiple of 4 (p2_quant_prepare refuses such K)");
    /* the reference reads the codes plane in int8w mode and the two planes otherwise (blas.c:1408) */
    int mode = current_mode() == P2H_INT8W ? P2H_INT8W : P2H_INT8;
    if (K == 0) { int8_empty_k(c, C, M, N, ldc, beta, who); return; }
    Entry *e = fv_weight(B, K, N);
    float *dA = upload_f32(c, &c->dA, &c->capA, (const float *)(const void *)A->q, M, K, K, who);
    float *dC = stage_c(c, C, M, N, ldc, beta != 0.0f, who);
    size_t wsb = 0;
    void *ws = workspace(c, mode, M, N, K, &wsb, who);
    check(p2h_fvb_gemm(mode, M, N, K, alpha, dA, K, e->w, beta, dC, N, ws, wsb, c->stream), who);
    finish_c(c, C, dC, M, N, ldc, who);
    entry_put(e);
}

void p2_sgemm_fvb_q8a(int M, int N, int K, float alpha, const QuantA *A, const FiveValueB *B, float beta, float *C,
                      int ldc)
{
    const long long t0 = now_ns();
    p2_sgemm_fvb_q8a_body(M, N, K, alpha, A, B, beta, C, ldc);
    stat_call(ST_FVB_CALLS, ST_FVB_NS, t0);
}

signed char *p2_fv_pack_codes(const FiveValueB *b, int K, int N)
{
    if (K % 4 != 0 || N % 16 != 0 || K <= 0 || N <= 0) return NULL;   /* blas.c:1393 */
    Ctx *c = ctx();
    Entry *e = fv_weight(b, K, N);
    size_t bytes = (size_t)K * N;
    signed char *host = (signed char *)malloc(bytes);
    void *d = p2h_malloc(bytes);
    if (!host || !d) {
        free(host);
        p2h_free(d);
        entry_put(e);
        return NULL;
    }
    int rc = p2h_fv_pack_codes(e->w, (signed char *)d, c->stream);
    if (rc == 0) rc = p2h_memcpy_d2h(host, d, bytes, c->stream);
    if (rc == 0) rc = p2h_stream_sync(c->stream);
    p2h_free(d);
    entry_put(e);
    if (rc != 0) {
        free(host);
        return NULL;
    }
    return host;
}

/* ── int8-table GEMMs ──────────────────────────────────────────────────────────────────────────────────────── */

static void p2_sgemm_q8b_body(int M, int N, int K, float alpha, const float *A, int lda, const signed char *B,
                  const float *scales, int ldb, float beta, float *C, int ldc)
{
    static const char who[] = "p2_sgemm_q8b";
    require_panel_aligned(N, who);
    Ctx *c = ctx();
    if (M <= 0 || N <= 0) return;
    if (alpha == 0.0f) { scale_only(c, C, M, N, ldc, beta, who); return; }
    int mode = current_mode();
    if (mode != P2H_EXACT && K == 0) { int8_empty_k(c, C, M, N, ldc, beta, who); return; }
    Entry *e = q8_weight(B, scales, ldb, K, N, c->stream);
    float *dA = upload_f32(c, &c->dA, &c->capA, A, M, K, lda, who);
    float *dC = stage_c(c, C, M, N, ldc, beta != 0.0f, who);
    size_t wsb = 0;
    void *ws = (mode != P2H_EXACT && K % 4 == 0) ? workspace_q8b(c, P2H_INT8W, M, N, K, &wsb, who) : NULL;
    check(p2h_q8b_gemm(mode, M, N, K, alpha, dA, K, (const signed char *)e->dq8, N, e->dsc, beta, dC, N, ws, wsb,
                       c->stream), who);
    finish_c(c, C, dC, M, N, ldc, who);
    entry_put(e);
}

void p2_sgemm_q8b(int M, int N, int K, float alpha, const float *A, int lda, const signed char *B,
                  const float *scales, int ldb, float beta, float *C, int ldc)
{
    const long long t0 = now_ns();
    p2_sgemm_q8b_body(M, N, K, alpha, A, lda, B, scales, ldb, beta, C, ldc);
    stat_call(ST_Q8B_CALLS, ST_Q8B_NS, t0);
}

static void p2_sgemm_q8b_q8a_body(int M, int N, int K, float alpha, const QuantA *A, const signed char *B, const float *scales,
                      int ldb, float beta, float *C, int ldc)
{
    static const char who[] = "p2_sgemm_q8b_q8a";
    require_panel_aligned(N, who);
    Ctx *c = ctx();
    if (M <= 0 || N <= 0) return;
    if (alpha == 0.0f) { scale_only(c, C, M, N, ldc, beta, who); return; }
    if (K % 4 != 0) die(who, "K is not a multiple of 4 (p2_quant_prepare refuses such K)");
    if (K == 0) { int8_empty_k(c, C, M, N, ldc, beta, who); return; }
    Entry *e = q8_weight(B, scales, ldb, K, N, c->stream);
    float *dA = upload_f32(c, &c->dA, &c->capA, (const float *)(const void *)A->q, M, K, K, who);
    float *dC = stage_c(c, C, M, N, ldc, beta != 0.0f, who);
    size_t wsb = 0;
    void *ws = workspace_q8b(c, P2H_INT8W, M, N, K, &wsb, who);
    check(p2h_q8b_gemm(P2H_INT8W, M, N, K, alpha, dA, K, (const signed char *)e->dq8, N, e->dsc, beta, dC, N, ws,
                       wsb, c->stream), who);
    finish_c(c, C, dC, M, N, ldc, who);
    entry_put(e);
}

void p2_sgemm_q8b_q8a(int M, int N, int K, float alpha, const QuantA *A, const signed char *B, const float *scales,
                      int ldb, float beta, float *C, int ldc)
{
    const long long t0 = now_ns();
    p2_sgemm_q8b_q8a_body(M, N, K, alpha, A, B, scales, ldb, beta, C, ldc);
    stat_call(ST_Q8B_CALLS, ST_Q8B_NS, t0);
}

/* ── fp32 GEMM ─────────────────────────────────────────────────────────────────────────────────────────────── */

static void sgemm_body(const char *who, P2Trans transA, P2Trans transB, int M, int N, int K, float alpha,
                       const float *A, int lda, const float *B, int ldb, float beta, float *C, int ldc)
{
    Ctx *c = ctx();
    if (M <= 0 || N <= 0) return;
    if (alpha == 0.0f || K <= 0) { scale_only(c, C, M, N, ldc, beta, who); return; }   /* blas.c:748-749 */
    int tA = transA == P2_TRANS, tB = transB == P2_TRANS;
    float *dA = tA ? upload_f32(c, &c->dA, &c->capA, A, K, M, lda, who)
                   : upload_f32(c, &c->dA, &c->capA, A, M, K, lda, who);
    float *dB = tB ? upload_f32(c, &c->dB, &c->capB, B, N, K, ldb, who)
                   : upload_f32(c, &c->dB, &c->capB, B, K, N, ldb, who);
    float *dC = stage_c(c, C, M, N, ldc, beta != 0.0f, who);
    check(p2h_sgemm(tA, tB, M, N, K, alpha, dA, tA ? M : K, dB, tB ? K : N, beta, dC, N, c->stream), who);
    finish_c(c, C, dC, M, N, ldc, who);
}

static void sgemm_any(const char *who, P2Trans transA, P2Trans transB, int M, int N, int K, float alpha,
                      const float *A, int lda, const float *B, int ldb, float beta, float *C, int ldc)
{
    const long long t0 = now_ns();
    sgemm_body(who, transA, transB, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
    stat_call(ST_SG_CALLS, ST_SG_NS, t0);
}

void p2_sgemm(P2Trans transA, P2Trans transB, int M, int N, int K, float alpha, const float *A, int lda,
              const float *B, int ldb, float beta, float *C, int ldc)
{
    sgemm_any("p2_sgemm", transA, transB, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
}

void p2_sgemm_st(P2Trans transA, P2Trans transB, int M, int N, int K, float alpha, const float *A, int lda,
                 const float *B, int ldb, float beta, float *C, int ldc)
{
    sgemm_any("p2_sgemm_st", transA, transB, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
}
