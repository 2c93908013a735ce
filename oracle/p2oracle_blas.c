/*  p2oracle_blas.c – the reference's quantised-GEMM entry points (csrc/blas.h) computed by the CPU oracle.
 *
 *  TEST INFRASTRUCTURE ONLY. It lets the reference engine (built from its own sources by oracle/Makefile) run its
 *  five-value and int8-table linears through the oracle's int8 / int8w arithmetic on a host whose reference build
 *  has only the exact route (blas.c:1021-1023, 1043-1045), so that end-to-end token ids of the GPU library can be
 *  compared with the same engine on the oracle. The fp32 GEMMs (p2_sgemm, p2_sgemm_st) stay the reference's own.
 *
 *  Entry points, each with the reference's signature and argument conventions (blas.h:38-79):
 *    p2_gemm_mode / p2_gemm_exact   mode latch from P2_GEMM / P2_EXACT once per process (blas.c:1027-1066), without
 *                                   the CPU-feature clause, as the GPU library latches it
 *    p2_quant_prepare / _row        per-thread rows of fp32 activations (the GEMM quantises them, p2o_quant_rows)
 *    p2_sgemm_fvb / _q8a            p2o_sgemm_fvb in the latched mode (q8a: the codes plane in int8w, two planes in
 *                                   int8; blas.c:1430-1437)
 *    p2_sgemm_q8b / _q8a            p2o_sgemm_q8b (blas.c:1439-1479)
 *    p2_fv_pack_codes               p2o_fv_pack_codes into malloc'd memory (blas.c:1372-1400)
 */
#include "../include/p2_blas.h"
#include "p2oracle.h"

#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int mode_latched = -1;
static pthread_once_t mode_once = PTHREAD_ONCE_INIT;

static void mode_init(void) { mode_latched = p2o_mode_from_env(getenv("P2_GEMM"), getenv("P2_EXACT")); }

static int mode_now(void)
{
    pthread_once(&mode_once, mode_init);
    return mode_latched;
}

int p2_gemm_exact(void) { return mode_now() == P2O_EXACT; }

const char *p2_gemm_mode(void)
{
    switch (mode_now()) {
    case P2O_INT8:  return "int8 dot products, exact weights";
    case P2O_INT8W: return "int8 dot products, int8 weights";
    default:        return "fp32 expansion (exact)";
    }
}

static void panel_aligned(int N, const char *who)   /* blas.c:989-995 */
{
    if (N % 16 != 0) {
        fprintf(stderr, "%s: N = %d is not a multiple of %d\n", who, N, 16);
        abort();
    }
}

/* per-thread fp32 rows handed out by p2_quant_prepare; one QuantA feeds one GEMM (phonon2.h:429-431) */
static __thread float *rows_buf;
static __thread size_t rows_cap;
static __thread float scales_dummy[1];

int p2_quant_prepare(QuantA *qa, int M, int K)
{
    if (mode_now() == P2O_EXACT || K % 4 != 0 || M < 0) return -1;   /* blas.c:1175 */
    size_t need = (size_t)(M > 0 ? M : 1) * (size_t)(K > 0 ? K : 1);
    if (need > rows_cap) {
        free(rows_buf);
        rows_buf = (float *)malloc(need * sizeof(float));
        if (!rows_buf) { rows_cap = 0; return -1; }
        rows_cap = need;
    }
    qa->q = (signed char *)(void *)rows_buf;
    qa->scales = scales_dummy;
    qa->M = M;
    qa->K = K;
    return 0;
}

void p2_quant_row(const QuantA *qa, int m, const float *row)
{
    memcpy((float *)(void *)qa->q + (size_t)m * qa->K, row, (size_t)qa->K * sizeof(float));
}

void p2_sgemm_fvb(int M, int N, int K, float alpha, const float *A, int lda, const FiveValueB *B, float beta,
                  float *C, int ldc)
{
    panel_aligned(N, "p2_sgemm_fvb");
    if (M <= 0 || N <= 0) return;
    p2o_sgemm_fvb(mode_now(), M, N, K, alpha, A, lda, B->signs, B->flags, B->lo, B->hi, beta, C, ldc);
}

void p2_sgemm_fvb_q8a(int M, int N, int K, float alpha, const QuantA *A, const FiveValueB *B, float beta, float *C,
                      int ldc)
{
    panel_aligned(N, "p2_sgemm_fvb_q8a");
    if (M <= 0 || N <= 0) return;
    int mode = mode_now() == P2O_INT8W ? P2O_INT8W : P2O_INT8;   /* blas.c:1408 */
    p2o_sgemm_fvb(mode, M, N, K, alpha, (const float *)(const void *)A->q, K, B->signs, B->flags, B->lo, B->hi,
                  beta, C, ldc);
}

void p2_sgemm_q8b(int M, int N, int K, float alpha, const float *A, int lda, const signed char *B,
                  const float *scales, int ldb, float beta, float *C, int ldc)
{
    panel_aligned(N, "p2_sgemm_q8b");
    if (M <= 0 || N <= 0) return;
    p2o_sgemm_q8b(mode_now(), M, N, K, alpha, A, lda, (const int8_t *)B, scales, ldb, beta, C, ldc);
}

void p2_sgemm_q8b_q8a(int M, int N, int K, float alpha, const QuantA *A, const signed char *B, const float *scales,
                      int ldb, float beta, float *C, int ldc)
{
    panel_aligned(N, "p2_sgemm_q8b_q8a");
    if (M <= 0 || N <= 0) return;
    p2o_sgemm_q8b(P2O_INT8W, M, N, K, alpha, (const float *)(const void *)A->q, K, (const int8_t *)B, scales, ldb,
                  beta, C, ldc);
}

signed char *p2_fv_pack_codes(const FiveValueB *b, int K, int N)
{
    if (K % 4 != 0 || N % 16 != 0 || K <= 0 || N <= 0) return NULL;   /* blas.c:1393 */
    signed char *out = (signed char *)malloc((size_t)K * N);
    if (out) p2o_fv_pack_codes(b->signs, b->flags, b->lo, b->hi, K, N, (int8_t *)out);
    return out;
}
