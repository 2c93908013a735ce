/*  p2_blas.h – the drop-in boundary: the reference's GEMM API (csrc/blas.h) served by libphonon2_gemm.so on one
 *  MI355X.
 *
 *  Every declaration below has the reference's name, C signature, argument meaning and error behaviour; a program
 *  built against the reference's blas.h and phonon2.h links against libphonon2_gemm.so instead of blas.o with no
 *  source change. Types are ABI-identical to the reference's (struct layout, enum values).
 *
 *  All pointers are host memory owned by the caller, as in the reference. Each call copies its operands to the GPU,
 *  runs the HIP kernels of libp2hip.so (include/p2hip.h) on the calling thread's stream and returns with C complete
 *  in host memory. Five-value and int8-table weights are uploaded once and cached on the device, keyed on their
 *  plane pointers and shape plus a content fingerprint (lo, hi and the first and last bytes of each plane);
 *  p2_gpu_weight_cache_clear() drops the cache (for callers that unmap and remap weights at the same address).
 *  Contract of the cache: a weight is immutable while its address is in use – the reference's weights are a read-only
 *  mmap (weights.c:551) – since a change in the middle of a plane at the same address is not seen. A caller that
 *  changes weights in place sets P2_GPU_WEIGHT_CACHE=0 (read once): every call then uploads its weight and frees the
 *  copy when it returns. Calls from many threads may share weights, and clearing the cache while they run is safe:
 *  a copy in use is freed by the last call using it.
 *
 *  Nothing falls back to the CPU: if the GPU library cannot start, the first call prints the reason and aborts.
 */
#ifndef P2_BLAS_H
#define P2_BLAS_H

/* P2Trans (blas.h:19-22) */
typedef enum {
    P2_NO_TRANS = 111,
    P2_TRANS    = 112
} P2Trans;

/* FiveValueB (blas.h:38-45): w[k][n] = (code − 1) · (flag ? hi[n] : lo[n]) with code the 2-bit field at
 * signs[k][n/4] bits 2·(n&3) (0 → −1, 1 → 0, 2 → +1) and flag bit (n&7) of flags[k][n/8]. */
typedef struct {
    const unsigned char *signs;  /* [K][N/4] */
    const unsigned char *flags;  /* [K][N/8] */
    const float         *lo;     /* [N] */
    const float         *hi;     /* [N] */
    const signed char   *codes;  /* optional pre-packed int8w codes (p2_fv_pack_codes) or NULL; this library reads the
                                    planes either way (the codes are a function of them) */
} FiveValueB;

#ifndef PHONON2_H
/* QuantA (phonon2.h:432-436). In this library q holds the K fp32 values of each row as p2_quant_row received them
 * (row m at byte offset 4·m·K); they are quantised on the GPU, with the reference's arithmetic, by the GEMM that
 * consumes them. Callers never read q or scales (tensor_ops.c:53, 57 read only M and K). */
typedef struct {
    signed char *q;
    float       *scales;
    int          M, K;
} QuantA;
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* blas.h:25-29 – C = alpha · op(A) · op(B) + beta · C, row-major. */
void p2_sgemm(P2Trans transA, P2Trans transB, int M, int N, int K, float alpha, const float *A, int lda,
              const float *B, int ldb, float beta, float *C, int ldc);

/* blas.h:32-36 – the same; safe to call from many threads at once. */
void p2_sgemm_st(P2Trans transA, P2Trans transB, int M, int N, int K, float alpha, const float *A, int lda,
                 const float *B, int ldb, float beta, float *C, int ldc);

/* blas.h:51 – the int8w codes [N/16][K/4][16][4] in malloc'd host memory (caller frees); NULL if K % 4 or
 * N % 16 is not 0 or on failure. */
signed char *p2_fv_pack_codes(const FiveValueB *b, int K, int N);

/* blas.h:54-57 – int8 weight table with one fp32 scale per column. N % 16 == 0 or abort. */
void p2_sgemm_q8b(int M, int N, int K, float alpha, const float *A, int lda, const signed char *B,
                  const float *scales, int ldb, float beta, float *C, int ldc);

/* blas.h:60-63 – the five-value GEMM. N % 16 == 0 or abort. */
void p2_sgemm_fvb(int M, int N, int K, float alpha, const float *A, int lda, const FiveValueB *B, float beta,
                  float *C, int ldc);

/* blas.h:67-68 – the mode, latched once from P2_GEMM / P2_EXACT (blas.c:1032-1047). */
const char *p2_gemm_mode(void);
int p2_gemm_exact(void);

/* blas.h:72-73 – pre-quantised activations. prepare returns −1 in exact mode or when K % 4 != 0. */
int  p2_quant_prepare(QuantA *qa, int M, int K);
void p2_quant_row(const QuantA *qa, int m, const float *row);

/* blas.h:76-79 – the int8 GEMMs on pre-quantised A; beta 0 stores, 1 accumulates, other values pre-scale C. */
void p2_sgemm_fvb_q8a(int M, int N, int K, float alpha, const QuantA *A, const FiveValueB *B, float beta, float *C,
                      int ldc);
void p2_sgemm_q8b_q8a(int M, int N, int K, float alpha, const QuantA *A, const signed char *B, const float *scales,
                      int ldb, float beta, float *C, int ldc);

/* No counterpart in the reference: drop every cached device copy of a weight (callers that free weights and map
 * new ones at the same addresses call it in between; p2_free_weights, weights.c:578-580, is where). */
void p2_gpu_weight_cache_clear(void);

/* No counterpart in the reference: the calls made since the last take, then reset. out[0..8]: five-value GEMM calls
 * (p2_sgemm_fvb, p2_sgemm_fvb_q8a) and ms inside them; int8-table calls and ms; fp32 p2_sgemm / p2_sgemm_st calls
 * and ms; ms of those spent uploading weights on first touch; MB of operands copied host to device and device to
 * host. The ms are summed over calling threads. For measuring what an engine window spends in the GEMMs. */
#define P2_GPU_STATS_N 9
void p2_gpu_stats_take(double out[P2_GPU_STATS_N]);

#ifdef __cplusplus
}
#endif

#endif /* P2_BLAS_H */
