/*  p2oracle.h – CPU restatement of phonon-2-c's five-value GEMM arithmetic (csrc/blas.c), for checking only.
 *
 *  TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 *  library, and only to check results against or as the CPU baseline; the product never links it.
 *
 *  Every function restates one piece of the reference and names the lines it follows. Pinning (what checks each
 *  function against something other than itself) is listed in the header comment of p2oracle.c.
 */
#ifndef P2ORACLE_H
#define P2ORACLE_H

#include <stdint.h>

/* Modes, as blas.c:1030 numbers them. */
enum { P2O_INT8 = 0, P2O_EXACT = 1, P2O_INT8W = 2 };

/* Plane packing from sign int8 [K][N] in {-1,0,1} and is_hi [K][N] (convert_weights.py:114-125). */
void p2o_pack_planes(const int8_t *sign, const uint8_t *is_hi, int K, int N, uint8_t *signs, uint8_t *flags);

/* Plane decode to the 2-bit sign code (0..3) and the flag bit of every weight (blas.h:38-45). */
void p2o_unpack_planes(const uint8_t *signs, const uint8_t *flags, int K, int N, uint8_t *code, uint8_t *flag);

/* The exact-mode fp32 weight of every (k, n): (code-1) · fmaf(flag, hi-lo, lo) (blas.c:877-897). */
void p2o_expand_exact(const uint8_t *signs, const uint8_t *flags, const float *lo, const float *hi,
                      int K, int N, float *W);

/* C = alpha · A · W + beta · C in exact mode (blas.c:60-70, 929-987, 155-186, 1481-1499). */
void p2o_sgemm_fvb_exact(int M, int N, int K, float alpha, const float *A, int lda,
                         const uint8_t *signs, const uint8_t *flags, const float *lo, const float *hi,
                         float beta, float *C, int ldc);

/* Row quantisation (blas.c:1114-1145): q [M][K] row-major int8, scales [M]. */
void p2o_quant_rows(const float *A, int M, int K, int lda, int8_t *q, float *scales);

/* Per-column int8w lo code clo[n] (blas.c:1319-1326). */
void p2o_clo(const float *lo, const float *hi, int N, uint8_t *clo);

/* int8w weight codes [K][N] row-major: (int8)((code-1) · (flag && code != 1 ? 127 : clo[n])) (blas.c:1222-1240). */
void p2o_codes_i8w(const uint8_t *signs, const uint8_t *flags, const float *lo, const float *hi, int K, int N,
                   int8_t *codes);

/* The same codes in the reference's kernel layout [N/16][K/4][16][4] (p2_fv_pack_codes, blas.c:1372-1400). */
void p2o_fv_pack_codes(const uint8_t *signs, const uint8_t *flags, const float *lo, const float *hi, int K, int N,
                       int8_t *packed);

/* The two int8 planes of the int8 mode: S = code-1, T = S masked by the flag (blas.c:1189-1220). */
void p2o_planes_i8(const uint8_t *signs, const uint8_t *flags, int K, int N, int8_t *S, int8_t *T);

/* Integer accumulators acc[M][N] = sum over k in [k0, k1) of q[m][k] · B[k][n] (blas.c:1256-1282). */
void p2o_acc_i32(const int8_t *q, int M, int K, const int8_t *B, int N, int k0, int k1, int32_t *acc);

/* The int8 GEMM on quantised A (blas.c:1296-1370): mode P2O_INT8W (codes) or P2O_INT8 (two planes); beta_zero
 * selects the store of the first 1024-row K block. C is read only when beta_zero == 0. */
void p2o_gemm_i8_run(int mode, int M, int N, int K, float alpha, const int8_t *q, const float *a_scales,
                     const uint8_t *signs, const uint8_t *flags, const float *lo, const float *hi,
                     int beta_zero, float *C, int ldc);

/* The int8-table GEMM on quantised A (blas.c:1296-1370 with the q8 plane, c1 = scales). */
void p2o_gemm_q8b_run(int M, int N, int K, float alpha, const int8_t *q, const float *a_scales,
                      const int8_t *B, int ldb, const float *scales, int beta_zero, float *C, int ldc);

/* The whole public entry: p2_sgemm_fvb in the given mode (blas.c:1481-1499, 1404-1428). */
void p2o_sgemm_fvb(int mode, int M, int N, int K, float alpha, const float *A, int lda,
                   const uint8_t *signs, const uint8_t *flags, const float *lo, const float *hi,
                   float beta, float *C, int ldc);

/* p2_sgemm_q8b in the given mode (blas.c:1448-1460, 806-836 for the exact expansion). */
void p2o_sgemm_q8b(int mode, int M, int N, int K, float alpha, const float *A, int lda,
                   const int8_t *B, const float *scales, int ldb, float beta, float *C, int ldc);

/* Producers (tensor_ops.c:204-268, 329-350, 437-463, 491-511; encoder.c:449-463, 554-568): LayerNorm and SiLU in the
 * reference's AVX2 order, and the four row producers that quantise what they make (q [rows][len], scales [rows]). */
void p2o_layer_norm_row(const float *x, const float *gamma, const float *beta, float *out, int len);
void p2o_swish_row(float *x, int len);
void p2o_ln_quant_rows(const float *X, int M, int D, int ldx, const float *gamma, const float *beta, int8_t *q,
                       float *scales);
void p2o_silu_quant_rows(const float *H, int M, int K, int ldh, int8_t *q, float *scales);
void p2o_concat_heads_quant_rows(const float *attn_h, int H, int T, int Dh, int8_t *q, float *scales);
void p2o_channel_major_quant_rows(const float *dw, int D, int T, int8_t *q, float *scales);

/* The conformer block between its linears, in the reference's order of operations, each operation rounded once:
 *   p2o_combine_softmax  scores (encoder.c:425-450) with p2_softmax's AVX2 route (tensor_ops.c:354-413)
 *   p2o_glu_channel_major  encoder.c:543-555 (expf, IEEE quotient)
 *   p2o_dwconv           p2_depthwise_conv1d (tensor_ops.c:559-648) as an fmaf chain per output
 *   p2o_dwconv_silu      p2o_dwconv, then p2_swish's AVX2 body (tensor_ops.c:437-463) over the channel-major result */
void p2o_combine_softmax(float *ac, const float *bd, int H, int T, float scale);
void p2o_glu_channel_major(const float *pw1, float *gated, int T, int D);
void p2o_dwconv(const float *x, const float *w, const float *b, float *out, int D, int T, int K);
void p2o_dwconv_silu(const float *x, const float *w, const float *b, float *out, int D, int T, int K);

/* The mode latch's decision for given P2_GEMM / P2_EXACT strings (NULL = unset), without the CPU-feature clause
 * (blas.c:1032-1047). */
int p2o_mode_from_env(const char *p2_gemm, const char *p2_exact);

#endif /* P2ORACLE_H */
