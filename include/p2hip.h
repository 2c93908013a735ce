/*  p2hip.h – the device-pointer C ABI of the MI355X five-value GEMM (libp2hip.so).
 *
 *  The thin layer the C host library (libphonon2_gemm.so, include/p2_blas.h) calls, and the entry points a caller
 *  with device-resident data uses directly. Plain C types only; streams are hipStream_t passed as void*, NULL means
 *  the calling thread's default stream of this library. Every kernel entry is asynchronous on its stream.
 *
 *  Errors: entries return 0 on success and a negative P2H_E_* code otherwise; p2h_last_error() gives the message
 *  (per thread). Nothing here falls back to the CPU: without a usable gfx950 device p2h_init fails.
 *
 *  Modes follow the reference's numbering (blas.c:1030): P2H_INT8 = 0 (A quantised, weights exact as two
 *  {-1,0,+1} planes), P2H_EXACT = 1 (fp32 expansion), P2H_INT8W = 2 (A and weights int8, the default).
 */
#ifndef P2HIP_H
#define P2HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { P2H_INT8 = 0, P2H_EXACT = 1, P2H_INT8W = 2 };

enum {
    P2H_OK = 0,
    P2H_E_ARG = -1,       /* a shape, stride, alignment or mode the entry does not accept */
    P2H_E_DEVICE = -2,    /* no usable gfx950 device, or a HIP call failed */
    P2H_E_NOMEM = -3,     /* device or pinned host allocation failed */
    P2H_E_WORKSPACE = -4  /* workspace missing or smaller than p2h_*_workspace_bytes */
};

/* Row padding of quantised activations: Q rows hold K int8 values, zero-filled up to a multiple of this. */
#define P2H_Q_KALIGN 128

/* Longest row a producer (p2h_*_quant_rows below) makes: the reference's widest producer row, P2_FF_DIM
 * (phonon2.h:76, the SiLU row buffer at tensor_ops.c:502). */
#define P2H_PROD_KMAX 4096

/* ── runtime ────────────────────────────────────────────────────────────────────────────────────────────────── */

int         p2h_init(void);                 /* device 0 must be gfx950; idempotent, thread-safe */
const char *p2h_last_error(void);
const char *p2h_device_name(void);          /* gcnArchName of the device in use */
int         p2h_device_cu_count(void);
/* Re-read the tuning and comparison switches (P2H_TILE, P2H_SPLIT_ROWS, P2H_EXACT_CHAIN, P2H_XF_STAGED, P2H_XF_TILE,
 * P2H_SGEMM_ANY, P2H_ATTENTION_FUSED, P2H_SILU_EPILOGUE, P2H_EXACT_EPILOGUE, P2H_STACK_NORM_PAIRS, P2H_CONV_QUANT,
 * P2H_CONV_TT, P2H_QUANT_RPW, P2H_DEVICE_SCOPE_STORES, P2H_RECORDS_IN_REGISTERS, P2H_XCD_ROWS) from the
 * environment. They are read once at initialisation; no launch reads the environment. No reference counterpart: for
 * tests and tuning runs that change a switch within one process. */
int         p2h_reload_switches(void);

void *p2h_stream_create(void);              /* a default-priority stream; NULL on failure */
int   p2h_stream_destroy(void *stream);
int   p2h_stream_sync(void *stream);
void *p2h_thread_stream(void);              /* this thread's stream (created on first use) */

void *p2h_malloc(size_t bytes);             /* device memory; NULL on failure */
int   p2h_free(void *dptr);
void *p2h_host_malloc(size_t bytes);        /* pinned host memory */
int   p2h_host_free(void *hptr);
int   p2h_memset(void *dptr, int value, size_t bytes, void *stream);
int   p2h_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream);
int   p2h_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream);
int   p2h_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream);
/* Row-strided copies: `rows` rows of `row_bytes`, source and destination pitches in bytes. */
int   p2h_memcpy2d_h2d(void *dst, size_t dpitch, const void *src, size_t spitch, size_t row_bytes, size_t rows,
                       void *stream);
int   p2h_memcpy2d_d2h(void *dst, size_t dpitch, const void *src, size_t spitch, size_t row_bytes, size_t rows,
                       void *stream);

/* Stream capture into a HIP graph, for launch-bound chains of these entry points (every kernel entry here is
 * capturable: none allocates, synchronises or records a memset). end returns an executable graph. */
int   p2h_capture_begin(void *stream);
int   p2h_capture_end(void *stream, void **graph_exec);
int   p2h_graph_launch(void *graph_exec, void *stream);
int   p2h_graph_destroy(void *graph_exec);

void *p2h_event_create(void);
int   p2h_event_destroy(void *event);
int   p2h_event_record(void *event, void *stream);
int   p2h_event_sync(void *event);
int   p2h_stream_wait_event(void *stream, void *event);   /* later work on stream waits for event (also in capture) */
float p2h_event_elapsed_ms(void *start, void *stop);   /* < 0 on error */
/* Keep the stream busy for about usec microseconds (≤ 1 s) with one sleeping wave, so that launches queued behind it
 * run back to back without host submission gaps: used to time single kernels. No counterpart in the reference. */
int   p2h_stream_hold(void *stream, unsigned usec);

/* ── five-value weights ─────────────────────────────────────────────────────────────────────────────────────────
 *  A device-resident five-value weight [K, N] (blas.h:38-45 FiveValueB; phonon2.h:116-126 Weight), made from the
 *  sign and flag planes as the reference stores them (signs [K][N/4], flags [K][N/8]) and lo[N], hi[N]: the 4-bit
 *  selector records every kernel reads (half a byte per weight), lo and hi, and the per-column epilogue tables
 *  derived on the device: clo[n] (blas.c:1319-1326), hi[n]/127 (blas.c:1327-1328), lo[n] and hi[n]-lo[n]
 *  (blas.c:1329-1333). The planes themselves are not kept. N % 16 == 0. */
typedef struct P2hWeight P2hWeight;

/* Upload from host memory (an mmap of weights.bin, weights.c:300-312); the planes pass through a device staging
 * buffer freed before the call returns. Synchronous. NULL on failure. */
P2hWeight *p2h_fv_weight_upload(const unsigned char *signs, const unsigned char *flags, const float *lo,
                                const float *hi, int K, int N);
/* Make a weight from planes already in device memory: the records are built from them during the call, lo and hi
 * are used in place (they must outlive the handle); the planes are not read again. Synchronous. */
P2hWeight *p2h_fv_weight_wrap(const void *d_signs, const void *d_flags, const float *d_lo, const float *d_hi,
                              int K, int N);
void   p2h_weight_free(P2hWeight *w);
int    p2h_weight_shape(const P2hWeight *w, int *K, int *N);
size_t p2h_weight_device_bytes(const P2hWeight *w);   /* bytes this handle allocated */

/* The int8w codes in the reference's kernel layout [N/16][K/4][16][4] (p2_fv_pack_codes, blas.c:1372-1400) into
 * d_codes (K·N bytes). K % 4 == 0. */
int p2h_fv_pack_codes(const P2hWeight *w, signed char *d_codes, void *stream);

/* ── activations ─────────────────────────────────────────────────────────────────────────────────────────────── */

/* Per-row int8 quantisation (blas.c:1114-1145): scale = amax/127 (1 for a zero row), q = round-half-even(x/scale
 * as x·(1/scale)) saturated, the K % 16 tail as lrintf(x/scale) clamped to ±127. K % 4 == 0.
 * Q is stored tiled for the matrix cores, as the reference's QuantA.q is private to its GEMM (blas.c:1151-1154):
 * rows are padded to Mp = roundup(M, 16) and columns to ldq (a multiple of P2H_Q_KALIGN, >= roundup(K,
 * P2H_Q_KALIGN)), pads written as 0, and byte (m, k) sits at
 *     ((m/16)·(ldq/64) + k/64)·1024 + ((k%64)/16·16 + m%16)·16 + k%16,
 * i.e. one 1 KB block per 16 rows × 64 columns. The buffer holds Mp·ldq bytes (p2h_q_bytes for ldq = p2h_q_ld). */
int p2h_quant_rows(int M, int K, const float *dA, int lda, signed char *dQ, int ldq, float *dScales, void *stream);
int p2h_q_ld(int K);              /* the smallest valid ldq for K */
size_t p2h_q_bytes(int M, int K); /* bytes of Q for M rows at ldq = p2h_q_ld(K) */

/* Producers: the rows a quantised linear reads, made and quantised in one launch, into the same tiled Q and scales
 * as p2h_quant_rows (same quantisation, same padding; ldq <= P2H_PROD_KMAX). Each computes in IEEE single precision
 * with every operation rounded as written:
 *   p2h_layer_norm_quant_rows     LayerNorm of each row of X [M][ldx] (eps 1e-5), then quantised
 *                                 (p2_layer_norm_quant_rows, tensor_ops.c:329-350 with p2_layer_norm, :204-268):
 *                                 the sums in the reference's AVX2 order (eight running lanes, then their
 *                                 pairwise sum), inv_std = 1/sqrtf(var + 1e-5) correctly rounded,
 *                                 y = fmaf((x − mean)·inv_std, gamma, beta). 1 <= D <= P2H_PROD_KMAX.
 *   p2h_silu_quant_rows           x · (1/(1 + e^−x)) of each row of H [M][ldh], e^x as p2_exp_avx2
 *                                 (tensor_ops.c:154-175), then quantised (p2_swish_quant_rows, tensor_ops.c:491-511).
 *                                 K % 8 == 0 (the reference's eight-wide route; its scalar tail calls expf).
 *   p2h_concat_heads_quant_rows   attention heads [H][T][Dh] as rows [T][H·Dh], quantised (concat_heads with a
 *                                 QuantA, encoder.c:449-463).
 *   p2h_channel_major_quant_rows  channel-major [D][T] as rows [T][D], quantised (channel_major_to_rows with a
 *                                 QuantA, encoder.c:554-568).
 * The reference's x86 build computes 1/sqrtf and 1/(1 + e) through approximate reciprocals refined by one Newton
 * step, so its LayerNorm and SiLU values differ from these in the last bits and a quantised code, rarely, by one. */
/* Self-check, no counterpart in the reference: the SiLU producer divides by 1 + e^-x (in [1, 2^126)) with the
 * hardware reciprocal and one Newton step; this compares that with the IEEE quotient for every float of [1, 2^126)
 * on the device and returns {mismatches, smallest mismatching bit pattern (or ~0), values checked}. Synchronous. */
int p2h_recip_selftest(unsigned long long *result3);

int p2h_layer_norm_quant_rows(int M, int D, const float *dX, int ldx, const float *dGamma, const float *dBeta,
                              signed char *dQ, int ldq, float *dScales, void *stream);
/* Two LayerNorms of the same rows in one pass (the block's output norm, then the next block's first norm:
 * encoder.c:623 then 342): Y = LayerNorm(X; gamma1, beta1) as fp32 rows [M][ldy] (Y may be X), then the int8 rows
 * and scales of LayerNorm(Y; gamma2, beta2), each as p2h_layer_norm_quant_rows / p2h_layer_norm_rows makes them, the
 * same bits. D <= 1024. */
int p2h_layer_norm2_quant_rows(int M, int D, const float *dX, int ldx, const float *dGamma1, const float *dBeta1,
                               float *dY, int ldy, const float *dGamma2, const float *dBeta2, signed char *dQ, int ldq,
                               float *dScales, void *stream);
int p2h_silu_quant_rows(int M, int K, const float *dH, int ldh, signed char *dQ, int ldq, float *dScales, void *stream);
int p2h_concat_heads_quant_rows(int H, int T, int Dh, const float *dAttnH, signed char *dQ, int ldq, float *dScales,
                                void *stream);
int p2h_channel_major_quant_rows(int D, int T, const float *dDW, signed char *dQ, int ldq, float *dScales, void *stream);

/* ── the five-value GEMM ─────────────────────────────────────────────────────────────────────────────────────── */

/* C = alpha · A · W + beta · C on quantised A (p2_sgemm_fvb_q8a, blas.c:1430-1437, and sgemm_i8_run,
 * blas.c:1296-1370): mode P2H_INT8W or P2H_INT8; beta 0 stores, 1 accumulates, any other value pre-scales C.
 * The int32 sums run over K blocks of 1024 rows and each block is folded into C in fp32 as the reference does. */
int p2h_fvb_gemm_q8a(int mode, int M, int N, int K, float alpha, const signed char *dQ, int ldq,
                     const float *dScales, const P2hWeight *w, float beta, float *dC, int ldc, void *workspace,
                     size_t workspace_bytes, void *stream);

/* p2h_fvb_gemm_q8a with the weight the caller multiplies next: while this product runs, its workgroups also read
 * the operand records that product will read (for the same M) into the memory-side cache, so its first loads do
 * not wait on HBM. Results are those of p2h_fvb_gemm_q8a; `next` may be NULL. No counterpart in the reference:
 * for callers that run a known sequence of linears (an encoder's 216 per window). Only the small-M tiles
 * (M <= 1024) read ahead. */
int p2h_fvb_gemm_q8a_next(int mode, int M, int N, int K, float alpha, const signed char *dQ, int ldq,
                          const float *dScales, const P2hWeight *w, float beta, float *dC, int ldc, void *workspace,
                          size_t workspace_bytes, const P2hWeight *next, void *stream);
/* C [M][N] = SiLU(alpha·A·W) (beta 0, ldc = N, N % 8 == 0): the feed-forward's up-projection followed by the SiLU
 * that p2_swish_quant_rows applies before quantising (tensor_ops.c:491-511, encoder.c:345-346), as the AVX2 body's
 * polynomial per element, the same bits as p2h_fvb_gemm_q8a then p2h_silu. Small-M tiles apply it as they store C;
 * the others by a second kernel. */
int p2h_fvb_gemm_q8a_silu(int mode, int M, int N, int K, float alpha, const signed char *dQ, int ldq,
                          const float *dScales, const P2hWeight *w, float *dC, void *workspace,
                          size_t workspace_bytes, void *stream);
/* The same product for `groups` (<= 32) weights of one shape [K, N] against the same quantised rows, C_q = alpha·A·W_q
 * + beta·C_q, in one launch where the small-M kernel serves the shape (M <= 1024, K <= 4096), otherwise one call per
 * weight; results are those of p2h_fvb_gemm_q8a per weight. No counterpart in the reference: it batches products
 * that share their activation rows, such as the 24 blocks' positional projections, which the reference runs as
 * p2_sgemm_fvb calls on the same positional rows (encoder.c:500). */
int p2h_fvb_gemm_q8a_grouped(int mode, int M, int N, int K, float alpha, const signed char *dQ, int ldq,
                             const float *dScales, const P2hWeight *const *w, int groups, float beta,
                             float *const *dC, int ldc, void *stream);
/* Bytes of workspace that let p2h_fvb_gemm_q8a split K across workgroups (0 when the call would not split). With
 * workspace NULL the call runs unsplit. A split call writes int32 partial sums per 1024-row block and a second
 * kernel adds them (exact) and folds the blocks in order, so results do not depend on the split. Calls sharing a
 * workspace must be stream-ordered. */
size_t p2h_fvb_q8a_workspace_bytes(int mode, int M, int N, int K);
/* The tile and split p2h_fvb_gemm_q8a chooses for a shape, as text (per thread; valid until the next call). */
const char *p2h_fvb_plan(int mode, int M, int N, int K, int with_workspace);

/* C = alpha · A · W + beta · C on fp32 A (p2_sgemm_fvb, blas.c:1481-1499): the int8 modes quantise A into the
 * workspace (at least p2h_fvb_workspace_bytes) and run p2h_fvb_gemm_q8a; P2H_EXACT (or K % 4 != 0) runs the fp32 expansion route, whose per-output
 * fmaf chain over k = 0..K-1 is the reference's exact kernel (blas.c:155-186, 929-987). */
int    p2h_fvb_gemm(int mode, int M, int N, int K, float alpha, const float *dA, int lda, const P2hWeight *w,
                    float beta, float *dC, int ldc, void *workspace, size_t workspace_bytes, void *stream);
size_t p2h_fvb_workspace_bytes(int mode, int M, int N, int K);

/* No counterpart in the reference: p2h_fvb_gemm for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc). It takes no workspace argument and allocates nothing:
 * its quantised rows and split partials live in a device array of P2H_NOALLOC_SCRATCH_BYTES that the library holds
 * on each GPU it runs on until the process ends. Shapes whose p2h_fvb_workspace_bytes exceeds that size are refused
 * with P2H_E_WORKSPACE (M = 6000 at K = 4096 fits: 24.6 MB). `stream` must be the caller's own (non-NULL). Calls on
 * one GPU share its array: calls that overlap in time on one GPU (other streams, other threads) race and must be
 * ordered by the caller. Nothing in the array needs to start at zero (every byte a kernel reads was written earlier
 * in the same call). Results are those of p2h_fvb_gemm. */
#define P2H_NOALLOC_SCRATCH_BYTES (32u << 20)
int    p2h_fvb_gemm_noalloc(int mode, int M, int N, int K, float alpha, const float *dA, int lda, const P2hWeight *w,
                            float beta, float *dC, int ldc, void *stream);
size_t p2h_noalloc_scratch_bytes(void);

/* The raw int32 accumulators sum_k q[m][k]·B[k][n] over all K of the int8 kernel (blas.c:1256-1282): for
 * P2H_INT8W B is the codes plane into dAcc; for P2H_INT8 the S plane into dAcc and the T plane into dAcc2. */
int p2h_fvb_acc_i32(int mode, int M, int N, int K, const signed char *dQ, int ldq, const P2hWeight *w,
                    int32_t *dAcc, int32_t *dAcc2, int ldacc, void *stream);

/* C = beta · C (scale_c, blas.c:60-70), the alpha == 0 case. */
int p2h_scale_c(int M, int N, float beta, float *dC, int ldc, void *stream);

/* ── int8-table weights (p2_sgemm_q8b / p2_sgemm_q8b_q8a, blas.c:1439-1479) ────────────────────────────────────
 *  B int8 [K][ldb] in device memory with one fp32 scale per column. N % 16 == 0. */
int p2h_q8b_gemm_q8a(int M, int N, int K, float alpha, const signed char *dQ, int ldq, const float *dScales,
                     const signed char *dB, int ldb, const float *dBscales, float beta, float *dC, int ldc,
                     void *stream);
/* p2_sgemm_q8b (blas.c:1439-1446): fp32 rows A quantised into the workspace (int8 modes), then the GEMM; P2H_EXACT
 * (or K % 4 != 0) runs the fp32 expansion. The workspace holds the quantised rows (it must have at least that many
 * bytes); with p2h_q8b_workspace_bytes bytes, a call with few rows and K beyond 1024 also splits K across workgroups
 * at the 1024-row blocks (int32 partial sums folded in order by a second kernel: the same bits). Stream-ordered. */
int p2h_q8b_gemm(int mode, int M, int N, int K, float alpha, const float *dA, int lda, const signed char *dB,
                 int ldb, const float *dBscales, float beta, float *dC, int ldc, void *workspace,
                 size_t workspace_bytes, void *stream);
/* Workspace bytes for p2h_q8b_gemm with room to split K (0 in P2H_EXACT or when K % 4 != 0). No counterpart in the
 * reference, which needs no device workspace. */
size_t p2h_q8b_workspace_bytes(int mode, int M, int N, int K);

/* ── fp32 GEMM (p2_sgemm, blas.h:25-29): C = alpha · op(A) · op(B) + beta · C, row-major, trans 0/1 ──────── *
 *  On the fp32 matrix cores: sums in their order, within fp32 rounding of the reference's. */
int p2h_sgemm(int transA, int transB, int M, int N, int K, float alpha, const float *dA, int lda,
              const float *dB, int ldb, float beta, float *dC, int ldc, void *stream);
/* The same for `batch` (<= 65535) products in one launch, entry b at A + b·strideA, B + b·strideB, C + b·strideC
 * (strides in floats): the per-head products of attention, which the reference runs as one p2_sgemm_st per
 * (head, row block) (heads_gemm, encoder.c:279-316, 505-519). */
int p2h_sgemm_batched(int transA, int transB, int M, int N, int K, float alpha, const float *dA, int lda,
                      long long strideA, const float *dB, int ldb, long long strideB, float beta, float *dC, int ldc,
                      long long strideC, int batch, void *stream);

/* ── the conformer block between its linears (device pointers, asynchronous) ────────────────────────────────────
 * The model's fixed widths: D = 1024 channels, 8 heads of 128 (phonon2.h:73-78); T frames, L = 2T − 1 positions.
 *   p2h_gather_heads       QKV [T][3D] (q | k | v) → Q_u = q + bias_u, Q_v = q + bias_v, V as [8][T][128] and K
 *                          transposed as [8][128][T] (gather_heads, encoder.c:366-404)
 *   p2h_transpose_pos      P [L][D] → [8][128][L] (transpose_pos, encoder.c:406-423)
 *   p2h_combine_softmax    AC [8·T][T] in place: softmax((AC + relative shift of BD [8·T][L]) / sqrt(128)) per row
 *                          (combine_softmax, encoder.c:425-450, p2_softmax's AVX2 route, tensor_ops.c:354-413: the
 *                          exponential of p2_exp_avx2, eight running sums, the tail T mod 8 with expf)
 *   p2h_glu_channel_major  pw1 [T][2D] → gated [D][T] = first half / (1 + e^−second half) (glu_to_channel_major,
 *                          encoder.c:543-555; expf)
 *   p2h_depthwise_conv_silu  dw [D][T] = SiLU(depthwise convolution of gated [D][T] with w [D][9], b [D], padding 4)
 *                          (p2_depthwise_conv1d then p2_swish, tensor_ops.c:559-648, 437-491; encoder.c:597-598)
 *   p2h_silu               x · sigmoid(x) in place on n floats (p2_swish, tensor_ops.c:437-491)
 *   p2h_add_residual       X [T][D] += alpha · Y (add_residual, encoder.c:252-275)
 *   p2h_layer_norm_rows    Y = LayerNorm(X) per row, eps 1e-5, X == Y allowed (p2_layer_norm_rows(_inplace),
 *                          tensor_ops.c:204-332), the same arithmetic as p2h_layer_norm_quant_rows
 *   p2h_concat_heads_rows  heads [8][T][128] → rows [T][D] fp32 (concat_heads, encoder.c:452-466)
 *   p2h_channel_major_rows channel-major [D][T] → rows [T][D] fp32 (channel_major_to_rows, encoder.c:557-571)
 * Transcendentals use expf where the reference calls libm (GLU, softmax and SiLU tails) and the reference's AVX2
 * polynomial where it does (softmax and SiLU bodies); every quotient and square root is correctly rounded. */
int p2h_gather_heads(int T, const float *dQKV, const float *dBiasU, const float *dBiasV, float *dQu, float *dQv,
                     float *dKt, float *dVh, void *stream);
int p2h_transpose_pos(int L, const float *dP, float *dPt, void *stream);
int p2h_combine_softmax(int T, float *dAC, const float *dBD, void *stream);
int p2h_glu_channel_major(int T, const float *dPW1, float *dGated, void *stream);
int p2h_depthwise_conv_silu(int T, const float *dGated, const float *dW, const float *dB, float *dOut, void *stream);
/* p2h_glu_channel_major then p2h_depthwise_conv_silu in one kernel (encoder.c:594-597): pw1 [T][2048] → out
 * [1024][T], the same bits, without the gated buffer. */
int p2h_glu_depthwise_conv_silu(int T, const float *dPW1, const float *dW, const float *dB, float *dOut,
                                void *stream);
/* The same with out [T][1024]: the transpose of the channel-major output, the rows that channel_major_to_rows
 * (encoder.c:554-568) would make for the pw2 linear; the same bits. */
int p2h_glu_depthwise_conv_silu_rows(int T, const float *dPW1, const float *dW, const float *dB, float *dOut,
                                     void *stream);
/* The int8 modes' form of the convolution module's middle (encoder.c:594-597 with channel_major_to_rows' QuantA
 * branch, encoder.c:554-568): GLU, depthwise convolution and SiLU of pw1's rows [T][2048], quantised per output row
 * into Q [roundup(T, 16)][ldq] (tiled as p2h_quant_rows stores it, pad rows and columns zero) and scales [T]: the
 * bits of p2h_glu_depthwise_conv_silu_rows followed by p2h_quant_rows, in one kernel, with no fp32 rows written.
 * No separate reference function: the reference runs these steps on the CPU between its linears. */
int p2h_glu_depthwise_conv_silu_quant_rows(int T, const float *dPW1, const float *dW, const float *dB,
                                           signed char *dQ, int ldq, float *dScales, void *stream);
int p2h_silu(size_t n, float *dX, void *stream);
int p2h_add_residual(int T, float *dX, const float *dY, float alpha, void *stream);
int p2h_layer_norm_rows(int M, int D, const float *dX, int ldx, const float *dGamma, const float *dBeta, float *dY,
                        int ldy, void *stream);
int p2h_concat_heads_rows(int T, const float *dAttnH, float *dY, void *stream);
int p2h_channel_major_rows(int T, const float *dDW, float *dY, void *stream);

/* Relative-position self-attention of all 8 heads between the projections (encoder.c:495-523: gather_heads,
 * transpose_pos, the two score products, combine_softmax and the product with V, heads_gemm encoder.c:279-316) in
 * one kernel: QKV [T][3·1024] (q | k | v rows), bias_u / bias_v [1024], the projected positional rows P
 * [2T − 1][1024] → attn_h [8][T][128]. The softmax is combine_softmax's arithmetic in its order; the score and
 * output products are fp32 matrix-core sums (another order than the reference's packed sgemm). T <= 768, every
 * pointer 16-byte aligned. */
#define P2H_ATTENTION_TMAX 768
int p2h_attention_heads(int T, const float *dQKV, const float *dBiasU, const float *dBiasV, const float *dP,
                        float *dAttnH, void *stream);
/* The same written as attn [T][1024], head h at columns 128·h: the rows concat_heads makes (encoder.c:449-463) for
 * the output linear; the same bits. */
int p2h_attention_rows(int T, const float *dQKV, const float *dBiasU, const float *dBiasV, const float *dP,
                       float *dAttn, void *stream);

/* One FastConformer block on the device (conformer_block, encoder.c:617-625): feed-forward ½, relative-position
 * self-attention, convolution module, feed-forward ½, final LayerNorm, on X [T][1024] in place. The five-value
 * linears run in `mode` (P2H_INT8W / P2H_INT8: LayerNorm, SiLU, head concatenation and the channel-major transpose
 * quantise their rows as they make them and the residuals are the GEMMs' beta-1 epilogues, as the reference's int8
 * path does; P2H_EXACT: fp32 rows, the fp32-input GEMM and separate residual adds, as its fp32 path does). PE is
 * the window's positional table [2T − 1][1024] (rel_pos_encoding, encoder.c:79-96), shared by every block. The
 * workspace is p2h_conformer_block_workspace_bytes(mode, T) bytes, 256-byte aligned. Norm vectors [1024], bias_u /
 * bias_v [8·128], dw_w [1024·9] and dw_b [1024] are device pointers. */
typedef struct P2hBlock {
    const float *norm_ff1_w, *norm_ff1_b;
    const P2hWeight *ff1_l1, *ff1_l2;            /* [1024, 4096], [4096, 1024] */
    const float *norm_sa_w, *norm_sa_b;
    const P2hWeight *qkv, *pos, *out;            /* [1024, 3072], [1024, 1024], [1024, 1024] */
    const float *bias_u, *bias_v;
    const float *norm_conv_w, *norm_conv_b;
    const P2hWeight *pw1, *pw2;                  /* [1024, 2048], [1024, 1024] */
    const float *dw_w, *dw_b;
    const float *norm_ff2_w, *norm_ff2_b;
    const P2hWeight *ff2_l1, *ff2_l2;
    const float *norm_out_w, *norm_out_b;
} P2hBlock;

size_t p2h_conformer_block_workspace_bytes(int mode, int T);
int    p2h_conformer_block(int mode, const P2hBlock *blk, int T, const float *dPE, float *dX, void *workspace,
                           size_t workspace_bytes, void *stream);

/* The block stack of one window (encode_blocks, encoder.c:628-644): blocks[0 .. n_blocks − 1] in order on x
 * [T][1024] in place, with the shared positional rows pe [2T − 1][1024]. The same results as p2h_conformer_block
 * called block after block, bit for bit; in the int8 modes the positional rows are quantised once and all the
 * blocks' positional projections run as grouped launches before the first block. The workspace is
 * p2h_conformer_stack_workspace_bytes(mode, T, n_blocks) bytes, 256-byte aligned (one block's, plus the n
 * projections in the int8 modes). */
size_t p2h_conformer_stack_workspace_bytes(int mode, int T, int n_blocks);
int    p2h_conformer_stack(int mode, const P2hBlock *blocks, int n_blocks, int T, const float *dPE, float *dX,
                           void *workspace, size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* P2HIP_H */
