/*  p2oracle.c – CPU restatement of phonon-2-c's five-value GEMM (csrc/blas.c), scalar and sequential.
 *
 *  TEST INFRASTRUCTURE ONLY: the reference for the HIP path's results and nothing else. Only tests/, __graft_entry__.smoke()
 *  and bench.py's cpu_baseline leg may load it.
 *
 *  Compiled without fast-math and with -ffp-contract=off: every rounding below is the one written.
 *
 *  What pins each function (tests/test_oracle_*.py):
 *    p2o_pack_planes / p2o_unpack_planes   round trip against an independent numpy decoder (np.unpackbits) and the
 *                                          generator's own packer; brute force on tiny K, N.
 *    p2o_expand_exact, p2o_sgemm_fvb_exact bit-exact against the reference's own p2_sgemm_fvb (exact mode, AVX2,
 *                                          built from its C sources) on committed golden vectors, including
 *                                          alpha/beta variants, ragged K, strides, non-fp16 lo/hi and code 3.
 *    p2o_sgemm_q8b (exact)                 bit-exact against the reference's p2_sgemm_q8b golden vectors.
 *    p2o_quant_rows                        invariants: |q·scale − x| ≤ scale/2, q in [−127, 127], the row maximum
 *                                          maps to ±127, zero rows give scale 1, power-of-two scaling of a row leaves
 *                                          q unchanged; ties to even on constructed rows; the K % 16 tail divides.
 *    p2o_clo / p2o_codes_i8w               invariants: codes in {0, ±clo, ±127}; clo = 127 when lo = hi; clo = 0
 *                                          when hi <= 0; |clo·hi/127 − lo| ≤ hi/254; int8 wrap for code 3.
 *    p2o_fv_pack_codes                     permutation of p2o_codes_i8w checked by an index-based numpy gather.
 *    p2o_acc_i32                           int64 numpy matmul of the same operands.
 *    p2o_gemm_i8_run / p2o_gemm_q8b_run    float64 evaluation of the same per-block products (≤ 1e-6 relative);
 *                                          the per-1024-block fmaf order is the restatement of blas.c:1355-1366.
 *    p2o_sgemm_fvb (int8 modes)            the above plus the quantisation error bound against the exact mode.
 *  Parity unpinned by a reference run: the int8/int8w routes cannot execute here (blas.c:1021-1023 compiles them only
 *  for AArch64 with the dot-product extension), so their fp32 rounding sequence rests on this restatement.
 */
#include "p2oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define KC_I8 1024   /* K rows per int8 block, blas.c:1025 */

/* ── planes (convert_weights.py:114-125, blas.h:38-45) ─────────────────────────────────────────────────────── */

void p2o_pack_planes(const int8_t *sign, const uint8_t *is_hi, int K, int N, uint8_t *signs, uint8_t *flags)
{
    for (int k = 0; k < K; k++) {
        for (int b = 0; b < N / 4; b++) {
            unsigned v = 0;
            for (int j = 0; j < 4; j++) v |= (unsigned)((sign[(size_t)k * N + 4 * b + j] + 1) & 3) << (2 * j);
            signs[(size_t)k * (N / 4) + b] = (uint8_t)v;
        }
        for (int b = 0; b < N / 8; b++) {
            unsigned v = 0;
            for (int j = 0; j < 8; j++) v |= (unsigned)(is_hi[(size_t)k * N + 8 * b + j] ? 1 : 0) << j;
            flags[(size_t)k * (N / 8) + b] = (uint8_t)v;
        }
    }
}

static inline int code_at(const uint8_t *signs, int N, int k, int n)
{
    return (signs[(size_t)k * (N / 4) + (n >> 2)] >> (2 * (n & 3))) & 3;
}

static inline int flag_at(const uint8_t *flags, int N, int k, int n)
{
    return (flags[(size_t)k * (N / 8) + (n >> 3)] >> (n & 7)) & 1;
}

void p2o_unpack_planes(const uint8_t *signs, const uint8_t *flags, int K, int N, uint8_t *code, uint8_t *flag)
{
    for (int k = 0; k < K; k++)
        for (int n = 0; n < N; n++) {
            code[(size_t)k * N + n] = (uint8_t)code_at(signs, N, k, n);
            flag[(size_t)k * N + n] = (uint8_t)flag_at(flags, N, k, n);
        }
}

/* ── exact route ───────────────────────────────────────────────────────────────────────────────────────────── */

/* blas.c:877-897 (AVX2 expansion, the x86 path): sign as a float (the LUT gives code − 1, so code 3 is +2) times
 * fmaf(flag, hi − lo, lo). */
static inline float exact_weight(int code, int flag, float lo, float hi)
{
    float d = hi - lo;
    return (float)(code - 1) * fmaf((float)flag, d, lo);
}

void p2o_expand_exact(const uint8_t *signs, const uint8_t *flags, const float *lo, const float *hi,
                      int K, int N, float *W)
{
    for (int k = 0; k < K; k++)
        for (int n = 0; n < N; n++)
            W[(size_t)k * N + n] = exact_weight(code_at(signs, N, k, n), flag_at(flags, N, k, n), lo[n], hi[n]);
}

/* blas.c:60-70 */
static void scale_c(float *C, int M, int N, int ldc, float beta)
{
    if (beta == 1.0f) return;
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            float *c = C + (size_t)i * ldc + j;
            *c = (beta == 0.0f) ? 0.0f : *c * beta;
        }
}

/* The exact kernel (blas.c:155-186 inside blas.c:960-985) keeps one fp32 accumulator per output and adds
 * fmaf(alpha·A[m][k], w[k][n], c) for k = 0 .. K−1 in order; the KC blocks store and reload C between blocks,
 * which does not change the value. */
static void exact_chain(int M, int N, int K, float alpha, const float *A, int lda, const float *W, float *C, int ldc)
{
    /* row at a time, k outer: every output still sees exactly the chain above, in k order */
    for (int m = 0; m < M; m++) {
        float *c = C + (size_t)m * ldc;
        for (int k = 0; k < K; k++) {
            float a = alpha * A[(size_t)m * lda + k];
            const float *w = W + (size_t)k * N;
            for (int n = 0; n < N; n++) c[n] = fmaf(a, w[n], c[n]);
        }
    }
}

void p2o_sgemm_fvb_exact(int M, int N, int K, float alpha, const float *A, int lda,
                         const uint8_t *signs, const uint8_t *flags, const float *lo, const float *hi,
                         float beta, float *C, int ldc)
{
    if (alpha == 0.0f) { scale_c(C, M, N, ldc, beta); return; }   /* blas.c:1488 */
    scale_c(C, M, N, ldc, beta);                                   /* blas.c:1495 */
    float *W = (float *)malloc((size_t)K * N * sizeof(float));
    p2o_expand_exact(signs, flags, lo, hi, K, N, W);
    exact_chain(M, N, K, alpha, A, lda, W, C, ldc);
    free(W);
}

/* ── int8 routes ───────────────────────────────────────────────────────────────────────────────────────────── */

static inline int8_t sat8(long v) { return (int8_t)(v > 127 ? 127 : v < -128 ? -128 : v); }

/* blas.c:1114-1145: amax over the row, scale = amax/127 (1 for a zero row), inv = 1/scale; the first K − K%16
 * entries round x·inv to nearest-even with saturation (vcvtnq_s32_f32 then two vqmovn), the tail rounds x/scale
 * with lrintf and clamps to ±127. */
static void quant_row(const float *row, int K, int8_t *q, float *scale_out)
{
    float amax = 0.0f;
    for (int k = 0; k < K; k++) { float v = fabsf(row[k]); if (v > amax) amax = v; }
    float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    *scale_out = scale;
    float inv = 1.0f / scale;
    int k16 = K / 16 * 16;
    for (int k = 0; k < k16; k++) q[k] = sat8(lrintf(row[k] * inv));
    for (int k = k16; k < K; k++) {
        long v = lrintf(row[k] / scale);
        q[k] = (int8_t)(v > 127 ? 127 : v < -127 ? -127 : v);
    }
}

void p2o_quant_rows(const float *A, int M, int K, int lda, int8_t *q, float *scales)
{
    for (int m = 0; m < M; m++) quant_row(A + (size_t)m * lda, K, q + (size_t)m * K, scales + m);
}

/* ── producers: the rows a quantised linear reads, made and quantised in one pass (tensor_ops.c, encoder.c) ────── */

/* The eight-lane horizontal sum of p2_hsum_avx2 (tensor_ops.c:182-190): v[i] + v[i+4], then pairs, then the two. */
static float hsum8(const float v[8])
{
    float s4[4];
    for (int i = 0; i < 4; i++) s4[i] = v[i] + v[i + 4];
    const float s20 = s4[0] + s4[2], s21 = s4[1] + s4[3];
    return s20 + s21;
}

/* p2_layer_norm, AVX2 route (tensor_ops.c:204-268): lane j of an 8-wide accumulator adds x[j], x[j+8], … in order,
 * the lanes meet in hsum8, the tail (len % 8) adds one by one; mean = sum/len; the variance accumulates
 * fmaf(d, d, ·) the same way; inv_std = 1/sqrtf(var + 1e-5); out = fmaf((x − mean)·inv_std, gamma, beta). Each
 * operation rounds once, as written here (built with -ffp-contract=off); the scalar tails (len % 8) take fmaf where the
 * source writes a product then a sum, as a contracting compiler builds them. The reference's -ffast-math x86 build
 * computes 1/sqrtf as vrsqrtss plus a Newton step and may reassociate the tails, so it agrees with this restatement
 * within 1e-6 of the row's rms, not bit for bit. */
void p2o_layer_norm_row(const float *x, const float *gamma, const float *beta, float *out, int len)
{
    const int body = len / 8 * 8;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < body; i += 8)
        for (int j = 0; j < 8; j++) acc[j] = acc[j] + x[i + j];
    float sum = hsum8(acc);
    for (int i = body; i < len; i++) sum += x[i];
    const float mean = sum / (float)len;
    for (int j = 0; j < 8; j++) acc[j] = 0.0f;
    for (int i = 0; i < body; i += 8)
        for (int j = 0; j < 8; j++) {
            const float d = x[i + j] - mean;
            acc[j] = fmaf(d, d, acc[j]);
        }
    float var_sum = hsum8(acc);
    for (int i = body; i < len; i++) {
        const float d = x[i] - mean;
        var_sum = fmaf(d, d, var_sum);
    }
    const float var = var_sum / (float)len;
    const float inv_std = 1.0f / sqrtf(var + 1e-5f);
    for (int i = 0; i < len; i++) out[i] = fmaf((x[i] - mean) * inv_std, gamma[i], beta[i]);
}

/* p2_exp_avx2 (tensor_ops.c:154-175): clamp to ±87, k = round-to-nearest-even(x·log2e), r = x − k·ln2 as one fmaf
 * (the reference's -ffast-math build contracts the source's product and difference the same way), degree-5 Horner in
 * fmaf, times 2^k built in the exponent. */
static float exp_avx2_lane(float x)
{
    x = fminf(fmaxf(x, -87.0f), 87.0f);
    const float kf = rintf(x * 1.44269504088896341f);
    const float r = fmaf(-kf, 0.69314718055994529f, x);
    float y = 1.0f / 120.0f;
    y = fmaf(y, r, 1.0f / 24.0f);
    y = fmaf(y, r, 1.0f / 6.0f);
    y = fmaf(y, r, 0.5f);
    y = fmaf(y, r, 1.0f);
    y = fmaf(y, r, 1.0f);
    union { uint32_t u; float f; } p;
    p.u = (uint32_t)((int32_t)kf + 127) << 23;
    return y * p.f;
}

/* swish_range, AVX2 route (tensor_ops.c:437-463): x · (1 / (1 + exp(−x))) in groups of eight, each operation rounded
 * as written; a tail uses p2_sigmoid (phonon2.h:38-46), expf clamped at 87. The reference's x86 build fuses 1 + y·2^k
 * into one fma and divides by vrcpps plus a Newton step, so its values agree with these within a few ulp. */
void p2o_swish_row(float *x, int len)
{
    const int body = len / 8 * 8;
    for (int i = 0; i < body; i++) {
        const float e = exp_avx2_lane(0.0f - x[i]);
        x[i] = x[i] * (1.0f / (1.0f + e));
    }
    for (int i = body; i < len; i++) x[i] *= 1.0f / (1.0f + expf(x[i] < -87.0f ? 87.0f : -x[i]));
}

/* p2_softmax, AVX2 route (tensor_ops.c:354-413): the maximum (order-free); over the elements below the last
 * multiple of eight, e = exp(x − max) summed into eight running lane sums in order (element j into lane j mod 8),
 * the lanes met as p2_hsum_avx2 pairs them (tensor_ops.c:182-190); the tail with expf added after them in order;
 * then every element times 1/sum. */
static void softmax_row(float *x, int len)
{
    const int body = len / 8 * 8;
    float mx = x[0];
    for (int i = 1; i < len; i++)
        if (x[i] > mx) mx = x[i];
    float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < body; i++) {
        x[i] = exp_avx2_lane(x[i] - mx);
        lane[i & 7] += x[i];
    }
    float sum = ((lane[0] + lane[4]) + (lane[2] + lane[6])) + ((lane[1] + lane[5]) + (lane[3] + lane[7]));
    for (int i = body; i < len; i++) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    const float inv = 1.0f / sum;
    for (int i = 0; i < len; i++) x[i] *= inv;
}

/* combine_softmax (encoder.c:425-450): row r of the [H·T, T] scores, query i = r mod T, reads its bd row from
 * position T − 1 − i (the relative shift); a = (ac + bd) · scale, then the softmax of the row. */
void p2o_combine_softmax(float *ac, const float *bd, int H, int T, float scale)
{
    const int L = 2 * T - 1;
    for (int r = 0; r < H * T; r++) {
        const int i = r % T;
        float *a = ac + (size_t)r * T;
        const float *b = bd + (size_t)r * L + (T - 1 - i);
        for (int j = 0; j < T; j++) a[j] = (a[j] + b[j]) * scale;
        softmax_row(a, T);
    }
}

/* glu_to_channel_major (encoder.c:543-555): gated[d][t] = pw1[t][d] / (1 + p2_expneg(pw1[t][D + d])), p2_expneg
 * clamping the exponent's argument at 87 (phonon2.h:38-41). */
void p2o_glu_channel_major(const float *pw1, float *gated, int T, int D)
{
    for (int t = 0; t < T; t++) {
        const float *row = pw1 + (size_t)t * 2 * D;
        for (int d = 0; d < D; d++) {
            const float g = row[D + d];
            gated[(size_t)d * T + t] = row[d] / (1.0f + expf(g < -87.0f ? 87.0f : -g));
        }
    }
}

/* depthwise_conv1d_channel (tensor_ops.c:559-627): padding (K − 1)/2, per output the bias then one fmaf per tap
 * inside the sequence in order of the tap, as the source's AVX2 body (tensor_ops.c:592-598) computes each of its
 * eight lanes. The source's scalar edges (t < pad, the last (T − 2·pad) mod 8 interior outputs, t ≥ T − pad) write
 * the same chain; an -ffast-math build may reassociate those, so there the reference's values can differ from these
 * in the last bits. */
void p2o_dwconv(const float *x, const float *w, const float *b, float *out, int D, int T, int K)
{
    const int pad = (K - 1) / 2;
    for (int d = 0; d < D; d++) {
        const float *xr = x + (size_t)d * T;
        float *orow = out + (size_t)d * T;
        for (int t = 0; t < T; t++) {
            float v = b[d];
            for (int k = 0; k < K; k++) {
                const int s = t - pad + k;
                if (s >= 0 && s < T) v = fmaf(xr[s], w[(size_t)d * K + k], v);
            }
            orow[t] = v;
        }
    }
}

/* the convolution module's depthwise step and activation (encoder.c:596-597): p2o_dwconv, then p2_swish
 * (tensor_ops.c:481-491) on the channel-major result, whose length D·T is a multiple of 16 at D = 1024, so every
 * element takes the eight-wide body. */
void p2o_dwconv_silu(const float *x, const float *w, const float *b, float *out, int D, int T, int K)
{
    p2o_dwconv(x, w, b, out, D, T, K);
    p2o_swish_row(out, D * T);
}

/* LayerNorm then quantise each row (p2_layer_norm_quant_rows, tensor_ops.c:329-350) */
void p2o_ln_quant_rows(const float *X, int M, int D, int ldx, const float *gamma, const float *beta, int8_t *q,
                       float *scales)
{
    float *row = (float *)malloc((size_t)D * sizeof(float));
    for (int m = 0; m < M; m++) {
        p2o_layer_norm_row(X + (size_t)m * ldx, gamma, beta, row, D);
        quant_row(row, D, q + (size_t)m * D, scales + m);
    }
    free(row);
}

/* SiLU then quantise each row (p2_swish_quant_rows, tensor_ops.c:491-511) */
void p2o_silu_quant_rows(const float *H, int M, int K, int ldh, int8_t *q, float *scales)
{
    float *row = (float *)malloc((size_t)K * sizeof(float));
    for (int m = 0; m < M; m++) {
        memcpy(row, H + (size_t)m * ldh, (size_t)K * sizeof(float));
        p2o_swish_row(row, K);
        quant_row(row, K, q + (size_t)m * K, scales + m);
    }
    free(row);
}

/* Heads [H, T, Dh] → rows [T, H·Dh], then quantise (concat_heads, encoder.c:449-463) */
void p2o_concat_heads_quant_rows(const float *attn_h, int H, int T, int Dh, int8_t *q, float *scales)
{
    const int D = H * Dh;
    float *row = (float *)malloc((size_t)D * sizeof(float));
    for (int t = 0; t < T; t++) {
        for (int h = 0; h < H; h++) memcpy(row + h * Dh, attn_h + ((size_t)h * T + t) * Dh, (size_t)Dh * sizeof(float));
        quant_row(row, D, q + (size_t)t * D, scales + t);
    }
    free(row);
}

/* Channel-major [D, T] → rows [T, D], then quantise (channel_major_to_rows, encoder.c:554-568) */
void p2o_channel_major_quant_rows(const float *dw, int D, int T, int8_t *q, float *scales)
{
    float *row = (float *)malloc((size_t)D * sizeof(float));
    for (int t = 0; t < T; t++) {
        for (int d = 0; d < D; d++) row[d] = dw[(size_t)d * T + t];
        quant_row(row, D, q + (size_t)t * D, scales + t);
    }
    free(row);
}

/* blas.c:1319-1326 */
static inline int clo_of(float lo, float hi)
{
    int c = hi > 0.0f ? (int)lrintf(127.0f * lo / hi) : 0;
    return c < 0 ? 0 : c > 127 ? 127 : c;
}

void p2o_clo(const float *lo, const float *hi, int N, uint8_t *clo)
{
    for (int n = 0; n < N; n++) clo[n] = (uint8_t)clo_of(lo[n], hi[n]);
}

/* blas.c:1193-1205 and 1229-1236: s = code − 1 as int8, t = s & −flag, magnitude 127 where t != 0 else clo, and
 * the code is the int8 product s · magnitude (vmulq_s8 wraps). */
static inline int8_t code_i8w(int code, int flag, int clo)
{
    int s = code - 1;
    int t = flag ? s : 0;
    int mag = t != 0 ? 127 : clo;
    return (int8_t)(uint8_t)((s * mag) & 0xFF);
}

void p2o_codes_i8w(const uint8_t *signs, const uint8_t *flags, const float *lo, const float *hi, int K, int N,
                   int8_t *codes)
{
    for (int k = 0; k < K; k++)
        for (int n = 0; n < N; n++)
            codes[(size_t)k * N + n] = code_i8w(code_at(signs, N, k, n), flag_at(flags, N, k, n),
                                                clo_of(lo[n], hi[n]));
}

/* blas.c:1229-1239 with vst4q_s8: per 16-column panel p, quad kq, column j, row i of the quad → offset
 * ((p·K/4 + kq)·16 + j)·4 + i. */
void p2o_fv_pack_codes(const uint8_t *signs, const uint8_t *flags, const float *lo, const float *hi, int K, int N,
                       int8_t *packed)
{
    for (int p = 0; p < N / 16; p++)
        for (int kq = 0; kq < K / 4; kq++)
            for (int j = 0; j < 16; j++) {
                int n = 16 * p + j;
                int clo = clo_of(lo[n], hi[n]);
                for (int i = 0; i < 4; i++) {
                    int k = 4 * kq + i;
                    packed[(((size_t)p * (K / 4) + kq) * 16 + j) * 4 + i] =
                        code_i8w(code_at(signs, N, k, n), flag_at(flags, N, k, n), clo);
                }
            }
}

/* blas.c:1189-1220 */
void p2o_planes_i8(const uint8_t *signs, const uint8_t *flags, int K, int N, int8_t *S, int8_t *T)
{
    for (int k = 0; k < K; k++)
        for (int n = 0; n < N; n++) {
            int s = code_at(signs, N, k, n) - 1;
            S[(size_t)k * N + n] = (int8_t)s;
            T[(size_t)k * N + n] = (int8_t)(flag_at(flags, N, k, n) ? s : 0);
        }
}

void p2o_acc_i32(const int8_t *q, int M, int K, const int8_t *B, int N, int k0, int k1, int32_t *acc)
{
    /* integer sums are exact, so the order of the k terms is free: a row of accumulators, k outer */
    for (int m = 0; m < M; m++) {
        int32_t *a = acc + (size_t)m * N;
        for (int n = 0; n < N; n++) a[n] = 0;
        for (int k = k0; k < k1; k++) {
            const int32_t qk = q[(size_t)m * K + k];
            const int8_t *b = B + (size_t)k * N;
            for (int n = 0; n < N; n++) a[n] += qk * (int32_t)b[n];
        }
    }
}

/* blas.c:1296-1370. Per K block of 1024 rows: f = (float)accS · c1 (+ fmaf((float)accT, c2, f) with two planes);
 * C = f · as on the storing first block, else C = fmaf(f, as, C); as = a_scale[m] · alpha. */
static void i8_epilogue_run(int two_planes, int M, int N, int K, float alpha, const int8_t *q, const float *a_scales,
                            const int8_t *B1, const int8_t *B2, const float *c1, const float *c2,
                            int beta_zero, float *C, int ldc)
{
    int32_t *accS = (int32_t *)malloc((size_t)M * N * sizeof(int32_t));
    int32_t *accT = two_planes ? (int32_t *)malloc((size_t)M * N * sizeof(int32_t)) : NULL;
    for (int kc = 0; kc < K; kc += KC_I8) {
        int k1 = kc + KC_I8 < K ? kc + KC_I8 : K;
        p2o_acc_i32(q, M, K, B1, N, kc, k1, accS);
        if (two_planes) p2o_acc_i32(q, M, K, B2, N, kc, k1, accT);
        int store = beta_zero && kc == 0;
        for (int m = 0; m < M; m++) {
            float as = a_scales[m] * alpha;
            for (int n = 0; n < N; n++) {
                float f = (float)accS[(size_t)m * N + n] * c1[n];
                if (two_planes) f = fmaf((float)accT[(size_t)m * N + n], c2[n], f);
                float *c = C + (size_t)m * ldc + n;
                *c = store ? f * as : fmaf(f, as, *c);
            }
        }
    }
    free(accS);
    free(accT);
}

void p2o_gemm_i8_run(int mode, int M, int N, int K, float alpha, const int8_t *q, const float *a_scales,
                     const uint8_t *signs, const uint8_t *flags, const float *lo, const float *hi,
                     int beta_zero, float *C, int ldc)
{
    float *c1 = (float *)malloc((size_t)N * sizeof(float));
    float *c2 = (float *)malloc((size_t)N * sizeof(float));
    if (mode == P2O_INT8W) {
        int8_t *codes = (int8_t *)malloc((size_t)K * N);
        p2o_codes_i8w(signs, flags, lo, hi, K, N, codes);
        for (int n = 0; n < N; n++) c1[n] = hi[n] * (1.0f / 127.0f);   /* blas.c:1327-1328 */
        i8_epilogue_run(0, M, N, K, alpha, q, a_scales, codes, NULL, c1, NULL, beta_zero, C, ldc);
        free(codes);
    } else {
        int8_t *S = (int8_t *)malloc((size_t)K * N), *T = (int8_t *)malloc((size_t)K * N);
        p2o_planes_i8(signs, flags, K, N, S, T);
        for (int n = 0; n < N; n++) { c1[n] = lo[n]; c2[n] = hi[n] - lo[n]; }   /* blas.c:1329-1333 */
        i8_epilogue_run(1, M, N, K, alpha, q, a_scales, S, T, c1, c2, beta_zero, C, ldc);
        free(S); free(T);
    }
    free(c1); free(c2);
}

void p2o_gemm_q8b_run(int M, int N, int K, float alpha, const int8_t *q, const float *a_scales,
                      const int8_t *B, int ldb, const float *scales, int beta_zero, float *C, int ldc)
{
    int8_t *Bc = (int8_t *)malloc((size_t)K * N);
    for (int k = 0; k < K; k++) memcpy(Bc + (size_t)k * N, B + (size_t)k * ldb, (size_t)N);
    i8_epilogue_run(0, M, N, K, alpha, q, a_scales, Bc, NULL, scales, NULL, beta_zero, C, ldc);
    free(Bc);
}

/* blas.c:1481-1499 with sgemm_i8 (blas.c:1415-1428) for the int8 modes. */
void p2o_sgemm_fvb(int mode, int M, int N, int K, float alpha, const float *A, int lda,
                   const uint8_t *signs, const uint8_t *flags, const float *lo, const float *hi,
                   float beta, float *C, int ldc)
{
    if (alpha == 0.0f) { scale_c(C, M, N, ldc, beta); return; }
    if (mode != P2O_EXACT && K % 4 == 0) {
        if (beta != 0.0f && beta != 1.0f) scale_c(C, M, N, ldc, beta);
        int8_t *q = (int8_t *)malloc((size_t)M * K);
        float *sc = (float *)malloc((size_t)(M > 0 ? M : 1) * sizeof(float));
        p2o_quant_rows(A, M, K, lda, q, sc);
        p2o_gemm_i8_run(mode, M, N, K, alpha, q, sc, signs, flags, lo, hi, beta == 0.0f, C, ldc);
        free(q); free(sc);
        return;
    }
    p2o_sgemm_fvb_exact(M, N, K, alpha, A, lda, signs, flags, lo, hi, beta, C, ldc);
}

/* blas.c:1448-1460; exact expansion w = (float)q · scale (blas.c:817-827, AVX2). */
void p2o_sgemm_q8b(int mode, int M, int N, int K, float alpha, const float *A, int lda,
                   const int8_t *B, const float *scales, int ldb, float beta, float *C, int ldc)
{
    if (alpha == 0.0f) { scale_c(C, M, N, ldc, beta); return; }
    if (mode != P2O_EXACT && K % 4 == 0) {
        if (beta != 0.0f && beta != 1.0f) scale_c(C, M, N, ldc, beta);
        int8_t *q = (int8_t *)malloc((size_t)M * K);
        float *sc = (float *)malloc((size_t)(M > 0 ? M : 1) * sizeof(float));
        p2o_quant_rows(A, M, K, lda, q, sc);
        p2o_gemm_q8b_run(M, N, K, alpha, q, sc, B, ldb, scales, beta == 0.0f, C, ldc);
        free(q); free(sc);
        return;
    }
    scale_c(C, M, N, ldc, beta);
    float *W = (float *)malloc((size_t)K * N * sizeof(float));
    for (int k = 0; k < K; k++)
        for (int n = 0; n < N; n++) W[(size_t)k * N + n] = (float)B[(size_t)k * ldb + n] * scales[n];
    exact_chain(M, N, K, alpha, A, lda, W, C, ldc);
    free(W);
}

int p2o_mode_from_env(const char *p2_gemm, const char *p2_exact)
{
    int mode = P2O_INT8W;
    if (p2_gemm && strcmp(p2_gemm, "exact") == 0) mode = P2O_EXACT;
    else if (p2_gemm && strcmp(p2_gemm, "int8") == 0) mode = P2O_INT8;
    else if (p2_gemm && strcmp(p2_gemm, "int8w") == 0) mode = P2O_INT8W;
    if (p2_exact && p2_exact[0] && p2_exact[0] != '0') mode = P2O_EXACT;
    return mode;
}
