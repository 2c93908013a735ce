/*  p2hip_kernels.h – gfx950 kernels of the five-value GEMM (included once, by p2hip.hip).
 *
 *  Kernels:
 *    fv_tables      per-column epilogue tables from lo/hi (blas.c:1319-1333)
 *    quant_rows     per-row int8 quantisation of fp32 activations (blas.c:1114-1145)
 *    gemm_i8        the int8 five-value GEMM on int8 MFMA (blas.c:1296-1370): packed planes → int8 codes in LDS,
 *                   v_mfma_i32_16x16x64_i8 with int32 accumulation, fp32 epilogue per 1024-row K block
 *    gemm_exact     the exact route (blas.c:838-987): fp32 panels expanded in LDS, one fmaf chain per output
 *    fv_pack_codes  the reference's pre-packed int8w code layout (blas.c:1372-1400)
 *    scale_c        C = beta · C (blas.c:60-70)
 */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace p2k {

typedef int v4i __attribute__((ext_vector_type(4)));

enum { MODE_INT8 = 0, MODE_EXACT = 1, MODE_INT8W = 2, MODE_Q8B = 3 };
enum { OUT_F32 = 0, OUT_ACC = 1 };

constexpr int kFoldRows = 1024;   /* K rows per fp32 fold of the int32 sums (KC_I8, blas.c:1025) */

/* ── per-column tables ─────────────────────────────────────────────────────────────────────────────────────── */

/* clo[n] = clamp(lrintf(127·lo/hi), 0, 127), 0 when hi <= 0 (blas.c:1319-1326); c1w[n] = hi·(1/127)
 * (blas.c:1327-1328); c2[n] = hi − lo (blas.c:1332). */
__global__ void fv_tables(int N, const float *__restrict__ lo, const float *__restrict__ hi,
                          uint8_t *__restrict__ clo, float *__restrict__ c1w, float *__restrict__ c2)
{
    int n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= N) return;
    float l = lo[n], h = hi[n];
    int c = 0;
    if (h > 0.0f) {
        float r = __builtin_rintf((127.0f * l) / h);
        c = r < 0.0f ? 0 : r > 127.0f ? 127 : (int)r;
    }
    clo[n] = (uint8_t)c;
    c1w[n] = h * (1.0f / 127.0f);
    c2[n] = h - l;
}

/* ── activation quantisation ───────────────────────────────────────────────────────────────────────────────── */

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

/* One wave per row. scale = amax/127 (1 for amax == 0), inv = 1/scale; the first K − K%16 entries become
 * sat8(rint(x·inv)), the tail lrintf(x/scale) clamped to ±127; columns K..kpad−1 of Q are zeroed. K % 4 == 0. */
__global__ __launch_bounds__(256) void quant_rows(int M, int K, int kpad, const float *__restrict__ A, int lda,
                                                  int vec_ok, int8_t *__restrict__ Q, int ldq,
                                                  float *__restrict__ scales)
{
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return;
    const float *row = A + (size_t)m * lda;
    float amax = 0.0f;
    for (int k = 4 * lane; k < K; k += 256) {
        float4 v;
        if (vec_ok) v = *reinterpret_cast<const float4 *>(row + k);
        else v = make_float4(row[k], row[k + 1], row[k + 2], row[k + 3]);
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    amax = wave_max(amax);
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / scale;
    const int k16 = K / 16 * 16;
    int8_t *qrow = Q + (size_t)m * ldq;
    for (int k = 4 * lane; k < kpad; k += 256) {
        uint32_t packed = 0;
        if (k < K) {
            float x[4];
            if (vec_ok) {
                float4 v = *reinterpret_cast<const float4 *>(row + k);
                x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
            } else {
                x[0] = row[k]; x[1] = row[k + 1]; x[2] = row[k + 2]; x[3] = row[k + 3];
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float r;
                if (k + i < k16) {
                    r = __builtin_rintf(x[i] * inv);
                    r = fminf(fmaxf(r, -128.0f), 127.0f);
                } else {
                    r = __builtin_rintf(x[i] / scale);
                    r = fminf(fmaxf(r, -127.0f), 127.0f);
                }
                packed |= ((uint32_t)(int)r & 0xFFu) << (8 * i);
            }
        }
        *reinterpret_cast<uint32_t *>(qrow + k) = packed;
    }
    if (lane == 0) scales[m] = scale;
}

/* ── the int8 GEMM ─────────────────────────────────────────────────────────────────────────────────────────── */

struct GemmArgs {
    int M, N, K;
    float alpha, beta;
    const int8_t *Q; int ldq; const float *a_scales;     /* quantised activations [M][ldq], row scales [M] */
    const uint8_t *signs; const uint8_t *flags;           /* five-value planes [K][N/4], [K][N/8] */
    const uint8_t *clo; const float *c1; const float *c2; /* per-column epilogue tables */
    const int8_t *B8; int ldb;                            /* int8 table [K][ldb] (MODE_Q8B) */
    float *C; int ldc; int c_vec4;                        /* fp32 output; c_vec4: ldc % 4 == 0 and C 16-B aligned */
    int32_t *acc1; int32_t *acc2; int ldacc;              /* OUT_ACC: raw sums */
    int tiles_n;                                          /* column tiles of the grid */
};

/* Tile geometry. Weight columns n play the MFMA "row" role and activation rows m the "column" role, so each lane's
 * four accumulators are four consecutive n of one output row (a 16-byte store). */
constexpr int BN = 128;          /* weight columns per workgroup */
constexpr int BM = 128;          /* activation rows per workgroup */
constexpr int BK = 128;          /* K rows per LDS stage */
constexpr int SB = BK + 16;      /* LDS row pitch in bytes: 9 × 16 B, so 8 consecutive rows hit 8 bank groups */
constexpr int TILE_BYTES = 128 * SB;

/* byte permute: result byte i = byte sel_i of the 8-byte value {hi:lo}, selectors 0-3 from lo, 4-7 from hi */
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel)
{
    return __builtin_amdgcn_perm(hi, lo, sel);
}

/* 4×4 byte transpose: out[q] byte r = in[r] byte q. */
__device__ __forceinline__ void transpose4x4(const uint32_t in[4], uint32_t out[4])
{
    uint32_t u0 = perm(in[1], in[0], 0x05010400u), u1 = perm(in[1], in[0], 0x07030602u);
    uint32_t v0 = perm(in[3], in[2], 0x05010400u), v1 = perm(in[3], in[2], 0x07030602u);
    out[0] = perm(v0, u0, 0x05040100u);
    out[1] = perm(v0, u0, 0x07060302u);
    out[2] = perm(v1, u1, 0x05040100u);
    out[3] = perm(v1, u1, 0x07060302u);
}

/* The code table of one column for the byte permute: selector code | flag << 2 (code = 2-bit sign code, flag = the
 * hi bit). int8w: (code−1)·(flag ? 127 : clo) as an int8 product (blas.c:1229-1236, vmulq_s8 wraps):
 *   lo dword [−clo, 0, clo, (int8)2·clo], hi dword [−127, 0, 127, (int8)254].
 * int8 two-plane: S = code−1 regardless of the flag, T = S where the flag is set (blas.c:1193-1205). */
__device__ __forceinline__ uint32_t i8w_lo_table(uint32_t clo)
{
    return ((0u - clo) & 0xFFu) | (clo << 16) | (((2u * clo) & 0xFFu) << 24);
}
constexpr uint32_t kI8wHiTable = 0xFE7F0081u;
constexpr uint32_t kPlaneS = 0x020100FFu;   /* [−1, 0, 1, 2] */

/* Rows k0..k0+3 (rq-th quad of the stage) × columns 16·cg..16·cg+15 of a five-value tile into the code tile(s):
 * column n, rows 4rq..4rq+3 land as one dword at row n, 16-byte chunk (rq/4) ^ (n/16 mod 8), dword rq mod 4. */
template <int MODE>
__device__ __forceinline__ void store_fv_codes(const uint32_t s[4], const uint32_t f[4], const uint32_t lo_tab[16],
                                               int8_t *tileB, int8_t *tileT, int cg, int rq)
{
    uint32_t X[4];
    transpose4x4(s, X);
    const uint32_t f01 = f[0] | (f[1] << 16), f23 = f[2] | (f[3] << 16);
    const uint32_t Y0 = perm(f23, f01, 0x06040200u), Y1 = perm(f23, f01, 0x07050301u);
    const int chunk = (rq >> 2) ^ (cg & 7);
    int8_t *base = tileB + (size_t)(16 * cg) * SB + chunk * 16 + (rq & 3) * 4;
    int8_t *baseT = tileT + (size_t)(16 * cg) * SB + chunk * 16 + (rq & 3) * 4;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint32_t sgn = (X[j >> 2] >> (2 * (j & 3))) & 0x03030303u;
        const uint32_t flg = ((j < 8 ? Y0 : Y1) >> (j & 7)) & 0x01010101u;
        const uint32_t sel = sgn | (flg << 2);
        if (MODE == MODE_INT8W) {
            *reinterpret_cast<uint32_t *>(base + j * SB) = perm(kI8wHiTable, lo_tab[j], sel);
        } else {
            *reinterpret_cast<uint32_t *>(base + j * SB) = perm(kPlaneS, kPlaneS, sel);
            *reinterpret_cast<uint32_t *>(baseT + j * SB) = perm(kPlaneS, 0u, sel);
        }
    }
}

/* An int8 table tile: rows 4rq..4rq+3, 16 columns from 16-byte row loads, transposed 4×4 per column quad. */
__device__ __forceinline__ void store_q8_codes(const uint4 r[4], int8_t *tileB, int cg, int rq)
{
    const int chunk = (rq >> 2) ^ (cg & 7);
    int8_t *base = tileB + (size_t)(16 * cg) * SB + chunk * 16 + (rq & 3) * 4;
    const uint32_t w[4][4] = {{r[0].x, r[0].y, r[0].z, r[0].w}, {r[1].x, r[1].y, r[1].z, r[1].w},
                              {r[2].x, r[2].y, r[2].z, r[2].w}, {r[3].x, r[3].y, r[3].z, r[3].w}};
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint32_t in[4] = {w[0][q], w[1][q], w[2][q], w[3][q]};
        uint32_t out[4];
        transpose4x4(in, out);
#pragma unroll
        for (int c = 0; c < 4; c++) *reinterpret_cast<uint32_t *>(base + (4 * q + c) * SB) = out[c];
    }
}

/* 256 threads, 4 waves as 2 (n) × 2 (m); each wave owns a 64 n × 64 m block: 4 × 4 MFMA tiles of 16 × 16.
 * Stage loop: global loads of stage t+1 are issued before the MFMAs of stage t and stored to the other LDS buffer
 * after them, one barrier per stage. MULTI (K > 1024) keeps an fp32 running sum per output across the 1024-row
 * folds; with K <= 1024 the single fold stores straight to C. */
template <int MODE, int OUT, bool MULTI>
__global__ __launch_bounds__(256, ((MODE == MODE_INT8 || MULTI) ? 1 : 2)) void gemm_i8(GemmArgs g)
{
    constexpr bool TWO = (MODE == MODE_INT8);
    __shared__ __attribute__((aligned(16))) int8_t sm[(TWO ? 6 : 4) * TILE_BYTES];
    /* LDS: activation tiles [2], code tiles [2], and the T-plane code tiles [2] of the two-plane mode */
    auto smA = [&](int b) { return sm + b * TILE_BYTES; };
    auto smB = [&](int b) { return sm + (2 + b) * TILE_BYTES; };
    auto smT = [&](int b) { return sm + ((TWO ? 4 : 2) + b) * TILE_BYTES; };

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wn = wave & 1, wm = wave >> 1;
    const int tile_n = blockIdx.x % g.tiles_n, tile_m = blockIdx.x / g.tiles_n;
    const int n0 = tile_n * BN, m0 = tile_m * BM;
    const int M = g.M, N = g.N, K = g.K;
    const int nk = (K + BK - 1) / BK;

    /* producer roles */
    const int cg = tid & 7, rq = tid >> 3;          /* B: 16-column group, 4-row quad */
    const bool col_ok = n0 + 16 * cg < N;
    const int a_chunk = tid & 7, a_row = tid >> 3;  /* A: 16-byte chunk, rows a_row + 32 i */

    uint32_t lo_tab[16];
    if (MODE == MODE_INT8W) {
#pragma unroll
        for (int j = 0; j < 16; j++) lo_tab[j] = col_ok ? i8w_lo_table(g.clo[n0 + 16 * cg + j]) : 0u;
    }

    uint4 ra[4];
    uint32_t rs[4], rf[4];
    uint4 rb[4];

    auto load_stage = [&](int t) {
        const int k0 = t * BK;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = m0 + a_row + 32 * i;
            ra[i] = m < M ? *reinterpret_cast<const uint4 *>(g.Q + (size_t)m * g.ldq + k0 + 16 * a_chunk)
                          : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int k = k0 + 4 * rq + r;
            const bool ok = col_ok && k < K;
            if (MODE == MODE_Q8B) {
                rb[r] = ok ? *reinterpret_cast<const uint4 *>(g.B8 + (size_t)k * g.ldb + n0 + 16 * cg)
                           : make_uint4(0, 0, 0, 0);
            } else {
                rs[r] = ok ? *reinterpret_cast<const uint32_t *>(g.signs + (size_t)k * (N / 4) + n0 / 4 + 4 * cg)
                           : 0x55555555u;   /* code 1 everywhere: zero weights */
                rf[r] = ok ? *reinterpret_cast<const uint16_t *>(g.flags + (size_t)k * (N / 8) + n0 / 8 + 2 * cg)
                           : 0u;
            }
        }
    };
    auto store_stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            *reinterpret_cast<uint4 *>(smA(buf) + (a_row + 32 * i) * SB + 16 * a_chunk) = ra[i];
        if (MODE == MODE_Q8B) store_q8_codes(rb, smB(buf), cg, rq);
        else store_fv_codes<MODE>(rs, rf, lo_tab, smB(buf), smT(buf), cg, rq);
    };

    v4i acc[4][4], accT[4][4];
    float run[MULTI ? 4 : 1][MULTI ? 4 : 1][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            acc[i][j] = v4i{0, 0, 0, 0};
            if (TWO) accT[i][j] = v4i{0, 0, 0, 0};
        }

    /* epilogue geometry of this lane: outputs (m_lane + 16 j, n_lane + 16 i + r) */
    const int n_lane = n0 + wn * 64 + 4 * (lane >> 4);
    const int m_lane = m0 + wm * 64 + (lane & 15);
    const bool beta_zero = g.beta == 0.0f;

    /* Fold the int32 sums of one K block into the fp32 result (blas.c:1355-1366): f = (float)acc · c1
     * (+ fmaf((float)accT, c2, f)); block 0 stores f · as (beta == 0) or fmaf(f, as, beta-scaled C), later blocks
     * fmaf(f, as, running). The last fold stores C. */
    auto fold = [&](int block, bool last) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = n_lane + 16 * i;
            const bool n_ok = n < N;
            float c1v[4] = {0, 0, 0, 0}, c2v[4] = {0, 0, 0, 0};
            if (n_ok) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    c1v[r] = g.c1[n + r];
                    if (TWO) c2v[r] = g.c2[n + r];
                }
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int m = m_lane + 16 * j;
                const bool ok = n_ok && m < M;
                const float as = m < M ? g.a_scales[m] * g.alpha : 0.0f;
                float *cp = g.C + (size_t)m * g.ldc + n;
                float cold[4] = {0, 0, 0, 0};
                if (block == 0 && !beta_zero && ok) {
                    if (g.c_vec4) {
                        float4 v = *reinterpret_cast<const float4 *>(cp);
                        cold[0] = v.x; cold[1] = v.y; cold[2] = v.z; cold[3] = v.w;
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; r++) cold[r] = cp[r];
                    }
                    if (g.beta != 1.0f) {
#pragma unroll
                        for (int r = 0; r < 4; r++) cold[r] = cold[r] * g.beta;
                    }
                }
                float out[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float f = (float)acc[i][j][r] * c1v[r];
                    if (TWO) f = __builtin_fmaf((float)accT[i][j][r], c2v[r], f);
                    float prev = cold[r];
                    if (MULTI && block > 0) prev = run[MULTI ? i : 0][MULTI ? j : 0][r];
                    out[r] = (block == 0 && beta_zero) ? f * as : __builtin_fmaf(f, as, prev);
                    if (MULTI) run[MULTI ? i : 0][MULTI ? j : 0][r] = out[r];
                }
                acc[i][j] = v4i{0, 0, 0, 0};
                if (TWO) accT[i][j] = v4i{0, 0, 0, 0};
                if (last && ok) {
                    if (g.c_vec4) {
                        *reinterpret_cast<float4 *>(cp) = make_float4(out[0], out[1], out[2], out[3]);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; r++) cp[r] = out[r];
                    }
                }
            }
        }
    };

    if (nk > 0) {
        load_stage(0);
        store_stage(0);
    }
    __syncthreads();

    int block = 0;
    for (int t = 0; t < nk; t++) {
        const int buf = t & 1;
        if (t + 1 < nk) load_stage(t + 1);
        const int8_t *tA = smA(buf), *tB = smB(buf), *tT = smT(buf);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 64) {
            const int g16 = (kk >> 4) + (lane >> 4);   /* this lane's 16-byte chunk along k */
            v4i a[4], b[4], bt[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int nl = wn * 64 + 16 * i + (lane & 15);
                const int off = nl * SB + 16 * (g16 ^ ((nl >> 4) & 7));
                a[i] = *reinterpret_cast<const v4i *>(tB + off);
                if (TWO) bt[i] = *reinterpret_cast<const v4i *>(tT + off);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int ml = wm * 64 + 16 * j + (lane & 15);
                b[j] = *reinterpret_cast<const v4i *>(tA + ml * SB + 16 * g16);
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
                    if (TWO) accT[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bt[i], b[j], accT[i][j], 0, 0, 0);
                }
        }
        if (t + 1 < nk) store_stage(buf ^ 1);
        if (OUT == OUT_F32) {
            const bool last = t + 1 == nk;
            if (MULTI) {
                if (((t + 1) * BK) % kFoldRows == 0 || last) fold(block++, last);
            } else if (last) {
                fold(0, true);
            }
        }
        __syncthreads();
    }

    if (OUT == OUT_ACC) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int n = n_lane + 16 * i, m = m_lane + 16 * j;
                if (m < M && n < N) {
                    *reinterpret_cast<v4i *>(g.acc1 + (size_t)m * g.ldacc + n) = acc[i][j];
                    if (TWO) *reinterpret_cast<v4i *>(g.acc2 + (size_t)m * g.ldacc + n) = accT[i][j];
                }
            }
    }
}

/* ── the exact route ───────────────────────────────────────────────────────────────────────────────────────── */

struct ExactArgs {
    int M, N, K;
    float alpha, beta;
    const float *A; int lda; int a_vec4;                  /* a_vec4: lda % 4 == 0 and A 16-B aligned */
    const uint8_t *signs; const uint8_t *flags; const float *lo; const float *hi;   /* five-value */
    const int8_t *B8; int ldb; const float *bscales;      /* int8 table */
    const float *Bf; int ldbf; int transA, transB;        /* plain fp32 B (p2_sgemm) */
    float *C; int ldc;
    int tiles_n;
};

constexpr int EBM = 64, EBN = 64, EBK = 32;

enum { EXB_FV = 0, EXB_Q8 = 1, EXB_F32 = 2 };

/* 256 threads; thread (tm, tn) owns rows 4tm..4tm+3 and columns 4tn..4tn+3 of a 64 × 64 tile. The B panel is
 * expanded to fp32 in LDS as blas.c:877-897 expands it (w = (code−1) · fmaf(flag, hi − lo, lo)), A enters LDS as
 * alpha·A (one fp32 product, as the micro-kernel forms it), and every output runs c = fmaf(alpha·A[m][k], w, c)
 * for k = 0..K−1 in order: the reference's exact kernel, bit for bit. */
template <int BKIND>
__global__ __launch_bounds__(256) void gemm_exact(ExactArgs g)
{
    __shared__ float sA[2][EBK][EBM + 1];
    __shared__ __attribute__((aligned(16))) float sW[2][EBK][EBN];

    const int tid = threadIdx.x;
    const int tn = tid & 15, tm = tid >> 4;
    const int tile_n = blockIdx.x % g.tiles_n, tile_m = blockIdx.x / g.tiles_n;
    const int n0 = tile_n * EBN, m0 = tile_m * EBM;
    const int M = g.M, N = g.N, K = g.K;

    /* A producer: row am, k offsets ak..ak+7 */
    const int am = tid >> 2, ak = (tid & 3) * 8;
    /* W producer: row wk, columns wn..wn+7 */
    const int wk = tid >> 3, wn = (tid & 7) * 8;
    const bool wcol_ok = n0 + wn < N;

    float wlo[8], wd[8];
    if (BKIND == EXB_FV || BKIND == EXB_Q8) {
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const int n = n0 + wn + c;
            const bool ok = n < N;
            if (BKIND == EXB_FV) {
                wlo[c] = ok ? g.lo[n] : 0.0f;
                wd[c] = ok ? g.hi[n] - wlo[c] : 0.0f;
            } else {
                wlo[c] = ok ? g.bscales[n] : 0.0f;
                wd[c] = 0.0f;
            }
        }
    }

    float ra[8], rw[8];
    auto load_stage = [&](int k0) {
        const int m = m0 + am;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const int k = k0 + ak + c;
            float v = 0.0f;
            if (m < M && k < K) v = g.transA ? g.A[(size_t)k * g.lda + m] : g.A[(size_t)m * g.lda + k];
            ra[c] = g.alpha * v;
        }
        const int k = k0 + wk;
        if (BKIND == EXB_FV) {
            uint32_t s = 0x5555u, f = 0;
            if (wcol_ok && k < K) {
                s = *reinterpret_cast<const uint16_t *>(g.signs + (size_t)k * (N / 4) + (n0 + wn) / 4);
                f = g.flags[(size_t)k * (N / 8) + (n0 + wn) / 8];
            }
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const int code = (s >> (2 * c)) & 3, fl = (f >> c) & 1;
                rw[c] = (float)(code - 1) * __builtin_fmaf((float)fl, wd[c], wlo[c]);
            }
        } else if (BKIND == EXB_Q8) {
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const int8_t q = (wcol_ok && k < K) ? g.B8[(size_t)k * g.ldb + n0 + wn + c] : (int8_t)0;
                rw[c] = (float)q * wlo[c];
            }
        } else {
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const int n = n0 + wn + c;
                float v = 0.0f;
                if (n < N && k < K) v = g.transB ? g.Bf[(size_t)n * g.ldbf + k] : g.Bf[(size_t)k * g.ldbf + n];
                rw[c] = v;
            }
        }
    };
    auto store_stage = [&](int buf) {
#pragma unroll
        for (int c = 0; c < 8; c++) sA[buf][ak + c][am] = ra[c];
        *reinterpret_cast<float4 *>(&sW[buf][wk][wn]) = make_float4(rw[0], rw[1], rw[2], rw[3]);
        *reinterpret_cast<float4 *>(&sW[buf][wk][wn + 4]) = make_float4(rw[4], rw[5], rw[6], rw[7]);
    };

    float c[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int m = m0 + 4 * tm + i;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int n = n0 + 4 * tn + j;
            float v = 0.0f;
            if (g.beta != 0.0f && m < M && n < N) {
                v = g.C[(size_t)m * g.ldc + n];
                if (g.beta != 1.0f) v = v * g.beta;
            }
            c[i][j] = v;
        }
    }

    const int nk = (K + EBK - 1) / EBK;
    if (nk > 0) {
        load_stage(0);
        store_stage(0);
    }
    __syncthreads();
    for (int t = 0; t < nk; t++) {
        const int buf = t & 1;
        if (t + 1 < nk) load_stage((t + 1) * EBK);
        const int kcount = min(EBK, K - t * EBK);
        for (int kk = 0; kk < kcount; kk++) {
            float a[4], w[4];
#pragma unroll
            for (int i = 0; i < 4; i++) a[i] = sA[buf][kk][4 * tm + i];
            const float4 wv = *reinterpret_cast<const float4 *>(&sW[buf][kk][4 * tn]);
            w[0] = wv.x; w[1] = wv.y; w[2] = wv.z; w[3] = wv.w;
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) c[i][j] = __builtin_fmaf(a[i], w[j], c[i][j]);
        }
        if (t + 1 < nk) store_stage(buf ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int m = m0 + 4 * tm + i;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int n = n0 + 4 * tn + j;
            if (m < M && n < N) g.C[(size_t)m * g.ldc + n] = c[i][j];
        }
    }
}

/* ── small kernels ─────────────────────────────────────────────────────────────────────────────────────────── */

/* One thread per (panel p, quad kq, column j): the dword of rows 4kq..4kq+3 at
 * out[((p·K/4 + kq)·16 + j)·4 ..] (vst4q_s8 order, blas.c:1229-1239). */
__global__ void fv_pack_codes(int K, int N, const uint8_t *__restrict__ signs, const uint8_t *__restrict__ flags,
                              const uint8_t *__restrict__ clo, uint32_t *__restrict__ out)
{
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)(N / 16) * (K / 4) * 16;
    if (idx >= total) return;
    const int j = (int)(idx % 16);
    const size_t pk = idx / 16;
    const int kq = (int)(pk % (K / 4));
    const int p = (int)(pk / (K / 4));
    const int n = 16 * p + j;
    const int cl = clo[n];
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int k = 4 * kq + i;
        const int code = (signs[(size_t)k * (N / 4) + (n >> 2)] >> (2 * (n & 3))) & 3;
        const int flag = (flags[(size_t)k * (N / 8) + (n >> 3)] >> (n & 7)) & 1;
        const int s = code - 1;
        const int mag = (flag && s != 0) ? 127 : cl;
        word |= ((uint32_t)(s * mag) & 0xFFu) << (8 * i);
    }
    out[idx] = word;
}

__global__ void scale_c(int M, int N, float beta, float *__restrict__ C, int ldc)
{
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)M * N) return;
    const int m = (int)(idx / N), n = (int)(idx % N);
    float *c = C + (size_t)m * ldc + n;
    *c = beta == 0.0f ? 0.0f : *c * beta;
}

}  // namespace p2k
