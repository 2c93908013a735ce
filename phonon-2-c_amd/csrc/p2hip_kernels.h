/*  p2hip_kernels.h – gfx950 kernels of the five-value GEMM (included once, by p2hip.hip).
 *
 *  Kernels:
 *    fv_tables      per-column epilogue tables from lo/hi (blas.c:1319-1333)
 *    quant_rows     per-row int8 quantisation of fp32 activations (blas.c:1114-1145)
 *    gemm_i8        the int8 five-value GEMM on int8 MFMA (blas.c:1296-1370): packed planes → int8 codes in LDS,
 *                   v_mfma_i32_16x16x64_i8 with int32 accumulation, fp32 epilogue per 1024-row K block
 *    gemm_fvs       the same for small M: operands streamed from global memory into registers, K split
 *                   across the waves of a workgroup, partial sums combined and folded through LDS
 *    gemm_exact     the exact route (blas.c:838-987): fp32 panels expanded in LDS, one fmaf chain per output
 *    fv_pack_codes  the reference's pre-packed int8w code layout (blas.c:1372-1400)
 *    fv_repack4     the planes re-laid per matrix-core operand (4 bits per weight) at upload
 *    scale_c        C = beta · C (blas.c:60-70)
 */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace p2k {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

enum { MODE_INT8 = 0, MODE_EXACT = 1, MODE_INT8W = 2, MODE_Q8B = 3 };
enum { OUT_F32 = 0, OUT_ACC = 1 };

constexpr int kFoldRows = 1024;   /* K rows per fp32 fold of the int32 sums (KC_I8, blas.c:1025) */
constexpr int kStoreSc1 = 16;     /* buffer store cache policy: sc1, device scope */
typedef unsigned v4u __attribute__((ext_vector_type(4)));

/* 16-byte stores at device scope (sc1) into one output of at most 2 GB. A plain store leaves its line dirty in the
 * XCD's L2, and the end of the kernel writes every dirty line back before the launch completes: about 2.8 µs once
 * 25 MB or more of output sit there, at M = 1500 as at M = 6000. Stores at device scope go through the L2 as they
 * are made. The scope travels on a buffer store, over a resource whose base must be the same for the whole wave
 * (32-bit byte offsets from it); `on` false, or an output over 2 GB, stores plainly. Only for whole row segments:
 * the quantised rows' 16-byte pieces, scattered over the operand layout, write through at a fraction of the rate
 * (quant_rows at M = 6000, K = 4096: 32.2 against 21.5 µs plainly). */
struct DevScopeOut {
    __amdgpu_buffer_rsrc_t r;
    char *base;
    bool on;
    __device__ __forceinline__ DevScopeOut(void *base_, size_t bytes, bool want)
        : base(static_cast<char *>(base_)), on(want && bytes <= 0x7fffffff)
    {
        r = __builtin_amdgcn_make_buffer_rsrc(base_, 0, on ? (int)bytes : 0, 0x00020000);
    }
    /* The whole offset is kept in the VGPR operand (soffset 0): a buffer store whose offset the compiler had split
     * into an SGPR soffset missed its store-data hazard wait on gfx950 and wrote the next store's data. */
    template <class V>
    __device__ __forceinline__ void st16(size_t off, V v) const
    {
        static_assert(sizeof(V) == 16, "16-byte stores");
        if (on) {
            int o = (int)off;
            asm volatile("" : "+v"(o));
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v), r, o, 0, kStoreSc1);
        } else {
            *reinterpret_cast<V *>(base + off) = v;
        }
    }
};

/* Quantised activations are stored tiled for the MFMA operand: per 16-row group and 64-column step one 1 KB block,
 * in which operand lane l (row l % 16, columns 16·(l / 16) .. +15) holds 16 consecutive bytes. Rows are padded to a
 * multiple of 16 and columns to ldq (a multiple of 128) with zeros. kst = ldq / 64. */
__host__ __device__ __forceinline__ size_t q_index(int m, int k, int kst)
{
    return ((size_t)(m >> 4) * kst + (k >> 6)) * 1024 + (size_t)(((((k >> 4) & 3) << 4) + (m & 15)) * 16) + (k & 15);
}

/* byte permute: result byte i = byte sel_i of the 8-byte value {hi:lo}, selectors 0-3 from lo, 4-7 from hi */
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel)
{
    return __builtin_amdgcn_perm(hi, lo, sel);
}

/* ── per-column tables ─────────────────────────────────────────────────────────────────────────────────────── */

/* clo[n] = clamp(lrintf(127·lo/hi), 0, 127), 0 when hi <= 0 (blas.c:1319-1326). The fold's other factors,
 * hi·(1/127) and hi − lo (blas.c:1327-1333), are made from lo and hi where they are used (c1_factor, c2_factor). */
__global__ void fv_tables(int N, const float *__restrict__ lo, const float *__restrict__ hi, uint8_t *__restrict__ clo)
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
}

/* ── activation quantisation ───────────────────────────────────────────────────────────────────────────────── */


/* Maximum over the wave: DPP within each row of 16 lanes, then the four row results. */
__device__ __forceinline__ float wave_max_dpp(float v)
{
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));  /* [1,0,3,2] */
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));  /* [2,3,0,1] */
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false))); /* half mirror */
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false))); /* mirror */
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

/* four int32 values in [-128, 127] → their low bytes packed little-endian */
__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d)
{
    const uint32_t lo = perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u), hi = perm((uint32_t)d, (uint32_t)c, 0x0c0c0400u);
    return perm(hi, lo, 0x05040100u);
}

/* 16 columns k0..k0+15 of one row (values x) into 16 bytes (blas.c:1114-1145): columns below k16 = K − K%16
 * become sat8(rint(x·inv)), the tail rint(x/scale) clamped to ±127, columns at or beyond K zero. */
__device__ __forceinline__ uint4 quant16(const float x[16], int k0, int K, int k16, float scale, float inv)
{
    int q[16];
    if (k0 + 16 <= k16) {
#pragma unroll
        for (int e = 0; e < 16; e++) q[e] = (int)__builtin_amdgcn_fmed3f(__builtin_rintf(x[e] * inv), -128.0f, 127.0f);
    } else {
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int k = k0 + e;
            const float body = __builtin_amdgcn_fmed3f(__builtin_rintf(x[e] * inv), -128.0f, 127.0f);
            const float tail = __builtin_amdgcn_fmed3f(__builtin_rintf(x[e] / scale), -127.0f, 127.0f);
            q[e] = (int)(k < k16 ? body : k < K ? tail : 0.0f);
        }
    }
    return make_uint4(pack4(q[0], q[1], q[2], q[3]), pack4(q[4], q[5], q[6], q[7]), pack4(q[8], q[9], q[10], q[11]),
                      pack4(q[12], q[13], q[14], q[15]));
}

/* 16 columns k0..k0+15 of a row, zeros at and beyond K (K % 4 == 0); every load is issued, out-of-range ones at
 * column 0 */
template <bool VEC>
__device__ __forceinline__ void load16(const float *__restrict__ row, int k0, int K, float x[16])
{
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int k = k0 + 4 * q;
        const bool ok = k < K;
        const int kk = ok ? k : 0;
        float4 v;
        if (VEC) v = *reinterpret_cast<const float4 *>(row + kk);
        else v = make_float4(row[kk], row[kk + 1], row[kk + 2], row[kk + 3]);
        x[4 * q] = ok ? v.x : 0.0f;
        x[4 * q + 1] = ok ? v.y : 0.0f;
        x[4 * q + 2] = ok ? v.z : 0.0f;
        x[4 * q + 3] = ok ? v.w : 0.0f;
    }
}

/* One wave per row of the padded row range, into the tiled layout (q_index). Lane l owns the 16-column chunks
 * 16·(l + 64c); with NCH > 0 the row (ldq <= 1024·NCH) stays in registers between the row maximum and the
 * quantisation, with NCH == 0 it is read twice. scale = amax/127 (1 for amax == 0), inv = 1/scale. Rows M..Mp−1 and
 * columns K..ldq−1 are written as zeros. VEC: lda % 4 == 0 and A 16-byte aligned. */
template <int NCH, bool VEC, int RPW = 4>
__global__ __launch_bounds__(64 * RPW) void quant_rows(int M, int Mp, int K, const float *__restrict__ A, int lda,
                                                       int8_t *__restrict__ Q, int ldq, float *__restrict__ scales)
{
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * RPW + (threadIdx.x >> 6);   /* RPW rows per workgroup of RPW waves */
    if (m >= Mp) return;
    const int kst = ldq / 64, k16 = K / 16 * 16;
    if (m >= M) {
        for (int k0 = 16 * lane; k0 < ldq; k0 += 1024)
            *reinterpret_cast<uint4 *>(Q + q_index(m, k0, kst)) = make_uint4(0u, 0u, 0u, 0u);
        return;
    }
    const float *row = A + (size_t)m * lda;
    if (NCH > 0) {
        float x[NCH > 0 ? NCH : 1][16];
        float amax = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            load16<VEC>(row, 16 * (lane + 64 * c), K, x[c]);
#pragma unroll
            for (int e = 0; e < 16; e++) amax = fmaxf(amax, fabsf(x[c][e]));
        }
        amax = wave_max_dpp(amax);
        const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / scale;
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            const int k0 = 16 * (lane + 64 * c);
            if (k0 < ldq) *reinterpret_cast<uint4 *>(Q + q_index(m, k0, kst)) = quant16(x[c], k0, K, k16, scale, inv);
        }
        if (lane == 0) scales[m] = scale;
        return;
    }
    float amax = 0.0f;
    for (int k0 = 16 * lane; k0 < K; k0 += 1024) {
        float x[16];
        load16<VEC>(row, k0, K, x);
#pragma unroll
        for (int e = 0; e < 16; e++) amax = fmaxf(amax, fabsf(x[e]));
    }
    amax = wave_max_dpp(amax);
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / scale;
    for (int k0 = 16 * lane; k0 < ldq; k0 += 1024) {
        float x[16];
        load16<VEC>(row, k0, K, x);
        *reinterpret_cast<uint4 *>(Q + q_index(m, k0, kst)) = quant16(x, k0, K, k16, scale, inv);
    }
    if (lane == 0) scales[m] = scale;
}

/* quant_rows with a workgroup of four waves per row, for a few long rows: each lane holds 16 · NCH values of
 * K ≤ 4096·NCH (four times fewer than one wave per row would), the waves' maxima meet in LDS. The maximum is exact
 * in any order, so the bits are quant_rows' own. */
template <int NCH, bool VEC>
__global__ __launch_bounds__(256) void quant_rows_w4(int M, int Mp, int K, const float *__restrict__ A, int lda,
                                                     int8_t *__restrict__ Q, int ldq, float *__restrict__ scales)
{
    __shared__ float wmax[4];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int m = blockIdx.x;
    if (m >= Mp) return;
    const int kst = ldq / 64, k16 = K / 16 * 16;
    if (m >= M) {
        for (int k0 = 16 * t; k0 < ldq; k0 += 4096)
            *reinterpret_cast<uint4 *>(Q + q_index(m, k0, kst)) = make_uint4(0u, 0u, 0u, 0u);
        return;
    }
    const float *row = A + (size_t)m * lda;
    float x[NCH][16];
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        load16<VEC>(row, 16 * (t + 256 * c), K, x[c]);
#pragma unroll
        for (int e = 0; e < 16; e++) amax = fmaxf(amax, fabsf(x[c][e]));
    }
    amax = wave_max_dpp(amax);
    if (lane == 0) wmax[w] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / scale;
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int k0 = 16 * (t + 256 * c);
        if (k0 < ldq) *reinterpret_cast<uint4 *>(Q + q_index(m, k0, kst)) = quant16(x[c], k0, K, k16, scale, inv);
    }
    if (t == 0) scales[m] = scale;
}

/* ── producers: make a quantised linear's input rows and quantise them in one pass ────────────────────────────── */

enum { PROD_SILU = 1, PROD_HEADS = 2, PROD_CMAJOR = 3, PROD_LN = 4 };

struct ProdArgs {
    int M, Mp, K;
    const float *X; int ldx;                  /* SILU, LN: rows [M][ldx]; HEADS: [H][T][Dh]; CMAJOR: [K][T] */
    int T, Dh;
    const float *gamma, *beta;                /* LN */
    int8_t *Q; int ldq; float *scales;
    float *Y; int ldy;                        /* when set: the made rows as fp32 [M][ldy] instead of quantised rows */
    const float *gamma2, *beta2;              /* LN2: the second LayerNorm's factors; the first one's rows go out */
    float *Y1; int ldy1;                      /* as fp32 [M][ldy1] (in place over X allowed) */
};

/* e^x as the reference's AVX2 exp (tensor_ops.c:154-175) in IEEE operations: clamp to ±87, k = rint(x·log2e),
 * r = fmaf(−k, ln2, x), degree-5 Horner in fmaf, times 2^k assembled in the exponent field. */
__device__ __forceinline__ float exp_p2(float x)
{
    x = fminf(fmaxf(x, -87.0f), 87.0f);
    const float kf = __builtin_rintf(__fmul_rn(x, 1.44269504088896341f));
    const float r = __builtin_fmaf(-kf, 0.69314718055994529f, x);
    float y = 1.0f / 120.0f;
    y = __builtin_fmaf(y, r, 1.0f / 24.0f);
    y = __builtin_fmaf(y, r, 1.0f / 6.0f);
    y = __builtin_fmaf(y, r, 0.5f);
    y = __builtin_fmaf(y, r, 1.0f);
    y = __builtin_fmaf(y, r, 1.0f);
    return __fmul_rn(y, __uint_as_float((uint32_t)((int)kf + 127) << 23));
}

/* 1/d correctly rounded for d in [1, 2^126): the hardware reciprocal (within 1 ulp) and one Newton step in fmaf.
 * recip_check compares it with the IEEE quotient for every float of that range (1,056,964,608 values, none differ on
 * gfx950; p2h_recip_selftest runs it). */
__device__ __forceinline__ float recip_ge1(float d)
{
    const float r = __builtin_amdgcn_rcpf(d);
    return __builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r);
}

/* x · sigmoid(x) = x · (1 / (1 + e^{−x})) (swish_range, tensor_ops.c:437-463), no operation contracted. exp_p2 clamps
 * its argument to ±87, so 1 + e^{−x} lies in [1, 0.72·2^126] and recip_ge1 gives the IEEE quotient. */
__device__ __forceinline__ float silu_p2(float x)
{
    return __fmul_rn(x, recip_ge1(__fadd_rn(1.0f, exp_p2(0.0f - x))));
}

/* Every float bit pattern b in [lo, hi): out[0] += how many recip_ge1 gets wrong against the IEEE quotient,
 * out[1] = the smallest such pattern (min), out[2] += how many were checked. */
__global__ void recip_check(uint32_t lo, uint32_t hi, unsigned long long *out)
{
    unsigned long long bad = 0, n = 0;
    for (uint64_t b = lo + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; b < hi;
         b += (uint64_t)gridDim.x * blockDim.x) {
        const float d = __uint_as_float((uint32_t)b);
        n++;
        if (__float_as_uint(recip_ge1(d)) != __float_as_uint(__fdiv_rn(1.0f, d))) {
            bad++;
            atomicMin(&out[1], (unsigned long long)b);
        }
    }
    atomicAdd(&out[0], bad);
    atomicAdd(&out[2], n);
}

/* One wave per row of the padded row range (WPR = 4: a workgroup of four waves per row, for few long rows), the
 * quantised row into the tiled layout as quant_rows does; the row is made on the way in:
 *   PROD_SILU    SiLU of row m of X (p2_swish_quant_rows, tensor_ops.c:491-511; K % 8 == 0)
 *   PROD_HEADS   row t of the head concatenation: element k = h·Dh + d is X[h][t][d] (encoder.c:449-463)
 *   PROD_CMAJOR  row t of the transpose of the channel-major X [K][T] (encoder.c:554-568)
 *   PROD_LN      LayerNorm of row m (p2_layer_norm_quant_rows, tensor_ops.c:204-268, 329-350): eight running sums,
 *                lane j adding elements j, j + 8, … in order, meet as p2_hsum_avx2 does (v[i] + v[i+4], then pairs);
 *                the same for fmaf(d, d, ·) with d = x − mean; inv_std = 1/sqrtf(var + 1e-5), square root and
 *                quotient correctly rounded (__builtin_sqrtf; the v_sqrt_f32 behind __fsqrt_rn is not);
 *                y = fmaf((x − mean)·inv_std, gamma, beta). The row is staged in LDS for the eight sums.
 * NCH chunks of 16 columns per lane (ldq <= 1024·WPR·NCH). LNR: LayerNorm's sums from registers (below). VEC: rows read as float4 — SILU / LN with K % 4 == 0,
 * ldx % 4 == 0 (LN: gamma and beta 16-byte aligned too); HEADS with Dh % 16 == 0; X 16-byte aligned. */
template <int KIND, int NCH, bool VEC, int WPR = 1, bool LNR = false, bool LN2 = false>
__global__ __launch_bounds__(256) void produce_rows(ProdArgs a)
{
    static_assert(WPR == 1 || (WPR == 4 && KIND != PROD_LN), "LayerNorm keeps one wave per row");
    __shared__ __align__(16) float stage[KIND == PROD_LN ? 4 * 8 * (128 * NCH + 20) : 1];
    __shared__ float wmax[4];
    constexpr int STRIDE = 64 * WPR;                       /* lanes per row */
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int m = blockIdx.x * (4 / WPR) + w / WPR;         /* with four waves per row, the workgroup's row */
    const int lr = (w % WPR) * 64 + lane;                   /* the thread's place among its row's lanes */
    if (m >= a.Mp) return;
    const int K = a.K, kst = a.ldq / 64, k16 = K / 16 * 16;
    if (m >= a.M) {
        if (a.Y) return;
        for (int k0 = 16 * lr; k0 < a.ldq; k0 += 16 * STRIDE)
            *reinterpret_cast<uint4 *>(a.Q + q_index(m, k0, kst)) = make_uint4(0u, 0u, 0u, 0u);
        return;
    }
    float x[NCH][16];
    /* the made row as fp32: 16-byte stores of the lane's 16 columns where the row is aligned and the chunk whole
     * (each store instruction then writes whole 128-byte lines), else one value at a time */
    auto store_row = [&](float *yr, const float (&v)[NCH][16]) __attribute__((always_inline)) {
        const bool al = (reinterpret_cast<uintptr_t>(yr) & 15) == 0;
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            const int k0 = 16 * (lr + STRIDE * c);
            if (al && k0 + 16 <= K) {
#pragma unroll
                for (int u = 0; u < 4; u++)
                    *reinterpret_cast<v4f *>(yr + k0 + 4 * u) = v4f{v[c][4 * u], v[c][4 * u + 1], v[c][4 * u + 2],
                                                                    v[c][4 * u + 3]};
            } else {
#pragma unroll
                for (int e = 0; e < 16; e++)
                    if (k0 + e < K) yr[k0 + e] = v[c][e];
            }
        }
    };
    /* LN: gamma and beta for the lane's columns, requested before the row's statistics need the wave for a while */
    constexpr int GB = KIND == PROD_LN && NCH <= 2 ? NCH : 1;
    float gam[GB][16], bet[GB][16];
    if (KIND == PROD_LN && NCH <= 2) {
#pragma unroll
        for (int c = 0; c < GB; c++) {
            const int k0 = 16 * (lane + 64 * c);
            if (VEC) {
                load16<true>(a.gamma, k0, K, gam[c]);
                load16<true>(a.beta, k0, K, bet[c]);
            } else {
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    gam[c][e] = k0 + e < K ? a.gamma[k0 + e] : 0.0f;
                    bet[c][e] = k0 + e < K ? a.beta[k0 + e] : 0.0f;
                }
            }
        }
    }
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int k0 = 16 * (lr + STRIDE * c);
        constexpr bool ROWS = KIND == PROD_SILU || KIND == PROD_LN;
        if (ROWS && VEC) {
            load16<true>(a.X + (size_t)m * a.ldx, k0, K, x[c]);
        } else if (ROWS) {
#pragma unroll
            for (int e = 0; e < 16; e++) x[c][e] = k0 + e < K ? a.X[(size_t)m * a.ldx + k0 + e] : 0.0f;
        } else if (KIND == PROD_HEADS && VEC) {   /* Dh % 16 == 0: the chunk lies in one head */
            const bool ok = k0 < K;
            const int h = ok ? k0 / a.Dh : 0;
            load16<true>(a.X + ((size_t)h * a.T + m) * a.Dh, ok ? k0 - h * a.Dh : 0, ok ? a.Dh : 0, x[c]);
        } else {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int k = k0 + e;
                float v = 0.0f;
                if (k < K) v = KIND == PROD_HEADS ? a.X[((size_t)(k / a.Dh) * a.T + m) * a.Dh + k % a.Dh]
                                                  : a.X[(size_t)k * a.T + m];
                x[c][e] = v;
            }
        }
        if (KIND == PROD_SILU) {
#pragma unroll
            for (int e = 0; e < 16; e++) x[c][e] = silu_p2(x[c][e]);
        }
    }
    if (KIND == PROD_LN) {
        /* LN2, two passes: LayerNorm(x), out as fp32 rows, then LayerNorm of those rows with gamma2 / beta2 (the
         * block's output norm followed by the next block's first norm, encoder.c:623 then 342) */
#pragma unroll
        for (int pass = 0; pass < (LN2 ? 2 : 1); pass++) {
            const float *gptr = pass ? a.gamma2 : a.gamma, *bptr = pass ? a.beta2 : a.beta;
            if (LN2 && pass == 1) {
                store_row(a.Y1 + (size_t)m * a.ldy1, x);
                if (NCH <= 2) {
#pragma unroll
                    for (int c = 0; c < GB; c++) {
                        const int k0 = 16 * (lane + 64 * c);
#pragma unroll
                        for (int e = 0; e < 16; e++) {
                            gam[c][e] = k0 + e < K ? a.gamma2[k0 + e] : 0.0f;
                            bet[c][e] = k0 + e < K ? a.beta2[k0 + e] : 0.0f;
                        }
                    }
                }
                __builtin_amdgcn_wave_barrier();   /* the first pass's reads of the staged row are done */
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            }
            /* The row in LDS by chain: element k at rt[(k % 8)·S + k / 8], so chain j's elements are contiguous and
             * read as float4; S = 128·NCH + 20 leaves each chain 16 elements of padding past its 128·NCH (a prefetch
             * of one batch past the end stays inside the chain's row) and puts the eight chains in different banks.
             * Lane L's element e of chunk c is k = 16·(L + 64c) + e: x[e] and x[e + 8] are neighbours in chain e.
             * Zeros beyond K. */
            constexpr int S = 128 * NCH + 20;
            float *rt = stage + w * 8 * S;
#pragma unroll
            for (int c = 0; c < NCH; c++)
#pragma unroll
                for (int e = 0; e < 8; e++)
                    *reinterpret_cast<float2 *>(rt + e * S + 2 * (lane + 64 * c)) = make_float2(x[c][e], x[c][e + 8]);
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            const int body = K / 8 * 8, n8 = body / 8, nb = n8 / 16;
            /* chain j = lane (j < 8): rt[j·S + 0 .. n8 − 1] in order, in batches of 16, the next batch's LDS reads in
             * flight while the current one is added */
            auto chain = [&](auto add) {
                float p = 0.0f;
                if (lane < 8) {
                    const float *cj = rt + lane * S;
                    auto add16 = [&](float p, const float4 (&v)[4]) {
#pragma unroll
                        for (int u = 0; u < 4; u++) p = add(add(add(add(p, v[u].x), v[u].y), v[u].z), v[u].w);
                        return p;
                    };
                    float4 va[4], vb[4];
#pragma unroll
                    for (int u = 0; u < 4; u++) va[u] = *reinterpret_cast<const float4 *>(cj + 4 * u);
                    int b = 0;
                    for (; b + 2 <= nb; b += 2) {   /* loads are unconditional: batch nb lies in the row's padding */
#pragma unroll
                        for (int u = 0; u < 4; u++)
                            vb[u] = *reinterpret_cast<const float4 *>(cj + 16 * (b + 1) + 4 * u);
                        __builtin_amdgcn_sched_barrier(0);   /* the next batch's reads stay ahead of these additions */
                        p = add16(p, va);
#pragma unroll
                        for (int u = 0; u < 4; u++)
                            va[u] = *reinterpret_cast<const float4 *>(cj + 16 * (b + 2) + 4 * u);
                        __builtin_amdgcn_sched_barrier(0);
                        p = add16(p, vb);
                    }
                    if (b < nb) p = add16(p, va);
                    for (int i = 16 * nb; i < n8; i++) p = add(p, cj[i]);
                }
                /* p2_hsum_avx2: lanes i and i + 4, then pairs */
                float v8[8];
#pragma unroll
                for (int j = 0; j < 8; j++) v8[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), j));
                return __fadd_rn(__fadd_rn(__fadd_rn(v8[0], v8[4]), __fadd_rn(v8[2], v8[6])),
                                 __fadd_rn(__fadd_rn(v8[1], v8[5]), __fadd_rn(v8[3], v8[7])));
            };
            /* LNR (NCH = 1, K = 1024 .. 1031: every LayerNorm of the encoder, chosen when the rows are few): each
             * chain's 128 elements read into registers once, for both sums, with one wait; the chains then run
             * without LDS round trips between batches. 4.5 against 5.3 us at 375 rows; at 6000 rows its 237 VGPRs
             * cost occupancy (13.0 against 11.3 us), so many rows take the LDS batches. */
            float4 cv[LNR ? 32 : 1];
            const bool whole = LNR && n8 == 128;
            if (LNR && whole) {   /* lanes 8.. read chain lane % 8 again (broadcast reads), their sums unused */
#pragma unroll
                for (int u = 0; u < (LNR ? 32 : 1); u++)
                    cv[u] = *reinterpret_cast<const float4 *>(rt + (lane & 7) * S + 4 * u);
            }
            auto chain_regs = [&](auto add) {
                float p = 0.0f;
#pragma unroll
                for (int u = 0; u < (LNR ? 32 : 1); u++) p = add(add(add(add(p, cv[u].x), cv[u].y), cv[u].z), cv[u].w);
                float v8[8];
#pragma unroll
                for (int j = 0; j < 8; j++) v8[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), j));
                return __fadd_rn(__fadd_rn(__fadd_rn(v8[0], v8[4]), __fadd_rn(v8[2], v8[6])),
                                 __fadd_rn(__fadd_rn(v8[1], v8[5]), __fadd_rn(v8[3], v8[7])));
            };
            auto add_sum = [](float p, float v) { return __fadd_rn(p, v); };
            auto at = [&](int k) { return rt[(k & 7) * S + (k >> 3)]; };
            float sum = whole ? chain_regs(add_sum) : chain(add_sum);
            for (int k = body; k < K; k++) sum = __fadd_rn(sum, at(k));
            const float mean = __fdiv_rn(sum, (float)K);
            auto add_sq = [mean](float p, float v) {
                const float d = __fsub_rn(v, mean);
                return __builtin_fmaf(d, d, p);
            };
            float var_sum = whole ? chain_regs(add_sq) : chain(add_sq);
            for (int k = body; k < K; k++) {
                const float d = __fsub_rn(at(k), mean);
                var_sum = __builtin_fmaf(d, d, var_sum);
            }
            const float inv_std = __fdiv_rn(1.0f, __builtin_sqrtf(__fadd_rn(__fdiv_rn(var_sum, (float)K), 1e-5f)));
#pragma unroll
            for (int c = 0; c < NCH; c++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int k = min(16 * (lane + 64 * c) + e, K - 1);
                    const float g = NCH <= 2 ? gam[NCH <= 2 ? c : 0][e] : gptr[k];
                    const float b = NCH <= 2 ? bet[NCH <= 2 ? c : 0][e] : bptr[k];
                    const float y = __builtin_fmaf(__fmul_rn(__fsub_rn(x[c][e], mean), inv_std), g, b);
                    x[c][e] = (16 * (lane + 64 * c) + e < K) ? y : 0.0f;
                }
    
        }
    }
    if (a.Y) {   /* fp32 rows (the exact route's LayerNorm, SiLU, head concatenation and transpose) */
        store_row(a.Y + (size_t)m * a.ldy, x);
        return;
    }
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; c++)
#pragma unroll
        for (int e = 0; e < 16; e++) amax = fmaxf(amax, fabsf(x[c][e]));
    amax = wave_max_dpp(amax);
    if (WPR > 1) {   /* the row's four waves meet in LDS (every wave of the workgroup is on this row) */
        if (lane == 0) wmax[w] = amax;
        __syncthreads();
        amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    }
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / scale;
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int k0 = 16 * (lr + STRIDE * c);
        if (k0 < a.ldq) *reinterpret_cast<uint4 *>(a.Q + q_index(m, k0, kst)) = quant16(x[c], k0, K, k16, scale, inv);
    }
    if (lr == 0) a.scales[m] = scale;
}

/* PROD_CMAJOR for K <= 1024, ldq <= 1024: a workgroup of 16 waves takes 16 consecutive rows t0..t0+15 of the
 * transpose of X [K][T]. Its threads read the 16 values X[d][t0..t0+15] of one channel d as one 64-byte segment
 * (produce_rows reads them a column element per lane), store them transposed into LDS (row stride 1028 floats, so
 * the 64 lanes of a store hit distinct banks and rows stay 16-byte aligned), then wave w quantises row t0 + w from
 * LDS exactly as produce_rows does. Rows at or beyond T read zeros and so write zero codes, as the padding needs. */
__global__ __launch_bounds__(1024) void cmajor_tile(ProdArgs a)
{
    constexpr int LD = 1024 + 4;
    __shared__ __align__(16) float tile[16 * LD];
    /* Tiles 2g and 2g + 1 read the two halves of the same 128-byte lines, so they go to workgroups 16p + x and
     * 16p + 8 + x (g = 8p + x), which the round-robin dispatch puts on the same XCD x, and the second finds the
     * lines in that XCD's L2. The grid is padded to a multiple of 16 workgroups; the padding ones exit. */
    const int b = (int)blockIdx.x, xcd = b % 8, slot = b / 8;
    const int tix = 2 * (8 * (slot / 2) + xcd) + slot % 2;
    if (tix >= a.Mp / 16) return;
    const int tid = threadIdx.x, t0 = tix * 16;
    const int K = a.K, T = a.T;
    {
        const int tr = tid & 15, dr = tid >> 4;
        const int t = t0 + tr;
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int d = dr + 64 * i;
            v[i] = (d < K && t < T) ? a.X[(size_t)d * T + t] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 16; i++) tile[tr * LD + dr + 64 * i] = v[i];
    }
    __syncthreads();
    const int lane = tid & 63, w = tid >> 6;
    const int m = t0 + w;
    const int kst = a.ldq / 64, k16 = K / 16 * 16, k0 = 16 * lane;
    float x[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float4 v = *reinterpret_cast<const float4 *>(&tile[w * LD + k0 + 4 * q]);
        x[4 * q] = v.x;
        x[4 * q + 1] = v.y;
        x[4 * q + 2] = v.z;
        x[4 * q + 3] = v.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; e++) amax = fmaxf(amax, fabsf(x[e]));
    amax = wave_max_dpp(amax);
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / scale;
    if (k0 < a.ldq) *reinterpret_cast<uint4 *>(a.Q + q_index(m, k0, kst)) = quant16(x, k0, K, k16, scale, inv);
    if (lane == 0 && m < a.M) a.scales[m] = scale;
}

/* ── the conformer block between its linears (encoder.c:252-613): attention and convolution internals ────── */

constexpr int kD = 1024, kH = 8, kDh = 128, kConvK = 9;   /* P2_D_MODEL, P2_N_HEADS, P2_HEAD_DIM, P2_CONV_KERNEL */

/* The head gather of encoder.c:366-404 without its transpose: Q_u = Q + bias_u, Q_v = Q + bias_v and V as [H, T, Dh]
 * from the fused rows QKV [T, 3D] (q | k | v); V is skipped when vh is null (a caller whose product reads V in
 * place). One thread per element, consecutive threads along d. */
__global__ __launch_bounds__(256) void gather_qv(int T, const float *__restrict__ qkv, const float *__restrict__ bu,
                                                 const float *__restrict__ bv, float *__restrict__ qu,
                                                 float *__restrict__ qv, float *__restrict__ vh)
{
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)T * kD) return;
    const int t = (int)(idx / kD), c = (int)(idx % kD), h = c / kDh, d = c % kDh;
    const float *row = qkv + (size_t)t * 3 * kD;
    const float q = row[c];
    const size_t o = ((size_t)h * T + t) * kDh + d;
    qu[o] = __fadd_rn(q, bu[c]);
    qv[o] = __fadd_rn(q, bv[c]);
    if (vh) vh[o] = row[2 * kD + c];
}

/* Per head transposed: dst[h][d][r] = src[r·ld + h·Dh + d] for r < rows (the keys of gather_heads, encoder.c:397-398,
 * and transpose_pos, encoder.c:406-423). A 32-row × 128-column tile of one head through LDS: reads along d, writes
 * along r. */
__global__ __launch_bounds__(256) void head_transpose(int rows, const float *__restrict__ src, int ld,
                                                      float *__restrict__ dst)
{
    __shared__ float tile[kDh][33];
    const int r0 = blockIdx.x * 32, h = blockIdx.y, tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int idx = tid + 256 * i, rl = idx / kDh, d = idx % kDh;
        if (r0 + rl < rows) tile[d][rl] = src[(size_t)(r0 + rl) * ld + h * kDh + d];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int idx = tid + 256 * i, d = idx / 32, rl = idx % 32;
        if (r0 + rl < rows) dst[((size_t)h * kDh + d) * rows + r0 + rl] = tile[d][rl];
    }
}

/* combine_softmax (encoder.c:425-450) with p2_softmax's AVX2 route (tensor_ops.c:354-413) in IEEE operations, eight
 * threads per row of the [H·T, T] scores: thread q takes the row's elements j ≡ q (mod 8). a[j] = (ac[j] + bd[j +
 * T − 1 − i]) · scale (the relative shift: row i of a head reads a window of its bd row); the maximum; for j below
 * the last multiple of eight, e = exp_p2(a − max) added to running sum q in order of j (the eight vector lanes),
 * the sums meeting as p2_hsum_avx2 does; the tail elements take expf and are added in order after them; then every
 * element times 1/sum. */
__global__ __launch_bounds__(256) void combine_softmax_rows(int rows, int T, float scale, float *__restrict__ ac,
                                                            const float *__restrict__ bd)
{
    const int r = blockIdx.x * 32 + (threadIdx.x >> 3), q = threadIdx.x & 7;
    const bool live = r < rows;
    const int i = live ? r % T : 0, L = 2 * T - 1, body = T / 8 * 8;
    float *a = ac + (size_t)(live ? r : 0) * T;
    const float *b = bd + (size_t)(live ? r : 0) * L + (T - 1 - i);
    float mx = -INFINITY;
    if (live)
        for (int j = q; j < T; j += 8) {
            const float v = __fmul_rn(__fadd_rn(a[j], b[j]), scale);
            a[j] = v;
            mx = fmaxf(mx, v);
        }
    mx = fmaxf(mx, __shfl_xor(mx, 1, 8));
    mx = fmaxf(mx, __shfl_xor(mx, 2, 8));
    mx = fmaxf(mx, __shfl_xor(mx, 4, 8));
    float lane_sum = 0.0f, tail = 0.0f;
    if (live) {
        for (int j = q; j < body; j += 8) {
            const float e = exp_p2(__fsub_rn(a[j], mx));
            a[j] = e;
            lane_sum = __fadd_rn(lane_sum, e);
        }
        if (body + q < T) {
            tail = expf(__fsub_rn(a[body + q], mx));
            a[body + q] = tail;
        }
    }
    /* p2_hsum_avx2: lanes q and q + 4, then q and q + 2, then 0 and 1 */
    float s = __fadd_rn(lane_sum, __shfl_down(lane_sum, 4, 8));
    s = __fadd_rn(s, __shfl_down(s, 2, 8));
    s = __fadd_rn(s, __shfl_down(s, 1, 8));
    s = __shfl(s, 0, 8);
    for (int k = 0; k < T - body; k++) s = __fadd_rn(s, __shfl(tail, k, 8));
    const float inv = __fdiv_rn(1.0f, s);
    if (live)
        for (int j = q; j < T; j += 8) a[j] = __fmul_rn(a[j], inv);
}

/* combine_softmax_rows' arithmetic with one wave per row (T <= 64·NM), four rows per workgroup. The row's scores are
 * read and written along j by all 64 lanes (lane l holds j = l + 64m in registers); the exponentials go to LDS by
 * chain, element j at chain j mod 8, place j / 8, so that lanes 0..7 run the eight sums of the AVX2 route's lanes
 * in order of j over contiguous float4 reads; the tail (expf) and p2_hsum_avx2's pairing follow on lane 0. Every
 * operation and its order are those of combine_softmax_rows: the results are the same bits. */
template <int NM>
__global__ __launch_bounds__(256) void combine_softmax_wave(int rows, int T, float scale, float *__restrict__ ac,
                                                            const float *__restrict__ bd)
{
    constexpr int S = 8 * NM + 4;   /* chain stride (floats): 64·NM / 8 places, 16 bytes of padding */
    __shared__ __align__(16) float chains[4][8 * S];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int r = blockIdx.x * 4 + w;
    if (r >= rows) return;
    const int i = r % T, L = 2 * T - 1, body = T / 8 * 8;
    float *a = ac + (size_t)r * T;
    const float *b = bd + (size_t)r * L + (T - 1 - i);
    float v[NM];
    float mx = -INFINITY;
#pragma unroll
    for (int m = 0; m < NM; m++) {
        const int j = lane + 64 * m;
        v[m] = j < T ? __fmul_rn(__fadd_rn(a[j], b[j]), scale) : -INFINITY;
        mx = fmaxf(mx, v[m]);
    }
    mx = wave_max_dpp(mx);
    float *ch = chains[w];
#pragma unroll
    for (int m = 0; m < NM; m++) {
        const int j = lane + 64 * m;
        if (j < body) v[m] = exp_p2(__fsub_rn(v[m], mx));
        else if (j < T) v[m] = expf(__fsub_rn(v[m], mx));
        if (j < T) ch[(j & 7) * S + (j >> 3)] = v[m];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    /* lane q < 8: the running sum of chain q over places 0 .. body/8 − 1 */
    float p = 0.0f;
    if (lane < 8) {
        const float *cq = ch + lane * S;
        const int n8 = body / 8;
        int k = 0;
        for (; k + 4 <= n8; k += 4) {
            const float4 x = *reinterpret_cast<const float4 *>(cq + k);
            p = __fadd_rn(__fadd_rn(__fadd_rn(__fadd_rn(p, x.x), x.y), x.z), x.w);
        }
        for (; k < n8; k++) p = __fadd_rn(p, cq[k]);
    }
    float l8[8];
#pragma unroll
    for (int q = 0; q < 8; q++) l8[q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), q));
    float s = __fadd_rn(__fadd_rn(__fadd_rn(l8[0], l8[4]), __fadd_rn(l8[2], l8[6])),
                        __fadd_rn(__fadd_rn(l8[1], l8[5]), __fadd_rn(l8[3], l8[7])));
    for (int j = body; j < T; j++) s = __fadd_rn(s, ch[(j & 7) * S + (j >> 3)]);
    const float inv = __fdiv_rn(1.0f, s);
#pragma unroll
    for (int m = 0; m < NM; m++) {
        const int j = lane + 64 * m;
        if (j < T) a[j] = __fmul_rn(v[m], inv);
    }
}

/* Direct global → LDS loads (16 bytes per lane into 16-byte lane slots at lds + 16·lane). Issued from inline
 * assembly so that the compiler adds no waits of its own for them: the GEMM waits for them explicitly (wait_vm),
 * and the compiler's waits for its own loads stay correct since the vector-memory counter retires in order. */
__device__ __forceinline__ void dma_16(const void *src, const void *lds)
{
    const uint32_t a = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(a) : "memory", "m0");
}

/* s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt left open); a compiler barrier for memory operations */
template <int N>
__device__ __forceinline__ void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
    asm volatile("" ::: "memory");
}

/* A 16-byte load into registers, issued from inline assembly as dma_16 is: the caller waits for it explicitly
 * (wait_vm) and then passes the registers through pin16, after which the compiler may read them. */
__device__ __forceinline__ v4u load16_async(const void *src)
{
    v4u r;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(src) : "memory");
    return r;
}
__device__ __forceinline__ void pin16(v4u &r) { asm volatile("" : "+v"(r)); }

/* this wave's LDS reads complete, then the workgroup barrier; no wait on vector memory */
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

/* Relative-position self-attention of one head for 16 query rows (encoder.c:495-523 between the projections): the
 * scores S[i][j] = (Q_u[i]·K[j] + Q_v[i]·P[j + T − 1 − i])·scale, their softmax over j as combine_softmax_rows
 * computes it (the AVX2 route's order, the same operations), and O[i] = Σ_j softmax(S)[i][j]·V[j], written to
 * out [8][T][128] (with `rows`, [T][1024]). Q_u = Q + bias_u and Q_v = Q + bias_v are formed as the operands load
 * (gather_heads' additions);
 * Q, K and V are read inside QKV [T][3·1024] and the positional rows inside P [2T − 1][1024], head h at column
 * offset 128·h. The scores live in LDS only: neither the [T, T] and [T, 2T − 1] products nor the half of the
 * positional product that no row reads is made. Products on v_mfma_f32_16x16x4_f32 (D = A·B with A's rows and B's
 * columns from lane % 16, the four k of a step from lane / 16): for a score tile the 16 keys or positions are A's
 * rows and the 16 queries B's columns, lane group g taking k = 16(s / 4) + 4g + s % 4 at step s (a row's 128 values
 * arrive as 16-byte loads, the four lanes of a row reading 64 contiguous bytes per load: with k = 32g + s each load
 * touched 64 cache lines and the loads' address processing bounded the kernel); for O the 16 output dimensions are
 * A's rows, the queries B's columns, j = 4s + g.
 * Eight waves: key and position tiles round-robin over the waves, two softmax rows each, 16 output dimensions
 * each. Grid 8·ceil(T / 16); T <= 64·NM. With NM <= 6 (T <= 384) the score tiles reach LDS by direct loads
 * (RING below: whole 128-byte lines per load instead of half lines, 2.5 us less at T = 375, the same bits); the
 * longer rows' scores leave no LDS room for the slots, and their tiles load into registers. */
template <int NM>
__global__ __launch_bounds__(512) void attention_rel(int T, float scale, const float *__restrict__ qkv,
                                                     const float *__restrict__ bu, const float *__restrict__ bv,
                                                     const float *__restrict__ P, float *__restrict__ out, int rows)
{
    constexpr int SP = 64 * NM + 4;   /* score row pitch (floats): 16 rows 4 banks apart */
    constexpr int CS = 8 * NM + 4;    /* softmax chain stride */
    constexpr int D3 = 3 * kD, NW = 8;
    /* RING: two 8 KB tile slots per wave, the softmax chains in the same space once the scores are made, and a slot
     * per lane for BD's out-of-range updates; else the chains (which also hold that slot) */
    constexpr bool RING = (16 * SP + NW * 2 * 2048 + NW * 64) * 4 <= 160 * 1024;
    static_assert(!RING || NW * 8 * CS <= NW * 2 * 2048, "chains inside the ring");
    __shared__ __align__(16) float S[16 * SP];
    __shared__ __align__(16) float ring[RING ? NW * 2 * 2048 : NW * 8 * CS];
    __shared__ __align__(16) float spare[RING ? NW * 64 : 1];
    float (*chains)[8 * CS] = reinterpret_cast<float (*)[8 * CS]>(ring);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, x = lane & 15;
    float *dslot = RING ? spare + 64 * w : chains[w];   /* this wave's per-lane slots for BD's outside updates */
    /* workgroups reach the 8 XCDs round-robin by linear id: head = id % 8 keeps each head's K, V and positional
     * rows in one XCD's L2 (with the head as the grid's second index every XCD fetched every head) */
    const int i0 = (int)(blockIdx.x / 8) * 16, h = (int)(blockIdx.x % 8);
    const int Tp = (T + 15) / 16 * 16, L = 2 * T - 1;

    /* this lane's query operands: row i0 + x (clamped; rows past T are computed and not stored), k = 16c + 4g + e
     * for c = 0..7, e = 0..3, held as element 4c + e (step s = 4c + e sums k = 16(s / 4) + 4g + s % 4 over the four
     * lane groups): one 16-byte load per c, and the four lanes of a row read 64 contiguous bytes at once */
    float qu[32], qv[32];
    {
        const int iq = min(i0 + x, T - 1);
        const float4 *q = reinterpret_cast<const float4 *>(qkv + (size_t)iq * D3 + h * kDh);
        const float4 *u = reinterpret_cast<const float4 *>(bu + h * kDh);
        const float4 *v = reinterpret_cast<const float4 *>(bv + h * kDh);
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const float4 a = q[4 * c + g], b = u[4 * c + g], d = v[4 * c + g];
            qu[4 * c] = __fadd_rn(a.x, b.x); qu[4 * c + 1] = __fadd_rn(a.y, b.y);
            qu[4 * c + 2] = __fadd_rn(a.z, b.z); qu[4 * c + 3] = __fadd_rn(a.w, b.w);
            qv[4 * c] = __fadd_rn(a.x, d.x); qv[4 * c + 1] = __fadd_rn(a.y, d.y);
            qv[4 * c + 2] = __fadd_rn(a.z, d.z); qv[4 * c + 3] = __fadd_rn(a.w, d.w);
        }
    }
    auto load_row = [&](const float *row, float (&r)[32]) __attribute__((always_inline)) {
        const float4 *r4 = reinterpret_cast<const float4 *>(row);
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const float4 a = r4[4 * c + g];
            r[4 * c] = a.x; r[4 * c + 1] = a.y; r[4 * c + 2] = a.z; r[4 * c + 3] = a.w;
        }
    };
    /* one 16 × 16 score tile: 32 steps on two accumulators (even and odd steps), added at the end */
    auto dot16 = [&](const float (&r)[32], const float (&qq)[32]) __attribute__((always_inline)) {
        v4f a0 = v4f{0.0f, 0.0f, 0.0f, 0.0f}, a1 = a0;
#pragma unroll
        for (int s = 0; s < 32; s += 2) {
            a0 = __builtin_amdgcn_mfma_f32_16x16x4f32(r[s], qq[s], a0, 0, 0, 0);
            a1 = __builtin_amdgcn_mfma_f32_16x16x4f32(r[s + 1], qq[s + 1], a1, 0, 0, 0);
        }
        return a0 + a1;   /* lane holds D[4g + e][x]: key / position 4g + e of the tile, query x */
    };
    /* BD, shifted into S: row i reads positions j + T − 1 − i, so the 16 rows need positions lbase .. 2T − 2 − i0 */
    const int ilast = min(i0 + 15, T - 1), lbase = T - 1 - ilast;
    const int n_ac = Tp / 16, n_bd = (2 * T - 1 - i0 - lbase + 15) / 16;
    /* each (i, j) is one lane's, once; a lane whose (i, j) lies outside the scores updates a slot of its own instead
     * (in the chain buffer without RING, written again before the softmax reads it), so the four reads and writes
     * need no branch */
    auto consume_bd = [&](int pt, v4f acc) __attribute__((always_inline)) {
        const int i = i0 + x;
        int at[4];
        float sv[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int j = lbase + 16 * pt + 4 * g + e - (T - 1 - i);
            at[e] = (i < T && j >= 0 && j < T) ? x * SP + j : -1;
            sv[e] = at[e] >= 0 ? S[at[e]] : dslot[lane];
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float r = __fmul_rn(__fadd_rn(sv[e], acc[e]), scale);
            if (at[e] >= 0) S[at[e]] = r;
            else dslot[lane] = r;
        }
    };
    if constexpr (RING) {
        /* Tiles (16 key or position rows × the head's 128 values, 8 KB) reach LDS by direct loads of two rows per
         * instruction, into two slots per wave: tile q + 2 is requested as soon as tile q is read out, so one tile
         * is always on its way while another is multiplied. Row r's 16-byte chunk cc lands at place cc ^ r of the
         * row, so the operand reads (lane (x, g): row x, chunks 4c + g) hit 16 distinct places of every 256-byte
         * window. Wave w takes AC tiles w, w + 8, … then BD tiles w, w + 8, …; no other wave reads its slots. */
        const int nac = n_ac > w ? (n_ac - w + NW - 1) / NW : 0;
        const int nbd = n_bd > w ? (n_bd - w + NW - 1) / NW : 0;
        const int n = nac + nbd;
        float *mine = ring + w * 2 * 2048;
        auto issue = [&](int q) __attribute__((always_inline)) {
            const bool ac = q < nac;
            const int t = w + NW * (ac ? q : q - nac);
            float *slot = mine + (q & 1) * 2048;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int r = 2 * k + (lane >> 5), cc = (lane & 31) ^ r;
                const float *row = ac ? qkv + (size_t)min(16 * t + r, T - 1) * D3 + kD + h * kDh
                                      : P + (size_t)min(lbase + 16 * t + r, L - 1) * kD + h * kDh;
                dma_16(row + 4 * cc, slot + 256 * k);
            }
        };
        auto read_tile = [&](int q, float (&r)[32]) __attribute__((always_inline)) {
            const float *slot = mine + (q & 1) * 2048 + x * 128;
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const float4 a = *reinterpret_cast<const float4 *>(slot + 4 * ((4 * c + g) ^ x));
                r[4 * c] = a.x; r[4 * c + 1] = a.y; r[4 * c + 2] = a.z; r[4 * c + 3] = a.w;
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   /* the slot is read out before it is refilled */
            if (q + 2 < n) issue(q + 2);
        };
        /* the query operands are in registers before the first direct load (the compiler's waits for its own
         * loads do not count the direct ones) */
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (n > 0) issue(0);
        if (n > 1) issue(1);
        int q = 0;
        for (; q < nac; q++) {   /* AC into S: S[x][16·kt + 4g + e] */
            if (q + 1 < n) wait_vm<8>(); else wait_vm<0>();
            float r[32];
            read_tile(q, r);
            const int kt = w + NW * q;
            *reinterpret_cast<v4f *>(&S[x * SP + 16 * kt + 4 * g]) = dot16(r, qu);
        }
        __syncthreads();   /* every AC tile is in S before BD adds to it */
        for (; q < n; q++) {
            if (q + 1 < n) wait_vm<8>(); else wait_vm<0>();
            float r[32];
            read_tile(q, r);
            consume_bd(w + NW * (q - nac), dot16(r, qv));
        }
    } else {
        /* tiles t = w, w + NW, … < n of one kind, in groups of MAXT: a group's rows are all requested before its
         * first product (the loads' latency, thousands of cycles from L2, is what bounds a tile; one tile in flight
         * at a time left the matrix cores idle most of the time) */
        constexpr int MAXT = 4;
        /* `between` runs once in every wave after the first group's loads are issued (the barrier before BD: its
         * rows are on their way while the other waves finish AC) */
        auto run_tiles = [&](int n, const float (&qq)[32], auto row_of, auto consume, auto between)
                             __attribute__((always_inline)) {
            float r[MAXT][32];
            int t0 = w;
#pragma unroll
            for (int q = 0; q < MAXT; q++)
                if (t0 + NW * q < n) load_row(row_of(t0 + NW * q), r[q]);
            between();
            while (t0 < n) {
#pragma unroll
                for (int q = 0; q < MAXT; q++)
                    if (t0 + NW * q < n) consume(t0 + NW * q, dot16(r[q], qq));
                t0 += NW * MAXT;
                if (t0 >= n) break;
#pragma unroll
                for (int q = 0; q < MAXT; q++)
                    if (t0 + NW * q < n) load_row(row_of(t0 + NW * q), r[q]);
            }
        };

        /* AC into S: S[x][16·kt + 4g + e] */
        run_tiles(n_ac, qu,
                  [&](int kt) { return qkv + (size_t)min(16 * kt + x, T - 1) * D3 + kD + h * kDh; },
                  [&](int kt, v4f acc) { *reinterpret_cast<v4f *>(&S[x * SP + 16 * kt + 4 * g]) = acc; }, [] {});
        run_tiles(n_bd, qv,
                  [&](int pt) { return P + (size_t)min(lbase + 16 * pt + x, L - 1) * kD + h * kDh; },
                  consume_bd,
                  [] { __syncthreads(); });
    }
    __syncthreads();
    /* O[i0 + x][16c + 4g + e] = Σ_j p[x][j]·V[j][16c + 4g + e], j = 4s + g, for output dimensions c = w, over
     * all steps: chunks of CH steps, the next chunk's V loaded while the current one is multiplied, four
     * accumulators (steps s mod 4) added at the end. V does not depend on the softmax, so the first chunk is
     * requested before it. */
    constexpr int CH = 24;
    const int c = w, sb = 0, se = Tp / 4;
    const float *vb = qkv + 2 * kD + h * kDh + 16 * c + x;
    auto load_v = [&](int s0, float (&vv)[CH]) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < CH; u++) vv[u] = vb[(size_t)min(4 * (s0 + u) + g, T - 1) * D3];   /* p = 0 past T */
    };
    float va[CH], vc[CH];
    if (sb < se) load_v(sb, va);
    /* softmax of rows w and w + 8 (combine_softmax_wave's arithmetic, the scores from LDS) */
    const int body = T / 8 * 8;
    for (int rr = w; rr < 16; rr += NW) {
        if (i0 + rr >= T) break;
        float *row = S + rr * SP;
        float v[NM];
        float mx = -INFINITY;
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const int j = lane + 64 * m;
            v[m] = j < T ? row[j] : -INFINITY;
            mx = fmaxf(mx, v[m]);
        }
        mx = wave_max_dpp(mx);
        float *ch = chains[w];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");   /* the previous row's chain reads are done */
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const int j = lane + 64 * m;
            if (j < body) v[m] = exp_p2(__fsub_rn(v[m], mx));
            else if (j < T) v[m] = expf(__fsub_rn(v[m], mx));
            if (j < T) ch[(j & 7) * CS + (j >> 3)] = v[m];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        float p = 0.0f;
        if (lane < 8) {
            const float *cq = ch + lane * CS;
            const int n8 = body / 8;
            int k = 0;
            for (; k + 4 <= n8; k += 4) {
                const float4 a = *reinterpret_cast<const float4 *>(cq + k);
                p = __fadd_rn(__fadd_rn(__fadd_rn(__fadd_rn(p, a.x), a.y), a.z), a.w);
            }
            for (; k < n8; k++) p = __fadd_rn(p, cq[k]);
        }
        float l8[8];
#pragma unroll
        for (int q = 0; q < 8; q++) l8[q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), q));
        float s = __fadd_rn(__fadd_rn(__fadd_rn(l8[0], l8[4]), __fadd_rn(l8[2], l8[6])),
                            __fadd_rn(__fadd_rn(l8[1], l8[5]), __fadd_rn(l8[3], l8[7])));
        float tv[7];   /* the tail's exponentials, read at once, added in order */
#pragma unroll
        for (int q = 0; q < 7; q++) tv[q] = ch[q * CS + (body >> 3)];   /* element body + q: chain q, place body / 8 */
#pragma unroll
        for (int q = 0; q < 7; q++)
            if (body + q < T) s = __fadd_rn(s, tv[q]);
        const float inv = __fdiv_rn(1.0f, s);
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const int j = lane + 64 * m;
            if (j < T) row[j] = __fmul_rn(v[m], inv);
            else if (j < Tp) row[j] = 0.0f;   /* the product with V runs over Tp keys */
        }
    }
    __syncthreads();
    const float *pr = S + x * SP + g;
    v4f a4[4];
#pragma unroll
    for (int q = 0; q < 4; q++) a4[q] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    auto mma_chunk = [&](int s0, const float (&vv)[CH]) __attribute__((always_inline)) {
        float pp[CH];
#pragma unroll
        for (int u = 0; u < CH; u++) {
            const float v = pr[4 * min(s0 + u, se - 1)];   /* read unconditionally, zero past the range */
            pp[u] = s0 + u < se ? v : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < CH; u++) a4[u % 4] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[u], pp[u], a4[u % 4], 0, 0, 0);
    };
    {
        int s0 = sb;
        while (s0 < se) {
            if (s0 + CH < se) load_v(s0 + CH, vc);
            mma_chunk(s0, va);
            s0 += CH;
            if (s0 >= se) break;
            if (s0 + CH < se) load_v(s0 + CH, va);
            mma_chunk(s0, vc);
            s0 += CH;
        }
    }
    const v4f acc = (a4[0] + a4[1]) + (a4[2] + a4[3]);
    /* rows: out [T][1024], head h at columns 128·h (concat_heads' layout, encoder.c:449-463); else [8][T][128] */
    const size_t at = rows ? (size_t)(i0 + x) * kD + h * kDh : ((size_t)h * T + i0 + x) * kDh;
    if (i0 + x < T) *reinterpret_cast<v4f *>(out + at + 16 * c + 4 * g) = acc;
}

/* glu_to_channel_major (encoder.c:543-555): gated[d][t] = pw1[t][d] / (1 + expf(−pw1[t][D + d])), the exponent's
 * argument clamped at 87 (p2_expneg, phonon2.h:38-41). A 32-frame × 64-channel tile through LDS: reads along d,
 * writes along t. */
__global__ __launch_bounds__(256) void glu_channel_major(int T, const float *__restrict__ pw1,
                                                         float *__restrict__ gated)
{
    __shared__ float tile[64][33];
    const int t0 = blockIdx.x * 32, d0 = blockIdx.y * 64, tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int idx = tid + 256 * i, tl = idx / 64, dl = idx % 64;
        if (t0 + tl < T) {
            const float *row = pw1 + (size_t)(t0 + tl) * 2 * kD;
            const float g = row[kD + d0 + dl];
            tile[dl][tl] = __fdiv_rn(row[d0 + dl], __fadd_rn(1.0f, expf(g < -87.0f ? 87.0f : -g)));
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int idx = tid + 256 * i, dl = idx / 32, tl = idx % 32;
        if (t0 + tl < T) gated[(size_t)(d0 + dl) * T + t0 + tl] = tile[dl][tl];
    }
}

/* p2_depthwise_conv1d (tensor_ops.c:559-648; kernel 9, padding 4, the BatchNorm folded into w and b) then p2_swish
 * over the result (tensor_ops.c:437-491): per channel d and frame t, v = b[d], then v = fmaf(x[t − 4 + k], w[d][k],
 * v) for the taps inside the sequence in order of k (the AVX2 route's fmadd chain; its scalar edges contract the
 * same way), out = v · (1 / (1 + e^−v)) as silu_p2. Channel-major [D][T] in and out, one thread per frame. */
__global__ __launch_bounds__(256) void dwconv_silu(int T, const float *__restrict__ x, const float *__restrict__ w,
                                                   const float *__restrict__ bias, float *__restrict__ out)
{
    const int d = blockIdx.y, t = blockIdx.x * 256 + threadIdx.x;
    if (t >= T) return;
    const float *xr = x + (size_t)d * T;
    float v = bias[d];
#pragma unroll
    for (int k = 0; k < kConvK; k++) {
        const int src = t - kConvK / 2 + k;
        if (src >= 0 && src < T) v = __builtin_fmaf(xr[src], w[d * kConvK + k], v);
    }
    out[(size_t)d * T + t] = silu_p2(v);
}

/* glu_channel_major and dwconv_silu in one pass (encoder.c:594-597): a 32-frame × 16-channel tile of the
 * depthwise convolution's output takes the GLU of frames t0 − 4 .. t0 + 35 of its channels into LDS (the halo is
 * computed twice, by both neighbouring tiles) and the channels' taps, then each output runs dwconv_silu's chain over
 * the LDS values. Every value is made by the same operations as in the two kernels, so the result is the same bits;
 * the gated [1024][T] buffer is never written. Grid (ceil(T / 32), 64): 768 workgroups at T = 375.
 * ROWS: out is [T][1024] (the transpose of the reference's channel-major output, as the next linear reads it),
 * consecutive threads writing consecutive channels of a frame; else [1024][T]. */
template <bool ROWS>
__global__ __launch_bounds__(256) void glu_dwconv_silu(int T, const float *__restrict__ pw1, const float *__restrict__ w,
                                                       const float *__restrict__ bias, float *__restrict__ out)
{
    constexpr int TT = 32, CB = 16, HALO = kConvK / 2, TW = TT + 2 * HALO;   /* 32-channel tiles: 1 us slower */
    __shared__ float gt[CB][TW + 1];
    __shared__ float wt[CB * kConvK + CB];
    const int t0 = blockIdx.x * TT, d0 = blockIdx.y * CB, tid = threadIdx.x;
    for (int i = tid; i < CB * kConvK + CB; i += 256)
        wt[i] = i < CB * kConvK ? w[d0 * kConvK + i] : bias[d0 + i - CB * kConvK];
    for (int i = tid; i < TW * CB; i += 256) {
        const int tl = i / CB, dl = i % CB, t = t0 - HALO + tl;
        float v = 0.0f;
        if (t >= 0 && t < T) {
            const float *row = pw1 + (size_t)t * 2 * kD;
            const float g = row[kD + d0 + dl];
            v = __fdiv_rn(row[d0 + dl], __fadd_rn(1.0f, expf(g < -87.0f ? 87.0f : -g)));
        }
        gt[dl][tl] = v;
    }
    __syncthreads();
    for (int i = tid; i < TT * CB; i += 256) {
        const int dl = ROWS ? i % CB : i / TT, tl = ROWS ? i / CB : i % TT, t = t0 + tl;
        if (t >= T) continue;
        float v = wt[CB * kConvK + dl];
#pragma unroll
        for (int k = 0; k < kConvK; k++) {
            const int src = t - HALO + k;
            if (src >= 0 && src < T) v = __builtin_fmaf(gt[dl][tl + k], wt[dl * kConvK + k], v);
        }
        if (ROWS) out[(size_t)t * kD + d0 + dl] = silu_p2(v);
        else out[(size_t)(d0 + dl) * T + t] = silu_p2(v);
    }
}

/* The convolution module's int8 form in one pass (encoder.c:594-597 and the QuantA branch of
 * channel_major_to_rows, encoder.c:554-568): GLU, depthwise convolution, SiLU and the per-row quantisation of the
 * output rows for pw2. A workgroup owns TT frames and all 1024 channels, one thread per channel: it makes the GLU of
 * its channel for frames t0 − 4 .. t0 + TT + 3 in registers, runs dwconv_silu's fmadd chain for its TT outputs and
 * writes them as rows to LDS; then one wave per row quantises it as quant_rows does (the row's 1024 values, 16 per
 * lane, its maximum across the wave, the same rounding), into the tiled layout with its scale. Every value is made
 * by the same operations as glu_dwconv_silu<true> followed by quant_rows, so the bits are theirs; neither the
 * fp32 rows nor the gated buffer reach memory. The workgroup with the last frames also writes the zero rows up to
 * the next multiple of 16. Grid ceil(T / TT). */
template <int TT>
__global__ __launch_bounds__(1024) void glu_dwconv_silu_quant(int T, const float *__restrict__ pw1,
                                                              const float *__restrict__ w,
                                                              const float *__restrict__ bias, int8_t *__restrict__ Q,
                                                              int ldq, float *__restrict__ scales)
{
    constexpr int HALO = kConvK / 2, TW = TT + 2 * HALO;
    static_assert(TT <= 16, "one wave per row: at most 16 rows per workgroup");
    __shared__ __attribute__((aligned(16))) float y[TT][kD + 4];
    const int d = threadIdx.x, t0 = blockIdx.x * TT;
    float gv[TW];
#pragma unroll
    for (int i = 0; i < TW; i++) {
        const int t = t0 - HALO + i;
        float v = 0.0f;
        if (t >= 0 && t < T) {
            const float *row = pw1 + (size_t)t * 2 * kD;
            const float g = row[kD + d];
            v = __fdiv_rn(row[d], __fadd_rn(1.0f, expf(g < -87.0f ? 87.0f : -g)));
        }
        gv[i] = v;
    }
    float taps[kConvK];
#pragma unroll
    for (int k = 0; k < kConvK; k++) taps[k] = w[d * kConvK + k];
    const float b = bias[d];
#pragma unroll
    for (int tl = 0; tl < TT; tl++) {
        const int t = t0 + tl;
        float v = b;
#pragma unroll
        for (int k = 0; k < kConvK; k++) {
            const int src = t - HALO + k;
            if (src >= 0 && src < T) v = __builtin_fmaf(gv[tl + k], taps[k], v);
        }
        y[tl][d] = silu_p2(v);
    }
    __syncthreads();
    const int lane = d & 63, wave = d >> 6;
    const int kst = ldq / 64;
    if (wave < TT) {
        const int m = t0 + wave;
        if (m < T) {
            float x[16];
            const float4 *src = reinterpret_cast<const float4 *>(&y[wave][16 * lane]);
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float4 v = src[c];
                x[4 * c] = v.x; x[4 * c + 1] = v.y; x[4 * c + 2] = v.z; x[4 * c + 3] = v.w;
            }
            float amax = 0.0f;
#pragma unroll
            for (int e = 0; e < 16; e++) amax = fmaxf(amax, fabsf(x[e]));
            amax = wave_max_dpp(amax);
            const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
            const float inv = 1.0f / scale;
            *reinterpret_cast<uint4 *>(Q + q_index(m, 16 * lane, kst)) = quant16(x, 16 * lane, kD, kD, scale, inv);
            for (int k0 = kD + 16 * lane; k0 < ldq; k0 += 1024)   /* columns beyond the row: zeros */
                *reinterpret_cast<uint4 *>(Q + q_index(m, k0, kst)) = make_uint4(0u, 0u, 0u, 0u);
            if (lane == 0) scales[m] = scale;
        }
    }
    /* the pad rows T .. roundup(T, 16) − 1 of the last row group, by the workgroup holding frame T − 1 */
    const int Mp = (T + 15) / 16 * 16;
    if (t0 <= T - 1 && T - 1 < t0 + TT)
        for (int i = d; i < (Mp - T) * (ldq / 16); i += 1024) {
            const int m = T + i / (ldq / 16), k0 = 16 * (i % (ldq / 16));
            *reinterpret_cast<uint4 *>(Q + q_index(m, k0, kst)) = make_uint4(0u, 0u, 0u, 0u);
        }
}

/* p2_swish on a flat array in place (tensor_ops.c:437-491): elements below the last multiple of eight as silu_p2,
 * the tail as x · p2_sigmoid(x) (expf clamped at 87, phonon2.h:38-46). */
__global__ __launch_bounds__(256) void silu_flat(size_t n, float *__restrict__ x)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    if (i < n / 8 * 8) x[i] = silu_p2(v);
    else x[i] = __fmul_rn(v, __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(v < -87.0f ? 87.0f : -v))));
}

/* add_residual (encoder.c:252-275): x += alpha · y as the AVX2 route's fmadd(y, alpha, x). */
__global__ __launch_bounds__(256) void axpy_rows(size_t n, float alpha, const float *__restrict__ y,
                                                 float *__restrict__ x)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = __builtin_fmaf(y[i], alpha, x[i]);
}

/* ── the int8 GEMM ─────────────────────────────────────────────────────────────────────────────────────────── */

struct GemmArgs {
    int M, N, K;
    float alpha, beta;
    const int8_t *Q; int ldq; const float *a_scales;     /* quantised activations [M][ldq], row scales [M] */
    const uint8_t *signs; const uint8_t *flags;           /* five-value planes [K][N/4], [K][N/8] */
    const uint8_t *clo; const float *c1; const float *c2; /* per-column epilogue factors (c1_factor, c2_factor) */
    int c1_hi;                                            /* 1: c1 holds hi, the factor is hi·(1/127) (int8w) */
    const int8_t *B8; int ldb;                            /* int8 table [K][ldb] (MODE_Q8B) */
    float *C; int ldc; int c_vec4;                        /* fp32 output; c_vec4: ldc % 4 == 0 and C 16-B aligned */
    int c_wt;                                             /* 1: C is stored at device scope (DevScopeOut) */
    int32_t *acc1; int32_t *acc2; int ldacc;              /* OUT_ACC: raw sums */
    int tiles_n, tiles_m;                                 /* output tiles of the grid */
    int kq;                                               /* K rounded up to 128: Q columns that may be read */
    int splits, split_rows;                               /* K splits; rows per split (divides 1024) */
    int32_t *part;                                        /* split partials [planes][splits][M][N] */
    const uint8_t *rec;                                   /* five-value operand records (fv_repack4) */
    int units;                                            /* 128-row K units of the records: K rounded up / 128 */
    int kst;                                              /* 64-column steps per 16-row group of Q: ldq / 64 */
    int mg_last, ng_last;                                 /* last 16-row group of Q, last 16-column group of C */
    const uint8_t *warm; int warm_lines;                  /* 128-byte lines a later kernel reads, loaded meanwhile */
    int act;                                              /* small-M tiles: 1 stores silu_p2 of each output */
    int xcd_rows;                                         /* small-M tiles: 0, or the rows of an XCD grid (below) */
};

/* The fold's per-column factors (blas.c:1316-1336), made from the weight's lo and hi as the reference makes them:
 * int8w c1 = hi·(1/127) (c1 holds hi, c1_hi = 1); int8 two-plane c1 = lo (c1 holds lo) and c2 = hi − lo (c2 holds
 * hi); the int8-table route's c1 is its column scale. */
__device__ __forceinline__ float c1_factor(const GemmArgs &g, int n)
{
    const float v = g.c1[n];
    return g.c1_hi ? v * (1.0f / 127.0f) : v;
}
__device__ __forceinline__ float c2_factor(const GemmArgs &g, int n) { return g.c2[n] - g.c1[n]; }



/* Tile geometry. Weight columns n play the MFMA "row" role and activation rows m the "column" role, so each lane's
 * four accumulators are four consecutive n of one output row (a 16-byte store). WN × WM waves; each wave owns
 * FN × FM MFMA tiles of 16 × 16. */
template <int BM_, int BN_, int WM_, int WN_, int BK_>
struct Geo {
    static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
    static constexpr int BK = BK_;           /* K rows per LDS stage (divides 1024) */
    static constexpr int SB = BK + 16;       /* LDS row pitch: an odd number of 16-byte chunks, so 8 consecutive rows
                                                hit 8 different bank groups */
    static constexpr int NT = 64 * WM * WN;
    static constexpr int FN = BN / WN / 16, FM = BM / WM / 16;
    static constexpr int A_CHUNKS = BM * (BK / 16);      /* 16-byte chunks of an activation stage */
    static constexpr int A_PER = A_CHUNKS / NT;
    static constexpr int CGS = BN / 16;                   /* 16-column groups */
    static constexpr int B_UNITS = (BK / 4) * CGS;        /* (4-row quad, column group) units of a weight stage */
    static constexpr int B_PER = (B_UNITS + NT - 1) / NT;
    static constexpr int A_BYTES = BM * SB, B_BYTES = BN * SB;
    static constexpr int LDS_ONE = 2 * A_BYTES + 2 * B_BYTES;   /* single-plane modes */
    static_assert(A_CHUNKS % NT == 0, "activation chunks must divide among the threads");
    static_assert(NT % CGS == 0, "a thread's column group must not change between its units");
    static_assert(FN >= 1 && FM >= 1, "wave tile");
    static_assert(1024 % BK == 0 && BK % 64 == 0, "stage depth");
};


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

/* Rows 4rq..4rq+3 of a stage × columns 16·cg..16·cg+15 of a five-value tile into the code tile(s): column n,
 * rows 4rq..4rq+3 land as one dword at LDS row n, 16-byte chunk (rq/4) ^ (n/16 mod 8), dword rq mod 4. */
template <int MODE, int SB>
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
template <int SB>
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

/* Workgroup → (output tile, K split). Workgroups are dealt to the 8 XCDs round-robin; when the count divides by 8
 * the index is remapped so each XCD runs one contiguous range of logical tiles – the splits of a tile and the
 * column tiles of a row band share that XCD's L2. */
__device__ __forceinline__ void tile_of(const GemmArgs &g, int &tile_n, int &tile_m, int &split)
{
    const int nb = (int)gridDim.x;
    int b = (int)blockIdx.x;
    if ((nb & 7) == 0) b = (b & 7) * (nb >> 3) + (b >> 3);
    split = b % g.splits;
    const int t = b / g.splits;
    tile_n = t % g.tiles_n;
    tile_m = t / g.tiles_n;
}

/* The int8 five-value GEMM (sgemm_i8_worker, blas.c:1296-1370) for one output tile and one K split.
 *  Stage loop: branch-free global loads of stage t+1 (addresses clamped in bounds, out-of-range values replaced
 *  afterwards) are issued before the MFMAs of stage t and written to the other LDS buffer after them.
 *  Folding the int32 sums into fp32 (blas.c:1355-1366): with one split, per 1024-row block in registers (MULTI keeps
 *  the running sum when K > 1024); with SPLIT, each workgroup writes its int32 partial sums and fold_splits, the
 *  next kernel on the stream, adds them per block (exact in int32) and folds the blocks in order. */
template <class G, int MODE, int OUT, bool MULTI, bool SPLIT>
__global__ __launch_bounds__(G::NT, ((MODE == MODE_INT8 || MULTI || G::NT > 256 || 2 * (G::LDS_ONE + 2048) > 160 * 1024) ? 1 : 2))
void gemm_i8(GemmArgs g)
{
    constexpr bool TWO = (MODE == MODE_INT8);
    constexpr bool FOLD = OUT == OUT_F32 && !SPLIT;   /* this kernel folds into fp32 C itself */
    constexpr int FN = G::FN, FM = G::FM, BK = G::BK, SB = G::SB;
    __shared__ __attribute__((aligned(16))) int8_t sm[2 * G::A_BYTES + (TWO ? 4 : 2) * G::B_BYTES];
    auto smA = [&](int b) { return sm + b * G::A_BYTES; };
    auto smB = [&](int b) { return sm + 2 * G::A_BYTES + b * G::B_BYTES; };
    auto smT = [&](int b) { return sm + 2 * G::A_BYTES + ((TWO ? 2 : 0) + b) * G::B_BYTES; };

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wn = wave % G::WN, wm = wave / G::WN;
    int tile_n, tile_m, split;
    tile_of(g, tile_n, tile_m, split);
    const int n0 = tile_n * G::BN, m0 = tile_m * G::BM;
    const int M = g.M, N = g.N, K = g.K;
    const int k_begin = split * g.split_rows;
    const int k_end = min(K, k_begin + g.split_rows);
    const int nk = (k_end - k_begin + BK - 1) / BK;

    /* B producer: column group cg (fixed), quads rq0 + u·(NT/CGS) */
    const int cg = tid % G::CGS, rq0 = tid / G::CGS;
    const bool col_ok = n0 + 16 * cg < N;
    const int cgc = col_ok ? cg : 0;   /* clamped column group for addressing */

    uint32_t lo_tab[16];
    if (MODE == MODE_INT8W) {
#pragma unroll
        for (int j = 0; j < 16; j++) lo_tab[j] = i8w_lo_table(g.clo[n0 + 16 * cgc + j]);
    }

    v4i acc[FN][FM], accT[TWO ? FN : 1][TWO ? FM : 1];
    float run[FOLD ? FN : 1][FOLD ? FM : 1][4];   /* fp32 outputs; with MULTI the running sum over K blocks */
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
        for (int j = 0; j < FM; j++) {
            acc[i][j] = v4i{0, 0, 0, 0};
            if (TWO) accT[TWO ? i : 0][TWO ? j : 0] = v4i{0, 0, 0, 0};
        }

    /* epilogue geometry of this lane: outputs (m_lane + 16 j, n_lane + 16 i + r) */
    const int n_lane = n0 + wn * (G::BN / G::WN) + 4 * (lane >> 4);
    const int m_lane = m0 + wm * (G::BM / G::WM) + (lane & 15);
    const bool beta_zero = g.beta == 0.0f;

    /* Epilogue factors of the tile – c1 (and c2) of its BN columns, as = a_scale·alpha of its BM rows – are loaded
     * into registers here, written to LDS with stage 0 and read from LDS by the fold, so no epilogue wait involves
     * the vector-memory counter that the C stores occupy. */
    static_assert(G::NT >= G::BN && G::NT >= G::BM, "one factor per thread");
    __shared__ __attribute__((aligned(16))) float f_c1[FOLD ? G::BN : 4], f_c2[FOLD && TWO ? G::BN : 4],
        f_as[FOLD ? G::BM : 4];
    float r_c1 = 0.0f, r_c2 = 0.0f, r_as = 0.0f;
    if (FOLD) {
        if (tid < G::BN) {
            const int n = min(n0 + tid, N - 1);
            r_c1 = c1_factor(g, n);
            if (TWO) r_c2 = c2_factor(g, n);
        }
        if (tid < G::BM) r_as = g.a_scales[min(m0 + tid, M - 1)] * g.alpha;
    }
    auto put_factors = [&]() {
        if (FOLD) {
            if (tid < G::BN) {
                f_c1[tid] = r_c1;
                if (TWO) f_c2[tid] = r_c2;
            }
            if (tid < G::BM) f_as[tid] = r_as;
        }
    };

    /* Per-lane byte offsets of this thread's loads, fixed for the whole K loop: a stage adds a uniform base, so the
     * loads address as (scalar base + 32-bit lane offset). */
    uint32_t a_off[G::A_PER], s_off[G::B_PER][4], f_off[G::B_PER][4], b8_off[G::B_PER][4];
#pragma unroll
    for (int i = 0; i < G::A_PER; i++) {
        const int c = tid + i * G::NT;
        const int row = c / (BK / 16), kc = c % (BK / 16);   /* row of the tile, 16-byte column chunk of the stage */
        a_off[i] = (uint32_t)(((row >> 4) * g.kst + (kc >> 2)) * 1024 + (((kc & 3) << 4) + (row & 15)) * 16);
    }
#pragma unroll
    for (int u = 0; u < G::B_PER; u++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = 4 * (rq0 + u * (G::NT / G::CGS)) + r;
            s_off[u][r] = (uint32_t)(row * (N / 4) + 4 * cgc);
            f_off[u][r] = (uint32_t)(row * (N / 8) + 2 * cgc);
            b8_off[u][r] = (uint32_t)(row * g.ldb + 16 * cgc);
        }

    uint4 ra[G::A_PER];
    uint32_t rs[G::B_PER][4], rf[G::B_PER][4];
    uint4 rb[G::B_PER][4];

    /* Interior tiles (every row, column and K row in range) run without any bounds arithmetic; edge tiles clamp
     * every address in bounds and mask the out-of-range values when they are written to LDS. Either way no load is
     * conditional, and none is waited on before the MFMAs of the current stage are issued. */
    const bool interior = m0 + G::BM <= M && n0 + G::BN <= N && (k_end - k_begin) % BK == 0;

    /* Fold one 1024-row K block into the lane's outputs (blas.c:1355-1366): f = (float)accS · c1 (+ fmaf((float)accT,
     * c2, f)); block 0 gives f · as (beta 0) or fmaf(f, as, beta-scaled C), later blocks fmaf(f, as, running). The
     * beta reads of C are the only global accesses and are issued before any store of this workgroup. */
    int block = 0;
    auto fold = [&](int blk) __attribute__((always_inline)) {
        const bool first = blk == 0;
#pragma unroll
        for (int i = 0; i < FN; i++) {
            const int nl = wn * (G::BN / G::WN) + 16 * i + 4 * (lane >> 4);
            const v4f c1 = *reinterpret_cast<const v4f *>(f_c1 + nl);
            v4f c2 = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            if (TWO) c2 = *reinterpret_cast<const v4f *>(f_c2 + nl);
            float cold[FM][4];
            if (first && !beta_zero) {
#pragma unroll
                for (int j = 0; j < FM; j++) {
                    const int n = min(n_lane + 16 * i, N - 4), m = min(m_lane + 16 * j, M - 1);
                    const float *cp = g.C + (size_t)m * g.ldc + n;
                    if (g.c_vec4) {
                        const v4f v = *reinterpret_cast<const v4f *>(cp);
                        cold[j][0] = v[0]; cold[j][1] = v[1]; cold[j][2] = v[2]; cold[j][3] = v[3];
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; r++) cold[j][r] = cp[r];
                    }
                }
                if (g.beta != 1.0f) {
#pragma unroll
                    for (int j = 0; j < FM; j++)
#pragma unroll
                        for (int r = 0; r < 4; r++) cold[j][r] = cold[j][r] * g.beta;
                }
            }
#pragma unroll
            for (int j = 0; j < FM; j++) {
                const float as = f_as[wm * (G::BM / G::WM) + 16 * j + (lane & 15)];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float f = (float)acc[i][j][r] * c1[r];
                    if (TWO) f = __builtin_fmaf((float)accT[TWO ? i : 0][TWO ? j : 0][r], c2[r], f);
                    const float prev = first ? cold[j][r] : run[FOLD ? i : 0][FOLD ? j : 0][r];
                    run[FOLD ? i : 0][FOLD ? j : 0][r] = (first && beta_zero) ? f * as : __builtin_fmaf(f, as, prev);
                }
                acc[i][j] = v4i{0, 0, 0, 0};
                if (TWO) accT[TWO ? i : 0][TWO ? j : 0] = v4i{0, 0, 0, 0};
            }
        }
    };

    auto body = [&](auto edge_tag) {
        constexpr bool EDGE = decltype(edge_tag)::value;
        auto load_stage = [&](int t) {
            const int k0 = k_begin + t * BK;
            if (!EDGE) {
                const int8_t *qk = g.Q + ((size_t)(m0 >> 4) * g.kst + (k0 >> 6)) * 1024;
#pragma unroll
                for (int i = 0; i < G::A_PER; i++) ra[i] = *reinterpret_cast<const uint4 *>(qk + a_off[i]);
                const uint8_t *sk = g.signs + (size_t)k0 * (N / 4) + n0 / 4;
                const uint8_t *fk = g.flags + (size_t)k0 * (N / 8) + n0 / 8;
                const int8_t *bk = g.B8 + (size_t)k0 * g.ldb + n0;
#pragma unroll
                for (int u = 0; u < G::B_PER; u++) {
                    if (G::B_UNITS % G::NT != 0 && rq0 + u * (G::NT / G::CGS) >= BK / 4) break;
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        if (MODE == MODE_Q8B) {
                            rb[u][r] = *reinterpret_cast<const uint4 *>(bk + b8_off[u][r]);
                        } else {
                            rs[u][r] = *reinterpret_cast<const uint32_t *>(sk + s_off[u][r]);
                            rf[u][r] = *reinterpret_cast<const uint16_t *>(fk + f_off[u][r]);
                        }
                    }
                }
                return;
            }
#pragma unroll
            for (int i = 0; i < G::A_PER; i++) {
                const int c = tid + i * G::NT;
                const int mc = min(m0 + c / (BK / 16), M - 1);
                const int kc = min(k0 + 16 * (c % (BK / 16)), g.kq - 16);
                ra[i] = *reinterpret_cast<const uint4 *>(g.Q + q_index(mc, kc, g.kst));
            }
#pragma unroll
            for (int u = 0; u < G::B_PER; u++) {
                const int rq = rq0 + u * (G::NT / G::CGS);
                if (G::B_UNITS % G::NT != 0 && rq >= BK / 4) break;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int kc = min(k0 + 4 * rq + r, K - 1);
                    if (MODE == MODE_Q8B) {
                        rb[u][r] = *reinterpret_cast<const uint4 *>(g.B8 + (size_t)kc * g.ldb + n0 + 16 * cgc);
                    } else {
                        rs[u][r] = *reinterpret_cast<const uint32_t *>(g.signs + (size_t)kc * (N / 4) + n0 / 4 + 4 * cgc);
                        rf[u][r] = *reinterpret_cast<const uint16_t *>(g.flags + (size_t)kc * (N / 8) + n0 / 8 + 2 * cgc);
                    }
                }
            }
        };
        auto store_stage = [&](int t, int buf) {
            const int k0 = k_begin + t * BK;
#pragma unroll
            for (int i = 0; i < G::A_PER; i++) {
                const int c = tid + i * G::NT;
                uint4 v = ra[i];
                if (EDGE) {
                    const bool ok = m0 + c / (BK / 16) < M && k0 + 16 * (c % (BK / 16)) < g.kq;
                    v = ok ? v : make_uint4(0, 0, 0, 0);
                }
                *reinterpret_cast<uint4 *>(smA(buf) + (c / (BK / 16)) * SB + 16 * (c % (BK / 16))) = v;
            }
#pragma unroll
            for (int u = 0; u < G::B_PER; u++) {
                const int rq = rq0 + u * (G::NT / G::CGS);
                if (G::B_UNITS % G::NT != 0 && rq >= BK / 4) break;
                if (MODE == MODE_Q8B) {
                    uint4 v[4];
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const bool ok = !EDGE || (col_ok && k0 + 4 * rq + r < k_end);
                        v[r] = ok ? rb[u][r] : make_uint4(0, 0, 0, 0);
                    }
                    store_q8_codes<SB>(v, smB(buf), cg, rq);
                } else {
                    uint32_t sv[4], fv[4];
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const bool ok = !EDGE || (col_ok && k0 + 4 * rq + r < k_end);
                        sv[r] = ok ? rs[u][r] : 0x55555555u;   /* code 1 everywhere: zero weights */
                        fv[r] = ok ? rf[u][r] : 0u;
                    }
                    store_fv_codes<MODE, SB>(sv, fv, lo_tab, smB(buf), smT(buf), cg, rq);
                }
            }
        };

        if (nk > 0) {
            load_stage(0);
            store_stage(0, 0);
        }
        put_factors();
        __syncthreads();

        for (int t = 0; t < nk; t++) {
            const int buf = t & 1;
            if (t + 1 < nk) load_stage(t + 1);
            const int8_t *tA = smA(buf), *tB = smB(buf), *tT = smT(buf);
#pragma unroll
            for (int kk = 0; kk < BK; kk += 64) {
                const int g16 = (kk >> 4) + (lane >> 4);   /* this lane's 16-byte chunk along k */
                v4i a[FN], b[FM], bt[TWO ? FN : 1];
#pragma unroll
                for (int i = 0; i < FN; i++) {
                    const int nl = wn * (G::BN / G::WN) + 16 * i + (lane & 15);
                    const int off = nl * SB + 16 * (g16 ^ ((nl >> 4) & 7));
                    a[i] = *reinterpret_cast<const v4i *>(tB + off);
                    if (TWO) bt[TWO ? i : 0] = *reinterpret_cast<const v4i *>(tT + off);
                }
#pragma unroll
                for (int j = 0; j < FM; j++) {
                    const int ml = wm * (G::BM / G::WM) + 16 * j + (lane & 15);
                    b[j] = *reinterpret_cast<const v4i *>(tA + ml * SB + 16 * g16);
                }
#pragma unroll
                for (int i = 0; i < FN; i++)
#pragma unroll
                    for (int j = 0; j < FM; j++) {
                        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
                        if (TWO)
                            accT[TWO ? i : 0][TWO ? j : 0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                                bt[TWO ? i : 0], b[j], accT[TWO ? i : 0][TWO ? j : 0], 0, 0, 0);
                    }
            }
            if (t + 1 < nk) store_stage(t + 1, buf ^ 1);
            if (FOLD && MULTI && t + 1 < nk && ((t + 1) * BK) % kFoldRows == 0) {
                fold(block);
                block++;
            }
            __syncthreads();
        }
    };
    if (interior) body(std::false_type{});
    else body(std::true_type{});

    if (FOLD) {
        if (nk == 0) return;
        fold(block);
        /* every output of the lane is final: one burst of 16-byte stores, nothing waited on after it */
        if (g.c_vec4) {
#pragma unroll
            for (int i = 0; i < FN; i++)
#pragma unroll
                for (int j = 0; j < FM; j++) {
                    const int n = n_lane + 16 * i, m = m_lane + 16 * j;
                    if (m < M && n < N)
                        *reinterpret_cast<v4f *>(g.C + (size_t)m * g.ldc + n) =
                            v4f{run[i][j][0], run[i][j][1], run[i][j][2], run[i][j][3]};
                }
        } else {
#pragma unroll
            for (int i = 0; i < FN; i++)
#pragma unroll
                for (int j = 0; j < FM; j++) {
                    const int n = n_lane + 16 * i, m = m_lane + 16 * j;
                    if (m < M && n < N) {
                        float *cp = g.C + (size_t)m * g.ldc + n;
#pragma unroll
                        for (int r = 0; r < 4; r++) cp[r] = run[i][j][r];
                    }
                }
        }
        return;
    }

    if (OUT == OUT_ACC) {
#pragma unroll
        for (int i = 0; i < FN; i++)
#pragma unroll
            for (int j = 0; j < FM; j++) {
                const int n = n_lane + 16 * i, m = m_lane + 16 * j;
                if (m < M && n < N) {
                    *reinterpret_cast<v4i *>(g.acc1 + (size_t)m * g.ldacc + n) = acc[i][j];
                    if (TWO) *reinterpret_cast<v4i *>(g.acc2 + (size_t)m * g.ldacc + n) = accT[TWO ? i : 0][TWO ? j : 0];
                }
            }
        return;
    }

    if (SPLIT) {   /* int32 partial sums of this split; fold_splits adds and folds them */
        const size_t plane = (size_t)g.splits * M * N;
#pragma unroll
        for (int i = 0; i < FN; i++)
#pragma unroll
            for (int j = 0; j < FM; j++) {
                const int n = n_lane + 16 * i, m = m_lane + 16 * j;
                if (m < M && n < N) {
                    int32_t *p = g.part + ((size_t)split * M + m) * N + n;
                    *reinterpret_cast<v4i *>(p) = acc[i][j];
                    if (TWO) *reinterpret_cast<v4i *>(p + plane) = accT[TWO ? i : 0][TWO ? j : 0];
                }
            }
    }
}

/* ── the five-value GEMM on operand records ──────────────────────────────────────────────────────────────────── */

/* Five-value planes → 4-bit selector records, the weight operand of every GEMM route. Record (column group cg, unit
 * u) holds 16 bytes per lane l, which serves column n = 16·cg + l % 16 and rows k = 128·u + 64·s + 16·(l / 16) +
 * 4·d + b (s = 0, 1: the two 64-row steps of the unit; d, b = 0..3): dword 2s + d/2, byte b, nibble d % 2 is the
 * byte-permute selector code | flag << 2 of row k. Rows k >= K hold code 1 (weight 0). Records are stored
 * [N/16][units][64][16 B], so a 16-column group streams along K. Half a byte per weight: one 16-byte load per lane
 * brings a whole 128-row unit, and an operand dword decodes with one mask (and one shift for odd d) before the
 * table permute. */
__global__ void fv_repack4(int K, int N, int units, const uint8_t *__restrict__ signs,
                           const uint8_t *__restrict__ flags, uint4 *__restrict__ rec)
{
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)(N / 16) * units * 64) return;
    const int l = (int)(idx % 64);
    const size_t gu = idx / 64;
    const int u = (int)(gu % units), cg = (int)(gu / units);
    const int n = 16 * cg + (l & 15), kq = l >> 4;
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    for (int s = 0; s < 2; s++)
        for (int d = 0; d < 4; d++)
            for (int b = 0; b < 4; b++) {
                const int k = 128 * u + 64 * s + 16 * kq + 4 * d + b;
                uint32_t code = 1u, flag = 0u;
                if (k < K) {
                    code = (signs[(size_t)k * (N / 4) + (n >> 2)] >> (2 * (n & 3))) & 3u;
                    flag = (flags[(size_t)k * (N / 8) + (n >> 3)] >> (n & 7)) & 1u;
                }
                w[2 * s + (d >> 1)] |= (code | (flag << 2)) << (8 * b + 4 * (d & 1));
            }
    rec[idx] = make_uint4(w[0], w[1], w[2], w[3]);
}

/* The selector nibble (code | flag << 2, fv_repack4's layout) of weight (k, n) lives in record (n / 16, k / 128),
 * lane 16·((k % 64) / 16) + n % 16, dword 2·((k % 128) / 64) + (k % 16) / 8, byte k % 4, nibble ((k % 16) / 4) % 2;
 * the four rows of a quad 4·q .. 4·q + 3 are the four bytes of one dword. This is that dword's byte offset in the
 * records and the nibble's shift within each byte. */
__device__ __forceinline__ size_t rec_quad_offset(int units, int k, int n, int &shift)
{
    const int u = k >> 7, s = (k >> 6) & 1, q = (k >> 4) & 3, d = (k >> 2) & 3;
    shift = 4 * (d & 1);
    return (((size_t)(n >> 4) * units + u) * 64 + 16 * q + (n & 15)) * 16 + 4 * (2 * s + (d >> 1));
}

template <int FM_, int FN_, int NW_, int D_>
struct FvGeo {
    static constexpr int FM = FM_, FN = FN_, NW = NW_, D = D_;
    static constexpr int NT = 64 * NW;
    static constexpr int BM = 16 * FM, BN = 16 * FN * NW;
    static constexpr int A_STAGE = 2 * FM * 1024;   /* FM row groups × two 64-row steps of activation operands */
    static constexpr int B_STAGE = FN * NW * 1024;  /* one weight record per 16-column group: 64 lanes × 16-B slots */
    static constexpr int STAGE = A_STAGE + B_STAGE;
    static constexpr int A_DMA = 2 * FM / NW;       /* activation DMAs per wave per stage */
    static constexpr int DMA = A_DMA + FN;          /* DMAs per wave per stage */
    static_assert((2 * FM) % NW == 0, "activation operands divide among the waves");
    static_assert(FN <= 4 && FM <= 16, "epilogue factors: one column and one row per thread");
    static_assert(D >= 2 && D * STAGE <= 160 * 1024, "LDS ring");
};

/* The int8 five-value GEMM (sgemm_i8_worker, blas.c:1296-1370) on operand records.
 *  A workgroup of NW waves owns a BM × BN output tile; wave w owns its FN 16-column groups for all FM 16-row groups,
 *  so each weight operand is decoded exactly once per workgroup, in registers, and feeds FM MFMAs.
 *  Operands stream through a ring of D LDS stages (two 64-row steps each) by direct global→LDS loads: stage t + D − 1
 *  is requested while stage t is computed, with one barrier per stage and no register staging.
 *  Folding into fp32 is as in gemm_i8: per 1024-row block in registers, or int32 partials per split for fold_splits. */
template <class G, int MODE, int OUT, bool MULTI, bool SPLIT, int OCC, bool CSHUF>
__device__ __forceinline__ void fv_tile(const GemmArgs &g)
{
    constexpr bool TWO = (MODE == MODE_INT8);
    constexpr bool FOLD = OUT == OUT_F32 && !SPLIT;
    constexpr int FM = G::FM, FN = G::FN, D = G::D, STAGE = G::STAGE;
    constexpr int UNITS_PER_FOLD = kFoldRows / 128;
    __shared__ __attribute__((aligned(16))) int8_t ring[D * STAGE];
    __shared__ __attribute__((aligned(16))) float f_c1[FOLD ? G::BN : 4], f_c2[FOLD && TWO ? G::BN : 4],
        f_as[FOLD ? G::BM : 4];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int tile_n, tile_m, split;
    tile_of(g, tile_n, tile_m, split);
    const int n0 = tile_n * G::BN, m0 = tile_m * G::BM;
    const int M = g.M, N = g.N;
    const int split_units = (g.split_rows + 127) / 128;
    const int u_begin = split * split_units;
    const int nst = max(0, min(g.units, u_begin + split_units) - u_begin);

    /* DMA sources of this lane (row and column groups clamped into the padded operands; their outputs are masked) */
    const int8_t *a_src[G::A_DMA];
    int a_dst[G::A_DMA];
#pragma unroll
    for (int q = 0; q < G::A_DMA; q++) {
        const int f = wave + q * G::NW;            /* operand f = 2·j + s of the stage */
        const int mg = min((m0 >> 4) + (f >> 1), g.mg_last);
        a_src[q] = g.Q + ((size_t)mg * g.kst + 2 * u_begin + (f & 1)) * 1024 + lane * 16;
        a_dst[q] = f * 1024;
    }
    const uint8_t *b_src[FN];
    uint32_t lo_tab[FN];
#pragma unroll
    for (int i = 0; i < FN; i++) {
        const int cg = min((n0 >> 4) + wave * FN + i, g.ng_last);
        b_src[i] = g.rec + ((size_t)cg * g.units + u_begin) * 1024 + lane * 16;
        if (MODE == MODE_INT8W) lo_tab[i] = i8w_lo_table(g.clo[16 * cg + (lane & 15)]);
    }
    auto issue = [&](int t) {   /* stage t → ring slot t % D */
        int8_t *slot = ring + (t % D) * STAGE;
#pragma unroll
        for (int q = 0; q < G::A_DMA; q++) dma_16(a_src[q] + (size_t)t * 2048, slot + a_dst[q]);
#pragma unroll
        for (int i = 0; i < FN; i++) {
            dma_16(b_src[i] + (size_t)t * 1024, slot + G::A_STAGE + (wave * FN + i) * 1024);
        }
    };
    /* epilogue factors: loaded before the first DMAs (so waiting for them waits for no DMA), into LDS before the
     * first barrier */
    float r_c1 = 0.0f, r_c2 = 0.0f, r_as = 0.0f;
    if (FOLD) {
        if (tid < G::BN) {
            const int n = min(n0 + tid, N - 1);
            r_c1 = c1_factor(g, n);
            if (TWO) r_c2 = c2_factor(g, n);
        }
        if (tid < G::BM) r_as = g.a_scales[min(m0 + tid, M - 1)];
    }
#pragma unroll
    for (int t = 0; t < D - 1; t++)
        if (t < nst) issue(t);
    if (FOLD) {
        r_as *= g.alpha;
        if (tid < G::BN) {
            f_c1[tid] = r_c1;
            if (TWO) f_c2[tid] = r_c2;
        }
        if (tid < G::BM) f_as[tid] = r_as;
    }

    v4i acc[FN][FM], accT[TWO ? FN : 1][TWO ? FM : 1];
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
        for (int j = 0; j < FM; j++) {
            acc[i][j] = v4i{0, 0, 0, 0};
            if (TWO) accT[TWO ? i : 0][TWO ? j : 0] = v4i{0, 0, 0, 0};
        }

    const int n_lane = n0 + wave * 16 * FN + 4 * (lane >> 4);   /* outputs (m_lane + 16 j, n_lane + 16 i + r) */
    const int m_lane = m0 + (lane & 15);
    const bool beta_zero = g.beta == 0.0f;
    float run[FOLD ? FN : 1][FOLD ? FM : 1][4];
    int block = 0;
    /* CASE 0: block 0 with beta 0 (f·as); 1: block 0 with beta-scaled C (fmaf(f, as, β·C)); 2: a later block
     * (fmaf(f, as, running)). Each case is straight-line code, selected by a uniform branch. */
    auto fold_case = [&](auto case_tag) __attribute__((always_inline)) {
        constexpr int CASE = decltype(case_tag)::value;
#pragma unroll
        for (int i = 0; i < FN; i++) {
            const int nl = wave * 16 * FN + 16 * i + 4 * (lane >> 4);
            const v4f c1 = *reinterpret_cast<const v4f *>(f_c1 + nl);
            v4f c2 = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            if (TWO) c2 = *reinterpret_cast<const v4f *>(f_c2 + nl);
            float cold[CASE == 1 ? FM : 1][4];
            if (CASE == 1) {
#pragma unroll
                for (int j = 0; j < FM; j++) {
                    const int n = min(n_lane + 16 * i, N - 4), m = min(m_lane + 16 * j, M - 1);
                    const float *cp = g.C + (size_t)m * g.ldc + n;
                    if (g.c_vec4) {
                        const v4f v = *reinterpret_cast<const v4f *>(cp);
                        cold[CASE == 1 ? j : 0][0] = v[0]; cold[CASE == 1 ? j : 0][1] = v[1];
                        cold[CASE == 1 ? j : 0][2] = v[2]; cold[CASE == 1 ? j : 0][3] = v[3];
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; r++) cold[CASE == 1 ? j : 0][r] = cp[r];
                    }
                }
                if (g.beta != 1.0f) {
#pragma unroll
                    for (int j = 0; j < FM; j++)
#pragma unroll
                        for (int r = 0; r < 4; r++) cold[CASE == 1 ? j : 0][r] = cold[CASE == 1 ? j : 0][r] * g.beta;
                }
            }
#pragma unroll
            for (int j = 0; j < FM; j++) {
                const float as = f_as[16 * j + (lane & 15)];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float f = (float)acc[i][j][r] * c1[r];
                    if (TWO) f = __builtin_fmaf((float)accT[TWO ? i : 0][TWO ? j : 0][r], c2[r], f);
                    float &out = run[FOLD ? i : 0][FOLD ? j : 0][r];
                    if (CASE == 0) out = f * as;
                    else if (CASE == 1) out = __builtin_fmaf(f, as, cold[CASE == 1 ? j : 0][r]);
                    else out = __builtin_fmaf(f, as, out);
                }
                acc[i][j] = v4i{0, 0, 0, 0};
                if (TWO) accT[TWO ? i : 0][TWO ? j : 0] = v4i{0, 0, 0, 0};
            }
        }
    };
    auto fold = [&](int blk) __attribute__((always_inline)) {
        if (blk > 0) fold_case(std::integral_constant<int, 2>{});
        else if (beta_zero) fold_case(std::integral_constant<int, 0>{});
        else fold_case(std::integral_constant<int, 1>{});
    };

    for (int t = 0; t < nst; t++) {
        /* this wave's DMAs of stage t have landed (D − 2 younger stages may still be in flight) ... */
        if (t + D - 2 < nst) wait_vm<G::DMA * (D - 2)>();
        else wait_vm<0>();
        /* ... and every wave's; every wave is also done reading the slot that stage t + D − 1 reuses */
        lds_barrier();
        if (t + D - 1 < nst) issue(t + D - 1);

        const int8_t *sa = ring + (t % D) * STAGE;
        const int8_t *sb = sa + G::A_STAGE + (wave * FN) * 1024 + lane * 16;
        /* all LDS reads of the stage first: FN weight records, 2·FM activation operands */
        uint32_t rw[FN][4];
#pragma unroll
        for (int i = 0; i < FN; i++) {
            const uint4 v = *reinterpret_cast<const uint4 *>(sb + i * 1024);
            rw[i][0] = v.x; rw[i][1] = v.y; rw[i][2] = v.z; rw[i][3] = v.w;
        }
        v4i av[2][FM];
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
            for (int j = 0; j < FM; j++)
                av[s2][j] = *reinterpret_cast<const v4i *>(sa + (2 * j + s2) * 1024 + lane * 16);
        /* weight operands of both 64-row steps */
        v4i bw[2][FN], bt[2][TWO ? FN : 1];
        auto decode = [&](auto step_tag) __attribute__((always_inline)) {
            constexpr int S = decltype(step_tag)::value;
#pragma unroll
            for (int i = 0; i < FN; i++)
#pragma unroll
                for (int d = 0; d < 4; d++) {
                    const uint32_t sel = (rw[i][2 * S + (d >> 1)] >> (4 * (d & 1))) & 0x07070707u;
                    if (MODE == MODE_INT8W) {
                        bw[S][i][d] = (int)perm(kI8wHiTable, lo_tab[i], sel);
                    } else {
                        bw[S][i][d] = (int)perm(kPlaneS, kPlaneS, sel);
                        bt[S][TWO ? i : 0][d] = (int)perm(kPlaneS, 0u, sel);
                    }
                }
        };
        auto mma = [&](auto step_tag) __attribute__((always_inline)) {
            constexpr int S = decltype(step_tag)::value;
#pragma unroll
            for (int j = 0; j < FM; j++)
#pragma unroll
                for (int i = 0; i < FN; i++) {
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw[S][i], av[S][j], acc[i][j], 0, 0, 0);
                    if (TWO)
                        accT[TWO ? i : 0][TWO ? j : 0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            bt[S][TWO ? i : 0], av[S][j], accT[TWO ? i : 0][TWO ? j : 0], 0, 0, 0);
                }
        };
        decode(std::integral_constant<int, 0>{});
        mma(std::integral_constant<int, 0>{});
        decode(std::integral_constant<int, 1>{});
        mma(std::integral_constant<int, 1>{});
        /* Issue order for the scheduler: the LDS reads, the step-0 decode, then step 0's MFMAs each followed by a
         * share of the step-1 decode (which the matrix cores' latency hides), then step 1's MFMAs. */
        constexpr int N_MFMA = FM * FN * (TWO ? 2 : 1);
        /* One step's decode is, per dword, an and, a perm and half a shift (int8w; the two-plane mode a perm more).
         * With four column groups per wave the scheduler gets exactly step 0's decode ahead of the first MFMA and
         * spreads step 1's over step 0's MFMAs (M = 1500 and 3000, 1024 → 4096: 4 % faster); with two, both steps'
         * decode goes first, which measured faster for 96 × 128 at K = 4096 (31.0 against 32.4 µs). */
        constexpr int DEC_VALU = FN >= 4 ? FN * 4 * (TWO ? 7 : 5) / 2 : FN * 4 * (TWO ? 6 : 5);
        constexpr int PER = (DEC_VALU + N_MFMA - 1) / N_MFMA;
        __builtin_amdgcn_sched_group_barrier(0x100, 3 * FN + 2 * FM, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, DEC_VALU, 0);
#pragma unroll
        for (int x = 0; x < N_MFMA; x++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, PER, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, N_MFMA, 0);
        if (FOLD && MULTI && t + 1 < nst && (t + 1) % UNITS_PER_FOLD == 0) {
            fold(block);
            block++;
        }
    }

    if (OUT == OUT_ACC) {
#pragma unroll
        for (int i = 0; i < FN; i++)
#pragma unroll
            for (int j = 0; j < FM; j++) {
                const int n = n_lane + 16 * i, m = m_lane + 16 * j;
                if (m < M && n < N) {
                    *reinterpret_cast<v4i *>(g.acc1 + (size_t)m * g.ldacc + n) = acc[i][j];
                    if (TWO) *reinterpret_cast<v4i *>(g.acc2 + (size_t)m * g.ldacc + n) = accT[TWO ? i : 0][TWO ? j : 0];
                }
            }
        return;
    }
    if (SPLIT) {   /* int32 partial sums of this split; fold_splits adds and folds them */
        const size_t plane = (size_t)g.splits * M * N;
#pragma unroll
        for (int i = 0; i < FN; i++)
#pragma unroll
            for (int j = 0; j < FM; j++) {
                const int n = n_lane + 16 * i, m = m_lane + 16 * j;
                if (m < M && n < N) {
                    int32_t *p = g.part + ((size_t)split * M + m) * N + n;
                    *reinterpret_cast<v4i *>(p) = acc[i][j];
                    if (TWO) *reinterpret_cast<v4i *>(p + plane) = accT[TWO ? i : 0][TWO ? j : 0];
                }
            }
        return;
    }
    if (nst == 0) return;
    fold(block);
    if (CSHUF) {
        /* The outputs are staged through the ring (idle once the last stage is read) and stored as whole row
         * segments: the matrix-core layout alone gives 16 rows × 64 bytes per store, which streams C to HBM at
         * about two thirds of the rate of full row segments. Chunks of CJ row groups, padded rows. */
        constexpr int SROW = G::BN + 4;
        constexpr int CJF = (D * STAGE) / (16 * SROW * 4);
        constexpr int CJ = CJF < FM ? CJF : FM;
        static_assert(CJ >= 1, "staging chunk");
        constexpr int LPR = G::BN / 4;   /* lanes per staged row */
        constexpr int RPI = 64 / LPR;    /* rows per store instruction */
        static_assert(64 % LPR == 0, "row segments per wave");
        float *stg = reinterpret_cast<float *>(ring);
        const int lr = lane / LPR, lc = lane % LPR;
        const DevScopeOut cout(g.C + (size_t)m0 * g.ldc, (size_t)min(G::BM, M - m0) * g.ldc * 4, g.c_wt);
        lds_barrier();
#pragma unroll
        for (int j0 = 0; j0 < FM; j0 += CJ) {
#pragma unroll
            for (int j = j0; j < j0 + CJ && j < FM; j++)
#pragma unroll
                for (int i = 0; i < FN; i++) {
                    const int nl = wave * 16 * FN + 16 * i + 4 * (lane >> 4);
                    *reinterpret_cast<v4f *>(stg + (16 * (j - j0) + (lane & 15)) * SROW + nl) =
                        v4f{run[i][j][0], run[i][j][1], run[i][j][2], run[i][j][3]};
                }
            lds_barrier();
            const int rows = 16 * (min(j0 + CJ, FM) - j0);
            for (int r = wave * RPI + lr; r < rows; r += 4 * RPI) {
                const int m = m0 + 16 * j0 + r, n = n0 + 4 * lc;
                if (m < M && n < N) {
                    const v4f v = *reinterpret_cast<const v4f *>(stg + r * SROW + 4 * lc);
                    if (g.c_vec4) {
                        cout.st16(((size_t)(m - m0) * g.ldc + n) * 4, v);
                    } else {
                        float *cp = g.C + (size_t)m * g.ldc + n;
                        cp[0] = v[0]; cp[1] = v[1]; cp[2] = v[2]; cp[3] = v[3];
                    }
                }
            }
            if (j0 + CJ < FM) lds_barrier();
        }
        return;
    }
    /* every output of the lane is final: one burst of 16-byte stores, nothing waited on after it */
    if (g.c_vec4) {
#pragma unroll
        for (int i = 0; i < FN; i++)
#pragma unroll
            for (int j = 0; j < FM; j++) {
                const int n = n_lane + 16 * i, m = m_lane + 16 * j;
                if (m < M && n < N)
                    *reinterpret_cast<v4f *>(g.C + (size_t)m * g.ldc + n) =
                        v4f{run[i][j][0], run[i][j][1], run[i][j][2], run[i][j][3]};
            }
    } else {
#pragma unroll
        for (int i = 0; i < FN; i++)
#pragma unroll
            for (int j = 0; j < FM; j++) {
                const int n = n_lane + 16 * i, m = m_lane + 16 * j;
                if (m < M && n < N) {
                    float *cp = g.C + (size_t)m * g.ldc + n;
#pragma unroll
                    for (int r = 0; r < 4; r++) cp[r] = run[i][j][r];
                }
            }
    }
}

/* The large-M int8w tiles with the weight records in registers (gemm_fv_rb, the production large-M kernel).
 *  As fv_tile, except that each wave loads its own FN weight records of stage t + 1 straight into registers while
 *  stage t is computed (a wave is the only reader of its columns' records, so they need no LDS and no barrier), and
 *  decodes step 0 of stage t + 1 among stage t's step-1 MFMAs: a stage starts on MFMAs as soon as its first
 *  activation operands are read from LDS. Only the activation operands go through the LDS ring (direct loads, one
 *  barrier per stage). Against the records in LDS: M = 1500 11.3 against 12.4 µs, M = 4099 24.8 against 27.1,
 *  M = 6000 32.5 against 33.7 (1024 → 4096). Two workgroups per CU; the output is folded and staged as in
 *  fv_tile (per 1024-row block, in order; C staged through LDS as whole row segments at device scope). */
template <class G, bool MULTI>
__device__ __forceinline__ void fv_tile_rb(const GemmArgs &g)
{
    constexpr int FM = G::FM, FN = G::FN, NW = G::NW, D = G::D, A_STAGE = G::A_STAGE, A_DMA = G::A_DMA;
    constexpr int UNITS_PER_FOLD = kFoldRows / 128;
    constexpr int SROW = G::BN + 4;                    /* staged C rows, padded */
    constexpr int CJ = FM < 3 ? FM : 3;                /* row groups per staging chunk */
    constexpr int RING = D * A_STAGE, STG = 16 * CJ * SROW * 4;
    __shared__ __attribute__((aligned(16))) int8_t ring[RING > STG ? RING : STG];
    __shared__ __attribute__((aligned(16))) float f_c1[G::BN], f_as[G::BM];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int tile_n, tile_m, split;
    tile_of(g, tile_n, tile_m, split);
    const int n0 = tile_n * G::BN, m0 = tile_m * G::BM;
    const int M = g.M, N = g.N;
    const int nst = g.units;

    /* sources of this lane (row and column groups clamped into the padded operands; their outputs are masked) */
    const int8_t *a_src[A_DMA];
    int a_dst[A_DMA];
#pragma unroll
    for (int q = 0; q < A_DMA; q++) {
        const int f = wave + q * NW;               /* operand f = 2·j + s of the stage */
        const int mg = min((m0 >> 4) + (f >> 1), g.mg_last);
        a_src[q] = g.Q + ((size_t)mg * g.kst + (f & 1)) * 1024 + lane * 16;
        a_dst[q] = f * 1024;
    }
    const uint8_t *b_src[FN];
    uint32_t lo_tab[FN];
#pragma unroll
    for (int i = 0; i < FN; i++) {
        const int cg = min((n0 >> 4) + wave * FN + i, g.ng_last);
        b_src[i] = g.rec + (size_t)cg * g.units * 1024 + lane * 16;
        lo_tab[i] = i8w_lo_table(g.clo[16 * cg + (lane & 15)]);
    }
    /* stage t's slot (t % D) filled with stage ts's activation operands (ts = t but past the last stage) */
    auto issue_a = [&](int t, int ts) __attribute__((always_inline)) {
        int8_t *slot = ring + (t % D) * A_STAGE;
#pragma unroll
        for (int q = 0; q < A_DMA; q++) dma_16(a_src[q] + (size_t)ts * 2048, slot + a_dst[q]);
    };

    /* epilogue factors first (so that waiting for them waits for nothing else), then stage 0 */
    float r_c1 = 0.0f, r_as = 0.0f;
    if (tid < G::BN) r_c1 = c1_factor(g, min(n0 + tid, N - 1));
    if (tid < G::BM) r_as = g.a_scales[min(m0 + tid, M - 1)];
    v4u rb0[FN], rb1[FN];
#pragma unroll
    for (int i = 0; i < FN; i++) rb0[i] = load16_async(b_src[i]);
#pragma unroll
    for (int t = 0; t < D - 1; t++) issue_a(t, min(t, nst - 1));
    if (tid < G::BN) f_c1[tid] = r_c1;
    if (tid < G::BM) f_as[tid] = r_as * g.alpha;

    auto decode = [&](auto step_tag, const v4u(&rb)[FN], v4i(&bw)[FN]) __attribute__((always_inline)) {
        constexpr int S = decltype(step_tag)::value;
#pragma unroll
        for (int i = 0; i < FN; i++)
#pragma unroll
            for (int d = 0; d < 4; d++) {
                const uint32_t sel = (rb[i][2 * S + (d >> 1)] >> (4 * (d & 1))) & 0x07070707u;
                bw[i][d] = (int)perm(kI8wHiTable, lo_tab[i], sel);
            }
    };

    v4i acc[FN][FM];
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
        for (int j = 0; j < FM; j++) acc[i][j] = v4i{0, 0, 0, 0};
    const int n_lane = n0 + wave * 16 * FN + 4 * (lane >> 4);   /* outputs (m_lane + 16 j, n_lane + 16 i + r) */
    const int m_lane = m0 + (lane & 15);
    const bool beta_zero = g.beta == 0.0f;
    float run[FN][FM][4];
    int block = 0;
    /* CASE 0: block 0 with beta 0 (f·as); 1: block 0 with beta-scaled C (fmaf(f, as, β·C)); 2: a later block */
    auto fold_case = [&](auto case_tag) __attribute__((always_inline)) {
        constexpr int CASE = decltype(case_tag)::value;
#pragma unroll
        for (int i = 0; i < FN; i++) {
            const int nl = wave * 16 * FN + 16 * i + 4 * (lane >> 4);
            const v4f c1 = *reinterpret_cast<const v4f *>(f_c1 + nl);
            float cold[CASE == 1 ? FM : 1][4];
            if (CASE == 1) {
#pragma unroll
                for (int j = 0; j < FM; j++) {
                    const int n = min(n_lane + 16 * i, N - 4), m = min(m_lane + 16 * j, M - 1);
                    const float *cp = g.C + (size_t)m * g.ldc + n;
                    if (g.c_vec4) {
                        const v4f v = *reinterpret_cast<const v4f *>(cp);
                        cold[CASE == 1 ? j : 0][0] = v[0]; cold[CASE == 1 ? j : 0][1] = v[1];
                        cold[CASE == 1 ? j : 0][2] = v[2]; cold[CASE == 1 ? j : 0][3] = v[3];
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; r++) cold[CASE == 1 ? j : 0][r] = cp[r];
                    }
                }
                if (g.beta != 1.0f) {
#pragma unroll
                    for (int j = 0; j < FM; j++)
#pragma unroll
                        for (int r = 0; r < 4; r++) cold[CASE == 1 ? j : 0][r] = cold[CASE == 1 ? j : 0][r] * g.beta;
                }
            }
#pragma unroll
            for (int j = 0; j < FM; j++) {
                const float as = f_as[16 * j + (lane & 15)];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float f = (float)acc[i][j][r] * c1[r];
                    float &out = run[i][j][r];
                    if (CASE == 0) out = f * as;
                    else if (CASE == 1) out = __builtin_fmaf(f, as, cold[CASE == 1 ? j : 0][r]);
                    else out = __builtin_fmaf(f, as, out);
                }
                acc[i][j] = v4i{0, 0, 0, 0};
            }
        }
    };
    auto fold = [&](int blk) __attribute__((always_inline)) {
        if (blk > 0) fold_case(std::integral_constant<int, 2>{});
        else if (beta_zero) fold_case(std::integral_constant<int, 0>{});
        else fold_case(std::integral_constant<int, 1>{});
    };

    v4i bw0[FN], bw1[FN];
    wait_vm<0>();
#pragma unroll
    for (int i = 0; i < FN; i++) pin16(rb0[i]);
    decode(std::integral_constant<int, 0>{}, rb0, bw0);

    /* stage t: its records in rc (step 0 already decoded into bw0); the next stage's records into rn */
    /* Loads retire in order: waiting until at most the youngest (D − 2) stages of activation loads are in flight
     * leaves every older load landed. */
    auto stage = [&](int t, v4u(&rc)[FN], v4u(&rn)[FN]) __attribute__((always_inline)) {
        wait_vm<(D - 2) * A_DMA>();   /* this wave's loads of stage t landed (the records of t + 1 too) ... */
        lds_barrier();   /* ... every wave's; every wave is also done reading the slot stage t + D − 1 reuses */
        /* stage t + 1's records and stage t + D − 1's activation operands; past the last stage, the last stage's
         * again (in bounds, unused), so that the stage is straight-line code */
        const int tn = min(t + 1, nst - 1), ta = min(t + D - 1, nst - 1);
#pragma unroll
        for (int i = 0; i < FN; i++) rn[i] = load16_async(b_src[i] + (size_t)tn * 1024);
        issue_a(t + D - 1, ta);
        const int8_t *sa = ring + (t % D) * A_STAGE;
        v4i av[2][FM];
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
            for (int j = 0; j < FM; j++)
                av[s2][j] = *reinterpret_cast<const v4i *>(sa + (2 * j + s2) * 1024 + lane * 16);
        /* step 0's MFMAs with step 1's decode among them ... */
        decode(std::integral_constant<int, 1>{}, rc, bw1);
#pragma unroll
        for (int j = 0; j < FM; j++)
#pragma unroll
            for (int i = 0; i < FN; i++)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw0[i], av[0][j], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * FM, 0);
#pragma unroll
        for (int x = 0; x < FM * FN; x++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, (FN * 10 + FM * FN - 1) / (FM * FN), 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        /* ... then step 1's, with the next stage's step-0 decode among them (its records have landed) */
        wait_vm<(D - 2) * A_DMA>();
#pragma unroll
        for (int i = 0; i < FN; i++) pin16(rn[i]);
        decode(std::integral_constant<int, 0>{}, rn, bw0);
#pragma unroll
        for (int j = 0; j < FM; j++)
#pragma unroll
            for (int i = 0; i < FN; i++)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw1[i], av[1][j], acc[i][j], 0, 0, 0);
#pragma unroll
        for (int x = 0; x < FM * FN; x++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, (FN * 10 + FM * FN - 1) / (FM * FN), 0);
        }
#pragma unroll
        for (int i = 0; i < FN; i++) asm volatile("" : "+v"(bw0[i]));   /* made here, not after the loop's branch */
        if (MULTI && t + 1 < nst && (t + 1) % UNITS_PER_FOLD == 0) {
            fold(block);
            block++;
        }
    };
    for (int t = 0; t < nst; t += 2) {
        stage(t, rb0, rb1);
        if (t + 1 < nst) stage(t + 1, rb1, rb0);
    }
    fold(block);

    /* C staged through LDS (idle once the last stage is read) and stored as whole row segments at device scope */
    constexpr int LPR = G::BN / 4;   /* lanes per staged row */
    constexpr int RPI = 64 / LPR;    /* rows per store instruction */
    static_assert(64 % LPR == 0, "row segments per wave");
    float *stg = reinterpret_cast<float *>(ring);
    const int lr = lane / LPR, lc = lane % LPR;
    const DevScopeOut cout(g.C + (size_t)m0 * g.ldc, (size_t)min(G::BM, M - m0) * g.ldc * 4, g.c_wt);
    lds_barrier();
#pragma unroll
    for (int j0 = 0; j0 < FM; j0 += CJ) {
#pragma unroll
        for (int j = j0; j < j0 + CJ && j < FM; j++)
#pragma unroll
            for (int i = 0; i < FN; i++) {
                const int nl = wave * 16 * FN + 16 * i + 4 * (lane >> 4);
                *reinterpret_cast<v4f *>(stg + (16 * (j - j0) + (lane & 15)) * SROW + nl) =
                    v4f{run[i][j][0], run[i][j][1], run[i][j][2], run[i][j][3]};
            }
        lds_barrier();
        const int rows = 16 * (min(j0 + CJ, FM) - j0);
        for (int r = wave * RPI + lr; r < rows; r += NW * RPI) {
            const int m = m0 + 16 * j0 + r, n = n0 + 4 * lc;
            if (m < M && n < N) {
                const v4f v = *reinterpret_cast<const v4f *>(stg + r * SROW + 4 * lc);
                if (g.c_vec4) {
                    cout.st16(((size_t)(m - m0) * g.ldc + n) * 4, v);
                } else {
                    float *cp = g.C + (size_t)m * g.ldc + n;
                    cp[0] = v[0]; cp[1] = v[1]; cp[2] = v[2]; cp[3] = v[3];
                }
            }
        }
        if (j0 + CJ < FM) lds_barrier();
    }
}

template <class G, bool MULTI>
__global__ __launch_bounds__(G::NT, 2) void gemm_fv_rb(GemmArgs g)
{
    fv_tile_rb<G, MULTI>(g);
}

template <class G, int MODE, int OUT, bool MULTI, bool SPLIT, int OCC = 1, bool CSHUF = false>
__global__ __launch_bounds__(G::NT, OCC) void gemm_fv(GemmArgs g)
{
    fv_tile<G, MODE, OUT, MULTI, SPLIT, OCC, CSHUF>(g);
}

/* ── the small-M five-value GEMM ─────────────────────────────────────────────────────────────────────────────── */

/* Small-M tile: a workgroup of W waves (four, or sixteen for long K) owns one BM × BN output tile (BM = 16·FM
 * activation rows, BN = 16·FN weight columns) and splits K among its waves. Each wave loads its operands straight from global memory into
 * registers – the tiled activations and the operand records are already in matrix-core order – two 128-row units
 * per load batch, the next batch in flight while the current one is decoded and multiplied. No LDS staging and no
 * barrier in the K loop. */
template <int FM_, int FN_, int CH_ = 2, int W_ = 4>
struct SmGeo {
    static constexpr int FM = FM_, FN = FN_;
    static constexpr int BM = 16 * FM, BN = 16 * FN;
    static constexpr int WAVES = W_, NT = 64 * W_;
    static constexpr int PITCH = BN + 4;     /* int32 per row of a partial tile in LDS */
    static constexpr int MAXSEG = W_;        /* K segments per tile (one per wave; K <= 4096) */
    static constexpr int CH = CH_;           /* 128-row units per load batch (two batches in registers) */
    static_assert(CH == 1 || CH == 2 || CH == 4 || CH == 8, "batches divide a segment's 8 units");
};

/* 128-row units per K segment of a small-M call with `waves` waves: up to 1024 rows, ceil(units / waves) inside the
 * one fold block; beyond, the smallest of 1, 2, 4, 8 that leaves at most one segment per wave, so that every
 * segment lies inside one 1024-row fold block and its int32 sum belongs to that block. */
__host__ __device__ __forceinline__ int sm_seg_units(int units, int waves)
{
    if (units <= 8) return (units + waves - 1) / waves;
    int d = 1;
    while (d < 8 && (units + d - 1) / d > waves) d *= 2;
    return d;
}

template <class G, int MODE, bool TWO_OUT>
__device__ __forceinline__ void sm_unit_mma(const v4i (&a)[2][G::FM], const uint32_t (&r)[G::FN][4],
                                            const uint32_t (&lo_tab)[G::FN], v4i (&acc)[G::FN][G::FM],
                                            v4i (&accT)[TWO_OUT ? G::FN : 1][TWO_OUT ? G::FM : 1])
{
#pragma unroll
    for (int s = 0; s < 2; s++) {
        v4i bw[G::FN], bt[TWO_OUT ? G::FN : 1];
#pragma unroll
        for (int i = 0; i < G::FN; i++)
#pragma unroll
            for (int d = 0; d < 4; d++) {
                const uint32_t sel = (r[i][2 * s + (d >> 1)] >> (4 * (d & 1))) & 0x07070707u;
                if (MODE == MODE_INT8W) {
                    bw[i][d] = (int)perm(kI8wHiTable, lo_tab[i], sel);
                } else {
                    bw[i][d] = (int)perm(kPlaneS, kPlaneS, sel);
                    bt[TWO_OUT ? i : 0][d] = (int)perm(kPlaneS, 0u, sel);
                }
            }
#pragma unroll
        for (int j = 0; j < G::FM; j++)
#pragma unroll
            for (int i = 0; i < G::FN; i++) {
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw[i], a[s][j], acc[i][j], 0, 0, 0);
                if (TWO_OUT)
                    accT[TWO_OUT ? i : 0][TWO_OUT ? j : 0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                        bt[TWO_OUT ? i : 0], a[s][j], accT[TWO_OUT ? i : 0][TWO_OUT ? j : 0], 0, 0, 0);
            }
    }
}

/* The int8 five-value GEMM for small M (sgemm_i8_worker, blas.c:1296-1370). Each wave accumulates int32 sums over its
 * K segments and writes them to LDS; after one barrier the workgroup adds the partial sums of each 1024-row block
 * (exact in int32) and folds the blocks into fp32 in order, exactly as the reference does per K block
 * (blas.c:1355-1366), storing C as whole row segments. */
template <class G, int MODE>
__device__ __forceinline__ void fvs_tile(const GemmArgs &g)
{
    constexpr bool TWO = (MODE == MODE_INT8);
    constexpr int FM = G::FM, FN = G::FN, BM = G::BM, BN = G::BN, PITCH = G::PITCH, CH = G::CH;
    constexpr int TILE = BM * PITCH;
    __shared__ __attribute__((aligned(16))) int32_t part[(TWO ? 2 : 1) * G::MAXSEG * TILE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    /* Workgroup b runs on XCD b % 8. By default consecutive workgroups take consecutive column tiles, so each XCD's
     * L2 fetches all the rows and an eighth of the weight records. With xcd_rows = a the XCDs form an a × (8 / a)
     * grid over the tiles: XCD x takes row block x / (8 / a) and column block x % (8 / a), its L2 fetching 1 / a of
     * the rows and a / 8 of the records. */
    int tile_n = blockIdx.x % g.tiles_n, tile_m = blockIdx.x / g.tiles_n;
    if (g.xcd_rows > 0) {
        const int a = g.xcd_rows, cb = 8 / a, x = (int)blockIdx.x & 7, l = (int)blockIdx.x >> 3;
        const int RB = g.tiles_m / a, CB = g.tiles_n / cb;
        tile_m = (x / cb) * RB + l / CB;
        tile_n = (x % cb) * CB + l % CB;
    }
    const int n0 = tile_n * BN, m0 = tile_m * BM;
    const int M = g.M, N = g.N, units = g.units;
    /* one 128-byte line per thread of the range a later kernel reads (the records of the caller's next weight),
     * requested before this tile's own loads, so that waiting for those (the vector-memory counter retires in
     * order) never waits behind it; the value is consumed as the wave ends */
    uint32_t warm = 0;
    if (g.warm) {
        const int t = blockIdx.x * G::NT + tid;
        if (t < g.warm_lines) warm = *reinterpret_cast<const uint32_t *>(g.warm + (size_t)t * 128);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int seg_units = sm_seg_units(units, G::WAVES);
    const int nseg = (units + seg_units - 1) / seg_units;

    /* per-lane operand addresses (row and column groups clamped into the padded operands; outputs are masked) */
    const int8_t *a_base[FM];
#pragma unroll
    for (int j = 0; j < FM; j++) {
        const int mg = min((m0 >> 4) + j, g.mg_last);
        a_base[j] = g.Q + (size_t)mg * g.kst * 1024 + lane * 16;
    }
    const uint8_t *b_base[FN];
    uint32_t clo[FN];   /* the columns' lo codes; their decode tables are built once the operand loads are issued */
#pragma unroll
    for (int i = 0; i < FN; i++) {
        const int cg = min((n0 >> 4) + i, g.ng_last);
        b_base[i] = g.rec + (size_t)cg * units * 1024 + lane * 16;
        clo[i] = MODE == MODE_INT8W ? g.clo[16 * cg + (lane & 15)] : 0u;
    }

    /* fold geometry: thread t owns rows t / (BN / 4) + RPP·p and four consecutive columns 4·(t % (BN / 4)). Its
     * epilogue factors are read here, ahead of the operands, so that their latency overlaps the operand loads'
     * instead of following the barrier (addresses clamped; the fold skips what lies outside C). */
    constexpr int TPR = BN / 4;                  /* threads per output row */
    constexpr int RPP = G::NT / TPR;             /* rows per pass */
    constexpr int PASSES = (BM + RPP - 1) / RPP;
    const int cq = tid % TPR, n = n0 + 4 * cq, r0 = tid / TPR;
    v4f c1 = *reinterpret_cast<const v4f *>(g.c1 + min(n, N - 4));
    v4f c2 = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if (TWO) c2 = *reinterpret_cast<const v4f *>(g.c2 + min(n, N - 4)) - c1;   /* hi − lo */
    if (g.c1_hi) c1 = c1 * (1.0f / 127.0f);                                      /* hi·(1/127) */
    float row_scale[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; p++) row_scale[p] = g.a_scales[min(m0 + r0 + RPP * p, M - 1)];

    v4i a[2][CH][2][FM];
    uint32_t r[2][CH][FN][4];
    auto load_batch = [&](int buf, int u0, int nu) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int u = min(u0 + c, u0 + nu - 1);   /* a short last batch reloads its last unit (never used) */
#pragma unroll
            for (int j = 0; j < FM; j++)
#pragma unroll
                for (int s = 0; s < 2; s++)
                    a[buf][c][s][j] = *reinterpret_cast<const v4i *>(a_base[j] + (size_t)(2 * u + s) * 1024);
#pragma unroll
            for (int i = 0; i < FN; i++) {
                const uint4 v = *reinterpret_cast<const uint4 *>(b_base[i] + (size_t)u * 1024);
                r[buf][c][i][0] = v.x; r[buf][c][i][1] = v.y; r[buf][c][i][2] = v.z; r[buf][c][i][3] = v.w;
            }
        }
    };

    /* one K segment per wave at most (K <= 4096), so no loop: a loop here makes the compiler wait for every load
     * above before it, the lo codes and the epilogue factors included */
    if (wave < nseg) {
        const int seg = wave;
        const int u_begin = seg * seg_units, u_end = min(units, u_begin + seg_units);
        v4i acc[FN][FM], accT[TWO ? FN : 1][TWO ? FM : 1];
#pragma unroll
        for (int i = 0; i < FN; i++)
#pragma unroll
            for (int j = 0; j < FM; j++) {
                acc[i][j] = v4i{0, 0, 0, 0};
                if (TWO) accT[TWO ? i : 0][TWO ? j : 0] = v4i{0, 0, 0, 0};
            }
        /* batches of CH units, the next batch loading while the current one is multiplied (at most 8 units) */
        load_batch(0, u_begin, min(CH, u_end - u_begin));
        __builtin_amdgcn_sched_barrier(0);
        uint32_t lo_tab[FN];
#pragma unroll
        for (int i = 0; i < FN; i++) lo_tab[i] = MODE == MODE_INT8W ? i8w_lo_table(clo[i]) : 0u;
#pragma unroll
        for (int b = 0; b < 8 / CH; b++) {
            const int u0 = u_begin + b * CH;
            if (u0 >= u_end) break;
            if (u0 + CH < u_end) load_batch((b + 1) & 1, u0 + CH, min(CH, u_end - u0 - CH));
#pragma unroll
            for (int c = 0; c < CH; c++)
                if (u0 + c < u_end) sm_unit_mma<G, MODE, TWO>(a[b & 1][c], r[b & 1][c], lo_tab, acc, accT);
        }
        /* this segment's int32 sums → LDS, [row][column] with padded rows */
        int32_t *dst = part + seg * TILE;
#pragma unroll
        for (int i = 0; i < FN; i++)
#pragma unroll
            for (int j = 0; j < FM; j++) {
                const int row = 16 * j + (lane & 15), col = 16 * i + 4 * (lane >> 4);
                *reinterpret_cast<v4i *>(dst + row * PITCH + col) = acc[i][j];
                if (TWO) *reinterpret_cast<v4i *>(dst + G::MAXSEG * TILE + row * PITCH + col) = accT[TWO ? i : 0][TWO ? j : 0];
            }
    }
    __syncthreads();

    /* fold */
    asm volatile("" ::"v"(warm));
    if (n >= N) return;
    const bool beta_zero = g.beta == 0.0f;
    const int nblocks = (units + 7) / 8;
    const int spb = units <= 8 ? nseg : 8 / seg_units;   /* segments per fold block */
    const DevScopeOut cout(g.C + (size_t)m0 * g.ldc, (size_t)min(BM, M - m0) * g.ldc * 4, g.c_wt);
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
        const int row = r0 + RPP * p, m = m0 + row;
        if (row >= BM || m >= M) break;
        const float as = row_scale[p] * g.alpha;
        float *cp = g.C + (size_t)m * g.ldc + n;
        float run[4];
        if (!beta_zero) {
            if (g.c_vec4) {
                const v4f v = *reinterpret_cast<const v4f *>(cp);
                run[0] = v[0]; run[1] = v[1]; run[2] = v[2]; run[3] = v[3];
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) run[e] = cp[e];
            }
            if (g.beta != 1.0f) {
#pragma unroll
                for (int e = 0; e < 4; e++) run[e] = run[e] * g.beta;
            }
        }
        for (int blk = 0; blk < nblocks; blk++) {
            /* the segments of this block: all of them below 1024 rows, else exactly the block's own */
            const int s0 = units <= 8 ? 0 : blk * spb, s1 = units <= 8 ? nseg : min(nseg, s0 + spb);
            v4i sum = v4i{0, 0, 0, 0}, sumT = v4i{0, 0, 0, 0};
            for (int sg = s0; sg < s1; sg++) {
                sum += *reinterpret_cast<const v4i *>(part + sg * TILE + row * PITCH + 4 * cq);
                if (TWO) sumT += *reinterpret_cast<const v4i *>(part + G::MAXSEG * TILE + sg * TILE + row * PITCH + 4 * cq);
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float f = (float)sum[e] * c1[e];
                if (TWO) f = __builtin_fmaf((float)sumT[e], c2[e], f);
                run[e] = (blk == 0 && beta_zero) ? f * as : __builtin_fmaf(f, as, run[e]);
            }
        }
        if (g.act) {   /* the feed-forward's SiLU (p2_swish_quant_rows' body, tensor_ops.c:491-511) on the output */
#pragma unroll
            for (int e = 0; e < 4; e++) run[e] = silu_p2(run[e]);
        }
        if (g.c_vec4) {
            cout.st16(((size_t)row * g.ldc + n) * 4, v4f{run[0], run[1], run[2], run[3]});
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) cp[e] = run[e];
        }
    }
}

template <class G, int MODE>
__global__ __launch_bounds__(G::NT, G::NT > 256 ? 1 : 2) void gemm_fvs(GemmArgs g)
{
    fvs_tile<G, MODE>(g);
}

/* Several five-value weights of one shape against the same quantised activations, one launch: blockIdx.y picks the
 * weight (its records, tables and output); everything else is gemm_fvs's. */
constexpr int kMaxGroups = 32;
struct GroupArgs {
    const uint8_t *rec[kMaxGroups];
    const uint8_t *clo[kMaxGroups];
    const float *c1[kMaxGroups];
    const float *c2[kMaxGroups];
    float *C[kMaxGroups];
};

template <class G, int MODE>
__global__ __launch_bounds__(G::NT, G::NT > 256 ? 1 : 2) void gemm_fvs_grouped(GemmArgs g, GroupArgs ga)
{
    GemmArgs h = g;
    const int q = blockIdx.y;
    h.rec = ga.rec[q]; h.clo = ga.clo[q]; h.c1 = ga.c1[q]; h.c2 = ga.c2[q]; h.C = ga.C[q];
    fvs_tile<G, MODE>(h);
}

/* The same for the large-M kernel's tiles (int8w, one split; blockIdx.x is the tile as in gemm_fv). */
template <class G, bool MULTI>
__global__ __launch_bounds__(G::NT, 2) void gemm_fv_grouped(GemmArgs g, GroupArgs ga)
{
    GemmArgs h = g;
    const int q = blockIdx.y;
    h.rec = ga.rec[q]; h.clo = ga.clo[q]; h.c1 = ga.c1[q]; h.c2 = ga.c2[q]; h.C = ga.C[q];
    fv_tile<G, MODE_INT8W, OUT_F32, MULTI, false, 2, true>(h);
}

/* The fold after a split GEMM: per output, the int32 partial sums of the splits inside each 1024-row block are
 * added (exact), then the blocks fold into fp32 in order exactly as the unsplit kernel folds them. One thread per
 * four consecutive outputs of a row. */
template <bool TWO>
__global__ __launch_bounds__(256) void fold_splits(GemmArgs g)
{
    const int M = g.M, N = g.N;
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= (size_t)M * (N / 4)) return;
    const int m = (int)(q / (N / 4)), n = 4 * (int)(q % (N / 4));
    const size_t plane = (size_t)g.splits * M * N;
    const int per_block = kFoldRows / g.split_rows;
    const int nblocks = (g.splits + per_block - 1) / per_block;
    const float as = g.a_scales[m] * g.alpha;
    float *cp = g.C + (size_t)m * g.ldc + n;
    float c1v[4], c2v[4] = {0, 0, 0, 0}, run[4] = {0, 0, 0, 0};
#pragma unroll
    for (int r = 0; r < 4; r++) {
        c1v[r] = c1_factor(g, n + r);
        if (TWO) c2v[r] = c2_factor(g, n + r);
    }
    if (g.beta != 0.0f) {
#pragma unroll
        for (int r = 0; r < 4; r++) run[r] = g.beta == 1.0f ? cp[r] : cp[r] * g.beta;
    }
    for (int b = 0; b < nblocks; b++) {
        v4i s1 = v4i{0, 0, 0, 0}, s2 = v4i{0, 0, 0, 0};
        const int s_end = min(g.splits, (b + 1) * per_block);
        for (int s = b * per_block; s < s_end; s++) {
            const int32_t *p = g.part + ((size_t)s * M + m) * N + n;
            s1 += *reinterpret_cast<const v4i *>(p);
            if (TWO) s2 += *reinterpret_cast<const v4i *>(p + plane);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float f = (float)s1[r] * c1v[r];
            if (TWO) f = __builtin_fmaf((float)s2[r], c2v[r], f);
            run[r] = (b == 0 && g.beta == 0.0f) ? f * as : __builtin_fmaf(f, as, run[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) cp[r] = run[r];
}

/* ── the exact route ───────────────────────────────────────────────────────────────────────────────────────── */

struct ExactArgs {
    int M, N, K;
    float alpha, beta;
    const float *A; int lda; int a_vec4;                  /* a_vec4: lda % 4 == 0 and A 16-B aligned */
    const uint8_t *signs; const uint8_t *flags; const float *lo; const float *hi;   /* five-value */
    const int8_t *B8; int ldb; const float *bscales;      /* int8 table */
    float *C; int ldc;
    int tiles_n;
    const uint8_t *rec; int units;                        /* 4-bit selector records (fv_repack4) for gemm_xf */
    int act;                                              /* gemm_xf: 1 stores silu_p2 of each output (beta 0,
                                                             ldc = N, N % 8 == 0: p2_swish's eight-wide body) */
};

constexpr int EBM = 64, EBN = 64, EBK = 32;

enum { EXB_FV = 0, EXB_Q8 = 1 };

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
            if (m < M && k < K) v = g.A[(size_t)m * g.lda + k];
            ra[c] = g.alpha * v;
        }
        const int k = k0 + wk;
        if (BKIND == EXB_FV) {   /* the 8 columns' selector nibbles of row k from the records (code 1 outside) */
            uint32_t sel[8];
#pragma unroll
            for (int c = 0; c < 8; c++) sel[c] = 1u;
            if (wcol_ok && k < K) {
                int shift;
                const uint8_t *rb = g.rec + rec_quad_offset(g.units, k & ~3, n0 + wn, shift) + (k & 3);
#pragma unroll
                for (int c = 0; c < 8; c++) sel[c] = (rb[16 * c] >> shift) & 7u;
            }
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const int code = (int)(sel[c] & 3u), fl = (int)(sel[c] >> 2);
                rw[c] = (float)(code - 1) * __builtin_fmaf((float)fl, wd[c], wlo[c]);
            }
        } else {
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const int8_t q = (wcol_ok && k < K) ? g.B8[(size_t)k * g.ldb + n0 + wn + c] : (int8_t)0;
                rw[c] = (float)q * wlo[c];
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

/* The exact-mode five-value GEMM on the fp32 matrix cores (sgemm_fvb_exact, blas.c:929-987): C = beta·C +
 * alpha·A·W with every weight expanded to fp32 as the reference expands it, w = (code − 1)·fmaf(flag, hi − lo, lo)
 * (blas.c:875-897), and the products summed in fp32 by v_mfma_f32_16x16x4_f32. The sum runs in a different order
 * from the reference's per-output fmaf chain (which gemm_exact keeps bit for bit), so outputs agree to fp32 rounding.
 * A workgroup of four waves owns a BM × BN tile and splits K among its waves, as gemm_fvs does: each wave streams its
 * units' weight records (the 4-bit selectors of fv_repack4) and fp32 rows, expands the weights in registers and
 * multiplies; lane l of the step t MFMA takes k = 16·(l / 16) + t of a 64-row step, which is the record's own order.
 * The four partial tiles meet in LDS and are added in wave order.
 * The fp32 rows reach the lanes in one of two ways, with the same MFMAs in the same order (the same bits):
 *   STAGED (K % 128 == 0 and VEC): each wave brings its 64-row K stages of the BM rows into its own LDS slot by
 *     direct loads of whole 256-byte row segments (four rows per instruction, 16-byte chunk c of row r stored at
 *     place c ^ (r % 16), so the operand reads below are free of bank conflicts); no barrier, each wave reads only its
 *     own slot. 43.3 → 31.5 us at M = 375, 1024 → 4096 (16.5 → 12.9 us at 1024 → 1024, 51.9 → 44.1 us at
 *     4096 → 1024): loads straight into the matrix-core layout touch 16 rows × 64 bytes per instruction, and the
 *     lines per instruction, not the bytes, set their pace.
 *   else: loads into registers in the matrix-core layout, units double-buffered.
 * VEC: K % 4 == 0, lda % 4 == 0 and A 16-byte aligned. */
template <int FM, int FN, bool VEC, bool STAGED = false>
__global__ __launch_bounds__(256, 2) void gemm_xf(ExactArgs g)
{
    static_assert(!STAGED || VEC, "the staged rows are read as 16-byte chunks");
    constexpr int NW = 4, NT = 64 * NW;
    constexpr int BM = 16 * FM, BN = 16 * FN, PITCH = BN + 4, TILE = BM * PITCH;
    constexpr int ABUF = BM * 256;                    /* STAGED: one 64-row K stage of one wave, BM rows × 256 bytes */
    constexpr int NQ = BM / 4;                        /* STAGED: direct loads per stage, four rows each */
    constexpr int SMEM = (STAGED && NW * ABUF > 4 * NW * TILE) ? NW * ABUF : 4 * NW * TILE;   /* bytes */
    __shared__ __attribute__((aligned(16))) int8_t smem[SMEM];   /* the partial tiles reuse the staging slots */
    float *part = reinterpret_cast<float *>(smem);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, grp = lane >> 4;
    const int tile_n = blockIdx.x % g.tiles_n, tile_m = blockIdx.x / g.tiles_n;
    const int n0 = tile_n * BN, m0 = tile_m * BM;
    const int M = g.M, N = g.N, K = g.K, units = g.units;
    const int su = (units + NW - 1) / NW;
    const int nseg = (units + su - 1) / su;
    const int u_begin = min(units, wave * su), u_end = min(units, u_begin + su);

    /* Every weight of column n is one of eight values, w = (code − 1)·fmaf(flag, hi − lo, lo) for the 4-bit
     * selector code | flag << 2: built once per tile into LDS (rows of 9 floats, so the 16 columns a wave reads
     * spread over the banks), then one extract and one LDS read per weight. */
    __shared__ float wtab[BN * 9];
    for (int c = tid; c < BN * 8; c += NT) {
        const int col = c >> 3, sel = c & 7, n = min(n0 + col, N - 1);
        const float lo = g.lo[n], d = g.hi[n] - lo;
        wtab[col * 9 + sel] = (float)((sel & 3) - 1) * __builtin_fmaf((float)(sel >> 2), d, lo);
    }
    int tcol[FN];
    const uint8_t *b_base[FN];
#pragma unroll
    for (int i = 0; i < FN; i++) {
        const int n = min(n0 + 16 * i + (lane & 15), N - 1);
        tcol[i] = (16 * i + (lane & 15)) * 9;
        b_base[i] = g.rec + (size_t)(n >> 4) * units * 1024 + lane * 16;
    }
    __syncthreads();
    const float *a_row[FM];
#pragma unroll
    for (int j = 0; j < FM; j++) a_row[j] = g.A + (size_t)min(m0 + 16 * j + (lane & 15), M - 1) * g.lda;

    v4f acc[FN][FM];
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
        for (int j = 0; j < FM; j++) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    auto load_x = [&](int j, int k0, float x[16]) __attribute__((always_inline)) {
        if (VEC) {
            load16<true>(a_row[j], k0, K, x);
        } else {
#pragma unroll
            for (int e = 0; e < 16; e++) x[e] = (k0 + e < K) ? a_row[j][k0 + e] : 0.0f;
        }
    };

    uint32_t r[2][FN][4];
    /* one 64-row step s of a unit whose records are r[rb]: 16 MFMA steps, each weight expanded once for the FM rows */
    auto mma_step = [&](int rb, int s, const float (&x)[FM][16]) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 16; t++) {
            const int d = t >> 2, b = t & 3;
            float w[FN];
#pragma unroll
            for (int i = 0; i < FN; i++)
                w[i] = wtab[tcol[i] + ((r[rb][i][2 * s + (d >> 1)] >> (8 * b + 4 * (d & 1))) & 7u)];
#pragma unroll
            for (int j = 0; j < FM; j++)
#pragma unroll
                for (int i = 0; i < FN; i++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(w[i], x[j][t], acc[i][j], 0, 0, 0);
        }
    };
    auto load_records = [&](int rb, int u) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < FN; i++) {
            const uint4 v = *reinterpret_cast<const uint4 *>(b_base[i] + (size_t)u * 1024);
            r[rb][i][0] = v.x; r[rb][i][1] = v.y; r[rb][i][2] = v.z; r[rb][i][3] = v.w;
        }
    };
    if constexpr (STAGED) {
        /* stage st = 2·(u − u_begin) + s into this wave's slot; load q brings rows 4q .. 4q + 3, lane L filling place
         * L % 16 of row 4q + L / 16 with that row's chunk (L % 16) ^ (row % 16) */
        const float *a_src[NQ];
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            const int rr = 4 * q + (lane >> 4);
            a_src[q] = g.A + (size_t)min(m0 + rr, M - 1) * g.lda + 4 * ((lane & 15) ^ (rr & 15));
        }
        int8_t *slot = smem + wave * ABUF;
        const int n_st = 2 * (u_end - u_begin);
        auto issue = [&](int st) __attribute__((always_inline)) {
            const int u = u_begin + (st >> 1);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   /* this wave's reads of the slot are complete */
#pragma unroll
            for (int q = 0; q < NQ; q++) dma_16(a_src[q] + 128 * u + 64 * (st & 1), slot + q * 1024);
            if ((st & 1) == 0) load_records(0, u);
        };
        auto compute = [&](int st) __attribute__((always_inline)) {
            float x[FM][16];
#pragma unroll
            for (int j = 0; j < FM; j++) {
                const int8_t *row = slot + (16 * j + (lane & 15)) * 256;
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) {
                    const float4 v = *reinterpret_cast<const float4 *>(row + 16 * ((4 * grp + q4) ^ (lane & 15)));
                    x[j][4 * q4] = v.x; x[j][4 * q4 + 1] = v.y; x[j][4 * q4 + 2] = v.z; x[j][4 * q4 + 3] = v.w;
                }
            }
            mma_step(0, st & 1, x);
        };
        /* one slot per wave, every load waited before its stage is multiplied: the other waves of the CU (up to four
         * per SIMD: 34 KB of LDS and at most 128 VGPRs per wave) cover each wave's wait. Two slots per wave with the
         * next stage in flight measured 5-14 % slower (the doubled LDS halves the workgroups per CU), and eight
         * waves splitting K no faster. */
        for (int st = 0; st < n_st; st += 2) {
            issue(st);        /* step 0 of the unit and its records */
            wait_vm<0>();
            compute(st);
            issue(st + 1);    /* step 1 */
            wait_vm<0>();
            compute(st + 1);
        }
        __syncthreads();   /* every wave is done with its slots: the partial tiles reuse the area */
    } else {
        /* units double-buffered in registers: unit u + 1 loads while unit u is expanded and multiplied */
        float x[2][2][FM][16];
        auto load_unit = [&](int buf, int u) __attribute__((always_inline)) {
            load_records(buf, u);
#pragma unroll
            for (int s = 0; s < 2; s++)
#pragma unroll
                for (int j = 0; j < FM; j++) load_x(j, 128 * u + 64 * s + 16 * grp, x[buf][s][j]);
        };
        auto mma_unit = [&](int buf) __attribute__((always_inline)) {
            mma_step(buf, 0, x[buf][0]);
            mma_step(buf, 1, x[buf][1]);
        };
        if (u_begin < u_end) load_unit(0, u_begin);
        for (int u = u_begin; u < u_end; u += 2) {
            if (u + 1 < u_end) load_unit(1, u + 1);
            mma_unit(0);
            if (u + 1 >= u_end) break;
            if (u + 2 < u_end) load_unit(0, u + 2);
            mma_unit(1);
        }
    }
    if (wave < nseg) {
        float *dst = part + wave * TILE;
#pragma unroll
        for (int i = 0; i < FN; i++)
#pragma unroll
            for (int j = 0; j < FM; j++)
                *reinterpret_cast<v4f *>(dst + (16 * j + (lane & 15)) * PITCH + 16 * i + 4 * grp) = acc[i][j];
    }
    __syncthreads();

    constexpr int TPR = BN / 4, RPP = NT / TPR;
    const int cq = tid % TPR, n = n0 + 4 * cq;
    if (n >= N) return;
    for (int row = tid / TPR; row < BM; row += RPP) {
        const int m = m0 + row;
        if (m >= M) break;
        v4f sum = *reinterpret_cast<const v4f *>(part + row * PITCH + 4 * cq);
        for (int sg = 1; sg < nseg; sg++) sum += *reinterpret_cast<const v4f *>(part + sg * TILE + row * PITCH + 4 * cq);
        float *cp = g.C + (size_t)m * g.ldc + n;
        if (n + 3 < N && (reinterpret_cast<uintptr_t>(cp) & 15) == 0) {   /* one 16-byte store */
            v4f c0 = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            if (g.beta != 0.0f) {
                c0 = *reinterpret_cast<const v4f *>(cp);
                if (g.beta != 1.0f) {
#pragma unroll
                    for (int e = 0; e < 4; e++) c0[e] = c0[e] * g.beta;
                }
            }
            v4f r;
#pragma unroll
            for (int e = 0; e < 4; e++) r[e] = __builtin_fmaf(g.alpha, sum[e], c0[e]);
            if (g.act) {
#pragma unroll
                for (int e = 0; e < 4; e++) r[e] = silu_p2(r[e]);
            }
            *reinterpret_cast<v4f *>(cp) = r;
            continue;
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            if (n + e >= N) break;
            const float c0 = g.beta == 0.0f ? 0.0f : (g.beta == 1.0f ? cp[e] : cp[e] * g.beta);
            const float r = __builtin_fmaf(g.alpha, sum[e], c0);
            cp[e] = g.act ? silu_p2(r) : r;
        }
    }
}

/* fp32 GEMMs on the matrix cores, batched with strides (p2_sgemm / p2_sgemm_st, blas.h:25-36, and the per-head
 * products of attention, encoder.c:279-316, 505-519): C_b = alpha·op(A_b)·op(B_b) + beta·C_b for b < batch, all
 * row-major; sgemm_f32 below. Sums run in the matrix cores' order (fp32 rounding, not the reference's order). */
struct SgemmArgs {
    int M, N, K;
    float alpha, beta;
    const float *A; int lda; long long sA; int transA;
    const float *B; int ldb; long long sB; int transB;
    float *C; int ldc; long long sC;
    int tiles_n, batch;
};

/* How an sgemm operand is read: LD_VEC, 16-byte loads (rows 16-byte aligned, row length a multiple of 4, so a run
 * of four is all in range or all out); LD_BUF, buffer loads through a descriptor whose range ends at the operand's
 * last element, an out-of-range element's offset pushed past that range so the hardware returns zero (no branch,
 * so the loads stay in flight; the operand spans less than 2 GiB); LD_ANY, element loads behind range checks. */
enum { LD_VEC = 0, LD_BUF = 1, LD_ANY = 2 };
constexpr uint32_t kBufDword3 = 0x00020000u;   /* raw buffer descriptor word 3 for gfx9 */

/* One operand's panel of a 32-row K stage in an sgemm workgroup of 256 threads. KMAJ: the panel is [k][x] (32 k-rows
 * of 64 values, the operand stored with x contiguous); else [x][k] (64 x-rows of 32 values, k contiguous). The panel
 * keeps that orientation in LDS: [k][x] rows 80 floats apart (≡ 16 mod 32: the 16-lane groups of an MFMA operand
 * read, one k-row each, fall in disjoint halves of the banks), [x][k] rows 34 apart (≡ 2 mod 32: lane (x, g) reads
 * bank 2x + g, distinct over a 32-lane pass), so no transpose happens at store time. Each thread moves 8 values:
 *   LD_VEC: two runs of 4 along the contiguous dimension, 16-byte loads (rows aligned, length a multiple of 4);
 *   else: 8 single values, consecutive lanes on consecutive columns, so each load instruction reads whole row
 *   segments; LD_BUF through a buffer descriptor (out-of-range offsets return zero, no branches), LD_ANY with range
 *   checks. Rows outside the operand, and columns past its row length, read as zeros. */
template <bool KMAJ, int LD>
struct SgPanel {
    static constexpr int S = KMAJ ? 80 : 34;          /* LDS row stride */
    static constexpr int CW = KMAJ ? 64 : 32;         /* panel row length */
    static constexpr int SIZE = KMAJ ? 32 * 80 : 64 * 34;
    const float *base;
    __amdgpu_buffer_rsrc_t rsrc;
    int ld, rows, len;                                /* operand: leading dimension, rows, valid values per row */

    /* panel origin: (row0, col0) in operand coordinates; thread tid; v: the thread's 8 values */
    __device__ __forceinline__ void load(int row0, int col0, int tid, float (&v)[8]) const
    {
        if (LD == LD_VEC) {
            const int r = KMAJ ? tid / 8 : tid / 4, c = KMAJ ? 8 * (tid % 8) : 8 * (tid % 4);
            const int gr = row0 + r;
            const bool rok = gr < rows;
            const float *row = base + (size_t)min(gr, rows - 1) * ld;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int gc = col0 + c + 4 * h;
                const bool ok = rok && gc < len;
                const float4 x = *reinterpret_cast<const float4 *>(row + (ok ? gc : 0));
                v[4 * h] = ok ? x.x : 0.0f;
                v[4 * h + 1] = ok ? x.y : 0.0f;
                v[4 * h + 2] = ok ? x.z : 0.0f;
                v[4 * h + 3] = ok ? x.w : 0.0f;
            }
        } else {
            const int c = tid % CW, gc = col0 + c;
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const int gr = row0 + q * (256 / CW) + tid / CW;
                const bool ok = gr < rows && gc < len;
                if (LD == LD_BUF) {
                    const int off = ok ? 4 * (gr * ld + gc) : (int)0x80000000u;
                    v[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc, off, 0, 0));
                } else {
                    v[q] = ok ? base[(size_t)gr * ld + gc] : 0.0f;
                }
            }
        }
    }
    __device__ __forceinline__ void store(float *panel, int tid, const float (&v)[8]) const
    {
        if (LD == LD_VEC) {
            const int r = KMAJ ? tid / 8 : tid / 4, c = KMAJ ? 8 * (tid % 8) : 8 * (tid % 4);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                float *d = panel + r * S + c + 4 * h;
                if (KMAJ) {
                    *reinterpret_cast<float4 *>(d) = make_float4(v[4 * h], v[4 * h + 1], v[4 * h + 2], v[4 * h + 3]);
                } else {   /* rows 34 floats apart: 8-byte aligned */
                    *reinterpret_cast<float2 *>(d) = make_float2(v[4 * h], v[4 * h + 1]);
                    *reinterpret_cast<float2 *>(d + 2) = make_float2(v[4 * h + 2], v[4 * h + 3]);
                }
            }
        } else {
            const int c = tid % CW;
#pragma unroll
            for (int q = 0; q < 8; q++) panel[(q * (256 / CW) + tid / CW) * S + c] = v[q];
        }
    }
    /* the MFMA operand element (k, x) */
    __device__ __forceinline__ static int at(int k, int x) { return KMAJ ? k * S + x : x * S + k; }
};

/* fp32 GEMM, C = alpha·op(A)·op(B) + beta·C, batched (the attention heads of heads_gemm, encoder.c:279-316; batch
 * index = workgroup id % batch). 64 × 64 tiles, four waves of 32 × 32, v_mfma_f32_16x16x4_f32 (B operand → lane
 * rows n, so a lane's four results are four consecutive n of one row). K advances in stages of 32 through two LDS
 * buffers per operand (SgPanel); each thread brings its 8 + 8 values of a stage into a three-slot register ring,
 * two stages ahead of the one being multiplied, and a stage's LDS operands are all requested before its first
 * MFMA (192 VGPRs would cost the third workgroup per CU that 576-tile launches need).
 * Stages past the end are loaded too (as zeros), so that every iteration issues the same loads and the compiler's
 * wait counts stay exact. TA: A stored [k][m]; TB: B stored [n][k]. LA / LB: how each operand is read (LD_*). */
template <bool TA, bool TB, int LA, int LB>
__global__ __launch_bounds__(256, 3) void sgemm_f32(SgemmArgs g)
{
    constexpr int BMS = 64, BNS = 64, BKS = 32, RING = 3, AHEAD = 2;
    using PA = SgPanel<TA, LA>;      /* A [k][m] is k-major */
    using PB = SgPanel<!TB, LB>;     /* B [k][n] is k-major */
    __shared__ __attribute__((aligned(16))) float sA[2][PA::SIZE];
    __shared__ __attribute__((aligned(16))) float sB[2][PB::SIZE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;                        /* this wave's 32 × 32 quarter */
    /* workgroups reach the 8 XCDs round-robin by linear id, so the batch index is the id's low part: with 8 (or a
     * multiple or divisor of 8) batches every XCD works on its own batches and their operands stay in its L2 */
    const int bat = (int)(blockIdx.x % (unsigned)g.batch), tile = (int)(blockIdx.x / (unsigned)g.batch);
    const int tile_n = tile % g.tiles_n, tile_m = tile / g.tiles_n;
    const int m0 = tile_m * BMS, n0 = tile_n * BNS;
    const float *A = g.A + (size_t)bat * g.sA;
    const float *B = g.B + (size_t)bat * g.sB;
    float *C = g.C + (size_t)bat * g.sC;
    const int M = g.M, N = g.N, K = g.K;
    PA pa;
    pa.base = A; pa.ld = g.lda; pa.rows = TA ? K : M; pa.len = TA ? M : K;
    pa.rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)A, (short)0, LA == LD_BUF ? 4 * ((pa.rows - 1) * pa.ld + pa.len) : 0,
                                                (int)kBufDword3);
    PB pb;
    pb.base = B; pb.ld = g.ldb; pb.rows = TB ? N : K; pb.len = TB ? K : N;
    pb.rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)B, (short)0, LB == LD_BUF ? 4 * ((pb.rows - 1) * pb.ld + pb.len) : 0,
                                                (int)kBufDword3);
    float ra[RING][8], rb[RING][8];
    auto load = [&](int t, float (&xa)[8], float (&xb)[8]) __attribute__((always_inline)) {
        const int k0 = t * BKS;
        if (TA) pa.load(k0, m0, tid, xa); else pa.load(m0, k0, tid, xa);
        if (TB) pb.load(n0, k0, tid, xb); else pb.load(k0, n0, tid, xb);
    };
    auto store = [&](int buf, const float (&xa)[8], const float (&xb)[8]) __attribute__((always_inline)) {
        pa.store(sA[buf], tid, xa);
        pb.store(sB[buf], tid, xb);
    };

    v4f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    const int nk = (K + BKS - 1) / BKS;
    /* stages past the end are loaded too (they read as zeros, from clamped addresses), so that every iteration
     * issues the same loads and the compiler's wait counts stay exact */
#pragma unroll
    for (int s = 0; s < AHEAD; s++) load(s, ra[s], rb[s]);
    store(0, ra[0], rb[0]);
    __syncthreads();
    for (int t0 = 0; t0 < nk; t0 += RING) {
#pragma unroll
        for (int u = 0; u < RING; u++) {   /* stage t = t0 + u sits in ring slot u and LDS buffer t & 1 */
            const int t = t0 + u, buf = t & 1;
            if (t >= nk) break;
            load(t + AHEAD, ra[(u + AHEAD) % RING], rb[(u + AHEAD) % RING]);
            /* the stage's operands, all requested before the first MFMA (one LDS latency per stage, not per step) */
            float a[BKS / 4][2], b[BKS / 4][2];
#pragma unroll
            for (int ks = 0; ks < BKS / 4; ks++) {
                const int kk = 4 * ks + (lane >> 4);
#pragma unroll
                for (int j = 0; j < 2; j++) a[ks][j] = sA[buf][PA::at(kk, 32 * wm + 16 * j + (lane & 15))];
#pragma unroll
                for (int i = 0; i < 2; i++) b[ks][i] = sB[buf][PB::at(kk, 32 * wn + 16 * i + (lane & 15))];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int ks = 0; ks < BKS / 4; ks++)
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(b[ks][i], a[ks][j], acc[i][j], 0, 0, 0);
            if (t + 1 < nk) store(buf ^ 1, ra[(u + 1) % RING], rb[(u + 1) % RING]);
            __syncthreads();
        }
    }
    /* lane l holds C[m][n .. n + 3] with m = m0 + 32·wm + 16·j + l % 16, n = n0 + 32·wn + 16·i + 4·(l / 16) */
    const bool vecC = g.ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(C) & 15) == 0;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int m = m0 + 32 * wm + 16 * j + (lane & 15), n = n0 + 32 * wn + 16 * i + 4 * (lane >> 4);
            if (m >= M) continue;
            float *cp = C + (size_t)m * g.ldc + n;
            if (vecC && n + 3 < N) {
                v4f c0 = v4f{0.0f, 0.0f, 0.0f, 0.0f};
                if (g.beta != 0.0f) {
                    c0 = *reinterpret_cast<const v4f *>(cp);
                    if (g.beta != 1.0f) c0 = c0 * g.beta;
                }
                v4f r;
#pragma unroll
                for (int e = 0; e < 4; e++) r[e] = __builtin_fmaf(g.alpha, acc[i][j][e], c0[e]);
                *reinterpret_cast<v4f *>(cp) = r;
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    if (n + e >= N) break;
                    const float c0 = g.beta == 0.0f ? 0.0f : (g.beta == 1.0f ? cp[e] : cp[e] * g.beta);
                    cp[e] = __builtin_fmaf(g.alpha, acc[i][j][e], c0);
                }
            }
        }
}

/* ── small kernels ─────────────────────────────────────────────────────────────────────────────────────────── */

/* One thread per (panel p, quad kq, column j): the dword of rows 4kq..4kq+3 at
 * out[((p·K/4 + kq)·16 + j)·4 ..] (vst4q_s8 order, blas.c:1229-1239), code = (code − 1)·(flag ? 127 : clo) as an
 * int8 product (blas.c:1233-1236), from the weight's 4-bit records. */
__global__ void fv_pack_codes(int K, int N, int units, const uint8_t *__restrict__ rec,
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
    int shift;
    const uint32_t w = *reinterpret_cast<const uint32_t *>(rec + rec_quad_offset(units, 4 * kq, n, shift));
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t sel = (w >> (8 * i + shift)) & 7u;
        const int code = (int)(sel & 3u), flag = (int)(sel >> 2);
        const int sv = code - 1;
        const int mag = (flag && sv != 0) ? 127 : cl;
        word |= ((uint32_t)(sv * mag) & 0xFFu) << (8 * i);
    }
    out[idx] = word;
}

/* Fill with a word value (a kernel rather than a memset node, so it may sit inside a captured graph). */
__global__ void fill_u32(uint32_t *__restrict__ p, size_t words, uint32_t value)
{
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < words) p[idx] = value;
}

/* One wave that sleeps until `ticks` of the constant-rate wall clock have passed, or `max_naps` naps of
 * s_sleep 127 (about 8k cycles each) have been taken, whichever comes first: the wait ends on either bound. */
__global__ __launch_bounds__(64) void stream_hold(unsigned long long ticks, unsigned max_naps)
{
    const unsigned long long t0 = wall_clock64();
    for (unsigned i = 0; i < max_naps && wall_clock64() - t0 < ticks; ++i) __builtin_amdgcn_s_sleep(127);
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
