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

#include <type_traits>

namespace p2k {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

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
    int tiles_n, tiles_m;                                 /* output tiles of the grid */
    int kq;                                               /* K rounded up to 128: Q columns that may be read */
    int splits, split_rows;                               /* K splits; rows per split (divides 1024) */
    int32_t *part;                                        /* split partials [planes][splits][M][N] */
};


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
            r_c1 = g.c1[n];
            if (TWO) r_c2 = g.c2[n];
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
        a_off[i] = (uint32_t)((c / (BK / 16)) * g.ldq + 16 * (c % (BK / 16)));
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
                const int8_t *qk = g.Q + (size_t)m0 * g.ldq + k0;
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
                ra[i] = *reinterpret_cast<const uint4 *>(g.Q + (size_t)mc * g.ldq + kc);
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
        c1v[r] = g.c1[n + r];
        if (TWO) c2v[r] = g.c2[n + r];
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

/* Fill with a word value (a kernel rather than a memset node, so it may sit inside a captured graph). */
__global__ void fill_u32(uint32_t *__restrict__ p, size_t words, uint32_t value)
{
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < words) p[idx] = value;
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
