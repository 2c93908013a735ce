/*  p2gen.c – seeded synthetic inputs for the five-value GEMM workloads (declared in include/p2gen.h).
 *
 *  PRNG: one xoshiro256** stream per tensor, seeded by SplitMix64 from seed ^ tensor_id. Uniforms are the top 24
 *  bits of a draw (exact in fp32). Normals are Irwin–Hall(12): the sum of twelve 24-bit uniforms minus 6, computed
 *  in integers and scaled by 2^-24, so no libm routine enters and every host produces the same bits.
 */
#include "p2gen.h"

#include <math.h>
#include <string.h>

typedef struct { uint64_t s[4]; } Xoshiro;

static uint64_t splitmix64(uint64_t *x)
{
    uint64_t z = (*x += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static void xo_seed(Xoshiro *g, uint64_t seed, uint64_t tensor_id)
{
    uint64_t x = seed ^ tensor_id;
    for (int i = 0; i < 4; i++) g->s[i] = splitmix64(&x);
}

static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

static inline uint64_t xo_next(Xoshiro *g)
{
    uint64_t *s = g->s;
    uint64_t r = rotl(s[1] * 5, 7) * 9;
    uint64_t t = s[1] << 17;
    s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return r;
}

static inline uint32_t u24(Xoshiro *g) { return (uint32_t)(xo_next(g) >> 40); }

static inline double unif(Xoshiro *g) { return (double)u24(g) * (1.0 / 16777216.0); }

static inline float irwin_hall12(Xoshiro *g)
{
    int64_t sum = 0;
    for (int i = 0; i < 12; i++) sum += u24(g);
    return (float)((double)(sum - 6 * 16777216ll) * (1.0 / 16777216.0));
}

float p2g_round_fp16(double x)
{
    if (x != x) return (float)x;
    double a = fabs(x);
    if (a == 0.0) return (float)x;
    if (a >= 65520.0) return x < 0 ? -INFINITY : INFINITY;   /* beyond the largest fp16 plus half an ulp */
    int e;
    frexp(a, &e);                 /* a = f · 2^e, f in [0.5, 1): the leading bit has weight 2^(e-1) */
    int lead = e - 1;
    if (lead < -14) lead = -14;   /* fp16 subnormals share the quantum 2^-24 */
    double quantum = ldexp(1.0, lead - 10);
    double r = nearbyint(a / quantum) * quantum;   /* exact scaling by a power of two, then round half to even */
    return (float)(x < 0 ? -r : r);
}

void p2g_activations(uint64_t seed, uint64_t tensor_id, int M, int K, float *A)
{
    Xoshiro g;
    xo_seed(&g, seed, tensor_id);
    size_t n = (size_t)M * K;
    for (size_t i = 0; i < n; i++) {
        float x = irwin_hall12(&g);
        if (u24(&g) < 16777u) x *= 20.0f;   /* 16777 / 2^24 ≈ 0.001 */
        A[i] = x;
    }
}

void p2g_fv_weight(uint64_t seed, uint64_t tensor_id, int K, int N,
                   unsigned char *signs, unsigned char *flags, float *lo, float *hi)
{
    Xoshiro g;
    xo_seed(&g, seed, tensor_id);
    for (int n = 0; n < N; n++) {
        double l = 0.005 + 0.015 * unif(&g);
        double h = l * (2.0 + 2.0 * unif(&g));
        lo[n] = p2g_round_fp16(l);
        hi[n] = p2g_round_fp16(h);
    }
    memset(signs, 0, (size_t)K * (N / 4));
    memset(flags, 0, (size_t)K * (N / 8));
    /* One draw per weight: bits 40-63 decide zero (p = 0.4), bit 0 the sign, bits 8-31 hi vs lo (p = 1/3). */
    const uint64_t zero_cut = (uint64_t)(0.4 * 16777216.0);   /* 6710886 */
    const uint64_t hi_cut = 16777216u / 3u;                   /* 5592405 */
    for (int k = 0; k < K; k++) {
        unsigned char *srow = signs + (size_t)k * (N / 4);
        unsigned char *frow = flags + (size_t)k * (N / 8);
        for (int n = 0; n < N; n++) {
            uint64_t r = xo_next(&g);
            unsigned code = 1, flag = 0;            /* code = sign + 1 */
            if ((r >> 40) >= zero_cut) {
                code = (r & 1) ? 2u : 0u;
                flag = ((r >> 8) & 0xFFFFFFu) < hi_cut;
            }
            srow[n >> 2] |= (unsigned char)(code << (2 * (n & 3)));
            frow[n >> 3] |= (unsigned char)(flag << (n & 7));
        }
    }
}

void p2g_i8_weight(uint64_t seed, uint64_t tensor_id, int K, int N, signed char *q8, float *scales)
{
    Xoshiro g;
    xo_seed(&g, seed, tensor_id);
    for (int n = 0; n < N; n++) scales[n] = p2g_round_fp16(0.0005 + 0.0015 * unif(&g));
    size_t kn = (size_t)K * N;
    for (size_t i = 0; i < kn; i++) q8[i] = (signed char)((int)(u24(&g) % 255u) - 127);
}
