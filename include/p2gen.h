/*  p2gen.h – seeded synthetic inputs for the five-value GEMM workloads (activations and five-value weights).
 *
 *  No counterpart in the reference's library: bench_gemm.c:15-29 draws its planes from rand(), which is neither
 *  portable nor seedable per tensor. These generators are portable integer arithmetic (SplitMix64 seeding
 *  xoshiro256**, Irwin–Hall(12) normals, fp16 rounding done by hand), so the same (seed, tensor id) gives the same
 *  bytes on every host, and every consumer (tests, benchmark, CPU baseline) can regenerate its inputs.
 *
 *  Weight statistics follow the five-value container: per output column n, lo ~ U(0.005, 0.02) and
 *  hi = lo · U(2, 4), both rounded to fp16 values as the container stores them (fermion_container.py:32-33);
 *  each weight is 0 with p = 0.4, ±lo with p = 0.4 and ±hi with p = 0.2, signs equiprobable, flag 0 on zeros
 *  (fermion_container.py:35-36). Planes are packed as convert_weights.py:114-125 packs them.
 */
#ifndef P2GEN_H
#define P2GEN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A[M][K] fp32, row stride K: Irwin–Hall(12) normals (mean 0, variance 1), each entry multiplied by 20 with
 * probability 0.001. */
void p2g_activations(uint64_t seed, uint64_t tensor_id, int M, int K, float *A);

/* A five-value weight [K, N]: signs [K][N/4], flags [K][N/8], lo[N], hi[N]. N % 8 == 0. */
void p2g_fv_weight(uint64_t seed, uint64_t tensor_id, int K, int N,
                   unsigned char *signs, unsigned char *flags, float *lo, float *hi);

/* An int8 weight table [K][N] (values uniform in [-127, 127]) with one fp32 scale per column, U(0.0005, 0.002)
 * rounded to fp16 – the shape of the reference's P2_W_I8 weights (phonon2.h:110-113). */
void p2g_i8_weight(uint64_t seed, uint64_t tensor_id, int K, int N, signed char *q8, float *scales);

/* Nearest fp16 value (round half to even) of x, returned widened to float. */
float p2g_round_fp16(double x);

#ifdef __cplusplus
}
#endif

#endif /* P2GEN_H */
