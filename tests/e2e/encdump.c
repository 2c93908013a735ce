/*  encdump.c – the reference engine's stages on one WAV file: log-mel, encoder, greedy decode.
 *
 *  Test infrastructure. oracle/Makefile links it with the reference's library sources in the same three ways as the
 *  reference CLI (its own GEMMs, the GPU library, the oracle), so tests can compare the encoder output (the frames
 *  after all 216 five-value linears and the projector) bit for bit, as well as the decoded token ids.
 *
 *  usage: encdump <weights_dir> <mono 16 kHz wav> <out.f32>
 *  Writes T × 640 fp32 encoder frames (phonon2.h:395, encoder.c:725-751) to out.f32 and prints "T <T>" and the
 *  token ids of p2_greedy_decode (phonon2.h:407) on stdout.
 *  ENCDUMP_REPEAT=n (default 1) runs p2_encoder n times on the same log-mel (the last run's frames are written) and
 *  prints the wall time of each run on stderr as "encoder_ms <ms>"; the first run of a GPU-linked build includes
 *  moving the weights to the device (unless P2_CACHE_CODES=1 moved them at load, weights.c:525-529). A GPU-linked
 *  build also prints, per run, "gpu_stats ..." from the library's call accounting: the time inside its GEMM entries
 *  (PCIe copies and kernels), the uploads among it, and the bytes copied each way.
 */
#include "phonon2.h"

#include <stdio.h>
#include <stdlib.h>
#include <time.h>

/* The GPU GEMM library's call accounting (include/p2_blas.h), present only in the GPU-linked builds. */
void p2_gpu_stats_take(double out[9]) __attribute__((weak));

static double now_ms(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6;
}

int main(int argc, char **argv)
{
    if (argc != 4) {
        fprintf(stderr, "usage: %s <weights_dir> <audio.wav> <out.f32>\n", argv[0]);
        return 2;
    }
    P2Engine *e = p2_engine_open(argv[1]);
    if (!e) return 1;
    float *audio = NULL;
    int n = 0, rate = 0, channels = 0;
    if (p2_wav_read(argv[2], &audio, &n, &rate, &channels) != 0 || channels != 1 || rate != P2_SAMPLE_RATE) {
        fprintf(stderr, "%s: a mono %d Hz WAV is expected\n", argv[2], P2_SAMPLE_RATE);
        return 1;
    }
    float *mel = NULL;
    int frames = 0;
    if (p2_mel_spectrogram(audio, n, &mel, &frames) != 0) return 1;
    const P2Model *m = p2_engine_model(e);
    float *enc = NULL;
    int T = 0;
    const char *rep = getenv("ENCDUMP_REPEAT");
    const int repeat = rep && atoi(rep) > 0 ? atoi(rep) : 1;
    if (p2_gpu_stats_take) {   /* what loading did (the uploads of P2_CACHE_CODES=1) is not a run's */
        double st[9];
        p2_gpu_stats_take(st);
        fprintf(stderr, "gpu_stats_load upload_ms %.3f\n", st[6]);
    }
    for (int r = 0; r < repeat; r++) {
        free(enc);
        enc = NULL;
        const double t0 = now_ms();
        if (p2_encoder(m, mel, frames, &enc, &T) != 0) return 1;
        fprintf(stderr, "encoder_ms %.3f\n", now_ms() - t0);
        if (p2_gpu_stats_take) {
            double st[9];
            p2_gpu_stats_take(st);
            fprintf(stderr, "gpu_stats fvb_calls %.0f fvb_ms %.3f q8b_calls %.0f q8b_ms %.3f sgemm_calls %.0f "
                            "sgemm_ms %.3f upload_ms %.3f h2d_mb %.3f d2h_mb %.3f\n",
                    st[0], st[1], st[2], st[3], st[4], st[5], st[6], st[7], st[8]);
        }
    }
    FILE *f = fopen(argv[3], "wb");
    if (!f || fwrite(enc, sizeof(float), (size_t)T * P2_JOINT_DIM, f) != (size_t)T * P2_JOINT_DIM) return 1;
    fclose(f);
    P2Token *toks = NULL;
    int nt = p2_greedy_decode(m, enc, T, &toks);
    printf("T %d\n", T);
    for (int i = 0; i < nt; i++) printf("%d%s", toks[i].id, i + 1 < nt ? " " : "\n");
    if (nt == 0) printf("\n");
    free(toks);
    free(enc);
    free(mel);
    free(audio);
    p2_engine_close(e);
    return 0;
}
