/*  ref_block.c – the reference engine's own conformer block as a callable library function.
 *
 *  TEST INFRASTRUCTURE ONLY. The block (encoder.c:617-625) and its attention and convolution pieces
 *  (encoder.c:366-613) are static functions of the reference's encoder.c, so this file includes that source file
 *  from the reference tree (oracle/Makefile passes -I to it; nothing of it is copied here) and exports thin entry
 *  points over those functions with plain pointers:
 *
 *    refblock_run              conformer_block (encoder.c:617-625) on x [T, 1024] in place, with the positional
 *                              rows pe [2T−1, 1024]; five-value weights as their sign/flag planes and lo/hi; or
 *                              one of its five steps (stage 0..4: feed_forward, self_attention, conv_module,
 *                              feed_forward, the final LayerNorm)
 *    refblock_pos_encoding     rel_pos_encoding (encoder.c:79-96), into a caller buffer
 *    refblock_gather_heads     gather_heads (encoder.c:366-404)
 *    refblock_transpose_pos    transpose_pos (encoder.c:406-423)
 *    refblock_combine_softmax  combine_softmax (encoder.c:425-450), scale 1/sqrt(128)
 *    refblock_concat_heads     concat_heads (encoder.c:452-466), fp32 rows
 *    refblock_glu              glu_to_channel_major (encoder.c:543-555)
 *    refblock_cm_to_rows       channel_major_to_rows (encoder.c:557-571), fp32 rows
 *    refblock_add_residual     add_residual (encoder.c:271-275)
 *
 *  oracle/Makefile links it twice: with the reference's blas.c (on x86 the exact route only, blas.c:1043-1045, so
 *  the block takes its fp32 path) and with the oracle's drop-in for the quantised GEMMs (p2oracle_blas.c: the block
 *  takes its int8 path in the mode P2_GEMM names).
 */
#include "encoder.c"

typedef struct {
    const unsigned char *signs, *flags;
    const float *lo, *hi;
    int K, N;
} RefFv;

typedef struct {
    const float *norm_ff1_w, *norm_ff1_b;
    RefFv ff1_l1, ff1_l2;
    const float *norm_sa_w, *norm_sa_b;
    RefFv qkv, pos, out;
    const float *bias_u, *bias_v;
    const float *norm_conv_w, *norm_conv_b;
    RefFv pw1, pw2;
    const float *dw_w, *dw_b;
    const float *norm_ff2_w, *norm_ff2_b;
    RefFv ff2_l1, ff2_l2;
    const float *norm_out_w, *norm_out_b;
} RefBlock;

static Weight fv_weight_of(RefFv w)
{
    Weight x;
    memset(&x, 0, sizeof x);
    x.kind = P2_W_FV;
    x.K = w.K;
    x.N = w.N;
    x.signs = w.signs;
    x.flags = w.flags;
    x.lo = w.lo;
    x.hi = w.hi;
    return x;
}

static void block_of(const RefBlock *b, ConformerBlock *blk)
{
    memset(blk, 0, sizeof *blk);
    blk->norm_ff1_w = b->norm_ff1_w; blk->norm_ff1_b = b->norm_ff1_b;
    blk->ff1.linear1_w = fv_weight_of(b->ff1_l1); blk->ff1.linear2_w = fv_weight_of(b->ff1_l2);
    blk->norm_sa_w = b->norm_sa_w; blk->norm_sa_b = b->norm_sa_b;
    blk->mha.qkv_w = fv_weight_of(b->qkv); blk->mha.pos_w = fv_weight_of(b->pos); blk->mha.out_w = fv_weight_of(b->out);
    blk->mha.bias_u = b->bias_u; blk->mha.bias_v = b->bias_v;
    blk->norm_conv_w = b->norm_conv_w; blk->norm_conv_b = b->norm_conv_b;
    blk->conv.pw1_w = fv_weight_of(b->pw1); blk->conv.pw2_w = fv_weight_of(b->pw2);
    blk->conv.dw_w = b->dw_w; blk->conv.dw_b = b->dw_b;
    blk->norm_ff2_w = b->norm_ff2_w; blk->norm_ff2_b = b->norm_ff2_b;
    blk->ff2.linear1_w = fv_weight_of(b->ff2_l1); blk->ff2.linear2_w = fv_weight_of(b->ff2_l2);
    blk->norm_out_w = b->norm_out_w; blk->norm_out_b = b->norm_out_b;
}

/* stage < 0: the whole block; 0..4: one of its five steps (encoder.c:619-623) on x */
int refblock_run(const RefBlock *b, const float *pe, float *x, int T, int stage)
{
    ConformerBlock blk;
    block_of(b, &blk);
    CfmWS ws;
    ws.cap = conformer_ws_peak(T);
    ws.buf = (float *)malloc(ws.cap * sizeof(float));
    if (!ws.buf) return -1;
    switch (stage) {
    case 0: feed_forward(blk.norm_ff1_w, blk.norm_ff1_b, &blk.ff1, x, T, &ws); break;
    case 1: self_attention(blk.norm_sa_w, blk.norm_sa_b, &blk.mha, pe, x, T, &ws); break;
    case 2: conv_module(blk.norm_conv_w, blk.norm_conv_b, &blk.conv, x, T, &ws); break;
    case 3: feed_forward(blk.norm_ff2_w, blk.norm_ff2_b, &blk.ff2, x, T, &ws); break;
    case 4: p2_layer_norm_rows_inplace(x, blk.norm_out_w, blk.norm_out_b, T, P2_D_MODEL); break;
    default: conformer_block(&blk, pe, x, T, &ws); break;
    }
    free(ws.buf);
    return 0;
}

void refblock_pos_encoding(int T, float *out)
{
    float *pe = rel_pos_encoding(T);
    memcpy(out, pe, (size_t)(2 * T - 1) * P2_D_MODEL * sizeof(float));
    free(pe);
}

void refblock_gather_heads(const float *QKV, const float *bias_u, const float *bias_v, float *Q_u, float *Q_v,
                           float *K_t, float *V_h, int T)
{
    struct gather_args g = { QKV, bias_u, bias_v, Q_u, Q_v, K_t, V_h, T };
    gather_heads(0, T, &g);
}

void refblock_transpose_pos(const float *P, float *P_t, int L)
{
    struct ptrans_args pt = { P, P_t, L };
    transpose_pos(0, L, &pt);
}

void refblock_combine_softmax(float *ac, const float *bd, int T)
{
    struct scores_args sc = { ac, bd, T, 1.0f / sqrtf((float)P2_HEAD_DIM) };
    combine_softmax(0, P2_N_HEADS * T, &sc);
}

void refblock_concat_heads(const float *attn_h, float *attn, int T)
{
    struct concat_args cc = { attn_h, attn, NULL, T };
    concat_heads(0, T, &cc);
}

void refblock_glu(const float *pw1, float *gated, int T)
{
    struct glu_args g = { pw1, gated, T };
    glu_to_channel_major(0, P2_D_MODEL, &g);
}

void refblock_cm_to_rows(const float *dw, float *act, int T)
{
    struct ct_args ct = { dw, act, NULL, T };
    channel_major_to_rows(0, T, &ct);
}

void refblock_add_residual(float *x, const float *y, int T, float alpha)
{
    add_residual(x, y, T, alpha);
}
