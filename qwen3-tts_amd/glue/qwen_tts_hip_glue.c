/*
 * qwen_tts_hip_glue.c — reference-side glue between qwen_tts_ctx_t (the reference's
 * qwen_tts.h) and libqwen_tts_hip.so (include/qwen_tts_hip.h).  A maintainer adds this
 * file to the reference's build, links libqwen_tts_hip.so, and calls these functions at
 * the places where the reference delegates to its CUDA backend.  Everything here is a field
 * copy plus the bookkeeping those call sites do (kv_len, dec_x); no arithmetic.
 */
#include "qwen_tts_hip_glue.h"

#include "ingot/safetensors.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* one matrix at precision prec; NULL w when that precision's pointer is absent */
static qwen_hip_mat_t hmat(const void *q4, const int8_t *i8, const float *sc, const uint16_t *bf, int prec) {
    qwen_hip_mat_t m = {NULL, NULL};
    if (prec == QWEN_HIP_Q4_0) m.w = q4;
    else if (prec == QWEN_HIP_INT8) { m.w = i8; m.scale = sc; }
    else m.w = bf;
    return m;
}

/* The layer records of a Talker (cp = 0) or CP (cp = 1) stack at the precision of layer
 * 0's q projection; -1 when any matrix of any layer lacks that precision (a mixed
 * model, e.g. the experimental q2 CP FFN: the CPU path keeps it). */
#define FILL_LAYER(dst, L, prec) do {                                                                  \
    (dst).q = hmat((L)->wq_q4, (L)->wq_int8, (L)->wq_scale, (L)->wq_bf16, prec);                          \
    (dst).k = hmat((L)->wk_q4, (L)->wk_int8, (L)->wk_scale, (L)->wk_bf16, prec);                          \
    (dst).v = hmat((L)->wv_q4, (L)->wv_int8, (L)->wv_scale, (L)->wv_bf16, prec);                          \
    (dst).o = hmat((L)->wo_q4, (L)->wo_int8, (L)->wo_scale, (L)->wo_bf16, prec);                          \
    (dst).gate_up = hmat((L)->gate_up_fused_q4, (L)->gate_up_fused_int8, (L)->gate_up_fused_scale,        \
                         (L)->gate_up_fused_bf16, prec);                                                  \
    (dst).down = hmat((L)->down_q4, (L)->down_int8, (L)->down_scale, (L)->down_bf16, prec);               \
    (dst).input_norm = (L)->input_norm; (dst).post_attn_norm = (L)->post_attn_norm;                       \
    (dst).q_norm = (L)->q_norm; (dst).k_norm = (L)->k_norm;                                                \
} while (0)

static int layer_complete(const qwen_hip_layer_t *l) {
    const qwen_hip_mat_t *m[6] = {&l->q, &l->k, &l->v, &l->o, &l->gate_up, &l->down};
    for (int i = 0; i < 6; i++) if (!m[i]->w) return 0;
    return l->input_norm && l->post_attn_norm && l->q_norm && l->k_norm;
}

static int talker_layers(const qwen_tts_ctx_t *ctx, qwen_hip_layer_t *out, int force_bf16) {
    const qwen_talker_layer_t *L0 = &ctx->layers[0];
    const int prec = force_bf16 ? QWEN_HIP_BF16 : L0->wq_q4 ? QWEN_HIP_Q4_0 : L0->wq_int8 ? QWEN_HIP_INT8 : QWEN_HIP_BF16;
    for (int l = 0; l < ctx->config.num_layers; l++) {
        const qwen_talker_layer_t *L = &ctx->layers[l];
        FILL_LAYER(out[l], L, prec);
        if (!layer_complete(&out[l])) return -1;
    }
    return prec;
}

void *qwen_hip_glue_talker_init(qwen_tts_ctx_t *ctx, int kv_max) {
    static qwen_hip_layer_t lay[QWEN_TTS_MAX_TALKER_LAYERS];
    const qwen_tts_config_t *c = &ctx->config;
    if (!qwen_hip_available() || c->num_layers > QWEN_TTS_MAX_TALKER_LAYERS) return NULL;
    const int prec = talker_layers(ctx, lay, 0);
    if (prec < 0) { fprintf(stderr, "hip: Talker weights of mixed precision; staying on the CPU path\n"); return NULL; }
    qwen_hip_talker_desc_t d;
    memset(&d, 0, sizeof d);
    d.hidden = c->hidden_size; d.inter = c->intermediate_size; d.n_heads = c->num_heads;
    d.n_kv_heads = c->num_kv_heads; d.head_dim = c->head_dim; d.n_layers = c->num_layers;
    d.kv_max = kv_max > 0 ? kv_max : ctx->kv_max;
    d.eps = c->rms_norm_eps; d.prec = prec; d.quantize_to = -1; d.layers = lay;
    d.final_norm = ctx->talker_norm;
    d.rope_cos = ctx->rope_cos; d.rope_sin = ctx->rope_sin; d.rope_len = ctx->rope_cache_len;
    return qwen_hip_talker_init(&d);          /* copies everything: lay may be reused */
}

int qwen_hip_glue_talker_step(void *state, qwen_tts_ctx_t *ctx, float *embed, float *hidden_out) {
    const int pos = ctx->kv_len;
    if (qwen_hip_talker_step(state, embed, hidden_out, pos) != 0) {
        fprintf(stderr, "hip: %s; staying on the CPU path\n", qwen_hip_last_error());
        return -1;
    }
    qwen_hip_talker_get_dec_x(state, ctx->dec_x);
    ctx->kv_len = pos + 1;
    return 0;
}

int qwen_hip_glue_upload_kv(void *state, qwen_tts_ctx_t *ctx, int prefill_len) {
    return qwen_hip_talker_upload_kv(state, ctx->kv_cache_k, ctx->kv_cache_v, ctx->kv_max, prefill_len);
}

int qwen_hip_glue_talker_prefill(void *state, qwen_tts_ctx_t *ctx, float *embeds, int seq) {
    static qwen_hip_layer_t bf[QWEN_TTS_MAX_TALKER_LAYERS];
    if (talker_layers(ctx, bf, 1) < 0) return -1;          /* the prefill runs on the bf16 weights (t.c:832-839) */
    if (qwen_hip_talker_prefill(state, bf, embeds, seq) != 0) return -1;
    ctx->kv_len = seq;
    qwen_hip_talker_get_dec_x(state, ctx->dec_x);
    return 0;
}

void *qwen_hip_glue_cp_init(qwen_tts_ctx_t *ctx) {
    static qwen_hip_layer_t lay[QWEN_TTS_MAX_CP_LAYERS];
    const qwen_tts_config_t *c = &ctx->config;
    if (!qwen_hip_available() || c->cp_num_layers > QWEN_TTS_MAX_CP_LAYERS) return NULL;
    const qwen_cp_layer_t *L0 = &ctx->cp_layers[0];
    const int prec = L0->wq_q4 ? QWEN_HIP_Q4_0 : L0->wq_int8 ? QWEN_HIP_INT8 : QWEN_HIP_BF16;
    for (int l = 0; l < c->cp_num_layers; l++) {
        const qwen_cp_layer_t *L = &ctx->cp_layers[l];
        if (L->gate_up_fused_q2 || L->down_q2) return NULL;   /* experimental q2 FFN: CPU path */
        FILL_LAYER(lay[l], L, prec);
        if (!layer_complete(&lay[l])) return NULL;
    }
    qwen_hip_cp_desc_t d;
    memset(&d, 0, sizeof d);
    d.cp.hidden = c->cp_hidden_size; d.cp.inter = c->cp_intermediate_size; d.cp.n_heads = c->cp_num_heads;
    d.cp.n_kv_heads = c->cp_num_kv_heads; d.cp.head_dim = c->cp_head_dim; d.cp.n_layers = c->cp_num_layers;
    d.cp.kv_max = ctx->cp_kv_max; d.cp.eps = c->rms_norm_eps; d.cp.prec = prec; d.cp.quantize_to = -1;
    d.cp.layers = lay; d.cp.final_norm = ctx->cp_norm;
    d.cp.rope_cos = ctx->cp_rope_cos; d.cp.rope_sin = ctx->cp_rope_sin; d.cp.rope_len = ctx->cp_rope_cache_len;
    d.codebook = c->codebook_size;
    d.lm_prec = ctx->cp_lm_head_q4[0] ? QWEN_HIP_Q4_0 : ctx->cp_lm_head_int8[0] ? QWEN_HIP_INT8 : QWEN_HIP_BF16;
    for (int g = 0; g < 15; g++) {
        d.lm_head[g] = hmat(ctx->cp_lm_head_q4[g], ctx->cp_lm_head_int8[g], ctx->cp_lm_head_scale[g],
                            ctx->cp_lm_head_bf16[g], d.lm_prec);
        if (!d.lm_head[g].w || !ctx->cp_codec_emb_bf16[g]) return NULL;
        d.cp_codec_emb[g] = ctx->cp_codec_emb_bf16[g];
    }
    d.talker_codec_emb = ctx->codec_embedding_bf16;
    d.codec_vocab = c->codec_vocab_size; d.talker_hidden = c->hidden_size; d.emb_dim = ctx->cp_emb_dim;
    if (ctx->cp_mtp_proj_int8) {
        d.mtp_prec = QWEN_HIP_INT8;
        d.mtp.w = ctx->cp_mtp_proj_int8; d.mtp.scale = ctx->cp_mtp_proj_scale;
    } else {
        d.mtp_prec = QWEN_HIP_BF16;
        d.mtp.w = ctx->cp_mtp_proj_bf16;        /* NULL when the hidden sizes agree: identity */
    }
    d.mtp_bias = ctx->cp_mtp_proj_bias;
    return qwen_hip_cp_init(&d);
}

int qwen_hip_glue_cp_predict(void *state, float *talker_hidden, int code0, int *out_codes) {
    return qwen_hip_cp_frame(state, talker_hidden, code0, out_codes);
}

int qwen_hip_glue_cp_step(void *state, qwen_tts_ctx_t *ctx, float *x, int pos) {
    if (qwen_hip_cp_step(state, x, pos) != 0) return -1;
    ctx->cp_kv_len = pos + 1;
    return 0;
}

int qwen_hip_glue_codec_sample(qwen_tts_ctx_t *ctx, int frame, int text_content_len, uint32_t *lcg) {
    const int expected = text_content_len * 3, start = expected * 2;
    float boost = 0.0f;
    if (expected > 0 && frame > start) {
        boost = 0.5f * (float)(frame - start);
        if (boost > 10.0f) boost = 10.0f;
    }
    float temp = ctx->temperature;
    int top_k = ctx->top_k;
    if (ctx->greedy_warmup > 0 && frame < ctx->greedy_warmup) { temp = 0.0f; top_k = 1; }
    return qwen_hip_op_codec_sample(ctx->logits, ctx->config.codec_vocab_size, frame, boost, temp, top_k, ctx->top_p,
                                    ctx->rep_penalty, ctx->prev_tokens, ctx->n_prev_tokens, lcg);
}

/* ---- speech decoder ----------------------------------------------------------------------- */
/* the getter of qwen_hip_sd_init over the reference's mmap: the tensor's own F32 bytes, as
 * get_f32 hands them to the CPU decoder (sd.c:77-80), checked for size and dtype */
static const float *glue_sd_get(void *user, const char *name, long long n_elems) {
    ingot_st *st = (ingot_st *)user;
    const ingot_st_tensor *t = ingot_st_find(st, name);
    if (!t || t->dtype != INGOT_DT_F32 || (long long)t->nelem != n_elems) return NULL;
    return (const float *)ingot_st_data(st, t);
}

void *qwen_hip_glue_sd_init(qwen_tts_ctx_t *ctx) {
    if (!ctx->speech_safetensors) return NULL;
    return qwen_hip_sd_init(glue_sd_get, ctx->speech_safetensors);
}

int qwen_hip_glue_sd_decode(void *state, const int *codes, int n_frames, float **audio_out, int *n_samples) {
    const int ns = n_frames * 1920;
    float *a = (float *)malloc((size_t)ns * sizeof(float));
    if (!a) return -1;
    const int got = qwen_hip_sd_decode(state, codes, n_frames, a, ns);
    if (got < 0) { free(a); return -1; }
    *audio_out = a;
    *n_samples = got;
    return 0;
}

/* ---- the backend vtable's HIP kind (qwen_tts_backend.h:34-49) ---------------------------- */
static void hip_backend_matvec_bf16(qwen_backend_t *b, float *y, const uint16_t *W, const float *x, int rows, int cols) {
    qwen_hip_matvec_bf16(b->impl, y, W, x, rows, cols);
}
static void hip_backend_matmat_bf16(qwen_backend_t *b, float *Y, const uint16_t *W, const float *X, int rows, int cols,
                                    int B) {
    qwen_hip_matmat_bf16(b->impl, Y, W, X, rows, cols, B);
}
static void hip_backend_free(qwen_backend_t *b) {
    if (!b) return;
    qwen_hip_free(b->impl);
    free(b);
}

qwen_backend_t *qwen_hip_glue_backend_new(void) {
    if (!qwen_hip_available()) return NULL;
    void *impl = qwen_hip_init();
    if (!impl) return NULL;
    qwen_backend_t *b = calloc(1, sizeof *b);
    if (!b) { qwen_hip_free(impl); return NULL; }
    b->kind = QWEN_BACKEND_HIP;
    b->name = "hip";
    b->impl = impl;
    b->matvec_bf16 = hip_backend_matvec_bf16;
    b->matmat_bf16 = hip_backend_matmat_bf16;
    b->free = hip_backend_free;
    return b;
}
