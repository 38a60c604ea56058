/*
 * ref_harness.c — test-only driver around the REFERENCE C engine.
 *
 * Built by oracle/Makefile together with the reference's own sources, compiled where
 * they lie under /root/reference (qwen_tts_talker.c, qwen_tts_code_predictor.c,
 * qwen_tts_kernels*.c, qwen_tts_thread.c, ingot core) into oracle/_ref/libqwen_ref.so.
 * Nothing here re-implements the model: it builds a qwen_tts_ctx_t the way
 * qwen_tts_load_ex does for the Talker/CP half (qwen_tts.c:556-696: config fields,
 * ingot_st_open_dir, qwen_talker_load, qwen_cp_load) and exposes plain-pointer
 * accessors so pytest can (a) run the reference's own qwen_talker_step /
 * qwen_cp_predict / quantizers as the checker and (b) hand the reference-loaded,
 * reference-quantized weight bytes to the HIP library under test.
 *
 * TEST INFRASTRUCTURE ONLY: tests/, the smoke check and bench.py's cpu_baseline leg
 * are the only callers.  It is never on the product path.
 */
#include "qwen_tts.h"
#include "qwen_tts_kernels.h"
#include "ingot/safetensors.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* The reference declares these at their call sites rather than in a header
 * (qwen_tts.c:236-241); same prototypes here. */
extern int qwen_talker_load(qwen_tts_ctx_t *ctx);
extern int qwen_cp_load(qwen_tts_ctx_t *ctx);
extern int qwen_talker_step(qwen_tts_ctx_t *ctx, float *embed, float *hidden_out);
extern int qwen_cp_predict(qwen_tts_ctx_t *ctx, float *talker_hidden, int code0, int *out_codes);
extern int qwen_talker_prefill(qwen_tts_ctx_t *ctx, float *input_embeds, int seq_len);

typedef struct {
    qwen_tts_ctx_t *ctx;
    int cfg[16];
} ref_handle_t;

enum { RC_HIDDEN, RC_LAYERS, RC_HEADS, RC_KVHEADS, RC_HEADDIM, RC_INTER, RC_VOCAB, RC_CODEBOOK,
       RC_TEXT_HIDDEN, RC_CP_HIDDEN, RC_CP_LAYERS, RC_CP_HEADS, RC_CP_KVHEADS, RC_CP_HEADDIM,
       RC_CP_INTER, RC_N };

/* cfg: int[15] in the RC_* order; eps/theta passed separately. */
void *ref_open(const char *dir, const int *cfg, float eps, float theta,
               int use_int8, int use_int4, int threads) {
    ref_handle_t *h = (ref_handle_t *)calloc(1, sizeof(*h));
    qwen_tts_ctx_t *ctx = (qwen_tts_ctx_t *)calloc(1, sizeof(qwen_tts_ctx_t));
    if (!h || !ctx) { free(h); free(ctx); return NULL; }
    memcpy(h->cfg, cfg, RC_N * sizeof(int));
    qwen_tts_config_t *c = &ctx->config;
    c->hidden_size = cfg[RC_HIDDEN];
    c->num_layers = cfg[RC_LAYERS];
    c->num_heads = cfg[RC_HEADS];
    c->num_kv_heads = cfg[RC_KVHEADS];
    c->head_dim = cfg[RC_HEADDIM];
    c->intermediate_size = cfg[RC_INTER];
    c->codec_vocab_size = cfg[RC_VOCAB];
    c->codebook_size = cfg[RC_CODEBOOK];
    c->text_hidden_size = cfg[RC_TEXT_HIDDEN];
    c->cp_hidden_size = cfg[RC_CP_HIDDEN];
    c->cp_num_layers = cfg[RC_CP_LAYERS];
    c->cp_num_heads = cfg[RC_CP_HEADS];
    c->cp_num_kv_heads = cfg[RC_CP_KVHEADS];
    c->cp_head_dim = cfg[RC_CP_HEADDIM];
    c->cp_intermediate_size = cfg[RC_CP_INTER];
    c->rms_norm_eps = eps;
    c->rope_theta = theta;
    ctx->silent = 1;
    ctx->use_int8 = use_int8;
    ctx->use_int4 = use_int4;
    ctx->temperature = 0.0f;
    ctx->rep_penalty = 1.0f;

    qwen_set_threads(threads > 0 ? threads : 1);

    char err[512];
    ingot_st *st = NULL;
    if (ingot_st_open_dir(&st, dir, err, sizeof err) != 0) {
        fprintf(stderr, "ref_open: %s\n", err);
        free(ctx); free(h); return NULL;
    }
    ctx->safetensors = st;
    if (qwen_talker_load(ctx) != 0 || qwen_cp_load(ctx) != 0) {
        fprintf(stderr, "ref_open: load failed\n");
        free(ctx); free(h); return NULL;
    }
    h->ctx = ctx;
    return h;
}

/* the reference context of a handle (for the glue under test) */
void *ref_ctx(void *hp) { return ((ref_handle_t *)hp)->ctx; }

void ref_set_threads(int n) { qwen_set_threads(n > 0 ? n : 1); }

/* ---- Talker ------------------------------------------------------------ */
int ref_talker_step(void *hp, const float *embed, float *hidden_out) {
    ref_handle_t *h = (ref_handle_t *)hp;
    /* qwen_talker_step copies embed into dec_x; it does not write through it. */
    return qwen_talker_step(h->ctx, (float *)embed, hidden_out);
}

/* Per-layer residuals: run the step with num_layers truncated to l+1 (l = 0..L-1);
 * ctx->dec_x then holds the residual after layer l (t.c:659-665).  Each truncated
 * run rewrites the KV slot at `pos` for layers <= l with the same bytes, so the final
 * full-depth run leaves the cache exactly as a single step would. */
int ref_talker_step_layers(void *hp, const float *embed, float *residuals /*[L][H]*/,
                           float *hidden_out) {
    ref_handle_t *h = (ref_handle_t *)hp;
    qwen_tts_ctx_t *ctx = h->ctx;
    int L = ctx->config.num_layers, H = ctx->config.hidden_size;
    int pos = ctx->kv_len;
    for (int l = 0; l < L; l++) {
        ctx->config.num_layers = l + 1;
        ctx->kv_len = pos;
        int rc = qwen_talker_step(ctx, (float *)embed, hidden_out);
        ctx->config.num_layers = L;
        if (rc != 0) return rc;
        memcpy(residuals + (size_t)l * H, ctx->dec_x, (size_t)H * sizeof(float));
    }
    ctx->kv_len = pos;
    return qwen_talker_step(ctx, (float *)embed, hidden_out);
}

/* The reference prefill (t.c:730-1038) over seq positions; embeds f32[seq][hidden] (the
 * reference copies it into its residual buffer and does not write through it).  Sets
 * kv_len = seq and dec_x = the last position's residual. */
int ref_talker_prefill(void *hp, const float *embeds, int seq) {
    ref_handle_t *h = (ref_handle_t *)hp;
    return qwen_talker_prefill(h->ctx, (float *)embeds, seq);
}

void ref_get_dec_x(void *hp, float *out) {
    ref_handle_t *h = (ref_handle_t *)hp;
    memcpy(out, h->ctx->dec_x, (size_t)h->ctx->config.hidden_size * sizeof(float));
}
/* Grow the reference's Talker KV cache to hold at least n positions before the caller
 * writes rows into it (the reference grows by doubling when a step needs room,
 * qwen_tts_talker.c:257-280; its buffers are released with free()).  Keeps rows
 * [0, kv_len).  Returns 0, or -1 when out of memory. */
int ref_kv_reserve(void *hp, int n) {
    qwen_tts_ctx_t *ctx = ((ref_handle_t *)hp)->ctx;
    if (n <= ctx->kv_max) return 0;
    int nm = ctx->kv_max;
    while (nm < n) nm *= 2;
    const size_t kvd = (size_t)ctx->config.num_kv_heads * ctx->config.head_dim, L = (size_t)ctx->config.num_layers;
    void *nk = NULL, *nv = NULL;
    if (posix_memalign(&nk, 64, L * nm * kvd * sizeof(uint16_t)) || posix_memalign(&nv, 64, L * nm * kvd * sizeof(uint16_t))) {
        free(nk); free(nv); return -1;
    }
    for (size_t l = 0; l < L; l++) {
        memcpy((uint16_t *)nk + l * nm * kvd, ctx->kv_cache_k + l * ctx->kv_max * kvd, (size_t)ctx->kv_len * kvd * 2);
        memcpy((uint16_t *)nv + l * nm * kvd, ctx->kv_cache_v + l * ctx->kv_max * kvd, (size_t)ctx->kv_len * kvd * 2);
    }
    free(ctx->kv_cache_k); free(ctx->kv_cache_v);
    ctx->kv_cache_k = (uint16_t *)nk; ctx->kv_cache_v = (uint16_t *)nv;
    ctx->kv_max = nm;
    return 0;
}
int ref_kv_len(void *hp) { return ((ref_handle_t *)hp)->ctx->kv_len; }
void ref_set_kv_len(void *hp, int n) { ((ref_handle_t *)hp)->ctx->kv_len = n; }
int ref_kv_max(void *hp) { return ((ref_handle_t *)hp)->ctx->kv_max; }
const uint16_t *ref_kv_k(void *hp) { return ((ref_handle_t *)hp)->ctx->kv_cache_k; }
const uint16_t *ref_kv_v(void *hp) { return ((ref_handle_t *)hp)->ctx->kv_cache_v; }
const float *ref_rope_cos(void *hp) { return ((ref_handle_t *)hp)->ctx->rope_cos; }
const float *ref_rope_sin(void *hp) { return ((ref_handle_t *)hp)->ctx->rope_sin; }
int ref_rope_len(void *hp) { return ((ref_handle_t *)hp)->ctx->rope_cache_len; }
const float *ref_talker_norm(void *hp) { return ((ref_handle_t *)hp)->ctx->talker_norm; }
const uint16_t *ref_codec_head(void *hp) { return ((ref_handle_t *)hp)->ctx->codec_head_bf16; }
const uint16_t *ref_codec_emb(void *hp) { return ((ref_handle_t *)hp)->ctx->codec_embedding_bf16; }

/* Weight accessor.  which: 0 q,1 k,2 v,3 o,4 gate_up (interleaved),5 down;
 * kind: 0 bf16, 1 int8, 2 int8 scale, 3 q4 blocks; norms via which 10..13
 * (10 input_norm, 11 post_attn_norm, 12 q_norm, 13 k_norm).  cp selects CP layers. */
const void *ref_layer_ptr(void *hp, int cp, int layer, int which, int kind) {
    qwen_tts_ctx_t *ctx = ((ref_handle_t *)hp)->ctx;
#define PICK(L) do { \
    switch (which) { \
    case 0: return kind==0?(const void*)L->wq_bf16:kind==1?(const void*)L->wq_int8:kind==2?(const void*)L->wq_scale:(const void*)L->wq_q4; \
    case 1: return kind==0?(const void*)L->wk_bf16:kind==1?(const void*)L->wk_int8:kind==2?(const void*)L->wk_scale:(const void*)L->wk_q4; \
    case 2: return kind==0?(const void*)L->wv_bf16:kind==1?(const void*)L->wv_int8:kind==2?(const void*)L->wv_scale:(const void*)L->wv_q4; \
    case 3: return kind==0?(const void*)L->wo_bf16:kind==1?(const void*)L->wo_int8:kind==2?(const void*)L->wo_scale:(const void*)L->wo_q4; \
    case 4: return kind==0?(const void*)L->gate_up_fused_bf16:kind==1?(const void*)L->gate_up_fused_int8:kind==2?(const void*)L->gate_up_fused_scale:(const void*)L->gate_up_fused_q4; \
    case 5: return kind==0?(const void*)L->down_bf16:kind==1?(const void*)L->down_int8:kind==2?(const void*)L->down_scale:(const void*)L->down_q4; \
    case 10: return L->input_norm; case 11: return L->post_attn_norm; \
    case 12: return L->q_norm; case 13: return L->k_norm; \
    default: return NULL; } } while (0)
    if (cp) { qwen_cp_layer_t *L = &ctx->cp_layers[layer]; PICK(L); }
    else    { qwen_talker_layer_t *L = &ctx->layers[layer]; PICK(L); }
#undef PICK
}

/* ---- Code Predictor ---------------------------------------------------- */
int ref_cp_predict(void *hp, const float *talker_hidden, int code0, int *out_codes) {
    return qwen_cp_predict(((ref_handle_t *)hp)->ctx, (float *)talker_hidden, code0, out_codes);
}
const float *ref_cp_norm(void *hp) { return ((ref_handle_t *)hp)->ctx->cp_norm; }
const uint16_t *ref_cp_kv_k(void *hp) { return ((ref_handle_t *)hp)->ctx->cp_kv_k; }
const uint16_t *ref_cp_kv_v(void *hp) { return ((ref_handle_t *)hp)->ctx->cp_kv_v; }
int ref_cp_kv_max(void *hp) { return ((ref_handle_t *)hp)->ctx->cp_kv_max; }
const float *ref_cp_rope_cos(void *hp) { return ((ref_handle_t *)hp)->ctx->cp_rope_cos; }
const float *ref_cp_rope_sin(void *hp) { return ((ref_handle_t *)hp)->ctx->cp_rope_sin; }
const float *ref_cp_dec_x(void *hp) { return ((ref_handle_t *)hp)->ctx->cp_dec_x; }
/* g in 0..14; kind 0 bf16, 1 int8, 2 scale, 3 q4 */
const void *ref_cp_lm_head(void *hp, int g, int kind) {
    qwen_tts_ctx_t *ctx = ((ref_handle_t *)hp)->ctx;
    return kind == 0 ? (const void *)ctx->cp_lm_head_bf16[g] : kind == 1 ? (const void *)ctx->cp_lm_head_int8[g]
         : kind == 2 ? (const void *)ctx->cp_lm_head_scale[g] : (const void *)ctx->cp_lm_head_q4[g];
}
const uint16_t *ref_cp_codec_emb(void *hp, int g) { return ((ref_handle_t *)hp)->ctx->cp_codec_emb_bf16[g]; }
int ref_cp_emb_dim(void *hp) { return ((ref_handle_t *)hp)->ctx->cp_emb_dim; }
/* kind 0 bf16 weight, 1 int8, 2 scale, 3 f32 bias */
const void *ref_cp_mtp(void *hp, int kind) {
    qwen_tts_ctx_t *ctx = ((ref_handle_t *)hp)->ctx;
    return kind == 0 ? (const void *)ctx->cp_mtp_proj_bf16 : kind == 1 ? (const void *)ctx->cp_mtp_proj_int8
         : kind == 2 ? (const void *)ctx->cp_mtp_proj_scale : (const void *)ctx->cp_mtp_proj_bias;
}

/* ---- Greedy codec-head rule (qwen_tts.c:1649-1694, qwen_tts_sampling.c:160-182) --
 * Runs the reference's own bf16 matvec and qwen_tts_sample(temp=0). */
extern int qwen_tts_sample(float *logits, int vocab_size, float temp, int top_k, float top_p,
                           float rep_penalty, int *prev_tokens, int n_prev);
int ref_codec_greedy(void *hp, const float *hidden, int frame, float *logits_out) {
    qwen_tts_ctx_t *ctx = ((ref_handle_t *)hp)->ctx;
    int V = ctx->config.codec_vocab_size, H = ctx->config.hidden_size;
    float *lg = (float *)malloc((size_t)V * sizeof(float));
    qwen_matvec_bf16(lg, ctx->codec_head_bf16, hidden, V, H);
    for (int t = 0; t < V; t++) {
        if (lg[t] > 100.0f) lg[t] = 100.0f;
        if (lg[t] < -100.0f) lg[t] = -100.0f;
    }
    for (int t = 2048; t < V; t++) if (t != QWEN_TTS_CODEC_EOS) lg[t] = -1e30f;
    if (frame < 2) lg[QWEN_TTS_CODEC_EOS] = -1e30f;
    if (logits_out) memcpy(logits_out, lg, (size_t)V * sizeof(float));
    int tok = qwen_tts_sample(lg, V, 0.0f, 1, 1.0f, 1.0f, NULL, 0);
    free(lg);
    return tok;
}

/* ---- Kernel-level passthroughs used as the checker ----------------------- */
void ref_quantize_int8(const uint16_t *src, int rows, int cols, int8_t *dst, float *scale) {
    qwen_quantize_bf16_to_int8(src, rows, cols, dst, scale);
}
void ref_quantize_q4_0(const uint16_t *src, int rows, int cols, void *dst) {
    qwen_quantize_bf16_to_q4_0(src, rows, cols, (q4_0_block_t *)dst);
}
void ref_matvec_bf16(float *y, const uint16_t *W, const float *x, int rows, int cols) {
    qwen_matvec_bf16(y, W, x, rows, cols);
}
void ref_matmat_bf16(float *Y, const uint16_t *W, const float *X, int rows, int cols, int B) {
    qwen_matmat_bf16(Y, W, X, rows, cols, B);
}
void ref_matvec_int8(float *y, const int8_t *W, const float *s, const float *x, int rows, int cols) {
    qwen_matvec_int8(y, W, s, x, rows, cols);
}
void ref_matvec_q4_0(float *y, const void *W, const float *x, int rows, int cols) {
    qwen_matvec_q4_0(y, (const q4_0_block_t *)W, x, rows, cols);
}
void ref_attention_bf16kv(float *out, const float *Q, const uint16_t *K, const uint16_t *V,
                          int seq_q, int seq_k, int nh, int nkv, int hd, float scale, int q_off) {
    qwen_causal_attention_bf16kv(out, Q, K, V, seq_q, seq_k, nh, nkv, hd, scale, q_off);
}
void ref_rms_norm(float *out, const float *x, const float *w, int seq, int dim, float eps) {
    qwen_rms_norm(out, x, w, seq, dim, eps);
}
void ref_swiglu(float *gu, int n) {
    float *tmp = (float *)malloc((size_t)n * sizeof(float));
    qwen_swiglu_inplace(gu, tmp, n);
    free(tmp);
}
int ref_argmax_matvec_bf16(const float *x, const uint16_t *W, int in_dim, int out_dim) {
    return qwen_argmax_matvec_bf16(x, W, in_dim, out_dim);
}
int ref_argmax_matvec_int8(const float *x, const int8_t *W, const float *s, int in_dim, int out_dim) {
    return qwen_argmax_matvec_int8(x, W, s, in_dim, out_dim);
}
int ref_argmax_matvec_q4_0(const float *x, const void *W, int in_dim, int out_dim) {
    return qwen_argmax_matvec_q4_0(x, (const q4_0_block_t *)W, in_dim, out_dim);
}
uint16_t ref_f32_to_f16(float f) { return qwen_f32_to_f16(f); }
/* qwen_tts_sample with the thread-local LCG state set from and returned to *seed. */
extern void qwen_set_seed(uint32_t seed);
extern uint32_t qwen_get_seed(void);
int ref_sample(float *logits, int n, float temp, int top_k, float top_p, float rep, int *prev, int n_prev,
               uint32_t *seed) {
    qwen_set_seed(*seed);
    int t = qwen_tts_sample(logits, n, temp, top_k, top_p, rep, prev, n_prev);
    *seed = qwen_get_seed();
    return t;
}
float ref_f16_to_f32(uint16_t h) { return qwen_f16_to_f32(h); }

/* Wall-clock helper for the CPU baseline: n consecutive Talker steps, returns seconds. */
double ref_time_talker_steps(void *hp, const float *embeds, int n, float *hidden_out) {
    struct timespec t0, t1;
    ref_handle_t *h = (ref_handle_t *)hp;
    int H = h->ctx->config.hidden_size;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (int i = 0; i < n; i++)
        qwen_talker_step(h->ctx, (float *)(embeds + (size_t)i * H), hidden_out);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

/* Same, with each step's wall time in seconds in times[n] (median / p90 for the baseline). */
void ref_time_talker_steps_each(void *hp, const float *embeds, int n, float *hidden_out, double *times) {
    ref_handle_t *h = (ref_handle_t *)hp;
    int H = h->ctx->config.hidden_size;
    for (int i = 0; i < n; i++) {
        struct timespec t0, t1;
        clock_gettime(CLOCK_MONOTONIC, &t0);
        qwen_talker_step(h->ctx, (float *)(embeds + (size_t)i * H), hidden_out);
        clock_gettime(CLOCK_MONOTONIC, &t1);
        times[i] = (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
    }
}

/* compiler that built this harness and the reference objects (same make run) */
const char *ref_build_info(void) { return "gcc " __VERSION__; }

/* per-head RMSNorm passthrough (checker for the device KV append) */
void ref_rms_norm_per_head(float *x, const float *w, int seq, int n_heads, int head_dim, float eps) {
    qwen_rms_norm_per_head(x, w, seq, n_heads, head_dim, eps);
}

/* ---- speech decoder (qwen_tts_speech_decoder.c) --------------------------------------
 * The reference's own loader and one-shot decode over an F32 safetensors file holding the
 * decoder's tensors (qwen_speech_decoder_load reads them by name, sd.c:372-578).  The
 * config fields the decoder reads are set to the 12 Hz codec's values (qwen_tts.c:207-223). */
extern int qwen_speech_decoder_load(qwen_tts_ctx_t *ctx);
extern int qwen_speech_decoder_decode(qwen_tts_ctx_t *ctx, const int *codes, int n_frames, float **audio_out,
                                      int *n_samples);

void *ref_sd_open(const char *path, int threads) {
    qwen_tts_ctx_t *ctx = calloc(1, sizeof *ctx);
    if (!ctx) return NULL;
    qwen_tts_config_t *c = &ctx->config;
    c->codebook_size = 2048;
    c->dec_num_layers = 8;
    c->dec_head_dim = 64;
    c->dec_rope_theta = 10000.0f;
    c->dec_rms_norm_eps = 1e-5f;
    ctx->silent = 1;
    qwen_set_threads(threads > 0 ? threads : 1);
    char err[512];
    ingot_st *st = NULL;
    if (ingot_st_open(&st, path, err, sizeof err) != 0) {
        fprintf(stderr, "ref_sd_open: %s\n", err);
        free(ctx);
        return NULL;
    }
    ctx->speech_safetensors = st;
    if (qwen_speech_decoder_load(ctx) != 0) {
        fprintf(stderr, "ref_sd_open: load failed\n");
        free(ctx);
        return NULL;
    }
    return ctx;
}

/* audio of n_frames x 16 codes into out[cap]; returns the sample count, or -1 */
int ref_sd_decode(void *h, const int *codes, int n_frames, float *out, int cap) {
    float *audio = NULL;
    int n = 0;
    if (qwen_speech_decoder_decode((qwen_tts_ctx_t *)h, codes, n_frames, &audio, &n) != 0 || !audio) return -1;
    if (n > cap) n = cap;
    memcpy(out, audio, (size_t)n * sizeof(float));
    free(audio);
    return n;
}

/* wall time of one decode in seconds (the CPU baseline of the device decoder) */
double ref_time_sd_decode(void *h, const int *codes, int n_frames) {
    struct timespec t0, t1;
    float *audio = NULL;
    int n = 0;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    const int rc = qwen_speech_decoder_decode((qwen_tts_ctx_t *)h, codes, n_frames, &audio, &n);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    free(audio);
    if (rc != 0) return -1.0;
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

/* the reference's exact streaming decode (qwen_speech_decoder_decode_streaming_st,
 * sd.c:1881-2389) with a state of its own */
extern void qwen_sd_stream_init(qwen_sd_stream_state_t *st);
extern void qwen_sd_stream_free(qwen_sd_stream_state_t *st);
extern int qwen_speech_decoder_decode_streaming_st(qwen_tts_ctx_t *ctx, qwen_sd_stream_state_t *st, const int *new_codes,
                                                   int new_frames, float **audio_out, int *n_samples);

void *ref_sd_stream_new(void) {
    qwen_sd_stream_state_t *st = calloc(1, sizeof *st);
    if (st) qwen_sd_stream_init(st);
    return st;
}

int ref_sd_stream_decode(void *h, void *st, const int *codes, int n_frames, float *out, int cap) {
    float *audio = NULL;
    int n = 0;
    if (qwen_speech_decoder_decode_streaming_st((qwen_tts_ctx_t *)h, (qwen_sd_stream_state_t *)st, codes, n_frames, &audio,
                                                &n) != 0 || !audio) return -1;
    if (n > cap) n = cap;
    memcpy(out, audio, (size_t)n * sizeof(float));
    free(audio);
    return n;
}

void ref_sd_stream_free(void *st) {
    if (!st) return;
    qwen_sd_stream_free((qwen_sd_stream_state_t *)st);
    free(st);
}
