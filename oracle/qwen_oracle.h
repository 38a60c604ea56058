/*
 * qwen_oracle.h — CPU restatement of the reference Talker / Code-Predictor decode
 * algorithm.  TEST INFRASTRUCTURE ONLY: this is the checker the HIP path is compared
 * against; it is never linked into, called by, or measured as the product.
 *
 * Plain scalar C, IEEE f32 (no -ffast-math), summation in index order.  Each function
 * cites the reference file:line it restates (paths relative to the reference root).
 * Weight and cache layouts are the reference's own:
 *   bf16 weights    uint16 [rows][cols] row-major
 *   int8 weights    int8  [rows][cols] + f32 scale[rows]
 *   q4_0 weights    18-byte blocks {u16 f16 scale; u8 qs[16]} [rows][cols/32]
 *   KV cache        bf16  [layer][kv_max][n_kv*head_dim]
 */
#ifndef QWEN_ORACLE_H
#define QWEN_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { QO_BF16 = 0, QO_INT8 = 1, QO_Q4_0 = 2 };

/* scalar conversions */
float    qo_bf16_to_f32(uint16_t b);
uint16_t qo_f32_to_bf16_trunc(float f);
float    qo_f16_to_f32(uint16_t h);
uint16_t qo_f32_to_f16(float f);

/* load-time quantizers and dequantizers */
void qo_quantize_int8(const uint16_t *src, int rows, int cols, int8_t *dst, float *scale);
void qo_quantize_q4_0(const uint16_t *src, int rows, int cols, uint8_t *blocks);
void qo_dequant_int8(const int8_t *w, const float *scale, int rows, int cols, float *out);
void qo_dequant_q4_0(const uint8_t *blocks, int rows, int cols, float *out);

/* matvecs: y[r] = sum_k W[r,k] x[k]; f32 accumulate (f64 twins for pinning) */
void qo_matvec(int prec, float *y, const void *W, const float *scale, const float *x, int rows, int cols);
void qo_matvec_f64(int prec, double *y, const void *W, const float *scale, const float *x, int rows, int cols);

/* elementwise / norm / rope / attention */
void qo_rms_norm(float *out, const float *x, const float *w, int dim, float eps);
void qo_rms_norm_per_head(float *x, const float *w, int n_heads, int head_dim, float eps);
void qo_rope_neox(float *x, int n_heads, int head_dim, const float *cos_t, const float *sin_t, int pos);
void qo_swiglu(float *gate_up, int n);
void qo_attention_bf16kv(float *out, const float *Q, const uint16_t *K, const uint16_t *V,
                         int seq_q, int seq_k, int n_heads, int n_kv, int head_dim,
                         float scale, int q_offset);
void qo_attention_f32(float *out, const float *Q, const float *K, const float *V,
                      int seq_q, int seq_k, int n_heads, int n_kv, int head_dim,
                      float scale, int q_offset);
int  qo_argmax(const float *v, int n);
int  qo_codec_greedy(const uint16_t *head, const float *hidden, int vocab, int hidden_dim,
                     int frame, float *logits_out);

/* ---- model-level ---------------------------------------------------------- */
typedef struct { const void *w; const float *scale; } qo_mat_t;
typedef struct {
    qo_mat_t q, k, v, o, gate_up, down;
    const float *input_norm, *post_attn_norm, *q_norm, *k_norm;
} qo_layer_t;
typedef struct {
    int hidden, inter, n_heads, n_kv_heads, head_dim, n_layers, kv_max;
    float eps;
    int prec;
    const qo_layer_t *layers;
    const float *final_norm;
    const float *rope_cos, *rope_sin;
    int rope_len;
    uint16_t *kv_k, *kv_v;   /* caller-owned [n_layers][kv_max][kv_dim] */
} qo_talker_t;

/* One decode step at position pos (qwen_tts_talker.c:537-699).  hidden_out = final
 * norm; dec_x_out (nullable) = pre-norm residual; residuals (nullable) = [L][H]. */
int qo_talker_step(const qo_talker_t *t, const float *embed, int pos,
                   float *hidden_out, float *dec_x_out, float *residuals);

/* Talker prefill of seq positions with bf16 weights (qwen_talker_prefill,
 * qwen_tts_talker.c:730-1038): fills cache rows [0, seq) of every layer, dec_x_out
 * (nullable) = the last position's residual. */
int qo_talker_prefill(const qo_talker_t *t, const float *embeds, int seq, float *dec_x_out);
/* One CP transformer pass over x (in/out residual) at pos (qwen_tts_code_predictor.c:737-761). */
int qo_cp_pass(const qo_talker_t *cp, float *x, int pos);

typedef struct {
    const qo_talker_t *cp;       /* CP layers; final_norm = cp_norm */
    const void *lm_head[15];     /* [codebook][cp_h] */
    const float *lm_scale[15];
    int lm_prec;
    const uint16_t *cp_emb[15];  /* bf16 [codebook][emb_dim] */
    const uint16_t *talker_codec_emb;  /* bf16 [codec_vocab][talker_h] */
    int talker_hidden, emb_dim, codebook, codec_vocab;
    const void *mtp_w; const float *mtp_scale; int mtp_prec; const float *mtp_bias; /* nullable */
} qo_cp_frame_t;

/* 16 passes + 15 argmax codes (qwen_tts_code_predictor.c:926-1045). */
int qo_cp_frame(const qo_cp_frame_t *f, const float *talker_hidden, int code0, int *out_codes);

/* qwen_tts_sample (qwen_tts_sampling.c:160-202) with the LCG state as *seed; when the draw
 * is not greedy, logits end holding the final (renormalised) distribution. */
int qo_sample(float *logits, int n, float temp, int top_k, float top_p, float rep, const int *prev, int n_prev,
              uint32_t *seed);
/* The codec-head rule of qwen_tts.c:1652-1679 in place (clip, specials, EOS). */
void qo_codec_rule(float *logits, int n, int frame, float eos_boost);

#ifdef __cplusplus
}
#endif
#endif
