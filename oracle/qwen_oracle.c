/*
 * qwen_oracle.c — CPU restatement of the reference decode algorithm (checker only).
 *
 * TEST INFRASTRUCTURE: only tests/, the smoke check and bench.py's cpu_baseline leg
 * load this library, and only to check results.  See qwen_oracle.h for layouts.
 * Reference citations are file:line relative to the reference root; k.c means
 * qwen_tts_kernels.c, t.c qwen_tts_talker.c, cp.c qwen_tts_code_predictor.c.
 *
 * Build: gcc -O2 -std=c11 (ISO mode, so no FMA contraction) — every product and sum
 * is a separately rounded IEEE f32 operation in index order.
 */
#include "qwen_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- scalar conversions -------------------------------------------------- */

/* bf16 -> f32 is a 16-bit left shift (t.c:93-97, k.c:583-588). */
float qo_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f; memcpy(&f, &u, 4); return f;
}

/* f32 -> bf16 for the KV cache is TRUNCATION, bits >> 16 (t.c:99-103, t.c:125-159). */
uint16_t qo_f32_to_bf16_trunc(float f) {
    uint32_t u; memcpy(&u, &f, 4); return (uint16_t)(u >> 16);
}

/* binary16 -> f32 as the reference's x86/portable branch computes it (k.h:162-179).
 * Normals, zeros, inf/NaN are the IEEE mapping.  Subnormals (exponent field 0,
 * mantissa m != 0) are normalised by shifting m left `sh` times until bit 10 is set
 * and given the f32 exponent field 112 - sh; IEEE would use 113 - sh, so the
 * reference's subnormal results are exactly half the IEEE value.  Parity follows the
 * reference, not IEEE (q4_0 block scales below 2^-14 take this branch). */
float qo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F, man = h & 0x3FF, bits;
    if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {
        uint32_t sh = 0;
        while (!(man & 0x400)) { man <<= 1; sh++; }
        bits = sign | ((112u - sh) << 23) | ((man & 0x3FF) << 13);
    }
    float f; memcpy(&f, &bits, 4); return f;
}

/* f32 -> f16 as the reference rounds it (k.h:180-201 x86 branch): overflow -> inf
 * (NaN is not preserved), subnormals by right shift with a half-up increment on the
 * first dropped bit, normals round half-UP on mantissa bit 12 with the carry allowed
 * to ripple into the exponent. */
uint16_t qo_f32_to_f16(float f) {
    uint32_t u; memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    int32_t e = (int32_t)((u >> 23) & 0xFF) - 112;   /* rebias 127 -> 15 */
    uint32_t m = u & 0x7FFFFFu;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t full = m | 0x800000u;
        uint32_t sh = (uint32_t)(14 - e);
        uint32_t r = full >> sh;
        if ((full >> (sh - 1)) & 1u) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = sign | ((uint32_t)e << 10) | (m >> 13);
    if (m & 0x1000u) r++;
    return (uint16_t)r;
}

/* ---- quantizers ---------------------------------------------------------- */

/* Per-row absmax int8 (k.c:2143-2238).  scale = amax/127 as the reference binary
 * computes it under -ffast-math (-freciprocal-math turns the division by the constant
 * into a multiply by its f32 reciprocal); inv = 127/amax; q = saturate(round(v*inv)),
 * round-half-even for the 8-wide vector body (_mm256_cvtps_epi32 under the default
 * MXCSR) and roundf (half away from zero) for the cols%8 tail. */
void qo_quantize_int8(const uint16_t *src, int rows, int cols, int8_t *dst, float *scale) {
    const float recip127 = 1.0f / 127.0f;
    int body = cols - cols % 8;
    for (int r = 0; r < rows; r++) {
        const uint16_t *row = src + (size_t)r * cols;
        float amax = 0.0f;
        for (int k = 0; k < cols; k++) {
            float a = fabsf(qo_bf16_to_f32(row[k]));
            if (a > amax) amax = a;
        }
        float s = amax * recip127;
        scale[r] = s;
        float inv = (s > 0.0f) ? 127.0f / amax : 0.0f;
        int8_t *d = dst + (size_t)r * cols;
        for (int k = 0; k < cols; k++) {
            float p = qo_bf16_to_f32(row[k]) * inv;
            long v = (k < body) ? lrintf(p) : (long)roundf(p);
            d[k] = (int8_t)(v < -128 ? -128 : (v > 127 ? 127 : v));
        }
    }
}

/* Weighted-LSQ q4_0 ("q4_0s1", k.c:2662-2726): per 32-block take the signed value of
 * the first max-|v| element, isc = -8/vmax, q = clamp(roundf(v*isc), -8, 7), then the
 * closed-form weighted least-squares scale s = sum(v^2 v q)/sum(v^2 q^2) in double,
 * stored as f16 with the reference rounding.  Nibble 2i is the low nibble of byte i,
 * 2i+1 the high nibble (k.h:207-210). */
void qo_quantize_q4_0(const uint16_t *src, int rows, int cols, uint8_t *blocks) {
    int nb = cols / 32;
    for (int r = 0; r < rows; r++) {
        for (int b = 0; b < nb; b++) {
            const uint16_t *blk = src + (size_t)r * cols + (size_t)b * 32;
            uint8_t *out = blocks + ((size_t)r * nb + b) * 18;
            float v[32], amax = 0.0f, vmax = 0.0f;
            for (int i = 0; i < 32; i++) {
                v[i] = qo_bf16_to_f32(blk[i]);
                float a = fabsf(v[i]);
                if (a > amax) { amax = a; vmax = v[i]; }
            }
            float isc = (vmax != 0.0f) ? -8.0f / vmax : 0.0f;
            int q[32];
            double num = 0.0, den = 0.0;
            for (int i = 0; i < 32; i++) {
                int t = (int)roundf(v[i] * isc);
                t = t < -8 ? -8 : (t > 7 ? 7 : t);
                q[i] = t;
                double w = (double)v[i] * (double)v[i];
                num += w * (double)v[i] * (double)t;
                den += w * (double)t * (double)t;
            }
            float s = (den > 0.0) ? (float)(num / den) : 0.0f;
            uint16_t h = qo_f32_to_f16(s);
            out[0] = (uint8_t)(h & 0xFF);
            out[1] = (uint8_t)(h >> 8);
            for (int i = 0; i < 16; i++)
                out[2 + i] = (uint8_t)((q[2 * i] + 8) | ((q[2 * i + 1] + 8) << 4));
        }
    }
}

/* int8 dequant as a value: q * scale (the matvec applies scale once per row,
 * k.c:2350-2351; this is the per-element view used for bit checks). */
void qo_dequant_int8(const int8_t *w, const float *scale, int rows, int cols, float *out) {
    for (int r = 0; r < rows; r++)
        for (int k = 0; k < cols; k++)
            out[(size_t)r * cols + k] = (float)w[(size_t)r * cols + k] * scale[r];
}

/* q4_0 dequant: (nib - 8) * f16_to_f32(scale) (k.c:2810-2819), exact in f32. */
void qo_dequant_q4_0(const uint8_t *blocks, int rows, int cols, float *out) {
    int nb = cols / 32;
    for (int r = 0; r < rows; r++)
        for (int b = 0; b < nb; b++) {
            const uint8_t *blk = blocks + ((size_t)r * nb + b) * 18;
            float s = qo_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            float *o = out + (size_t)r * cols + (size_t)b * 32;
            for (int i = 0; i < 16; i++) {
                o[2 * i] = (float)((int)(blk[2 + i] & 0x0F) - 8) * s;
                o[2 * i + 1] = (float)((int)(blk[2 + i] >> 4) - 8) * s;
            }
        }
}

/* ---- matvecs --------------------------------------------------------------- */

static inline float w_at(int prec, const void *W, int cols, int r, int k) {
    if (prec == QO_BF16) return qo_bf16_to_f32(((const uint16_t *)W)[(size_t)r * cols + k]);
    if (prec == QO_INT8) return (float)((const int8_t *)W)[(size_t)r * cols + k];
    const uint8_t *blk = (const uint8_t *)W + ((size_t)r * (cols / 32) + k / 32) * 18;
    int i = k % 32;
    int nib = (i & 1) ? (blk[2 + i / 2] >> 4) : (blk[2 + i / 2] & 0x0F);
    return (float)(nib - 8) * qo_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
}

/* bf16: y = sum bf16(W)x (k.c:1091-1100); int8: y = (sum (float)q x) * scale
 * (k.c:2548-2599, scale applied once per row); q4_0: y = sum ((nib-8)*s) x
 * (k.c:2729-2824). */
void qo_matvec(int prec, float *y, const void *W, const float *scale, const float *x,
               int rows, int cols) {
    for (int r = 0; r < rows; r++) {
        float acc = 0.0f;
        for (int k = 0; k < cols; k++) acc += w_at(prec, W, cols, r, k) * x[k];
        y[r] = (prec == QO_INT8) ? acc * scale[r] : acc;
    }
}

void qo_matvec_f64(int prec, double *y, const void *W, const float *scale, const float *x,
                   int rows, int cols) {
    for (int r = 0; r < rows; r++) {
        double acc = 0.0;
        for (int k = 0; k < cols; k++) acc += (double)w_at(prec, W, cols, r, k) * (double)x[k];
        y[r] = (prec == QO_INT8) ? acc * (double)scale[r] : acc;
    }
}

/* ---- norms, RoPE, SwiGLU ------------------------------------------------------ */

/* out = x * (1/sqrt(mean(x^2)+eps)) * w, evaluated (x*inv)*w (k.c:292-382). */
void qo_rms_norm(float *out, const float *x, const float *w, int dim, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < dim; i++) ss += x[i] * x[i];
    float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = 0; i < dim; i++) out[i] = (x[i] * inv) * w[i];
}

/* Per-head RMSNorm with one shared [head_dim] gain (k.c:486-577). */
void qo_rms_norm_per_head(float *x, const float *w, int n_heads, int head_dim, float eps) {
    for (int h = 0; h < n_heads; h++) qo_rms_norm(x + (size_t)h * head_dim, x + (size_t)h * head_dim, w, head_dim, eps);
}

/* NeoX split-half rotation (t.c:203-251): for i < hd/2,
 * x1' = x1*c - x2*s, x2' = x2*c + x1*s, c/s from row `pos` of the [npos][hd/2] tables.
 * The AVX2 body evaluates these as fmsub(x1,c,x2*s) / fmadd(x2,c,x1*s): one rounding
 * for the product x2*s (resp. x1*s) and one for the fused multiply-add. */
void qo_rope_neox(float *x, int n_heads, int head_dim, const float *cos_t, const float *sin_t, int pos) {
    int half = head_dim / 2;
    const float *c = cos_t + (size_t)pos * half, *s = sin_t + (size_t)pos * half;
    for (int h = 0; h < n_heads; h++) {
        float *xh = x + (size_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            float x1 = xh[i], x2 = xh[i + half];
            xh[i] = fmaf(x1, c[i], -(x2 * s[i]));
            xh[i + half] = fmaf(x2, c[i], x1 * s[i]);
        }
    }
}

/* SwiGLU over interleaved [g0,u0,g1,u1,...] -> out[i] = g/(1+expf(-g))*u, in place
 * into the first n floats (k.c:3857-3878). */
void qo_swiglu(float *gu, int n) {
    for (int i = 0; i < n; i++) {
        float g = gu[2 * i], u = gu[2 * i + 1];
        gu[i] = g / (1.0f + expf(-g)) * u;
    }
}

/* ---- attention -------------------------------------------------------------- */

/* Causal GQA attention over a bf16 KV cache, online softmax exactly as
 * k.c:3704-3846: kvh = h / (nh/nkv); max=-1e30, sum=0, o=0; per key s=(q.k)*scale;
 * if s>max: c=expf(max-s), sum=sum*c+1, o=o*c+v, max=s; else w=expf(s-max),
 * sum+=w, o+=w*v; finally o *= 1/sum.  K/V rows are [seq][n_kv*hd]. */
void qo_attention_bf16kv(float *out, const float *Q, const uint16_t *K, const uint16_t *V,
                         int seq_q, int seq_k, int n_heads, int n_kv, int head_dim,
                         float scale, int q_offset) {
    int hpk = n_heads / n_kv, qh = n_heads * head_dim, kvh_dim = n_kv * head_dim;
    for (int h = 0; h < n_heads; h++) {
        int g = h / hpk;
        for (int i = 0; i < seq_q; i++) {
            const float *q = Q + (size_t)i * qh + (size_t)h * head_dim;
            float *o = out + (size_t)i * qh + (size_t)h * head_dim;
            int k_end = q_offset + i + 1;
            if (k_end > seq_k) k_end = seq_k;
            float mx = -1e30f, sum = 0.0f;
            for (int d = 0; d < head_dim; d++) o[d] = 0.0f;
            for (int j = 0; j < k_end; j++) {
                const uint16_t *kr = K + (size_t)j * kvh_dim + (size_t)g * head_dim;
                const uint16_t *vr = V + (size_t)j * kvh_dim + (size_t)g * head_dim;
                float s = 0.0f;
                for (int d = 0; d < head_dim; d++) s += q[d] * qo_bf16_to_f32(kr[d]);
                s *= scale;
                if (s > mx) {
                    float c = expf(mx - s);
                    sum = sum * c + 1.0f;
                    for (int d = 0; d < head_dim; d++) o[d] = o[d] * c + qo_bf16_to_f32(vr[d]);
                    mx = s;
                } else {
                    float w = expf(s - mx);
                    sum += w;
                    for (int d = 0; d < head_dim; d++) o[d] += qo_bf16_to_f32(vr[d]) * w;
                }
            }
            if (sum > 0.0f) {
                float inv = 1.0f / sum;
                for (int d = 0; d < head_dim; d++) o[d] *= inv;
            }
        }
    }
}

/* The same online softmax over f32 K/V rows (qwen_causal_attention, k.c:3454-3560), used
 * by the Talker prefill on the f32 q/k/v it has just computed (t.c:901-907). */
void qo_attention_f32(float *out, const float *Q, const float *K, const float *V,
                      int seq_q, int seq_k, int n_heads, int n_kv, int head_dim,
                      float scale, int q_offset) {
    int hpk = n_heads / n_kv, qh = n_heads * head_dim, kvh_dim = n_kv * head_dim;
    for (int h = 0; h < n_heads; h++) {
        int g = h / hpk;
        for (int i = 0; i < seq_q; i++) {
            const float *q = Q + (size_t)i * qh + (size_t)h * head_dim;
            float *o = out + (size_t)i * qh + (size_t)h * head_dim;
            int k_end = q_offset + i + 1;
            if (k_end > seq_k) k_end = seq_k;
            float mx = -1e30f, sum = 0.0f;
            for (int d = 0; d < head_dim; d++) o[d] = 0.0f;
            for (int j = 0; j < k_end; j++) {
                const float *kr = K + (size_t)j * kvh_dim + (size_t)g * head_dim;
                const float *vr = V + (size_t)j * kvh_dim + (size_t)g * head_dim;
                float s = 0.0f;
                for (int d = 0; d < head_dim; d++) s += q[d] * kr[d];
                s *= scale;
                if (s > mx) {
                    float c = expf(mx - s);
                    sum = sum * c + 1.0f;
                    for (int d = 0; d < head_dim; d++) o[d] = o[d] * c + vr[d];
                    mx = s;
                } else {
                    float w = expf(s - mx);
                    sum += w;
                    for (int d = 0; d < head_dim; d++) o[d] += vr[d] * w;
                }
            }
            if (sum > 0.0f) {
                float inv = 1.0f / sum;
                for (int d = 0; d < head_dim; d++) o[d] *= inv;
            }
        }
    }
}

/* Greedy argmax, lowest index on ties (strict >, qwen_tts_sampling.c:175-182). */
int qo_argmax(const float *v, int n) {
    int best = 0; float bv = v[0];
    for (int i = 1; i < n; i++) if (v[i] > bv) { bv = v[i]; best = i; }
    return best;
}

/* Codec head + greedy code0 (qwen_tts.c:1649-1694): bf16 matvec, clip to [-100,100],
 * tokens [2048, vocab) except EOS 2150 -> -1e30, EOS -> -1e30 on frames 0-1, greedy
 * (rep-penalty 1.0 and no EOS boost in the synthetic harness). */
int qo_codec_greedy(const uint16_t *head, const float *hidden, int vocab, int hidden_dim,
                    int frame, float *logits_out) {
    float *lg = (float *)malloc((size_t)vocab * sizeof(float));
    if (!lg) return -1;
    qo_matvec(QO_BF16, lg, head, NULL, hidden, vocab, hidden_dim);
    for (int t = 0; t < vocab; t++) {
        if (lg[t] > 100.0f) lg[t] = 100.0f;
        if (lg[t] < -100.0f) lg[t] = -100.0f;
    }
    for (int t = 2048; t < vocab; t++) if (t != 2150) lg[t] = -1e30f;
    if (frame < 2 && vocab > 2150) lg[2150] = -1e30f;
    if (logits_out) memcpy(logits_out, lg, (size_t)vocab * sizeof(float));
    int tok = qo_argmax(lg, vocab);
    free(lg);
    return tok;
}

/* ---- one transformer layer (t.c:580-690 == cp.c:595-717) --------------------- */

typedef struct {
    float *xn, *q, *k, *v, *attn, *proj, *gu;
} qo_scratch_t;

static int scratch_alloc(qo_scratch_t *s, const qo_talker_t *t) {
    int H = t->hidden, qd = t->n_heads * t->head_dim, kvd = t->n_kv_heads * t->head_dim;
    s->xn = malloc((size_t)H * 4); s->q = malloc((size_t)qd * 4);
    s->k = malloc((size_t)kvd * 4); s->v = malloc((size_t)kvd * 4);
    s->attn = malloc((size_t)qd * 4); s->proj = malloc((size_t)H * 4);
    s->gu = malloc((size_t)2 * t->inter * 4);
    return (s->xn && s->q && s->k && s->v && s->attn && s->proj && s->gu) ? 0 : -1;
}
static void scratch_free(qo_scratch_t *s) {
    free(s->xn); free(s->q); free(s->k); free(s->v); free(s->attn); free(s->proj); free(s->gu);
}

/* x: residual (in/out); xn: on entry rmsnorm(x, input_norm[l]); on exit the next
 * layer's input norm (when l+1 < L) — the reference's fused residual+norm placement. */
static void layer_body(const qo_talker_t *t, int l, float *x, qo_scratch_t *s, int pos) {
    const qo_layer_t *ly = &t->layers[l];
    int H = t->hidden, F = t->inter, nh = t->n_heads, nkv = t->n_kv_heads, hd = t->head_dim;
    int qd = nh * hd, kvd = nkv * hd;
    qo_matvec(t->prec, s->q, ly->q.w, ly->q.scale, s->xn, qd, H);
    qo_matvec(t->prec, s->k, ly->k.w, ly->k.scale, s->xn, kvd, H);
    qo_matvec(t->prec, s->v, ly->v.w, ly->v.scale, s->xn, kvd, H);
    qo_rms_norm_per_head(s->q, ly->q_norm, nh, hd, t->eps);
    qo_rms_norm_per_head(s->k, ly->k_norm, nkv, hd, t->eps);
    qo_rope_neox(s->q, nh, hd, t->rope_cos, t->rope_sin, pos);
    qo_rope_neox(s->k, nkv, hd, t->rope_cos, t->rope_sin, pos);
    size_t lay = (size_t)l * t->kv_max * kvd;
    for (int i = 0; i < kvd; i++) {
        t->kv_k[lay + (size_t)pos * kvd + i] = qo_f32_to_bf16_trunc(s->k[i]);
        t->kv_v[lay + (size_t)pos * kvd + i] = qo_f32_to_bf16_trunc(s->v[i]);
    }
    qo_attention_bf16kv(s->attn, s->q, t->kv_k + lay, t->kv_v + lay, 1, pos + 1, nh, nkv, hd,
                        1.0f / sqrtf((float)hd), pos);
    qo_matvec(t->prec, s->proj, ly->o.w, ly->o.scale, s->attn, H, qd);
    for (int i = 0; i < H; i++) x[i] += s->proj[i];
    qo_rms_norm(s->xn, x, ly->post_attn_norm, H, t->eps);
    qo_matvec(t->prec, s->gu, ly->gate_up.w, ly->gate_up.scale, s->xn, 2 * F, H);
    qo_swiglu(s->gu, F);
    qo_matvec(t->prec, s->proj, ly->down.w, ly->down.scale, s->gu, H, F);
    for (int i = 0; i < H; i++) x[i] += s->proj[i];
    if (l + 1 < t->n_layers) qo_rms_norm(s->xn, x, t->layers[l + 1].input_norm, H, t->eps);
}

int qo_talker_step(const qo_talker_t *t, const float *embed, int pos,
                   float *hidden_out, float *dec_x_out, float *residuals) {
    if (pos < 0 || pos >= t->kv_max || pos >= t->rope_len) return -1;
    int H = t->hidden;
    qo_scratch_t s;
    float *x = malloc((size_t)H * 4);
    if (!x || scratch_alloc(&s, t) != 0) { free(x); return -1; }
    memcpy(x, embed, (size_t)H * 4);
    qo_rms_norm(s.xn, x, t->layers[0].input_norm, H, t->eps);
    for (int l = 0; l < t->n_layers; l++) {
        layer_body(t, l, x, &s, pos);
        if (residuals) memcpy(residuals + (size_t)l * H, x, (size_t)H * 4);
    }
    if (hidden_out) qo_rms_norm(hidden_out, x, t->final_norm, H, t->eps);
    if (dec_x_out) memcpy(dec_x_out, x, (size_t)H * 4);
    scratch_free(&s); free(x);
    return 0;
}

/* Talker prefill of seq positions (qwen_talker_prefill, t.c:730-1038), bf16 weights
 * (the reference's prefill reads the bf16 layer weights whatever the decode precision,
 * t.c:832-839, 845-847).  X[s] = embeds[s]; per layer, for every position s:
 * xn = rmsnorm(X[s], input_norm); q|k|v = W . xn (f32 sums); per-head q/k norm; NeoX RoPE
 * at position s (t.c:887-895); cache rows s = bf16 truncation of k, v (t.c:897-899);
 * causal attention over the f32 q/k/v of positions <= s (t.c:901-907); X[s] += W_o . attn;
 * xn = rmsnorm(X[s], post_norm); X[s] += W_down . SwiGLU(W_gu . xn) (t.c:909-1010).
 * dec_x_out = X[seq-1] (t.c:1032-1033). */
int qo_talker_prefill(const qo_talker_t *t, const float *embeds, int seq, float *dec_x_out) {
    if (t->prec != QO_BF16 || seq < 1 || seq > t->kv_max || seq > t->rope_len) return -1;
    int H = t->hidden, F = t->inter, nh = t->n_heads, nkv = t->n_kv_heads, hd = t->head_dim;
    int qd = nh * hd, kvd = nkv * hd;
    float *X = malloc((size_t)seq * H * 4), *xn = malloc((size_t)H * 4);
    float *Q = malloc((size_t)seq * qd * 4), *K = malloc((size_t)seq * kvd * 4), *V = malloc((size_t)seq * kvd * 4);
    float *A = malloc((size_t)seq * qd * 4), *proj = malloc((size_t)H * 4), *gu = malloc((size_t)2 * F * 4);
    int rc = -1;
    if (!X || !xn || !Q || !K || !V || !A || !proj || !gu) goto done;
    memcpy(X, embeds, (size_t)seq * H * 4);
    for (int l = 0; l < t->n_layers; l++) {
        const qo_layer_t *ly = &t->layers[l];
        for (int s = 0; s < seq; s++) {
            float *q = Q + (size_t)s * qd, *k = K + (size_t)s * kvd, *v = V + (size_t)s * kvd;
            qo_rms_norm(xn, X + (size_t)s * H, ly->input_norm, H, t->eps);
            qo_matvec(QO_BF16, q, ly->q.w, NULL, xn, qd, H);
            qo_matvec(QO_BF16, k, ly->k.w, NULL, xn, kvd, H);
            qo_matvec(QO_BF16, v, ly->v.w, NULL, xn, kvd, H);
            qo_rms_norm_per_head(q, ly->q_norm, nh, hd, t->eps);
            qo_rms_norm_per_head(k, ly->k_norm, nkv, hd, t->eps);
            qo_rope_neox(q, nh, hd, t->rope_cos, t->rope_sin, s);
            qo_rope_neox(k, nkv, hd, t->rope_cos, t->rope_sin, s);
            size_t row = ((size_t)l * t->kv_max + s) * kvd;
            for (int i = 0; i < kvd; i++) {
                t->kv_k[row + i] = qo_f32_to_bf16_trunc(k[i]);
                t->kv_v[row + i] = qo_f32_to_bf16_trunc(v[i]);
            }
        }
        qo_attention_f32(A, Q, K, V, seq, seq, nh, nkv, hd, 1.0f / sqrtf((float)hd), 0);
        for (int s = 0; s < seq; s++) {
            float *x = X + (size_t)s * H;
            qo_matvec(QO_BF16, proj, ly->o.w, NULL, A + (size_t)s * qd, H, qd);
            for (int i = 0; i < H; i++) x[i] += proj[i];
            qo_rms_norm(xn, x, ly->post_attn_norm, H, t->eps);
            qo_matvec(QO_BF16, gu, ly->gate_up.w, NULL, xn, 2 * F, H);
            qo_swiglu(gu, F);
            qo_matvec(QO_BF16, proj, ly->down.w, NULL, gu, H, F);
            for (int i = 0; i < H; i++) x[i] += proj[i];
        }
    }
    if (dec_x_out) memcpy(dec_x_out, X + (size_t)(seq - 1) * H, (size_t)H * 4);
    rc = 0;
done:
    free(X); free(xn); free(Q); free(K); free(V); free(A); free(proj); free(gu);
    return rc;
}

int qo_cp_pass(const qo_talker_t *cp, float *x, int pos) {
    if (pos < 0 || pos >= cp->kv_max || pos >= cp->rope_len) return -1;
    qo_scratch_t s;
    if (scratch_alloc(&s, cp) != 0) return -1;
    qo_rms_norm(s.xn, x, cp->layers[0].input_norm, cp->hidden, cp->eps);
    for (int l = 0; l < cp->n_layers; l++) layer_body(cp, l, x, &s, pos);
    scratch_free(&s);
    return 0;
}

/* small_to_mtp_projection (cp.c:907-924): dst = W src (+bias) or a copy of cp_h. */
static void mtp(const qo_cp_frame_t *f, float *dst, const float *src) {
    int cph = f->cp->hidden;
    if (f->mtp_w) {
        qo_matvec(f->mtp_prec, dst, f->mtp_w, f->mtp_scale, src, cph, f->emb_dim);
        if (f->mtp_bias) for (int i = 0; i < cph; i++) dst[i] += f->mtp_bias[i];
    } else {
        memcpy(dst, src, (size_t)cph * 4);
    }
}

int qo_cp_frame(const qo_cp_frame_t *f, const float *talker_hidden, int code0, int *out_codes) {
    const qo_talker_t *cp = f->cp;
    int cph = cp->hidden, E = f->emb_dim;
    float *x = malloc((size_t)cph * 4), *x1 = malloc((size_t)cph * 4);
    float *xn = malloc((size_t)cph * 4), *emb = malloc((size_t)(E > f->talker_hidden ? E : f->talker_hidden) * 4);
    float *lg = malloc((size_t)f->codebook * 4);
    if (!x || !x1 || !xn || !emb || !lg) { free(x); free(x1); free(xn); free(emb); free(lg); return -1; }
    mtp(f, x, talker_hidden);
    if (f->talker_codec_emb && code0 >= 0 && code0 < f->codec_vocab) {
        for (int i = 0; i < f->talker_hidden; i++)
            emb[i] = qo_bf16_to_f32(f->talker_codec_emb[(size_t)code0 * f->talker_hidden + i]);
        mtp(f, x1, emb);
    } else {
        memset(x1, 0, (size_t)cph * 4);
    }
    qo_cp_pass(cp, x, 0);
    memcpy(x, x1, (size_t)cph * 4);
    qo_cp_pass(cp, x, 1);
    for (int g = 0; g < 15; g++) {
        if (g > 0) {
            int prev = out_codes[g - 1];
            if (f->cp_emb[g - 1] && prev >= 0 && prev < f->codebook) {
                for (int i = 0; i < E; i++) emb[i] = qo_bf16_to_f32(f->cp_emb[g - 1][(size_t)prev * E + i]);
                mtp(f, x, emb);
            } else {
                memset(x, 0, (size_t)cph * 4);
            }
            qo_cp_pass(cp, x, g + 1);
        }
        qo_rms_norm(xn, x, cp->final_norm, cph, cp->eps);
        qo_matvec(f->lm_prec, lg, f->lm_head[g], f->lm_scale[g], xn, f->codebook, cph);
        /* fused argmax+matvec keeps best=-1e30 and a strict > (k.c:4652-4759) */
        int best = 0; float bv = -1e30f;
        for (int i = 0; i < f->codebook; i++) if (lg[i] > bv) { bv = lg[i]; best = i; }
        out_codes[g] = best;
    }
    free(x); free(x1); free(xn); free(emb); free(lg);
    return 0;
}

/* ---- sampling (qwen_tts_sampling.c) ---------------------------------------------------
 * The steps of qwen_tts_sample in the reference's order and with its sequential sums:
 * repetition penalty (sampling.c:165-173), greedy below temp 1e-6 (:176-182), softmax with
 * 1/temp (:52-62), top-k threshold = k-th largest value with multiplicity (:96-111; here by
 * a sorted copy instead of quickselect: same value), top-p by selection of the running
 * maximum until the cumulative sum exceeds p, ties resolved by the same swap sequence
 * (:114-146), renormalisation (:195-198), LCG draw over the cumulative sum (:38-42,
 * :149-157). */
static int qo_cmp_desc(const void *a, const void *b) {
    float x = *(const float *)a, y = *(const float *)b;
    return (x < y) - (x > y);
}

int qo_sample(float *lg, int n, float temp, int top_k, float top_p, float rep, const int *prev, int n_prev,
              uint32_t *seed) {
    if (rep != 1.0f && n_prev > 0)
        for (int j = 0; j < n_prev; j++) {
            int t = prev[j];
            if (t >= 0 && t < n) lg[t] = lg[t] > 0 ? lg[t] / rep : lg[t] * rep;
        }
    if (temp < 1e-6f) {
        int best = 0;
        for (int i = 1; i < n; i++) if (lg[i] > lg[best]) best = i;
        return best;
    }
    float mx = lg[0];
    for (int i = 1; i < n; i++) if (lg[i] > mx) mx = lg[i];
    float inv = 1.0f / temp, sum = 0.f;
    for (int i = 0; i < n; i++) { lg[i] = expf((lg[i] - mx) * inv); sum += lg[i]; }
    for (int i = 0; i < n; i++) lg[i] /= sum;
    if (top_k > 0 && top_k < n) {
        float *tmp = (float *)malloc((size_t)n * sizeof(float));
        memcpy(tmp, lg, (size_t)n * sizeof(float));
        qsort(tmp, (size_t)n, sizeof(float), qo_cmp_desc);
        float thr = tmp[top_k - 1];
        free(tmp);
        for (int i = 0; i < n; i++) if (lg[i] < thr) lg[i] = 0.f;
    }
    if (top_p < 1.0f && top_p > 0.0f) {
        int *idx = (int *)malloc((size_t)n * sizeof(int));
        for (int i = 0; i < n; i++) idx[i] = i;
        float cum = 0.f;
        int cut = n;
        for (int i = 0; i < n; i++) {
            int m = i;
            for (int j = i + 1; j < n; j++) if (lg[idx[j]] > lg[idx[m]]) m = j;
            int t = idx[i]; idx[i] = idx[m]; idx[m] = t;
            cum += lg[idx[i]];
            if (cum > top_p) { cut = i + 1; break; }
        }
        for (int i = cut; i < n; i++) lg[idx[i]] = 0.f;
        free(idx);
    }
    float s2 = 0.f;
    for (int i = 0; i < n; i++) s2 += lg[i];
    if (s2 > 0) for (int i = 0; i < n; i++) lg[i] /= s2;
    *seed = *seed * 1103515245u + 12345u;
    float r = (float)((*seed >> 16) & 0x7FFF) / 32768.0f, cum = 0.f;
    for (int i = 0; i < n; i++) {
        cum += lg[i];
        if (r < cum) return i;
    }
    return n - 1;
}

void qo_codec_rule(float *lg, int n, int frame, float eos_boost) {
    for (int t = 0; t < n; t++) {
        if (lg[t] > 100.0f) lg[t] = 100.0f;
        if (lg[t] < -100.0f) lg[t] = -100.0f;
    }
    for (int t = 2048; t < n; t++) if (t != 2150) lg[t] = -1e30f;
    if (n > 2150) {
        if (frame < 2) lg[2150] = -1e30f;
        lg[2150] += eos_boost;
    }
}
