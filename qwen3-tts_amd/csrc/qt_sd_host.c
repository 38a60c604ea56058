/* qt_sd_host.c — host side of the device speech decoder (qt_sd.hip): weights by the reference's
 * tensor names (qwen_speech_decoder_load, qwen_tts_speech_decoder.c:372-578) rearranged
 * into the implicit-GEMM layouts, and the one-shot decode sequence of
 * qwen_speech_decoder_decode (sd.c:579-1290) as kernel launches on one stream.
 *
 * Layouts on the device (all f32): activations [T][C]; a conv or linear layer is
 * W[phase][tap][K = in][N = out] with per-tap input row offsets:
 *   linear   [out][in]              -> one tap, offset 0 (W transposed);
 *   conv1d   [out][in][k], dil d    -> k taps, offsets (p - k + 1) d;
 *   convT    [in][out][2s], stride s-> s phases (output rows t*s + z), taps: column z at
 *            offset 0 and column z + s at offset -1 (when z + s < kernel).
 */
#include "qwen_tts_hip.h"
#include "qt_launch.h"

#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define SD_CB 256
#define SD_CBSIZE 2048
#define SD_ROPE_POS 8000
#define SD_SPF 1920               /* samples per frame */

enum { SD_BIAS = 1, SD_GELU = 2, SD_CSCALE = 4, SD_RESID = 8, SD_SNAKE = 16, SD_SNAKE2 = 32 };

typedef struct {
    float *w, *b;
    int K, N, ntap, phases;
    int off[8];
} sd_conv_t;

typedef struct { float *a, *ib; } sd_snake_t;

typedef struct {
    float *n1, *n2, *ls1, *ls2;
    sd_conv_t qkv, o, gu, dn;
} sd_layer_t;

typedef struct {
    hipStream_t st;
    float *cb;                    /* [16][2048][256] dequantised codebooks */
    sd_conv_t vq, pre, inp, outp, init;
    sd_layer_t L[8];
    float *fnorm;
    struct { sd_conv_t up, pw1, pw2; float *dw, *db, *lw, *lb, *gamma; } cn[2];
    struct { sd_snake_t s; sd_conv_t up; struct { sd_snake_t s1, s2; sd_conv_t c1, c2; } r[3]; } blk[4];
    sd_snake_t fs;
    float *fw, *fb;
    float *rope_c, *rope_s;       /* [8000][32] */
    /* workspace, grown to the largest call */
    int cap;
    float *E, *V, *P, *H, *XN, *QKV, *A, *GU, *M, *LAT, *big[3];
    int *dcodes; float *daudio;
    void **allocs; int n_allocs, cap_allocs;
} sd_t;

static const int UP_RATE[4] = {8, 5, 4, 3}, UP_CH[4] = {768, 384, 192, 96}, DIL[3] = {1, 3, 9};

/* ---- allocation bookkeeping ------------------------------------------------------------ */
static void *sd_dalloc(sd_t *s, size_t bytes) {
    void *p = NULL;
    if (s->n_allocs == s->cap_allocs) {
        int nc = s->cap_allocs ? 2 * s->cap_allocs : 256;
        void **na = (void **)realloc(s->allocs, (size_t)nc * sizeof *na);
        if (!na) return NULL;
        s->allocs = na; s->cap_allocs = nc;
    }
    if (hipMalloc(&p, bytes ? bytes : 4) != hipSuccess) return NULL;
    s->allocs[s->n_allocs++] = p;
    return p;
}

void qwen_hip_sd_free(void *state) {
    sd_t *s = (sd_t *)state;
    if (!s) return;
    if (s->st) (void)hipStreamSynchronize(s->st);
    for (int i = 0; i < s->n_allocs; i++) (void)hipFree(s->allocs[i]);
    free(s->allocs);
    float *ws[] = {s->E, s->V, s->P, s->H, s->XN, s->QKV, s->A, s->GU, s->M, s->LAT, s->big[0], s->big[1], s->big[2],
                   s->daudio};
    for (size_t i = 0; i < sizeof ws / sizeof ws[0]; i++) if (ws[i]) (void)hipFree(ws[i]);
    if (s->dcodes) (void)hipFree(s->dcodes);
    if (s->st) (void)hipStreamDestroy(s->st);
    free(s);
}

/* ---- weights ------------------------------------------------------------------------------ */
typedef struct {
    qwen_hip_sd_get_fn get;
    void *user;
    sd_t *s;
    float *tmp; size_t tmp_n;
    int bad;
} sd_ld_t;

static const float *sd_get(sd_ld_t *L, const char *name, long long n) {
    if (L->bad) return NULL;
    const float *p = L->get(L->user, name, n);
    if (!p) {
        if (!qwen_hip_last_error()[0] || !strstr(qwen_hip_last_error(), name))
            qt_seterr("sd_init: missing tensor %s (%lld floats)", name, n);
        L->bad = 1;
    }
    return p;
}

static float *sd_tmp(sd_ld_t *L, size_t n) {
    if (n > L->tmp_n) {
        free(L->tmp);
        L->tmp = (float *)malloc(n * sizeof(float));
        L->tmp_n = L->tmp ? n : 0;
        if (!L->tmp) { qt_seterr("sd_init: out of host memory"); L->bad = 1; }
    }
    return L->tmp;
}

/* host f32 -> new device buffer (synchronous: the host source may be reused) */
static float *sd_put(sd_ld_t *L, const float *src, size_t n) {
    if (L->bad || !src) return NULL;
    float *d = (float *)sd_dalloc(L->s, n * sizeof(float));
    if (!d || hipMemcpy(d, src, n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
        qt_seterr("sd_init: device allocation or upload failed");
        L->bad = 1;
        return NULL;
    }
    return d;
}

static float *sd_vec(sd_ld_t *L, const char *name, long long n) { return sd_put(L, sd_get(L, name, n), (size_t)n); }

static sd_snake_t sd_snake(sd_ld_t *L, const char *pa, const char *pb, int n) {
    sd_snake_t r = {NULL, NULL};
    float *la = sd_vec(L, pa, n), *lb = sd_vec(L, pb, n);
    if (L->bad) return r;
    r.a = (float *)sd_dalloc(L->s, (size_t)n * sizeof(float));
    r.ib = (float *)sd_dalloc(L->s, (size_t)n * sizeof(float));
    if (!r.a || !r.ib || qt_launch_sd_snake_params(la, lb, r.a, r.ib, n, L->s->st) != hipSuccess) L->bad = 1;
    return r;
}

/* linear [out][in] (+ bias) -> one tap [in][out] */
static sd_conv_t sd_linear(sd_ld_t *L, const char *wn, const char *bn, int out, int in) {
    sd_conv_t c; memset(&c, 0, sizeof c);
    c.K = in; c.N = out; c.ntap = 1; c.phases = 1;
    const float *w = sd_get(L, wn, (long long)out * in);
    float *t = sd_tmp(L, (size_t)out * in);
    if (L->bad) return c;
    for (int o = 0; o < out; o++) for (int i = 0; i < in; i++) t[(size_t)i * out + o] = w[(size_t)o * in + i];
    c.w = sd_put(L, t, (size_t)out * in);
    if (bn) c.b = sd_vec(L, bn, out);
    return c;
}

/* causal conv [out][in][k], dilation d -> k taps [p][in][out] at offsets (p - k + 1) d */
static sd_conv_t sd_conv(sd_ld_t *L, const char *wn, const char *bn, int out, int in, int k, int d) {
    sd_conv_t c; memset(&c, 0, sizeof c);
    c.K = in; c.N = out; c.ntap = k; c.phases = 1;
    for (int p = 0; p < k; p++) c.off[p] = (p - k + 1) * d;
    const float *w = sd_get(L, wn, (long long)out * in * k);
    float *t = sd_tmp(L, (size_t)out * in * k);
    if (L->bad) return c;
    for (int o = 0; o < out; o++)
        for (int i = 0; i < in; i++)
            for (int p = 0; p < k; p++) t[((size_t)p * in + i) * out + o] = w[((size_t)o * in + i) * k + p];
    c.w = sd_put(L, t, (size_t)out * in * k);
    if (bn) c.b = sd_vec(L, bn, out);
    return c;
}

/* causal transposed conv [in][out][k], stride s (k <= 2s) -> s phases of taps at offsets
 * 0 (column z) and -1 (column z + s; zero where z + s >= k) */
static sd_conv_t sd_convt(sd_ld_t *L, const char *wn, const char *bn, int in, int out, int k, int s) {
    sd_conv_t c; memset(&c, 0, sizeof c);
    c.K = in; c.N = out; c.phases = s; c.ntap = k > s ? 2 : 1;
    c.off[0] = 0; c.off[1] = -1;
    const float *w = sd_get(L, wn, (long long)in * out * k);
    const size_t per = (size_t)in * out;
    float *t = sd_tmp(L, (size_t)s * c.ntap * per);
    if (L->bad) return c;
    for (int z = 0; z < s; z++)
        for (int p = 0; p < c.ntap; p++) {
            const int col = z + p * s;
            float *dst = t + ((size_t)z * c.ntap + p) * per;
            for (int i = 0; i < in; i++)
                for (int o = 0; o < out; o++) dst[(size_t)i * out + o] = col < k ? w[((size_t)i * out + o) * k + col] : 0.f;
        }
    c.w = sd_put(L, t, (size_t)s * c.ntap * per);
    if (bn) c.b = sd_vec(L, bn, out);
    return c;
}

void *qwen_hip_sd_init(qwen_hip_sd_get_fn get, void *user) {
    int ndev = 0;
    if (!get) { qt_seterr("sd_init: no tensor getter"); return NULL; }
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) { qt_seterr("sd_init: no HIP device"); return NULL; }
    sd_t *s = (sd_t *)calloc(1, sizeof *s);
    if (!s) { qt_seterr("sd_init: out of host memory"); return NULL; }
    sd_ld_t L = {get, user, s, NULL, 0, 0};
    char nm[160], nb[160];
    if (hipStreamCreateWithFlags(&s->st, hipStreamNonBlocking) != hipSuccess) { qt_seterr("sd_init: stream"); goto fail; }
    /* codebooks: EMA sums over usage, on the device */
    s->cb = (float *)sd_dalloc(s, (size_t)16 * SD_CBSIZE * SD_CB * sizeof(float));
    if (!s->cb) { qt_seterr("sd_init: device allocation failed"); goto fail; }
    for (int k = 0; k < 16 && !L.bad; k++) {
        const char *pfx = k == 0 ? "decoder.quantizer.rvq_first.vq.layers.0._codebook" : NULL;
        char pb[128];
        if (!pfx) { snprintf(pb, sizeof pb, "decoder.quantizer.rvq_rest.vq.layers.%d._codebook", k - 1); pfx = pb; }
        snprintf(nm, sizeof nm, "%s.embedding_sum", pfx);
        snprintf(nb, sizeof nb, "%s.cluster_usage", pfx);
        float *es = sd_vec(&L, nm, (long long)SD_CBSIZE * SD_CB), *cu = sd_vec(&L, nb, SD_CBSIZE);
        if (L.bad) break;
        if (qt_launch_sd_cb_dequant(es, cu, s->cb + (size_t)k * SD_CBSIZE * SD_CB, SD_CBSIZE, SD_CB, s->st) != hipSuccess ||
            hipStreamSynchronize(s->st) != hipSuccess) { qt_seterr("sd_init: codebook dequantisation failed"); goto fail; }
    }
    /* VQ projections as one K = 512 product of [codebook 0 | sum of 1..15] rows */
    {
        s->vq.K = 2 * SD_CB; s->vq.N = 512; s->vq.ntap = 1; s->vq.phases = 1;
        const float *w1 = sd_get(&L, "decoder.quantizer.rvq_first.output_proj.weight", 512LL * SD_CB);
        float *t = sd_tmp(&L, (size_t)2 * SD_CB * 512);
        if (!L.bad) for (int o = 0; o < 512; o++) for (int i = 0; i < SD_CB; i++) t[(size_t)i * 512 + o] = w1[(size_t)o * SD_CB + i];
        const float *w2 = sd_get(&L, "decoder.quantizer.rvq_rest.output_proj.weight", 512LL * SD_CB);
        if (!L.bad) for (int o = 0; o < 512; o++) for (int i = 0; i < SD_CB; i++) t[(size_t)(SD_CB + i) * 512 + o] = w2[(size_t)o * SD_CB + i];
        s->vq.w = sd_put(&L, t, (size_t)2 * SD_CB * 512);
    }
    s->pre = sd_conv(&L, "decoder.pre_conv.conv.weight", "decoder.pre_conv.conv.bias", 1024, 512, 3, 1);
    s->inp = sd_linear(&L, "decoder.pre_transformer.input_proj.weight", "decoder.pre_transformer.input_proj.bias", 512, 1024);
    for (int l = 0; l < 8 && !L.bad; l++) {
        sd_layer_t *y = &s->L[l];
#define LN(sfx) (snprintf(nm, sizeof nm, "decoder.pre_transformer.layers.%d.%s", l, sfx), nm)
        y->n1 = sd_vec(&L, LN("input_layernorm.weight"), 512);
        y->n2 = sd_vec(&L, LN("post_attention_layernorm.weight"), 512);
        y->ls1 = sd_vec(&L, LN("self_attn_layer_scale.scale"), 512);
        y->ls2 = sd_vec(&L, LN("mlp_layer_scale.scale"), 512);
        /* q | k | v as one [512][3072] tap, gate | up as one [512][2048] tap */
        {
            y->qkv.K = 512; y->qkv.N = 3072; y->qkv.ntap = 1; y->qkv.phases = 1;
            float *t = sd_tmp(&L, (size_t)512 * 3072);
            const char *nmq[3] = {"self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight"};
            for (int q = 0; q < 3 && !L.bad; q++) {
                const float *w = sd_get(&L, LN(nmq[q]), 1024LL * 512);
                if (L.bad) break;
                for (int o = 0; o < 1024; o++) for (int i = 0; i < 512; i++) t[(size_t)i * 3072 + q * 1024 + o] = w[(size_t)o * 512 + i];
            }
            y->qkv.w = sd_put(&L, t, (size_t)512 * 3072);
        }
        y->o = sd_linear(&L, LN("self_attn.o_proj.weight"), NULL, 512, 1024);
        {
            y->gu.K = 512; y->gu.N = 2048; y->gu.ntap = 1; y->gu.phases = 1;
            float *t = sd_tmp(&L, (size_t)512 * 2048);
            const char *nmg[2] = {"mlp.gate_proj.weight", "mlp.up_proj.weight"};
            for (int q = 0; q < 2 && !L.bad; q++) {
                const float *w = sd_get(&L, LN(nmg[q]), 1024LL * 512);
                if (L.bad) break;
                for (int o = 0; o < 1024; o++) for (int i = 0; i < 512; i++) t[(size_t)i * 2048 + q * 1024 + o] = w[(size_t)o * 512 + i];
            }
            y->gu.w = sd_put(&L, t, (size_t)512 * 2048);
        }
        y->dn = sd_linear(&L, LN("mlp.down_proj.weight"), NULL, 512, 1024);
#undef LN
    }
    s->fnorm = sd_vec(&L, "decoder.pre_transformer.norm.weight", 512);
    s->outp = sd_linear(&L, "decoder.pre_transformer.output_proj.weight", "decoder.pre_transformer.output_proj.bias", 1024, 512);
    for (int b = 0; b < 2 && !L.bad; b++) {
#define CN(sfx) (snprintf(nm, sizeof nm, "decoder.upsample.%d.%s", b, sfx), nm)
#define CB(sfx) (snprintf(nb, sizeof nb, "decoder.upsample.%d.%s", b, sfx), nb)
        s->cn[b].up = sd_convt(&L, CN("0.conv.weight"), CB("0.conv.bias"), 1024, 1024, 2, 2);
        s->cn[b].dw = sd_vec(&L, CN("1.dwconv.conv.weight"), 1024 * 7);
        s->cn[b].db = sd_vec(&L, CN("1.dwconv.conv.bias"), 1024);
        s->cn[b].lw = sd_vec(&L, CN("1.norm.weight"), 1024);
        s->cn[b].lb = sd_vec(&L, CN("1.norm.bias"), 1024);
        s->cn[b].gamma = sd_vec(&L, CN("1.gamma"), 1024);
        s->cn[b].pw1 = sd_linear(&L, CN("1.pwconv1.weight"), CB("1.pwconv1.bias"), 4096, 1024);
        s->cn[b].pw2 = sd_linear(&L, CN("1.pwconv2.weight"), CB("1.pwconv2.bias"), 1024, 4096);
#undef CN
#undef CB
    }
    s->init = sd_conv(&L, "decoder.decoder.0.conv.weight", "decoder.decoder.0.conv.bias", 1536, 1024, 7, 1);
    {
        int cin = 1536;
        for (int b = 0; b < 4 && !L.bad; b++) {
            const int r = UP_RATE[b], c = UP_CH[b];
#define BN(sfx) (snprintf(nm, sizeof nm, "decoder.decoder.%d.block.%s", b + 1, sfx), nm)
#define BB(sfx) (snprintf(nb, sizeof nb, "decoder.decoder.%d.block.%s", b + 1, sfx), nb)
            s->blk[b].s = sd_snake(&L, BN("0.alpha"), BB("0.beta"), cin);
            s->blk[b].up = sd_convt(&L, BN("1.conv.weight"), BB("1.conv.bias"), cin, c, 2 * r, r);
            for (int u = 0; u < 3 && !L.bad; u++) {
                char sa[64], sb[64];
                snprintf(sa, sizeof sa, "%d.act1.alpha", u + 2); snprintf(sb, sizeof sb, "%d.act1.beta", u + 2);
                s->blk[b].r[u].s1 = sd_snake(&L, BN(sa), BB(sb), c);
                snprintf(sa, sizeof sa, "%d.act2.alpha", u + 2); snprintf(sb, sizeof sb, "%d.act2.beta", u + 2);
                s->blk[b].r[u].s2 = sd_snake(&L, BN(sa), BB(sb), c);
                snprintf(sa, sizeof sa, "%d.conv1.conv.weight", u + 2); snprintf(sb, sizeof sb, "%d.conv1.conv.bias", u + 2);
                s->blk[b].r[u].c1 = sd_conv(&L, BN(sa), BB(sb), c, c, 7, DIL[u]);
                snprintf(sa, sizeof sa, "%d.conv2.conv.weight", u + 2); snprintf(sb, sizeof sb, "%d.conv2.conv.bias", u + 2);
                s->blk[b].r[u].c2 = sd_conv(&L, BN(sa), BB(sb), c, c, 1, 1);
            }
#undef BN
#undef BB
            cin = c;
        }
    }
    s->fs = sd_snake(&L, "decoder.decoder.5.alpha", "decoder.decoder.5.beta", 96);
    s->fw = sd_vec(&L, "decoder.decoder.6.conv.weight", 96 * 7);
    s->fb = sd_vec(&L, "decoder.decoder.6.conv.bias", 1);
    if (L.bad) goto fail;
    /* RoPE tables of the pre-transformer: angle = pos / theta^(2i/64) (sd.c:455-463) */
    {
        float *c = sd_tmp(&L, (size_t)2 * SD_ROPE_POS * 32);
        if (L.bad) goto fail;
        for (int p = 0; p < SD_ROPE_POS; p++)
            for (int i = 0; i < 32; i++) {
                const float ang = (float)p / powf(10000.0f, (float)(2 * i) / 64.0f);
                c[p * 32 + i] = cosf(ang);
                c[SD_ROPE_POS * 32 + p * 32 + i] = sinf(ang);
            }
        s->rope_c = sd_put(&L, c, (size_t)SD_ROPE_POS * 32);
        s->rope_s = sd_put(&L, c + SD_ROPE_POS * 32, (size_t)SD_ROPE_POS * 32);
    }
    if (L.bad || hipStreamSynchronize(s->st) != hipSuccess) goto fail;
    free(L.tmp);
    return s;
fail:
    free(L.tmp);
    if (!qwen_hip_last_error()[0]) qt_seterr("sd_init failed");
    qwen_hip_sd_free(s);
    return NULL;
}

/* ---- decode --------------------------------------------------------------------------------- */
static size_t sd_big_floats(int n) {
    /* the largest [T][C] of the conv stages: block 4 at T = 1920 n, C = 96 (ConvNeXt pw1
     * [4n][4096] and the others are smaller) */
    return (size_t)SD_SPF * n * 96 + 64;
}

static int sd_reserve(sd_t *s, int n) {
    if (n <= s->cap) return 0;
    float **ws[] = {&s->E, &s->V, &s->P, &s->H, &s->XN, &s->QKV, &s->A, &s->GU, &s->M, &s->LAT, &s->big[0], &s->big[1],
                    &s->big[2], &s->daudio};
    const size_t sz[] = {512, 512, 1024, 512, 512, 3072, 1024, 2048, 1024, 1024, 0, 0, 0, SD_SPF};
    (void)hipStreamSynchronize(s->st);
    for (size_t i = 0; i < sizeof ws / sizeof ws[0]; i++) {
        if (*ws[i]) (void)hipFree(*ws[i]);
        *ws[i] = NULL;
        const size_t f = sz[i] ? sz[i] * (size_t)n : sd_big_floats(n);
        if (hipMalloc((void **)ws[i], f * sizeof(float)) != hipSuccess) { s->cap = 0; qt_seterr("sd_decode: out of device memory for %d frames", n); return -1; }
    }
    if (s->dcodes) (void)hipFree(s->dcodes);
    s->dcodes = NULL;
    if (hipMalloc((void **)&s->dcodes, (size_t)n * 16 * sizeof(int)) != hipSuccess) { s->cap = 0; qt_seterr("sd_decode: out of device memory"); return -1; }
    s->cap = n;
    return 0;
}

static hipError_t sd_run(const sd_t *s, const sd_conv_t *c, const float *X, int Tx, int T, float *Y, int epi,
                         const float *cscale, const float *R) {
    return qt_launch_sd_gemm(X, c->K, Tx, 0, c->w, c->K, c->N, c->ntap, c->off, c->phases, T, Y, c->N,
                             c->b, cscale, R, NULL, NULL, NULL, epi | (c->b ? SD_BIAS : 0), 0, s->st);
}

/* the same with a snake on the output: in place (Y2 == NULL) or into Y2 beside Y */
static hipError_t sd_run_snake(const sd_t *s, const sd_conv_t *c, const float *X, int Tx, int T, float *Y, int epi,
                               const float *R, const sd_snake_t *sn, float *Y2) {
    return qt_launch_sd_gemm(X, c->K, Tx, 0, c->w, c->K, c->N, c->ntap, c->off, c->phases, T, Y, c->N, c->b, NULL, R,
                             sn->a, sn->ib, Y2, epi | (c->b ? SD_BIAS : 0) | (Y2 ? SD_SNAKE2 : SD_SNAKE), 0, s->st);
}

#define SCK(call) do { hipError_t e_ = (call); if (e_ != hipSuccess) { \
    qt_seterr("sd_decode: %s -> %s", #call, hipGetErrorString(e_)); return -1; } } while (0)

/* VQ + pre-transformer: codes -> s->LAT [n][1024] (sd.c:599-1044) */
static int sd_enqueue_latent(sd_t *s, const int *d_codes, int n) {
    const hipStream_t st = s->st;
    SCK(qt_launch_sd_vq(d_codes, s->cb, s->E, n, SD_CBSIZE, st));
    SCK(sd_run(s, &s->vq, s->E, n, n, s->V, 0, NULL, NULL));
    SCK(sd_run(s, &s->pre, s->V, n, n, s->P, 0, NULL, NULL));
    SCK(sd_run(s, &s->inp, s->P, n, n, s->H, 0, NULL, NULL));
    for (int l = 0; l < 8; l++) {
        const sd_layer_t *y = &s->L[l];
        SCK(qt_launch_sd_rmsnorm(s->H, y->n1, s->XN, n, 512, 1e-5f, st));
        SCK(sd_run(s, &y->qkv, s->XN, n, n, s->QKV, 0, NULL, NULL));
        SCK(qt_launch_sd_rope(s->QKV, s->rope_c, s->rope_s, n, 0, 0, st));
        SCK(qt_launch_sd_attn(s->QKV, s->A, n, 0, 0, 72, 0.125f, st));
        SCK(sd_run(s, &y->o, s->A, n, n, s->H, SD_CSCALE | SD_RESID, y->ls1, s->H));
        SCK(qt_launch_sd_rmsnorm(s->H, y->n2, s->XN, n, 512, 1e-5f, st));
        SCK(sd_run(s, &y->gu, s->XN, n, n, s->GU, 0, NULL, NULL));
        SCK(qt_launch_sd_swiglu(s->GU, s->M, n, 1024, st));
        SCK(sd_run(s, &y->dn, s->M, n, n, s->H, SD_CSCALE | SD_RESID, y->ls2, s->H));
    }
    SCK(qt_launch_sd_rmsnorm(s->H, s->fnorm, s->XN, n, 512, 1e-5f, st));
    SCK(sd_run(s, &s->outp, s->XN, n, n, s->LAT, 0, NULL, NULL));
    return 0;
}

/* the decode on device buffers, enqueued on the state's stream */
static int sd_enqueue(sd_t *s, const int *d_codes, int n, float *d_audio) {
    const hipStream_t st = s->st;
    if (sd_enqueue_latent(s, d_codes, n)) return -1;
    /* ConvNeXt upsamplers: sig [T][1024] -> [2T][1024] each */
    float *sig = s->LAT, *b0 = s->big[0], *b1 = s->big[1], *b2 = s->big[2];
    int T = n;
    for (int b = 0; b < 2; b++) {
        float *up = b == 0 ? b0 : b2, *dl = b == 0 ? b1 : b0, *pw = b == 0 ? b2 : b1;
        SCK(sd_run(s, &s->cn[b].up, sig, T, T, up, 0, NULL, NULL));
        T *= 2;
        SCK(qt_launch_sd_dwln(up, s->cn[b].dw, s->cn[b].db, s->cn[b].lw, s->cn[b].lb, dl, T, 1024, 0, st));
        SCK(sd_run(s, &s->cn[b].pw1, dl, T, T, pw, SD_GELU, NULL, NULL));
        SCK(sd_run(s, &s->cn[b].pw2, pw, T, T, up, SD_CSCALE | SD_RESID, s->cn[b].gamma, up));
        sig = up;
    }
    /* sig == b2 here; initial conv 1024 -> 1536, its output through block 1's input snake.
     * Every snake of the upsampler is applied by the GEMM that produces its input:
     * transposed conv -> signal + snake1(signal) of unit 1; conv1 -> snake2 in place;
     * conv2 (+ residual) -> signal + snake1 of the next unit, or, after unit 3, the signal
     * through the next block's input snake (or the final snake) in place. */
    SCK(sd_run_snake(s, &s->init, sig, T, T, b0, 0, NULL, &s->blk[0].s, NULL));
    float *cur = b0, *f1 = b1, *f2 = b2;
    for (int b = 0; b < 4; b++) {
        const int r = UP_RATE[b];
        SCK(sd_run_snake(s, &s->blk[b].up, cur, T, T, f1, 0, NULL, &s->blk[b].r[0].s1, f2));
        T *= r;
        { float *t_ = cur; cur = f1; f1 = f2; f2 = t_; }  /* cur: signal, f1: snake1(signal) */
        for (int u = 0; u < 3; u++) {
            SCK(sd_run_snake(s, &s->blk[b].r[u].c1, f1, T, T, f2, 0, NULL, &s->blk[b].r[u].s2, NULL));
            if (u < 2)
                SCK(sd_run_snake(s, &s->blk[b].r[u].c2, f2, T, T, cur, SD_RESID, cur, &s->blk[b].r[u + 1].s1, f1));
            else
                SCK(sd_run_snake(s, &s->blk[b].r[u].c2, f2, T, T, cur, SD_RESID, cur, b < 3 ? &s->blk[b + 1].s : &s->fs,
                                 NULL));
        }
    }
    SCK(qt_launch_sd_final(cur, s->fw, s->fb, d_audio, T, 96, 0, st));
    return 0;
}

int qwen_hip_sd_decode_device(void *state, const int *d_codes, int n_frames, float *d_audio) {
    sd_t *s = (sd_t *)state;
    if (!s || !d_codes || !d_audio) { qt_seterr("sd_decode_device: null argument"); return -1; }
    if (n_frames < 1 || n_frames > SD_ROPE_POS) { qt_seterr("sd_decode_device: %d frames (1..%d)", n_frames, SD_ROPE_POS); return -1; }
    if (sd_reserve(s, n_frames)) return -1;
    return sd_enqueue(s, d_codes, n_frames, d_audio);
}

int qwen_hip_sd_decode(void *state, const int *codes, int n_frames, float *audio_out, int max_samples) {
    sd_t *s = (sd_t *)state;
    if (!s || !codes || !audio_out) { qt_seterr("sd_decode: null argument"); return -1; }
    if (n_frames < 1 || n_frames > SD_ROPE_POS) { qt_seterr("sd_decode: %d frames (1..%d)", n_frames, SD_ROPE_POS); return -1; }
    const long long ns = (long long)n_frames * SD_SPF;
    if (max_samples < ns) { qt_seterr("sd_decode: %d frames need %lld samples, buffer holds %d", n_frames, ns, max_samples); return -1; }
    if (sd_reserve(s, n_frames)) return -1;
    SCK(hipMemcpyAsync(s->dcodes, codes, (size_t)n_frames * 16 * sizeof(int), hipMemcpyHostToDevice, s->st));
    if (sd_enqueue(s, s->dcodes, n_frames, s->daudio)) return -1;
    SCK(hipMemcpyAsync(audio_out, s->daudio, (size_t)ns * sizeof(float), hipMemcpyDeviceToHost, s->st));
    SCK(hipStreamSynchronize(s->st));
    return (int)ns;
}

int qwen_hip_sd_latent(void *state, const int *codes, int n_frames, float *latent_out) {
    sd_t *s = (sd_t *)state;
    if (!s || !codes || !latent_out) { qt_seterr("sd_latent: null argument"); return -1; }
    if (n_frames < 1 || n_frames > SD_ROPE_POS) { qt_seterr("sd_latent: %d frames (1..%d)", n_frames, SD_ROPE_POS); return -1; }
    if (sd_reserve(s, n_frames)) return -1;
    SCK(hipMemcpyAsync(s->dcodes, codes, (size_t)n_frames * 16 * sizeof(int), hipMemcpyHostToDevice, s->st));
    if (sd_enqueue_latent(s, s->dcodes, n_frames)) return -1;
    SCK(hipMemcpyAsync(latent_out, s->LAT, (size_t)n_frames * 1024 * sizeof(float), hipMemcpyDeviceToHost, s->st));
    SCK(hipStreamSynchronize(s->st));
    return 0;
}

void *qwen_hip_sd_stream(void *state) { return state ? (void *)((sd_t *)state)->st : NULL; }

/* ---- single-layer entry points (parity tests of the implicit GEMM) ------------------------ */
typedef struct { const float *w; long long n; } sd_one_t;
static const float *sd_one_get(void *user, const char *name, long long n) {
    const sd_one_t *o = (const sd_one_t *)user;
    (void)name;
    return n == o->n ? o->w : NULL;
}

/* one layer through the decoder's GEMM: conv (kernel k, dilation d) when stride == 0, else a
 * transposed conv of that stride; X [Tin][Cin] time-major host array, Y [Tout][Cout] */
static int sd_op(float *Y, const float *X, const float *W, const float *bias, int Tin, int Cin, int Cout, int k, int d,
                 int stride, int tile) {
    sd_t tmp;
    memset(&tmp, 0, sizeof tmp);
    float *dx = NULL, *dy = NULL;
    int rc = -1;
    if (!Y || !X || !W || Tin < 1 || Cin < 16 || Cin % 16 || Cout < 4 || Cout % 4 || k < 1 ||
        (stride ? (k > 2 * stride || stride > 64) : k > 8) || (tile && tile != 16 && tile != 32 && tile != 64 && tile != 128)) {
        qt_seterr("op_sd_conv: bad shape (Cin multiple of 16, Cout of 4; conv kernel 1..8, transposed kernel <= 2 stride)");
        return -1;
    }
    sd_one_t one = {W, (long long)Cout * Cin * k};
    sd_ld_t L = {sd_one_get, &one, &tmp, NULL, 0, 0};
    if (hipStreamCreateWithFlags(&tmp.st, hipStreamNonBlocking) != hipSuccess) { qt_seterr("op_sd_conv: stream"); return -1; }
    sd_conv_t c = stride ? sd_convt(&L, "w", NULL, Cin, Cout, k, stride) : sd_conv(&L, "w", NULL, Cout, Cin, k, d);
    if (!L.bad && bias) c.b = sd_put(&L, bias, (size_t)Cout);
    free(L.tmp);
    const int Tout = stride ? Tin * stride : Tin;
    if (L.bad) goto done;
    if (hipMalloc((void **)&dx, (size_t)Tin * Cin * sizeof(float)) != hipSuccess ||
        hipMalloc((void **)&dy, (size_t)Tout * Cout * sizeof(float)) != hipSuccess) { qt_seterr("op_sd_conv: alloc"); goto done; }
    if (hipMemcpy(dx, X, (size_t)Tin * Cin * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) goto done;
    if (qt_launch_sd_gemm(dx, Cin, Tin, 0, c.w, Cin, Cout, c.ntap, c.off, c.phases, Tin, dy, Cout, c.b, NULL, NULL, NULL,
                          NULL, NULL, c.b ? SD_BIAS : 0, tile, tmp.st) != hipSuccess ||
        hipMemcpyAsync(Y, dy, (size_t)Tout * Cout * sizeof(float), hipMemcpyDeviceToHost, tmp.st) != hipSuccess ||
        hipStreamSynchronize(tmp.st) != hipSuccess) { qt_seterr("op_sd_conv: launch failed"); goto done; }
    rc = 0;
done:
    if (dx) (void)hipFree(dx);
    if (dy) (void)hipFree(dy);
    for (int i = 0; i < tmp.n_allocs; i++) (void)hipFree(tmp.allocs[i]);
    free(tmp.allocs);
    (void)hipStreamDestroy(tmp.st);
    return rc;
}

int qwen_hip_op_sd_conv(float *Y, const float *X, const float *W, const float *bias, int T, int Cin, int Cout,
                        int kernel, int dilation, int tile) {
    if (dilation < 1) { qt_seterr("op_sd_conv: dilation %d", dilation); return -1; }
    return sd_op(Y, X, W, bias, T, Cin, Cout, kernel, dilation, 0, tile);
}

int qwen_hip_op_sd_conv_transpose(float *Y, const float *X, const float *W, const float *bias, int Tin, int Cin,
                                  int Cout, int kernel, int stride, int tile) {
    if (stride < 1) { qt_seterr("op_sd_conv_transpose: stride %d", stride); return -1; }
    return sd_op(Y, X, W, bias, Tin, Cin, Cout, kernel, 1, stride, tile);
}

/* ---- streaming decode (qwen_speech_decoder_decode_streaming_st, sd.c:1881-2389) ------------
 * The reference's streaming contract: each call takes new frames and returns exactly
 * their 1920 samples each, equal to that slice of a one-shot decode (so the ConvNeXt
 * LayerNorm is the one-shot decode's E[x^2] - mean^2; the reference's streaming path
 * computes a two-pass one, qwen_tts_speech_decoder.c:1343-1352).  Here every stage whose
 * kernel looks back in time keeps the previous chunk's last rows in front of its input
 * buffer (history rows at negative indices, zero before the first chunk, which is the
 * causal padding): pre-conv 2 rows, the pre-transformer's roped q|k|v 71 rows per layer
 * (window 72, positions continue across chunks), the ConvNeXt depthwise convs 6, the initial
 * conv 6, each block's transposed conv 1 (its input: the previous block's signal, or the
 * initial conv's output), each residual unit's dilated conv 6 d, the final conv 6.  The GEMM
 * reads those rows through its negative tap offsets, so a chunk computes only its own rows,
 * in the same arithmetic order as the one-shot decode (chunking does not change a bit). */
#define SDS_CAP 32            /* frames per internal chunk (longer calls are split) */
#define SDS_KH 71             /* key history of the 72-frame attention window */

typedef struct { float *p; int H, C; } sds_buf_t;   /* [H history + rows][C] */

typedef struct {
    sd_t *sd;
    int frames;               /* frames decoded so far */
    sds_buf_t V, Q[8], U[2], I, C0, S[4], F1[4][3];
    float *E, *P, *Hh, *XN, *A, *GU, *M, *LAT, *CN0, *D, *PW, *F2;
    int *dcodes; float *daudio;
    void **allocs; int n_allocs;
} sds_t;

static float *sds_alloc(sds_t *q, size_t floats) {
    void *p = NULL;
    if (hipMalloc(&p, floats * sizeof(float)) != hipSuccess) return NULL;
    void **na = (void **)realloc(q->allocs, (size_t)(q->n_allocs + 1) * sizeof *na);
    if (!na) { (void)hipFree(p); return NULL; }
    q->allocs = na;
    q->allocs[q->n_allocs++] = p;
    return (float *)p;
}

static int sds_buf(sds_t *q, sds_buf_t *b, int H, int rows, int C) {
    b->H = H; b->C = C;
    b->p = sds_alloc(q, (size_t)(H + rows) * C);
    return b->p ? 0 : -1;
}

static float *sds_new_rows(const sds_buf_t *b) { return b->p + (size_t)b->H * b->C; }

void qwen_hip_sd_stream_free(void *state) {
    sds_t *q = (sds_t *)state;
    if (!q) return;
    if (q->sd && q->sd->st) (void)hipStreamSynchronize(q->sd->st);
    for (int i = 0; i < q->n_allocs; i++) (void)hipFree(q->allocs[i]);
    free(q->allocs);
    if (q->dcodes) (void)hipFree(q->dcodes);
    free(q);
}

/* every history back to zero: the next call starts a new utterance (qwen_sd_stream_init) */
int qwen_hip_sd_stream_reset(void *state) {
    sds_t *q = (sds_t *)state;
    if (!q) { qt_seterr("sd_stream_reset: null state"); return -1; }
    sds_buf_t *bs[] = {&q->V, &q->U[0], &q->U[1], &q->I, &q->C0, &q->S[0], &q->S[1], &q->S[2], &q->S[3]};
    for (size_t i = 0; i < sizeof bs / sizeof bs[0]; i++)
        if (hipMemsetAsync(bs[i]->p, 0, (size_t)bs[i]->H * bs[i]->C * sizeof(float), q->sd->st) != hipSuccess) goto fail;
    for (int l = 0; l < 8; l++)
        if (hipMemsetAsync(q->Q[l].p, 0, (size_t)q->Q[l].H * q->Q[l].C * sizeof(float), q->sd->st) != hipSuccess) goto fail;
    for (int b = 0; b < 4; b++)
        for (int u = 0; u < 3; u++)
            if (hipMemsetAsync(q->F1[b][u].p, 0, (size_t)q->F1[b][u].H * q->F1[b][u].C * sizeof(float), q->sd->st) != hipSuccess)
                goto fail;
    if (hipStreamSynchronize(q->sd->st) != hipSuccess) goto fail;
    q->frames = 0;
    return 0;
fail:
    qt_seterr("sd_stream_reset: device memset failed");
    return -1;
}

void *qwen_hip_sd_stream_new(void *sd_state) {
    sd_t *s = (sd_t *)sd_state;
    if (!s) { qt_seterr("sd_stream_new: null decoder state"); return NULL; }
    sds_t *q = (sds_t *)calloc(1, sizeof *q);
    if (!q) { qt_seterr("sd_stream_new: out of host memory"); return NULL; }
    q->sd = s;
    const int n = SDS_CAP;
    int bad = 0;
    bad |= sds_buf(q, &q->V, 2, n, 512);
    for (int l = 0; l < 8; l++) bad |= sds_buf(q, &q->Q[l], SDS_KH, n, 3072);
    bad |= sds_buf(q, &q->U[0], 6, 2 * n, 1024);
    bad |= sds_buf(q, &q->U[1], 6, 4 * n, 1024);
    bad |= sds_buf(q, &q->I, 6, 4 * n, 1024);
    bad |= sds_buf(q, &q->C0, 1, 4 * n, 1536);
    int T = 4 * n;
    for (int b = 0; b < 4; b++) {
        T *= UP_RATE[b];
        bad |= sds_buf(q, &q->S[b], b < 3 ? 1 : 6, T, UP_CH[b]);
        for (int u = 0; u < 3; u++) bad |= sds_buf(q, &q->F1[b][u], 6 * DIL[u], T, UP_CH[b]);
    }
    const size_t sz[] = {(size_t)n * 512, (size_t)n * 1024, (size_t)n * 512, (size_t)n * 512, (size_t)n * 1024, (size_t)n * 2048,
                         (size_t)n * 1024, (size_t)n * 1024, (size_t)2 * n * 1024, (size_t)4 * n * 1024,
                         (size_t)4 * n * 4096, (size_t)T * 96};
    float **ws[] = {&q->E, &q->P, &q->Hh, &q->XN, &q->A, &q->GU, &q->M, &q->LAT, &q->CN0, &q->D, &q->PW, &q->F2};
    for (size_t i = 0; i < sizeof ws / sizeof ws[0]; i++) if (!(*ws[i] = sds_alloc(q, sz[i]))) bad = 1;
    if (!(q->daudio = sds_alloc(q, (size_t)n * SD_SPF))) bad = 1;
    if (hipMalloc((void **)&q->dcodes, (size_t)n * 16 * sizeof(int)) != hipSuccess) bad = 1;
    if (bad) { qt_seterr("sd_stream_new: out of device memory"); qwen_hip_sd_stream_free(q); return NULL; }
    if (qwen_hip_sd_stream_reset(q)) { qwen_hip_sd_stream_free(q); return NULL; }
    return q;
}

static hipError_t sds_gemm(const sd_t *s, const sd_conv_t *c, const float *X, int xlo, int T, float *Y, int epi,
                           const float *cscale, const float *R, const sd_snake_t *sn, float *Y2) {
    int e = epi | (c->b ? SD_BIAS : 0);
    if (sn) e |= Y2 ? SD_SNAKE2 : SD_SNAKE;
    return qt_launch_sd_gemm(X, c->K, T, xlo, c->w, c->K, c->N, c->ntap, c->off, c->phases, T, Y, c->N, c->b, cscale, R,
                             sn ? sn->a : NULL, sn ? sn->ib : NULL, Y2, e, 0, s->st);
}

/* one chunk of n <= SDS_CAP frames: codes already in q->dcodes, audio into q->daudio */
static int sds_chunk(sds_t *q, int n) {
    sd_t *s = q->sd;
    const hipStream_t st = s->st;
    const int fb = q->frames;
    SCK(qt_launch_sd_vq(q->dcodes, s->cb, q->E, n, SD_CBSIZE, st));
    SCK(sds_gemm(s, &s->vq, q->E, 0, n, sds_new_rows(&q->V), 0, NULL, NULL, NULL, NULL));
    SCK(sds_gemm(s, &s->pre, sds_new_rows(&q->V), -q->V.H, n, q->P, 0, NULL, NULL, NULL, NULL));
    SCK(sds_gemm(s, &s->inp, q->P, 0, n, q->Hh, 0, NULL, NULL, NULL, NULL));
    const int kh = fb < SDS_KH ? fb : SDS_KH;
    for (int l = 0; l < 8; l++) {
        const sd_layer_t *y = &s->L[l];
        SCK(qt_launch_sd_rmsnorm(q->Hh, y->n1, q->XN, n, 512, 1e-5f, st));
        SCK(sds_gemm(s, &y->qkv, q->XN, 0, n, sds_new_rows(&q->Q[l]), 0, NULL, NULL, NULL, NULL));
        SCK(qt_launch_sd_rope(q->Q[l].p, s->rope_c, s->rope_s, n, SDS_KH, fb, st));
        SCK(qt_launch_sd_attn(q->Q[l].p, q->A, n, SDS_KH, SDS_KH - kh, 72, 0.125f, st));
        SCK(sds_gemm(s, &y->o, q->A, 0, n, q->Hh, SD_CSCALE | SD_RESID, y->ls1, q->Hh, NULL, NULL));
        SCK(qt_launch_sd_rmsnorm(q->Hh, y->n2, q->XN, n, 512, 1e-5f, st));
        SCK(sds_gemm(s, &y->gu, q->XN, 0, n, q->GU, 0, NULL, NULL, NULL, NULL));
        SCK(qt_launch_sd_swiglu(q->GU, q->M, n, 1024, st));
        SCK(sds_gemm(s, &y->dn, q->M, 0, n, q->Hh, SD_CSCALE | SD_RESID, y->ls2, q->Hh, NULL, NULL));
    }
    SCK(qt_launch_sd_rmsnorm(q->Hh, s->fnorm, q->XN, n, 512, 1e-5f, st));
    SCK(sds_gemm(s, &s->outp, q->XN, 0, n, q->LAT, 0, NULL, NULL, NULL, NULL));
    /* ConvNeXt upsamplers (the transposed convs look back 0 rows, the depthwise convs 6) */
    int T = n;
    const float *cin = q->LAT;
    for (int b = 0; b < 2; b++) {
        float *up = sds_new_rows(&q->U[b]);
        float *out = b == 0 ? q->CN0 : sds_new_rows(&q->I);
        SCK(sds_gemm(s, &s->cn[b].up, cin, 0, T, up, 0, NULL, NULL, NULL, NULL));
        T *= 2;
        SCK(qt_launch_sd_dwln(up, s->cn[b].dw, s->cn[b].db, s->cn[b].lw, s->cn[b].lb, q->D, T, 1024, -q->U[b].H, st));
        SCK(sds_gemm(s, &s->cn[b].pw1, q->D, 0, T, q->PW, SD_GELU, NULL, NULL, NULL, NULL));
        SCK(sds_gemm(s, &s->cn[b].pw2, q->PW, 0, T, out, SD_CSCALE | SD_RESID, s->cn[b].gamma, up, NULL, NULL));
        cin = out;
    }
    /* initial conv (6 rows back), output through block 1's input snake */
    SCK(sds_gemm(s, &s->init, sds_new_rows(&q->I), -q->I.H, T, sds_new_rows(&q->C0), 0, NULL, NULL, &s->blk[0].s, NULL));
    const sds_buf_t *in = &q->C0;
    for (int b = 0; b < 4; b++) {
        const int r = UP_RATE[b];
        float *sig = sds_new_rows(&q->S[b]);
        SCK(sds_gemm(s, &s->blk[b].up, sds_new_rows(in), -in->H, T, sig, 0, NULL, NULL, &s->blk[b].r[0].s1,
                     sds_new_rows(&q->F1[b][0])));
        T *= r;
        for (int u = 0; u < 3; u++) {
            SCK(sds_gemm(s, &s->blk[b].r[u].c1, sds_new_rows(&q->F1[b][u]), -q->F1[b][u].H, T, q->F2, 0, NULL, NULL,
                         &s->blk[b].r[u].s2, NULL));
            if (u < 2)
                SCK(sds_gemm(s, &s->blk[b].r[u].c2, q->F2, 0, T, sig, SD_RESID, NULL, sig, &s->blk[b].r[u + 1].s1,
                             sds_new_rows(&q->F1[b][u + 1])));
            else
                SCK(sds_gemm(s, &s->blk[b].r[u].c2, q->F2, 0, T, sig, SD_RESID, NULL, sig, b < 3 ? &s->blk[b + 1].s : &s->fs,
                             NULL));
        }
        in = &q->S[b];
    }
    SCK(qt_launch_sd_final(sds_new_rows(&q->S[3]), s->fw, s->fb, q->daudio, T, 96, -q->S[3].H, st));
    /* histories for the next chunk: each buffer's last H rows (of H + its rows this chunk) */
    SCK(qt_launch_sd_shift(q->V.p, q->V.H, n, 512, st));
    for (int l = 0; l < 8; l++) SCK(qt_launch_sd_shift(q->Q[l].p, SDS_KH, n, 3072, st));
    SCK(qt_launch_sd_shift(q->U[0].p, q->U[0].H, 2 * n, 1024, st));
    SCK(qt_launch_sd_shift(q->U[1].p, q->U[1].H, 4 * n, 1024, st));
    SCK(qt_launch_sd_shift(q->I.p, q->I.H, 4 * n, 1024, st));
    SCK(qt_launch_sd_shift(q->C0.p, q->C0.H, 4 * n, 1536, st));
    T = 4 * n;
    for (int b = 0; b < 4; b++) {
        T *= UP_RATE[b];
        SCK(qt_launch_sd_shift(q->S[b].p, q->S[b].H, T, UP_CH[b], st));
        for (int u = 0; u < 3; u++) SCK(qt_launch_sd_shift(q->F1[b][u].p, q->F1[b][u].H, T, UP_CH[b], st));
    }
    q->frames += n;
    return 0;
}

int qwen_hip_sd_stream_decode(void *state, const int *new_codes, int new_frames, float *audio_out, int max_samples) {
    sds_t *q = (sds_t *)state;
    if (!q || !new_codes || !audio_out) { qt_seterr("sd_stream_decode: null argument"); return -1; }
    if (new_frames < 1 || q->frames + new_frames > SD_ROPE_POS) {
        qt_seterr("sd_stream_decode: %d new frames after %d (at most %d in a stream)", new_frames, q->frames, SD_ROPE_POS);
        return -1;
    }
    const long long ns = (long long)new_frames * SD_SPF;
    if (max_samples < ns) { qt_seterr("sd_stream_decode: %d frames need %lld samples, buffer holds %d", new_frames, ns, max_samples); return -1; }
    for (int off = 0; off < new_frames; off += SDS_CAP) {
        const int n = new_frames - off < SDS_CAP ? new_frames - off : SDS_CAP;
        SCK(hipMemcpyAsync(q->dcodes, new_codes + (size_t)off * 16, (size_t)n * 16 * sizeof(int), hipMemcpyHostToDevice,
                           q->sd->st));
        if (sds_chunk(q, n)) return -1;
        SCK(hipMemcpyAsync(audio_out + (size_t)off * SD_SPF, q->daudio, (size_t)n * SD_SPF * sizeof(float),
                           hipMemcpyDeviceToHost, q->sd->st));
    }
    SCK(hipStreamSynchronize(q->sd->st));
    return (int)ns;
}
