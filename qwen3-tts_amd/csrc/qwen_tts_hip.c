/*
 * qwen_tts_hip.c — host side of the MI355X decode-step library (C, HIP runtime API).
 *
 * What the reference's qwen_tts_cuda_talker.cu host code does (resident weights + KV,
 * one graph per step, device-side position; qwen_tts_cuda_talker.cu:313-438), redone
 * for gfx950:
 *   - weights are uploaded once into the device encodings of qt_device.h (Q|K|V rows
 *     concatenated into one matrix per layer so the QKV projection is one launch;
 *     int8 the reference's signed bytes; q4_0 split into qs rows + f16 scale bits);
 *   - the KV cache stays bf16 on the device (the reference keeps f32 with truncated
 *     mantissas, qwen_tts_cuda_talker.cu:203-208, 350-351), head-major
 *     [layer][kv_head][kv_max][128], so upload is a strided memcpy of the host bits and
 *     a chunk of keys of one head is contiguous;
 *   - a layer is 5 launches: norm+QKV, attention (q/k norm + RoPE + KV append +
 *     split-K + merge), O+residual, norm+gate_up+SwiGLU, down+residual; the step
 *     (n_layers*5 + 1 launches) is captured once into a hipGraph and replayed with the
 *     position read on the device.
 * Every HIP call is checked; a failure marks the state dead and is reported through
 * qwen_hip_last_error().
 */
#include "qwen_tts_hip.h"
#include "qt_launch.h"

#include <hip/hip_runtime_api.h>
#include <math.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static __thread char g_err[512];
const char *qwen_hip_last_error(void) { return g_err; }

#define SETERR(...) do { snprintf(g_err, sizeof g_err, __VA_ARGS__); fprintf(stderr, "[qwen_hip] %s\n", g_err); } while (0)

/* error text from the kernel files (same channel as SETERR) */
void qt_seterr(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    fprintf(stderr, "[qwen_hip] %s\n", g_err);
}
#define HCK(call) do { hipError_t e_ = (call); if (e_ != hipSuccess) { \
    SETERR("%s:%d %s -> %s", __FILE__, __LINE__, #call, hipGetErrorString(e_)); goto fail; } } while (0)
#define REQ(cond, ...) do { if (!(cond)) { SETERR(__VA_ARGS__); goto fail; } } while (0)
/* split-K partials of the bf16 projection GEMMs (prefill, bf16 batch): 32 MiB; the
 * launcher splits K only while its grid is short of the CUs, which bounds the partials
 * well inside this, and never beyond it */
#define PF_PART_FLOATS ((long long)8 << 20)

/* ---- device matrices --------------------------------------------------------------- */

typedef struct {
    int prec, rows, cols;
    uint8_t *w;        /* chunk rows (bf16 bits | int8 q | q4 qs) */
    float *scale;      /* int8 */
    uint16_t *s16;     /* q4 f16 scale bits */
} dmat_t;

static size_t row_bytes(int prec, int cols) {
    return prec == QWEN_HIP_BF16 ? (size_t)cols * 2 : prec == QWEN_HIP_INT8 ? (size_t)cols : (size_t)cols / 2;
}

static int dmat_alloc(dmat_t *m, int prec, int rows, int cols) {
    memset(m, 0, sizeof *m);
    m->prec = prec; m->rows = rows; m->cols = cols;
    HCK(hipMalloc((void **)&m->w, row_bytes(prec, cols) * rows));
    if (prec == QWEN_HIP_INT8) HCK(hipMalloc((void **)&m->scale, (size_t)rows * sizeof(float)));
    if (prec == QWEN_HIP_Q4_0) HCK(hipMalloc((void **)&m->s16, (size_t)rows * (cols / 32) * sizeof(uint16_t)));
    return 0;
fail:
    return -1;
}

static void dmat_free(dmat_t *m) {
    if (m->w) (void)hipFree(m->w);
    if (m->scale) (void)hipFree(m->scale);
    if (m->s16) (void)hipFree(m->s16);
    memset(m, 0, sizeof *m);
}

/* Copy a source matrix (reference host layout, precision src_prec, host or device
 * memory) into rows [r0, r0+rows) of m, converting to m->prec on the device.
 * tmp: device scratch of at least rows*cols*2 bytes. */
static int dmat_put(dmat_t *m, int r0, const qwen_hip_mat_t *src, int src_prec, int rows, hipStream_t st, void *tmp) {
    const int cols = m->cols;
    REQ(src && src->w, "missing weight pointer");
    if (src_prec == m->prec) {
        if (m->prec == QWEN_HIP_BF16) {
            HCK(hipMemcpyAsync(m->w + (size_t)r0 * cols * 2, src->w, (size_t)rows * cols * 2, hipMemcpyDefault, st));
        } else if (m->prec == QWEN_HIP_INT8) {
            REQ(src->scale, "int8 weight without scale");
            HCK(hipMemcpyAsync(m->w + (size_t)r0 * cols, src->w, (size_t)rows * cols, hipMemcpyDefault, st));
            HCK(hipMemcpyAsync(m->scale + r0, src->scale, (size_t)rows * sizeof(float), hipMemcpyDefault, st));
        } else {
            size_t nb = (size_t)rows * (cols / 32);
            HCK(hipMemcpyAsync(tmp, src->w, nb * 18, hipMemcpyDefault, st));
            HCK(qt_launch_repack_q4((const uint8_t *)tmp, nb, m->w + (size_t)r0 * (cols / 2),
                                    m->s16 + (size_t)r0 * (cols / 32), st));
        }
    } else {
        REQ(src_prec == QWEN_HIP_BF16, "can only quantize from bf16 (got prec %d -> %d)", src_prec, m->prec);
        HCK(hipMemcpyAsync(tmp, src->w, (size_t)rows * cols * 2, hipMemcpyDefault, st));
        if (m->prec == QWEN_HIP_INT8)
            HCK(qt_launch_quant_int8((const uint16_t *)tmp, rows, cols, m->w + (size_t)r0 * cols, m->scale + r0, st));
        else
            HCK(qt_launch_quant_q4((const uint16_t *)tmp, rows, cols, m->w + (size_t)r0 * (cols / 2),
                                   m->s16 + (size_t)r0 * (cols / 32), st));
    }
    HCK(hipStreamSynchronize(st));   /* tmp is reused by the next put */
    return 0;
fail:
    return -1;
}

static hipError_t mv(const dmat_t *m, int epi, int norm, const float *vin, const float *nw, float eps,
                     float *out, float *resid, const float *bias, hipStream_t st) {
    return qt_launch_mv(m->prec, epi, norm, vin, nw, eps, m->w, m->scale, m->s16, m->rows, m->cols,
                        out, resid, bias, NULL, st);
}

static float *up_f32(const float *src, size_t n, hipStream_t st) {
    float *d = NULL;
    if (!src) { SETERR("missing f32 tensor"); return NULL; }
    if (hipMalloc((void **)&d, n * sizeof(float)) != hipSuccess) { SETERR("hipMalloc %zu f32 failed", n); return NULL; }
    if (hipMemcpyAsync(d, src, n * sizeof(float), hipMemcpyDefault, st) != hipSuccess) {
        (void)hipFree(d); SETERR("upload f32 failed"); return NULL;
    }
    return d;
}

/* One layer's K or V between the host cache rows (position-major [n][n_kv*hd], the
 * reference's kv_cache_k/v layer slice, contiguous) and the device cache (head-major
 * [n_kv][kv_max][hd]): one contiguous copy through a device staging buffer plus a
 * relayout kernel, instead of one strided copy per head with 256-byte rows (which
 * pageable memory serves at tens of MB/s).  stage holds n*n_kv*hd bf16. */
/* Host -> device copies from pageable memory (the reference's KV after its CPU prefill)
 * through two pinned buffers: the CPU copies the next piece of the source into one buffer
 * with UP_THREADS threads while the DMA engine moves the previous piece out of the other.
 * On the MI355X box, 235 MB moved at 40-43 GB/s this way.  hipMemcpy from the same pageable
 * source moved at 25-29 GB/s: it stages through the runtime's own pinned buffers with one
 * copying thread.  As with a pageable hipMemcpyAsync, the source may be reused once the call
 * returns: the DMA still in flight reads the pinned buffer only. */
#define UP_PIECE ((size_t)4 << 20)
#define UP_THREADS 4
typedef struct { void *pin[2]; hipEvent_t ev[2]; int nb; } hpipe_t;

typedef struct { char *d; const char *s; size_t n; } hcopy_t;
static void *hcopy_run(void *p) {
    const hcopy_t *j = (const hcopy_t *)p;
    memcpy(j->d, j->s, j->n);
    return NULL;
}
/* memcpy over up to UP_THREADS page-aligned slices: the calling thread copies the first,
 * and a slice whose thread could not be created is copied by the caller too */
static void par_memcpy(void *dst, const void *src, size_t n) {
    pthread_t th[UP_THREADS];
    hcopy_t jb[UP_THREADS];
    int run[UP_THREADS] = {0};
    const int nt = n >= ((size_t)UP_THREADS << 20) ? UP_THREADS : 1;
    const size_t per = ((n + nt - 1) / nt + 4095) & ~(size_t)4095;
    for (int t = 0; t < nt; t++) {
        const size_t o = (size_t)t * per;
        jb[t].d = (char *)dst + o;
        jb[t].s = (const char *)src + o;
        jb[t].n = o >= n ? 0 : (o + per > n ? n - o : per);
        if (t > 0 && jb[t].n) run[t] = pthread_create(&th[t], NULL, hcopy_run, &jb[t]) == 0;
    }
    hcopy_run(&jb[0]);
    for (int t = 1; t < nt; t++) {
        if (run[t]) pthread_join(th[t], NULL);
        else if (jb[t].n) hcopy_run(&jb[t]);
    }
}
static void hpipe_free(hpipe_t *p) {
    for (int b = 0; b < 2; b++) {
        if (p->pin[b]) (void)hipHostFree(p->pin[b]);
        if (p->ev[b]) (void)hipEventDestroy(p->ev[b]);
    }
    memset(p, 0, sizeof *p);
}
/* the pinned buffers and events of a pipe that runs on stream st (pinning takes
 * milliseconds: the Talker makes its pipe at init, other owners on first use) */
static hipError_t hpipe_init(hpipe_t *p, hipStream_t st) {
    hipError_t e;
    if (p->pin[0] && p->pin[1]) return hipSuccess;
    hpipe_free(p);
    for (int b = 0; b < 2; b++) {
        if ((e = hipHostMalloc(&p->pin[b], UP_PIECE, hipHostMallocDefault)) ||
            (e = hipEventCreateWithFlags(&p->ev[b], hipEventDisableTiming)) || (e = hipEventRecord(p->ev[b], st))) {
            hpipe_free(p);
            return e;
        }
    }
    return hipSuccess;
}
/* `bytes` from pageable host memory to device memory, in order on stream st (one stream
 * per pipe) */
static hipError_t hpipe_upload(hpipe_t *p, void *dev, const void *host, size_t bytes, hipStream_t st) {
    hipError_t e;
    if ((e = hpipe_init(p, st))) return e;
    for (size_t o = 0; o < bytes; o += UP_PIECE) {
        const size_t n = bytes - o < UP_PIECE ? bytes - o : UP_PIECE;
        const int b = p->nb;
        p->nb ^= 1;
        if ((e = hipEventSynchronize(p->ev[b]))) return e;   /* the copy that last read this buffer is done */
        par_memcpy(p->pin[b], (const char *)host + o, n);
        if ((e = hipMemcpyAsync((char *)dev + o, p->pin[b], n, hipMemcpyHostToDevice, st))) return e;
        if ((e = hipEventRecord(p->ev[b], st))) return e;
    }
    return hipSuccess;
}

/* n positions of one layer's K or V between the host rows [n][nkv*hd] and the device's
 * head-major cache, through the device staging buffer and the relayout kernel; uploads
 * go through the pinned pipe */
static hipError_t kv_xfer(uint16_t *dev_heads, int kv_max, uint16_t *host_rows, int n, int nkv, int hd, int upload,
                          uint16_t *stage, hpipe_t *pipe, hipStream_t st) {
    hipError_t e;
    const size_t bytes = (size_t)n * nkv * hd * sizeof(uint16_t);
    if (n <= 0) return hipSuccess;
    if (upload) {
        if ((e = hpipe_upload(pipe, stage, host_rows, bytes, st))) return e;
        return qt_launch_kv_relayout(stage, dev_heads, n, nkv, hd, kv_max, 1, st);
    }
    if ((e = qt_launch_kv_relayout(dev_heads, stage, n, nkv, hd, kv_max, 0, st))) return e;
    return hipMemcpyAsync(host_rows, stage, bytes, hipMemcpyDefault, st);
}

/* ---- one stack of transformer layers on the device (Talker: 28, CP: 5) ------------ */

typedef struct {
    int H, F, nh, nkv, hd, L, kv_max, qd, kvd, prec, rope_len, attn_G;
    int step_G;                /* key chunks per kv head of the single-stream step's attention */
    int step_onepass;          /* ...and each chunk as one softmax (qt_launch_attn_onepass) */
    float eps;
    dmat_t *qkv, *o, *gu, *dn;
    float **in_norm, **post_norm, **qn, **kn;
    float *final_norm, *rope_cos, *rope_sin;
    uint16_t *kc, *vc;         /* [L][nkv][kv_max][hd] */
    float *qkvbuf, *attn, *hbuf;
    float *part; unsigned *cnt;
    uint16_t *kv_stage;        /* [kv_max][n_kv*hd]: KV upload/download staging, made on first use */
    hpipe_t up;                /* pinned buffers of the KV upload */
} stack_t;

static void stack_free(stack_t *s) {
    for (int l = 0; l < s->L; l++) {
        if (s->qkv) dmat_free(&s->qkv[l]);
        if (s->o) dmat_free(&s->o[l]);
        if (s->gu) dmat_free(&s->gu[l]);
        if (s->dn) dmat_free(&s->dn[l]);
        if (s->in_norm && s->in_norm[l]) (void)hipFree(s->in_norm[l]);
        if (s->post_norm && s->post_norm[l]) (void)hipFree(s->post_norm[l]);
        if (s->qn && s->qn[l]) (void)hipFree(s->qn[l]);
        if (s->kn && s->kn[l]) (void)hipFree(s->kn[l]);
    }
    free(s->qkv); free(s->o); free(s->gu); free(s->dn);
    free(s->in_norm); free(s->post_norm); free(s->qn); free(s->kn);
    void *bufs[] = {s->final_norm, s->rope_cos, s->rope_sin, s->kc, s->vc, s->qkvbuf, s->attn, s->hbuf, s->part, s->cnt,
                    s->kv_stage};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) if (bufs[i]) (void)hipFree(bufs[i]);
    hpipe_free(&s->up);
    memset(s, 0, sizeof *s);
}

#define KV_LIMIT 8192   /* the largest cache the attention grid covers (qt_attn_grid) */

static int stack_init(stack_t *s, const qwen_hip_talker_desc_t *d, hipStream_t st) {
    void *tmp = NULL;
    memset(s, 0, sizeof *s);
    REQ(d && d->layers, "null descriptor");
    REQ(d->head_dim == 128, "head_dim %d unsupported (128 only)", d->head_dim);
    REQ(d->n_kv_heads > 0 && d->n_heads % d->n_kv_heads == 0, "bad head counts %d/%d", d->n_heads, d->n_kv_heads);
    REQ(d->kv_max > 0 && qt_attn_grid(d->kv_max) > 0, "kv_max %d out of range (1..8192)", d->kv_max);
    REQ(d->rope_cos && d->rope_sin && d->rope_len > 0, "missing rope tables");
    REQ(d->prec >= 0 && d->prec <= 2, "bad prec %d", d->prec);
    s->H = d->hidden; s->F = d->inter; s->nh = d->n_heads; s->nkv = d->n_kv_heads; s->hd = d->head_dim;
    s->L = d->n_layers; s->kv_max = d->kv_max; s->eps = d->eps;
    s->qd = s->nh * s->hd; s->kvd = s->nkv * s->hd;
    s->prec = (d->quantize_to >= 0) ? d->quantize_to : d->prec;
    REQ(s->prec == d->prec || d->prec == QWEN_HIP_BF16, "quantize_to needs bf16 source weights");
    if (s->prec == QWEN_HIP_Q4_0)
        REQ(s->H % 32 == 0 && s->F % 32 == 0 && s->qd % 32 == 0, "q4_0 needs dims divisible by 32");
    /* the whole rope table (up to the largest cache), so that the KV cache can grow */
    s->rope_len = d->rope_len < KV_LIMIT ? d->rope_len : KV_LIMIT;
    /* split-K grid: short caches (the CP's <= 64 positions) use one chunk per kv head */
    s->attn_G = s->kv_max <= 128 ? 1 : qt_attn_grid(s->kv_max);
    s->step_G = s->attn_G;
    const int L = s->L, H = s->H, F = s->F;
    s->qkv = calloc(L, sizeof(dmat_t)); s->o = calloc(L, sizeof(dmat_t));
    s->gu = calloc(L, sizeof(dmat_t)); s->dn = calloc(L, sizeof(dmat_t));
    s->in_norm = calloc(L, sizeof(float *)); s->post_norm = calloc(L, sizeof(float *));
    s->qn = calloc(L, sizeof(float *)); s->kn = calloc(L, sizeof(float *));
    REQ(s->qkv && s->o && s->gu && s->dn && s->in_norm && s->post_norm && s->qn && s->kn, "host alloc failed");
    size_t tmp_bytes = (size_t)2 * F * H * 2;
    if ((size_t)(s->qd + 2 * s->kvd) * H * 2 > tmp_bytes) tmp_bytes = (size_t)(s->qd + 2 * s->kvd) * H * 2;
    HCK(hipMalloc(&tmp, tmp_bytes));
    for (int l = 0; l < L; l++) {
        const qwen_hip_layer_t *ly = &d->layers[l];
        REQ(dmat_alloc(&s->qkv[l], s->prec, s->qd + 2 * s->kvd, H) == 0, "alloc qkv");
        REQ(dmat_put(&s->qkv[l], 0, &ly->q, d->prec, s->qd, st, tmp) == 0, "upload q (layer %d)", l);
        REQ(dmat_put(&s->qkv[l], s->qd, &ly->k, d->prec, s->kvd, st, tmp) == 0, "upload k (layer %d)", l);
        REQ(dmat_put(&s->qkv[l], s->qd + s->kvd, &ly->v, d->prec, s->kvd, st, tmp) == 0, "upload v (layer %d)", l);
        REQ(dmat_alloc(&s->o[l], s->prec, H, s->qd) == 0, "alloc o");
        REQ(dmat_put(&s->o[l], 0, &ly->o, d->prec, H, st, tmp) == 0, "upload o (layer %d)", l);
        REQ(dmat_alloc(&s->gu[l], s->prec, 2 * F, H) == 0, "alloc gate_up");
        REQ(dmat_put(&s->gu[l], 0, &ly->gate_up, d->prec, 2 * F, st, tmp) == 0, "upload gate_up (layer %d)", l);
        REQ(dmat_alloc(&s->dn[l], s->prec, H, F) == 0, "alloc down");
        REQ(dmat_put(&s->dn[l], 0, &ly->down, d->prec, H, st, tmp) == 0, "upload down (layer %d)", l);
        REQ((s->in_norm[l] = up_f32(ly->input_norm, H, st)) != NULL, "input_norm %d", l);
        REQ((s->post_norm[l] = up_f32(ly->post_attn_norm, H, st)) != NULL, "post_norm %d", l);
        REQ((s->qn[l] = up_f32(ly->q_norm, s->hd, st)) != NULL, "q_norm %d", l);
        REQ((s->kn[l] = up_f32(ly->k_norm, s->hd, st)) != NULL, "k_norm %d", l);
    }
    REQ((s->final_norm = up_f32(d->final_norm, H, st)) != NULL, "final_norm");
    REQ((s->rope_cos = up_f32(d->rope_cos, (size_t)s->rope_len * (s->hd / 2), st)) != NULL, "rope_cos");
    REQ((s->rope_sin = up_f32(d->rope_sin, (size_t)s->rope_len * (s->hd / 2), st)) != NULL, "rope_sin");
    size_t kvn = (size_t)L * s->nkv * s->kv_max * s->hd;
    HCK(hipMalloc((void **)&s->kc, kvn * 2));
    HCK(hipMalloc((void **)&s->vc, kvn * 2));
    HCK(hipMemsetAsync(s->kc, 0, kvn * 2, st));
    HCK(hipMemsetAsync(s->vc, 0, kvn * 2, st));
    HCK(hipMalloc((void **)&s->qkvbuf, (size_t)(s->qd + 2 * s->kvd) * sizeof(float)));
    HCK(hipMalloc((void **)&s->attn, (size_t)s->qd * sizeof(float)));
    HCK(hipMalloc((void **)&s->hbuf, (size_t)(F > H ? F : H) * sizeof(float)));
    HCK(hipMalloc((void **)&s->part, (size_t)s->nkv * s->attn_G * (s->nh / s->nkv) * 130 * sizeof(float)));
    HCK(hipMalloc((void **)&s->cnt, (size_t)s->nkv * sizeof(unsigned)));
    HCK(hipMemsetAsync(s->cnt, 0, (size_t)s->nkv * sizeof(unsigned), st));
    HCK(hipStreamSynchronize(st));
    (void)hipFree(tmp);
    return 0;
fail:
    if (tmp) (void)hipFree(tmp);
    stack_free(s);
    return -1;
}

/* The layers of one pass: x (device residual) in/out, position read from d_pos.
 * Mirrors qwen_talker_step's layer loop (qwen_tts_talker.c:580-690) and
 * cp_layer_body (qwen_tts_code_predictor.c:595-717). */
static hipError_t stack_body_ex(stack_t *s, float *x, const int *d_pos, hipStream_t st, float *layer_out) {
    hipError_t e;
    const float scale = 1.0f / sqrtf((float)s->hd);
    for (int l = 0; l < s->L; l++) {
        const size_t lay = (size_t)l * s->nkv * s->kv_max * s->hd;
        if ((e = mv(&s->qkv[l], QT_EPI_STORE, 1, x, s->in_norm[l], s->eps, s->qkvbuf, NULL, NULL, st))) return e;
        if ((e = (s->step_onepass ? qt_launch_attn_onepass : qt_launch_attn)(
                     1, s->qkvbuf, s->qn[l], s->kn[l], s->rope_cos, s->rope_sin, s->eps, d_pos, 0,
                                s->kc + lay, s->vc + lay, s->hd, (long long)s->kv_max * s->hd, s->nh, s->nkv,
                                s->hd, scale, s->part, s->cnt, s->step_G, s->attn, st))) return e;
        if ((e = mv(&s->o[l], QT_EPI_RESID, 0, s->attn, NULL, s->eps, NULL, x, NULL, st))) return e;
        if ((e = mv(&s->gu[l], QT_EPI_SWIGLU, 1, x, s->post_norm[l], s->eps, s->hbuf, NULL, NULL, st))) return e;
        if ((e = mv(&s->dn[l], QT_EPI_RESID, 0, s->hbuf, NULL, s->eps, NULL, x, NULL, st))) return e;
        if (layer_out && (e = qt_launch_copy_f32(x, layer_out + (size_t)l * s->H, s->H, st))) return e;
    }
    return hipSuccess;
}

static hipError_t stack_body(stack_t *s, float *x, const int *d_pos, hipStream_t st) {
    return stack_body_ex(s, x, d_pos, st, NULL);
}

/* ---- Talker state ------------------------------------------------------------------ */

typedef struct {
    stack_t s;
    hipStream_t st;
    float *io;              /* device [hidden_out H | x H] */
    int *d_pos;             /* device: position of the next step */
    int *d_frame, *d_tok, *d_hist;
    float *h_in, *h_out;    /* pinned: embed in; [hidden | x] out */
    int *h_pos;
    hipGraphExec_t exec, gexec;
    int graph_ready, ggraph_ready, greedy_ready;
    int dev_pos;            /* host mirror of *d_pos (-1 unknown) */
    int dead;
    /* greedy loop */
    const uint16_t *head_host, *emb_host;
    uint16_t *codec_head, *codec_emb;
    int codec_vocab;
    float *logits;
    dmat_t head_m;
    int hist_len;
    /* sampled loop: token history (prev tokens + drawn tokens), LCG state, EOS flag;
     * allocated once at init (QT_SAMPLE_HIST_MAX entries) */
    int *smp_hist;
    uint32_t *smp_seed;
    int *smp_done;
    /* device frame loop: the 16 codes of every frame of a call, the text-side pad embedding */
    int *gen_codes;         /* [QT_SAMPLE_HIST_MAX][16] */
    float *gen_pad;         /* [H] */
    /* persistent single-kernel step (qt_pstep.hip) */
    int ps_on;
    void *ps_layers;        /* device layer table */
    unsigned long long *ps_ring;   /* tagged activation words */
    int rs_on;              /* the role-specialised kernel (qt_rstep.hip) runs the fused step: 1 its 1.7B
                             * build, 2 its 0.6B build (qt_rstep06.hip), 3 its 0.6B bf16 build
                             * (qt_rstep06b.hip), 4 its 1.7B q4_0 build (qt_rstep4.hip) */
    unsigned *rs_reg;       /* its hand-off words, [2][L][layer block], sentinel when empty */
    unsigned long long *rs_slots;  /* its tagged winner words */
    float *ps_xin;          /* step-0 input of a launch */
    unsigned *ps_epoch;     /* tag of the next step */
    int *ps_err;
    int *h_err;             /* pinned */
    /* Talker prefill (qt_prefill.hip): bf16 projection weights (the step's own when they
     * are bf16, else owned copies made on the first prefill) and position buffers */
    dmat_t *pf_qkv, *pf_o, *pf_gu, *pf_dn;
    int pf_cap;             /* positions the buffers below hold */
    float *pf_x, *pf_qkvb, *pf_attn, *pf_h;
    float *pf_e;            /* the last prefill's embeddings (pf_x becomes the residual stream) */
    float *pf_part;         /* split-K partial sums, PF_PART_FLOATS */
    uint16_t *pf_p;         /* activation planes [3][spad][max(H, qd, F)] */
} talker_t;

/* QWEN_HIP_RSTEP=0 keeps the single-role persistent kernel (qt_pstep.hip) for shapes the
 * role-specialised one (qt_rstep.hip) also covers. */
static int rstep_enabled(void) {
    static int on = -1;
    if (on < 0) { const char *e = getenv("QWEN_HIP_RSTEP"); on = !(e && e[0] == '0'); }
    return on;
}

/* Which build of the role-specialised kernel covers the stack: 1 (1.7B int8), 2 (0.6B int8),
 * 3 (0.6B bf16), 4 (1.7B q4_0), 0 none. */
static int rs_kind(const stack_t *s) {
    if (!rstep_enabled()) return 0;
    if (qt_rstep_supported(s->prec, s->H, s->F, s->nh, s->nkv, s->hd, s->kv_max, s->L)) return 1;
    if (qt_rstep06_supported(s->prec, s->H, s->F, s->nh, s->nkv, s->hd, s->kv_max, s->L)) return 2;
    if (qt_rstep06b_supported(s->prec, s->H, s->F, s->nh, s->nkv, s->hd, s->kv_max, s->L)) return 3;
    if (qt_rstep4_supported(s->prec, s->H, s->F, s->nh, s->nkv, s->hd, s->kv_max, s->L)) return 4;
    return 0;
}
static size_t rs_region_words(int rk, int L) {
    return rk == 4 ? qt_rstep4_region_words(L) : rk == 3 ? qt_rstep06b_region_words(L)
         : rk == 2 ? qt_rstep06_region_words(L) : qt_rstep_region_words(L);
}
static size_t rs_slot_words(int rk) {
    return rk == 4 ? qt_rstep4_slot_words() : rk == 3 ? qt_rstep06b_slot_words()
         : rk == 2 ? qt_rstep06_slot_words() : qt_rstep_slot_words();
}

static int persistent_enabled(void) {
    static int on = -1;
    if (on < 0) { const char *e = getenv("QWEN_HIP_PERSISTENT"); on = !(e && e[0] == '0'); }
    return on;
}

static void talker_destroy(talker_t *t) {
    if (!t) return;
    if (t->graph_ready) (void)hipGraphExecDestroy(t->exec);
    if (t->ggraph_ready) (void)hipGraphExecDestroy(t->gexec);
    if (t->pf_qkv) {
        for (int l = 0; l < t->s.L; l++) {
            dmat_free(&t->pf_qkv[l]); dmat_free(&t->pf_o[l]); dmat_free(&t->pf_gu[l]); dmat_free(&t->pf_dn[l]);
        }
        free(t->pf_qkv); free(t->pf_o); free(t->pf_gu); free(t->pf_dn);
    }
    stack_free(&t->s);
    void *bufs[] = {t->io, t->d_pos, t->d_frame, t->d_tok, t->d_hist, t->codec_head, t->codec_emb, t->logits,
                    t->smp_hist, t->smp_seed, t->smp_done, t->gen_codes, t->gen_pad,
                    t->ps_layers, t->ps_ring, t->ps_xin, t->ps_epoch, t->ps_err, t->rs_reg, t->rs_slots,
                    t->pf_x, t->pf_qkvb, t->pf_attn, t->pf_h, t->pf_p, t->pf_part, t->pf_e};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) if (bufs[i]) (void)hipFree(bufs[i]);
    if (t->h_in) (void)hipHostFree(t->h_in);
    if (t->h_out) (void)hipHostFree(t->h_out);
    if (t->h_pos) (void)hipHostFree(t->h_pos);
    if (t->h_err) (void)hipHostFree(t->h_err);
    if (t->st) (void)hipStreamDestroy(t->st);
    free(t);
}

/* Resources of the persistent step: activation ring, layer table, barrier blocks. */
static int ps_setup(talker_t *t) {
    stack_t *s = &t->s;
    void *host_tab = NULL;
    const size_t lb = qt_pstep_layer_bytes();
    const size_t words = qt_pstep_ring_words(s->H, s->F, s->L);
    const unsigned one = 1;   /* ring words start with tag 0: the first step is tag 1 */
    const int rk = rs_kind(s);
    if (rk) {
        /* hand-off words start empty (0xFF bytes: the sentinel), winner words with tag 0;
         * the per-kernel step splits attention into the same key chunks */
        const size_t rw = rs_region_words(rk, s->L), sw = rs_slot_words(rk);
        HCK(hipMalloc((void **)&t->rs_reg, rw * sizeof(unsigned)));
        HCK(hipMalloc((void **)&t->rs_slots, sw * sizeof(unsigned long long)));
        HCK(hipMemsetAsync(t->rs_reg, 0xFF, rw * sizeof(unsigned), t->st));
        HCK(hipMemsetAsync(t->rs_slots, 0, sw * sizeof(unsigned long long), t->st));
        s->step_G = qt_rstep_chunks();
        s->step_onepass = 1;
        t->rs_on = rk;
    }
    HCK(hipMalloc((void **)&t->ps_ring, (t->rs_on ? 1 : words) * sizeof(unsigned long long)));
    HCK(hipMalloc((void **)&t->ps_epoch, 64));
    HCK(hipMalloc((void **)&t->ps_err, 64));
    HCK(hipMalloc((void **)&t->ps_xin, (size_t)s->H * sizeof(float)));
    HCK(hipHostMalloc((void **)&t->h_err, 64, hipHostMallocDefault));
    HCK(hipMemsetAsync(t->ps_ring, 0, (t->rs_on ? 1 : words) * sizeof(unsigned long long), t->st));
    HCK(hipMemsetAsync(t->ps_err, 0, 64, t->st));
    HCK(hipMemcpyAsync(t->ps_epoch, &one, sizeof one, hipMemcpyHostToDevice, t->st));
    host_tab = calloc((size_t)s->L, lb);
    REQ(host_tab, "host alloc");
    for (int l = 0; l < s->L; l++) {
        const uint8_t *w[4] = {s->qkv[l].w, s->o[l].w, s->gu[l].w, s->dn[l].w};
        const float *sc[4] = {s->qkv[l].scale, s->o[l].scale, s->gu[l].scale, s->dn[l].scale};
        const uint16_t *s16[4] = {s->qkv[l].s16, s->o[l].s16, s->gu[l].s16, s->dn[l].s16};
        qt_pstep_fill_layer((char *)host_tab + (size_t)l * lb, w, sc, s16, s->in_norm[l], s->post_norm[l], s->qn[l], s->kn[l]);
    }
    HCK(hipMalloc(&t->ps_layers, (size_t)s->L * lb));
    HCK(hipMemcpy(t->ps_layers, host_tab, (size_t)s->L * lb, hipMemcpyHostToDevice));
    HCK(hipStreamSynchronize(t->st));
    free(host_tab);
    t->ps_on = 1;
    return 0;
fail:
    free(host_tab);
    return -1;
}

/* One launch of the persistent kernel: n_steps decode steps (with_head: greedy loop).
 * layer_out (role-specialised kernel only, may be NULL): every layer's output x of the
 * launch's last step, [L][H]. */
static hipError_t ps_launch_ex(talker_t *t, int n_steps, int with_head, float *layer_out) {
    stack_t *s = &t->s;
    if (t->rs_on)
        return (t->rs_on == 4 ? qt_launch_rstep4 : t->rs_on == 3 ? qt_launch_rstep06b
                : t->rs_on == 2 ? qt_launch_rstep06 : qt_launch_rstep)(t->ps_layers, s->L, s->final_norm, s->rope_cos, s->rope_sin, s->kc, s->vc, s->kv_max, s->eps,
                               1.0f / sqrtf((float)s->hd), t->rs_reg, t->rs_slots, t->io, t->io + s->H, t->ps_xin, t->d_pos,
                               t->ps_epoch, t->ps_err, n_steps, with_head,
                               with_head ? (const uint16_t *)t->head_m.w : NULL, with_head ? t->codec_emb : NULL,
                               t->codec_vocab, t->d_frame, t->d_hist, t->hist_len, layer_out, t->st);
    return qt_launch_pstep(s->prec, s->H, t->ps_layers, s->L, s->final_norm, s->rope_cos, s->rope_sin, s->kc, s->vc,
                           s->kv_max, s->eps, 1.0f / sqrtf((float)s->hd), t->ps_ring, t->io, t->io + s->H, t->ps_xin,
                           t->d_pos, t->ps_epoch, t->ps_err, n_steps, with_head,
                           with_head ? (const uint16_t *)t->head_m.w : NULL, with_head ? t->codec_emb : NULL,
                           t->codec_vocab, t->d_frame, t->d_hist, t->hist_len, t->st);
}
static hipError_t ps_launch(talker_t *t, int n_steps, int with_head) { return ps_launch_ex(t, n_steps, with_head, NULL); }

/* After a synchronous persistent launch: the kernel's own error flag. */
static int ps_check(talker_t *t) {
    if (t->h_err[0] != 0) {
        SETERR("persistent decode step: a wait for another workgroup's data timed out (device error flag set)");
        return -1;
    }
    return 0;
}

/* ---- KV capacity growth (kv_cache_grow, qwen_tts_talker.c:257-280) -------------------------
 * The capacity doubles until it holds `required` positions (at most KV_LIMIT); the cache is
 * copied into the larger one on the device (one strided copy each for K and V: the rows of
 * one (layer, kv head) are contiguous), the attention split follows the new capacity, the
 * captured graphs are dropped (they hold the old cache), and the fused step keeps running:
 * past the role-specialised kernel's capacity the single-role persistent kernel takes over,
 * with the same device position, step tag and next input. */
static int ps_reselect(talker_t *t) {
    stack_t *s = &t->s;
    if (rs_kind(s)) {
        s->step_G = qt_rstep_chunks();
        s->step_onepass = 1;
        return 0;
    }
    /* both fused kernels cover the same shapes, and the single-role one every capacity */
    REQ(persistent_enabled() && qt_pstep_supported(s->prec, s->H, s->F, s->nh, s->nkv, s->hd, s->kv_max),
        "no fused kernel for a cache of %d positions", s->kv_max);
    if (t->rs_on) {
        /* tags carry over: ring words start at tag 0, older than any step's */
        const size_t words = qt_pstep_ring_words(s->H, s->F, s->L);
        (void)hipFree(t->rs_reg); (void)hipFree(t->rs_slots); (void)hipFree(t->ps_ring);
        t->rs_reg = NULL; t->rs_slots = NULL; t->ps_ring = NULL; t->rs_on = 0;
        HCK(hipMalloc((void **)&t->ps_ring, words * sizeof(unsigned long long)));
        HCK(hipMemsetAsync(t->ps_ring, 0, words * sizeof(unsigned long long), t->st));
        HCK(hipStreamSynchronize(t->st));
    }
    return 0;
fail:
    return -1;
}

static int talker_grow_kv(talker_t *t, int required) {
    stack_t *s = &t->s;
    uint16_t *nk = NULL, *nv = NULL;
    float *npart = NULL;
    if (required <= s->kv_max) return 0;
    REQ(required <= KV_LIMIT, "a KV cache of %d positions exceeds %d", required, KV_LIMIT);
    REQ(required <= s->rope_len, "position %d is past the rope table (%d positions)", required - 1, s->rope_len);
    int nm = s->kv_max;
    while (nm < required) nm *= 2;
    if (nm > KV_LIMIT) nm = KV_LIMIT;
    HCK(hipStreamSynchronize(t->st));
    const size_t rows = (size_t)s->L * s->nkv, opitch = (size_t)s->kv_max * s->hd * 2, npitch = (size_t)nm * s->hd * 2;
    HCK(hipMalloc((void **)&nk, rows * npitch));
    HCK(hipMalloc((void **)&nv, rows * npitch));
    HCK(hipMemsetAsync(nk, 0, rows * npitch, t->st));
    HCK(hipMemsetAsync(nv, 0, rows * npitch, t->st));
    HCK(hipMemcpy2DAsync(nk, npitch, s->kc, opitch, opitch, rows, hipMemcpyDeviceToDevice, t->st));
    HCK(hipMemcpy2DAsync(nv, npitch, s->vc, opitch, opitch, rows, hipMemcpyDeviceToDevice, t->st));
    const int G = nm <= 128 ? 1 : qt_attn_grid(nm);
    if (G != s->attn_G)
        HCK(hipMalloc((void **)&npart, (size_t)s->nkv * G * (s->nh / s->nkv) * 130 * sizeof(float)));
    HCK(hipStreamSynchronize(t->st));
    (void)hipFree(s->kc); (void)hipFree(s->vc);
    s->kc = nk; s->vc = nv; nk = nv = NULL;
    if (npart) { (void)hipFree(s->part); s->part = npart; npart = NULL; }
    s->kv_max = nm; s->attn_G = G; s->step_G = G; s->step_onepass = 0;
    if (s->kv_stage) { (void)hipFree(s->kv_stage); s->kv_stage = NULL; }
    if (t->graph_ready) { (void)hipGraphExecDestroy(t->exec); t->graph_ready = 0; }
    if (t->ggraph_ready) { (void)hipGraphExecDestroy(t->gexec); t->ggraph_ready = 0; }
    if (t->ps_on && ps_reselect(t) != 0) { t->dead = 1; return -1; }
    return 0;
fail:
    if (nk) (void)hipFree(nk);
    if (nv) (void)hipFree(nv);
    if (npart) (void)hipFree(npart);
    return -1;
}

int qwen_hip_talker_grow_kv(void *state, int required) {
    talker_t *t = (talker_t *)state;
    if (!t || t->dead) { SETERR("talker state is dead or NULL"); return -1; }
    return talker_grow_kv(t, required);
}
int qwen_hip_talker_kv_max(void *state) { return state ? ((talker_t *)state)->s.kv_max : -1; }

void *qwen_hip_talker_init(const qwen_hip_talker_desc_t *desc) {
    talker_t *t = calloc(1, sizeof *t);
    if (!t) { SETERR("out of host memory"); return NULL; }
    HCK(hipStreamCreateWithFlags(&t->st, hipStreamNonBlocking));
    if (stack_init(&t->s, desc, t->st) != 0) goto fail;   /* g_err already set */
    /* the KV hand-off's pinned pipe and device staging, so that upload_kv only copies */
    HCK(hpipe_init(&t->s.up, t->st));
    HCK(hipMalloc((void **)&t->s.kv_stage, (size_t)t->s.kv_max * t->s.kvd * sizeof(uint16_t)));
    /* one small copy and relayout now: the runtime's first-use costs of both (2.7 ms on the
     * MI355X box) belong to init, not to the first hand-off */
    HCK(hipMemcpyAsync(t->s.kv_stage, t->s.up.pin[0], 4096, hipMemcpyHostToDevice, t->st));
    HCK(qt_launch_kv_relayout(t->s.kc, t->s.kv_stage, 1, t->s.nkv, t->s.hd, t->s.kv_max, 0, t->st));
    HCK(hipStreamSynchronize(t->st));
    const int H = t->s.H;
    t->hist_len = 4096;
    HCK(hipMalloc((void **)&t->io, (size_t)2 * H * sizeof(float)));
    HCK(hipMalloc((void **)&t->d_pos, sizeof(int)));
    HCK(hipMalloc((void **)&t->d_frame, sizeof(int)));
    HCK(hipMalloc((void **)&t->d_tok, sizeof(int)));
    HCK(hipMalloc((void **)&t->d_hist, (size_t)t->hist_len * sizeof(int)));
    HCK(hipMalloc((void **)&t->smp_hist, (size_t)QT_SAMPLE_HIST_MAX * sizeof(int)));
    HCK(hipMalloc((void **)&t->smp_seed, 64));
    HCK(hipMalloc((void **)&t->smp_done, 64));
    HCK(hipMalloc((void **)&t->gen_codes, (size_t)QT_SAMPLE_HIST_MAX * 16 * sizeof(int)));
    HCK(hipMalloc((void **)&t->gen_pad, (size_t)H * sizeof(float)));
    HCK(hipHostMalloc((void **)&t->h_in, (size_t)H * sizeof(float), hipHostMallocDefault));
    HCK(hipHostMalloc((void **)&t->h_out, (size_t)2 * H * sizeof(float), hipHostMallocDefault));
    HCK(hipHostMalloc((void **)&t->h_pos, 4 * sizeof(int), hipHostMallocDefault));
    HCK(hipMemsetAsync(t->io, 0, (size_t)2 * H * sizeof(float), t->st));
    HCK(hipStreamSynchronize(t->st));
    t->dev_pos = -1;
    if (persistent_enabled() && qt_pstep_supported(t->s.prec, H, t->s.F, t->s.nh, t->s.nkv, t->s.hd, t->s.kv_max)) {
        if (ps_setup(t) != 0) goto fail;
    }
    return t;
fail:
    talker_destroy(t);
    return NULL;
}

void qwen_hip_talker_free(void *state) { talker_destroy((talker_t *)state); }
void *qwen_hip_talker_stream(void *state) { return state ? (void *)((talker_t *)state)->st : NULL; }
int qwen_hip_talker_fused(void *state) { return state ? ((talker_t *)state)->ps_on : -1; }
int qwen_hip_talker_fused_kernel(void *state) {
    if (!state) return -1;
    const talker_t *t = (const talker_t *)state;
    return t->ps_on ? (t->rs_on ? 2 : 1) : 0;
}

static hipError_t talker_body(talker_t *t) {
    hipError_t e;
    float *x = t->io + t->s.H;
    if ((e = stack_body(&t->s, x, t->d_pos, t->st))) return e;
    /* final norm into io[0:H); advances *d_pos for the next step */
    return qt_launch_rmsnorm(x, t->s.final_norm, t->io, t->s.H, t->s.eps, t->d_pos, t->st);
}

static int capture(hipStream_t st, hipGraphExec_t *exec, hipError_t (*body)(void *), void *arg) {
    hipGraph_t g = NULL;
    hipError_t be;
    HCK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    be = body(arg);
    {
        hipError_t ee = hipStreamEndCapture(st, &g);
        if (be != hipSuccess || ee != hipSuccess) {
            SETERR("graph capture failed: %s / %s", hipGetErrorString(be), hipGetErrorString(ee));
            if (g) (void)hipGraphDestroy(g);
            return -1;
        }
    }
    HCK(hipGraphInstantiate(exec, g, NULL, NULL, 0));
    (void)hipGraphDestroy(g);
    return 0;
fail:
    if (g) (void)hipGraphDestroy(g);
    return -1;
}

static hipError_t talker_body_cb(void *a) { return talker_body((talker_t *)a); }

/* QWEN_HIP_GRAPH=0 replays the same launch sequence directly on the stream instead of
 * through a captured hipGraph (profilers that cannot trace graph replays; A/B checks). */
static int graphs_enabled(void) {
    static int on = -1;
    if (on < 0) { const char *e = getenv("QWEN_HIP_GRAPH"); on = !(e && e[0] == '0'); }
    return on;
}

static int talker_set_pos(talker_t *t, int pos) {
    if (t->dev_pos == pos) return 0;
    t->h_pos[0] = pos;
    HCK(hipMemcpyAsync(t->d_pos, t->h_pos, sizeof(int), hipMemcpyHostToDevice, t->st));
    /* h_pos is reused: make sure the copy has consumed it before the host changes it */
    HCK(hipStreamSynchronize(t->st));
    t->dev_pos = pos;
    return 0;
fail:
    return -1;
}

static int talker_step_impl(talker_t *t, const float *embed, float *hidden_out, int pos, int use_graph) {
    if (!t || t->dead) { SETERR("talker state is dead or NULL"); return -1; }
    const int H = t->s.H;
    if (pos >= 0 && talker_grow_kv(t, pos + 1) != 0) return -1;   /* qwen_talker_step grows first (t.c:574) */
    REQ(pos >= 0 && pos < t->s.kv_max && pos < t->s.rope_len, "pos %d out of range (kv_max %d, rope %d)",
        pos, t->s.kv_max, t->s.rope_len);
    if (talker_set_pos(t, pos) != 0) goto fail;
    memcpy(t->h_in, embed, (size_t)H * sizeof(float));
    if (use_graph && t->ps_on) {
        HCK(hipMemcpyAsync(t->ps_xin, t->h_in, (size_t)H * sizeof(float), hipMemcpyHostToDevice, t->st));
        HCK(ps_launch(t, 1, 0));
        HCK(hipMemcpyAsync(t->h_out, t->io, (size_t)2 * H * sizeof(float), hipMemcpyDeviceToHost, t->st));
        HCK(hipMemcpyAsync(t->h_err, t->ps_err, sizeof(int), hipMemcpyDeviceToHost, t->st));
        HCK(hipStreamSynchronize(t->st));
        if (ps_check(t) != 0) goto fail;
        t->dev_pos = pos + 1;
        if (hidden_out) memcpy(hidden_out, t->h_out, (size_t)H * sizeof(float));
        return 0;
    }
    HCK(hipMemcpyAsync(t->io + H, t->h_in, (size_t)H * sizeof(float), hipMemcpyHostToDevice, t->st));
    if (use_graph && graphs_enabled()) {
        if (!t->graph_ready) {
            if (capture(t->st, &t->exec, talker_body_cb, t) != 0) goto fail;
            t->graph_ready = 1;
        }
        HCK(hipGraphLaunch(t->exec, t->st));
    } else {
        HCK(talker_body(t));
    }
    HCK(hipMemcpyAsync(t->h_out, t->io, (size_t)2 * H * sizeof(float), hipMemcpyDeviceToHost, t->st));
    HCK(hipStreamSynchronize(t->st));
    t->dev_pos = pos + 1;
    if (hidden_out) memcpy(hidden_out, t->h_out, (size_t)H * sizeof(float));
    return 0;
fail:
    if (t) { t->dead = 1; t->dev_pos = -1; }
    return -1;
}

int qwen_hip_talker_step(void *state, const float *embed, float *hidden_out, int pos) {
    return talker_step_impl((talker_t *)state, embed, hidden_out, pos, 1);
}
int qwen_hip_talker_step_nograph(void *state, const float *embed, float *hidden_out, int pos) {
    return talker_step_impl((talker_t *)state, embed, hidden_out, pos, 0);
}

void qwen_hip_talker_get_dec_x(void *state, float *out) {
    talker_t *t = (talker_t *)state;
    if (t && out) memcpy(out, t->h_out + t->s.H, (size_t)t->s.H * sizeof(float));
}

/* One step that also returns the residual after every layer (residuals[L][H]): the
 * device twin of the per-layer check the reference tests use (running the step with
 * num_layers truncated, qwen_tts_talker.c:659-665).  On the fused path the values are the
 * persistent kernel's own: its activation ring keeps every layer's output x (phase E,
 * tagged with the step number) until the slot is reused two steps later, so they are read
 * back after the launch and their tags are checked.  On the per-kernel path x is copied
 * after each layer of an ungraphed step.  Allocates a temporary device buffer (a
 * diagnostic, not a hot-path call). */
int qwen_hip_talker_step_layers(void *state, const float *embed, float *residuals, float *hidden_out, int pos) {
    talker_t *t = (talker_t *)state;
    void *tmp = NULL;
    unsigned long long *words = NULL;
    if (!t || t->dead) { SETERR("talker state is dead or NULL"); return -1; }
    if (!embed || !residuals) { SETERR("null argument"); return -1; }
    stack_t *s = &t->s;
    const int H = s->H, L = s->L;
    if (pos >= 0 && talker_grow_kv(t, pos + 1) != 0) return -1;
    if (pos < 0 || pos >= s->kv_max || pos >= s->rope_len) { SETERR("pos %d out of range", pos); return -1; }
    if (talker_set_pos(t, pos) != 0) goto fail;
    memcpy(t->h_in, embed, (size_t)H * sizeof(float));
    if (t->ps_on && t->rs_on) {
        HCK(hipMalloc(&tmp, (size_t)L * H * sizeof(float)));
        HCK(hipMemcpyAsync(t->ps_xin, t->h_in, (size_t)H * sizeof(float), hipMemcpyHostToDevice, t->st));
        HCK(ps_launch_ex(t, 1, 0, (float *)tmp));
        HCK(hipMemcpyAsync(t->h_out, t->io, (size_t)2 * H * sizeof(float), hipMemcpyDeviceToHost, t->st));
        HCK(hipMemcpyAsync(t->h_err, t->ps_err, sizeof(int), hipMemcpyDeviceToHost, t->st));
        HCK(hipMemcpyAsync(residuals, tmp, (size_t)L * H * sizeof(float), hipMemcpyDeviceToHost, t->st));
        HCK(hipStreamSynchronize(t->st));
        (void)hipFree(tmp);
        tmp = NULL;
        if (ps_check(t) != 0) goto fail;
        t->dev_pos = pos + 1;
    } else if (t->ps_on) {
        unsigned tag = 0;
        HCK(hipMemcpyAsync(t->ps_xin, t->h_in, (size_t)H * sizeof(float), hipMemcpyHostToDevice, t->st));
        HCK(ps_launch(t, 1, 0));
        HCK(hipMemcpyAsync(t->h_out, t->io, (size_t)2 * H * sizeof(float), hipMemcpyDeviceToHost, t->st));
        HCK(hipMemcpyAsync(t->h_err, t->ps_err, sizeof(int), hipMemcpyDeviceToHost, t->st));
        HCK(hipMemcpyAsync(&tag, t->ps_epoch, sizeof tag, hipMemcpyDeviceToHost, t->st));
        HCK(hipStreamSynchronize(t->st));
        if (ps_check(t) != 0) goto fail;
        t->dev_pos = pos + 1;
        words = (unsigned long long *)malloc((size_t)H * sizeof *words);
        REQ(words, "host alloc");
        for (int l = 0; l < L; l++) {
            const size_t off = qt_pstep_ring_x_offset(H, s->F, L, 0, l);   /* a 1-step launch runs at parity 0 */
            HCK(hipMemcpy(words, t->ps_ring + off, (size_t)H * sizeof *words, hipMemcpyDeviceToHost));
            for (int i = 0; i < H; i++) {
                REQ((unsigned)(words[i] >> 32) == tag - 1u, "ring word of layer %d carries tag %u, expected %u", l,
                    (unsigned)(words[i] >> 32), tag - 1u);
                const unsigned bits = (unsigned)words[i];
                memcpy(residuals + (size_t)l * H + i, &bits, sizeof bits);
            }
        }
        free(words);
    } else {
        HCK(hipMalloc(&tmp, (size_t)L * H * sizeof(float)));
        HCK(hipMemcpyAsync(t->io + H, t->h_in, (size_t)H * sizeof(float), hipMemcpyHostToDevice, t->st));
        HCK(stack_body_ex(s, t->io + H, t->d_pos, t->st, (float *)tmp));
        HCK(qt_launch_rmsnorm(t->io + H, s->final_norm, t->io, H, s->eps, t->d_pos, t->st));
        HCK(hipMemcpyAsync(t->h_out, t->io, (size_t)2 * H * sizeof(float), hipMemcpyDeviceToHost, t->st));
        HCK(hipMemcpyAsync(residuals, tmp, (size_t)L * H * sizeof(float), hipMemcpyDeviceToHost, t->st));
        HCK(hipStreamSynchronize(t->st));
        (void)hipFree(tmp);
        t->dev_pos = pos + 1;
    }
    if (hidden_out) memcpy(hidden_out, t->h_out, (size_t)H * sizeof(float));
    return 0;
fail:
    free(words);
    if (tmp) (void)hipFree(tmp);
    t->dead = 1; t->dev_pos = -1;
    return -1;
}

int qwen_hip_talker_upload_kv(void *state, const uint16_t *kv_k, const uint16_t *kv_v, int host_kv_max,
                              int prefill_len) {
    talker_t *t = (talker_t *)state;
    if (!t || t->dead) { SETERR("talker state is dead or NULL"); return -1; }
    stack_t *s = &t->s;
    if (prefill_len <= 0) return 0;
    if (prefill_len <= host_kv_max && talker_grow_kv(t, prefill_len) != 0) return -1;
    REQ(prefill_len <= s->kv_max && prefill_len <= host_kv_max, "prefill_len %d exceeds kv_max", prefill_len);
    REQ(kv_k && kv_v, "null KV");
    if (!s->kv_stage) HCK(hipMalloc((void **)&s->kv_stage, (size_t)s->kv_max * s->kvd * sizeof(uint16_t)));
    for (int l = 0; l < s->L; l++) {
        const size_t lay = (size_t)l * s->nkv * s->kv_max * s->hd, src = (size_t)l * host_kv_max * s->kvd;
        HCK(kv_xfer(s->kc + lay, s->kv_max, (uint16_t *)kv_k + src, prefill_len, s->nkv, s->hd, 1, s->kv_stage, &s->up, t->st));
        HCK(kv_xfer(s->vc + lay, s->kv_max, (uint16_t *)kv_v + src, prefill_len, s->nkv, s->hd, 1, s->kv_stage, &s->up, t->st));
    }
    HCK(hipStreamSynchronize(t->st));
    return 0;
fail:
    return -1;
}

/* positions [0, n) of a stack's cache into the host layout [L][host_kv_max][n_kv * hd] */
static int stack_download_kv(stack_t *s, hipStream_t st, uint16_t *kv_k, uint16_t *kv_v, int host_kv_max, int n) {
    REQ(n >= 0 && n <= s->kv_max && n <= host_kv_max, "n %d out of range", n);
    if (n == 0) return 0;
    REQ(kv_k && kv_v, "null KV");
    if (!s->kv_stage) HCK(hipMalloc((void **)&s->kv_stage, (size_t)s->kv_max * s->kvd * sizeof(uint16_t)));
    for (int l = 0; l < s->L; l++) {
        const size_t lay = (size_t)l * s->nkv * s->kv_max * s->hd, dst = (size_t)l * host_kv_max * s->kvd;
        HCK(kv_xfer(s->kc + lay, s->kv_max, kv_k + dst, n, s->nkv, s->hd, 0, s->kv_stage, NULL, st));
        HCK(kv_xfer(s->vc + lay, s->kv_max, kv_v + dst, n, s->nkv, s->hd, 0, s->kv_stage, NULL, st));
    }
    HCK(hipStreamSynchronize(st));
    return 0;
fail:
    return -1;
}

int qwen_hip_talker_download_kv(void *state, uint16_t *kv_k, uint16_t *kv_v, int host_kv_max, int n) {
    talker_t *t = (talker_t *)state;
    if (!t) { SETERR("NULL state"); return -1; }
    return stack_download_kv(&t->s, t->st, kv_k, kv_v, host_kv_max, n);
}

/* -- Talker prefill (qwen_talker_prefill, qwen_tts_talker.c:730-1038) ------------------ */

/* The prefill's layer loop (qwen_tts_talker.c:780-1030) over pf_x (seq residual rows):
 * planes of the normed input -> q|k|v GEMM, whose reduce does the per-head norm, RoPE and
 * KV store -> causal
 * attention, written as the O projection's planes -> O GEMM + residual, whose reduce also
 * writes the planes of the post-attention-normed residual -> gate|up GEMM + SwiGLU, written
 * as the down projection's planes -> down GEMM + residual, whose reduce writes the next
 * layer's input planes.  The fused reduces need the split-K workspace to hold all the
 * partials (seq x 2F for SwiGLU, seq x H for the residuals); beyond that the f32 rows and
 * a separate plane kernel. */
static hipError_t pf_layers(talker_t *t, const dmat_t *wq, const dmat_t *wo, const dmat_t *wgu, const dmat_t *wdn,
                            int seq) {
    stack_t *s = &t->s;
    const int L = s->L, H = s->H, F = s->F, qd = s->qd, qkvr = s->qd + 2 * s->kvd;
    const float scale = 1.0f / sqrtf((float)s->hd);
    const int h_planes = (long long)seq * 2 * F <= PF_PART_FLOATS;
    const int x_planes = (long long)seq * H <= PF_PART_FLOATS;
    hipError_t e;
#define PFE(x) do { if ((e = (x)) != hipSuccess) return e; } while (0)
    for (int l = 0; l < L; l++) {
        const size_t lay = (size_t)l * s->nkv * s->kv_max * s->hd;
        /* layer 0's input planes; later layers get them from the previous down projection */
        if (l == 0 || !x_planes) PFE(qt_launch_pf_pieces(t->pf_x, H, seq, H, s->in_norm[l], s->eps, t->pf_p, t->st));
        if ((long long)seq * qkvr <= PF_PART_FLOATS) {
            PFE(qt_launch_pf_gemm_qkv_post((const uint16_t *)wq[l].w, t->pf_p, seq, qkvr, H, t->pf_qkvb, qkvr, s->nh, s->nkv,
                                           s->qn[l], s->kn[l], s->rope_cos, s->rope_sin, s->eps, s->kc + lay,
                                           s->vc + lay, s->kv_max, t->pf_part, PF_PART_FLOATS, t->st));
        } else {
            PFE(qt_launch_pf_gemm(QT_PF_STORE, (const uint16_t *)wq[l].w, t->pf_p, seq, qkvr, H, t->pf_qkvb, qkvr, t->pf_part, PF_PART_FLOATS, t->st));
            PFE(qt_launch_pf_qkv_post(t->pf_qkvb, qkvr, seq, s->nh, s->nkv, s->qn[l], s->kn[l], s->rope_cos, s->rope_sin,
                                      s->eps, s->kc + lay, s->vc + lay, s->kv_max, t->st));
        }
        int att_planes = 0;
        PFE(qt_launch_pf_attn_planes(t->pf_qkvb, qkvr, seq, s->nh, s->nkv, scale, t->pf_attn, qd, t->pf_p, &att_planes,
                                     t->st));
        if (!att_planes) PFE(qt_launch_pf_pieces(t->pf_attn, qd, seq, qd, NULL, 0.f, t->pf_p, t->st));
        if (x_planes) {
            PFE(qt_launch_pf_gemm_resid_planes((const uint16_t *)wo[l].w, t->pf_p, seq, H, qd, t->pf_x, H, s->post_norm[l],
                                               s->eps, t->pf_p, t->pf_part, PF_PART_FLOATS, t->st));
        } else {
            PFE(qt_launch_pf_gemm(QT_PF_RESID, (const uint16_t *)wo[l].w, t->pf_p, seq, H, qd, t->pf_x, H, t->pf_part, PF_PART_FLOATS, t->st));
            PFE(qt_launch_pf_pieces(t->pf_x, H, seq, H, s->post_norm[l], s->eps, t->pf_p, t->st));
        }
        if (h_planes) {
            PFE(qt_launch_pf_gemm_swiglu_planes((const uint16_t *)wgu[l].w, t->pf_p, seq, 2 * F, H, t->pf_p, t->pf_part,
                                                PF_PART_FLOATS, t->st));
        } else {
            PFE(qt_launch_pf_gemm(QT_PF_SWIGLU, (const uint16_t *)wgu[l].w, t->pf_p, seq, 2 * F, H, t->pf_h, F, t->pf_part, PF_PART_FLOATS, t->st));
            PFE(qt_launch_pf_pieces(t->pf_h, F, seq, F, NULL, 0.f, t->pf_p, t->st));
        }
        if (x_planes && l + 1 < L)
            PFE(qt_launch_pf_gemm_resid_planes((const uint16_t *)wdn[l].w, t->pf_p, seq, H, F, t->pf_x, H, s->in_norm[l + 1],
                                               s->eps, t->pf_p, t->pf_part, PF_PART_FLOATS, t->st));
        else
            PFE(qt_launch_pf_gemm(QT_PF_RESID, (const uint16_t *)wdn[l].w, t->pf_p, seq, H, F, t->pf_x, H, t->pf_part, PF_PART_FLOATS, t->st));
    }
#undef PFE
    return hipSuccess;
}

/* bf16 copies of the projection weights for the prefill (the reference's prefill reads
 * the bf16 layer weights whatever the decode precision, t.c:832-839). */
static int pf_weights(talker_t *t, const qwen_hip_layer_t *ly) {
    stack_t *s = &t->s;
    const int L = s->L, H = s->H, F = s->F, qd = s->qd, kvd = s->kvd;
    void *tmp = NULL;
    size_t tb = (size_t)2 * F * H * 2;
    if ((size_t)(qd + 2 * kvd) * H * 2 > tb) tb = (size_t)(qd + 2 * kvd) * H * 2;
    t->pf_qkv = calloc(L, sizeof(dmat_t)); t->pf_o = calloc(L, sizeof(dmat_t));
    t->pf_gu = calloc(L, sizeof(dmat_t)); t->pf_dn = calloc(L, sizeof(dmat_t));
    REQ(t->pf_qkv && t->pf_o && t->pf_gu && t->pf_dn, "host alloc failed");
    HCK(hipMalloc(&tmp, tb));
    for (int l = 0; l < L; l++) {
        REQ(dmat_alloc(&t->pf_qkv[l], QWEN_HIP_BF16, qd + 2 * kvd, H) == 0, "alloc prefill qkv");
        REQ(dmat_put(&t->pf_qkv[l], 0, &ly[l].q, QWEN_HIP_BF16, qd, t->st, tmp) == 0, "upload q %d", l);
        REQ(dmat_put(&t->pf_qkv[l], qd, &ly[l].k, QWEN_HIP_BF16, kvd, t->st, tmp) == 0, "upload k %d", l);
        REQ(dmat_put(&t->pf_qkv[l], qd + kvd, &ly[l].v, QWEN_HIP_BF16, kvd, t->st, tmp) == 0, "upload v %d", l);
        REQ(dmat_alloc(&t->pf_o[l], QWEN_HIP_BF16, H, qd) == 0, "alloc prefill o");
        REQ(dmat_put(&t->pf_o[l], 0, &ly[l].o, QWEN_HIP_BF16, H, t->st, tmp) == 0, "upload o %d", l);
        REQ(dmat_alloc(&t->pf_gu[l], QWEN_HIP_BF16, 2 * F, H) == 0, "alloc prefill gate_up");
        REQ(dmat_put(&t->pf_gu[l], 0, &ly[l].gate_up, QWEN_HIP_BF16, 2 * F, t->st, tmp) == 0, "upload gate_up %d", l);
        REQ(dmat_alloc(&t->pf_dn[l], QWEN_HIP_BF16, H, F) == 0, "alloc prefill down");
        REQ(dmat_put(&t->pf_dn[l], 0, &ly[l].down, QWEN_HIP_BF16, H, t->st, tmp) == 0, "upload down %d", l);
    }
    (void)hipFree(tmp);
    return 0;
fail:
    if (tmp) (void)hipFree(tmp);
    return -1;
}

static void pf_free_bufs(talker_t *t) {
    void *b[] = {t->pf_x, t->pf_qkvb, t->pf_attn, t->pf_h, t->pf_p, t->pf_part, t->pf_e};
    for (size_t i = 0; i < sizeof b / sizeof b[0]; i++) if (b[i]) (void)hipFree(b[i]);
    t->pf_x = t->pf_qkvb = t->pf_attn = t->pf_h = t->pf_part = t->pf_e = NULL; t->pf_p = NULL; t->pf_cap = 0;
}

int qwen_hip_talker_prefill(void *state, const qwen_hip_layer_t *bf16_layers, const float *embeds, int seq) {
    talker_t *t = (talker_t *)state;
    if (!t || t->dead) { SETERR("talker state is dead or NULL"); return -1; }
    stack_t *s = &t->s;
    const int H = s->H, F = s->F, qd = s->qd, qkvr = s->qd + 2 * s->kvd;
    /* argument errors leave the state usable */
    if (!embeds) { SETERR("null embeds"); return -1; }
    if (seq >= 1 && seq <= s->rope_len && talker_grow_kv(t, seq) != 0) return -1;   /* t.c:773 */
    if (seq < 1 || seq > s->kv_max || seq > s->rope_len) {
        SETERR("seq %d out of range (1..%d)", seq, s->kv_max < s->rope_len ? s->kv_max : s->rope_len);
        return -1;
    }
    if (H % 64 || F % 64 || qkvr % 64 || qd % 64) { SETERR("prefill needs hidden, inter, q|k|v rows, q dim divisible by 64"); return -1; }
    const dmat_t *wq = s->qkv, *wo = s->o, *wgu = s->gu, *wdn = s->dn;
    if (s->prec != QWEN_HIP_BF16) {
        if (!t->pf_qkv) {
            if (!bf16_layers) { SETERR("prefill of a non-bf16 state needs the bf16 layer weights"); return -1; }
            if (pf_weights(t, bf16_layers) != 0) goto fail;
        }
        wq = t->pf_qkv; wo = t->pf_o; wgu = t->pf_gu; wdn = t->pf_dn;
    }
    if (seq > t->pf_cap) {
        pf_free_bufs(t);
        const int sp = qt_pf_spad(seq);
        int km = H > qd ? H : qd;
        if (F > km) km = F;
        HCK(hipMalloc((void **)&t->pf_x, (size_t)seq * H * sizeof(float)));
        HCK(hipMalloc((void **)&t->pf_qkvb, (size_t)seq * qkvr * sizeof(float)));
        HCK(hipMalloc((void **)&t->pf_attn, (size_t)seq * qd * sizeof(float)));
        HCK(hipMalloc((void **)&t->pf_h, (size_t)seq * F * sizeof(float)));
        HCK(hipMalloc((void **)&t->pf_p, (size_t)3 * sp * km * sizeof(uint16_t)));
        HCK(hipMalloc((void **)&t->pf_part, (size_t)PF_PART_FLOATS * sizeof(float)));
        HCK(hipMalloc((void **)&t->pf_e, (size_t)seq * H * sizeof(float)));
        t->pf_cap = seq;
    }
    HCK(hipMemcpyAsync(t->pf_e, embeds, (size_t)seq * H * sizeof(float), hipMemcpyDefault, t->st));
    HCK(hipMemcpyAsync(t->pf_x, t->pf_e, (size_t)seq * H * sizeof(float), hipMemcpyDeviceToDevice, t->st));
    HCK(pf_layers(t, wq, wo, wgu, wdn, seq));
    /* dec_x = the last position's residual (t.c:1032-1033), where get_dec_x reads it */
    HCK(hipMemcpyAsync(t->io + H, t->pf_x + (size_t)(seq - 1) * H, (size_t)H * sizeof(float), hipMemcpyDeviceToDevice, t->st));
    HCK(hipMemcpyAsync(t->h_out + H, t->io + H, (size_t)H * sizeof(float), hipMemcpyDeviceToHost, t->st));
    HCK(hipStreamSynchronize(t->st));
    return 0;
fail:
    t->dead = 1;
    return -1;
}

/* Benchmark entry: enqueue n prefills of the last prefill's embeddings (kept on the
 * device) without host synchronisation; each one rewrites the cache rows and dec_x
 * exactly as that prefill did. */
int qwen_hip_talker_prefill_async(void *state, int seq, int n) {
    talker_t *t = (talker_t *)state;
    if (!t || t->dead) { SETERR("talker state is dead or NULL"); return -1; }
    stack_t *s = &t->s;
    const int H = s->H;
    if (seq < 1 || seq > t->pf_cap || n < 0) { SETERR("call qwen_hip_talker_prefill with at least seq positions first"); return -1; }
    const dmat_t *wq = s->prec == QWEN_HIP_BF16 ? s->qkv : t->pf_qkv, *wo = s->prec == QWEN_HIP_BF16 ? s->o : t->pf_o;
    const dmat_t *wgu = s->prec == QWEN_HIP_BF16 ? s->gu : t->pf_gu, *wdn = s->prec == QWEN_HIP_BF16 ? s->dn : t->pf_dn;
    if (!wq) { SETERR("no prefill weights"); return -1; }
    if (!t->pf_e) { SETERR("no prefill inputs"); return -1; }
    for (int it = 0; it < n; it++) {
        HCK(hipMemcpyAsync(t->pf_x, t->pf_e, (size_t)seq * H * sizeof(float), hipMemcpyDeviceToDevice, t->st));
        HCK(pf_layers(t, wq, wo, wgu, wdn, seq));
        HCK(hipMemcpyAsync(t->io + H, t->pf_x + (size_t)(seq - 1) * H, (size_t)H * sizeof(float), hipMemcpyDeviceToDevice,
                           t->st));
    }
    return 0;
fail:
    t->dead = 1;
    return -1;
}

/* -- resident greedy loop: step -> codec head -> greedy code0 -> next embed ---------- */

static hipError_t greedy_body(void *a) {
    talker_t *t = (talker_t *)a;
    hipError_t e;
    const int H = t->s.H;
    float *x = t->io + H;
    if ((e = stack_body(&t->s, x, t->d_pos, t->st))) return e;
    /* final norm fused into the codec head: the head matvec normalises x with
     * talker_norm and also writes the normed hidden to io[0:H) */
    if ((e = qt_launch_mv(t->head_m.prec, QT_EPI_STORE, 1, x, t->s.final_norm, t->s.eps, t->head_m.w, NULL, NULL,
                          t->head_m.rows, t->head_m.cols, t->logits, NULL, NULL, t->io, t->st))) return e;
    /* greedy code0, next embedding into x, frame and position advance */
    return qt_launch_select(t->logits, t->codec_vocab, 1, t->d_frame, 1, t->d_tok, t->d_hist, t->hist_len,
                            t->codec_emb, H, x, t->d_pos, t->st);
}

/* codec head (bf16) and embedding table on the device, re-uploaded when the caller's
 * arrays change */
static int head_setup(talker_t *t, const uint16_t *codec_head, const uint16_t *codec_emb, int codec_vocab) {
    const int H = t->s.H;
    if (t->head_host != codec_head || t->emb_host != codec_emb || t->codec_vocab != codec_vocab) {
        if (t->ggraph_ready) { (void)hipGraphExecDestroy(t->gexec); t->ggraph_ready = 0; }
        t->greedy_ready = 0;
        dmat_free(&t->head_m);
        if (t->codec_emb) (void)hipFree(t->codec_emb);
        if (t->logits) (void)hipFree(t->logits);
        t->codec_emb = NULL; t->logits = NULL;
        qwen_hip_mat_t hm = {codec_head, NULL};
        REQ(dmat_alloc(&t->head_m, QWEN_HIP_BF16, codec_vocab, H) == 0, "alloc codec head");
        REQ(dmat_put(&t->head_m, 0, &hm, QWEN_HIP_BF16, codec_vocab, t->st, NULL) == 0, "upload codec head");
        HCK(hipMalloc((void **)&t->codec_emb, (size_t)codec_vocab * H * 2));
        HCK(hipMemcpy(t->codec_emb, codec_emb, (size_t)codec_vocab * H * 2, hipMemcpyDefault));
        HCK(hipMalloc((void **)&t->logits, (size_t)codec_vocab * sizeof(float)));
        t->head_host = codec_head; t->emb_host = codec_emb; t->codec_vocab = codec_vocab;
    }
    return 0;
fail:
    return -1;
}

int qwen_hip_talker_greedy(void *state, const uint16_t *codec_head, const uint16_t *codec_emb, int codec_vocab,
                           const float *embed, int pos, int frame0, int n_steps, int *tokens_out,
                           float *hidden_out) {
    talker_t *t = (talker_t *)state;
    if (!t || t->dead) { SETERR("talker state is dead or NULL"); return -1; }
    const int H = t->s.H;
    REQ(codec_head && codec_emb && codec_vocab > 0, "missing codec head/embedding");
    REQ(n_steps >= 0 && n_steps <= t->hist_len, "n_steps %d out of range", n_steps);
    REQ(frame0 >= 0, "frame0 %d must be >= 0", frame0);
    REQ(tokens_out || n_steps == 0, "null tokens_out");
    if (pos >= 0 && talker_grow_kv(t, pos + n_steps) != 0) return -1;
    REQ(pos >= 0 && pos + n_steps <= t->s.kv_max && pos + n_steps <= t->s.rope_len, "positions exceed kv_max");
    if (head_setup(t, codec_head, codec_emb, codec_vocab) != 0) goto fail;
    if (talker_set_pos(t, pos) != 0) goto fail;
    t->h_pos[1] = frame0;
    HCK(hipMemcpyAsync(t->d_frame, t->h_pos + 1, sizeof(int), hipMemcpyHostToDevice, t->st));
    memcpy(t->h_in, embed, (size_t)H * sizeof(float));
    if (t->ps_on && codec_vocab == 3072) {
        HCK(hipMemcpyAsync(t->ps_xin, t->h_in, (size_t)H * sizeof(float), hipMemcpyHostToDevice, t->st));
        t->greedy_ready = 2;
        if (n_steps > 0) HCK(ps_launch(t, n_steps, 1));
    } else {
    HCK(hipMemcpyAsync(t->io + H, t->h_in, (size_t)H * sizeof(float), hipMemcpyHostToDevice, t->st));
    if (graphs_enabled() && !t->ggraph_ready) {
        if (capture(t->st, &t->gexec, greedy_body, t) != 0) goto fail;
        t->ggraph_ready = 1;
    }
    t->greedy_ready = 1;
    for (int i = 0; i < n_steps; i++) HCK(graphs_enabled() ? hipGraphLaunch(t->gexec, t->st) : greedy_body(t));
    }
    {
        int *hist = (int *)malloc((size_t)t->hist_len * sizeof(int));
        REQ(hist, "host alloc");
        hipError_t e1 = hipMemcpyAsync(hist, t->d_hist, (size_t)t->hist_len * sizeof(int), hipMemcpyDeviceToHost, t->st);
        hipError_t e2 = hipMemcpyAsync(t->h_out, t->io, (size_t)2 * H * sizeof(float), hipMemcpyDeviceToHost, t->st);
        hipError_t e4 = t->ps_on ? hipMemcpyAsync(t->h_err, t->ps_err, sizeof(int), hipMemcpyDeviceToHost, t->st) : hipSuccess;
        hipError_t e3 = hipStreamSynchronize(t->st);
        if (e1 || e2 || e3 || e4) { free(hist); SETERR("greedy readback failed"); goto fail; }
        if (t->greedy_ready == 2 && ps_check(t) != 0) { free(hist); goto fail; }
        for (int i = 0; i < n_steps; i++) tokens_out[i] = hist[(frame0 + i) % t->hist_len];
        free(hist);
    }
    t->dev_pos = pos + n_steps;
    if (hidden_out) memcpy(hidden_out, t->h_out, (size_t)H * sizeof(float));
    return 0;
fail:
    if (t) { t->dead = 1; t->dev_pos = -1; }
    return -1;
}

/* Sampled frame loop on the device (qwen_tts.c:1649-1721, code0 only): per step the Talker
 * step, the final norm fused into the codec head, the codec-head rule (clip, special-token
 * mask, EOS masked on frames 0-1, EOS boost after 2 x 3 x text_len frames) +
 * qwen_tts_sample (k_sample) with the repetition penalty over the code0 history
 * (prev_tokens, then every token drawn here, appended as qwen_tts.c:1721 appends them) and
 * the next input = codec_emb[token].  Frames below greedy_warmup draw greedily
 * (qwen_tts.c:1688-1692).  The reference leaves its loop at EOS (qwen_tts.c:1716-1719): here
 * the first EOS sets a device flag, after which the sampler writes EOS without drawing
 * (the LCG state and the history stop where the reference's do) and the remaining steps'
 * results are discarded.  Logits, history and LCG state stay on the device until the end;
 * nothing is allocated per call. */
int qwen_hip_talker_sample(void *state, const uint16_t *codec_head, const uint16_t *codec_emb, int codec_vocab,
                           const float *embed, int pos, int frame0, int n_steps, const qwen_hip_sample_params_t *sp,
                           const int *prev_tokens, int n_prev, uint32_t *seed, int *tokens_out, float *hidden_out) {
    talker_t *t = (talker_t *)state;
    if (!t || t->dead) { SETERR("talker state is dead or NULL"); return -1; }
    const int H = t->s.H;
    if (!codec_head || !codec_emb || codec_vocab <= 2150 || codec_vocab > 4096 || !seed || !sp ||
        (n_steps > 0 && !tokens_out) || n_steps < 0 || frame0 < 0 || n_prev < 0 || (n_prev > 0 && !prev_tokens) || !embed) {
        SETERR("talker_sample: bad arguments"); return -1;
    }
    if ((long long)n_prev + n_steps + 1 > QT_SAMPLE_HIST_MAX) {
        SETERR("talker_sample: history of %d + %d tokens exceeds %d", n_prev, n_steps, QT_SAMPLE_HIST_MAX - 1); return -1;
    }
    if (pos >= 0 && talker_grow_kv(t, pos + n_steps) != 0) return -1;
    if (pos < 0 || pos + n_steps > t->s.kv_max || pos + n_steps > t->s.rope_len) {
        SETERR("talker_sample: positions exceed kv_max"); return -1;
    }
    if (head_setup(t, codec_head, codec_emb, codec_vocab) != 0) goto fail;
    if (talker_set_pos(t, pos) != 0) goto fail;
    if (n_prev > 0) HCK(hipMemcpyAsync(t->smp_hist, prev_tokens, (size_t)n_prev * sizeof(int), hipMemcpyHostToDevice, t->st));
    t->h_pos[2] = (int)*seed;
    t->h_pos[3] = 0;
    HCK(hipMemcpyAsync(t->smp_seed, t->h_pos + 2, sizeof(uint32_t), hipMemcpyHostToDevice, t->st));
    HCK(hipMemcpyAsync(t->smp_done, t->h_pos + 3, sizeof(int), hipMemcpyHostToDevice, t->st));
    /* the step's input: the fused kernel reads it from ps_xin, the per-kernel step works on
     * the residual io[H:2H] in place */
    float *xin = t->ps_on ? t->ps_xin : t->io + H;
    memcpy(t->h_in, embed, (size_t)H * sizeof(float));
    HCK(hipMemcpyAsync(xin, t->h_in, (size_t)H * sizeof(float), hipMemcpyHostToDevice, t->st));
    const int expected = sp->text_len * 3, boost_start = expected * 2;
    for (int i = 0; i < n_steps; i++) {
        float *x = t->io + H;
        const int frame = frame0 + i;
        float boost = 0.0f;
        if (expected > 0 && frame > boost_start) {
            boost = 0.5f * (float)(frame - boost_start);
            if (boost > 10.0f) boost = 10.0f;
        }
        const int warm = sp->greedy_warmup > 0 && frame < sp->greedy_warmup;
        /* one decode step: the fused kernel (one launch; it leaves the residual in io[H:2H],
         * bit-identical to the per-kernel layers, and advances the position) or the layers */
        if (t->ps_on) HCK(ps_launch(t, 1, 0));
        else HCK(stack_body(&t->s, x, t->d_pos, t->st));
        HCK(qt_launch_mv(t->head_m.prec, QT_EPI_STORE, 1, x, t->s.final_norm, t->s.eps, t->head_m.w, NULL, NULL,
                         t->head_m.rows, t->head_m.cols, t->logits, NULL, NULL, t->io, t->st));
        HCK(qt_launch_sample(t->logits, codec_vocab, 1, frame, boost, warm ? 0.0f : sp->temperature,
                             warm ? 1 : sp->top_k, sp->top_p, sp->rep_penalty, t->smp_hist, n_prev + i, t->smp_seed,
                             t->smp_hist + n_prev + i, t->smp_done, t->st));
        HCK(qt_launch_gather(t->smp_hist + n_prev + i, codec_vocab, t->codec_emb, H, xin, t->st));
        if (!t->ps_on) HCK(qt_launch_advance_pos(t->d_pos, 1, t->st));
    }
    if (n_steps > 0)
        HCK(hipMemcpyAsync(tokens_out, t->smp_hist + n_prev, (size_t)n_steps * sizeof(int), hipMemcpyDeviceToHost, t->st));
    HCK(hipMemcpyAsync(t->h_pos + 2, t->smp_seed, sizeof(uint32_t), hipMemcpyDeviceToHost, t->st));
    HCK(hipMemcpyAsync(t->h_out, t->io, (size_t)2 * H * sizeof(float), hipMemcpyDeviceToHost, t->st));
    if (t->ps_on) HCK(hipMemcpyAsync(t->h_err, t->ps_err, sizeof(int), hipMemcpyDeviceToHost, t->st));
    HCK(hipStreamSynchronize(t->st));
    if (t->ps_on && ps_check(t) != 0) goto fail;
    *seed = (uint32_t)t->h_pos[2];
    if (hidden_out) memcpy(hidden_out, t->h_out, (size_t)H * sizeof(float));
    t->dev_pos = pos + n_steps;
    t->greedy_ready = 0;            /* the fused greedy loop's input is stale: re-seed it with talker_greedy */
    int n_gen = n_steps;
    for (int i = 0; i < n_steps; i++)
        if (tokens_out[i] == 2150) { n_gen = i + 1; break; }
    return n_gen;
fail:
    t->dead = 1; t->dev_pos = -1;
    return -1;
}

int qwen_hip_talker_greedy_async(void *state, int n_steps) {
    talker_t *t = (talker_t *)state;
    if (!t || t->dead || !t->greedy_ready) { SETERR("greedy loop not initialised"); return -1; }
    if (t->dev_pos >= 0 && talker_grow_kv(t, t->dev_pos + n_steps) != 0) return -1;
    REQ(t->dev_pos >= 0 && t->dev_pos + n_steps <= t->s.kv_max && t->dev_pos + n_steps <= t->s.rope_len,
        "positions exceed kv_max");
    if (t->greedy_ready == 2) {
        if (n_steps > 0) HCK(ps_launch(t, n_steps, 1));
    } else {
        if (graphs_enabled() && !t->ggraph_ready) {       /* dropped when the cache grew */
            if (capture(t->st, &t->gexec, greedy_body, t) != 0) goto fail;
            t->ggraph_ready = 1;
        }
        for (int i = 0; i < n_steps; i++) HCK(graphs_enabled() ? hipGraphLaunch(t->gexec, t->st) : greedy_body(t));
    }
    t->dev_pos += n_steps;
    return 0;
fail:
    if (t) t->dead = 1;
    return -1;
}

int qwen_hip_talker_sync(void *state) {
    talker_t *t = (talker_t *)state;
    if (!t) return -1;
    if (t->ps_on) HCK(hipMemcpyAsync(t->h_err, t->ps_err, sizeof(int), hipMemcpyDeviceToHost, t->st));
    HCK(hipStreamSynchronize(t->st));
    if (t->ps_on && ps_check(t) != 0) goto fail;
    return 0;
fail:
    t->dead = 1;
    return -1;
}

/* Enqueue n launches of one kernel of the step (benchmark/profiling aid, no sync):
 * kernel 0 norm+QKV, 1 attention (at the current device position), 2 O+residual,
 * 3 norm+gate_up+SwiGLU, 4 down+residual, 5 final norm (position not advanced). */
int qwen_hip_talker_launch_kernel(void *state, int kernel, int layer, int n) {
    talker_t *t = (talker_t *)state;
    if (!t || t->dead) { SETERR("talker state is dead or NULL"); return -1; }
    stack_t *s = &t->s;
    REQ(layer >= 0 && layer < s->L && kernel >= 0 && kernel <= 5 && n >= 0, "bad kernel/layer");
    REQ(t->dev_pos >= 0 && t->dev_pos < s->kv_max, "device position unknown: run a step first");
    float *x = t->io + s->H;
    const size_t lay = (size_t)layer * s->nkv * s->kv_max * s->hd;
    for (int i = 0; i < n; i++) {
        switch (kernel) {
        case 0: HCK(mv(&s->qkv[layer], QT_EPI_STORE, 1, x, s->in_norm[layer], s->eps, s->qkvbuf, NULL, NULL, t->st)); break;
        case 1: HCK((s->step_onepass ? qt_launch_attn_onepass : qt_launch_attn)(
                        1, s->qkvbuf, s->qn[layer], s->kn[layer], s->rope_cos, s->rope_sin, s->eps, t->d_pos, 0,
                                   s->kc + lay, s->vc + lay, s->hd, (long long)s->kv_max * s->hd, s->nh, s->nkv,
                                   s->hd, 1.0f / sqrtf((float)s->hd), s->part, s->cnt, s->step_G, s->attn, t->st)); break;
        case 2: HCK(mv(&s->o[layer], QT_EPI_STORE, 0, s->attn, NULL, s->eps, s->hbuf, NULL, NULL, t->st)); break;
        case 3: HCK(mv(&s->gu[layer], QT_EPI_SWIGLU, 1, x, s->post_norm[layer], s->eps, s->hbuf, NULL, NULL, t->st)); break;
        case 4: HCK(mv(&s->dn[layer], QT_EPI_STORE, 0, s->hbuf, NULL, s->eps, s->attn, NULL, NULL, t->st)); break;
        case 5: HCK(qt_launch_rmsnorm(x, s->final_norm, t->io, s->H, s->eps, NULL, t->st)); break;
        }
    }
    return 0;
fail:
    return -1;
}

int qwen_hip_talker_dequant(void *state, int layer, int which, int r0, int n, float *out) {
    talker_t *t = (talker_t *)state;
    float *d = NULL;
    if (!t) { SETERR("NULL state"); return -1; }
    stack_t *s = &t->s;
    REQ(layer >= 0 && layer < s->L && which >= 0 && which <= 5, "bad layer/which");
    const dmat_t *m = which <= 2 ? &s->qkv[layer] : which == 3 ? &s->o[layer] : which == 4 ? &s->gu[layer] : &s->dn[layer];
    int off = which == 1 ? s->qd : which == 2 ? s->qd + s->kvd : 0;
    int lim = which == 0 ? s->qd : which <= 2 ? s->kvd : m->rows;
    REQ(r0 >= 0 && n >= 0 && r0 + n <= lim, "row range out of bounds");
    HCK(hipMalloc((void **)&d, (size_t)n * m->cols * sizeof(float) + 4));
    HCK(qt_launch_dequant(m->prec, m->w, m->scale, m->s16, m->cols, off + r0, n, d, t->st));
    HCK(hipMemcpyAsync(out, d, (size_t)n * m->cols * sizeof(float), hipMemcpyDeviceToHost, t->st));
    HCK(hipStreamSynchronize(t->st));
    (void)hipFree(d);
    return 0;
fail:
    if (d) (void)hipFree(d);
    return -1;
}

/* ---- Code Predictor state ------------------------------------------------------------ */

typedef struct {
    stack_t s;
    hipStream_t st;
    int codebook, lm_prec, codec_vocab, talker_hidden, emb_dim;
    dmat_t lm[15];
    uint16_t *cp_emb[15];
    uint16_t *talker_emb;
    dmat_t mtp; int has_mtp; float *mtp_bias;
    float *x, *ebuf, *logits, *th;   /* device */
    int *d_posv;                          /* [64]: 0..63, per-pass positions */
    int *d_codes;                         /* [16]: [0] = code0, [1..15] = out codes */
    float *h_x; int *h_codes;             /* pinned */
    hipGraphExec_t fexec, pexec;
    int fready, pready, frame_ready;
    int *d_steppos;
    /* two-position prefill (positions 0 and 1 as one two-column pass) */
    int prefill2;                         /* 1: the frame starts with cp_prefill2_body */
    float *x2, *qkv2, *attn2, *h2;        /* device [2][H], [2][QKV], [2][qd], [2][F] */
    int8_t *pc2; float *ps2;              /* activation pieces of the two columns */
    /* the whole frame as one launch of the role-specialised kernel's 0.6B build: int8 layers,
     * lm heads and mtp projection (qt_launch_rstep06_cp) or all of them bf16
     * (qt_launch_rstep06b_cp) */
    int rs_ok, rs_on;                     /* available / in use */
    int rs_bf16;                          /* the bf16 build */
    void *rs_layers;                      /* device layer table */
    unsigned *rs_reg; unsigned long long *rs_slots;
    void **rs_tab;                        /* device [45]: lm heads, their scales, input tables */
    unsigned *rs_epoch; int *rs_err, *rs_pos;
    float *rs_io;                         /* [2H]: final-normed and raw x of the last pass */
    int dead;
} cp_t;

static void cp_destroy(cp_t *c) {
    if (!c) return;
    if (c->fready) (void)hipGraphExecDestroy(c->fexec);
    if (c->pready) (void)hipGraphExecDestroy(c->pexec);
    stack_free(&c->s);
    for (int g = 0; g < 15; g++) { dmat_free(&c->lm[g]); if (c->cp_emb[g]) (void)hipFree(c->cp_emb[g]); }
    dmat_free(&c->mtp);
    void *bufs[] = {c->talker_emb, c->mtp_bias, c->x, c->ebuf, c->logits, c->th, c->d_posv, c->d_codes, c->d_steppos,
                    c->x2, c->qkv2, c->attn2, c->h2, c->pc2, c->ps2, c->rs_layers, c->rs_reg, c->rs_slots, c->rs_tab,
                    c->rs_epoch, c->rs_err, c->rs_pos, c->rs_io};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) if (bufs[i]) (void)hipFree(bufs[i]);
    if (c->h_x) (void)hipHostFree(c->h_x);
    if (c->h_codes) (void)hipHostFree(c->h_codes);
    if (c->st) (void)hipStreamDestroy(c->st);
    free(c);
}

/* The role-specialised frame's resources, when the CP qualifies: the 0.6B geometry, one
 * precision (int8 or bf16) in every layer, lm head and the mtp projection (which must map the
 * 2048-wide Talker hidden state).  The per-kernel path then splits its attention into the
 * same key chunks with the same one-pass arithmetic; with int8 weights the two frames give
 * the same bits, with bf16 weights the projections sum the same exact products in the MFMA's
 * order instead of k_mv's. */
static int cp_rs_setup(cp_t *c) {
    stack_t *s = &c->s;
    void *host_tab = NULL;
    void *ptab[45];
    const unsigned one = 1;
    const int wp = c->lm_prec;
    if (!rstep_enabled() || (wp != QWEN_HIP_INT8 && wp != QWEN_HIP_BF16)) return 0;
    if (c->has_mtp && (c->mtp.prec != wp || c->emb_dim != 2048 || c->talker_hidden != 2048)) return 0;
    const int rk = wp == QWEN_HIP_BF16 ? 3 : 2;
    if (!(rk == 3 ? qt_rstep06b_supported : qt_rstep06_supported)(s->prec, s->H, s->F, s->nh, s->nkv, s->hd,
                                                                   s->kv_max, s->L)) return 0;
    for (int l = 0; l < s->L; l++)
        if (s->qkv[l].prec != wp || s->o[l].prec != wp || s->gu[l].prec != wp || s->dn[l].prec != wp) return 0;
    const size_t lb = qt_pstep_layer_bytes();
    const size_t rw = rs_region_words(rk, s->L), sw = rs_slot_words(rk);
    HCK(hipMalloc((void **)&c->rs_reg, rw * sizeof(unsigned)));
    HCK(hipMalloc((void **)&c->rs_slots, sw * sizeof(unsigned long long)));
    HCK(hipMemsetAsync(c->rs_reg, 0xFF, rw * sizeof(unsigned), c->st));
    HCK(hipMemsetAsync(c->rs_slots, 0, sw * sizeof(unsigned long long), c->st));
    HCK(hipMalloc((void **)&c->rs_epoch, 64));
    HCK(hipMalloc((void **)&c->rs_err, 64));
    HCK(hipMalloc((void **)&c->rs_pos, 64));
    HCK(hipMalloc((void **)&c->rs_io, (size_t)2 * s->H * sizeof(float)));
    HCK(hipMemsetAsync(c->rs_err, 0, 64, c->st));
    HCK(hipMemsetAsync(c->rs_pos, 0, 64, c->st));
    HCK(hipMemcpyAsync(c->rs_epoch, &one, sizeof one, hipMemcpyHostToDevice, c->st));
    for (int g = 0; g < 15; g++) {
        ptab[g] = (void *)c->lm[g].w;
        ptab[15 + g] = (void *)c->lm[g].scale;
        ptab[30 + g] = g == 0 ? (void *)c->talker_emb : (void *)c->cp_emb[g - 1];
    }
    HCK(hipMalloc((void **)&c->rs_tab, sizeof ptab));
    HCK(hipMemcpy(c->rs_tab, ptab, sizeof ptab, hipMemcpyHostToDevice));
    host_tab = calloc((size_t)s->L, lb);
    REQ(host_tab, "host alloc");
    for (int l = 0; l < s->L; l++) {
        const uint8_t *w[4] = {s->qkv[l].w, s->o[l].w, s->gu[l].w, s->dn[l].w};
        const float *sc[4] = {s->qkv[l].scale, s->o[l].scale, s->gu[l].scale, s->dn[l].scale};
        const uint16_t *s16[4] = {s->qkv[l].s16, s->o[l].s16, s->gu[l].s16, s->dn[l].s16};
        qt_pstep_fill_layer((char *)host_tab + (size_t)l * lb, w, sc, s16, s->in_norm[l], s->post_norm[l], s->qn[l], s->kn[l]);
    }
    HCK(hipMalloc(&c->rs_layers, (size_t)s->L * lb));
    HCK(hipMemcpy(c->rs_layers, host_tab, (size_t)s->L * lb, hipMemcpyHostToDevice));
    HCK(hipStreamSynchronize(c->st));
    free(host_tab);
    s->step_G = qt_rstep_chunks();
    s->step_onepass = 1;
    c->rs_ok = c->rs_on = 1;
    c->rs_bf16 = rk == 3;
    return 0;
fail:
    free(host_tab);
    return -1;
}

static hipError_t cp_rs_launch_on(cp_t *c, hipStream_t st) {
    stack_t *s = &c->s;
    return (c->rs_bf16 ? qt_launch_rstep06b_cp : qt_launch_rstep06_cp)(c->rs_layers, s->L, s->final_norm, s->rope_cos, s->rope_sin, s->kc, s->vc, s->kv_max,
                                s->eps, 1.0f / sqrtf((float)s->hd), c->rs_reg, c->rs_slots, c->rs_io, c->rs_io + s->H,
                                c->th, c->rs_pos, c->rs_epoch, c->rs_err, 16, (const void *const *)c->rs_tab,
                                c->codebook, c->d_codes, c->has_mtp ? c->mtp.w : NULL,
                                c->has_mtp ? c->mtp.scale : NULL, c->has_mtp ? c->mtp_bias : NULL, st);
}
static hipError_t cp_rs_launch(cp_t *c) { return cp_rs_launch_on(c, c->st); }

void *qwen_hip_cp_init(const qwen_hip_cp_desc_t *d) {
    cp_t *c = calloc(1, sizeof *c);
    void *tmp = NULL;
    if (!c) { SETERR("out of host memory"); return NULL; }
    REQ(d, "null descriptor");
    HCK(hipStreamCreateWithFlags(&c->st, hipStreamNonBlocking));
    if (stack_init(&c->s, &d->cp, c->st) != 0) goto fail;   /* g_err already set */
    c->codebook = d->codebook; c->codec_vocab = d->codec_vocab;
    c->talker_hidden = d->talker_hidden; c->emb_dim = d->emb_dim;
    c->lm_prec = (d->cp.quantize_to >= 0) ? d->cp.quantize_to : d->lm_prec;
    const int H = c->s.H;
    REQ(c->s.kv_max >= 16, "CP kv_max must hold 16 positions");
    size_t tb = (size_t)c->codebook * (H > c->emb_dim ? H : c->emb_dim) * 2 + 64;
    HCK(hipMalloc(&tmp, tb));
    for (int g = 0; g < 15; g++) {
        REQ(dmat_alloc(&c->lm[g], c->lm_prec, c->codebook, H) == 0, "alloc lm_head");
        REQ(dmat_put(&c->lm[g], 0, &d->lm_head[g], d->lm_prec, c->codebook, c->st, tmp) == 0, "upload lm_head %d", g);
        REQ(d->cp_codec_emb[g], "missing cp codec embedding %d", g);
        HCK(hipMalloc((void **)&c->cp_emb[g], (size_t)c->codebook * c->emb_dim * 2));
        HCK(hipMemcpy(c->cp_emb[g], d->cp_codec_emb[g], (size_t)c->codebook * c->emb_dim * 2, hipMemcpyDefault));
    }
    REQ(d->talker_codec_emb, "missing talker codec embedding");
    HCK(hipMalloc((void **)&c->talker_emb, (size_t)c->codec_vocab * c->talker_hidden * 2));
    HCK(hipMemcpy(c->talker_emb, d->talker_codec_emb, (size_t)c->codec_vocab * c->talker_hidden * 2, hipMemcpyDefault));
    c->has_mtp = d->mtp.w != NULL;
    if (c->has_mtp) {
        int mp = d->mtp_prec;
        /* a quantized CP has its mtp projection in int8 too, as the reference quantizes it
         * for both --int8 and --int4 (qwen_tts_code_predictor.c:474-476) */
        const int qt = d->cp.quantize_to;
        const int mdst = (mp == QWEN_HIP_BF16 && (qt == QWEN_HIP_INT8 || qt == QWEN_HIP_Q4_0)) ? QWEN_HIP_INT8 : mp;
        REQ(dmat_alloc(&c->mtp, mdst, H, c->emb_dim) == 0, "alloc mtp");
        REQ(dmat_put(&c->mtp, 0, &d->mtp, mp, H, c->st, tmp) == 0, "upload mtp");
        REQ(d->mtp_bias, "mtp projection without bias");
        REQ((c->mtp_bias = up_f32(d->mtp_bias, H, c->st)) != NULL, "mtp bias");
    } else {
        REQ(c->emb_dim == H && c->talker_hidden == H, "no mtp projection but emb_dim != cp_hidden");
    }
    int E = c->emb_dim > c->talker_hidden ? c->emb_dim : c->talker_hidden;
    HCK(hipMalloc((void **)&c->x, (size_t)H * sizeof(float)));
    HCK(hipMalloc((void **)&c->ebuf, (size_t)E * sizeof(float)));
    HCK(hipMalloc((void **)&c->th, (size_t)E * sizeof(float)));
    HCK(hipMalloc((void **)&c->logits, (size_t)c->codebook * sizeof(float)));
    HCK(hipMalloc((void **)&c->d_posv, 64 * sizeof(int)));
    HCK(hipMalloc((void **)&c->d_codes, 16 * sizeof(int)));
    HCK(hipMalloc((void **)&c->d_steppos, sizeof(int)));
    HCK(hipHostMalloc((void **)&c->h_x, (size_t)(E > H ? E : H) * sizeof(float), hipHostMallocDefault));
    HCK(hipHostMalloc((void **)&c->h_codes, 64 * sizeof(int), hipHostMallocDefault));
    for (int i = 0; i < 64; i++) c->h_codes[i] = i;
    HCK(hipMemcpy(c->d_posv, c->h_codes, 64 * sizeof(int), hipMemcpyHostToDevice));
    (void)hipFree(tmp);
    tmp = NULL;
    if (cp_rs_setup(c) != 0) goto fail;
    return c;
fail:
    if (tmp) (void)hipFree(tmp);
    cp_destroy(c);
    return NULL;
}

/* the CP cache after a frame or passes: positions [0, n) as the reference keeps
 * ctx->cp_kv_k / cp_kv_v ([layer][cp_kv_max][kv_dim]) */
int qwen_hip_cp_download_kv(void *state, uint16_t *kv_k, uint16_t *kv_v, int host_kv_max, int n) {
    cp_t *c = (cp_t *)state;
    if (!c) { SETERR("NULL state"); return -1; }
    return stack_download_kv(&c->s, c->st, kv_k, kv_v, host_kv_max, n);
}

void qwen_hip_cp_free(void *state) { cp_destroy((cp_t *)state); }
void *qwen_hip_cp_stream(void *state) { return state ? (void *)((cp_t *)state)->st : NULL; }

/* dst = mtp(src) (qwen_tts_code_predictor.c:907-924) */
static hipError_t cp_project(cp_t *c, const float *src, float *dst) {
    if (c->has_mtp)
        return mv(&c->mtp, QT_EPI_BIAS, 0, src, NULL, c->s.eps, dst, NULL, c->mtp_bias, c->st);
    return qt_launch_copy_f32(src, dst, c->s.H, c->st);
}

static hipError_t cp_pass_body(void *a) {
    cp_t *c = (cp_t *)a;
    return stack_body(&c->s, c->x, c->d_steppos, c->st);
}

/* Positions 0 and 1 of a frame as one two-column pass: the device twin of cp_prefill2
 * (qwen_tts_code_predictor.c:816-902).  x2 = [x0 | x1] (residuals, not normed).  Every
 * projection reads its int8 weights once for both columns (pieces + MFMA, the batched
 * projection of qt_batch.hip); per-head norm, RoPE, KV append and attention run per
 * position in order, so position 1 attends to the key/value that position 0 appended.
 * Mathematically the two sequential passes; the projections round differently (exact
 * integer products of 3-plane activation pieces instead of f32 dot products), the same
 * kind of difference the reference accepts for its B=2 matmat. */
static hipError_t cp_prefill2_body(cp_t *c) {
    stack_t *s = &c->s;
    hipError_t e;
    const int H = s->H, F = s->F, QKV = s->qd + 2 * s->kvd;
    const float scale = 1.0f / sqrtf((float)s->hd);
    for (int l = 0; l < s->L; l++) {
        const size_t lay = (size_t)l * s->nkv * s->kv_max * s->hd;
        if ((e = qt_launch_bpieces(c->x2, H, s->in_norm[l], s->eps, H, 2, 16, c->pc2, c->ps2, c->st))) return e;
        if ((e = qt_launch_bgemm_i8(QT_EPI_STORE, s->qkv[l].w, s->qkv[l].scale, QKV, H, c->pc2, c->ps2, 2, 16, c->qkv2, QKV,
                                    c->st))) return e;
        for (int p = 0; p < 2; p++)
            if ((e = qt_launch_attn(1, c->qkv2 + (size_t)p * QKV, s->qn[l], s->kn[l], s->rope_cos, s->rope_sin, s->eps,
                                    c->d_posv + p, 0, s->kc + lay, s->vc + lay, s->hd, (long long)s->kv_max * s->hd, s->nh,
                                    s->nkv, s->hd, scale, s->part, s->cnt, s->attn_G, c->attn2 + (size_t)p * s->qd,
                                    c->st))) return e;
        if ((e = qt_launch_bpieces(c->attn2, s->qd, NULL, s->eps, s->qd, 2, 16, c->pc2, c->ps2, c->st))) return e;
        if ((e = qt_launch_bgemm_i8(QT_EPI_RESID, s->o[l].w, s->o[l].scale, H, s->qd, c->pc2, c->ps2, 2, 16, c->x2, H,
                                    c->st))) return e;
        if ((e = qt_launch_bpieces(c->x2, H, s->post_norm[l], s->eps, H, 2, 16, c->pc2, c->ps2, c->st))) return e;
        if ((e = qt_launch_bgemm_i8(QT_EPI_SWIGLU, s->gu[l].w, s->gu[l].scale, 2 * F, H, c->pc2, c->ps2, 2, 16, c->h2, F,
                                    c->st))) return e;
        if ((e = qt_launch_bpieces(c->h2, F, NULL, s->eps, F, 2, 16, c->pc2, c->ps2, c->st))) return e;
        if ((e = qt_launch_bgemm_i8(QT_EPI_RESID, s->dn[l].w, s->dn[l].scale, H, F, c->pc2, c->ps2, 2, 16, c->x2, H,
                                    c->st))) return e;
    }
    return hipSuccess;
}

/* Mode switch of the two-position prefill (the reference's QWEN_CP_PREFILL2,
 * qwen_tts_code_predictor.c:783-807): on needs int8 weights in every CP layer.  The
 * frame graph is rebuilt on the next frame. */
int qwen_hip_cp_set_prefill2(void *state, int on) {
    cp_t *c = (cp_t *)state;
    if (!c || c->dead) { SETERR("CP state is dead or NULL"); return -1; }
    stack_t *s = &c->s;
    if (on) {
        for (int l = 0; l < s->L; l++)
            REQ(s->qkv[l].prec == QWEN_HIP_INT8 && s->o[l].prec == QWEN_HIP_INT8 && s->gu[l].prec == QWEN_HIP_INT8 &&
                s->dn[l].prec == QWEN_HIP_INT8, "CP prefill2 needs int8 weights in every layer");
        REQ(s->H % 64 == 0 && s->F % 64 == 0 && s->qd % 64 == 0, "CP prefill2 needs dims divisible by 64");
        if (!c->x2) {
            const int K = s->F > s->H ? (s->F > s->qd ? s->F : s->qd) : (s->H > s->qd ? s->H : s->qd);
            HCK(hipMalloc((void **)&c->x2, (size_t)2 * s->H * sizeof(float)));
            HCK(hipMalloc((void **)&c->qkv2, (size_t)2 * (s->qd + 2 * s->kvd) * sizeof(float)));
            HCK(hipMalloc((void **)&c->attn2, (size_t)2 * s->qd * sizeof(float)));
            HCK(hipMalloc((void **)&c->h2, (size_t)2 * s->F * sizeof(float)));
            HCK(hipMalloc((void **)&c->pc2, (size_t)K * 3 * 16));
            HCK(hipMalloc((void **)&c->ps2, 16 * sizeof(float)));
        }
    }
    if (c->prefill2 != (on != 0) && c->fready) {
        (void)hipGraphExecDestroy(c->fexec);
        c->fready = 0;
        c->frame_ready = 0;
    }
    c->prefill2 = on != 0;
    return 0;
fail:
    return -1;
}

/* x0, x1: host f32[cp_hidden] residuals in/out; positions 0 and 1 (their KV rows are
 * written).  The device twin of cp_prefill2(ctx, mode, x0, x1). */
int qwen_hip_cp_prefill2(void *state, float *x0, float *x1) {
    cp_t *c = (cp_t *)state;
    if (!c || c->dead) { SETERR("CP state is dead or NULL"); return -1; }
    if (!x0 || !x1) { SETERR("null residuals"); return -1; }            /* argument errors leave the state usable */
    if (!c->x2) { SETERR("CP prefill2 is not enabled (qwen_hip_cp_set_prefill2)"); return -1; }
    const int H = c->s.H;
    memcpy(c->h_x, x0, (size_t)H * sizeof(float));
    HCK(hipMemcpyAsync(c->x2, c->h_x, (size_t)H * sizeof(float), hipMemcpyHostToDevice, c->st));
    HCK(hipStreamSynchronize(c->st));
    memcpy(c->h_x, x1, (size_t)H * sizeof(float));
    HCK(hipMemcpyAsync(c->x2 + H, c->h_x, (size_t)H * sizeof(float), hipMemcpyHostToDevice, c->st));
    HCK(cp_prefill2_body(c));
    HCK(hipMemcpyAsync(c->h_x, c->x2, (size_t)H * sizeof(float), hipMemcpyDeviceToHost, c->st));
    HCK(hipStreamSynchronize(c->st));
    memcpy(x0, c->h_x, (size_t)H * sizeof(float));
    HCK(hipMemcpyAsync(c->h_x, c->x2 + H, (size_t)H * sizeof(float), hipMemcpyDeviceToHost, c->st));
    HCK(hipStreamSynchronize(c->st));
    memcpy(x1, c->h_x, (size_t)H * sizeof(float));
    return 0;
fail:
    if (c) c->dead = 1;
    return -1;
}

/* The whole frame (qwen_tts_code_predictor.c:926-1045) as one launch sequence:
 * th = talker hidden (device), d_codes[0] = code0. */
static hipError_t cp_frame_body(void *a) {
    cp_t *c = (cp_t *)a;
    hipError_t e;
    const int H = c->s.H;
    /* Without the mtp projection an embedding row is the next pass's input itself, so the
     * gathers write straight into the residual buffers (no copy kernel). */
    const int mtp = c->has_mtp;
    if (c->prefill2) {
        if ((e = cp_project(c, c->th, c->x2))) return e;
        if ((e = qt_launch_gather(c->d_codes, c->codec_vocab, c->talker_emb, c->talker_hidden,
                                  mtp ? c->ebuf : c->x2 + H, c->st))) return e;
        if (mtp && (e = cp_project(c, c->ebuf, c->x2 + H))) return e;
        if ((e = cp_prefill2_body(c))) return e;
        if ((e = qt_launch_copy_f32(c->x2 + H, c->x, H, c->st))) return e;
    } else {
        /* pass 0 on the projected Talker hidden state; code0's embedding, the input of
         * pass 1, is looked up once pass 0 has consumed x */
        if ((e = cp_project(c, c->th, c->x))) return e;
        if ((e = stack_body(&c->s, c->x, c->d_posv + 0, c->st))) return e;
        if ((e = qt_launch_gather(c->d_codes, c->codec_vocab, c->talker_emb, c->talker_hidden,
                                  mtp ? c->ebuf : c->x, c->st))) return e;
        if (mtp && (e = cp_project(c, c->ebuf, c->x))) return e;
        if ((e = stack_body(&c->s, c->x, c->d_posv + 1, c->st))) return e;
    }
    for (int g = 0; g < 15; g++) {
        if (g > 0) {
            if (mtp && (e = cp_project(c, c->ebuf, c->x))) return e;
            if ((e = stack_body(&c->s, c->x, c->d_posv + g + 1, c->st))) return e;
        }
        if ((e = mv(&c->lm[g], QT_EPI_STORE, 1, c->x, c->s.final_norm, c->s.eps, c->logits, NULL, NULL, c->st))) return e;
        /* the argmax also gathers code g+1's row of the next embedding table (the input
         * of pass g+2), the lookup of qwen_tts_code_predictor.c:1008-1017 */
        if ((e = qt_launch_select(c->logits, c->codebook, 0, NULL, 0, c->d_codes + g + 1, NULL, 0,
                                  g < 14 ? c->cp_emb[g] : NULL, c->emb_dim, mtp ? c->ebuf : c->x, NULL, c->st)))
            return e;
    }
    return hipSuccess;
}

/* cp_frame_body with every launch on stream st (the ungraphed frame inside another
 * state's stream, for QWEN_HIP_GRAPH=0) */
static hipError_t cp_frame_body_on(cp_t *c, hipStream_t st) {
    hipStream_t own = c->st;
    c->st = st;
    hipError_t e = cp_frame_body(c);
    c->st = own;
    return e;
}

int qwen_hip_cp_frame(void *state, const float *talker_hidden, int code0, int *out_codes) {
    cp_t *c = (cp_t *)state;
    if (!c || c->dead) { SETERR("CP state is dead or NULL"); return -1; }
    memcpy(c->h_x, talker_hidden, (size_t)c->talker_hidden * sizeof(float));
    c->h_codes[0] = code0;
    HCK(hipMemcpyAsync(c->th, c->h_x, (size_t)c->talker_hidden * sizeof(float), hipMemcpyHostToDevice, c->st));
    HCK(hipMemcpyAsync(c->d_codes, c->h_codes, sizeof(int), hipMemcpyHostToDevice, c->st));
    if (c->rs_on && !c->prefill2) {
        HCK(cp_rs_launch(c));
        c->frame_ready = 1;
        HCK(hipMemcpyAsync(c->h_codes + 16, c->d_codes, 16 * sizeof(int), hipMemcpyDeviceToHost, c->st));
        HCK(hipMemcpyAsync(c->h_codes + 32, c->rs_err, sizeof(int), hipMemcpyDeviceToHost, c->st));
        HCK(hipStreamSynchronize(c->st));
        REQ(c->h_codes[32] == 0, "CP frame: a wait for another workgroup's data timed out (device error flag set)");
        for (int g = 0; g < 15; g++) out_codes[g] = c->h_codes[16 + 1 + g];
        for (int i = 0; i < 16; i++) c->h_codes[16 + i] = 0;
        c->h_codes[0] = 0;
        return 0;
    }
    if (graphs_enabled() && !c->fready) {
        if (capture(c->st, &c->fexec, cp_frame_body, c) != 0) goto fail;
        c->fready = 1;
    }
    c->frame_ready = 1;
    HCK(graphs_enabled() ? hipGraphLaunch(c->fexec, c->st) : cp_frame_body(c));
    HCK(hipMemcpyAsync(c->h_codes + 16, c->d_codes, 16 * sizeof(int), hipMemcpyDeviceToHost, c->st));
    HCK(hipStreamSynchronize(c->st));
    for (int g = 0; g < 15; g++) out_codes[g] = c->h_codes[16 + 1 + g];
    for (int i = 0; i < 16; i++) c->h_codes[16 + i] = 0;
    c->h_codes[0] = 0;
    return 0;
fail:
    if (c) c->dead = 1;
    return -1;
}

int qwen_hip_cp_frame_async(void *state, int n_frames) {
    cp_t *c = (cp_t *)state;
    if (!c || c->dead || !c->frame_ready) { SETERR("CP frame not initialised"); return -1; }
    if (c->rs_on && !c->prefill2) {
        for (int i = 0; i < n_frames; i++) HCK(cp_rs_launch(c));
        return 0;
    }
    REQ(c->fready || !graphs_enabled(), "CP frame graph not captured");
    for (int i = 0; i < n_frames; i++) HCK(graphs_enabled() ? hipGraphLaunch(c->fexec, c->st) : cp_frame_body(c));
    return 0;
fail:
    c->dead = 1;
    return -1;
}

int qwen_hip_cp_sync(void *state) {
    cp_t *c = (cp_t *)state;
    if (!c) return -1;
    HCK(hipStreamSynchronize(c->st));
    if (c->rs_ok) {
        int e = 0;
        HCK(hipMemcpy(&e, c->rs_err, sizeof e, hipMemcpyDeviceToHost));
        REQ(e == 0, "CP frame: a wait for another workgroup's data timed out (device error flag set)");
    }
    return 0;
fail:
    c->dead = 1;
    return -1;
}

/* Frames on the role-specialised kernel (on = 1, the default where the CP qualifies) or
 * on the per-kernel graph (0); int8 weights give the same bits both ways, bf16 weights the
 * same codes with K/V within f32 rounding.  Returns the mode in effect. */
int qwen_hip_cp_fused(void *state, int on) {
    cp_t *c = (cp_t *)state;
    if (!c || c->dead) { SETERR("CP state is dead or NULL"); return -1; }
    HCK(hipStreamSynchronize(c->st));
    c->rs_on = on && c->rs_ok;
    c->frame_ready = 0;       /* the next frame call sets the inputs of the new mode */
    return c->rs_on;
fail:
    c->dead = 1;
    return -1;
}

int qwen_hip_cp_step(void *state, float *x, int pos) {
    cp_t *c = (cp_t *)state;
    if (!c || c->dead) { SETERR("CP state is dead or NULL"); return -1; }
    REQ(pos >= 0 && pos < c->s.kv_max && pos < c->s.rope_len, "CP pos %d out of range", pos);
    const int H = c->s.H;
    memcpy(c->h_x, x, (size_t)H * sizeof(float));
    c->h_codes[32] = pos;
    HCK(hipMemcpyAsync(c->x, c->h_x, (size_t)H * sizeof(float), hipMemcpyHostToDevice, c->st));
    HCK(hipMemcpyAsync(c->d_steppos, c->h_codes + 32, sizeof(int), hipMemcpyHostToDevice, c->st));
    if (graphs_enabled() && !c->pready) {
        if (capture(c->st, &c->pexec, cp_pass_body, c) != 0) goto fail;
        c->pready = 1;
    }
    HCK(graphs_enabled() ? hipGraphLaunch(c->pexec, c->st) : cp_pass_body(c));
    HCK(hipMemcpyAsync(c->h_x, c->x, (size_t)H * sizeof(float), hipMemcpyDeviceToHost, c->st));
    HCK(hipStreamSynchronize(c->st));
    memcpy(x, c->h_x, (size_t)H * sizeof(float));
    return 0;
fail:
    if (c) c->dead = 1;
    return -1;
}

/* ---- the whole frame loop on the device ------------------------------------------------- */

/* The Talker + Code Predictor frame loop of qwen_tts_generate (qwen_tts.c:1649-1778, the
 * non-streaming path) with no host round trip per frame.  Per frame f, on the Talker's
 * stream: codec head over the last normed hidden state -> codec-head rule (EOS boost,
 * greedy warmup) + qwen_tts_sample with the code0 history (k_sample) -> the CP frame
 * (its captured graph: mtp projection, 16 passes, 15 greedy lm-head picks) for that
 * hidden state and code0 -> next input codec_emb[code0] + sum_g cp_codec_emb[g][code_g] +
 * tts_pad (k_frame_embed) -> one Talker step (the fused persistent kernel reading that
 * input from device memory, or the per-kernel step).  hidden0 is the normed hidden state
 * the loop starts from (the prefill's last position, or the previous call's last step);
 * the first step runs at pos.  As in the reference, the frame whose code0 is EOS ends the
 * utterance: it is not a frame, and from it on the sampler draws nothing (the LCG state
 * and the history stop there); the remaining frames' work runs and is discarded.
 * codes_out[n_frames][16] (code0, then the 15 CP codes); returns the number of frames
 * generated (codes_out[n][0] == 2150 marks where EOS was drawn, when n < n_frames), or -1.
 * The CP state must not be used on its own stream meanwhile.  Allocates nothing. */
int qwen_hip_generate(void *talker_state, void *cp_state, const uint16_t *codec_head, const uint16_t *codec_emb,
                      int codec_vocab, const float *tts_pad, const float *hidden0, int pos, int frame0, int n_frames,
                      const qwen_hip_sample_params_t *sp, const int *prev_tokens, int n_prev, uint32_t *seed,
                      int *codes_out, float *hidden_out) {
    talker_t *t = (talker_t *)talker_state;
    cp_t *c = (cp_t *)cp_state;
    if (!t || t->dead || !c || c->dead) { SETERR("generate: talker or CP state is dead or NULL"); return -1; }
    const int H = t->s.H;
    if (!codec_head || !codec_emb || codec_vocab <= 2150 || codec_vocab > 4096 || !tts_pad || !hidden0 || !sp || !seed ||
        (n_frames > 0 && !codes_out) || n_frames < 0 || frame0 < 0 || n_prev < 0 || (n_prev > 0 && !prev_tokens)) {
        SETERR("generate: bad arguments"); return -1;
    }
    if (c->talker_hidden != H || c->codec_vocab != codec_vocab || c->emb_dim != H) {
        SETERR("generate: CP state built for talker hidden %d / vocab %d / emb_dim %d, Talker has %d / %d",
               c->talker_hidden, c->codec_vocab, c->emb_dim, H, codec_vocab);
        return -1;
    }
    if ((long long)n_prev + n_frames + 1 > QT_SAMPLE_HIST_MAX) {
        SETERR("generate: history of %d + %d tokens exceeds %d", n_prev, n_frames, QT_SAMPLE_HIST_MAX - 1); return -1;
    }
    if (pos >= 0 && talker_grow_kv(t, pos + n_frames) != 0) return -1;
    if (pos < 0 || pos + n_frames > t->s.kv_max || pos + n_frames > t->s.rope_len) {
        SETERR("generate: positions exceed kv_max"); return -1;
    }
    if (head_setup(t, codec_head, codec_emb, codec_vocab) != 0) goto fail;
    const int cp_fused = c->rs_on && !c->prefill2;   /* the CP frame as one launch */
    if (!cp_fused && graphs_enabled() && !c->fready) {
        if (capture(c->st, &c->fexec, cp_frame_body, c) != 0) goto fail;
        c->fready = 1;
    }
    HCK(hipStreamSynchronize(c->st));               /* nothing of the CP's own stream still runs */
    c->frame_ready = 1;
    if (talker_set_pos(t, pos) != 0) goto fail;
    if (n_prev > 0) HCK(hipMemcpyAsync(t->smp_hist, prev_tokens, (size_t)n_prev * sizeof(int), hipMemcpyHostToDevice, t->st));
    t->h_pos[2] = (int)*seed;
    t->h_pos[3] = 0;
    HCK(hipMemcpyAsync(t->smp_seed, t->h_pos + 2, sizeof(uint32_t), hipMemcpyHostToDevice, t->st));
    HCK(hipMemcpyAsync(t->smp_done, t->h_pos + 3, sizeof(int), hipMemcpyHostToDevice, t->st));
    HCK(hipMemcpyAsync(t->gen_pad, tts_pad, (size_t)H * sizeof(float), hipMemcpyHostToDevice, t->st));
    memcpy(t->h_in, hidden0, (size_t)H * sizeof(float));
    HCK(hipMemcpyAsync(t->io, t->h_in, (size_t)H * sizeof(float), hipMemcpyHostToDevice, t->st));
    {
        const uint16_t *cpe[15];
        for (int g = 0; g < 15; g++) cpe[g] = c->cp_emb[g];
        const int expected = sp->text_len * 3, boost_start = expected * 2;
        for (int i = 0; i < n_frames; i++) {
            const int frame = frame0 + i;
            float boost = 0.0f;
            if (expected > 0 && frame > boost_start) {
                boost = 0.5f * (float)(frame - boost_start);
                if (boost > 10.0f) boost = 10.0f;
            }
            const int warm = sp->greedy_warmup > 0 && frame < sp->greedy_warmup;
            int *tok = t->smp_hist + n_prev + i;
            /* code0 from the last normed hidden state (io[0:H]) */
            HCK(qt_launch_mv(t->head_m.prec, QT_EPI_STORE, 0, t->io, NULL, t->s.eps, t->head_m.w, NULL, NULL,
                             t->head_m.rows, t->head_m.cols, t->logits, NULL, NULL, NULL, t->st));
            HCK(qt_launch_sample(t->logits, codec_vocab, 1, frame, boost, warm ? 0.0f : sp->temperature,
                                 warm ? 1 : sp->top_k, sp->top_p, sp->rep_penalty, t->smp_hist, n_prev + i, t->smp_seed,
                                 tok, t->smp_done, t->st));
            /* the CP frame for (hidden, code0) */
            HCK(qt_launch_copy_f32(t->io, c->th, H, t->st));
            HCK(hipMemcpyAsync(c->d_codes, tok, sizeof(int), hipMemcpyDeviceToDevice, t->st));
            HCK(cp_fused ? cp_rs_launch_on(c, t->st)
                         : graphs_enabled() ? hipGraphLaunch(c->fexec, t->st) : cp_frame_body_on(c, t->st));
            HCK(hipMemcpyAsync(t->gen_codes + (size_t)16 * i, c->d_codes, 16 * sizeof(int), hipMemcpyDeviceToDevice, t->st));
            /* next input, then the Talker step */
            float *xin = t->ps_on ? t->ps_xin : t->io + H;
            HCK(qt_launch_frame_embed(c->d_codes, codec_vocab, c->codebook, t->codec_emb, cpe, t->gen_pad, H, xin, t->st));
            if (t->ps_on) HCK(ps_launch(t, 1, 0));
            else HCK(talker_body(t));
        }
    }
    if (n_frames > 0)
        HCK(hipMemcpyAsync(codes_out, t->gen_codes, (size_t)n_frames * 16 * sizeof(int), hipMemcpyDeviceToHost, t->st));
    HCK(hipMemcpyAsync(t->h_pos + 2, t->smp_seed, sizeof(uint32_t), hipMemcpyDeviceToHost, t->st));
    HCK(hipMemcpyAsync(t->h_out, t->io, (size_t)2 * H * sizeof(float), hipMemcpyDeviceToHost, t->st));
    if (t->ps_on) HCK(hipMemcpyAsync(t->h_err, t->ps_err, sizeof(int), hipMemcpyDeviceToHost, t->st));
    if (cp_fused) HCK(hipMemcpyAsync(t->h_err + 1, c->rs_err, sizeof(int), hipMemcpyDeviceToHost, t->st));
    HCK(hipStreamSynchronize(t->st));
    if (t->ps_on && ps_check(t) != 0) goto fail;
    REQ(!cp_fused || t->h_err[1] == 0, "generate: the CP frame's wait for another workgroup's data timed out");
    *seed = (uint32_t)t->h_pos[2];
    if (hidden_out) memcpy(hidden_out, t->h_out, (size_t)H * sizeof(float));
    t->dev_pos = pos + n_frames;
    t->greedy_ready = 0;
    {
        int n_gen = n_frames;
        for (int i = 0; i < n_frames; i++)
            if (codes_out[(size_t)16 * i] == 2150) { n_gen = i; break; }
        return n_gen;
    }
fail:
    t->dead = 1; t->dev_pos = -1;
    return -1;
}

/* ---- batched steps: B streams over one state's resident weights -------------------- */
/* Twin of qwen_cuda_talker_batch_* / qwen_cuda_cp_batch_* (qwen_tts_cuda_talker.cu:595-648,
 * 879-915) and of the CPU batch_talker_step_impl (qwen_tts_talker.c:1192-1270): B
 * sequences, each at its own position pos_arr[b] (ragged), each with its own bf16 KV
 * cache; the weights are the single state's (never freed here), read ONCE per step for
 * all streams.  Per layer (int8 weights):
 *   pieces(RMSNorm(x)) -> MFMA QKV -> attention (q/k norm, RoPE, KV append, split-K over
 *   each stream's own length, B streams in one grid) -> pieces(attn) -> MFMA O + residual
 *   -> pieces(RMSNorm(x)) -> MFMA gate|up + SwiGLU -> pieces(h) -> MFMA down + residual,
 * captured once into a hipGraph (positions live on the device).  q4_0 weights take the
 * same pieces into qt_launch_bgemm_q4 (per-32-block integer sums, block scale in f32);
 * bf16 weights take the prefill's projection GEMM (three exact bf16 activation planes on
 * the bf16 MFMA, split K for the residual projections).  Every weight is read once per
 * step for all B streams in every precision. */

#define QWEN_HIP_BATCH_MAX 64

typedef struct {
    const stack_t *s;          /* borrowed weights / norms / rope tables */
    int B, Bp, kv_max, is_cp, attn_G;
    float *layer_out;          /* diagnostic (ungraphed steps only): every layer's x, [L][B][H] */
    hipStream_t st;
    uint16_t *kc, *vc;         /* [B][L][nkv][kv_max][hd] */
    float *x, *qkv, *attn, *h, *hid;
    int8_t *pc; float *ps;     /* activation pieces [Kmax/64][3*Bp][64], scales [Bp] */
    uint16_t *pf_p; float *pf_part; /* bf16: activation planes [3][64][Kmax], split-K partials (PF_PART_FLOATS) */
    int *g2_part; unsigned *g2_cnt; /* int8: split-K tiles and counters of qt_launch_bgemm2_i8 */
    int fold;                  /* int8: pieces made inside each projection launch (qt_launch_bgemm2_i8_px) */
    unsigned *px_sync;         /* in-launch pieces: count + per-workgroup go flags (128-byte lines), error word */
    int px_wgs;                /* workgroups px_sync has flags for */
    float *part; unsigned *cnt;
    int *d_pos;                /* [B] */
    float *h_io; int *h_pos;   /* pinned */
    hipGraphExec_t exec; int graph_ready, stepped;   /* stepped: a batch_step has run (inputs set) */
    int last_async;            /* steps replayed since the last batch_step */
    uint16_t *kv_stage;        /* [kv_max][n_kv*hd]: slot upload/download staging, made on first use */
    hpipe_t up;                /* pinned buffers of the slot upload */
    int dead;
} batch_t;

static void batch_destroy(batch_t *bt) {
    if (!bt) return;
    if (bt->graph_ready) (void)hipGraphExecDestroy(bt->exec);
    void *bufs[] = {bt->kc, bt->vc, bt->x, bt->qkv, bt->attn, bt->h, bt->hid, bt->pc, bt->ps, bt->part, bt->cnt, bt->d_pos,
                    bt->kv_stage, bt->pf_p, bt->pf_part, bt->g2_part, bt->g2_cnt, bt->px_sync};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) if (bufs[i]) (void)hipFree(bufs[i]);
    hpipe_free(&bt->up);
    if (bt->h_io) (void)hipHostFree(bt->h_io);
    if (bt->h_pos) (void)hipHostFree(bt->h_pos);
    if (bt->st) (void)hipStreamDestroy(bt->st);
    free(bt);
}

/* int8: every projection of the layer runs k_bgemm2_i8 and takes in-launch pieces */
static int batch_px_ok(const batch_t *bt) {
    const stack_t *s = bt->s;
    if (s->prec != QWEN_HIP_INT8 || !bt->px_sync) return 0;
    const int shp[4][2] = {{s->qd + 2 * s->kvd, s->H}, {s->H, s->qd}, {2 * s->F, s->H}, {s->H, s->F}};
    for (int i = 0; i < 4; i++) {
        int kb_, S_, rt_, nc; size_t pi;
        const int n = qt_bgemm2_px_wgs(shp[i][0], shp[i][1], bt->Bp);
        if (!qt_bgemm2_plan(shp[i][0], shp[i][1], bt->Bp, &kb_, &S_, &rt_, &pi, &nc) || (S_ > 1 && !bt->g2_part) ||
            n == 0 || n > bt->px_wgs) return 0;
    }
    return 1;
}

static batch_t *batch_create(const stack_t *s, int B, int is_cp) {
    batch_t *bt = calloc(1, sizeof *bt);
    if (!bt) { SETERR("out of host memory"); return NULL; }
    REQ(B >= 1 && B <= QWEN_HIP_BATCH_MAX, "batch size %d out of range (1..%d)", B, QWEN_HIP_BATCH_MAX);
    REQ(s->H % 64 == 0 && s->F % 64 == 0 && s->qd % 64 == 0, "batched step needs dims divisible by 64");
    bt->s = s; bt->B = B; bt->Bp = (B + 15) & ~15; bt->kv_max = s->kv_max; bt->is_cp = is_cp;
    HCK(hipStreamCreateWithFlags(&bt->st, hipStreamNonBlocking));
    const size_t per = (size_t)s->L * s->nkv * bt->kv_max * s->hd;
    const int K = s->F > s->H ? (s->F > s->qd ? s->F : s->qd) : (s->H > s->qd ? s->H : s->qd);
    HCK(hipMalloc((void **)&bt->kc, (size_t)B * per * 2));
    HCK(hipMalloc((void **)&bt->vc, (size_t)B * per * 2));
    HCK(hipMemsetAsync(bt->kc, 0, (size_t)B * per * 2, bt->st));
    HCK(hipMemsetAsync(bt->vc, 0, (size_t)B * per * 2, bt->st));
    HCK(hipMalloc((void **)&bt->x, (size_t)B * s->H * sizeof(float)));
    HCK(hipMalloc((void **)&bt->hid, (size_t)B * s->H * sizeof(float)));
    HCK(hipMalloc((void **)&bt->qkv, (size_t)B * (s->qd + 2 * s->kvd) * sizeof(float)));
    HCK(hipMalloc((void **)&bt->attn, (size_t)B * s->qd * sizeof(float)));
    HCK(hipMalloc((void **)&bt->h, (size_t)B * s->F * sizeof(float)));
    HCK(hipMalloc((void **)&bt->pc, (size_t)K * 3 * bt->Bp));
    HCK(hipMalloc((void **)&bt->ps, (size_t)bt->Bp * sizeof(float)));
    if (s->prec == QWEN_HIP_BF16) {
        HCK(hipMalloc((void **)&bt->pf_p, (size_t)3 * qt_pf_spad(B) * K * sizeof(uint16_t)));
        HCK(hipMalloc((void **)&bt->pf_part, (size_t)PF_PART_FLOATS * sizeof(float)));
    }
    if (s->prec == QWEN_HIP_INT8) {
        /* workspace of the largest split-K plan over the layer's four projections */
        const int shp[4][2] = {{s->qd + 2 * s->kvd, s->H}, {s->H, s->qd}, {2 * s->F, s->H}, {s->H, s->F}};
        size_t pmax = 0; int cmax = 0;
        for (int i = 0; i < 4; i++) {
            int kb_, S_, rt_, nc; size_t pi;
            if (qt_bgemm2_plan(shp[i][0], shp[i][1], bt->Bp, &kb_, &S_, &rt_, &pi, &nc)) {
                if (pi > pmax) pmax = pi;
                if (nc > cmax) cmax = nc;
            }
        }
        if (pmax) {
            HCK(hipMalloc((void **)&bt->g2_part, pmax * sizeof(int)));
            HCK(hipMalloc((void **)&bt->g2_cnt, (size_t)cmax * sizeof(unsigned)));
            HCK(hipMemsetAsync(bt->g2_cnt, 0, (size_t)cmax * sizeof(unsigned), bt->st));
        }
        for (int i = 0; i < 4; i++) {
            const int n = qt_bgemm2_px_wgs(shp[i][0], shp[i][1], bt->Bp);
            if (n > bt->px_wgs) bt->px_wgs = n;
        }
        const size_t words = (size_t)32 * (2 + bt->px_wgs);   /* count, flags, error word */
        HCK(hipMalloc((void **)&bt->px_sync, words * sizeof(unsigned)));
        HCK(hipMemsetAsync(bt->px_sync, 0, words * sizeof(unsigned), bt->st));
        bt->fold = batch_px_ok(bt);
    }
    bt->attn_G = s->attn_G;      /* its own: the single state's may change when its cache grows */
    HCK(hipMalloc((void **)&bt->part, (size_t)B * s->nkv * bt->attn_G * (s->nh / s->nkv) * 130 * sizeof(float)));
    HCK(hipMalloc((void **)&bt->cnt, (size_t)B * s->nkv * sizeof(unsigned)));
    HCK(hipMemsetAsync(bt->cnt, 0, (size_t)B * s->nkv * sizeof(unsigned), bt->st));
    HCK(hipMalloc((void **)&bt->d_pos, (size_t)B * sizeof(int)));
    HCK(hipHostMalloc((void **)&bt->h_io, (size_t)B * s->H * sizeof(float), hipHostMallocDefault));
    HCK(hipHostMalloc((void **)&bt->h_pos, (size_t)B * sizeof(int), hipHostMallocDefault));
    HCK(hipStreamSynchronize(bt->st));
    return bt;
fail:
    batch_destroy(bt);
    return NULL;
}

/* dst[b] = W . src[b] (+ epilogue) for the B streams.  Pieces of src (optionally
 * RMS-normalised with nw) are computed first on the int8 path. */
static hipError_t batch_proj(batch_t *bt, const dmat_t *m, int epi, const float *nw, const float *src, long long sstride,
                             float *dst, long long dstride) {
    const stack_t *s = bt->s;
    hipError_t e;
    if (m->prec == QWEN_HIP_BF16) {
        if ((e = qt_launch_pf_pieces(src, (int)sstride, bt->B, m->cols, nw, s->eps, bt->pf_p, bt->st))) return e;
        return qt_launch_pf_gemm(epi, (const uint16_t *)m->w, bt->pf_p, bt->B, m->rows, m->cols, dst, (int)dstride,
                                 bt->pf_part, PF_PART_FLOATS, bt->st);
    }
    if (m->prec == QWEN_HIP_INT8 && bt->fold)
        return qt_launch_bgemm2_i8_px(epi, m->w, m->scale, m->rows, m->cols, src, sstride, nw, s->eps, bt->pc, bt->ps,
                                      bt->B, bt->Bp, dst, dstride, bt->g2_part, bt->g2_cnt, bt->px_sync, bt->px_wgs,
                                      bt->px_sync + 32 * (1 + bt->px_wgs), bt->st);
    if ((e = qt_launch_bpieces(src, sstride, nw, s->eps, m->cols, bt->B, bt->Bp, bt->pc, bt->ps, bt->st))) return e;
    if (m->prec == QWEN_HIP_INT8) {
        int kb_, S_, rt_, nc; size_t pi;
        if (qt_bgemm2_plan(m->rows, m->cols, bt->Bp, &kb_, &S_, &rt_, &pi, &nc) && (S_ == 1 || bt->g2_part))
            return qt_launch_bgemm2_i8(epi, m->w, m->scale, m->rows, m->cols, bt->pc, bt->ps, bt->B, bt->Bp, dst, dstride,
                                       bt->g2_part, bt->g2_cnt, bt->st);
        return qt_launch_bgemm_i8(epi, m->w, m->scale, m->rows, m->cols, bt->pc, bt->ps, bt->B, bt->Bp, dst, dstride, bt->st);
    }
    return qt_launch_bgemm_q4(epi, m->w, m->s16, m->rows, m->cols, bt->pc, bt->ps, bt->B, bt->Bp, dst, dstride, bt->st);
}

static hipError_t batch_body(void *arg) {
    batch_t *bt = (batch_t *)arg;
    const stack_t *s = bt->s;
    hipError_t e;
    const float scale = 1.0f / sqrtf((float)s->hd);
    const int H = s->H, F = s->F, QKV = s->qd + 2 * s->kvd;
    const long long per = (long long)s->L * s->nkv * bt->kv_max * s->hd;
    /* bf16 weights: each reduce writes the next projection's input planes (the SwiGLU
     * output, the normed residual), so only layer 0's input and the attention output get a
     * plane kernel of their own */
    const int fused = s->prec == QWEN_HIP_BF16 && (long long)bt->B * 2 * F <= PF_PART_FLOATS;
    for (int l = 0; l < s->L; l++) {
        const size_t lay = (size_t)l * s->nkv * bt->kv_max * s->hd;
        if (fused) {
            if (l == 0 && (e = qt_launch_pf_pieces(bt->x, H, bt->B, H, s->in_norm[0], s->eps, bt->pf_p, bt->st))) return e;
            if ((e = qt_launch_pf_gemm(QT_PF_STORE, (const uint16_t *)s->qkv[l].w, bt->pf_p, bt->B, QKV, H, bt->qkv, QKV,
                                       bt->pf_part, PF_PART_FLOATS, bt->st))) return e;
        } else if ((e = batch_proj(bt, &s->qkv[l], QT_EPI_STORE, s->in_norm[l], bt->x, H, bt->qkv, QKV))) return e;
        if ((e = qt_launch_attn_b(bt->qkv, QKV, s->qn[l], s->kn[l], s->rope_cos, s->rope_sin, s->eps, bt->d_pos,
                                  bt->kc + lay, bt->vc + lay, per, s->hd, (long long)bt->kv_max * s->hd, s->nh, s->nkv,
                                  s->hd, scale, bt->part, (long long)s->nkv * bt->attn_G * (s->nh / s->nkv) * 130,
                                  bt->cnt, bt->attn_G, bt->attn, s->qd, bt->B, bt->st))) return e;
        if (fused) {
            if ((e = qt_launch_pf_pieces(bt->attn, s->qd, bt->B, s->qd, NULL, 0.f, bt->pf_p, bt->st))) return e;
            if ((e = qt_launch_pf_gemm_resid_planes((const uint16_t *)s->o[l].w, bt->pf_p, bt->B, H, s->qd, bt->x, H,
                                                    s->post_norm[l], s->eps, bt->pf_p, bt->pf_part, PF_PART_FLOATS,
                                                    bt->st))) return e;
            if ((e = qt_launch_pf_gemm_swiglu_planes((const uint16_t *)s->gu[l].w, bt->pf_p, bt->B, 2 * F, H, bt->pf_p,
                                                     bt->pf_part, PF_PART_FLOATS, bt->st))) return e;
            if (l + 1 < s->L)
                e = qt_launch_pf_gemm_resid_planes((const uint16_t *)s->dn[l].w, bt->pf_p, bt->B, H, F, bt->x, H,
                                                   s->in_norm[l + 1], s->eps, bt->pf_p, bt->pf_part, PF_PART_FLOATS, bt->st);
            else
                e = qt_launch_pf_gemm(QT_PF_RESID, (const uint16_t *)s->dn[l].w, bt->pf_p, bt->B, H, F, bt->x, H,
                                      bt->pf_part, PF_PART_FLOATS, bt->st);
            if (e) return e;
        } else {
            if ((e = batch_proj(bt, &s->o[l], QT_EPI_RESID, NULL, bt->attn, s->qd, bt->x, H))) return e;
            if ((e = batch_proj(bt, &s->gu[l], QT_EPI_SWIGLU, s->post_norm[l], bt->x, H, bt->h, F))) return e;
            if ((e = batch_proj(bt, &s->dn[l], QT_EPI_RESID, NULL, bt->h, F, bt->x, H))) return e;
        }
        if (bt->layer_out &&
            (e = hipMemcpyAsync(bt->layer_out + (size_t)l * bt->B * H, bt->x, (size_t)bt->B * H * sizeof(float),
                                hipMemcpyDeviceToDevice, bt->st))) return e;
    }
    if (bt->is_cp) return qt_launch_advance_pos(bt->d_pos, bt->B, bt->st);
    /* hid = final_norm(x) per stream, positions advanced by the same launch */
    return qt_launch_rmsnorm_rows_to(bt->x, bt->hid, s->final_norm, bt->B, H, s->eps, bt->d_pos, bt->st);
}

/* After a synchronisation: fails (and marks the state dead) if an in-launch pieces wait
 * gave up on the device. */
static int batch_check_err(batch_t *bt) {
    unsigned w = 0;
    if (!bt->px_sync) return 0;
    HCK(hipMemcpy(&w, bt->px_sync + 32 * (1 + bt->px_wgs), sizeof w, hipMemcpyDeviceToHost));
    REQ(w == 0, "batched step: a projection gave up waiting for its in-launch activation pieces");
    return 0;
fail:
    bt->dead = 1;
    return -1;
}

/* One batched step: x[b] <- in[b] (host), positions <- pos_arr, run, out[b] <- hid or x. */
static int batch_step_run(batch_t *bt, const float *in, const int *pos_arr, float *out, int use_graph) {
    if (!bt || bt->dead) { SETERR("batch state is dead or NULL"); return -1; }
    const stack_t *s = bt->s;
    const int B = bt->B, H = s->H;
    REQ(in && pos_arr, "null embeds / positions");
    for (int b = 0; b < B; b++)
        REQ(pos_arr[b] >= 0 && pos_arr[b] < bt->kv_max && pos_arr[b] < s->rope_len,
            "stream %d: pos %d out of range (kv_max %d, rope %d)", b, pos_arr[b], bt->kv_max, s->rope_len);
    memcpy(bt->h_io, in, (size_t)B * H * sizeof(float));
    memcpy(bt->h_pos, pos_arr, (size_t)B * sizeof(int));
    bt->last_async = 0;
    HCK(hipMemcpyAsync(bt->x, bt->h_io, (size_t)B * H * sizeof(float), hipMemcpyHostToDevice, bt->st));
    HCK(hipMemcpyAsync(bt->d_pos, bt->h_pos, (size_t)B * sizeof(int), hipMemcpyHostToDevice, bt->st));
    if (use_graph && graphs_enabled()) {
        if (!bt->graph_ready) {
            if (capture(bt->st, &bt->exec, batch_body, bt) != 0) goto fail;
            bt->graph_ready = 1;
        }
        HCK(hipGraphLaunch(bt->exec, bt->st));
    } else {
        HCK(batch_body(bt));
    }
    bt->stepped = 1;
    HCK(hipMemcpyAsync(bt->h_io, bt->is_cp ? bt->x : bt->hid, (size_t)B * H * sizeof(float), hipMemcpyDeviceToHost, bt->st));
    HCK(hipStreamSynchronize(bt->st));
    if (batch_check_err(bt)) return -1;
    if (out) memcpy(out, bt->h_io, (size_t)B * H * sizeof(float));
    return 0;
fail:
    if (bt) bt->dead = 1;
    return -1;
}

static int batch_step_impl(batch_t *bt, const float *in, const int *pos_arr, float *out) {
    return batch_step_run(bt, in, pos_arr, out, 1);
}

/* Diagnostic: one ungraphed batched step that also returns the residual x of every stream
 * after every layer (residuals host [L][B][H]).  Allocates a temporary device buffer. */
int qwen_hip_talker_batch_step_layers(void *state, const float *embeds, const int *pos_arr, float *residuals,
                                      float *hidden_out) {
    batch_t *bt = (batch_t *)state;
    float *tmp = NULL;
    if (!bt || bt->dead) { SETERR("batch state is dead or NULL"); return -1; }
    if (!residuals) { SETERR("null residuals"); return -1; }
    const size_t n = (size_t)bt->s->L * bt->B * bt->s->H;
    HCK(hipMalloc((void **)&tmp, n * sizeof(float)));
    bt->layer_out = tmp;
    const int rc = batch_step_run(bt, embeds, pos_arr, hidden_out, 0);
    bt->layer_out = NULL;
    if (rc == 0) {
        HCK(hipMemcpy(residuals, tmp, n * sizeof(float), hipMemcpyDeviceToHost));
    }
    (void)hipFree(tmp);
    return rc;
fail:
    bt->layer_out = NULL;
    if (tmp) (void)hipFree(tmp);
    return -1;
}

void *qwen_hip_talker_batch_init(void *single, int B) {
    talker_t *t = (talker_t *)single;
    if (!t || t->dead) { SETERR("batch init: single state is dead or NULL"); return NULL; }
    return batch_create(&t->s, B, 0);
}
int qwen_hip_talker_batch_step(void *state, const float *embeds, const int *pos_arr, float *hidden_out) {
    return batch_step_impl((batch_t *)state, embeds, pos_arr, hidden_out);
}
int qwen_hip_talker_batch_upload_slot(void *state, int b, const uint16_t *kv_k, const uint16_t *kv_v, int src_kv_max,
                                      int prefill_len) {
    batch_t *bt = (batch_t *)state;
    if (!bt || bt->dead) { SETERR("batch state is dead or NULL"); return -1; }
    const stack_t *s = bt->s;
    if (prefill_len <= 0) return 0;
    REQ(b >= 0 && b < bt->B, "slot %d out of range", b);
    REQ(kv_k && kv_v, "null KV");
    REQ(prefill_len <= bt->kv_max && prefill_len <= src_kv_max, "prefill_len %d exceeds kv_max", prefill_len);
    const size_t per = (size_t)s->L * s->nkv * bt->kv_max * s->hd;
    if (!bt->kv_stage) HCK(hipMalloc((void **)&bt->kv_stage, (size_t)bt->kv_max * s->kvd * sizeof(uint16_t)));
    for (int l = 0; l < s->L; l++) {
        const size_t dst = (size_t)b * per + (size_t)l * s->nkv * bt->kv_max * s->hd;
        const size_t src = (((size_t)b * s->L + l) * src_kv_max) * s->kvd;
        HCK(kv_xfer(bt->kc + dst, bt->kv_max, (uint16_t *)kv_k + src, prefill_len, s->nkv, s->hd, 1, bt->kv_stage, &bt->up, bt->st));
        HCK(kv_xfer(bt->vc + dst, bt->kv_max, (uint16_t *)kv_v + src, prefill_len, s->nkv, s->hd, 1, bt->kv_stage, &bt->up, bt->st));
    }
    HCK(hipStreamSynchronize(bt->st));
    return 0;
fail:
    return -1;
}
int qwen_hip_talker_batch_download_slot(void *state, int b, uint16_t *kv_k, uint16_t *kv_v, int dst_kv_max, int n) {
    batch_t *bt = (batch_t *)state;
    if (!bt) { SETERR("NULL batch state"); return -1; }
    const stack_t *s = bt->s;
    REQ(b >= 0 && b < bt->B, "slot %d out of range", b);
    REQ(n >= 0 && n <= bt->kv_max && n <= dst_kv_max, "n %d out of range", n);
    if (n == 0) return 0;
    const size_t per = (size_t)s->L * s->nkv * bt->kv_max * s->hd;
    REQ(kv_k && kv_v, "null KV");
    if (!bt->kv_stage) HCK(hipMalloc((void **)&bt->kv_stage, (size_t)bt->kv_max * s->kvd * sizeof(uint16_t)));
    for (int l = 0; l < s->L; l++) {
        const size_t src = (size_t)b * per + (size_t)l * s->nkv * bt->kv_max * s->hd;
        const size_t dst = (((size_t)b * s->L + l) * dst_kv_max) * s->kvd;
        HCK(kv_xfer(bt->kc + src, bt->kv_max, kv_k + dst, n, s->nkv, s->hd, 0, bt->kv_stage, NULL, bt->st));
        HCK(kv_xfer(bt->vc + src, bt->kv_max, kv_v + dst, n, s->nkv, s->hd, 0, bt->kv_stage, NULL, bt->st));
    }
    HCK(hipStreamSynchronize(bt->st));
    return 0;
fail:
    return -1;
}
/* Benchmark entry: n more batched steps replaying the last batch_step's inputs, every
 * stream advancing one position per step on the device, no host sync.  The caller
 * keeps max(pos) + n within kv_max. */
int qwen_hip_talker_batch_step_async(void *state, int n_steps) {
    batch_t *bt = (batch_t *)state;
    if (!bt || bt->dead || !bt->stepped) { SETERR("batch state not initialised by a batch_step call"); return -1; }
    int maxp = 0;
    for (int b = 0; b < bt->B; b++) if (bt->h_pos[b] > maxp) maxp = bt->h_pos[b];
    bt->last_async += n_steps;
    REQ(maxp + bt->last_async < bt->kv_max && maxp + bt->last_async < bt->s->rope_len,
        "replayed positions would pass kv_max %d", bt->kv_max);
    for (int i = 0; i < n_steps; i++) HCK(bt->graph_ready ? hipGraphLaunch(bt->exec, bt->st) : batch_body(bt));
    return 0;
fail:
    bt->dead = 1;
    return -1;
}
int qwen_hip_talker_batch_sync(void *state) {
    batch_t *bt = (batch_t *)state;
    if (!bt) return -1;
    HCK(hipStreamSynchronize(bt->st));
    return batch_check_err(bt);
fail:
    bt->dead = 1;
    return -1;
}
/* int8 projections: make the activation pieces inside each projection launch (on = 1,
 * the default where every projection shape allows it) or in a launch of their own (0).
 * The two give the same bytes; the switch is for tests and measurement.  Returns the
 * mode in effect, -1 on error. */
int qwen_hip_batch_fold_pieces(void *state, int on) {
    batch_t *bt = (batch_t *)state;
    if (!bt || bt->dead) { SETERR("batch state is dead or NULL"); return -1; }
    const int want = on && batch_px_ok(bt);
    if (want != bt->fold) {
        HCK(hipStreamSynchronize(bt->st));
        if (bt->graph_ready) { (void)hipGraphExecDestroy(bt->exec); bt->graph_ready = 0; }
        bt->fold = want;
    }
    return bt->fold;
fail:
    bt->dead = 1;
    return -1;
}
void *qwen_hip_talker_batch_stream(void *state) { return state ? (void *)((batch_t *)state)->st : NULL; }
void qwen_hip_talker_batch_free(void *state) { batch_destroy((batch_t *)state); }


/* CP batch twins (qwen_tts_cuda_talker.cu:879-915): x[B][cp_hidden] host residuals in
 * place, one 5-layer pass per stream at pos_arr[b] (each stream's own CP KV). */
void *qwen_hip_cp_batch_init(void *single, int B) {
    cp_t *c = (cp_t *)single;
    if (!c || c->dead) { SETERR("CP batch init: single state is dead or NULL"); return NULL; }
    return batch_create(&c->s, B, 1);
}
int qwen_hip_cp_batch_step(void *state, float *x, const int *pos_arr) {
    return batch_step_impl((batch_t *)state, x, pos_arr, x);
}
void qwen_hip_cp_batch_free(void *state) { batch_destroy((batch_t *)state); }

/* ---- level 1: per-op backend + kernel-API parity surface ----------------------------- */

typedef struct { const void *host; int rows, cols; dmat_t m; } wcache_t;
typedef struct {
    hipStream_t st;
    wcache_t *cache; int ncache, capcache;
} backend_t;

int qwen_hip_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n > 0;
}

void *qwen_hip_init(void) {
    backend_t *b = calloc(1, sizeof *b);
    if (!b) return NULL;
    if (!qwen_hip_available()) { SETERR("no HIP device"); free(b); return NULL; }
    if (hipStreamCreateWithFlags(&b->st, hipStreamNonBlocking) != hipSuccess) { SETERR("stream create failed"); free(b); return NULL; }
    return b;
}

void qwen_hip_free(void *ctx) {
    backend_t *b = (backend_t *)ctx;
    if (!b) return;
    for (int i = 0; i < b->ncache; i++) dmat_free(&b->cache[i].m);
    free(b->cache);
    (void)hipStreamDestroy(b->st);
    free(b);
}

static dmat_t *cached_bf16(backend_t *b, const uint16_t *W, int rows, int cols) {
    for (int i = 0; i < b->ncache; i++)
        if (b->cache[i].host == W && b->cache[i].rows == rows && b->cache[i].cols == cols) return &b->cache[i].m;
    if (b->ncache == b->capcache) {
        int nc = b->capcache ? 2 * b->capcache : 64;
        wcache_t *n = realloc(b->cache, (size_t)nc * sizeof *n);
        if (!n) return NULL;
        b->cache = n; b->capcache = nc;
    }
    wcache_t *e = &b->cache[b->ncache];
    qwen_hip_mat_t src = {W, NULL};
    if (dmat_alloc(&e->m, QWEN_HIP_BF16, rows, cols) != 0) return NULL;
    if (dmat_put(&e->m, 0, &src, QWEN_HIP_BF16, rows, b->st, NULL) != 0) { dmat_free(&e->m); return NULL; }
    e->host = W; e->rows = rows; e->cols = cols;
    b->ncache++;
    return &e->m;
}

void qwen_hip_matvec_bf16(void *ctx, float *y, const uint16_t *W, const float *x, int rows, int cols) {
    qwen_hip_matmat_bf16(ctx, y, W, x, rows, cols, 1);
}

void qwen_hip_matmat_bf16(void *ctx, float *Y, const uint16_t *W, const float *X, int rows, int cols, int B) {
    backend_t *b = (backend_t *)ctx;
    float *dx = NULL, *dy = NULL, *hx = NULL, *hy = NULL;
    uint16_t *dp = NULL;
    dmat_t *m;
    REQ(b && B >= 1 && B <= 64, "bad backend call");
    REQ((m = cached_bf16(b, W, rows, cols)) != NULL, "weight upload failed");
    HCK(hipMalloc((void **)&dx, (size_t)cols * B * sizeof(float)));
    HCK(hipMalloc((void **)&dy, (size_t)rows * B * sizeof(float)));
    hx = malloc((size_t)cols * B * sizeof(float)); hy = malloc((size_t)rows * B * sizeof(float));
    REQ(hx && hy, "host alloc");
    /* X is [cols][B] row-major: gather column b into a contiguous vector */
    for (int k = 0; k < cols; k++) for (int j = 0; j < B; j++) hx[(size_t)j * cols + k] = X[(size_t)k * B + j];
    HCK(hipMemcpyAsync(dx, hx, (size_t)cols * B * sizeof(float), hipMemcpyHostToDevice, b->st));
    if (rows % 64 == 0 && cols % 64 == 0) {
        /* weights read once for all B columns: exact bf16 planes of X on the bf16 MFMA */
        HCK(hipMalloc((void **)&dp, (size_t)3 * qt_pf_spad(B) * cols * sizeof(uint16_t)));
        HCK(qt_launch_pf_pieces(dx, cols, B, cols, NULL, 0.f, dp, b->st));
        HCK(qt_launch_pf_gemm(QT_PF_STORE, (const uint16_t *)m->w, dp, B, rows, cols, dy, rows, NULL, 0, b->st));
    } else {
        for (int j = 0; j < B; j++)
            HCK(mv(m, QT_EPI_STORE, 0, dx + (size_t)j * cols, NULL, 0.f, dy + (size_t)j * rows, NULL, NULL, b->st));
    }
    HCK(hipMemcpyAsync(hy, dy, (size_t)rows * B * sizeof(float), hipMemcpyDeviceToHost, b->st));
    HCK(hipStreamSynchronize(b->st));
    for (int r = 0; r < rows; r++) for (int j = 0; j < B; j++) Y[(size_t)r * B + j] = hy[(size_t)j * rows + r];
fail:
    if (dx) (void)hipFree(dx);
    if (dy) (void)hipFree(dy);
    if (dp) (void)hipFree(dp);
    free(hx); free(hy);
}

/* a private stream for the one-shot op entry points */
static hipStream_t op_stream(void) {
    static hipStream_t s = NULL;
    if (!s && hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) s = NULL;
    return s;
}

static int op_matvec(int prec, float *y, const void *W, const float *scale, const float *x, int rows, int cols) {
    hipStream_t st = op_stream();
    dmat_t m; memset(&m, 0, sizeof m);
    float *dx = NULL, *dy = NULL; void *tmp = NULL;
    qwen_hip_mat_t src = {W, scale};
    REQ(st, "no stream");
    REQ(rows > 0 && cols > 0, "bad shape");
    REQ(dmat_alloc(&m, prec, rows, cols) == 0, "alloc");
    if (prec == QWEN_HIP_Q4_0) HCK(hipMalloc(&tmp, (size_t)rows * (cols / 32) * 18 + 16));
    REQ(dmat_put(&m, 0, &src, prec, rows, st, tmp) == 0, "upload");
    HCK(hipMalloc((void **)&dx, (size_t)cols * sizeof(float)));
    HCK(hipMalloc((void **)&dy, (size_t)rows * sizeof(float)));
    HCK(hipMemcpyAsync(dx, x, (size_t)cols * sizeof(float), hipMemcpyHostToDevice, st));
    HCK(mv(&m, QT_EPI_STORE, 0, dx, NULL, 0.f, dy, NULL, NULL, st));
    HCK(hipMemcpyAsync(y, dy, (size_t)rows * sizeof(float), hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    dmat_free(&m); (void)hipFree(dx); (void)hipFree(dy); if (tmp) (void)hipFree(tmp);
    return 0;
fail:
    dmat_free(&m); if (dx) (void)hipFree(dx); if (dy) (void)hipFree(dy); if (tmp) (void)hipFree(tmp);
    return -1;
}

/* Y[rows][B] = W @ X[cols][B] (row-major f32, B <= 64, cols a multiple of 64) on the
 * batched MFMA kernels: exact int8 activation pieces against int8 (qt_launch_bgemm_i8) or
 * q4_0 (qt_launch_bgemm_q4) weights, each weight read once for all B columns. */
static int op_matmat(int prec, float *Y, const void *W, const float *scale, const float *X, int rows, int cols, int B) {
    hipStream_t st = op_stream();
    dmat_t m; memset(&m, 0, sizeof m);
    float *dx = NULL, *dy = NULL, *hx = NULL, *hy = NULL, *ps = NULL;
    int8_t *pc = NULL; void *tmp = NULL;
    int *g2p = NULL; unsigned *g2c = NULL;
    qwen_hip_mat_t src = {W, scale};
    const int Bp = (B + 15) & ~15;
    REQ(st, "no stream");
    REQ(rows > 0 && cols > 0 && cols % 64 == 0 && cols <= 8192, "bad shape %dx%d (cols: multiple of 64, <= 8192)", rows, cols);
    REQ(B >= 1 && B <= 64, "B %d out of range (1..64)", B);
    REQ(dmat_alloc(&m, prec, rows, cols) == 0, "alloc");
    if (prec == QWEN_HIP_Q4_0) HCK(hipMalloc(&tmp, (size_t)rows * (cols / 32) * 18 + 16));
    REQ(dmat_put(&m, 0, &src, prec, rows, st, tmp) == 0, "upload");
    hx = malloc((size_t)B * cols * sizeof(float)); hy = malloc((size_t)B * rows * sizeof(float));
    REQ(hx && hy, "host alloc");
    for (int k = 0; k < cols; k++) for (int j = 0; j < B; j++) hx[(size_t)j * cols + k] = X[(size_t)k * B + j];
    HCK(hipMalloc((void **)&dx, (size_t)B * cols * sizeof(float)));
    HCK(hipMalloc((void **)&dy, (size_t)B * rows * sizeof(float)));
    HCK(hipMalloc((void **)&pc, (size_t)cols * 3 * Bp));
    HCK(hipMalloc((void **)&ps, (size_t)Bp * sizeof(float)));
    HCK(hipMemcpyAsync(dx, hx, (size_t)B * cols * sizeof(float), hipMemcpyHostToDevice, st));
    HCK(qt_launch_bpieces(dx, cols, NULL, 0.f, cols, B, Bp, pc, ps, st));
    if (prec == QWEN_HIP_INT8) {
        int kb_, S_, rt_, nc; size_t pi;
        if (qt_bgemm2_plan(rows, cols, Bp, &kb_, &S_, &rt_, &pi, &nc)) {
            if (pi) {
                HCK(hipMalloc((void **)&g2p, pi * sizeof(int)));
                HCK(hipMalloc((void **)&g2c, (size_t)nc * sizeof(unsigned)));
                HCK(hipMemsetAsync(g2c, 0, (size_t)nc * sizeof(unsigned), st));
            }
            HCK(qt_launch_bgemm2_i8(QT_EPI_STORE, m.w, m.scale, rows, cols, pc, ps, B, Bp, dy, rows, g2p, g2c, st));
        } else {
            HCK(qt_launch_bgemm_i8(QT_EPI_STORE, m.w, m.scale, rows, cols, pc, ps, B, Bp, dy, rows, st));
        }
    } else
        HCK(qt_launch_bgemm_q4(QT_EPI_STORE, m.w, m.s16, rows, cols, pc, ps, B, Bp, dy, rows, st));
    HCK(hipMemcpyAsync(hy, dy, (size_t)B * rows * sizeof(float), hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    for (int r = 0; r < rows; r++) for (int j = 0; j < B; j++) Y[(size_t)r * B + j] = hy[(size_t)j * rows + r];
    dmat_free(&m); (void)hipFree(dx); (void)hipFree(dy); (void)hipFree(pc); (void)hipFree(ps);
    if (tmp) (void)hipFree(tmp);
    if (g2p) (void)hipFree(g2p);
    if (g2c) (void)hipFree(g2c);
    free(hx); free(hy);
    return 0;
fail:
    dmat_free(&m);
    if (dx) (void)hipFree(dx);
    if (dy) (void)hipFree(dy);
    if (pc) (void)hipFree(pc);
    if (ps) (void)hipFree(ps);
    if (tmp) (void)hipFree(tmp);
    if (g2p) (void)hipFree(g2p);
    if (g2c) (void)hipFree(g2c);
    free(hx); free(hy);
    return -1;
}

/* qwen_matmat_int8 (qwen_tts_kernels.h:121-122): Y[rows][B] = (W*scale) @ X[cols][B]. */
int qwen_hip_op_matmat_int8(float *Y, const int8_t *W, const float *scale, const float *X, int rows, int cols, int B) {
    return op_matmat(QWEN_HIP_INT8, Y, W, scale, X, rows, cols, B);
}
/* qwen_matmat_q4_0 (qwen_tts_kernels.h:226-227): Y[rows][B] = dequant(W) @ X[cols][B]. */
int qwen_hip_op_matmat_q4_0(float *Y, const void *W, const float *X, int rows, int cols, int B) {
    return op_matmat(QWEN_HIP_Q4_0, Y, W, NULL, X, rows, cols, B);
}

int qwen_hip_op_matvec_bf16(float *y, const uint16_t *W, const float *x, int rows, int cols) {
    return op_matvec(QWEN_HIP_BF16, y, W, NULL, x, rows, cols);
}
int qwen_hip_op_matvec_int8(float *y, const int8_t *W, const float *scale, const float *x, int rows, int cols) {
    return op_matvec(QWEN_HIP_INT8, y, W, scale, x, rows, cols);
}
int qwen_hip_op_matvec_q4_0(float *y, const void *W, const float *x, int rows, int cols) {
    if (cols % 32) { SETERR("q4_0 needs cols %% 32 == 0"); return -1; }
    return op_matvec(QWEN_HIP_Q4_0, y, W, NULL, x, rows, cols);
}

int qwen_hip_op_argmax_matvec(int prec, const float *x, const void *W, const float *scale, int in_dim, int out_dim) {
    hipStream_t st = op_stream();
    dmat_t m; memset(&m, 0, sizeof m);
    float *dx = NULL, *dy = NULL; int *dt = NULL; void *tmp = NULL; int tok = -1;
    qwen_hip_mat_t src = {W, scale};
    REQ(st, "no stream");
    REQ(dmat_alloc(&m, prec, out_dim, in_dim) == 0, "alloc");
    if (prec == QWEN_HIP_Q4_0) HCK(hipMalloc(&tmp, (size_t)out_dim * (in_dim / 32) * 18 + 16));
    REQ(dmat_put(&m, 0, &src, prec, out_dim, st, tmp) == 0, "upload");
    HCK(hipMalloc((void **)&dx, (size_t)in_dim * sizeof(float)));
    HCK(hipMalloc((void **)&dy, (size_t)out_dim * sizeof(float)));
    HCK(hipMalloc((void **)&dt, sizeof(int)));
    HCK(hipMemcpyAsync(dx, x, (size_t)in_dim * sizeof(float), hipMemcpyHostToDevice, st));
    HCK(mv(&m, QT_EPI_STORE, 0, dx, NULL, 0.f, dy, NULL, NULL, st));
    HCK(qt_launch_select(dy, out_dim, 0, NULL, 0, dt, NULL, 0, NULL, 0, NULL, NULL, st));
    HCK(hipMemcpyAsync(&tok, dt, sizeof(int), hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
fail:
    dmat_free(&m); if (dx) (void)hipFree(dx); if (dy) (void)hipFree(dy); if (dt) (void)hipFree(dt);
    if (tmp) (void)hipFree(tmp);
    return tok;
}

/* Sampling (qwen_tts_sampling.c:160-202, optionally behind the codec-head rule of
 * qwen_tts.c:1652-1679) on the op stream: logits, history and LCG state up, token and
 * state back. */
static int op_sample(int rule, int frame, float eos_boost, const float *logits, int vocab, float temp, int top_k,
                     float top_p, float rep, const int *prev, int n_prev, uint32_t *seed) {
    hipStream_t st = op_stream();
    float *dl = NULL; int *dp = NULL, *dt = NULL; uint32_t *ds = NULL; int tok = -1, out = -1;
    REQ(st, "no stream");
    REQ(logits && seed && vocab > 0 && vocab <= 4096, "sampling needs logits, a seed and 1 <= vocab <= 4096");
    REQ(n_prev >= 0 && (n_prev == 0 || prev), "n_prev > 0 needs prev_tokens");
    HCK(hipMalloc((void **)&dl, (size_t)vocab * sizeof(float)));
    HCK(hipMalloc((void **)&dt, sizeof(int)));
    HCK(hipMalloc((void **)&ds, sizeof(uint32_t)));
    if (n_prev > 0) {
        HCK(hipMalloc((void **)&dp, (size_t)n_prev * sizeof(int)));
        HCK(hipMemcpyAsync(dp, prev, (size_t)n_prev * sizeof(int), hipMemcpyHostToDevice, st));
    }
    HCK(hipMemcpyAsync(dl, logits, (size_t)vocab * sizeof(float), hipMemcpyHostToDevice, st));
    HCK(hipMemcpyAsync(ds, seed, sizeof(uint32_t), hipMemcpyHostToDevice, st));
    HCK(qt_launch_sample(dl, vocab, rule, frame, eos_boost, temp, top_k, top_p, rep, dp, n_prev, ds, dt, NULL, st));
    HCK(hipMemcpyAsync(&tok, dt, sizeof(int), hipMemcpyDeviceToHost, st));
    HCK(hipMemcpyAsync(seed, ds, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    out = tok;
fail:
    if (dl) (void)hipFree(dl);
    if (dp) (void)hipFree(dp);
    if (dt) (void)hipFree(dt);
    if (ds) (void)hipFree(ds);
    return out;
}
int qwen_hip_op_sample(const float *logits, int vocab, float temp, int top_k, float top_p, float rep_penalty,
                       const int *prev_tokens, int n_prev, uint32_t *seed) {
    return op_sample(0, 0, 0.f, logits, vocab, temp, top_k, top_p, rep_penalty, prev_tokens, n_prev, seed);
}
int qwen_hip_op_codec_sample(const float *logits, int vocab, int frame, float eos_boost, float temp, int top_k,
                             float top_p, float rep_penalty, const int *prev_tokens, int n_prev, uint32_t *seed) {
    return op_sample(1, frame, eos_boost, logits, vocab, temp, top_k, top_p, rep_penalty, prev_tokens, n_prev, seed);
}

int qwen_hip_op_causal_attention_bf16kv(float *out, const float *Q, const uint16_t *K, const uint16_t *V,
                                        int seq_q, int seq_k, int n_heads, int n_kv_heads, int head_dim,
                                        float scale, int q_offset) {
    hipStream_t st = op_stream();
    float *dq = NULL, *dout = NULL, *part = NULL; uint16_t *dk = NULL, *dv = NULL; unsigned *cnt = NULL;
    REQ(st, "no stream");
    REQ(head_dim == 128 && seq_q > 0 && seq_k > 0 && n_kv_heads > 0, "unsupported attention shape");
    const int qh = n_heads * head_dim, kvd = n_kv_heads * head_dim;
    const int G = qt_attn_grid(seq_k);
    const int hpk = n_heads / n_kv_heads;
    REQ(G > 0, "seq_k %d exceeds the split-K grid (8192 keys)", seq_k);
    HCK(hipMalloc((void **)&dq, (size_t)seq_q * qh * sizeof(float)));
    HCK(hipMalloc((void **)&dout, (size_t)seq_q * qh * sizeof(float)));
    HCK(hipMalloc((void **)&dk, (size_t)seq_k * kvd * 2));
    HCK(hipMalloc((void **)&dv, (size_t)seq_k * kvd * 2));
    HCK(hipMalloc((void **)&part, (size_t)n_kv_heads * G * hpk * 130 * sizeof(float)));
    HCK(hipMalloc((void **)&cnt, (size_t)n_kv_heads * sizeof(unsigned)));
    HCK(hipMemsetAsync(cnt, 0, (size_t)n_kv_heads * sizeof(unsigned), st));
    HCK(hipMemcpyAsync(dq, Q, (size_t)seq_q * qh * sizeof(float), hipMemcpyHostToDevice, st));
    HCK(hipMemcpyAsync(dk, K, (size_t)seq_k * kvd * 2, hipMemcpyHostToDevice, st));
    HCK(hipMemcpyAsync(dv, V, (size_t)seq_k * kvd * 2, hipMemcpyHostToDevice, st));
    for (int i = 0; i < seq_q; i++) {
        int k_end = q_offset + i + 1;
        if (k_end > seq_k) k_end = seq_k;
        if (k_end <= 0) {
            HCK(hipMemsetAsync(dout + (size_t)i * qh, 0, (size_t)qh * sizeof(float), st));
            continue;
        }
        HCK(qt_launch_attn(0, dq + (size_t)i * qh, NULL, NULL, NULL, NULL, 0.f, NULL, k_end, dk, dv, kvd, head_dim,
                           n_heads, n_kv_heads, head_dim, scale, part, cnt, G, dout + (size_t)i * qh, st));
    }
    HCK(hipMemcpyAsync(out, dout, (size_t)seq_q * qh * sizeof(float), hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    (void)hipFree(dq); (void)hipFree(dout); (void)hipFree(dk); (void)hipFree(dv); (void)hipFree(part); (void)hipFree(cnt);
    return 0;
fail:
    if (dq) (void)hipFree(dq);
    if (dout) (void)hipFree(dout);
    if (dk) (void)hipFree(dk);
    if (dv) (void)hipFree(dv);
    if (part) (void)hipFree(part);
    if (cnt) (void)hipFree(cnt);
    return -1;
}

int qwen_hip_op_rms_norm(float *out, const float *x, const float *w, int seq, int dim, float eps) {
    hipStream_t st = op_stream();
    float *dx = NULL, *dw = NULL, *dout = NULL;
    REQ(st && seq > 0 && dim > 0, "bad args");
    HCK(hipMalloc((void **)&dx, (size_t)seq * dim * sizeof(float)));
    HCK(hipMalloc((void **)&dout, (size_t)seq * dim * sizeof(float)));
    HCK(hipMalloc((void **)&dw, (size_t)dim * sizeof(float)));
    HCK(hipMemcpyAsync(dx, x, (size_t)seq * dim * sizeof(float), hipMemcpyHostToDevice, st));
    HCK(hipMemcpyAsync(dw, w, (size_t)dim * sizeof(float), hipMemcpyHostToDevice, st));
    for (int s = 0; s < seq; s++)
        HCK(qt_launch_rmsnorm(dx + (size_t)s * dim, dw, dout + (size_t)s * dim, dim, eps, NULL, st));
    HCK(hipMemcpyAsync(out, dout, (size_t)seq * dim * sizeof(float), hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    (void)hipFree(dx); (void)hipFree(dout); (void)hipFree(dw);
    return 0;
fail:
    if (dx) (void)hipFree(dx);
    if (dout) (void)hipFree(dout);
    if (dw) (void)hipFree(dw);
    return -1;
}

int qwen_hip_op_rms_norm_per_head(float *x, const float *w, int seq, int n_heads, int head_dim, float eps) {
    hipStream_t st = op_stream();
    float *dx = NULL, *dw = NULL;
    const size_t n = (size_t)seq * n_heads * head_dim;
    REQ(st && seq > 0 && n_heads > 0 && head_dim > 0, "bad args");
    HCK(hipMalloc((void **)&dx, n * sizeof(float)));
    HCK(hipMalloc((void **)&dw, (size_t)head_dim * sizeof(float)));
    HCK(hipMemcpyAsync(dx, x, n * sizeof(float), hipMemcpyHostToDevice, st));
    HCK(hipMemcpyAsync(dw, w, (size_t)head_dim * sizeof(float), hipMemcpyHostToDevice, st));
    HCK(qt_launch_rmsnorm_rows(dx, dw, seq * n_heads, head_dim, eps, st));
    HCK(hipMemcpyAsync(x, dx, n * sizeof(float), hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    (void)hipFree(dx); (void)hipFree(dw);
    return 0;
fail:
    if (dx) (void)hipFree(dx);
    if (dw) (void)hipFree(dw);
    return -1;
}

/* The prefill projection on its own: Y[S][N] = X[S][K] . W[N][K]^T (epi 0), Y += (epi 1),
 * or SwiGLU of the interleaved rows into Y[S][N/2] (epi 2); host pointers, W bf16. */
int qwen_hip_op_prefill_gemm(float *Y, const uint16_t *W, const float *X, int S, int N, int K, int epi) {
    hipStream_t st = op_stream();
    uint16_t *dw = NULL, *dp = NULL;
    float *dx = NULL, *dy = NULL, *dpart = NULL;
    REQ(st, "no stream");
    REQ(S >= 1 && N >= 64 && K >= 64 && N % 64 == 0 && K % 64 == 0 && epi >= 0 && epi <= 2, "bad shape/epi");
    const int ny = epi == QT_PF_SWIGLU ? N / 2 : N;
    HCK(hipMalloc((void **)&dw, (size_t)N * K * 2));
    HCK(hipMalloc((void **)&dx, (size_t)S * K * sizeof(float)));
    HCK(hipMalloc((void **)&dy, (size_t)S * ny * sizeof(float)));
    HCK(hipMalloc((void **)&dp, (size_t)3 * qt_pf_spad(S) * K * 2));
    HCK(hipMalloc((void **)&dpart, (size_t)4 * S * N * sizeof(float)));
    HCK(hipMemcpyAsync(dw, W, (size_t)N * K * 2, hipMemcpyHostToDevice, st));
    HCK(hipMemcpyAsync(dx, X, (size_t)S * K * sizeof(float), hipMemcpyHostToDevice, st));
    if (epi == QT_PF_RESID) HCK(hipMemcpyAsync(dy, Y, (size_t)S * ny * sizeof(float), hipMemcpyHostToDevice, st));
    HCK(qt_launch_pf_pieces(dx, K, S, K, NULL, 0.f, dp, st));
    HCK(qt_launch_pf_gemm(epi, dw, dp, S, N, K, dy, ny, dpart, 4LL * S * N, st));
    HCK(hipMemcpyAsync(Y, dy, (size_t)S * ny * sizeof(float), hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    (void)hipFree(dw); (void)hipFree(dx); (void)hipFree(dy); (void)hipFree(dp); (void)hipFree(dpart);
    return 0;
fail:
    if (dpart) (void)hipFree(dpart);
    if (dw) (void)hipFree(dw);
    if (dx) (void)hipFree(dx);
    if (dy) (void)hipFree(dy);
    if (dp) (void)hipFree(dp);
    return -1;
}

/* The prefill's causal attention alone: out[S][nh*128] from QKV host f32[S][(nh+2nkv)*128]
 * (q | k | v rows as the prefill holds them after norm and RoPE). */
int qwen_hip_op_prefill_attention(float *out, const float *QKV, int S, int nh, int nkv, float scale) {
    hipStream_t st = op_stream();
    float *dq = NULL, *dout = NULL;
    REQ(st && S >= 1 && nh > 0 && nkv > 0 && nh % nkv == 0, "bad args");
    const int ld = (nh + 2 * nkv) * 128;
    HCK(hipMalloc((void **)&dq, (size_t)S * ld * sizeof(float)));
    HCK(hipMalloc((void **)&dout, (size_t)S * nh * 128 * sizeof(float)));
    HCK(hipMemcpyAsync(dq, QKV, (size_t)S * ld * sizeof(float), hipMemcpyHostToDevice, st));
    HCK(qt_launch_pf_attn(dq, ld, S, nh, nkv, scale, dout, nh * 128, st));
    HCK(hipMemcpyAsync(out, dout, (size_t)S * nh * 128 * sizeof(float), hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    (void)hipFree(dq); (void)hipFree(dout);
    return 0;
fail:
    if (dq) (void)hipFree(dq);
    if (dout) (void)hipFree(dout);
    return -1;
}

int qwen_hip_op_swiglu(float *out, const float *gate_up, int n) {
    hipStream_t st = op_stream();
    float *dg = NULL, *dout = NULL;
    REQ(st && n > 0, "bad args");
    HCK(hipMalloc((void **)&dg, (size_t)2 * n * sizeof(float)));
    HCK(hipMalloc((void **)&dout, (size_t)n * sizeof(float)));
    HCK(hipMemcpyAsync(dg, gate_up, (size_t)2 * n * sizeof(float), hipMemcpyHostToDevice, st));
    HCK(qt_launch_swiglu(dg, dout, n, st));
    HCK(hipMemcpyAsync(out, dout, (size_t)n * sizeof(float), hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    (void)hipFree(dg); (void)hipFree(dout);
    return 0;
fail:
    if (dg) (void)hipFree(dg);
    if (dout) (void)hipFree(dout);
    return -1;
}

int qwen_hip_op_quantize_int8(const uint16_t *src, int rows, int cols, int8_t *dst, float *scale) {
    hipStream_t st = op_stream();
    uint16_t *ds = NULL; uint8_t *dq = NULL; float *dsc = NULL;
    REQ(st && rows > 0 && cols > 0, "bad args");
    HCK(hipMalloc((void **)&ds, (size_t)rows * cols * 2));
    HCK(hipMalloc((void **)&dq, (size_t)rows * cols));
    HCK(hipMalloc((void **)&dsc, (size_t)rows * sizeof(float)));
    HCK(hipMemcpyAsync(ds, src, (size_t)rows * cols * 2, hipMemcpyHostToDevice, st));
    HCK(qt_launch_quant_int8(ds, rows, cols, dq, dsc, st));
    HCK(hipMemcpyAsync(dst, dq, (size_t)rows * cols, hipMemcpyDeviceToHost, st));
    HCK(hipMemcpyAsync(scale, dsc, (size_t)rows * sizeof(float), hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    (void)hipFree(ds); (void)hipFree(dq); (void)hipFree(dsc);
    return 0;
fail:
    if (ds) (void)hipFree(ds);
    if (dq) (void)hipFree(dq);
    if (dsc) (void)hipFree(dsc);
    return -1;
}

int qwen_hip_op_quantize_q4_0(const uint16_t *src, int rows, int cols, void *dst_blocks) {
    hipStream_t st = op_stream();
    uint16_t *ds = NULL, *s16 = NULL; uint8_t *qs = NULL, *hq = NULL; uint16_t *hs = NULL;
    const size_t nb = (size_t)rows * (cols / 32);
    REQ(st && rows > 0 && cols > 0 && cols % 32 == 0, "bad args");
    HCK(hipMalloc((void **)&ds, (size_t)rows * cols * 2));
    HCK(hipMalloc((void **)&qs, nb * 16));
    HCK(hipMalloc((void **)&s16, nb * 2));
    HCK(hipMemcpyAsync(ds, src, (size_t)rows * cols * 2, hipMemcpyHostToDevice, st));
    HCK(qt_launch_quant_q4(ds, rows, cols, qs, s16, st));
    hq = malloc(nb * 16); hs = malloc(nb * 2);
    REQ(hq && hs, "host alloc");
    HCK(hipMemcpyAsync(hq, qs, nb * 16, hipMemcpyDeviceToHost, st));
    HCK(hipMemcpyAsync(hs, s16, nb * 2, hipMemcpyDeviceToHost, st));
    HCK(hipStreamSynchronize(st));
    for (size_t b = 0; b < nb; b++) {
        uint8_t *o = (uint8_t *)dst_blocks + b * 18;
        o[0] = (uint8_t)(hs[b] & 0xFF); o[1] = (uint8_t)(hs[b] >> 8);
        memcpy(o + 2, hq + b * 16, 16);
    }
    free(hq); free(hs);
    (void)hipFree(ds); (void)hipFree(qs); (void)hipFree(s16);
    return 0;
fail:
    free(hq); free(hs);
    if (ds) (void)hipFree(ds);
    if (qs) (void)hipFree(qs);
    if (s16) (void)hipFree(s16);
    return -1;
}
