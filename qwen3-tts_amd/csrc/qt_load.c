/*
 * qt_load.c — the Talker's weights straight from the model file to the device.
 *
 * The reference maps model.safetensors (ingot's mmap loader, qwen_tts_talker.c:105-122,
 * third_party/ingot/src/safetensors.c), keeps the bf16 matrices in host memory, builds
 * the fused gate|up matrix on the host (qwen_tts_talker.c:378-388) and quantizes on the
 * host (qwen_tts_talker.c:286-317).  Here the file's bytes go to device memory through two
 * pinned staging buffers (pread of the next chunk while the previous one is copied), the
 * gate|up interleave runs on the device, and the state is built by qwen_hip_talker_init
 * from those device copies (which also quantizes on the device when asked): no host copy
 * of the model is made.
 *
 * safetensors: 8-byte little-endian header length N, N bytes of JSON
 *   {"__metadata__": {...}, "<name>": {"dtype": "BF16", "shape": [r, c],
 *    "data_offsets": [begin, end]}, ...}
 * then the data; offsets are relative to byte 8 + N.  The scanner below reads exactly that
 * shape of JSON (objects, arrays, strings with escapes, integers); every tensor the step
 * needs is looked up and checked (dtype, shape, extent within the file) before any GPU
 * call, so a malformed or mismatched file fails with a message and nothing allocated.
 */
#define _GNU_SOURCE
#include "qwen_tts_hip.h"
#include "qt_launch.h"

#include <hip/hip_runtime_api.h>
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

enum { ST_BF16 = 0, ST_F32 = 1, ST_F16 = 2, ST_OTHER = 3 };

typedef struct {
    char *name;
    int dtype, ndim;
    long long shape[4];
    unsigned long long off0, off1;     /* relative to the data start */
} st_tensor_t;

typedef struct {
    int fd;
    unsigned long long data_start, file_size;
    int n, cap;
    st_tensor_t *t;
} st_file_t;

/* ---- JSON scanning ---------------------------------------------------------------------- */

typedef struct { const char *p, *end; } scan_t;

static void sk_ws(scan_t *s) { while (s->p < s->end && (*s->p == ' ' || *s->p == '\n' || *s->p == '\r' || *s->p == '\t')) s->p++; }
static int sk_ch(scan_t *s, char c) { sk_ws(s); if (s->p < s->end && *s->p == c) { s->p++; return 1; } return 0; }

/* a string into a fresh buffer (escapes \" \\ \/ kept as the character; \uXXXX refused) */
static char *sk_str(scan_t *s) {
    sk_ws(s);
    if (s->p >= s->end || *s->p != '"') return NULL;
    s->p++;
    const char *b = s->p;
    size_t n = 0;
    for (const char *q = b; q < s->end && *q != '"'; q++, n++) if (*q == '\\') q++;
    char *out = (char *)malloc(n + 1);
    if (!out) return NULL;
    size_t k = 0;
    while (s->p < s->end && *s->p != '"') {
        if (*s->p == '\\') {
            s->p++;
            if (s->p >= s->end || *s->p == 'u') { free(out); return NULL; }
        }
        out[k++] = *s->p++;
    }
    if (s->p >= s->end) { free(out); return NULL; }
    s->p++;
    out[k] = 0;
    return out;
}

static int sk_int(scan_t *s, long long *v) {
    sk_ws(s);
    char *e = NULL;
    errno = 0;
    long long x = strtoll(s->p, &e, 10);
    if (e == s->p || errno) return -1;
    s->p = e;
    *v = x;
    return 0;
}

/* skip one JSON value of any kind */
static int sk_skip(scan_t *s) {
    sk_ws(s);
    if (s->p >= s->end) return -1;
    char c = *s->p;
    if (c == '"') { char *t = sk_str(s); if (!t) return -1; free(t); return 0; }
    if (c == '{' || c == '[') {
        const char close = c == '{' ? '}' : ']';
        s->p++;
        if (sk_ch(s, close)) return 0;
        for (;;) {
            if (c == '{') { char *k = sk_str(s); if (!k) return -1; free(k); if (!sk_ch(s, ':')) return -1; }
            if (sk_skip(s)) return -1;
            if (sk_ch(s, ',')) continue;
            return sk_ch(s, close) ? 0 : -1;
        }
    }
    while (s->p < s->end && *s->p != ',' && *s->p != '}' && *s->p != ']') s->p++;   /* number / literal */
    return 0;
}

static int parse_tensor(scan_t *s, st_tensor_t *t) {
    if (!sk_ch(s, '{')) return -1;
    int have_dt = 0, have_sh = 0, have_off = 0;
    if (!sk_ch(s, '}'))
        for (;;) {
            char *k = sk_str(s);
            if (!k || !sk_ch(s, ':')) { free(k); return -1; }
            if (!strcmp(k, "dtype")) {
                char *v = sk_str(s);
                if (!v) { free(k); return -1; }
                t->dtype = !strcmp(v, "BF16") ? ST_BF16 : !strcmp(v, "F32") ? ST_F32 : !strcmp(v, "F16") ? ST_F16 : ST_OTHER;
                free(v);
                have_dt = 1;
            } else if (!strcmp(k, "shape")) {
                if (!sk_ch(s, '[')) { free(k); return -1; }
                t->ndim = 0;
                if (!sk_ch(s, ']'))
                    for (;;) {
                        long long v;
                        if (sk_int(s, &v) || t->ndim >= 4) { free(k); return -1; }
                        t->shape[t->ndim++] = v;
                        if (sk_ch(s, ',')) continue;
                        if (!sk_ch(s, ']')) { free(k); return -1; }
                        break;
                    }
                have_sh = 1;
            } else if (!strcmp(k, "data_offsets")) {
                long long a, b;
                if (!sk_ch(s, '[') || sk_int(s, &a) || !sk_ch(s, ',') || sk_int(s, &b) || !sk_ch(s, ']') || a < 0 || b < a) {
                    free(k);
                    return -1;
                }
                t->off0 = (unsigned long long)a; t->off1 = (unsigned long long)b;
                have_off = 1;
            } else if (sk_skip(s)) {
                free(k);
                return -1;
            }
            free(k);
            if (sk_ch(s, ',')) continue;
            if (!sk_ch(s, '}')) return -1;
            break;
        }
    return (have_dt && have_sh && have_off) ? 0 : -1;
}

static void st_close(st_file_t *f) {
    if (f->fd >= 0) close(f->fd);
    for (int i = 0; i < f->n; i++) free(f->t[i].name);
    free(f->t);
    memset(f, 0, sizeof *f);
    f->fd = -1;
}

static int st_open(st_file_t *f, const char *path) {
    char buf[4096];
    unsigned char len8[8];
    struct stat sb;
    char *hdr = NULL;
    memset(f, 0, sizeof *f);
    f->fd = -1;
    if (stat(path, &sb) == 0 && S_ISDIR(sb.st_mode)) {
        snprintf(buf, sizeof buf, "%s/model.safetensors", path);
        path = buf;
    }
    f->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (f->fd < 0) { qt_seterr("load: cannot open %s: %s", path, strerror(errno)); return -1; }
    if (fstat(f->fd, &sb) != 0 || pread(f->fd, len8, 8, 0) != 8) { qt_seterr("load: %s: cannot read the header length", path); goto fail; }
    unsigned long long N = 0;
    for (int i = 7; i >= 0; i--) N = (N << 8) | len8[i];
    f->file_size = (unsigned long long)sb.st_size;
    if (N == 0 || N > (1ull << 30) || 8 + N > f->file_size) { qt_seterr("load: %s: bad header length %llu", path, N); goto fail; }
    hdr = (char *)malloc(N);
    if (!hdr || pread(f->fd, hdr, N, 8) != (ssize_t)N) { qt_seterr("load: %s: cannot read the header", path); goto fail; }
    f->data_start = 8 + N;
    scan_t s = {hdr, hdr + N};
    if (!sk_ch(&s, '{')) { qt_seterr("load: %s: header is not a JSON object", path); goto fail; }
    if (!sk_ch(&s, '}'))
        for (;;) {
            char *k = sk_str(&s);
            if (!k || !sk_ch(&s, ':')) { free(k); qt_seterr("load: %s: malformed header", path); goto fail; }
            if (!strcmp(k, "__metadata__")) {
                free(k);
                if (sk_skip(&s)) { qt_seterr("load: %s: malformed __metadata__", path); goto fail; }
            } else {
                if (f->n == f->cap) {
                    int nc = f->cap ? 2 * f->cap : 256;
                    st_tensor_t *nt = (st_tensor_t *)realloc(f->t, (size_t)nc * sizeof *nt);
                    if (!nt) { free(k); qt_seterr("load: out of host memory"); goto fail; }
                    f->t = nt; f->cap = nc;
                }
                st_tensor_t *t = &f->t[f->n];
                memset(t, 0, sizeof *t);
                t->name = k;
                f->n++;
                if (parse_tensor(&s, t)) { qt_seterr("load: %s: malformed entry for %s", path, k); goto fail; }
                if (f->data_start + t->off1 > f->file_size) { qt_seterr("load: %s: %s extends past the end of the file", path, k); goto fail; }
            }
            if (sk_ch(&s, ',')) continue;
            if (!sk_ch(&s, '}')) { qt_seterr("load: %s: malformed header", path); goto fail; }
            break;
        }
    free(hdr);
    return 0;
fail:
    free(hdr);
    st_close(f);
    return -1;
}

static const st_tensor_t *st_find(const st_file_t *f, const char *name) {
    for (int i = 0; i < f->n; i++) if (!strcmp(f->t[i].name, name)) return &f->t[i];
    return NULL;
}

/* the tensor `name` with dtype (ST_BF16, or ST_BF16/ST_F32 for norms when any_float) and shape */
static const st_tensor_t *st_need(const st_file_t *f, const char *name, int any_float, long long d0, long long d1) {
    const st_tensor_t *t = st_find(f, name);
    if (!t) { qt_seterr("load: missing tensor %s", name); return NULL; }
    const int es = t->dtype == ST_F32 ? 4 : 2;
    const int ok_dt = t->dtype == ST_BF16 || (any_float && t->dtype == ST_F32);
    const long long n = d1 > 0 ? d0 * d1 : d0;
    const int ok_sh = d1 > 0 ? (t->ndim == 2 && t->shape[0] == d0 && t->shape[1] == d1) : (t->ndim == 1 && t->shape[0] == d0);
    if (!ok_dt || !ok_sh || t->off1 - t->off0 != (unsigned long long)n * es) {
        qt_seterr("load: tensor %s has dtype %d / %d dims [%lld, %lld] / %llu bytes, expected %s [%lld%s%lld]", name, t->dtype,
                  t->ndim, t->shape[0], t->ndim > 1 ? t->shape[1] : 0, t->off1 - t->off0, any_float ? "BF16/F32" : "BF16", d0,
                  d1 > 0 ? ", " : "", d1 > 0 ? d1 : 0);
        return NULL;
    }
    return t;
}

/* ---- file -> device ----------------------------------------------------------------------- */

#define LD_CHUNK ((size_t)32 << 20)

typedef struct {
    const st_file_t *f;
    hipStream_t st;
    void *stage[2];
    hipEvent_t ev[2];
    int used[2], next;
} loader_t;

/* bytes [off0, off1) of the data section -> dst (device) through the pinned buffers */
static int ld_copy(loader_t *L, const st_tensor_t *t, void *dst) {
    unsigned long long pos = L->f->data_start + t->off0, end = L->f->data_start + t->off1;
    char *d = (char *)dst;
    while (pos < end) {
        const int b = L->next;
        L->next ^= 1;
        if (L->used[b] && hipEventSynchronize(L->ev[b]) != hipSuccess) { qt_seterr("load: staging copy failed"); return -1; }
        size_t n = (size_t)(end - pos) < LD_CHUNK ? (size_t)(end - pos) : LD_CHUNK, got = 0;
        while (got < n) {
            ssize_t r = pread(L->f->fd, (char *)L->stage[b] + got, n - got, (off_t)(pos + got));
            if (r <= 0) { qt_seterr("load: read of %s failed: %s", t->name, r < 0 ? strerror(errno) : "end of file"); return -1; }
            got += (size_t)r;
        }
        if (hipMemcpyAsync(d, L->stage[b], n, hipMemcpyHostToDevice, L->st) != hipSuccess ||
            hipEventRecord(L->ev[b], L->st) != hipSuccess) {
            qt_seterr("load: copy to the device failed");
            return -1;
        }
        L->used[b] = 1;
        d += n;
        pos += n;
    }
    return 0;
}

/* a small f32 vector (norm gains, BF16 or F32 in the file) read on the host */
static float *ld_f32(const st_file_t *f, const st_tensor_t *t, long long n) {
    float *out = (float *)malloc((size_t)n * sizeof(float));
    if (!out) { qt_seterr("load: out of host memory"); return NULL; }
    const size_t bytes = (size_t)(t->off1 - t->off0);
    void *raw = malloc(bytes);
    if (!raw || pread(f->fd, raw, bytes, (off_t)(f->data_start + t->off0)) != (ssize_t)bytes) {
        free(raw); free(out);
        qt_seterr("load: read of %s failed", t->name);
        return NULL;
    }
    if (t->dtype == ST_F32) memcpy(out, raw, (size_t)n * sizeof(float));
    else
        for (long long i = 0; i < n; i++) {
            uint32_t u = (uint32_t)((const uint16_t *)raw)[i] << 16;    /* bf16 -> f32: exact (ingot dtype.c:270-275) */
            memcpy(&out[i], &u, sizeof u);
        }
    free(raw);
    return out;
}

void *qwen_hip_talker_load_file(const char *model_path, const qwen_hip_talker_desc_t *shape) {
    st_file_t f;
    loader_t L;
    void *state = NULL;
    const int nm = 6;
    memset(&L, 0, sizeof L);
    if (!model_path || !shape) { qt_seterr("load: null argument"); return NULL; }
    const int nl = shape->n_layers, H = shape->hidden, F = shape->inter, hd = shape->head_dim;
    if (nl <= 0 || nl > 64 || H <= 0 || F <= 0 || hd <= 0 || shape->n_heads <= 0 || shape->n_kv_heads <= 0 || H % 8 || F % 8) {
        qt_seterr("load: bad dimensions in the descriptor"); return NULL;
    }
    if (st_open(&f, model_path)) return NULL;
    const long long qd = (long long)shape->n_heads * hd, kvd = (long long)shape->n_kv_heads * hd;
    /* every tensor checked before the first GPU call */
    const st_tensor_t *(*T)[10] = calloc((size_t)nl, sizeof *T);
    const st_tensor_t *fn_t;
    float **norms = calloc((size_t)nl * 4, sizeof(float *));
    float *final_norm = NULL;
    uint16_t **dev = calloc((size_t)nl * nm, sizeof(uint16_t *));   /* q k v o gate_up down, device bf16 */
    uint16_t *dgate = NULL, *dup = NULL;
    qwen_hip_layer_t *lay = calloc((size_t)nl, sizeof *lay);
    if (!T || !norms || !dev || !lay) { qt_seterr("load: out of host memory"); goto fail; }
    for (int l = 0; l < nl; l++) {
        char nmb[256];
#define NEED(i, sfx, anyf, d0, d1) do { snprintf(nmb, sizeof nmb, "talker.model.layers.%d.%s", l, sfx); \
        if (!(T[l][i] = st_need(&f, nmb, anyf, d0, d1))) goto fail; } while (0)
        NEED(0, "self_attn.q_proj.weight", 0, qd, H);
        NEED(1, "self_attn.k_proj.weight", 0, kvd, H);
        NEED(2, "self_attn.v_proj.weight", 0, kvd, H);
        NEED(3, "self_attn.o_proj.weight", 0, H, qd);
        NEED(4, "mlp.gate_proj.weight", 0, F, H);
        NEED(5, "mlp.up_proj.weight", 0, F, H);
        NEED(6, "mlp.down_proj.weight", 0, H, F);
        NEED(7, "input_layernorm.weight", 1, H, 0);
        NEED(8, "post_attention_layernorm.weight", 1, H, 0);
        NEED(9, "self_attn.q_norm.weight", 1, hd, 0);
#undef NEED
    }
    if (!(fn_t = st_need(&f, "talker.model.norm.weight", 1, H, 0))) goto fail;
    for (int l = 0; l < nl; l++) {
        char nmb[256];
        snprintf(nmb, sizeof nmb, "talker.model.layers.%d.self_attn.k_norm.weight", l);
        const st_tensor_t *kn = st_need(&f, nmb, 1, hd, 0);
        if (!kn) goto fail;
        if (!(norms[4 * l + 0] = ld_f32(&f, T[l][7], H)) || !(norms[4 * l + 1] = ld_f32(&f, T[l][8], H)) ||
            !(norms[4 * l + 2] = ld_f32(&f, T[l][9], hd)) || !(norms[4 * l + 3] = ld_f32(&f, kn, hd)))
            goto fail;
    }
    if (!(final_norm = ld_f32(&f, fn_t, H))) goto fail;

    /* file -> device */
    if (!qwen_hip_available()) { qt_seterr("load: no HIP device"); goto fail; }
    if (hipStreamCreateWithFlags(&L.st, hipStreamNonBlocking) != hipSuccess) { qt_seterr("load: stream create failed"); goto fail; }
    for (int b = 0; b < 2; b++)
        if (hipHostMalloc(&L.stage[b], LD_CHUNK, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&L.ev[b], hipEventDisableTiming) != hipSuccess) {
            qt_seterr("load: pinned staging allocation failed"); goto fail;
        }
    L.f = &f;
    if (hipMalloc((void **)&dgate, (size_t)F * H * 2) != hipSuccess || hipMalloc((void **)&dup, (size_t)F * H * 2) != hipSuccess) {
        qt_seterr("load: device allocation failed"); goto fail;
    }
    for (int l = 0; l < nl; l++) {
        const long long rows[6] = {qd, kvd, kvd, H, 2LL * F, H}, cols[6] = {H, H, H, qd, H, F};
        for (int i = 0; i < nm; i++)
            if (hipMalloc((void **)&dev[l * nm + i], (size_t)(rows[i] * cols[i] * 2)) != hipSuccess) {
                qt_seterr("load: device allocation failed"); goto fail;
            }
        if (ld_copy(&L, T[l][0], dev[l * nm + 0]) || ld_copy(&L, T[l][1], dev[l * nm + 1]) ||
            ld_copy(&L, T[l][2], dev[l * nm + 2]) || ld_copy(&L, T[l][3], dev[l * nm + 3]) ||
            ld_copy(&L, T[l][4], dgate) || ld_copy(&L, T[l][5], dup) || ld_copy(&L, T[l][6], dev[l * nm + 5]))
            goto fail;
        if (qt_launch_interleave_rows(dgate, dup, dev[l * nm + 4], F, H, L.st) != hipSuccess ||
            hipStreamSynchronize(L.st) != hipSuccess) {     /* dgate/dup are reused by the next layer */
            qt_seterr("load: gate|up interleave failed"); goto fail;
        }
        qwen_hip_layer_t *ly = &lay[l];
        ly->q.w = dev[l * nm + 0]; ly->k.w = dev[l * nm + 1]; ly->v.w = dev[l * nm + 2];
        ly->o.w = dev[l * nm + 3]; ly->gate_up.w = dev[l * nm + 4]; ly->down.w = dev[l * nm + 5];
        ly->input_norm = norms[4 * l + 0]; ly->post_attn_norm = norms[4 * l + 1];
        ly->q_norm = norms[4 * l + 2]; ly->k_norm = norms[4 * l + 3];
    }
    {
        qwen_hip_talker_desc_t d = *shape;
        d.prec = QWEN_HIP_BF16;
        d.layers = lay;
        d.final_norm = final_norm;
        state = qwen_hip_talker_init(&d);        /* copies / quantizes from the device buffers */
    }
fail:
    if (L.st) (void)hipStreamSynchronize(L.st);
    for (int b = 0; b < 2; b++) {
        if (L.stage[b]) (void)hipHostFree(L.stage[b]);
        if (L.ev[b]) (void)hipEventDestroy(L.ev[b]);
    }
    if (L.st) (void)hipStreamDestroy(L.st);
    if (dev) for (int i = 0; i < nl * nm; i++) if (dev[i]) (void)hipFree(dev[i]);
    if (dgate) (void)hipFree(dgate);
    if (dup) (void)hipFree(dup);
    if (norms) for (int i = 0; i < nl * 4; i++) free(norms[i]);
    free(norms); free(final_norm); free(dev); free(lay); free(T);
    st_close(&f);
    return state;
}

/* ---- speech decoder from its safetensors file ------------------------------------------- */
typedef struct {
    st_file_t f;
    float *buf;
    size_t cap;
} sd_src_t;

/* qwen_hip_sd_get_fn over the file: the F32 tensor `name` of n floats, read into a buffer
 * that the next call reuses */
static const float *sd_file_get(void *user, const char *name, long long n) {
    sd_src_t *S = (sd_src_t *)user;
    const st_tensor_t *t = st_find(&S->f, name);
    if (!t) { qt_seterr("load: missing tensor %s", name); return NULL; }
    if (t->dtype != ST_F32 || t->off1 - t->off0 != (unsigned long long)n * 4) {
        qt_seterr("load: tensor %s is dtype %d with %llu bytes, expected F32 with %lld floats", name, t->dtype,
                  t->off1 - t->off0, n);
        return NULL;
    }
    if ((size_t)n > S->cap) {
        free(S->buf);
        S->buf = (float *)malloc((size_t)n * sizeof(float));
        S->cap = S->buf ? (size_t)n : 0;
        if (!S->buf) { qt_seterr("load: out of host memory"); return NULL; }
    }
    size_t got = 0, bytes = (size_t)n * 4;
    while (got < bytes) {
        ssize_t r = pread(S->f.fd, (char *)S->buf + got, bytes - got, (off_t)(S->f.data_start + t->off0 + got));
        if (r <= 0) { qt_seterr("load: read of %s failed", name); return NULL; }
        got += (size_t)r;
    }
    return S->buf;
}

void *qwen_hip_sd_load_file(const char *path) {
    char buf[4096];
    struct stat sb;
    if (!path) { qt_seterr("load: null path"); return NULL; }
    if (stat(path, &sb) == 0 && S_ISDIR(sb.st_mode)) {
        snprintf(buf, sizeof buf, "%s/speech_decoder.safetensors", path);
        path = buf;
    }
    sd_src_t S;
    memset(&S, 0, sizeof S);
    if (st_open(&S.f, path)) return NULL;
    void *state = qwen_hip_sd_init(sd_file_get, &S);
    st_close(&S.f);
    free(S.buf);
    return state;
}
