// qt_misc.hip — small kernels around the decode step: final RMSNorm, greedy
// codec-head / lm-head selection, embedding gather, load-time weight preparation
// (int8 quantizer, q4_0 repack, int8 re-encoding) and a dequantiser for bit checks.
#include "qt_device.h"

// out = RMSNorm(x)*w (qwen_tts_kernels.c:292-382); optionally advance *d_pos by one
// (the resident decode loop's device-side position).  One 1024-thread workgroup; every
// thread issues its (<= 4) loads before using any, so the kernel pays one memory latency.
#define QT_BIG 1024
__device__ __forceinline__ float big_block_sum(float v, float *red) {
    v = group_sum<64>(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < QT_BIG / 64; i++) t += red[i];
    return t;
}

__global__ __launch_bounds__(QT_BIG) void k_rmsnorm(const float *x, const float *w, float *out, int n,
                                                    float eps, int *d_pos) {
    __shared__ float red[QT_BIG / 64];
    float xv[4], wv[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i = threadIdx.x + k * QT_BIG;
        xv[k] = i < n ? x[i] : 0.f;
        wv[k] = i < n ? w[i] : 0.f;
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) ss += xv[k] * xv[k];
    const float tot = big_block_sum(ss, red);
    const float inv = 1.0f / sqrtf(tot / (float)n + eps);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i = threadIdx.x + k * QT_BIG;
        if (i < n) out[i] = (xv[k] * inv) * wv[k];
    }
    if (d_pos && threadIdx.x == 0) *d_pos += 1;
}

extern "C" hipError_t qt_launch_rmsnorm(const float *x, const float *w, float *out, int n, float eps,
                                        int *d_pos, hipStream_t st) {
    if (n <= 0 || n > 4 * QT_BIG) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(QT_BIG), 0, st, x, w, out, n, eps, d_pos);
    return hipGetLastError();
}

// Per-row RMSNorm of `rows` vectors of length n (per-head norm, k.c:486-577), in place.
// Per-row RMSNorm of `rows` vectors of length n (per-head norm, k.c:486-577): out row b =
// RMSNorm(x row b) * w (in place when out == x); pos != NULL: workgroup b also advances
// pos[b] (the batched step's position advance, folded into its final norm).
// Lane t accumulates x[t], x[t + 64], ... in index order; the loads go out eight at a time
// (one memory round trip per 512 elements, not per 64), the sums in the same order.
__global__ __launch_bounds__(64) void k_rmsnorm_rows(const float *x, float *out, const float *w, int n, float eps,
                                                     int *pos) {
    const float *r = x + (size_t)blockIdx.x * n;
    float *o = out + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (int i0 = threadIdx.x; i0 < n; i0 += 64 * 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = i0 + 64 * k < n ? r[i0 + 64 * k] : 0.f;
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (i0 + 64 * k < n) ss += v[k] * v[k];
    }
    ss = group_sum<64>(ss);
    float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i0 = threadIdx.x; i0 < n; i0 += 64 * 8) {
        float v[8], g[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const bool ok = i0 + 64 * k < n;
            v[k] = ok ? r[i0 + 64 * k] : 0.f;
            g[k] = ok ? w[i0 + 64 * k] : 0.f;
        }
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (i0 + 64 * k < n) o[i0 + 64 * k] = (v[k] * inv) * g[k];
    }
    if (pos && threadIdx.x == 0) pos[blockIdx.x] += 1;
}

extern "C" hipError_t qt_launch_rmsnorm_rows(float *x, const float *w, int rows, int n, float eps,
                                             hipStream_t st) {
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(rows), dim3(64), 0, st, x, x, w, n, eps, (int *)NULL);
    return hipGetLastError();
}
extern "C" hipError_t qt_launch_rmsnorm_rows_to(const float *x, float *out, const float *w, int rows, int n,
                                                float eps, int *pos, hipStream_t st) {
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(rows), dim3(64), 0, st, x, out, w, n, eps, pos);
    return hipGetLastError();
}

// SwiGLU over interleaved pairs, out[i] = g/(1+expf(-g))*u (k.c:3857-3878).
__global__ void k_swiglu(const float *gu, float *out, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) { float g = gu[2 * i], u = gu[2 * i + 1]; out[i] = g / (1.0f + expf(-g)) * u; }
}
extern "C" hipError_t qt_launch_swiglu(const float *gu, float *out, int n, hipStream_t st) {
    hipLaunchKernelGGL(k_swiglu, dim3((n + 255) / 256), dim3(256), 0, st, gu, out, n);
    return hipGetLastError();
}

// Greedy pick over `n` logits, lowest index on ties.  mode 0: plain argmax with the
// fused argmax-matvec start value -1e30 (qwen_tts_kernels.c:4652-4759, CP lm heads);
// mode 1: the codec-head rule of qwen_tts.c:1652-1663 + qwen_tts_sampling.c:175-182
// (clip to +-100, tokens >= 2048 except EOS 2150 masked, EOS masked while the frame
// index *d_frame < 2).  Writes the token to tok[0] and, when hist != NULL, to
// hist[*d_frame % hist_len]; advance != 0 increments *d_frame.  When emb != NULL it
// also gathers the next input embedding out[i] = bf16(emb[tok*emb_dim + i])
// (qwen_tts.c:919-924).  One workgroup.
__global__ __launch_bounds__(QT_BIG) void k_select(const float *logits, int n, int mode, int *d_frame, int advance,
                                                   int *tok, int *hist, int hist_len, const uint16_t *emb,
                                                   int emb_dim, float *out, int *d_pos) {
    __shared__ float bv_s[QT_BIG / 64];
    __shared__ int bi_s[QT_BIG / 64];
    __shared__ int t_s;
    const int frame = d_frame ? *d_frame : 0;
    float lv[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i = threadIdx.x + k * QT_BIG;
        lv[k] = i < n ? logits[i] : -INFINITY;
    }
    float bv = (mode == 0) ? -1e30f : -INFINITY;
    int bi = 0x7FFFFFFF;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i = threadIdx.x + k * QT_BIG;
        if (i >= n) continue;
        float v = lv[k];
        if (mode == 1) {
            v = fminf(fmaxf(v, -100.0f), 100.0f);
            if (i >= 2048 && i != 2150) v = -1e30f;
            if (i == 2150 && frame < 2) v = -1e30f;
        }
        if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(bv, o, 64);
        int oi = __shfl_xor(bi, o, 64);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { bv_s[wave] = bv; bi_s[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = bv_s[0]; int ix = bi_s[0];
        for (int w = 1; w < QT_BIG / 64; w++)
            if (bv_s[w] > b || (bv_s[w] == b && bi_s[w] < ix)) { b = bv_s[w]; ix = bi_s[w]; }
        if (ix == 0x7FFFFFFF) ix = 0;   // nothing beat the start value: index 0
        tok[0] = ix;
        if (hist) hist[frame % hist_len] = ix;
        t_s = ix;
        if (advance && d_frame) *d_frame = frame + 1;
        if (d_pos) *d_pos += 1;
    }
    __syncthreads();
    if (emb) {
        const int t = t_s;
        for (int i = threadIdx.x; i < emb_dim; i += QT_BIG) out[i] = bf16f(emb[(size_t)t * emb_dim + i]);
    }
}

extern "C" hipError_t qt_launch_select(const float *logits, int n, int mode, int *d_frame, int advance, int *tok,
                                       int *hist, int hist_len, const uint16_t *emb, int emb_dim, float *out,
                                       int *d_pos, hipStream_t st) {
    if (n <= 0 || n > 4 * QT_BIG) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_select, dim3(1), dim3(QT_BIG), 0, st, logits, n, mode, d_frame, advance, tok, hist,
                       hist_len, emb, emb_dim, out, d_pos);
    return hipGetLastError();
}

__global__ void k_copy_f32(const float *src, float *dst, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) dst[i] = src[i];
}
extern "C" hipError_t qt_launch_copy_f32(const float *src, float *dst, int n, hipStream_t st) {
    hipLaunchKernelGGL(k_copy_f32, dim3(4), dim3(256), 0, st, src, dst, n);
    return hipGetLastError();
}

// x[i] = bf16(table[tok*dim + i]), tok read on device (embedding gather).
__global__ void k_gather(const int *tok, int tok_max, const uint16_t *table, int dim, float *out) {
    const int t = *tok;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < dim; i += gridDim.x * blockDim.x)
        out[i] = (t >= 0 && t < tok_max) ? bf16f(table[(size_t)t * dim + i]) : 0.0f;
}
extern "C" hipError_t qt_launch_gather(const int *tok, int tok_max, const uint16_t *table, int dim, float *out,
                                       hipStream_t st) {
    hipLaunchKernelGGL(k_gather, dim3(4), dim3(256), 0, st, tok, tok_max, table, dim, out);
    return hipGetLastError();
}

// ---- load-time weight preparation ------------------------------------------------

// Per-row absmax int8 quantizer, bit-exact with the reference binary
// (qwen_tts_kernels.c:2143-2238 compiled with -O3 -ffast-math): scale = amax*(1/127)
// (the constant division becomes a multiply by the f32 reciprocal), inv = 127/amax,
// q = round-half-even(v*inv) on the 8-wide body, roundf on the cols%8 tail, saturated.
// Output in the device encoding u = q ^ 0x80.  One workgroup per row.
__global__ __launch_bounds__(QT_WG) void k_quant_int8(const uint16_t *src, int cols, uint8_t *dst, float *scale) {
    __shared__ float red[QT_WAVES];
    const uint16_t *row = src + (size_t)blockIdx.x * cols;
    float amax = 0.f;
    for (int k = threadIdx.x; k < cols; k += QT_WG) amax = fmaxf(amax, fabsf(bf16f(row[k])));
    amax = group_max<64>(amax);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = amax * (1.0f / 127.0f);
    const float inv = (s > 0.f) ? 127.0f / amax : 0.f;
    if (threadIdx.x == 0) scale[blockIdx.x] = s;
    const int body = cols - cols % 8;
    for (int k = threadIdx.x; k < cols; k += QT_WG) {
        const float p = bf16f(row[k]) * inv;
        int v = (k < body) ? (int)__builtin_rintf(p) : (int)roundf(p);
        v = v < -128 ? -128 : (v > 127 ? 127 : v);
        dst[(size_t)blockIdx.x * cols + k] = (uint8_t)(v & 0xFF);
    }
}
extern "C" hipError_t qt_launch_quant_int8(const uint16_t *src, int rows, int cols, uint8_t *dst, float *scale,
                                           hipStream_t st) {
    hipLaunchKernelGGL(k_quant_int8, dim3(rows), dim3(QT_WG), 0, st, src, cols, dst, scale);
    return hipGetLastError();
}

// Reference q4_0 blocks {u16 scale; u8 qs[16]} (18 B, qwen_tts_kernels.h:206-210) ->
// qs rows [rows][cols/2] + f16 scale bits [rows][cols/32].  Pure byte moves.
__global__ void k_repack_q4(const uint8_t *blocks, size_t nblocks, uint8_t *qs, uint16_t *s16) {
    size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; b < nblocks; b += stride) {
        const uint8_t *src = blocks + b * 18;
        s16[b] = (uint16_t)(src[0] | (src[1] << 8));
        uint8_t *d = qs + b * 16;
#pragma unroll
        for (int i = 0; i < 16; i++) d[i] = src[2 + i];
    }
}
extern "C" hipError_t qt_launch_repack_q4(const uint8_t *blocks, size_t nblocks, uint8_t *qs, uint16_t *s16,
                                          hipStream_t st) {
    hipLaunchKernelGGL(k_repack_q4, dim3(1024), dim3(256), 0, st, blocks, nblocks, qs, s16);
    return hipGetLastError();
}

// Weighted-LSQ q4_0 quantizer (qwen_tts_kernels.c:2662-2726) into the device layout
// (qs rows + f16 scale bits).  One thread per 32-block; double accumulation in index
// order.  The reference build may vectorise its double sums in another order, but each
// term (v^2 * v * q, v^2 * q^2 of bf16 v and q in [-8, 7]) is an exact double and the
// sums' last-place rounding does not reach the f16 rounding of the scale, so the bytes
// are the reference's (tested bit for bit).
__device__ uint16_t ref_f32_to_f16(float f) {
    uint32_t u = __float_as_uint(f);
    uint32_t sign = (u >> 16) & 0x8000u;
    int e = (int)((u >> 23) & 0xFF) - 112;
    uint32_t m = u & 0x7FFFFFu;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t full = m | 0x800000u, sh = (uint32_t)(14 - e);
        uint32_t r = full >> sh;
        if ((full >> (sh - 1)) & 1u) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = sign | ((uint32_t)e << 10) | (m >> 13);
    if (m & 0x1000u) r++;
    return (uint16_t)r;
}

__global__ void k_quant_q4(const uint16_t *src, int rows, int cols, uint8_t *qs, uint16_t *s16) {
    const int nb = cols / 32;
    size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= (size_t)rows * nb) return;
    const uint16_t *blk = src + b * 32;   // rows are contiguous: block b = row*nb + j
    float v[32], amax = 0.f, vmax = 0.f;
    for (int i = 0; i < 32; i++) {
        v[i] = bf16f(blk[i]);
        float a = fabsf(v[i]);
        if (a > amax) { amax = a; vmax = v[i]; }
    }
    const float isc = (vmax != 0.f) ? -8.0f / vmax : 0.f;
    int q[32];
    double num = 0.0, den = 0.0;
    for (int i = 0; i < 32; i++) {
        int t = (int)roundf(v[i] * isc);
        t = t < -8 ? -8 : (t > 7 ? 7 : t);
        q[i] = t;
        double w = (double)v[i] * (double)v[i];
        num = __dadd_rn(num, __dmul_rn(__dmul_rn(w, (double)v[i]), (double)t));
        den = __dadd_rn(den, __dmul_rn(__dmul_rn(w, (double)t), (double)t));
    }
    const float s = (den > 0.0) ? (float)(num / den) : 0.f;
    s16[b] = ref_f32_to_f16(s);
    uint8_t *d = qs + b * 16;
    for (int i = 0; i < 16; i++) d[i] = (uint8_t)((q[2 * i] + 8) | ((q[2 * i + 1] + 8) << 4));
}
extern "C" hipError_t qt_launch_quant_q4(const uint16_t *src, int rows, int cols, uint8_t *qs, uint16_t *s16,
                                         hipStream_t st) {
    size_t nb = (size_t)rows * (cols / 32);
    hipLaunchKernelGGL(k_quant_q4, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, st, src, rows, cols, qs, s16);
    return hipGetLastError();
}

// Dequantise rows [r0, r0+n) of a device matrix to f32 (bit-exactness checks):
// bf16 -> f32 shift; int8 -> (float)q * scale; q4 -> (nib-8) * f16(scale).
__global__ void k_dequant(int prec, const uint8_t *w, const float *scale, const uint16_t *s16, int cols,
                          int r0, int n, float *out) {
    size_t total = (size_t)n * cols;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const int r = r0 + (int)(i / cols), k = (int)(i % cols);
        float v;
        if (prec == QT_BF16) v = bf16f(reinterpret_cast<const uint16_t *>(w)[(size_t)r * cols + k]);
        else if (prec == QT_INT8) v = (float)(int)(int8_t)w[(size_t)r * cols + k] * scale[r];
        else {
            const uint8_t byte = w[(size_t)r * (cols / 2) + k / 2];
            const int nib = (k & 1) ? (byte >> 4) : (byte & 0xF);
            v = (float)(nib - 8) * ref_f16_to_f32(s16[(size_t)r * (cols / 32) + k / 32]);
        }
        out[i] = v;
    }
}
extern "C" hipError_t qt_launch_dequant(int prec, const uint8_t *w, const float *scale, const uint16_t *s16,
                                        int cols, int r0, int n, float *out, hipStream_t st) {
    hipLaunchKernelGGL(k_dequant, dim3(512), dim3(256), 0, st, prec, w, scale, s16, cols, r0, n, out);
    return hipGetLastError();
}

// Fill a buffer with zeros (graph-capturable replacement for hipMemsetAsync).
__global__ void k_zero_u32(uint32_t *p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0;
}
extern "C" hipError_t qt_launch_zero_u32(uint32_t *p, size_t n, hipStream_t st) {
    hipLaunchKernelGGL(k_zero_u32, dim3(64), dim3(256), 0, st, p, n);
    return hipGetLastError();
}

// KV layout change between the reference's host cache rows (position-major:
// [n][n_kv*head_dim] bf16, qwen_tts.h:513-518) and the device cache (head-major:
// [n_kv][kv_max][head_dim], one contiguous row per head and position).  One thread per
// 16-byte chunk (8 bf16): reads of a position's row are contiguous, and so are the
// writes of one head's row.  to_heads = 1: rows -> heads (upload), 0: heads -> rows.
__global__ void k_kv_relayout(const uint4 *src, uint4 *dst, int n, int nkv, int hd, long long kv_max, int to_heads) {
    const int cpr = hd / 8;                              // 16-byte chunks per head row
    const long long total = (long long)n * nkv * cpr;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (long long)gridDim.x * blockDim.x) {
        const int c = (int)(i % cpr);
        const long long t = i / cpr;
        const int g = (int)(t % nkv);
        const long long p = t / nkv;
        const long long row_idx = (p * nkv + g) * cpr + c;           // position-major
        const long long head_idx = ((long long)g * kv_max + p) * cpr + c;   // head-major
        if (to_heads) dst[head_idx] = src[row_idx];
        else dst[row_idx] = src[head_idx];
    }
}
extern "C" hipError_t qt_launch_kv_relayout(const uint16_t *src, uint16_t *dst, int n, int nkv, int hd, int kv_max,
                                            int to_heads, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    if (hd % 8 || nkv <= 0 || kv_max < n) return hipErrorInvalidValue;
    const long long total = (long long)n * nkv * (hd / 8);
    long long blocks = (total + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(k_kv_relayout, dim3((unsigned)blocks), dim3(256), 0, st, (const uint4 *)src, (uint4 *)dst, n, nkv,
                       hd, (long long)kv_max, to_heads);
    return hipGetLastError();
}

// Next Talker input of the frame loop (qwen_tts.c:1768-1778): e = codec_emb[code0] (bf16 -> f32,
// zeros for an out-of-range code, lookup_codec_embed qwen_tts.c:919-924), then += each CP
// group's embedding row cp_emb[g][codes[g + 1]] in g order (skipped when out of range,
// qwen_bf16_accum_f32 k.c:3900-3925), then += tts_pad; one f32 add at a time per element,
// as the reference does, so the result is bit-identical.  codes[0] = code0, codes[1..15].
struct QtFrameEmb { const uint16_t *g[15]; };
__global__ void k_frame_embed(const int *codes, int vocab, int codebook, const uint16_t *codec_emb, QtFrameEmb cp,
                              const float *pad, int H, float *out) {
    const int c0 = codes[0];
    int cg[15];
#pragma unroll
    for (int g = 0; g < 15; g++) cg[g] = codes[g + 1];
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < H; i += gridDim.x * blockDim.x) {
        float e = (c0 >= 0 && c0 < vocab) ? bf16f(codec_emb[(size_t)c0 * H + i]) : 0.0f;
#pragma unroll
        for (int g = 0; g < 15; g++)
            if (cg[g] >= 0 && cg[g] < codebook) e = __fadd_rn(e, bf16f(cp.g[g][(size_t)cg[g] * H + i]));
        out[i] = __fadd_rn(e, pad[i]);
    }
}
extern "C" hipError_t qt_launch_frame_embed(const int *codes, int vocab, int codebook, const uint16_t *codec_emb,
                                            const uint16_t *const cp_emb[15], const float *pad, int H, float *out,
                                            hipStream_t st) {
    QtFrameEmb cp;
    for (int g = 0; g < 15; g++) {
        if (!cp_emb[g]) return hipErrorInvalidValue;
        cp.g[g] = cp_emb[g];
    }
    hipLaunchKernelGGL(k_frame_embed, dim3((H + 255) / 256), dim3(256), 0, st, codes, vocab, codebook, codec_emb, cp, pad,
                       H, out);
    return hipGetLastError();
}

// gate|up row interleave on the device (the reference loader does it on the host,
// qwen_tts_talker.c:378-388): out row 2r = gate row r, out row 2r+1 = up row r; bf16 rows
// of `cols` elements, copied as 16-byte chunks (cols % 8 == 0).
__global__ void k_interleave_rows(const uint4 *gate, const uint4 *up, uint4 *out, int rows, int cpr) {
    const long long total = (long long)rows * cpr;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (long long)gridDim.x * blockDim.x) {
        const long long r = i / cpr, c = i % cpr;
        out[(2 * r) * cpr + c] = gate[i];
        out[(2 * r + 1) * cpr + c] = up[i];
    }
}
extern "C" hipError_t qt_launch_interleave_rows(const uint16_t *gate, const uint16_t *up, uint16_t *out, int rows, int cols,
                                                hipStream_t st) {
    if (rows <= 0 || cols <= 0 || cols % 8) return hipErrorInvalidValue;
    const long long total = (long long)rows * (cols / 8);
    long long blocks = (total + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(k_interleave_rows, dim3((unsigned)blocks), dim3(256), 0, st, (const uint4 *)gate, (const uint4 *)up,
                       (uint4 *)out, rows, cols / 8);
    return hipGetLastError();
}
