// qt_sd.hip — the speech decoder (codes -> 24 kHz audio) on gfx950.
//
// The reference's one-shot decode (qwen_speech_decoder_decode, qwen_tts_speech_decoder.c:
// 579-1290) is a VQ lookup, an 8-layer windowed-attention transformer over the frames and
// a convolutional upsampler (ConvNeXt x2, then four blocks of transposed conv + dilated
// residual units) to 1920 samples per frame.  All of it is f32.  Here every activation is
// kept time-major ([T][C], channels contiguous), and every projection, convolution and
// transposed convolution is one implicit GEMM on the f32 matrix cores:
//
//   Y[t*os + z][n] = epi( sum over taps p, channels k of X[t + off_p][k] * W[z][p][k][n] )
//
// (rows of X outside [xlo, Tx) read as zero: the causal left padding; the streaming decode
// keeps the previous chunk's last rows at negative indices, xlo < 0).  A causal conv of
// kernel K and dilation d has taps off_p = (p - K + 1) d; a transposed conv of stride s
// and kernel 2s is s phases z (output rows t*s + z), each with taps at offsets 0 and -1
// (kernel columns z and z + s); a linear layer is one tap.  The epilogue adds a bias,
// applies GELU, scales per column (layer scale, ConvNeXt gamma), adds a residual and
// applies the snake activation that the next layer needs on its input (so no separate
// pass over the activation: the upsampler's snakes all live in the producing GEMM).
// Products accumulate in f32 in MFMA order (the reference sums in loop order): the
// results agree to f32 rounding, not bitwise.
#include "qt_device.h"

typedef float qt_sd_f4 __attribute__((ext_vector_type(4)));

#define SD_WG 256
#define SD_KC 16                 // K chunk staged per step (the 16- and 32-row tiles stage 64 where K allows)
#define SD_MAXTAP 8

enum { SD_EPI_BIAS = 1, SD_EPI_GELU = 2, SD_EPI_CSCALE = 4, SD_EPI_RESID = 8, SD_EPI_SNAKE = 16, SD_EPI_SNAKE2 = 32 };

struct SdGemmArgs {
    const float *X; int ldx, Tx, xlo;     // input rows [xlo, Tx) of a [.][ldx] buffer (xlo <= 0: history rows)
    const float *W;                       // [phases][ntap][K][N]
    int K, N, ntap;
    int off[SD_MAXTAP];
    int T;                                // output rows per phase (t < T)
    float *Y; int ldy, os;                // output row t*os + phase
    const float *bias, *cscale;
    const float *R;                       // residual, same indexing as Y (may alias Y)
    const float *sa, *sib;                // SNAKE: Y = snake(v) with per-column a, 1/b
    float *Y2;                            // SNAKE2: Y = v and Y2 = snake(v) (same indexing)
    int epi;
};

__device__ __forceinline__ float sd_gelu(float x) {
    return 0.5f * x * (1.0f + erff(x * 0.7071067811865476f));
}

// snake (k.c:4472-4600): x + (1/b) sin(a x)^2 with a = e^alpha, 1/b = e^-beta per channel
__device__ __forceinline__ float sd_snake(float x, float a, float ib) {
    const float s = sinf(a * x);
    return fmaf(ib, s * s, x);
}

// TM x TN output tile (16, 32 or 64 x 64, or 128 x 128), four waves of a 2 x 2 grid (a
// 1 x 4 grid for TM = 16), each a grid of 16 x 16 MFMA tiles; K in chunks of KC (16, or
// 64 for the small tiles where K allows) staged through LDS (two buffers).  The global
// loads of the next P chunks sit in a ring of P register slots: a chunk's loads are
// issued P - 1 chunks before it is staged, which hides HBM latency when only a few
// workgroups share a CU (a streaming chunk of a few frames gives the long-K convolutions
// a few dozen tiles).  The fetch index is clamped to the last chunk rather than guarded,
// so the loads are straight-line code and the compiler counts them exactly.  Every
// output element sums its products four k at a time in ascending k, one MFMA after
// another, whatever TM, TN, P and KC are, so every tile gives the same bits.
// The 128 x 128 tile reads each A and B value from LDS once per four MFMAs (twice as
// many as the 64 x 64 tile's two).
// v_mfma_f32_16x16x4_f32: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16] and
// receives D[4 (l / 16) + r][l % 16], r < 4.
template <int TM, int TN, int P, int KC>
__global__ __launch_bounds__(SD_WG) void k_sd_gemm(SdGemmArgs a) {
    static_assert(P >= 2 && P % 2 == 0, "chunk c sits in LDS buffer c & 1 == slot & 1");
    static_assert(KC == 16 || KC == 64, "K chunk");
    // A chunk is TM x KC floats = TM * KC / 4 float4s; where that is fewer than the 256
    // threads (16 or 32 rows at KC = 16) the spare waves load a copy of the same rows
    // (same addresses, nothing staged)
    constexpr int AF4 = TM * KC / 4, AQ = AF4 >= SD_WG ? AF4 / SD_WG : 1;   // A float4 loads per thread
    constexpr int BQ = KC * TN / (4 * SD_WG);                               // B float4 loads per thread
    constexpr int AS = KC + (KC == 16 ? 1 : 17);   // A row stride = 17 mod 32 floats: 16 rows spread over banks
    constexpr int WMW = TM >= 32 ? 2 : 1, WNW = 4 / WMW;     // wave grid: WMW along M, WNW along N
    constexpr int BS = TN + 16;                        // B row stride: rows k, k+1 on opposite bank halves
    constexpr int MI = TM / (16 * WMW), NJ = TN / (16 * WNW);   // 16 x 16 MFMA tiles per wave
    static_assert(MI >= 1 && NJ >= 1 && TN % 64 == 0 && BQ >= 1, "tile shape");
    __shared__ float As[2][TM * AS];
    __shared__ float Bs[2][KC * BS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = blockIdx.x * TM, n0 = blockIdx.y * TN, z = blockIdx.z;
    const float *W = a.W + (size_t)z * a.ntap * a.K * a.N;
    const int kpt = a.K / KC, nch = a.ntap * kpt;
    // ring slots hold the loads as issued (clamped rows and columns); which of them are
    // real (am: bit q of the slot's A loads, bok: B columns inside N) is applied when a
    // slot is staged, so the loads have no use before then and nothing branches around them
    float4 av[P][AQ], bv[P][BQ];
    unsigned amk[P];
    unsigned bok = 0;
#pragma unroll
    for (int q = 0; q < BQ; q++) bok |= (n0 + ((tid + q * SD_WG) % (TN / 4)) * 4 < a.N) ? 1u << q : 0u;
    auto fetch = [&](int c, float4 (&ra)[AQ], float4 (&rb)[BQ], unsigned &am) {
        const int p = c / kpt, k0 = (c - p * kpt) * KC;
#pragma unroll
        for (int q = 0; q < AQ; q++) {
            const int f = tid + q * SD_WG, ar = (f / (KC / 4)) % TM, ac = (f % (KC / 4)) * 4;
            const int xr = t0 + ar + a.off[p];
            const bool ok = t0 + ar < a.T && xr >= a.xlo && xr < a.Tx;
            const int xc = min(max(xr, a.xlo), a.Tx - 1);   // in bounds; the value is dropped when !ok
            ra[q] = *reinterpret_cast<const float4 *>(a.X + (ptrdiff_t)xc * a.ldx + k0 + ac);
            am = ok ? am | (1u << q) : am & ~(1u << q);
        }
#pragma unroll
        for (int q = 0; q < BQ; q++) {
            const int f = tid + q * SD_WG, br = f / (TN / 4), bc = (f % (TN / 4)) * 4;
            const int nc = min(n0 + bc, a.N - 4);
            rb[q] = *reinterpret_cast<const float4 *>(W + ((size_t)p * a.K + k0 + br) * a.N + nc);
        }
    };
    auto stage = [&](int buf, const float4 (&ra)[AQ], const float4 (&rb)[BQ], unsigned am) {
        // masks on the bits, value by value (a select of whole float4s becomes a select of
        // their addresses, which moves the ring to scratch)
#pragma unroll
        for (int q = 0; q < AQ; q++) {
            const int f = tid + q * SD_WG, ar = f / (KC / 4), ac = (f % (KC / 4)) * 4;
            if (AF4 < SD_WG && f >= AF4) continue;    // the copies (whole waves)
            const unsigned m = 0u - ((am >> q) & 1u);
            float *as = As[buf] + ar * AS + ac;
            as[0] = __uint_as_float(__float_as_uint(ra[q].x) & m);
            as[1] = __uint_as_float(__float_as_uint(ra[q].y) & m);
            as[2] = __uint_as_float(__float_as_uint(ra[q].z) & m);
            as[3] = __uint_as_float(__float_as_uint(ra[q].w) & m);
        }
#pragma unroll
        for (int q = 0; q < BQ; q++) {
            const int f = tid + q * SD_WG, br = f / (TN / 4), bc = (f % (TN / 4)) * 4;
            const unsigned m = 0u - ((bok >> q) & 1u);
            *reinterpret_cast<float4 *>(Bs[buf] + br * BS + bc) =
                make_float4(__uint_as_float(__float_as_uint(rb[q].x) & m), __uint_as_float(__float_as_uint(rb[q].y) & m),
                            __uint_as_float(__float_as_uint(rb[q].z) & m), __uint_as_float(__float_as_uint(rb[q].w) & m));
        }
    };
    const int wm = (wave / WNW) * (TM / WMW), wn = (wave % WNW) * (TN / WNW);
    const int li = lane & 15, lk = lane >> 4;
    qt_sd_f4 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[i][j] = qt_sd_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < P; s++) fetch(min(s, nch - 1), av[s], bv[s], amk[s]);
    stage(0, av[0], bv[0], amk[0]);
    __syncthreads();
    for (int c0 = 0; c0 < nch; c0 += P) {
#pragma unroll
        for (int s = 0; s < P; s++) {
            const int c = c0 + s;
            // slot s held chunk c, staged one step ago: refill it with chunk c + P (loads
            // issued on every path, so the waits before each stage count them exactly)
            fetch(min(c + P, nch - 1), av[s], bv[s], amk[s]);
            if (c < nch) {
                const float *as = As[s & 1], *bs = Bs[s & 1];
#pragma unroll
                for (int kk = 0; kk < KC; kk += 4) {
                    float fa[MI], fb[NJ];
#pragma unroll
                    for (int i = 0; i < MI; i++) fa[i] = as[(wm + 16 * i + li) * AS + kk + lk];
#pragma unroll
                    for (int j = 0; j < NJ; j++) fb[j] = bs[(kk + lk) * BS + wn + 16 * j + li];
#pragma unroll
                    for (int i = 0; i < MI; i++)
#pragma unroll
                        for (int j = 0; j < NJ; j++)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i], fb[j], acc[i][j], 0, 0, 0);
                }
                if (c + 1 < nch) stage((s & 1) ^ 1, av[(s + 1) % P], bv[(s + 1) % P], amk[(s + 1) % P]);
                __syncthreads();
            }
        }
    }
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int n = n0 + wn + 16 * j + li;
            if (n >= a.N) continue;
            const float bn = (a.epi & SD_EPI_BIAS) ? a.bias[n] : 0.f;
            const float sn = (a.epi & SD_EPI_CSCALE) ? a.cscale[n] : 1.f;
            const float pa = (a.epi & (SD_EPI_SNAKE | SD_EPI_SNAKE2)) ? a.sa[n] : 0.f;
            const float pb = (a.epi & (SD_EPI_SNAKE | SD_EPI_SNAKE2)) ? a.sib[n] : 0.f;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t = t0 + wm + 16 * i + 4 * lk + r;
                if (t >= a.T) continue;
                const size_t o = (size_t)(t * a.os + z) * a.ldy + n;
                float v = acc[i][j][r];
                if (a.epi & SD_EPI_BIAS) v += bn;
                if (a.epi & SD_EPI_GELU) v = sd_gelu(v);
                if (a.epi & SD_EPI_CSCALE) v *= sn;
                if (a.epi & SD_EPI_RESID) v = a.R[o] + v;
                if (a.epi & SD_EPI_SNAKE2) {
                    a.Y[o] = v;
                    a.Y2[o] = sd_snake(v, pa, pb);
                } else {
                    a.Y[o] = (a.epi & SD_EPI_SNAKE) ? sd_snake(v, pa, pb) : v;
                }
            }
        }
}

// ---- elementwise / small kernels ---------------------------------------------------------

// codebook = embedding_sum / max(cluster_usage, 1e-5) (sd.c:383-405), [rows][dim]
__global__ void k_sd_cb_dequant(const float *es, const float *cu, float *cb, int rows, int dim) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < (size_t)rows * dim) cb[i] = es[i] / fmaxf(cu[i / dim], 1e-5f);
}

// exp of the snake log-parameters: a = e^alpha, ib = e^-beta (k.c:4475-4476)
__global__ void k_sd_snake_params(const float *la, const float *lb, float *a, float *ib, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) { a[i] = expf(la[i]); ib[i] = expf(-lb[i]); }
}

// per frame: E[f][0:256] = codebook 0 row, E[f][256:512] = sum of codebooks 1..15 rows in
// order (sd.c:604-625); codes outside [0, 2048) add nothing
__global__ void k_sd_vq(const int *codes, const float *cb, float *E, int cbsize) {
    const int f = blockIdx.x, d = threadIdx.x;        // 256 threads = codebook dim
    const int *c = codes + f * 16;
    const int c0 = c[0];
    E[(size_t)f * 512 + d] = (c0 >= 0 && c0 < cbsize) ? cb[(size_t)c0 * 256 + d] : 0.f;
    float s = 0.f;
    for (int k = 1; k < 16; k++) {
        const int ck = c[k];
        if (ck >= 0 && ck < cbsize) s += cb[((size_t)k * cbsize + ck) * 256 + d];
    }
    E[(size_t)f * 512 + 256 + d] = s;
}

// RMSNorm of rows (qwen_rms_norm, k.c:292-382): out = x * (1/sqrt(mean(x^2) + eps)) * w
__global__ __launch_bounds__(SD_WG) void k_sd_rmsnorm(const float *x, const float *w, float *out, int C, float eps) {
    __shared__ float red[QT_WAVES];
    const float *xr = x + (size_t)blockIdx.x * C;
    float ss = 0.f;
    for (int i = threadIdx.x; i < C; i += SD_WG) ss = fmaf(xr[i], xr[i], ss);
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)C + eps);
    for (int i = threadIdx.x; i < C; i += SD_WG) out[(size_t)blockIdx.x * C + i] = (xr[i] * inv) * w[i];
}

// NeoX split-half RoPE of q and k (columns [0, 1024) and [1024, 2048) of a [.][3072] row),
// 16 heads of 64, tables [pos][32] (sd.c:790-860): rows row0 .. row0 + T - 1 at positions
// pos0 .. pos0 + T - 1
__global__ void k_sd_rope(float *qkv, const float *cs, const float *sn, int T, int row0, int pos0) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;      // (t, which, head, pair)
    if (i >= T * 2 * 16 * 32) return;
    const int pr = i & 31, h = (i >> 5) & 15, which = (i >> 9) & 1, t = i >> 10;
    float *v = qkv + (size_t)(row0 + t) * 3072 + which * 1024 + h * 64;
    const int p = pos0 + t;
    const float c = cs[p * 32 + pr], s = sn[p * 32 + pr];
    const float x1 = v[pr], x2 = v[pr + 32];
    v[pr] = x1 * c - x2 * s;
    v[pr + 32] = x2 * c + x1 * s;
}

// windowed causal attention (qwen_causal_attention_windowed, k.c:3579-3700; seq_q == seq_k,
// q_offset 0): the query at buffer row q0 + t of head h over keys [max(kmin, q0 + t + 1 -
// window), q0 + t] (kmin: the first row holding a key; the streaming decode keeps the
// previous chunks' last window - 1 keys in rows [kmin, q0)).  One wave per (t, h): lanes take
// keys for the scores (dot over 64 dims), then lanes take dims for the weighted sum of values.
__global__ __launch_bounds__(SD_WG) void k_sd_attn(const float *qkv, float *out, int T, int q0, int kmin, int window,
                                                   float scale) {
    __shared__ float sq[QT_WAVES][64];
    __shared__ float sp[QT_WAVES][128];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int item = blockIdx.x * QT_WAVES + wave;
    if (item >= T * 16) return;
    const int t = item >> 4, h = item & 15, qr = q0 + t;
    const int j0 = max(kmin, qr + 1 - window), nk = qr + 1 - j0;   // nk <= window <= 128
    sq[wave][lane] = qkv[(size_t)qr * 3072 + h * 64 + lane];
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    float sc[2];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int j = r * 64 + lane;
        float s = -INFINITY;
        if (j < nk) {
            const float *kr = qkv + (size_t)(j0 + j) * 3072 + 1024 + h * 64;
            float d = 0.f;
            for (int e = 0; e < 64; e += 4) {
                const float4 kv = *reinterpret_cast<const float4 *>(kr + e);
                d = fmaf(sq[wave][e], kv.x, d); d = fmaf(sq[wave][e + 1], kv.y, d);
                d = fmaf(sq[wave][e + 2], kv.z, d); d = fmaf(sq[wave][e + 3], kv.w, d);
            }
            s = d * scale;
        }
        sc[r] = s;
        mx = fmaxf(mx, s);
    }
    mx = group_max<64>(mx);
    float l = 0.f;
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int j = r * 64 + lane;
        const float p = j < nk ? expf(sc[r] - mx) : 0.f;
        sp[wave][j] = p;
        l += p;
    }
    l = group_sum<64>(l);
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    float o = 0.f;
    for (int j = 0; j < nk; j++) o = fmaf(sp[wave][j], qkv[(size_t)(j0 + j) * 3072 + 2048 + h * 64 + lane], o);
    out[(size_t)t * 1024 + h * 64 + lane] = o * (1.0f / l);
}

// m[t][i] = g / (1 + e^-g) * u for the [T][2C] gate|up rows (sd.c:946-950)
__global__ void k_sd_swiglu(const float *gu, float *m, int T, int C) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)T * C) return;
    const size_t t = i / C, c = i % C;
    const float g = gu[t * 2 * C + c], u = gu[t * 2 * C + C + c];
    m[i] = g / (1.0f + expf(-g)) * u;
}

// ConvNeXt: depthwise causal conv (k = 7, pad 6) + LayerNorm over the channels of each
// time step (mean and E[x^2] - mean^2, eps 1e-5), sd.c:1086-1116.  One workgroup per t;
// input rows before xlo (<= 0) read as zero.
__global__ __launch_bounds__(SD_WG) void k_sd_dwln(const float *x, const float *dw, const float *db, const float *lw,
                                                   const float *lb, float *out, int T, int C, int xlo) {
    __shared__ float red[QT_WAVES];
    const int t = blockIdx.x;
    float v[4];
    float s = 0.f, s2 = 0.f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int c = threadIdx.x + q * SD_WG;
        float d = 0.f;
        if (c < C) {
            d = db[c];
            for (int j = 0; j < 7; j++) {
                const int ti = t - 6 + j;
                if (ti >= xlo) d = fmaf(dw[c * 7 + j], x[(size_t)ti * C + c], d);
            }
        }
        v[q] = d;
        s += d;
        s2 = fmaf(d, d, s2);
    }
    s = block_sum(s, red);
    __syncthreads();
    s2 = block_sum(s2, red);
    const float mean = s / (float)C;
    const float var = s2 / (float)C - mean * mean;
    const float inv = 1.0f / sqrtf(var + 1e-5f);
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int c = threadIdx.x + q * SD_WG;
        if (c < C) out[(size_t)t * C + c] = (v[q] - mean) * inv * lw[c] + lb[c];
    }
}

// final conv to one channel (k = 7, pad 6) + clamp to [-1, 1] (sd.c:1259-1279); x [T][C]
// already through the final snake (rows before xlo <= 0 read as zero).  A workgroup takes
// 64 samples: the 70 input rows they
// need go to LDS (row stride C + 1, so the 64 lanes of a read, one row each, hit distinct
// banks); wave w sums channels [w C/4, (w+1) C/4) for its lane's sample, and the four
// partial sums are added in wave order.
#define SD_FIN_T 64
__global__ __launch_bounds__(SD_WG) void k_sd_final(const float *x, const float *w, const float *b, float *audio, int T,
                                                    int C, int xlo) {
    extern __shared__ float xs[];                        // [70][C + 1]
    __shared__ float part[QT_WAVES][SD_FIN_T];
    const int t0 = blockIdx.x * SD_FIN_T, ld = C + 1;
    for (int i = threadIdx.x; i < (SD_FIN_T + 6) * C; i += SD_WG) {
        const int r = i / C, c = i % C, ti = t0 - 6 + r;
        xs[r * ld + c] = (ti >= xlo && ti < T) ? x[(size_t)ti * C + c] : 0.f;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int cw = C / QT_WAVES, c0 = wave * cw;
    float s = 0.f;
    for (int c = c0; c < c0 + cw; c++)
#pragma unroll
        for (int j = 0; j < 7; j++) s = fmaf(w[c * 7 + j], xs[(lane + j) * ld + c], s);
    part[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && t0 + lane < T) {
        const float v = b[0] + part[0][lane] + part[1][lane] + part[2][lane] + part[3][lane];
        audio[t0 + lane] = fminf(fmaxf(v, -1.0f), 1.0f);
    }
}

// streaming history: the last H rows of a buffer's [H + T] rows become its first H rows.
// Source and destination overlap when T < H (a chunk of fewer new rows than the history),
// so a workgroup owns 64 columns whole: its four waves read all H rows of them into
// registers (loads of every row in flight at once), wait for the data, meet at one
// barrier, and only then store.  No other workgroup touches those columns.
#define SD_SHIFT_MAXH 96
__global__ __launch_bounds__(SD_WG) void k_sd_shift(float *buf, int H, int T, int C) {
    constexpr int NR = SD_SHIFT_MAXH / 4;
    const int c = blockIdx.x * 64 + (threadIdx.x & 63), r0 = threadIdx.x >> 6;
    float v[NR];
#pragma unroll
    for (int i = 0; i < NR; i++) {
        const int r = r0 + 4 * i;
        v[i] = (c < C && r < H) ? buf[(size_t)(T + r) * C + c] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < NR; i++) asm volatile("" : "+v"(v[i]));   // every load has returned
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NR; i++) {
        const int r = r0 + 4 * i;
        if (c < C && r < H) buf[(size_t)r * C + c] = v[i];
    }
}

// ---- launchers ----------------------------------------------------------------------------

// tile: 0 = by size (128 x 128 where that still gives two workgroups per CU, else the
// largest of 64, 32, 16 rows x 64 columns that fills the CUs), 16, 32, 64 or 128 = forced.
// Every tile sums each output's products in the same order, so the choice never changes
// a result bit.
extern "C" hipError_t qt_launch_sd_gemm(const float *X, int ldx, int Tx, int xlo, const float *W, int K, int N, int ntap,
                                        const int *off, int phases, int T, float *Y, int ldy, const float *bias,
                                        const float *cscale, const float *R, const float *sa, const float *sib,
                                        float *Y2, int epi, int tile, hipStream_t st) {
    if (!X || !W || !Y || K <= 0 || K % SD_KC || N <= 0 || N % 4 || ntap < 1 || ntap > SD_MAXTAP || phases < 1 ||
        T <= 0 || Tx <= 0 || xlo > 0 || ldx % 4 || ldx < K || ldy < N)
        return hipErrorInvalidValue;
    if (((epi & 1) && !bias) || ((epi & 4) && !cscale) || ((epi & 8) && !R)) return hipErrorInvalidValue;
    if ((epi & (SD_EPI_SNAKE | SD_EPI_SNAKE2)) && (!sa || !sib)) return hipErrorInvalidValue;
    if ((epi & SD_EPI_SNAKE2) && (!Y2 || (epi & SD_EPI_SNAKE))) return hipErrorInvalidValue;
    SdGemmArgs a;
    a.X = X; a.ldx = ldx; a.Tx = Tx; a.xlo = xlo; a.W = W; a.K = K; a.N = N; a.ntap = ntap;
    for (int i = 0; i < SD_MAXTAP; i++) a.off[i] = i < ntap ? off[i] : 0;
    a.T = T; a.Y = Y; a.ldy = ldy; a.os = phases; a.bias = bias; a.cscale = cscale; a.R = R; a.epi = epi;
    a.sa = sa; a.sib = sib; a.Y2 = Y2;
    const long long nt = (long long)((N + 63) / 64) * phases;
    const long long big = (long long)((T + 127) / 128) * ((N + 127) / 128) * phases;
    if (tile == 0) {
        // the largest row tile whose grid still gives every CU a workgroup: a streaming
        // chunk of a few frames leaves T at 10..320 rows, where 64-row tiles would be
        // mostly padding on a few dozen CUs
        if (N >= 128 && big >= 512) tile = 128;
        else if ((T + 63) / 64 * nt >= 256) tile = 64;
        else if ((T + 31) / 32 * nt >= 256) tile = 32;
        else tile = 16;
    }
    if (tile == 128) {
        dim3 grid((T + 127) / 128, (N + 127) / 128, phases);
        hipLaunchKernelGGL((k_sd_gemm<128, 128, 2, 16>), grid, dim3(SD_WG), 0, st, a);
    } else if (tile == 64) {
        dim3 grid((T + 63) / 64, (N + 63) / 64, phases);
        hipLaunchKernelGGL((k_sd_gemm<64, 64, 2, 16>), grid, dim3(SD_WG), 0, st, a);
    } else if (tile == 32 || tile == 16) {
        // the small tiles stage 64-wide K chunks where K allows: a quarter of the barriers
        // and LDS round trips per MFMA (the per-element order is the same)
        dim3 grid((T + tile - 1) / tile, (N + 63) / 64, phases);
        const bool k64 = K % 64 == 0;
        if (tile == 32) {
            if (k64) hipLaunchKernelGGL((k_sd_gemm<32, 64, 4, 64>), grid, dim3(SD_WG), 0, st, a);
            else hipLaunchKernelGGL((k_sd_gemm<32, 64, 8, 16>), grid, dim3(SD_WG), 0, st, a);
        } else {
            if (k64) hipLaunchKernelGGL((k_sd_gemm<16, 64, 4, 64>), grid, dim3(SD_WG), 0, st, a);
            else hipLaunchKernelGGL((k_sd_gemm<16, 64, 8, 16>), grid, dim3(SD_WG), 0, st, a);
        }
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

extern "C" hipError_t qt_launch_sd_cb_dequant(const float *es, const float *cu, float *cb, int rows, int dim,
                                              hipStream_t st) {
    const size_t n = (size_t)rows * dim;
    hipLaunchKernelGGL(k_sd_cb_dequant, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, es, cu, cb, rows, dim);
    return hipGetLastError();
}
extern "C" hipError_t qt_launch_sd_snake_params(const float *la, const float *lb, float *a, float *ib, int n,
                                                hipStream_t st) {
    hipLaunchKernelGGL(k_sd_snake_params, dim3((n + 255) / 256), dim3(256), 0, st, la, lb, a, ib, n);
    return hipGetLastError();
}
extern "C" hipError_t qt_launch_sd_vq(const int *codes, const float *cb, float *E, int n, int cbsize, hipStream_t st) {
    hipLaunchKernelGGL(k_sd_vq, dim3(n), dim3(256), 0, st, codes, cb, E, cbsize);
    return hipGetLastError();
}
extern "C" hipError_t qt_launch_sd_rmsnorm(const float *x, const float *w, float *out, int T, int C, float eps,
                                           hipStream_t st) {
    hipLaunchKernelGGL(k_sd_rmsnorm, dim3(T), dim3(SD_WG), 0, st, x, w, out, C, eps);
    return hipGetLastError();
}
extern "C" hipError_t qt_launch_sd_rope(float *qkv, const float *cs, const float *sn, int T, int row0, int pos0,
                                        hipStream_t st) {
    const int n = T * 1024;
    hipLaunchKernelGGL(k_sd_rope, dim3((n + 255) / 256), dim3(256), 0, st, qkv, cs, sn, T, row0, pos0);
    return hipGetLastError();
}
extern "C" hipError_t qt_launch_sd_attn(const float *qkv, float *out, int T, int q0, int kmin, int window, float scale,
                                        hipStream_t st) {
    if (window <= 0 || window > 128 || kmin < 0 || kmin > q0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_sd_attn, dim3((T * 16 + QT_WAVES - 1) / QT_WAVES), dim3(SD_WG), 0, st, qkv, out, T, q0, kmin,
                       window, scale);
    return hipGetLastError();
}
extern "C" hipError_t qt_launch_sd_swiglu(const float *gu, float *m, int T, int C, hipStream_t st) {
    const size_t n = (size_t)T * C;
    hipLaunchKernelGGL(k_sd_swiglu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, gu, m, T, C);
    return hipGetLastError();
}
extern "C" hipError_t qt_launch_sd_dwln(const float *x, const float *dw, const float *db, const float *lw, const float *lb,
                                        float *out, int T, int C, int xlo, hipStream_t st) {
    if (C > 4 * SD_WG || xlo > 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_sd_dwln, dim3(T), dim3(SD_WG), 0, st, x, dw, db, lw, lb, out, T, C, xlo);
    return hipGetLastError();
}
extern "C" hipError_t qt_launch_sd_final(const float *x, const float *w, const float *b, float *audio, int T, int C,
                                         int xlo, hipStream_t st) {
    if (C % QT_WAVES || C > 256 || xlo > 0) return hipErrorInvalidValue;
    const size_t lds = (size_t)(SD_FIN_T + 6) * (C + 1) * sizeof(float);
    hipLaunchKernelGGL(k_sd_final, dim3((T + SD_FIN_T - 1) / SD_FIN_T), dim3(SD_WG), lds, st, x, w, b, audio, T, C, xlo);
    return hipGetLastError();
}

extern "C" hipError_t qt_launch_sd_shift(float *buf, int H, int T, int C, hipStream_t st) {
    if (H <= 0) return hipSuccess;
    if (H > SD_SHIFT_MAXH || T <= 0 || C <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_sd_shift, dim3((C + 63) / 64), dim3(SD_WG), 0, st, buf, H, T, C);
    return hipGetLastError();
}
