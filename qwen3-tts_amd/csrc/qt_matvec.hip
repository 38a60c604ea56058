// qt_matvec.hip — weight-streaming matvec kernels for the decode step (gfx950).
//
// One kernel family covers every projection of a Talker / Code-Predictor layer:
//   y = W . f(v)   with  f = identity or RMSNorm(v)*g   (NORM)
// and an epilogue (EPI):
//   STORE   y[r] = acc                        (QKV, logits)
//   RESID   x[r] += acc                       (O and down projections, residual add)
//   SWIGLU  h[i] = silu(acc[2i]) * acc[2i+1]  (interleaved gate|up rows)
//   BIAS    y[r] = acc + bias[r]              (CP small_to_mtp_projection)
// Numerics follow the reference CPU path: f32 activations, f32 accumulation (bf16,
// q4_0); int8 weights meet the activation as exact int8 pieces (qt_device.h) summed in
// int32, so the dot is the exact one to ~2^-27 relative; the int8 row scale is applied
// once per row (qwen_tts_kernels.c:2350-2351), q4 block value
// (nib-8)*f16(scale) (qwen_tts_kernels.c:2810-2819), SwiGLU g/(1+expf(-g))*u
// (qwen_tts_kernels.c:3857-3878), RMSNorm (x*inv)*w (qwen_tts_kernels.c:292-382).
//
// Work split: a wave owns NR*(64/LPR) consecutive rows; each row is split over LPR
// lanes, lane `sub` holding the 16-byte chunks c = sub + LPR*j (j < CPL) of it, so
// NR*CPL independent 128-bit weight loads are in flight per lane and consecutive lanes
// read consecutive 16-byte chunks (1 KiB per wave per load instruction).
// Latency (about 1 us per cold miss on MI355X) is paid once: every load the wave needs
// (weights, its slice of the input vector, norm gains, row scales, residual values) is
// issued at entry, before any of them is consumed.  The input slice a lane needs is
// exactly the columns of its chunks, read straight from global memory (coalesced; the
// four waves of a workgroup share it through L1), and an LPR-lane group covers the whole
// vector, so the RMSNorm statistic is a group reduction: no LDS staging, no barrier.
#include "qt_device.h"

template <int PREC> struct QtPrec;
template <> struct QtPrec<QT_BF16> { static constexpr int EPC = 8; };
template <> struct QtPrec<QT_INT8> { static constexpr int EPC = 16; };
template <> struct QtPrec<QT_Q4> { static constexpr int EPC = 32; };

__device__ __forceinline__ size_t qt_row_bytes(int prec, int cols) {
    return prec == QT_BF16 ? (size_t)cols * 2 : prec == QT_INT8 ? (size_t)cols : (size_t)cols / 2;
}

struct QtMvArgs {
    const float *vin;    // input vector [cols]
    const float *nw;     // RMSNorm gain [cols] (NORM)
    float eps;
    QtMat M;
    float *out;          // STORE/SWIGLU/BIAS output
    float *resid;        // RESID target
    const float *bias;   // BIAS
    float *nout;         // NORM: if set, workgroup 0 / wave 0 also writes RMSNorm(vin)*nw here
};

template <int EPI>
__device__ __forceinline__ void qt_epilogue(const QtMvArgs &a, int row, float acc) {
    if (EPI == QT_EPI_STORE) a.out[row] = acc;
    else if (EPI == QT_EPI_RESID) a.resid[row] += acc;
    else if (EPI == QT_EPI_BIAS) a.out[row] = acc + a.bias[row];
}

__device__ __forceinline__ float qt_silu_mul(float g, float u) {
    return g / (1.0f + expf(-g)) * u;
}

template <int PREC, int LPR, int CPL, int NR, int EPI, bool NORM>
__global__ __launch_bounds__(QT_WG) void k_mv(QtMvArgs a) {
    constexpr int EPC = QtPrec<PREC>::EPC;
    constexpr int RPW = NR * (64 / LPR);
    constexpr int COLS = LPR * CPL * EPC;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = lane / LPR, sub = lane % LPR;
    const int row0 = (blockIdx.x * QT_WAVES + wave) * RPW + grp * NR;
    const int rows = a.M.rows;
    constexpr size_t rb = PREC == QT_BF16 ? (size_t)COLS * 2 : PREC == QT_INT8 ? (size_t)COLS : (size_t)COLS / 2;

    // ---- every load up front ----
    uint4 wv[NR][CPL];
    float sc[NR][CPL];
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const int row = row0 + r;
#pragma unroll
        for (int j = 0; j < CPL; j++) {
            const int c = sub + LPR * j;
            if (row < rows) {
                wv[r][j] = ld_chunk(a.M.w + (size_t)row * rb + (size_t)c * 16);
                if (PREC == QT_Q4) sc[r][j] = ref_f16_to_f32(a.M.s16[(size_t)row * (COLS / 32) + c]);
            } else {
                wv[r][j] = make_uint4(0, 0, 0, 0);
                sc[r][j] = 0.f;
            }
        }
    }
    float4 xv[CPL][EPC / 4];
    float4 gv[CPL][EPC / 4];
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        const int c = sub + LPR * j;
#pragma unroll
        for (int q = 0; q < EPC / 4; q++) {
            xv[j][q] = *reinterpret_cast<const float4 *>(a.vin + c * EPC + 4 * q);
            if (NORM) gv[j][q] = *reinterpret_cast<const float4 *>(a.nw + c * EPC + 4 * q);
        }
    }
    float rsc[NR], rres[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const int row = row0 + r;
        const bool ok = sub == 0 && row < rows;
        rsc[r] = (PREC == QT_INT8 && ok) ? a.M.scale[row] : 1.0f;
        rres[r] = ((EPI == QT_EPI_RESID || EPI == QT_EPI_BIAS) && ok)
                      ? (EPI == QT_EPI_RESID ? a.resid[row] : a.bias[row]) : 0.f;
    }

    // ---- input slice (RMS-normalised when NORM) in element order ----
    float xe[CPL][EPC];
#pragma unroll
    for (int j = 0; j < CPL; j++)
#pragma unroll
        for (int q = 0; q < EPC / 4; q++) {
            xe[j][4 * q + 0] = xv[j][q].x; xe[j][4 * q + 1] = xv[j][q].y;
            xe[j][4 * q + 2] = xv[j][q].z; xe[j][4 * q + 3] = xv[j][q].w;
        }
    float pc_m = 0.f;       // int8: bound of max|input| for the pieces' scale
    if (NORM) {
        float ss = 0.f;
        if (PREC == QT_INT8) {
            // the fused step's order (its gather): virtual thread t = lane + 64 w (w < 4)
            // accumulates x[t + 256 k]^2 over k, butterfly per w, the four sums in order;
            // the scale bound is inv * max|x*g| * (1 + 2^-20) (qt_pstep.hip, pc_norm_scale)
            static_assert(PREC != QT_INT8 || (LPR == 64 && COLS % 256 == 0), "int8 norm order");
            float mg = 0.f;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                float p = 0.f;
#pragma unroll
                for (int k = 0; k < COLS / 256; k++) {
                    const float v = a.vin[lane + 64 * w + 256 * k];
                    p = fmaf(v, v, p);
                }
                ss = w == 0 ? group_sum<64>(p) : ss + group_sum<64>(p);
            }
#pragma unroll
            for (int j = 0; j < CPL; j++)
#pragma unroll
                for (int q = 0; q < EPC / 4; q++) {
                    mg = fmaxf(mg, fabsf(xv[j][q].x * gv[j][q].x)); mg = fmaxf(mg, fabsf(xv[j][q].y * gv[j][q].y));
                    mg = fmaxf(mg, fabsf(xv[j][q].z * gv[j][q].z)); mg = fmaxf(mg, fabsf(xv[j][q].w * gv[j][q].w));
                }
            pc_m = group_max<LPR>(mg);
        } else {
#pragma unroll
            for (int j = 0; j < CPL; j++)
#pragma unroll
                for (int e = 0; e < EPC; e++) ss = fmaf(xe[j][e], xe[j][e], ss);
            ss = group_sum<LPR>(ss);
        }
        const float inv = 1.0f / sqrtf(ss / (float)COLS + a.eps);
        if (PREC == QT_INT8) pc_m = (inv * pc_m) * (1.0f + 0x1p-20f);
#pragma unroll
        for (int j = 0; j < CPL; j++)
#pragma unroll
            for (int q = 0; q < EPC / 4; q++) {
                xe[j][4 * q + 0] = (xe[j][4 * q + 0] * inv) * gv[j][q].x;
                xe[j][4 * q + 1] = (xe[j][4 * q + 1] * inv) * gv[j][q].y;
                xe[j][4 * q + 2] = (xe[j][4 * q + 2] * inv) * gv[j][q].z;
                xe[j][4 * q + 3] = (xe[j][4 * q + 3] * inv) * gv[j][q].w;
            }
        if (a.nout && blockIdx.x == 0 && wave == 0 && grp == 0) {
#pragma unroll
            for (int j = 0; j < CPL; j++)
#pragma unroll
                for (int q = 0; q < EPC / 4; q++)
                    *reinterpret_cast<float4 *>(a.nout + (sub + LPR * j) * EPC + 4 * q) =
                        make_float4(xe[j][4 * q], xe[j][4 * q + 1], xe[j][4 * q + 2], xe[j][4 * q + 3]);
        }
    }
    // int8: the exact pieces of the (normalised) input; the maximum is a group reduction
    // (the LPR lanes of a group hold the whole vector), so every group agrees on s
    uint4 pl[PREC == QT_INT8 ? CPL : 1][4];
    float pcs = 0.f;
    if (PREC == QT_INT8) {
        if (!NORM) {
            float mx = 0.f;
#pragma unroll
            for (int j = 0; j < CPL; j++)
#pragma unroll
                for (int e = 0; e < EPC; e++) mx = fmaxf(mx, fabsf(xe[j][e]));
            pc_m = group_max<LPR>(mx);
        }
        const QtPcScale ps = qt_pc_scale(pc_m);
        pcs = ps.s;
#pragma unroll
        for (int j = 0; j < CPL; j++) {
            float v16[16];
#pragma unroll
            for (int e = 0; e < 16; e++) v16[e] = xe[j][e];
            qt_pc16(v16, ps.isc, pl[j]);
        }
    }
    // operand order of the weight chunk: bf16 natural; q4 word m holds elements
    // 8m..8m+7 with the even ones in the low nibbles
    float xr[CPL][EPC];
    float xsum[CPL];
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        if (PREC == QT_INT8) { xsum[j] = 0.f; continue; }
        if (PREC == QT_Q4) {
#pragma unroll
            for (int m = 0; m < 4; m++)
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    xr[j][m * 4 + b] = xe[j][8 * m + 2 * b];
                    xr[j][16 + m * 4 + b] = xe[j][8 * m + 2 * b + 1];
                }
        } else {
#pragma unroll
            for (int e = 0; e < EPC; e++) xr[j][e] = xe[j][e];
        }
        float s = 0.f;
        if (PREC != QT_BF16) {
#pragma unroll
            for (int e = 0; e < EPC; e++) s += xr[j][e];
        }
        xsum[j] = s;
    }

    float acc[NR];
    if (PREC == QT_INT8) {
        // the 4*NR plane sums (row r, plane q at 4r+q), exact in int32
        int d[4 * NR], D[4 * NR];
#pragma unroll
        for (int i = 0; i < 4 * NR; i++) d[i] = 0;
#pragma unroll
        for (int r = 0; r < NR; r++)
#pragma unroll
            for (int j = 0; j < CPL; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) d[4 * r + q] = qt_dot16(wv[r][j], pl[j][q], d[4 * r + q]);
        if constexpr (LPR == 64) {
            wave_sum_i_scatter<4 * NR>(d, D);
        } else {
#pragma unroll
            for (int i = 0; i < 4 * NR; i++) D[i] = group_sum_i<LPR>(d[i]);
        }
#pragma unroll
        for (int r = 0; r < NR; r++) acc[r] = qt_pc_dot(D[4 * r], D[4 * r + 1], D[4 * r + 2], D[4 * r + 3], pcs);
    }
#pragma unroll
    for (int r = 0; r < NR; r++) {
        if (PREC == QT_INT8) continue;
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; j++) {
            const uint32_t w4[4] = {wv[r][j].x, wv[r][j].y, wv[r][j].z, wv[r][j].w};
            if (PREC == QT_BF16) {
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    s = fmaf(bf_lo(w4[m]), xr[j][2 * m], s);
                    s = fmaf(bf_hi(w4[m]), xr[j][2 * m + 1], s);
                }
            } else {
                float t = 0.f;
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    const uint32_t lo = w4[m] & 0x0F0F0F0Fu, hi = (w4[m] >> 4) & 0x0F0F0F0Fu;
                    t = fmaf((float)(lo & 0xFFu), xr[j][m * 4 + 0], t);
                    t = fmaf((float)((lo >> 8) & 0xFFu), xr[j][m * 4 + 1], t);
                    t = fmaf((float)((lo >> 16) & 0xFFu), xr[j][m * 4 + 2], t);
                    t = fmaf((float)(lo >> 24), xr[j][m * 4 + 3], t);
                    t = fmaf((float)(hi & 0xFFu), xr[j][16 + m * 4 + 0], t);
                    t = fmaf((float)((hi >> 8) & 0xFFu), xr[j][16 + m * 4 + 1], t);
                    t = fmaf((float)((hi >> 16) & 0xFFu), xr[j][16 + m * 4 + 2], t);
                    t = fmaf((float)(hi >> 24), xr[j][16 + m * 4 + 3], t);
                }
                s = fmaf(sc[r][j], fmaf(-8.0f, xsum[j], t), s);
            }
        }
        acc[r] = group_sum<LPR>(s);
    }

    if (sub == 0) {
        if (EPI == QT_EPI_SWIGLU) {
#pragma unroll
            for (int r = 0; r < NR; r += 2) {
                const int row = row0 + r;
                if (row + 1 < rows) {
                    const float g = __fmul_rn(acc[r], rsc[r]), u = __fmul_rn(acc[r + 1], rsc[r + 1]);
                    a.out[row >> 1] = qt_silu_mul(g, u);
                }
            }
        } else {
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const int row = row0 + r;
                if (row < rows) {
                    const float v = __fmul_rn(acc[r], rsc[r]);
                    if (EPI == QT_EPI_STORE) a.out[row] = v;
                    else if (EPI == QT_EPI_RESID) a.resid[row] = __fadd_rn(rres[r], v);
                    else a.out[row] = __fadd_rn(v, rres[r]);
                }
            }
        }
    }
}

// Generic fallback for shapes the tuned instantiations do not cover (per-op API with
// arbitrary rows/cols): one wave per row (pair of rows for SWIGLU), lane-strided
// scalar reads, same numerics.
template <int PREC, int EPI, bool NORM>
__global__ __launch_bounds__(QT_WG) void k_mv_generic(QtMvArgs a) {
    extern __shared__ float xs[];
    __shared__ float red[QT_WAVES];
    const int cols = a.M.cols, rows = a.M.rows;
    // staging without the float4 assumption
    float ss = 0.f;
    for (int i = threadIdx.x; i < cols; i += QT_WG) {
        float v = a.vin[i];
        xs[i] = v;
        if (NORM) ss += v * v;
    }
    if (NORM) {
        float tot = block_sum(ss, red);
        float inv = 1.0f / sqrtf(tot / (float)cols + a.eps);
        __syncthreads();
        for (int i = threadIdx.x; i < cols; i += QT_WG) {
            xs[i] = (xs[i] * inv) * a.nw[i];
            if (a.nout && blockIdx.x == 0) a.nout[i] = xs[i];
        }
    }
    __syncthreads();
    QtPcScale ps = {0.f, 0.f};
    if (PREC == QT_INT8) {          // scale of the exact pieces: block maximum of |x|
        float mx = 0.f;
        for (int i = threadIdx.x; i < cols; i += QT_WG) mx = fmaxf(mx, fabsf(xs[i]));
        mx = group_max<64>(mx);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
        __syncthreads();
        mx = 0.f;
#pragma unroll
        for (int i = 0; i < QT_WAVES; i++) mx = fmaxf(mx, red[i]);
        ps = qt_pc_scale(mx);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int per = (EPI == QT_EPI_SWIGLU) ? 2 : 1;
    const int row0 = (blockIdx.x * QT_WAVES + wave) * per;
    float acc[2] = {0.f, 0.f};
    for (int r = 0; r < per; r++) {
        const int row = row0 + r;
        if (row >= rows) break;
        if (PREC == QT_INT8) {
            int d[4] = {0, 0, 0, 0};
            for (int k = lane; k < cols; k += 64) {
                const int q = (int)(int8_t)a.M.w[(size_t)row * cols + k];
                const uint32_t t = qt_pc_word(xs[k], ps.isc);
#pragma unroll
                for (int i = 0; i < 4; i++) d[i] += q * ((int)((t >> (8 * i)) & 0xFFu) - 128);
            }
#pragma unroll
            for (int q = 0; q < 4; q++) d[q] = group_sum_i<64>(d[q]);
            acc[r] = qt_pc_dot(d[0], d[1], d[2], d[3], ps.s) * a.M.scale[row];
            continue;
        }
        float s = 0.f;
        for (int k = lane; k < cols; k += 64) {
            float w;
            if (PREC == QT_BF16) {
                w = bf16f(reinterpret_cast<const uint16_t *>(a.M.w)[(size_t)row * cols + k]);
            } else {
                const uint8_t byte = a.M.w[(size_t)row * (cols / 2) + k / 2];
                const int nib = (k & 1) ? (byte >> 4) : (byte & 0xF);
                w = (float)(nib - 8) * ref_f16_to_f32(a.M.s16[(size_t)row * (cols / 32) + k / 32]);
            }
            s = fmaf(w, xs[k], s);
        }
        acc[r] = group_sum<64>(s);
    }
    if (lane == 0) {
        if (EPI == QT_EPI_SWIGLU) {
            if (row0 + 1 < rows) a.out[row0 >> 1] = qt_silu_mul(acc[0], acc[1]);
        } else if (row0 < rows) {
            qt_epilogue<EPI>(a, row0, acc[0]);
        }
    }
}

// ---------------------------------------------------------------------------------
// q4_0 matvec in the arithmetic of the role-specialised step's q4_0 build (qt_rstep.hip,
// QTile16), so that the per-kernel q4_0 step and the fused one give the same bits: the
// input's exact int8 pieces (the int8 path's scale rule: max|x| or, under RMSNorm, the
// fused step's statistics order and bound), per 32-weight block the exact integer plane
// sums of (n - 8) * piece joined into f = hi * 2^16 + lo (two exact 23-bit halves), and
// per row the blocks' d * f accumulated by fmaf in that kernel's order: the K range in
// four slices, in each slice two chains (blocks 2s + h of the slice, s ascending, h = 0,
// 1), the four slices' chain sums added in slice order per h, the two h sums added, times
// the pieces' scale.  Eight lanes take a row (lane 2w + h runs chain (w, h)), 32 rows per
// workgroup; the pieces of the whole input are made once per workgroup into LDS, each
// 16-column group stored even columns first (the low nibbles' order).
template <int COLS, int EPI, bool NORM>
__global__ __launch_bounds__(QT_WG) void k_mv_q4r(QtMvArgs a) {
    static_assert(COLS % 256 == 0, "four slices of whole block pairs");
    constexpr int NBS = COLS / 128;            // blocks per slice
    constexpr int NS = NBS / 2;                // blocks per chain
    constexpr int EPT = COLS / QT_WG;          // input elements per thread
    __shared__ __align__(16) uint32_t pcw[COLS];   // 4 planes x COLS bytes
    __shared__ float red[2 * QT_WAVES];
    uint8_t *pc = reinterpret_cast<uint8_t *>(pcw);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int k = lane & 7, w = k >> 1, h = k & 1;
    const int row = (blockIdx.x * QT_WAVES + wave) * 8 + (lane >> 3);
    const bool rok = row < a.M.rows;
    // ---- every load up front: the chain's blocks and scales, the input, the gains ----
    uint4 wq[NS];
    float d[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int b = w * NBS + 2 * s + h;
        wq[s] = rok ? ld_chunk(a.M.w + (size_t)row * (COLS / 2) + (size_t)b * 16) : make_uint4(0, 0, 0, 0);
        d[s] = rok ? ref_f16_to_f32(a.M.s16[(size_t)row * (COLS / 32) + b]) : 0.f;
    }
    float x[EPT], g[EPT];
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        x[j] = a.vin[tid + QT_WG * j];
        g[j] = NORM ? a.nw[tid + QT_WG * j] : 1.0f;
    }
    float rres = 0.f;
    if ((EPI == QT_EPI_RESID || EPI == QT_EPI_BIAS) && rok && k == 0)
        rres = EPI == QT_EPI_RESID ? a.resid[row] : a.bias[row];
    // ---- statistics (thread t: elements t + 256 j; waves in order) and the pieces ----
    float ss = 0.f, m = 0.f;
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        if (NORM) ss = fmaf(x[j], x[j], ss);
        m = fmaxf(m, fabsf(NORM ? x[j] * g[j] : x[j]));
    }
    if (NORM) ss = group_sum<64>(ss);
    m = group_max<64>(m);
    if (lane == 0) { red[2 * wave] = ss; red[2 * wave + 1] = m; }
    __syncthreads();
    float inv = 1.f;
    QtPcScale ps;
    {
        float S = red[0], M = red[1];
#pragma unroll
        for (int v = 1; v < QT_WAVES; v++) { S += red[2 * v]; M = fmaxf(M, red[2 * v + 1]); }
        if (NORM) {
            inv = 1.0f / sqrtf(S / (float)COLS + a.eps);
            ps = qt_pc_scale((inv * M) * (1.0f + 0x1p-20f));
        } else {
            ps = qt_pc_scale(M);
        }
    }
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        const int e = tid + QT_WG * j;
        const float v = NORM ? (x[j] * inv) * g[j] : x[j];
        if (NORM && a.nout && blockIdx.x == 0) a.nout[e] = v;
        const uint32_t t = qt_pc_word(v, ps.isc);      // biased digits
        const int pos = 16 * (e >> 4) + ((e & 1) ? 8 : 0) + ((e & 15) >> 1);
#pragma unroll
        for (int q = 0; q < 4; q++) pc[q * COLS + pos] = (uint8_t)(((t >> (8 * q)) & 0xFFu) ^ 0x80u);
    }
    __syncthreads();
    // ---- the chain ----
    float acc = 0.f;
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int b = w * NBS + 2 * s + h;
        const uint32_t w4[4] = {wq[s].x, wq[s].y, wq[s].z, wq[s].w};
        int D[4], P[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint4 p0 = *reinterpret_cast<const uint4 *>(pc + q * COLS + 32 * b);
            const uint4 p1 = *reinterpret_cast<const uint4 *>(pc + q * COLS + 32 * b + 16);
            const uint32_t W[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
            int dq = 0, pq = 0;
#pragma unroll
            for (int mm = 0; mm < 4; mm++) {
                // word mm: elements 8mm .. 8mm+7, even ones in the low nibbles
                const uint32_t ev = W[4 * (mm >> 1) + (mm & 1)], od = W[4 * (mm >> 1) + 2 + (mm & 1)];
                dq = __builtin_amdgcn_sdot4((int)(w4[mm] & 0x0F0F0F0Fu), (int)ev, dq, false);
                dq = __builtin_amdgcn_sdot4((int)((w4[mm] >> 4) & 0x0F0F0F0Fu), (int)od, dq, false);
                pq = __builtin_amdgcn_sdot4((int)ev, 0x01010101, pq, false);
                pq = __builtin_amdgcn_sdot4((int)od, 0x01010101, pq, false);
            }
            D[q] = dq; P[q] = pq;
        }
        const int lo = D[0] + (D[1] << 8) - 8 * (P[0] + 256 * P[1]);
        const int hi = D[2] + (D[3] << 8) - 8 * (P[2] + 256 * P[3]);
        acc = fmaf(d[s], fmaf((float)hi, 65536.f, (float)lo), acc);
    }
    // ---- slices in order per h, then the two h sums, times the pieces' scale ----
    const int base = lane & ~7;
    const float c0 = __shfl(acc, base + h, 64), c1 = __shfl(acc, base + 2 + h, 64);
    const float c2 = __shfl(acc, base + 4 + h, 64), c3 = __shfl(acc, base + 6 + h, 64);
    const float dh = ((c0 + c1) + c2) + c3;
    const float v = (__shfl(dh, base, 64) + __shfl(dh, base + 1, 64)) * ps.s;
    if (EPI == QT_EPI_SWIGLU) {
        const float u = __shfl(v, (lane + 8) & 63, 64);   // the odd row of the pair
        if (k == 0 && ((lane >> 3) & 1) == 0 && row + 1 < a.M.rows) a.out[row >> 1] = qt_silu_mul(v, u);
    } else if (k == 0 && rok) {
        if (EPI == QT_EPI_STORE) a.out[row] = v;
        else if (EPI == QT_EPI_RESID) a.resid[row] = __fadd_rn(rres, v);
        else a.out[row] = __fadd_rn(v, rres);
    }
}

template <int COLS, int EPI, bool NORM>
static hipError_t launch_q4r(const QtMvArgs &a, hipStream_t st) {
    const int grid = (a.M.rows + 8 * QT_WAVES - 1) / (8 * QT_WAVES);
    hipLaunchKernelGGL((k_mv_q4r<COLS, EPI, NORM>), dim3(grid), dim3(QT_WG), 0, st, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// host-side dispatch (C ABI, used by qwen_tts_hip.c)

template <int PREC, int LPR, int CPL, int NR, int EPI, bool NORM>
static hipError_t launch_tuned(const QtMvArgs &a, hipStream_t st) {
    constexpr int RPW = NR * (64 / LPR);
    const int per_wg = RPW * QT_WAVES;
    const int grid = (a.M.rows + per_wg - 1) / per_wg;
    hipLaunchKernelGGL((k_mv<PREC, LPR, CPL, NR, EPI, NORM>), dim3(grid), dim3(QT_WG), 0, st, a);
    return hipGetLastError();
}

template <int PREC, int EPI, bool NORM>
static hipError_t launch_generic(const QtMvArgs &a, hipStream_t st) {
    const int per = (EPI == QT_EPI_SWIGLU) ? 2 : 1;
    const int grid = (a.M.rows + per * QT_WAVES - 1) / (per * QT_WAVES);
    hipLaunchKernelGGL((k_mv_generic<PREC, EPI, NORM>), dim3(grid), dim3(QT_WG),
                       (size_t)a.M.cols * sizeof(float), st, a);
    return hipGetLastError();
}

// Rows per lane-group: the largest of {4, 2, 1} (at most NRMAX) that still gives >= 2048
// waves (two per SIMD on 256 CUs), >= 1024 for int8, whose per-wave input work (norm, max,
// the four activation planes) is shared by more rows that way; SwiGLU needs gate/up row
// pairs, so NR >= 2 there.
template <int PREC, int LPR, int CPL, int NRMAX, int EPI, bool NORM>
static hipError_t launch_nr(const QtMvArgs &a, hipStream_t st) {
    constexpr int G = 64 / LPR;
    constexpr int MW = PREC == QT_INT8 ? 1024 : 2048;
    const int rows = a.M.rows;
    if (NRMAX >= 4 && rows / (4 * G) >= MW) return launch_tuned<PREC, LPR, CPL, 4, EPI, NORM>(a, st);
    if (NRMAX >= 2 && (EPI == QT_EPI_SWIGLU || rows / (2 * G) >= MW))
        return launch_tuned<PREC, LPR, CPL, 2, EPI, NORM>(a, st);
    if (EPI == QT_EPI_SWIGLU) return launch_tuned<PREC, LPR, CPL, 2, EPI, NORM>(a, st);
    return launch_tuned<PREC, LPR, CPL, 1, EPI, NORM>(a, st);
}

// (prec, cols) -> tuned instantiation: one 16-byte chunk per lane per load, CPL chunks
// per row per lane, NR*CPL independent 128-bit loads in flight per lane.
template <int EPI, bool NORM>
static hipError_t dispatch(int prec, const QtMvArgs &a, hipStream_t st) {
    const int c = a.M.cols;
    const bool aligned = ((uintptr_t)a.M.w % 16 == 0) && ((uintptr_t)a.vin % 16 == 0);
    if (aligned) {
        if (prec == QT_BF16) {
            switch (c) {
            case 1024: return launch_nr<QT_BF16, 64, 2, 4, EPI, NORM>(a, st);
            case 2048: return launch_nr<QT_BF16, 64, 4, 2, EPI, NORM>(a, st);
            case 3072: return launch_nr<QT_BF16, 64, 6, 2, EPI, NORM>(a, st);
            case 6144: return launch_nr<QT_BF16, 64, 12, 2, EPI, NORM>(a, st);
            }
        } else if (prec == QT_INT8) {
            switch (c) {
            case 1024: return launch_nr<QT_INT8, 64, 1, 4, EPI, NORM>(a, st);
            case 2048: return launch_nr<QT_INT8, 64, 2, 4, EPI, NORM>(a, st);
            case 3072: return launch_nr<QT_INT8, 64, 3, 4, EPI, NORM>(a, st);
            case 6144: return launch_nr<QT_INT8, 64, 6, 2, EPI, NORM>(a, st);
            }
        } else {
            // q4_0: the fused step's arithmetic and order (k_mv_q4r)
            switch (c) {
            case 1024: return launch_q4r<1024, EPI, NORM>(a, st);
            case 2048: return launch_q4r<2048, EPI, NORM>(a, st);
            case 3072: return launch_q4r<3072, EPI, NORM>(a, st);
            case 6144: return launch_q4r<6144, EPI, NORM>(a, st);
            }
        }
    }
    if (prec == QT_BF16) return launch_generic<QT_BF16, EPI, NORM>(a, st);
    if (prec == QT_INT8) return launch_generic<QT_INT8, EPI, NORM>(a, st);
    return launch_generic<QT_Q4, EPI, NORM>(a, st);
}

extern "C" hipError_t qt_launch_mv(int prec, int epi, int norm, const float *vin, const float *nw,
                                   float eps, const uint8_t *w, const float *scale,
                                   const uint16_t *s16, int rows, int cols, float *out,
                                   float *resid, const float *bias, float *nout, hipStream_t st) {
    QtMvArgs a;
    a.vin = vin; a.nw = nw; a.eps = eps;
    a.M.w = w; a.M.scale = scale; a.M.s16 = s16; a.M.rows = rows; a.M.cols = cols;
    a.out = out; a.resid = resid; a.bias = bias; a.nout = nout;
    if (rows <= 0 || cols <= 0) return hipErrorInvalidValue;
    if (epi == QT_EPI_SWIGLU && (rows & 1)) return hipErrorInvalidValue;
    if (prec == QT_Q4 && (cols % 32)) return hipErrorInvalidValue;
    if ((size_t)cols * sizeof(float) > 64 * 1024) return hipErrorInvalidValue;
    switch (epi) {
    case QT_EPI_STORE: return norm ? dispatch<QT_EPI_STORE, true>(prec, a, st) : dispatch<QT_EPI_STORE, false>(prec, a, st);
    case QT_EPI_RESID: return norm ? dispatch<QT_EPI_RESID, true>(prec, a, st) : dispatch<QT_EPI_RESID, false>(prec, a, st);
    case QT_EPI_SWIGLU: return norm ? dispatch<QT_EPI_SWIGLU, true>(prec, a, st) : dispatch<QT_EPI_SWIGLU, false>(prec, a, st);
    case QT_EPI_BIAS: return norm ? dispatch<QT_EPI_BIAS, true>(prec, a, st) : dispatch<QT_EPI_BIAS, false>(prec, a, st);
    }
    return hipErrorInvalidValue;
}
