// qt_batch.hip — weight-shared projections for B concurrent decode streams (gfx950).
//
// The batched step (qwen_tts_talker.c:1192-1270, batch_talker_step_impl; CUDA twin
// qwen_tts_cuda_talker.cu:441-560) reads every weight matrix ONCE per step for all B
// streams: Y[b][r] = W[r,:] . X[b][:].  With B = 32 that is a real dense contraction
// (32 x rows x cols), so it runs on the matrix cores with the int8 weights as they are:
//
//   Activation pieces.  Each stream's f32 activation row x (length K) is split exactly
//   into three int8 planes with one power-of-two scale s = 2^(e-6), 2^e <= max|x| < 2^(e+1):
//       x/s = p1 + p2*2^-7 + p3*2^-14 + e3,   p1 in [-128,127], p2,p3 in [0,127],
//       0 <= e3 < 2^-14,
//   every step (scale, floor, subtract, *128) exact in f32 except y - floor(y) for y in
//   (-1/2, 0), which can round by 2^-25 (and, within 2^-25 of 0, up to 1: planes 2 and 3 are
//   held to 127), so |x - s*(p1+p2/128+p3/16384)| < s*(2^-14 + 2^-25) <= max|x| * 2^-19.9.
//   Integer products.  v_mfma_i32_16x16x64_i8 accumulates q*p exactly in int32
//   (|sum| <= 128*128*6144 < 2^31), so the three dot products C1, C2, C3 are exact and
//   independent of summation order; y = s * (C1 + C2/128 + C3/16384) is formed in f64
//   (exact) and rounded once, then multiplied by the row scale as the reference does
//   (qwen_tts_kernels.c:2350-2351).  Against the reference's f32 accumulation the result
//   differs by the f32 rounding of its own sum (~1e-7 relative), nothing systematic.
//
// Layouts.  Weights: the device int8 rows of qt_device.h (signed bytes q), fed to the
// MFMA as they are.  Pieces: [K/64][3*Bp][64] int8, column
// col = piece*Bp + b (Bp = B rounded up to 16; padding columns are zero), so the MFMA B
// operand of N-tile t at k-block kb is one contiguous KiB (16 columns x 64 bytes).
// MFMA operand mapping (16x16x64, wave64): lane l supplies 16 bytes of A row (l % 16)
// and of B column (l % 16) for the same k group (l / 16); lane l receives D rows
// 4*(l/16)+i (i < 4) of column l % 16.  A and B use the same k mapping, so any k order
// within a group gives the same exact integer dot product.
//
// Work split (k_bgemm_i8, any K that is a multiple of 64): one workgroup per 16 weight
// rows, one wave per 512 columns of K, partial int32 tiles summed through LDS.  The
// batched step uses k_bgemm2_i8 (below) where K is a multiple of 1024.
#include "qt_device.h"

typedef int qt_v4i __attribute__((ext_vector_type(4)));

#define QT_BG_KW 512           // K columns per wave
#define QT_BG_MAXW 16          // waves per workgroup at most (K <= 8192)

// ---- activation pieces ---------------------------------------------------------------
// The pieces of one stream are made by a group of QT_BP_T threads (four waves): thread t
// holds the float4 groups g = t + QT_BP_T*j (elements 4g .. 4g+3) in registers, one load
// round; the RMSNorm sum of squares (norm_w != NULL, qwen_tts_kernels.c:292-382) and the
// maximum are one in-wave reduction each plus a four-entry LDS combine in a fixed order,
// so every maker of a stream's pieces (k_bpieces, or the first workgroups of a
// k_bgemm2_i8 launch) produces the same bytes.  Each thread writes its four elements of
// each plane as one dword.  A padding stream (xb == NULL) gets zero pieces and S = 0.
#define QT_BP_T 256            // threads per stream
#define QT_BP_J 8              // float4 groups per thread: K <= 8192
struct BpStream {
    float4 v[QT_BP_J], w[QT_BP_J];
    // issue the loads (x row and gains); the caller may issue other loads before finish()
    __device__ __forceinline__ void load(const float *xb, const float *norm_w, int K, int t) {
        const int ng = K >> 2;
#pragma unroll
        for (int j = 0; j < QT_BP_J; j++) {
            const int g = t + QT_BP_T * j;
            v[j] = (xb && g < ng) ? *reinterpret_cast<const float4 *>(xb + 4 * g) : make_float4(0.f, 0.f, 0.f, 0.f);
            w[j] = (norm_w && g < ng) ? *reinterpret_cast<const float4 *>(norm_w + 4 * g) : make_float4(1.f, 1.f, 1.f, 1.f);
        }
    }
    // plane `plane` of x / s = p1 + p2/128 + p3/16384 + e3 (the exact split of the file header)
    __device__ __forceinline__ static unsigned split(float x, float isc, int plane) {
        const float y = x * isc;                 // |y| < 128, exact
        const float f1 = floorf(y);
        // y - f1 is exact for |y| >= 1 and for y >= 0; for y in (-1/2, 0) it can round,
        // and for -2^-25 < y < 0 it rounds up to 1.0, which would make plane 2 128 (an
        // int8 -128): planes 2 and 3 are held to 127, so p1 + 127/128 + 127/16384 =
        // p1 + 1 - 2^-14 stands for such a y, still within 2^-14 of it
        const float r1 = (y - f1) * 128.0f;      // [0, 128]
        const float f2 = fminf(floorf(r1), 127.0f);
        if (plane == 0) return (unsigned)(int)f1 & 255u;
        if (plane == 1) return (unsigned)(int)f2 & 255u;
        const float r2 = (r1 - f2) * 128.0f;
        return (unsigned)(int)fminf(floorf(r2), 127.0f) & 255u;
    }
    // normalise, scale, split and store; red: 8 floats of LDS owned by this group.
    // Contains one workgroup barrier per reduction (norm must be the same for every group
    // of a workgroup).  AGENT: stores at device scope (read by workgroups on other XCDs in
    // the same launch).
    template <bool AGENT>
    __device__ __forceinline__ void finish(bool norm, float eps, int K, int b, int Bp, int8_t *P, float *S, float *red,
                                           int t) {
        const int lane = t & 63, wv = t >> 6, ng = K >> 2;
        if (norm) {
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < QT_BP_J; j++) {
                ss = fmaf(v[j].x, v[j].x, ss); ss = fmaf(v[j].y, v[j].y, ss);
                ss = fmaf(v[j].z, v[j].z, ss); ss = fmaf(v[j].w, v[j].w, ss);
            }
            ss = group_sum<64>(ss);
            if (lane == 0) red[wv] = ss;
            __syncthreads();
            const float inv = 1.0f / sqrtf((((red[0] + red[1]) + red[2]) + red[3]) / (float)K + eps);
#pragma unroll
            for (int j = 0; j < QT_BP_J; j++) {
                v[j].x = (v[j].x * inv) * w[j].x; v[j].y = (v[j].y * inv) * w[j].y;
                v[j].z = (v[j].z * inv) * w[j].z; v[j].w = (v[j].w * inv) * w[j].w;
            }
        }
        float m = 0.f;
#pragma unroll
        for (int j = 0; j < QT_BP_J; j++)
            m = fmaxf(fmaxf(m, fmaxf(fabsf(v[j].x), fabsf(v[j].y))), fmaxf(fabsf(v[j].z), fabsf(v[j].w)));
        m = group_max<64>(m);
        if (lane == 0) red[4 + wv] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
        // s = 2^(e-6) with 2^e <= m < 2^(e+1); m == 0 (or not finite) -> all pieces zero
        const bool ok = m > 0.f && m <= 3.0e38f;
        const int ex = ok ? ilogbf(m) : 0;
        const float sc = ok ? ldexpf(1.0f, ex - 6) : 0.f, isc = ok ? ldexpf(1.0f, 6 - ex) : 0.f;
        const size_t cs = (size_t)3 * Bp * 64;
#pragma unroll
        for (int j = 0; j < QT_BP_J; j++) {
            const int g = t + QT_BP_T * j;
            if (g >= ng) break;
            unsigned q[3] = {0u, 0u, 0u};
            if (ok) {
#pragma unroll
                for (int p = 0; p < 3; p++)
                    q[p] = split(v[j].x, isc, p) | split(v[j].y, isc, p) << 8 | split(v[j].z, isc, p) << 16 |
                           split(v[j].w, isc, p) << 24;
            }
            const int k0 = 4 * g;
            unsigned *d = reinterpret_cast<unsigned *>(P + (size_t)(k0 >> 6) * cs + (size_t)b * 64 + (k0 & 63));
#pragma unroll
            for (int p = 0; p < 3; p++) {
                if (AGENT) __hip_atomic_store(d + p * Bp * 16, q[p], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else d[p * Bp * 16] = q[p];
            }
        }
        if (t == 0) {
            if (AGENT) st_agent(S + b, sc);
            else S[b] = sc;
        }
    }
};

// One QT_BP_T-thread workgroup per padded stream b < Bp; x row b at x + b*xstride;
// norm_w != NULL: the pieces are of RMSNorm(x)*w, else of x.
__global__ __launch_bounds__(QT_BP_T) void k_bpieces(const float *x, long long xstride, const float *norm_w, float eps,
                                                     int K, int B, int Bp, int8_t *P, float *S) {
    __shared__ float red[8];
    const int b = blockIdx.x;
    BpStream bs;
    bs.load(b < B ? x + (size_t)b * xstride : nullptr, norm_w, K, threadIdx.x);
    bs.finish<false>(norm_w != nullptr, eps, K, b, Bp, P, S, red, threadIdx.x);
}

// ---- int8 weights x activation pieces --------------------------------------------------
struct QtBgArgs {
    const uint8_t *w;     // device int8 rows (signed q), [rows][K]
    const float *scale;   // [rows]
    int rows, K;
    const int8_t *P;      // pieces [K/64][3*Bp][64]
    const float *S;       // [Bp]
    int B;
    float *out;           // STORE: out[b*ostride + r]; SWIGLU: out[b*ostride + r/2]; RESID: out[b*ostride + r] +=
    long long ostride;
};

template <int NT, int EPI>
__global__ __launch_bounds__(QT_BG_MAXW * 64) void k_bgemm_i8(QtBgArgs a) {
    constexpr int BP = NT * 16 / 3;                // padded streams
    __shared__ int red[NT][4][64];                 // summed int32 tiles
    const int nw = blockDim.x >> 6;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r0 = blockIdx.x * 16;
    const int m = lane & 15, grp = lane >> 4;
    const int row = min(r0 + m, a.rows - 1);       // rows past the end repeat the last (discarded)
    const uint8_t *wr = a.w + (size_t)row * a.K;
    const size_t cs = (size_t)3 * BP * 64;

    qt_v4i acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = qt_v4i{0, 0, 0, 0};
    const int kw0 = wave * QT_BG_KW;
    const int nkb = max(0, min(QT_BG_KW, a.K - kw0)) >> 6;   // wave-uniform
    // the wave's weights (8 k-blocks of 16 rows x 64 bytes) all in flight at once
    uint4 wa[QT_BG_KW / 64];
#pragma unroll
    for (int kb = 0; kb < QT_BG_KW / 64; kb++)
        wa[kb] = kb < nkb ? *reinterpret_cast<const uint4 *>(wr + kw0 + kb * 64 + grp * 16) : make_uint4(0, 0, 0, 0);
    // B fragments: every load of a full 512-column slice is unconditional, so the
    // compiler can issue them ahead of the MFMAs that consume them
    auto block = [&](int kb) {
        const int k = kw0 + kb * 64;
        const qt_v4i A = qt_v4i{(int)wa[kb].x, (int)wa[kb].y, (int)wa[kb].z, (int)wa[kb].w};
        const int8_t *pb = a.P + (size_t)(k >> 6) * cs + (size_t)m * 64 + grp * 16;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const uint4 pv = *reinterpret_cast<const uint4 *>(pb + (size_t)t * 16 * 64);
            const qt_v4i Bv = qt_v4i{(int)pv.x, (int)pv.y, (int)pv.z, (int)pv.w};
            acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, Bv, acc[t], 0, 0, 0);
        }
    };
    if (nkb == QT_BG_KW / 64) {
#pragma unroll
        for (int kb = 0; kb < QT_BG_KW / 64; kb++) block(kb);
    } else {
#pragma unroll
        for (int kb = 0; kb < QT_BG_KW / 64; kb++)
            if (kb < nkb) block(kb);
    }
    // sum the waves' tiles (exact; wave 0 stores, the others add in wave order)
    for (int w = 0; w < nw; w++) {
        if (wave == w) {
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) red[t][i][lane] = (w == 0 ? 0 : red[t][i][lane]) + acc[t][i];
        }
        __syncthreads();
    }
    // epilogue: thread j -> (local row j / BP, stream j % BP)
    for (int j = tid; j < 16 * BP; j += blockDim.x) {
        const int rl = j / BP, b = j % BP, r = r0 + rl;
        if (b >= a.B || r >= a.rows) continue;
        if (EPI == QT_EPI_SWIGLU && (rl & 1)) continue;
        auto val = [&](int rr) -> float {   // rr: local row
            const int t0 = b >> 4, ln = (rr >> 2) * 16 + (b & 15), i = rr & 3;
            const double c = (double)red[t0][i][ln] + (double)red[t0 + BP / 16][i][ln] * (1.0 / 128.0) +
                             (double)red[t0 + 2 * BP / 16][i][ln] * (1.0 / 16384.0);
            const float dot = (float)(c * (double)a.S[b]);
            return __fmul_rn(dot, a.scale[r0 + rr]);
        };
        float *ob = a.out + (size_t)b * a.ostride;
        if (EPI == QT_EPI_STORE) ob[r] = val(rl);
        else if (EPI == QT_EPI_RESID) ob[r] = __fadd_rn(ob[r], val(rl));
        else if (EPI == QT_EPI_SWIGLU) {
            const float g = val(rl), u = val(rl + 1);
            ob[r >> 1] = g / (1.0f + expf(-g)) * u;
        }
    }
}

// ---- int8 weights x activation pieces, tall tiles and split K --------------------------
// The batched step's projections have 2048-12288 rows and K = 1024..6144.  A workgroup
// of QT_B2_W waves owns RT row tiles (16*RT rows) and one of S equal K ranges; wave w
// takes KB consecutive k-blocks of 64 of that range.  Every weight fragment and every B
// fragment of the wave is issued at entry (all of a workgroup's HBM and L2 traffic in
// flight at once: one memory latency, not one per k-block), together with the
// epilogue's operands (row scales, stream scales, the residual rows), so the only
// dependent round trip left is the split-K hand-off.  Each B fragment feeds the RT row
// tiles.  After the MFMAs each wave parks its int32 tiles in LDS; one barrier; then
// each thread sums, over the waves, the three plane sums of the outputs it writes and
// folds them into one exact integer T = C1*2^14 + C2*2^7 + C3 (|T| < 2^42), so that
// s * (C1 + C2/128 + C3/16384) = s * T * 2^-14 is formed exactly in f64 and rounded
// once, as in k_bgemm_i8.  With S > 1 each workgroup publishes its T values (agent-scope
// stores), counts itself in with a device-scope atomic, and the last of the S
// workgroups of a row group adds the others' T (integers: the order cannot change the
// result; all of its loads are issued before any is added) and writes the outputs, then
// re-arms the counter for the next call.  Outputs of one workgroup are numbered
// unit u = b * NRU + q (stream b, row q; SwiGLU: row pair q), so consecutive threads
// write consecutive rows of one stream.
#define QT_B2_W 8
struct QtBg2Args {
    const uint8_t *w; const float *scale;
    int rows, K;
    const int8_t *P; const float *S;
    int B;
    float *out; long long ostride;
    long long *part;    // S > 1: [gridDim.x][S][units][1 or 2] exact sums
    unsigned *cnt;      // S > 1: [gridDim.x], zero between calls
    // Pieces made in the same launch (px != NULL): the pieces of px (rows of pxstride,
    // RMS-normalised with pnorm when it is set) are written to P and S by the launch itself.
    const float *px; long long pxstride; const float *pnorm; float eps;
    unsigned *sync;     // px: word 0 the makers' count, word 32*(1+g) workgroup g's go flag (one
                        // 128-byte line each); all zero between calls
    unsigned *err;      // px: set to 1 if a wait for the pieces gave up
};

// registers of a (NT, RT, KB) wave: B fragments, weight fragments, accumulators
__host__ __device__ constexpr int qt_b2_regs(int nt, int rt, int kb) { return 4 * (kb * nt + rt * kb + rt * nt); }
// LDS row of 64 ints (one accumulator register of a 16x16 tile) padded to 68, so the
// sums that read the same register of 16 consecutive rows hit 16 different banks
#define QT_B2_ROW 68
__host__ __device__ constexpr bool qt_b2_ok(int nt, int rt, int kb) {
    return qt_b2_regs(nt, rt, kb) <= 220 && QT_B2_W * rt * nt * 4 * QT_B2_ROW * 4 <= 159 * 1024;
}

template <int NT, int EPI, int RT, int KB>
__global__ __launch_bounds__(QT_B2_W * 64) void k_bgemm2_i8(QtBg2Args a) {
    constexpr int BP = NT * 16 / 3, NTH = QT_B2_W * 64, NR = 16 * RT;
    constexpr int TILE = RT * NT * 4 * QT_B2_ROW;     // ints of one wave's tiles (padded rows)
    constexpr bool SW = EPI == QT_EPI_SWIGLU;
    constexpr int NRU = SW ? NR / 2 : NR;             // output rows (SwiGLU: row pairs)
    constexpr int NU = NRU * BP, PU = (NU + NTH - 1) / NTH, H = SW ? 2 : 1;
    __shared__ int wred[QT_B2_W][TILE];
    __shared__ unsigned last_flag;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m = lane & 15, grp = lane >> 4;
    const int x = blockIdx.x, z = blockIdx.y, S = gridDim.y;
    const int r0 = x * NR;
    const int kw0 = z * (a.K / S) + wave * KB * 64;
    const size_t cs = (size_t)3 * BP * 64;

    // In-launch pieces: workgroups 0 .. BP/2-1 in dispatch order (blockIdx.x fastest) each
    // make the pieces of streams 2i and 2i+1 (one per half of the workgroup: every 128-byte
    // line of P is written by one workgroup), store them at device scope, wait for the
    // stores to be acknowledged and count themselves in; the last maker to count in re-arms
    // the count and raises every workgroup's go flag (one line per workgroup: no line is
    // polled by more than one workgroup).  Every workgroup issues its weight loads first,
    // then waits for its flag and clears it.  The makers never wait before they publish and
    // are dispatched before every waiter, so the wait ends.  The B fragments are then read
    // with ordinary loads: no L2 holds a line of P when the launch starts (the launch
    // boundary's cache maintenance, which the two-launch form relies on too) and none is
    // filled before the flags rise, except by its one maker.  The scales S are read at
    // device scope.
    const bool fold = a.px != nullptr;
    const int lin = x + gridDim.x * z;
    __shared__ float bp_red[2][8];
    __shared__ unsigned mk_last;
    BpStream bs;
    const bool maker = fold && lin < BP / 2;
    const int bmk = 2 * lin + (tid >> 8);                  // maker: its stream
    if (maker) bs.load(bmk < a.B ? a.px + (size_t)bmk * a.pxstride : nullptr, a.pnorm, a.K, tid & (QT_BP_T - 1));
    uint4 wa[RT][KB];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const uint8_t *wr = a.w + (size_t)min(r0 + 16 * rt + m, a.rows - 1) * a.K + kw0 + grp * 16;
#pragma unroll
        for (int kb = 0; kb < KB; kb++) wa[rt][kb] = *reinterpret_cast<const uint4 *>(wr + kb * 64);
    }
    if (fold) {
        if (maker) {
            bs.finish<true>(a.pnorm != nullptr, a.eps, a.K, bmk, BP, const_cast<int8_t *>(a.P), const_cast<float *>(a.S),
                            bp_red[tid >> 8], tid & (QT_BP_T - 1));
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (tid == 0)
                mk_last = __hip_atomic_fetch_add(&a.sync[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                          (unsigned)(BP / 2 - 1);
            __syncthreads();
            if (mk_last) {   // every maker's stores are acknowledged
                if (tid == 0) __hip_atomic_store(&a.sync[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                for (int i = tid; i < (int)(gridDim.x * gridDim.y); i += NTH)
                    __hip_atomic_store(&a.sync[32 * (1 + i)], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        if (tid == 0) {
            unsigned *flag = &a.sync[32 * (1 + lin)], spins = 0;
            while (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u) {
                if (++spins > (1u << 21)) {   // seconds: a maker is missing; flag it and go on
                    __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            __hip_atomic_store(flag, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
    }
    const int8_t *pbase = a.P + (size_t)(kw0 >> 6) * cs + (size_t)m * 64 + grp * 16;
    uint4 bv[KB][NT];
#pragma unroll
    for (int kb = 0; kb < KB; kb++)
#pragma unroll
        for (int t = 0; t < NT; t++) bv[kb][t] = *reinterpret_cast<const uint4 *>(pbase + (size_t)kb * cs + (size_t)t * 16 * 64);
    // epilogue operands of this thread's units
    float e_sc[PU][H], e_S[PU], e_res[PU];
#pragma unroll
    for (int u = 0; u < PU; u++) {
        const int j = tid + u * NTH, b = j / NRU, r = r0 + (SW ? 2 : 1) * (j % NRU);
        const bool ok = j < NU && b < a.B && r < a.rows;
#pragma unroll
        for (int h = 0; h < H; h++) e_sc[u][h] = ok ? a.scale[r + h] : 0.f;
        e_S[u] = ok ? (fold ? ld_agent(a.S + b) : a.S[b]) : 0.f;
        e_res[u] = (ok && EPI == QT_EPI_RESID) ? a.out[(size_t)b * a.ostride + r] : 0.f;
    }
    qt_v4i acc[RT][NT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[rt][t] = qt_v4i{0, 0, 0, 0};
#pragma unroll
    for (int kb = 0; kb < KB; kb++)
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const qt_v4i A = qt_v4i{(int)wa[rt][kb].x, (int)wa[rt][kb].y, (int)wa[rt][kb].z, (int)wa[rt][kb].w};
#pragma unroll
            for (int t = 0; t < NT; t++)
                acc[rt][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                    A, qt_v4i{(int)bv[kb][t].x, (int)bv[kb][t].y, (int)bv[kb][t].z, (int)bv[kb][t].w}, acc[rt][t], 0, 0, 0);
        }
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) wred[wave][((rt * NT + t) * 4 + i) * QT_B2_ROW + lane] = acc[rt][t][i];
    __syncthreads();
    // exact sums of this thread's outputs: D row 4(l/16)+i, column l%16 of tile (rt, t)
    long long T[PU][H];
#pragma unroll
    for (int u = 0; u < PU; u++) {
        const int j = tid + u * NTH, b = j / NRU, q = j % NRU;
#pragma unroll
        for (int h = 0; h < H; h++) {
            long long v = 0;
            if (j < NU) {
                const int rr = (SW ? 2 : 1) * q + h, rt = rr >> 4, lr = rr & 15;
                const int e = ((rt * NT + (b >> 4)) * 4 + (lr & 3)) * QT_B2_ROW + (lr >> 2) * 16 + (b & 15);
                int c[3] = {0, 0, 0};
#pragma unroll
                for (int w = 0; w < QT_B2_W; w++)
#pragma unroll
                    for (int p = 0; p < 3; p++) c[p] += wred[w][e + p * (BP / 16) * 4 * QT_B2_ROW];
                v = (long long)c[0] * 16384 + (long long)c[1] * 128 + (long long)c[2];
            }
            T[u][h] = v;
        }
    }
    if (S > 1) {
        long long *mine = a.part + ((size_t)x * S + z) * NU * H;
#pragma unroll
        for (int u = 0; u < PU; u++)
#pragma unroll
            for (int h = 0; h < H; h++)
                if (tid + u * NTH < NU)
                    __hip_atomic_store(mine + (size_t)(tid + u * NTH) * H + h, T[u][h], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        // Ordering without release/acquire fences: the partials are agent-scope atomic
        // stores (sc1: written through to the device coherence point, never left dirty in
        // an XCD's L2), the count is incremented only after s_waitcnt has seen every one of
        // them acknowledged, and the last workgroup reads the others' partials with
        // agent-scope atomic loads (sc1: not served from a stale L1/L2 line) issued after
        // its own increment returned the final count.  An agent-scope acq_rel increment
        // plus acquire fence would add an L2 write-back and invalidate per workgroup:
        // measured 3.07 -> 3.35 ms per batched step (32 ragged streams, 1.7B int8).
        if (tid == 0)
            last_flag = __hip_atomic_fetch_add(&a.cnt[x], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                        (unsigned)(S - 1);
        __syncthreads();
        if (!last_flag) return;
        for (int zz = 0; zz < S; zz++) {
            if (zz == z) continue;
            const long long *other = a.part + ((size_t)x * S + zz) * NU * H;
            long long t[PU][H];
#pragma unroll
            for (int u = 0; u < PU; u++)
#pragma unroll
                for (int h = 0; h < H; h++)
                    t[u][h] = (tid + u * NTH < NU)
                                  ? __hip_atomic_load(other + (size_t)(tid + u * NTH) * H + h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                  : 0;
#pragma unroll
            for (int u = 0; u < PU; u++)
#pragma unroll
                for (int h = 0; h < H; h++) T[u][h] += t[u][h];
        }
        if (tid == 0) __hip_atomic_store(&a.cnt[x], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int u = 0; u < PU; u++) {
        const int j = tid + u * NTH, b = j / NRU, r = r0 + (SW ? 2 : 1) * (j % NRU);
        if (j >= NU || b >= a.B || r >= a.rows) continue;
        float y[H];
#pragma unroll
        for (int h = 0; h < H; h++) {
            const float dot = (float)((double)T[u][h] * 0x1p-14 * (double)e_S[u]);
            y[h] = __fmul_rn(dot, e_sc[u][h]);
        }
        float *ob = a.out + (size_t)b * a.ostride;
        if (EPI == QT_EPI_STORE) ob[r] = y[0];
        else if (EPI == QT_EPI_RESID) ob[r] = __fadd_rn(e_res[u], y[0]);
        else ob[r >> 1] = y[0] / (1.0f + expf(-y[0])) * y[H - 1];
    }
}

// The tiling qt_launch_bgemm2_i8 uses for a (rows, K) projection: KB k-blocks per wave,
// S K ranges, RT row tiles per workgroup.  KB is the largest of {6, 4, 2} dividing
// K/512 whose fragments fit the register budget; K ranges are split further (KB 4 -> 2,
// 6 -> 2) while fewer than 128 workgroups would run; RT grows to 3 while more than 256
// row-tile jobs remain per full grid and the registers and LDS allow.  Returns 0 if the
// shape has none (K not a multiple of 1024, or no NT for Bp), else fills the workspace
// it needs (ints of the split-K sums and counters; 0 when S == 1).
extern "C" int qt_bgemm2_plan(int rows, int K, int Bp, int *kb, int *S, int *rt, size_t *part_ints, int *n_cnt) {
    if (rows <= 0 || K <= 0 || K % 1024 || (Bp != 16 && Bp != 32 && Bp != 48 && Bp != 64)) return 0;
    const int NT = 3 * Bp / 16, nblk = K / 512;
    int KB = 0;
    const int cand[3] = {6, 4, 2};
    for (int i = 0; i < 3 && !KB; i++)
        if (nblk % cand[i] == 0 && qt_b2_ok(NT, 1, cand[i])) KB = cand[i];
    if (!KB) return 0;
    int SS = nblk / KB;
    const int tiles = (rows + 15) / 16;
    if (tiles * SS < 128 && KB > 2) { SS *= KB / 2; KB = 2; }
    int RT = tiles * SS / 256;
    RT = RT < 1 ? 1 : RT > 3 ? 3 : RT;
    while (RT > 1 && !qt_b2_ok(NT, RT, KB)) RT--;
    const int gx = (tiles + RT - 1) / RT;
    *kb = KB; *S = SS; *rt = RT;
    *part_ints = SS > 1 ? (size_t)gx * SS * 16 * RT * Bp * 2 : 0;
    *n_cnt = SS > 1 ? gx : 0;
    return 1;
}

template <int NT, int E, int RT, int KB>
static void qt_b2_go(const QtBg2Args &a, dim3 grid, hipStream_t st, hipError_t &err) {
    if constexpr (qt_b2_ok(NT, RT, KB))
        hipLaunchKernelGGL((k_bgemm2_i8<NT, E, RT, KB>), grid, dim3(QT_B2_W * 64), 0, st, a);
    else
        err = hipErrorInvalidValue;
}
template <int NT, int E, int RT>
static void qt_b2_kb(int KB, const QtBg2Args &a, dim3 grid, hipStream_t st, hipError_t &err) {
    if (KB == 6) qt_b2_go<NT, E, RT, 6>(a, grid, st, err);
    else if (KB == 4) qt_b2_go<NT, E, RT, 4>(a, grid, st, err);
    else qt_b2_go<NT, E, RT, 2>(a, grid, st, err);
}
template <int NT, int E>
static void qt_b2_rt(int RT, int KB, const QtBg2Args &a, dim3 grid, hipStream_t st, hipError_t &err) {
    if (RT == 1) qt_b2_kb<NT, E, 1>(KB, a, grid, st, err);
    else if (RT == 2) qt_b2_kb<NT, E, 2>(KB, a, grid, st, err);
    else qt_b2_kb<NT, E, 3>(KB, a, grid, st, err);
}
template <int NT>
static void qt_b2_epi(int epi, int RT, int KB, const QtBg2Args &a, dim3 grid, hipStream_t st, hipError_t &err) {
    if (epi == QT_EPI_STORE) qt_b2_rt<NT, QT_EPI_STORE>(RT, KB, a, grid, st, err);
    else if (epi == QT_EPI_RESID) qt_b2_rt<NT, QT_EPI_RESID>(RT, KB, a, grid, st, err);
    else if (epi == QT_EPI_SWIGLU) qt_b2_rt<NT, QT_EPI_SWIGLU>(RT, KB, a, grid, st, err);
    else err = hipErrorInvalidValue;
}

// part / cnt: workspace from qt_bgemm2_plan (cnt zeroed once at allocation; the kernel
// re-arms it).  Returns hipErrorInvalidValue for shapes without a plan.
static hipError_t b2_launch(int epi, const uint8_t *w, const float *scale, int rows, int K, const float *px,
                            long long pxstride, const float *pnorm, float eps, const int8_t *P, const float *S, int B,
                            int Bp, float *out, long long ostride, int *part, unsigned *cnt, unsigned *sync,
                            int sync_wgs, unsigned *derr, hipStream_t st) {
    int KB, SS, RT, ncnt; size_t pints;
    if (rows <= 0 || B <= 0 || B > Bp || !qt_bgemm2_plan(rows, K, Bp, &KB, &SS, &RT, &pints, &ncnt)) return hipErrorInvalidValue;
    if (epi == QT_EPI_SWIGLU && (rows & 1)) return hipErrorInvalidValue;
    if (SS > 1 && (!part || !cnt)) return hipErrorInvalidValue;
    QtBg2Args a;
    a.w = w; a.scale = scale; a.rows = rows; a.K = K; a.P = P; a.S = S; a.B = B; a.out = out; a.ostride = ostride;
    a.part = reinterpret_cast<long long *>(part); a.cnt = cnt;
    a.px = px; a.pxstride = pxstride; a.pnorm = pnorm; a.eps = eps; a.sync = sync; a.err = derr;
    const dim3 grid(((rows + 15) / 16 + RT - 1) / RT, SS);
    // the in-launch pieces need Bp/2 makers, all in the first row of the grid, and the
    // pieces routine's register row (K <= 8192)
    if (px && (!sync || !derr || (int)grid.x < Bp / 2 || (int)(grid.x * grid.y) > sync_wgs ||
               K > QT_BP_T * 4 * QT_BP_J)) return hipErrorInvalidValue;
    hipError_t err = hipSuccess;
    if (Bp == 16) qt_b2_epi<3>(epi, RT, KB, a, grid, st, err);
    else if (Bp == 32) qt_b2_epi<6>(epi, RT, KB, a, grid, st, err);
    else if (Bp == 48) qt_b2_epi<9>(epi, RT, KB, a, grid, st, err);
    else qt_b2_epi<12>(epi, RT, KB, a, grid, st, err);
    if (err != hipSuccess) return err;
    return hipGetLastError();
}

extern "C" hipError_t qt_launch_bgemm2_i8(int epi, const uint8_t *w, const float *scale, int rows, int K,
                                          const int8_t *P, const float *S, int B, int Bp, float *out, long long ostride,
                                          int *part, unsigned *cnt, hipStream_t st) {
    return b2_launch(epi, w, scale, rows, K, nullptr, 0, nullptr, 0.f, P, S, B, Bp, out, ostride, part, cnt, nullptr, 0,
                     nullptr, st);
}

// The same with the activation pieces made inside the launch (one launch instead of
// qt_launch_bpieces + qt_launch_bgemm2_i8, same bytes in P and S, same outputs): x rows
// of xstride, RMS-normalised with norm_w when it is set.  sync: two zeroed words that the
// kernel re-arms; err: set to 1 if a wait for the pieces gave up (the outputs are then
// invalid).  Needs a grid of at least Bp/2 row groups and sync of 32*(1 + sync_wgs) words
// with sync_wgs at least the launch's workgroups (qt_bgemm2_px_wgs).
extern "C" hipError_t qt_launch_bgemm2_i8_px(int epi, const uint8_t *w, const float *scale, int rows, int K,
                                             const float *x, long long xstride, const float *norm_w, float eps, int8_t *P,
                                             float *S, int B, int Bp, float *out, long long ostride, int *part,
                                             unsigned *cnt, unsigned *sync, int sync_wgs, unsigned *err,
                                             hipStream_t st) {
    if (!x) return hipErrorInvalidValue;
    return b2_launch(epi, w, scale, rows, K, x, xstride, norm_w, eps, P, S, B, Bp, out, ostride, part, cnt, sync,
                     sync_wgs, err, st);
}

// Workgroups of the qt_launch_bgemm2_i8_px launch for the shape, 0 if it does not take it.
extern "C" int qt_bgemm2_px_wgs(int rows, int K, int Bp) {
    int KB, SS, RT, nc; size_t pi;
    if (!qt_bgemm2_plan(rows, K, Bp, &KB, &SS, &RT, &pi, &nc)) return 0;
    const int gx = ((rows + 15) / 16 + RT - 1) / RT;
    return gx >= Bp / 2 && K <= QT_BP_T * 4 * QT_BP_J ? gx * SS : 0;
}

// ---- q4_0 weights x activation pieces -------------------------------------------------
// Y[b][r] = sum over 32-blocks j of d[r][j] * sum_{k in j} (nib[r][k] - 8) * x[b][k]
// (qwen_matmat_q4_0, qwen_tts_kernels.c:1954; dequant (nib-8)*f16(scale), k.c:2810-2819),
// weights read once for all streams.  (nib - 8) is an exact int8, so each block's three
// piece sums C1, C2, C3 are exact int32 MFMA results; C = C1*2^14 + C2*2^7 + C3 is exact in
// int32 (|C| < 2^30), and x = s * 2^-14 * (p1*2^14 + p2*2^7 + p3) gives the block's dot as
// s * 2^-14 * C: one rounding to f32 per block, then d * 2^-14 (exact: a power-of-two
// multiple of an f16) folded in by one fma into the f32 row sum.  The block scale must
// stay outside the integer sum, so every MFMA covers one block: the 64-k operand of
// v_mfma_i32_16x16x64_i8 spans two blocks (lane groups 0-1 and 2-3), and two MFMAs take
// the same B fragment with the other block's A lanes zeroed.
// Weight layout: the device q4 rows (qt_device.h) -- K/2 bytes per row, byte i holds
// elements 2i (low nibble) and 2i+1 (high) -- and f16 scale bits s16[rows][K/32].
struct QtBgQ4Args {
    const uint8_t *w;       // [rows][K/2]
    const uint16_t *s16;    // [rows][K/32]
    int rows, K;
    const int8_t *P;        // pieces [K/64][3*Bp][64]
    const float *S;         // [Bp]
    int B;
    float *out;
    long long ostride;
};

// 8 bytes of q4 (16 nibbles, elements e0..e15 in order) -> 16 int8 (e - 8), element order
__device__ __forceinline__ qt_v4i q4_unpack16(uint2 w) {
    const uint32_t l0 = ((w.x & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;   // bytes: e0 e2 e4 e6 (minus 8)
    const uint32_t h0 = (((w.x >> 4) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;   // e1 e3 e5 e7
    const uint32_t l1 = ((w.y & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
    const uint32_t h1 = (((w.y >> 4) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
    // v_perm_b32(hi, lo, sel): selector bytes 0-3 pick lo's bytes, 4-7 hi's
    return qt_v4i{(int)__builtin_amdgcn_perm(h0, l0, 0x05010400u), (int)__builtin_amdgcn_perm(h0, l0, 0x07030602u),
                  (int)__builtin_amdgcn_perm(h1, l1, 0x05010400u), (int)__builtin_amdgcn_perm(h1, l1, 0x07030602u)};
}

// KB k-blocks of 64 per wave, at most 8 waves (KB = 16 for K > 4096), so a lane may hold
// 256 registers: a ring of RING blocks' B fragments, the block's MFMA results and the q4
// weights.  Every load a block needs is issued well before it: the weights of all KB
// blocks and the first RING blocks' B fragments at entry (a consumed ring slot is refilled
// with the block RING ahead; indices clamped to the last block instead of guarded, so the
// loads are straight-line code and the compiler counts them), and the workgroup's block
// scales go to LDS at entry, so no block waits on a dependent global load.
#define QT_BQ_MAXW 8
template <int NT, int EPI, int KB>
__global__ __launch_bounds__(QT_BQ_MAXW * 64) void k_bgemm_q4(QtBgQ4Args a) {
    constexpr int BP = NT * 16 / 3, NS = BP / 16;   // padded streams, stream tiles
    constexpr int RING = KB < 30 / NT ? KB : (30 / NT > 2 ? 30 / NT : 2);
    __shared__ float wred[QT_BQ_MAXW][NS][4][64];   // each wave's partial row sums
    __shared__ float sres[16 * BP], sS[BP];         // residual rows [row][stream], stream scales
    __shared__ float ssc[16][QT_BQ_MAXW * KB * 2];  // block scales x 2^-14 of the 16 rows
    const int nw = blockDim.x >> 6;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r0 = blockIdx.x * 16;
    const int m = lane & 15, grp = lane >> 4;
    const int row = min(r0 + m, a.rows - 1);       // rows past the end repeat the last (discarded)
    const int nb32 = a.K >> 5;
    const uint8_t *wr = a.w + (size_t)row * (a.K >> 1);
    const size_t cs = (size_t)3 * BP * 64;
    const int kw0 = wave * KB * 64;
    const int nkb = max(0, min(KB * 64, a.K - kw0)) >> 6;   // wave-uniform

    const int kl = max(nkb - 1, 0);                          // last block of this wave (clamp)
    uint2 wq[KB];
#pragma unroll
    for (int kb = 0; kb < KB; kb++)
        wq[kb] = *reinterpret_cast<const uint2 *>(wr + ((kw0 + min(kb, kl) * 64) >> 1) + grp * 8);
    // B fragments of block kb, ring slot kb % RING
    auto loadB = [&](qt_v4i (&Bv)[NT], int kb) {
        const int8_t *pb = a.P + (size_t)((kw0 >> 6) + kb) * cs + (size_t)m * 64 + grp * 16;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const uint4 pv = *reinterpret_cast<const uint4 *>(pb + (size_t)t * 16 * 64);
            Bv[t] = qt_v4i{(int)pv.x, (int)pv.y, (int)pv.z, (int)pv.w};
        }
    };
    qt_v4i Br[RING][NT];
#pragma unroll
    for (int r = 0; r < RING; r++) loadB(Br[r], min(r, kl));
    // block scales of the workgroup's 16 rows, times 2^-14, into LDS
    for (int i = tid; i < 16 * nb32; i += (int)blockDim.x) {
        const int rl = i / nb32, b = i % nb32;
        ssc[rl][b] = ref_f16_to_f32(a.s16[(size_t)min(r0 + rl, a.rows - 1) * nb32 + b]) * 0x1p-14f;
    }

    // the epilogue's operands (stream scales, residual rows) into LDS right behind the
    // weight loads, instead of one dependent load per output at the end
    for (int i = tid; i < 16 * BP; i += (int)blockDim.x) {
        const int rl = i / BP, b = i % BP, r = r0 + rl;
        sres[i] = (EPI == QT_EPI_RESID && b < a.B && r < a.rows) ? a.out[(size_t)b * a.ostride + r] : 0.f;
    }
    for (int i = tid; i < BP; i += (int)blockDim.x) sS[i] = i < a.B ? a.S[i] : 0.f;
    __syncthreads();                                // block scales in LDS
    float acc[NS][4];
#pragma unroll
    for (int s = 0; s < NS; s++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[s][i] = 0.f;
    // one block's three piece sums -> C = C1*2^14 + C2*2^7 + C3 (exact), times d*2^-14 into acc
    auto fold = [&](const qt_v4i (&c)[NT], int blk) {
        float d[4];
#pragma unroll
        for (int i = 0; i < 4; i++) d[i] = ssc[4 * grp + i][(kw0 >> 5) + blk];
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int v = (c[s][i] << 14) + (c[NS + s][i] << 7) + c[2 * NS + s][i];
                acc[s][i] = fmaf((float)v, d[i], acc[s][i]);
            }
    };
    auto block = [&](int kb, const qt_v4i (&Bv)[NT]) {
        const qt_v4i A = q4_unpack16(wq[kb]);
        const qt_v4i Z = qt_v4i{0, 0, 0, 0};
        const qt_v4i A0 = grp < 2 ? A : Z, A1 = grp < 2 ? Z : A;
        qt_v4i c[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) c[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, Bv[t], Z, 0, 0, 0);
        fold(c, 2 * kb);
#pragma unroll
        for (int t = 0; t < NT; t++) c[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, Bv[t], Z, 0, 0, 0);
        fold(c, 2 * kb + 1);
    };
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
        if (kb < nkb) block(kb, Br[kb % RING]);   // wave-uniform; a guard, not a break, so the loop unrolls fully
        if (kb + RING < KB) loadB(Br[kb % RING], min(kb + RING, kl));
        __builtin_amdgcn_sched_barrier(0);
    }
    // the waves' partial row sums: each wave parks its own, one barrier, then every output
    // is summed over the waves in wave order from 0.0f (the order fixes the f32 result)
#pragma unroll
    for (int s = 0; s < NS; s++)
#pragma unroll
        for (int i = 0; i < 4; i++) wred[wave][s][i][lane] = acc[s][i];
    __syncthreads();
    auto val = [&](int rr, int b) -> float {
        float t = 0.f;
        for (int w = 0; w < nw; w++) t += wred[w][b >> 4][rr & 3][(rr >> 2) * 16 + (b & 15)];
        return t * sS[b];
    };
    for (int j = tid; j < 16 * BP; j += (int)blockDim.x) {
        const int rl = j / BP, b = j % BP, r = r0 + rl;
        if (b >= a.B || r >= a.rows) continue;
        if (EPI == QT_EPI_SWIGLU && (rl & 1)) continue;
        float *ob = a.out + (size_t)b * a.ostride;
        if (EPI == QT_EPI_STORE) ob[r] = val(rl, b);
        else if (EPI == QT_EPI_RESID) ob[r] = __fadd_rn(sres[j], val(rl, b));
        else if (EPI == QT_EPI_SWIGLU) {
            const float g = val(rl, b), u = val(rl + 1, b);
            ob[r >> 1] = g / (1.0f + expf(-g)) * u;
        }
    }
}

extern "C" hipError_t qt_launch_bgemm_q4(int epi, const uint8_t *w, const uint16_t *s16, int rows, int K,
                                         const int8_t *P, const float *S, int B, int Bp, float *out, long long ostride,
                                         hipStream_t st) {
    if (rows <= 0 || K <= 0 || (K & 63) || K > 16 * 64 * QT_BQ_MAXW || B <= 0 || B > Bp) return hipErrorInvalidValue;
    if (epi == QT_EPI_SWIGLU && (rows & 1)) return hipErrorInvalidValue;
    QtBgQ4Args a;
    a.w = w; a.s16 = s16; a.rows = rows; a.K = K; a.P = P; a.S = S; a.B = B; a.out = out; a.ostride = ostride;
    const int kb = K > 8 * 64 * QT_BQ_MAXW ? 16 : 8;
    const int nw = (K + kb * 64 - 1) / (kb * 64);
    dim3 grid((rows + 15) / 16), block(nw * 64);
#define QT_BQ_KB(NT_, E_)                                                                              \
    if (kb == 8) hipLaunchKernelGGL((k_bgemm_q4<NT_, E_, 8>), grid, block, 0, st, a);                   \
    else hipLaunchKernelGGL((k_bgemm_q4<NT_, E_, 16>), grid, block, 0, st, a);
#define QT_BQ_CASE(NT_)                                                                                   \
    if (epi == QT_EPI_STORE) { QT_BQ_KB(NT_, QT_EPI_STORE) }                                              \
    else if (epi == QT_EPI_RESID) { QT_BQ_KB(NT_, QT_EPI_RESID) }                                         \
    else if (epi == QT_EPI_SWIGLU) { QT_BQ_KB(NT_, QT_EPI_SWIGLU) }                                       \
    else return hipErrorInvalidValue;
    if (Bp == 16) { QT_BQ_CASE(3) }
    else if (Bp == 32) { QT_BQ_CASE(6) }
    else if (Bp == 48) { QT_BQ_CASE(9) }
    else if (Bp == 64) { QT_BQ_CASE(12) }
    else return hipErrorInvalidValue;
#undef QT_BQ_CASE
#undef QT_BQ_KB
    return hipGetLastError();
}

extern "C" hipError_t qt_launch_bpieces(const float *x, long long xstride, const float *norm_w, float eps, int K, int B,
                                        int Bp, int8_t *P, float *S, hipStream_t st) {
    if (K <= 0 || (K & 63) || B <= 0 || Bp < B || (Bp & 15) || Bp > 64) return hipErrorInvalidValue;
    if (K > QT_BP_T * 4 * QT_BP_J) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_bpieces, dim3(Bp), dim3(QT_BP_T), 0, st, x, xstride, norm_w, eps, K, B, Bp, P, S);
    return hipGetLastError();
}

// Bp: padded stream count of the pieces (16, 32, 48, 64).
extern "C" hipError_t qt_launch_bgemm_i8(int epi, const uint8_t *w, const float *scale, int rows, int K,
                                         const int8_t *P, const float *S, int B, int Bp, float *out,
                                         long long ostride, hipStream_t st) {
    if (rows <= 0 || K <= 0 || (K & 63) || K > QT_BG_KW * QT_BG_MAXW || B <= 0 || B > Bp) return hipErrorInvalidValue;
    if (epi == QT_EPI_SWIGLU && (rows & 1)) return hipErrorInvalidValue;
    QtBgArgs a;
    a.w = w; a.scale = scale; a.rows = rows; a.K = K; a.P = P; a.S = S; a.B = B; a.out = out; a.ostride = ostride;
    const int nw = (K + QT_BG_KW - 1) / QT_BG_KW;
    dim3 grid((rows + 15) / 16), block(nw * 64);
#define QT_BG_CASE(NT_)                                                                                   \
    if (epi == QT_EPI_STORE) hipLaunchKernelGGL((k_bgemm_i8<NT_, QT_EPI_STORE>), grid, block, 0, st, a);   \
    else if (epi == QT_EPI_RESID) hipLaunchKernelGGL((k_bgemm_i8<NT_, QT_EPI_RESID>), grid, block, 0, st, a); \
    else if (epi == QT_EPI_SWIGLU) hipLaunchKernelGGL((k_bgemm_i8<NT_, QT_EPI_SWIGLU>), grid, block, 0, st, a); \
    else return hipErrorInvalidValue;
    if (Bp == 16) { QT_BG_CASE(3) }
    else if (Bp == 32) { QT_BG_CASE(6) }
    else if (Bp == 48) { QT_BG_CASE(9) }
    else if (Bp == 64) { QT_BG_CASE(12) }
    else return hipErrorInvalidValue;
#undef QT_BG_CASE
    return hipGetLastError();
}

// pos[b] += 1 for b < n: the batched step's device positions advance after each step,
// so replays of a captured step walk every stream forward by one position.
__global__ void k_advance_pos(int *pos, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) pos[i] += 1;
}
extern "C" hipError_t qt_launch_advance_pos(int *pos, int n, hipStream_t st) {
    if (n <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_advance_pos, dim3((n + 63) / 64), dim3(64), 0, st, pos, n);
    return hipGetLastError();
}
