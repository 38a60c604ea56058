// qt_prefill.hip — Talker prefill (qwen_talker_prefill, qwen_tts_talker.c:730-1038) on gfx950.
//
// The reference runs the prompt's positions as dense projections Y[seq][out] =
// Xn[seq][in] . W^T over the bf16 layer weights with f32 sums (sgemm or
// qwen_matmat_bf16, t.c:845-847, 913, 964, 990), per-head q/k RMSNorm, NeoX RoPE at each
// position, the bf16-truncated K/V store (t.c:897-899), causal attention over the f32
// q/k/v (t.c:901-907), O + residual, RMSNorm + gate|up + SwiGLU, down + residual.
//
// Projections here run on the bf16 matrix cores.  The f32 activations are split
// into three bf16 planes whose sum is each value exactly (x truncated to bf16, the
// truncated rest, the remaining <= 8 significant bits; qt_attn_mf.h); W . x = sum over
// the planes of W . x_p, and each bf16 x bf16 product is exact in f32, so the three
// MFMAs per k-step accumulate, in f32, the exact products of the f32 activations with
// the bf16 weights.  Both operands are read row-major exactly as stored: the MFMA A
// operand is 16 weight rows x 8 consecutive k, the B operand 16 positions x 8
// consecutive k of one plane, so neither needs a transpose.
#include "qt_attn_mf.h"

#define QT_PF_WG 256

// ---- activation planes ---------------------------------------------------------------
// Row s < S of X (ldx floats apart), optionally RMS-normalised with gain (the reference's
// qwen_rms_norm: out = (x * inv) * w, inv = 1/sqrt(mean(x^2) + eps), k.c:292-382), as
// three bf16 planes P[p][s][K] (plane stride Sp*K); rows S <= s < Sp are zero.
__global__ __launch_bounds__(QT_PF_WG) void k_pf_pieces(const float *X, int ldx, int S, int Sp, int K,
                                                         const float *gain, float eps, uint16_t *P) {
    __shared__ float red[QT_WAVES];
    const int s = blockIdx.x, tid = threadIdx.x;
    const size_t plane = (size_t)Sp * K;
    uint16_t *p0 = P + (size_t)s * K;
    if (s >= S) {
        for (int k = tid * 8; k < K; k += QT_PF_WG * 8)
#pragma unroll
            for (int p = 0; p < 3; p++) *reinterpret_cast<uint4 *>(p0 + p * plane + k) = make_uint4(0u, 0u, 0u, 0u);
        return;
    }
    const float *x = X + (size_t)s * ldx;
    float inv = 1.0f;
    if (gain) {
        float ss = 0.f;
        for (int k = tid; k < K; k += QT_PF_WG) ss = fmaf(x[k], x[k], ss);
        ss = block_sum(ss, red);
        inv = 1.0f / sqrtf(ss / (float)K + eps);
    }
    for (int k = tid * 4; k < K; k += QT_PF_WG * 4) {
        float4 v = *reinterpret_cast<const float4 *>(x + k);
        if (gain) {
            const float4 g = *reinterpret_cast<const float4 *>(gain + k);
            v.x = (v.x * inv) * g.x; v.y = (v.y * inv) * g.y; v.z = (v.z * inv) * g.z; v.w = (v.w * inv) * g.w;
        }
        uint16_t pc[3][4];
        const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; i++) qt_put_pieces(&pc[0][i], 4, e[i]);
#pragma unroll
        for (int p = 0; p < 3; p++)
            *reinterpret_cast<uint2 *>(p0 + p * plane + k) =
                make_uint2((uint32_t)pc[p][0] | ((uint32_t)pc[p][1] << 16), (uint32_t)pc[p][2] | ((uint32_t)pc[p][3] << 16));
    }
}

// ---- projection GEMM ------------------------------------------------------------------
// Y = X . W^T: W bf16 [N][K] row-major, X as the planes P[3][Sp][K].  Workgroup tile:
// 64*NR weight rows x 64 positions; wave w takes rows [16*NR*w, 16*NR*(w+1)) of it and
// every position; the weight fragments go straight from HBM to registers (each wave reads
// its own rows once), the planes' tile is shared through LDS.
//   PF_STORE   Y[s][n] = acc
//   PF_RESID   Y[s][n] += acc                     (O, down: the residual stream)
//   PF_SWIGLU  rows 2i, 2i+1 are gate_i, up_i (the reference's interleaved gate|up,
//              t.c:378-388): Y[s][i] = g / (1 + e^-g) * u  (qwen_swiglu_inplace, k.c:3857)
// (the same values as in qt_launch.h, which the .hip sources do not include)
enum { QT_PF_STORE = 0, QT_PF_RESID = 1, QT_PF_SWIGLU = 2 };

// NST chunks of 64 k are in flight: each chunk's planes (3 x 64
// positions x 128 B) go straight from HBM into LDS stage c % NST by global_load_lds (no
// registers; lane L of a 1-KiB copy fills slot L%8 of row 8b + L/8 and fetches the chunk
// that belongs there: chunk c of row r sits at slot c ^ ((r >> 1) & 7), so the 16 lanes of
// a B-operand read (rows j, one chunk) hit 16 different bank groups), and its weight
// fragments into registers, NST - 1 chunks ahead.  One barrier per chunk: after the wait
// for chunk c, every wave is also done with chunk c - 1, whose stage takes chunk
// c + NST - 1.  blockIdx.z selects one of gridDim.z equal K ranges (split K): with
// PF_PART the workgroup stores its partial tile at Y + z * S * ldy (k_pf_reduce adds the
// ranges in order).
enum { QT_PF_PART = 3 };
template <int N>
__device__ __forceinline__ void qt_vmcnt() {   // wait until at most N vector-memory ops are outstanding
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Two waves per SIMD for the two-stage tile (amdgpu_waves_per_eu(2)): the 256-row tile
// with two stages fits in 202 registers per lane, so two workgroups share a CU and hide
// each other's chunk waits (the three-stage 256-row tile held 304 registers, one wave per
// SIMD); the four-stage tiles' 96 KB of LDS allow one workgroup per CU anyway.
template <int EPI, int NR, int NST>
__global__ __launch_bounds__(QT_PF_WG) __attribute__((amdgpu_waves_per_eu(NST == 2 ? 2 : 1))) void k_pf_gemm2(const uint16_t *__restrict__ W, const uint16_t *__restrict__ P,
                                                        int S, int Sp, int K, float *Y, int ldy) {
    constexpr int KC = 64, ST = 64, STB = 3 * ST * KC * 2;      // one stage: 24 KiB
    constexpr int NB = STB / 1024 / QT_WAVES;                   // 1-KiB copies per wave per chunk (6)
    constexpr int OPS = NB + 2 * NR;                            // vector-memory ops per wave per chunk
    static_assert(NB * 1024 * QT_WAVES == STB, "copy split");
    __shared__ __align__(16) uint8_t sp[NST * STB];             // NST stages
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, kg = lane >> 4;
    const int n0 = blockIdx.x * (64 * NR) + wave * 16 * NR;
    const int s0 = blockIdx.y * ST;
    const int kr = K / gridDim.z, k0 = blockIdx.z * kr, nch = kr / KC;
    const size_t plane = (size_t)Sp * K;
    if (EPI == QT_PF_PART) Y += (size_t)blockIdx.z * S * ldy;

    // this lane's source of each 1-KiB copy (chunk offset added per chunk)
    const uint16_t *src[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int row = 8 * (wave * NB + b) + (lane >> 3), c = (lane & 7) ^ ((row >> 1) & 7);
        src[b] = P + (row / ST) * plane + (size_t)(s0 + row % ST) * K + k0 + 8 * c;
    }
    const uint16_t *wrow[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) wrow[r] = W + (size_t)(n0 + 16 * r + j) * K + k0 + 8 * kg;
    qt_u32x4 a[NST][2][NR];
    auto issue = [&](int c, int st) {   // chunk c into stage st (compile-time st)
        uint8_t *dst = sp + st * STB + (wave * NB) * 1024;
#pragma unroll
        for (int b = 0; b < NB; b++)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(src[b] + c * KC),
                                             (__attribute__((address_space(3))) void *)(dst + b * 1024), 16, 0, 0);
    };
    qt_f32x4 acc[NR][4];
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[r][t] = qt_f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int c = 0; c < NST - 1; c++)
        if (c < nch) {
            issue(c, c);
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int r = 0; r < NR; r++) a[c][ks][r] = *reinterpret_cast<const qt_u32x4 *>(wrow[r] + c * KC + 32 * ks);
        }
    const int f = j >> 1;                               // row swizzle of this lane's B rows
    for (int cb = 0; cb < nch; cb += NST) {
#pragma unroll
        for (int u = 0; u < NST; u++) {
            const int c = cb + u;
            if (c >= nch) break;
            if (c + NST - 2 < nch) qt_vmcnt<(NST - 2) * OPS>();
            else qt_vmcnt<0>();
            __syncthreads();
            const int cn = c + NST - 1;                  // stage (u + NST - 1) % NST held chunk c - 1
            if (cn < nch) {
                issue(cn, (u + NST - 1) % NST);
#pragma unroll
                for (int ks = 0; ks < 2; ks++)
#pragma unroll
                    for (int r = 0; r < NR; r++)
                        a[(u + NST - 1) % NST][ks][r] = *reinterpret_cast<const qt_u32x4 *>(wrow[r] + cn * KC + 32 * ks);
            }
            const uint8_t *stg = sp + u * STB;
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                qt_u32x4 b[4][3];
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int p = 0; p < 3; p++)
                        b[t][p] = qt_lds16(stg + (p * ST + 16 * t + j) * (KC * 2) + 16 * ((4 * ks + kg) ^ f));
#pragma unroll
                for (int r = 0; r < NR; r++)
#pragma unroll
                    for (int t = 0; t < 4; t++)
#pragma unroll
                        for (int p = 0; p < 3; p++) acc[r][t] = qt_mfma_bf16(a[u][ks][r], b[t][p], acc[r][t]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int s = s0 + 16 * t + j, n = n0 + 16 * r + 4 * kg;
            if (s >= S) continue;
            const qt_f32x4 v = acc[r][t];
            if constexpr (EPI == QT_PF_SWIGLU) {
                const float g0 = v[0], u0 = v[1], g1 = v[2], u1 = v[3];
                *reinterpret_cast<float2 *>(Y + (size_t)s * ldy + (n >> 1)) =
                    make_float2(g0 / (1.0f + expf(-g0)) * u0, g1 / (1.0f + expf(-g1)) * u1);
            } else {
                float4 *y = reinterpret_cast<float4 *>(Y + (size_t)s * ldy + n);
                if constexpr (EPI == QT_PF_RESID) {
                    const float4 o = *y;
                    *y = make_float4(o.x + v[0], o.y + v[1], o.z + v[2], o.w + v[3]);
                } else {
                    *y = make_float4(v[0], v[1], v[2], v[3]);
                }
            }
        }
}

// acc = sum over the nz K ranges of part[z][s][n..n+3], ranges in order (each range's
// loads issued before the adds), then the projection's epilogue: Y = acc (STORE),
// Y += acc (RESID), or the SwiGLU of the interleaved gate|up pairs into Y[s][n/2..n/2+1].
__device__ __forceinline__ float4 pf_sum_ranges(const float *part, int nz, int S, int N, int s, int n) {
    float4 acc = *reinterpret_cast<const float4 *>(part + (size_t)s * N + n);
    constexpr int ZB = 8;
    for (int z0 = 1; z0 < nz; z0 += ZB) {
        float4 v[ZB];
#pragma unroll
        for (int k = 0; k < ZB; k++)
            if (z0 + k < nz) v[k] = *reinterpret_cast<const float4 *>(part + ((size_t)(z0 + k) * S + s) * N + n);
#pragma unroll
        for (int k = 0; k < ZB; k++)
            if (z0 + k < nz) { acc.x += v[k].x; acc.y += v[k].y; acc.z += v[k].z; acc.w += v[k].w; }
    }
    return acc;
}

template <int EPI>
__global__ __launch_bounds__(QT_PF_WG) void k_pf_reduce(const float *part, int nz, int S, int N, float *Y, int ldy) {
    const int i = blockIdx.x * QT_PF_WG + threadIdx.x;
    if (i >= S * N / 4) return;
    const int s = i / (N / 4), n = 4 * (i % (N / 4));
    const float4 acc = pf_sum_ranges(part, nz, S, N, s, n);
    if constexpr (EPI == QT_PF_SWIGLU) {
        *reinterpret_cast<float2 *>(Y + (size_t)s * ldy + (n >> 1)) =
            make_float2(acc.x / (1.0f + expf(-acc.x)) * acc.y, acc.z / (1.0f + expf(-acc.z)) * acc.w);
    } else {
        float4 *y = reinterpret_cast<float4 *>(Y + (size_t)s * ldy + n);
        if constexpr (EPI == QT_PF_RESID) {
            const float4 o = *y;
            *y = make_float4(o.x + acc.x, o.y + acc.y, o.z + acc.z, o.w + acc.w);
        } else {
            *y = acc;
        }
    }
}

// The SwiGLU epilogue of the summed K ranges written straight as the three planes of h,
// the down projection's input (F = N/2 columns, P[p][s][F], plane stride Sp*F; rows
// S <= s < Sp zero): the same h values and the same pieces as k_pf_reduce<SWIGLU> followed
// by k_pf_pieces, one launch fewer.
__global__ __launch_bounds__(QT_PF_WG) void k_pf_reduce_swiglu_planes(const float *part, int nz, int S, int Sp, int N,
                                                                      uint16_t *P) {
    const int i = blockIdx.x * QT_PF_WG + threadIdx.x;
    if (i >= Sp * N / 4) return;
    const int s = i / (N / 4), n = 4 * (i % (N / 4));
    const int F = N / 2;
    const size_t plane = (size_t)Sp * F;
    uint16_t *dst = P + (size_t)s * F + (n >> 1);
    if (s >= S) {
#pragma unroll
        for (int p = 0; p < 3; p++) *reinterpret_cast<uint32_t *>(dst + p * plane) = 0u;
        return;
    }
    const float4 acc = pf_sum_ranges(part, nz, S, N, s, n);
    // rounded products (__fmul_rn: no contraction into the piece split), as stored by k_pf_reduce
    const float h0 = __fmul_rn(acc.x / (1.0f + expf(-acc.x)), acc.y), h1 = __fmul_rn(acc.z / (1.0f + expf(-acc.z)), acc.w);
    uint16_t pc[3][2];
    qt_put_pieces(&pc[0][0], 2, h0);
    qt_put_pieces(&pc[0][1], 2, h1);
#pragma unroll
    for (int p = 0; p < 3; p++)
        *reinterpret_cast<uint32_t *>(dst + p * plane) = (uint32_t)pc[p][0] | ((uint32_t)pc[p][1] << 16);
}

// The residual epilogue of the summed K ranges for one position row per workgroup (Y[s] +=
// acc, as k_pf_reduce<RESID>), then that row RMS-normalised with `gain` and written as the
// next projection's three input planes (P[p][s][N], plane stride Sp*N; rows S <= s < Sp
// zero): the row is kept in LDS and the norm and pieces are k_pf_pieces' arithmetic in its
// order (thread t sums x[t + 256 j]^2, block_sum, (x * inv) * g), one launch fewer.
__global__ __launch_bounds__(QT_PF_WG) void k_pf_reduce_resid_planes(const float *part, int nz, int S, int Sp, int N,
                                                                     float *Y, int ldy, const float *gain, float eps,
                                                                     uint16_t *P) {
    extern __shared__ __align__(16) float xr[];
    __shared__ float red[QT_WAVES];
    const int s = blockIdx.x, tid = threadIdx.x;
    const size_t plane = (size_t)Sp * N;
    uint16_t *p0 = P + (size_t)s * N;
    if (s >= S) {
        for (int k = tid * 8; k < N; k += QT_PF_WG * 8)
#pragma unroll
            for (int p = 0; p < 3; p++) *reinterpret_cast<uint4 *>(p0 + p * plane + k) = make_uint4(0u, 0u, 0u, 0u);
        return;
    }
    for (int n = 4 * tid; n < N; n += 4 * QT_PF_WG) {
        const float4 acc = pf_sum_ranges(part, nz, S, N, s, n);
        float4 *y = reinterpret_cast<float4 *>(Y + (size_t)s * ldy + n);
        const float4 o = *y;
        const float4 r = make_float4(o.x + acc.x, o.y + acc.y, o.z + acc.z, o.w + acc.w);
        *y = r;
        *reinterpret_cast<float4 *>(xr + n) = r;
    }
    __syncthreads();
    float ss = 0.f;
    for (int k = tid; k < N; k += QT_PF_WG) ss = fmaf(xr[k], xr[k], ss);
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)N + eps);
    for (int k = tid * 4; k < N; k += QT_PF_WG * 4) {
        float4 v = *reinterpret_cast<const float4 *>(xr + k);
        const float4 g = *reinterpret_cast<const float4 *>(gain + k);
        v.x = (v.x * inv) * g.x; v.y = (v.y * inv) * g.y; v.z = (v.z * inv) * g.z; v.w = (v.w * inv) * g.w;
        uint16_t pc[3][4];
        const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; i++) qt_put_pieces(&pc[0][i], 4, e[i]);
#pragma unroll
        for (int p = 0; p < 3; p++)
            *reinterpret_cast<uint2 *>(p0 + p * plane + k) =
                make_uint2((uint32_t)pc[p][0] | ((uint32_t)pc[p][1] << 16), (uint32_t)pc[p][2] | ((uint32_t)pc[p][3] << 16));
    }
}

// ---- per-head q/k norm, RoPE, KV store ---------------------------------------------
// Position s = blockIdx.x of QKV [S][ld] (q | k | v rows as the projection wrote them):
// q and k heads RMS-normalised with their [128] gains (qwen_rms_norm_per_head,
// k.c:486-577) and rotated at position s (apply_rope_neox_inplace, t.c:203-251:
// x1' = x1 c - x2 s, x2' = x2 c + x1 s), in place; the cache rows s of kv head g get the
// bf16 truncation of k and v (t.c:897-899).  One wave per head row, lane d holding
// elements d and d + 64 (the RoPE pair).
__global__ __launch_bounds__(QT_PF_WG) void k_pf_qkv_post(float *QKV, int ld, int nh, int nkv, const float *qn,
                                                           const float *kn, const float *rc, const float *rs, float eps,
                                                           uint16_t *kc, uint16_t *vc, long long kv_max) {
    const int s = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float *row = QKV + (size_t)s * ld;
    const float c = rc[(size_t)s * 64 + lane], sn = rs[(size_t)s * 64 + lane];
    for (int hr = wave; hr < nh + 2 * nkv; hr += QT_WAVES) {
        float *x = row + hr * 128;
        const float x0 = x[lane], x1 = x[lane + 64];
        if (hr < nh + nkv) {
            const bool isk = hr >= nh;
            const float *w = isk ? kn : qn;
            const float ss = group_sum<64>(x0 * x0 + x1 * x1);
            const float inv = 1.0f / sqrtf(ss / 128.0f + eps);
            const float n0 = (x0 * inv) * w[lane], n1 = (x1 * inv) * w[lane + 64];
            const float r0 = fmaf(n0, c, -(n1 * sn)), r1 = fmaf(n1, c, n0 * sn);
            x[lane] = r0;
            x[lane + 64] = r1;
            if (isk) {
                uint16_t *kd = kc + ((size_t)(hr - nh) * kv_max + s) * 128;
                kd[lane] = f2bf_trunc(r0);
                kd[lane + 64] = f2bf_trunc(r1);
            }
        } else {
            uint16_t *vd = vc + ((size_t)(hr - nh - nkv) * kv_max + s) * 128;
            vd[lane] = f2bf_trunc(x0);
            vd[lane + 64] = f2bf_trunc(x1);
        }
    }
}

// The q|k|v projection's summed K ranges for one position row per workgroup, kept in LDS,
// then k_pf_qkv_post's work on that row (per-head q/k norm, RoPE, KV store) with the same
// arithmetic; the row (q, k rotated, v as summed) is written once.  One launch fewer.
struct PfQkvPost {
    int nh, nkv;
    const float *qn, *kn, *rc, *rs;
    float eps;
    uint16_t *kc, *vc;
    long long kv_max;
};
__global__ __launch_bounds__(QT_PF_WG) void k_pf_reduce_qkv_post(const float *part, int nz, int S, int N, float *QKV,
                                                                 int ld, PfQkvPost a) {
    extern __shared__ __align__(16) float xr[];
    const int s = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int n = 4 * tid; n < N; n += 4 * QT_PF_WG)
        *reinterpret_cast<float4 *>(xr + n) = pf_sum_ranges(part, nz, S, N, s, n);
    __syncthreads();
    float *row = QKV + (size_t)s * ld;
    const float c = a.rc[(size_t)s * 64 + lane], sn = a.rs[(size_t)s * 64 + lane];
    for (int hr = wave; hr < a.nh + 2 * a.nkv; hr += QT_WAVES) {
        float *x = row + hr * 128;
        const float x0 = xr[hr * 128 + lane], x1 = xr[hr * 128 + lane + 64];
        if (hr < a.nh + a.nkv) {
            const bool isk = hr >= a.nh;
            const float *w = isk ? a.kn : a.qn;
            const float ss = group_sum<64>(x0 * x0 + x1 * x1);
            const float inv = 1.0f / sqrtf(ss / 128.0f + a.eps);
            const float n0 = (x0 * inv) * w[lane], n1 = (x1 * inv) * w[lane + 64];
            const float r0 = fmaf(n0, c, -(n1 * sn)), r1 = fmaf(n1, c, n0 * sn);
            x[lane] = r0;
            x[lane + 64] = r1;
            if (isk) {
                uint16_t *kd = a.kc + ((size_t)(hr - a.nh) * a.kv_max + s) * 128;
                kd[lane] = f2bf_trunc(r0);
                kd[lane + 64] = f2bf_trunc(r1);
            }
        } else {
            x[lane] = x0;
            x[lane + 64] = x1;
            uint16_t *vd = a.vc + ((size_t)(hr - a.nh - a.nkv) * a.kv_max + s) * 128;
            vd[lane] = f2bf_trunc(x0);
            vd[lane + 64] = f2bf_trunc(x1);
        }
    }
}

// ---- causal attention, tiled -------------------------------------------------------
// The same attention for 64 queries of one head per workgroup, over 64-key blocks held in
// LDS (flash-style: per block, row max -> rescale of the running sums -> P.V).  Thread t
// takes queries r = t/16 + 16a (a = 0..3) and, for the scores, keys t%16 + 16b, for P.V
// the dims 4(t%16) + 64h + e (h = 0..1, e = 0..3); the 16 threads of a query row are one
// DPP row, so row max and row sum are 16-lane reductions.  K rows are padded to 132
// floats so the 16 key rows a wave reads at one offset fall in 16 different bank groups.
#define QT_PF_KP 132
// P != NULL: the output goes out as the three planes of the O projection's input
// (P[p][s][nh*128], plane stride Sp*nh*128; the same pieces k_pf_pieces makes of the f32
// output), and the workgroup of the last query tile zeroes rows S <= s < Sp of its head.
template <int QA>   // queries per thread: 16 * QA queries per workgroup
__global__ __launch_bounds__(QT_PF_WG) void k_pf_fattn(const float *QKV, int ld, int S, int nh, int nkv, float scale,
                                                        float *A, int lda, uint16_t *P, int Sp) {
    constexpr int QB = 16 * QA;
    __shared__ __align__(16) float qs[QB][128];
    __shared__ __align__(16) float ks[64][QT_PF_KP];
    __shared__ __align__(16) float vs[64][128];
    __shared__ __align__(16) float ps[QB][68];
    const int tid = threadIdx.x, rq = tid >> 4, cg = tid & 15;
    const int q0 = blockIdx.x * QB, h = blockIdx.y, g = h / (nh / nkv);
    const int qd = nh * 128, kvd = nkv * 128;
    // Q block (rows past S: zeros)
    for (int i = tid; i < QB * 32; i += QT_PF_WG) {
        const int r = i >> 5, c = (i & 31) * 4, q = q0 + r;
        *reinterpret_cast<float4 *>(&qs[r][c]) =
            q < S ? *reinterpret_cast<const float4 *>(QKV + (size_t)q * ld + h * 128 + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float m[QA], l[QA], o[QA][8];
#pragma unroll
    for (int a = 0; a < QA; a++) {
        m[a] = -INFINITY; l[a] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) o[a][e] = 0.f;
    }
    const int nkb = (q0 + QB - 1) / 64 + 1;              // key blocks up to the one holding the last query
    for (int kb = 0; kb < nkb; kb++) {
        const int j0 = kb * 64;
        __syncthreads();                                // previous block's K/V/P reads done
        for (int i = tid; i < 64 * 32; i += QT_PF_WG) {
            const int r = i >> 5, c = (i & 31) * 4, j = j0 + r;
            float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
            if (j < S) {
                kv = *reinterpret_cast<const float4 *>(QKV + (size_t)j * ld + qd + g * 128 + c);
                vv = *reinterpret_cast<const float4 *>(QKV + (size_t)j * ld + qd + kvd + g * 128 + c);
            }
            *reinterpret_cast<float4 *>(&ks[r][c]) = kv;
            *reinterpret_cast<float4 *>(&vs[r][c]) = vv;
        }
        __syncthreads();
        // scores of queries rq + 16a with keys cg + 16b
        float sc[QA][4];
#pragma unroll
        for (int a = 0; a < QA; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) sc[a][b] = 0.f;
        for (int d = 0; d < 128; d += 4) {
            float4 qv[QA], kv[4];
#pragma unroll
            for (int a = 0; a < QA; a++) qv[a] = *reinterpret_cast<const float4 *>(&qs[rq + 16 * a][d]);
#pragma unroll
            for (int b = 0; b < 4; b++) kv[b] = *reinterpret_cast<const float4 *>(&ks[cg + 16 * b][d]);
#pragma unroll
            for (int a = 0; a < QA; a++)
#pragma unroll
                for (int b = 0; b < 4; b++)
                    sc[a][b] = fmaf(qv[a].w, kv[b].w, fmaf(qv[a].z, kv[b].z, fmaf(qv[a].y, kv[b].y, fmaf(qv[a].x, kv[b].x, sc[a][b]))));
        }
        // causal mask (keys after the query, keys past S), block max, rescale, P
#pragma unroll
        for (int a = 0; a < QA; a++) {
            const int q = q0 + rq + 16 * a;
            float bm = -INFINITY;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int j = j0 + cg + 16 * b;
                sc[a][b] = (j <= q && j < S) ? sc[a][b] * scale : -INFINITY;
                bm = fmaxf(bm, sc[a][b]);
            }
            bm = group_max<16>(bm);
            const float mn = fmaxf(m[a], bm);
            const float mr = mn == -INFINITY ? 0.f : mn;   // a query row past S has no key at all
            const float c = expf(m[a] - mr);
            float rs = 0.f;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const float pv = expf(sc[a][b] - mr);
                ps[rq + 16 * a][cg + 16 * b] = pv;
                rs += pv;
            }
            l[a] = l[a] * c + group_sum<16>(rs);
            m[a] = mn;
#pragma unroll
            for (int e = 0; e < 8; e++) o[a][e] *= c;
        }
        __syncthreads();
        // o[a][4h + e] += sum_j P[rq + 16a][j] * V[j][64h + 4cg + e]
        for (int jj = 0; jj < 64; jj++) {
            const float4 v0 = *reinterpret_cast<const float4 *>(&vs[jj][4 * cg]);
            const float4 v1 = *reinterpret_cast<const float4 *>(&vs[jj][64 + 4 * cg]);
#pragma unroll
            for (int a = 0; a < QA; a++) {
                const float pv = ps[rq + 16 * a][jj];
                o[a][0] = fmaf(pv, v0.x, o[a][0]); o[a][1] = fmaf(pv, v0.y, o[a][1]);
                o[a][2] = fmaf(pv, v0.z, o[a][2]); o[a][3] = fmaf(pv, v0.w, o[a][3]);
                o[a][4] = fmaf(pv, v1.x, o[a][4]); o[a][5] = fmaf(pv, v1.y, o[a][5]);
                o[a][6] = fmaf(pv, v1.z, o[a][6]); o[a][7] = fmaf(pv, v1.w, o[a][7]);
            }
        }
    }
    if (P) {
        const int K = nh * 128;
        const size_t plane = (size_t)Sp * K;
#pragma unroll
        for (int a = 0; a < QA; a++) {
            const int q = q0 + rq + 16 * a;
            if (q >= S) continue;
            const float inv = 1.0f / l[a];
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                uint16_t pc[3][4];
#pragma unroll
                for (int e = 0; e < 4; e++) qt_put_pieces(&pc[0][e], 4, __fmul_rn(o[a][4 * hh + e], inv));
                uint16_t *dst = P + (size_t)q * K + h * 128 + 64 * hh + 4 * cg;
#pragma unroll
                for (int p = 0; p < 3; p++)
                    *reinterpret_cast<uint2 *>(dst + p * plane) =
                        make_uint2((uint32_t)pc[p][0] | ((uint32_t)pc[p][1] << 16), (uint32_t)pc[p][2] | ((uint32_t)pc[p][3] << 16));
            }
        }
        if (blockIdx.x == gridDim.x - 1)
            for (int i = threadIdx.x; i < (Sp - S) * 32; i += QT_PF_WG) {
                uint16_t *dst = P + (size_t)(S + i / 32) * K + h * 128 + 4 * (i % 32);
#pragma unroll
                for (int p = 0; p < 3; p++) *reinterpret_cast<uint2 *>(dst + p * plane) = make_uint2(0u, 0u);
            }
        return;
    }
#pragma unroll
    for (int a = 0; a < QA; a++) {
        const int q = q0 + rq + 16 * a;
        if (q >= S) continue;
        const float inv = 1.0f / l[a];
        float *out = A + (size_t)q * lda + h * 128;
        *reinterpret_cast<float4 *>(out + 4 * cg) = make_float4(o[a][0] * inv, o[a][1] * inv, o[a][2] * inv, o[a][3] * inv);
        *reinterpret_cast<float4 *>(out + 64 + 4 * cg) = make_float4(o[a][4] * inv, o[a][5] * inv, o[a][6] * inv, o[a][7] * inv);
    }
}

// ---- launchers -------------------------------------------------------------------------
// Positions are padded to a multiple of QT_PF_SPAD for the planes (the GEMM's position
// tile); weight rows must be a multiple of 64 and K a multiple of 64.
#define QT_PF_SPAD 64

extern "C" int qt_pf_spad(int S) { return (S + QT_PF_SPAD - 1) / QT_PF_SPAD * QT_PF_SPAD; }

extern "C" hipError_t qt_launch_pf_pieces(const float *X, int ldx, int S, int K, const float *gain, float eps,
                                          uint16_t *P, hipStream_t st) {
    if (S <= 0 || K <= 0 || K % 8 || ldx % 4) return hipErrorInvalidValue;
    const int Sp = qt_pf_spad(S);
    hipLaunchKernelGGL(k_pf_pieces, dim3(Sp), dim3(QT_PF_WG), 0, st, X, ldx, S, Sp, K, gain, eps, P);
    return hipGetLastError();
}

// part: workspace of 4 * S * N floats for split K (nullable: no split).  The residual
// projections (few weight rows) split K so the grid fills the CUs; the partial ranges
// are added in order (deterministic).
// Tile and K split of a projection: a weight tile of 256, 192, 128 or 64 rows (a taller
// tile reuses each LDS read of the planes over more rows and runs more MFMAs per barrier)
// with its K split where needed into 2^k equal ranges of at least four 64-k chunks whose
// partials fit in part_cap floats (added in order by k_pf_reduce), so that the grid
// reaches 256 workgroups; among such plans the one with the least work on the busiest CU,
// else the largest grid.  Measured on the 1.7B prefill (128 / 512 positions): with the
// three-stage 256-row tile 4.16 / 9.46 ms against 4.53 / 10.72 preferring an unsplit
// shorter tile, 4.50 / 10.22 splitting to 512 workgroups, 4.27 / 9.46 with two-chunk
// ranges; with the two-stage tiles at two waves per SIMD 3.94 / 8.73 (splitting to 512
// workgroups 4.50 / 9.56); choosing by the busiest CU's work (192-row tiles for gate|up:
// 512 workgroups, two on every CU, where 256-row tiles gave 384) 3.64 / 7.79.
static void qt_pf_plan(int S, int Sp, int N, int K, long long part_cap, int &nr, int &sk) {
    // per-CU load of a plan: workgroups per CU (ceil over 256) x rows per workgroup / K ranges;
    // among the plans that reach 256 workgroups the lightest, the taller tile on a tie
    const long long sy = Sp / 64;
    long long best = -1;
    double bcost = 1e30;
    bool reach = false;
    nr = 1; sk = 1;
    const int rs[4] = {4, 3, 2, 1};
    for (int ri = 0; ri < 4; ri++) {
        const int r = rs[ri];
        if (N % (64 * r)) continue;
        const long long g = (long long)(N / (64 * r)) * sy;
        int k = 1;
        while (g * k < 256 && (K / 64) % (2 * k) == 0 && K / 64 / (2 * k) >= 4 && 2LL * k * S * N <= part_cap) k *= 2;
        if (g * k >= 256) {
            const double cost = (double)((g * k + 255) / 256) * r / k;
            if (!reach || cost < bcost) { nr = r; sk = k; bcost = cost; }
            reach = true;
        } else if (!reach && g * k > best) {
            best = g * k; nr = r; sk = k;
        }
    }
}

// Pout != NULL (SwiGLU only): h goes out as the three planes of the next projection's
// input (k_pf_reduce_swiglu_planes) instead of f32 rows; needs part with S*N <= part_cap.
// Pout with RESID: Y += the product as usual, then RMSNorm(Y row) * gain goes out as the
// next projection's input planes (k_pf_reduce_resid_planes); needs part, S*N <= part_cap.
// qp != NULL (STORE into the q|k|v rows Y): k_pf_reduce_qkv_post finishes the rows.
static hipError_t pf_gemm(int epi, const uint16_t *W, const uint16_t *P, int S, int N, int K, float *Y, int ldy,
                          float *part, long long part_cap, uint16_t *Pout, const float *gain, float eps,
                          hipStream_t st, const PfQkvPost *qp = nullptr) {
    constexpr int NST = 4;
    if (qp && (epi != QT_PF_STORE || Pout || !part || (long long)S * N > part_cap || N != (qp->nh + 2 * qp->nkv) * 128 ||
               (size_t)N * 4 > 64 * 1024 || S > qp->kv_max))
        return hipErrorInvalidValue;
    if (S <= 0 || N <= 0 || K <= 0 || N % 64 || K % 64 || epi < 0 || epi > 2) return hipErrorInvalidValue;
    if (Pout ? ((epi != QT_PF_SWIGLU && !(epi == QT_PF_RESID && gain && Y && ldy >= N && ldy % 4 == 0 &&
                                          (size_t)N * 4 <= 64 * 1024)) ||
                !part || (long long)S * N > part_cap)
             : (epi != QT_PF_SWIGLU ? (ldy < N || ldy % 4) : (ldy < N / 2 || ldy % 2)))
        return hipErrorInvalidValue;
    const int Sp = qt_pf_spad(S);
    int nr, sk;
    qt_pf_plan(S, Sp, N, K, part ? part_cap : 0, nr, sk);
    const int gx = N / (64 * nr);
    const dim3 grid(gx, Sp / 64, sk);
#define QT_PF_GEMM(E, OUT, LD)                                                                                         \
    if (nr == 4) hipLaunchKernelGGL((k_pf_gemm2<E, 4, 2>), grid, dim3(QT_PF_WG), 0, st, W, P, S, Sp, K, OUT, LD);    \
    else if (nr == 3) hipLaunchKernelGGL((k_pf_gemm2<E, 3, 2>), grid, dim3(QT_PF_WG), 0, st, W, P, S, Sp, K, OUT, LD); \
    else if (nr == 2) hipLaunchKernelGGL((k_pf_gemm2<E, 2, NST>), grid, dim3(QT_PF_WG), 0, st, W, P, S, Sp, K, OUT, LD); \
    else hipLaunchKernelGGL((k_pf_gemm2<E, 1, NST>), grid, dim3(QT_PF_WG), 0, st, W, P, S, Sp, K, OUT, LD);
    if (qp) {
        QT_PF_GEMM(QT_PF_PART, part, N)
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(k_pf_reduce_qkv_post, dim3(S), dim3(QT_PF_WG), (size_t)N * sizeof(float), st, part, sk, S, N, Y,
                           ldy, *qp);
    } else if (Pout) {
        QT_PF_GEMM(QT_PF_PART, part, N)
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (epi == QT_PF_SWIGLU)
            hipLaunchKernelGGL(k_pf_reduce_swiglu_planes, dim3((Sp * N / 4 + QT_PF_WG - 1) / QT_PF_WG), dim3(QT_PF_WG), 0,
                               st, part, sk, S, Sp, N, Pout);
        else
            hipLaunchKernelGGL(k_pf_reduce_resid_planes, dim3(Sp), dim3(QT_PF_WG), (size_t)N * sizeof(float), st, part, sk,
                               S, Sp, N, Y, ldy, gain, eps, Pout);
    } else if (sk > 1) {
        QT_PF_GEMM(QT_PF_PART, part, N)
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const dim3 rg((S * N / 4 + QT_PF_WG - 1) / QT_PF_WG);
        if (epi == QT_PF_STORE) hipLaunchKernelGGL(k_pf_reduce<QT_PF_STORE>, rg, dim3(QT_PF_WG), 0, st, part, sk, S, N, Y, ldy);
        else if (epi == QT_PF_RESID) hipLaunchKernelGGL(k_pf_reduce<QT_PF_RESID>, rg, dim3(QT_PF_WG), 0, st, part, sk, S, N, Y, ldy);
        else hipLaunchKernelGGL(k_pf_reduce<QT_PF_SWIGLU>, rg, dim3(QT_PF_WG), 0, st, part, sk, S, N, Y, ldy);
    } else if (epi == QT_PF_STORE) {
        QT_PF_GEMM(QT_PF_STORE, Y, ldy)
    } else if (epi == QT_PF_RESID) {
        QT_PF_GEMM(QT_PF_RESID, Y, ldy)
    } else {
        QT_PF_GEMM(QT_PF_SWIGLU, Y, ldy)
    }
#undef QT_PF_GEMM
    return hipGetLastError();
}

extern "C" hipError_t qt_launch_pf_gemm(int epi, const uint16_t *W, const uint16_t *P, int S, int N, int K, float *Y,
                                        int ldy, float *part, long long part_cap, hipStream_t st) {
    return pf_gemm(epi, W, P, S, N, K, Y, ldy, part, part_cap, NULL, NULL, 0.f, st);
}
extern "C" hipError_t qt_launch_pf_gemm_swiglu_planes(const uint16_t *W, const uint16_t *P, int S, int N, int K,
                                                      uint16_t *Pout, float *part, long long part_cap, hipStream_t st) {
    return pf_gemm(QT_PF_SWIGLU, W, P, S, N, K, NULL, 0, part, part_cap, Pout, NULL, 0.f, st);
}
extern "C" hipError_t qt_launch_pf_gemm_qkv_post(const uint16_t *W, const uint16_t *P, int S, int N, int K, float *QKV,
                                                  int ld, int nh, int nkv, const float *qn, const float *kn,
                                                  const float *rc, const float *rs, float eps, uint16_t *kc, uint16_t *vc,
                                                  long long kv_max, float *part, long long part_cap, hipStream_t st) {
    if (nh <= 0 || nkv <= 0 || nh % nkv) return hipErrorInvalidValue;
    const PfQkvPost qp = {nh, nkv, qn, kn, rc, rs, eps, kc, vc, kv_max};
    return pf_gemm(QT_PF_STORE, W, P, S, N, K, QKV, ld, part, part_cap, NULL, NULL, 0.f, st, &qp);
}
extern "C" hipError_t qt_launch_pf_gemm_resid_planes(const uint16_t *W, const uint16_t *P, int S, int N, int K, float *Y,
                                                     int ldy, const float *gain, float eps, uint16_t *Pout, float *part,
                                                     long long part_cap, hipStream_t st) {
    return pf_gemm(QT_PF_RESID, W, P, S, N, K, Y, ldy, part, part_cap, Pout, gain, eps, st);
}

extern "C" hipError_t qt_launch_pf_qkv_post(float *QKV, int ld, int S, int nh, int nkv, const float *qn,
                                            const float *kn, const float *rc, const float *rs, float eps, uint16_t *kc,
                                            uint16_t *vc, long long kv_max, hipStream_t st) {
    if (S <= 0 || nh <= 0 || nkv <= 0 || nh % nkv || S > kv_max) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pf_qkv_post, dim3(S), dim3(QT_PF_WG), 0, st, QKV, ld, nh, nkv, qn, kn, rc, rs, eps, kc, vc,
                       kv_max);
    return hipGetLastError();
}

// ---- causal attention on the f32 matrix cores -----------------------------------------
// 64 queries of one head per workgroup, 16 per wave, over 64-key blocks staged in LDS (K
// rows [key][dim]; V transposed, [dim][key]).  v_mfma_f32_16x16x4_f32 (lane l supplies
// A[l%16][l/16] and B[l/16][l%16], receives D[4(l/16)+r][l%16]) computes the scores
// transposed, S^T = K . Q^T, with k-step s of lane group g taking dim 32g + s: each lane
// keeps its query's 32 dims (32g .. 32g+31) in registers and reads a key's four dims of
// four steps as one float4.  Lane l then holds the scores of query l%16 with keys
// 16t + 4g + r (tile t, register r) -- exactly the A operand of P.V when k-step s of tile
// t takes key 16t + 4g + s, so the probabilities never leave the registers; the B
// operand (4 keys of one dim) is one float4 of the transposed V.  Softmax per block as
// in k_pf_fattn (scale, causal mask, block max, e^(s - m), running sums), the per-query
// statistics exchanged across the four lane groups with shuffles; the P.V result rows
// (queries 4g + r) take their rescale factors from the lanes that own those queries.
#define QT_PF_VTP 68   // V^T row pitch (64 keys + 4: the float4 reads of a wave spread over banks)
// P != NULL: output as the O projection's input planes, as k_pf_fattn does.
__global__ __launch_bounds__(QT_PF_WG) __attribute__((amdgpu_waves_per_eu(2))) void k_pf_fattn_mf(
    const float *QKV, int ld, int S, int nh, int nkv, float scale, float *A, int lda, uint16_t *P, int Sp) {
    __shared__ __align__(16) float ks[64][QT_PF_KP];
    __shared__ __align__(16) float vt[128][QT_PF_VTP];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 15, g = lane >> 4;
    const int h = blockIdx.y, kvh = h / (nh / nkv);
    const int q0 = blockIdx.x * 64, qw = q0 + 16 * wave, q = qw + li;
    const int qd = nh * 128, kvd = nkv * 128;
    float qf[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 v = q < S ? *reinterpret_cast<const float4 *>(QKV + (size_t)q * ld + h * 128 + 32 * g + 4 * i)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
        qf[4 * i] = v.x; qf[4 * i + 1] = v.y; qf[4 * i + 2] = v.z; qf[4 * i + 3] = v.w;
    }
    float m = -INFINITY, l = 0.f;           // statistics of query q (the same in the four lane groups)
    qt_f32x4 o[8];                          // O[query 4g + r][dim 16 dt + li]
#pragma unroll
    for (int dt = 0; dt < 8; dt++) o[dt] = qt_f32x4{0.f, 0.f, 0.f, 0.f};
    const int nkb = (min(q0 + 64, S) - 1) / 64 + 1;
    // the next block's K and V rows wait in registers while the current block computes
    // (thread t: rows t/32 + 8i, float4 column t%32, i < 8)
    constexpr int NP = 64 * 32 / QT_PF_WG;
    float4 pk[NP], pv[NP];
    auto fetch = [&](int j0) {
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int r = (tid >> 5) + 8 * i, c = (tid & 31) * 4, j = j0 + r;
            pk[i] = pv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (j < S) {
                pk[i] = *reinterpret_cast<const float4 *>(QKV + (size_t)j * ld + qd + kvh * 128 + c);
                pv[i] = *reinterpret_cast<const float4 *>(QKV + (size_t)j * ld + qd + kvd + kvh * 128 + c);
            }
        }
    };
    fetch(0);
    for (int kb = 0; kb < nkb; kb++) {
        const int j0 = kb * 64;
        __syncthreads();                                // previous block's K / V reads done
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int r = (tid >> 5) + 8 * i, c = (tid & 31) * 4;
            *reinterpret_cast<float4 *>(&ks[r][c]) = pk[i];
            vt[c][r] = pv[i].x; vt[c + 1][r] = pv[i].y; vt[c + 2][r] = pv[i].z; vt[c + 3][r] = pv[i].w;
        }
        __syncthreads();
        if (kb + 1 < nkb) fetch(j0 + 64);
        if (j0 > qw + 15) continue;                     // every query of this wave precedes the block (wave-uniform)
        qt_f32x4 st[4];
#pragma unroll
        for (int t = 0; t < 4; t++) st[t] = qt_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s4 = 0; s4 < 8; s4++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const float4 kv = *reinterpret_cast<const float4 *>(&ks[16 * t + li][32 * g + 4 * s4]);
                st[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.x, qf[4 * s4], st[t], 0, 0, 0);
                st[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.y, qf[4 * s4 + 1], st[t], 0, 0, 0);
                st[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.z, qf[4 * s4 + 2], st[t], 0, 0, 0);
                st[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.w, qf[4 * s4 + 3], st[t], 0, 0, 0);
            }
        float bm = -INFINITY;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int j = j0 + 16 * t + 4 * g + r;
                const float sv = (j <= q && j < S) ? st[t][r] * scale : -INFINITY;
                st[t][r] = sv;
                bm = fmaxf(bm, sv);
            }
        bm = fmaxf(bm, __shfl_xor(bm, 16));
        bm = fmaxf(bm, __shfl_xor(bm, 32));
        const float mn = fmaxf(m, bm);
        const float mr = mn == -INFINITY ? 0.f : mn;     // a query row past S has no key at all
        const float alpha = expf(m - mr);
        float rs = 0.f;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float pv = expf(st[t][r] - mr);
                st[t][r] = pv;
                rs += pv;
            }
        rs += __shfl_xor(rs, 16);
        rs += __shfl_xor(rs, 32);
        l = l * alpha + rs;
        m = mn;
        float ar[4];
#pragma unroll
        for (int r = 0; r < 4; r++) ar[r] = __shfl(alpha, 4 * g + r);
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++) o[dt][r] *= ar[r];
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                const float4 vv = *reinterpret_cast<const float4 *>(&vt[16 * dt + li][16 * t + 4 * g]);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(st[t][0], vv.x, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(st[t][1], vv.y, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(st[t][2], vv.z, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(st[t][3], vv.w, o[dt], 0, 0, 0);
            }
    }
    float lr[4];
#pragma unroll
    for (int r = 0; r < 4; r++) lr[r] = 1.0f / __shfl(l, 4 * g + r);
    if (P) {
        const size_t plane = (size_t)Sp * qd;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int qq = qw + 4 * g + r;
            if (qq >= S) continue;
#pragma unroll
            for (int dt = 0; dt < 8; dt++)
                qt_put_pieces(P + (size_t)qq * qd + h * 128 + 16 * dt + li, (int)plane, __fmul_rn(o[dt][r], lr[r]));
        }
        if (blockIdx.x == gridDim.x - 1)
            for (int i = tid; i < (Sp - S) * 32; i += QT_PF_WG) {
                uint16_t *dst = P + (size_t)(S + i / 32) * qd + h * 128 + 4 * (i % 32);
#pragma unroll
                for (int p = 0; p < 3; p++) *reinterpret_cast<uint2 *>(dst + p * plane) = make_uint2(0u, 0u);
            }
        return;
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int qq = qw + 4 * g + r;
        if (qq >= S) continue;
#pragma unroll
        for (int dt = 0; dt < 8; dt++) A[(size_t)qq * lda + h * 128 + 16 * dt + li] = o[dt][r] * lr[r];
    }
}

// P != NULL (with planes): the output is written as the O projection's input planes
// (rows padded to qt_pf_spad(S)) and *planes = 1; otherwise A gets the f32 rows.
static hipError_t pf_attn(const float *QKV, int ld, int S, int nh, int nkv, float scale, float *A, int lda,
                          uint16_t *P, int *planes, hipStream_t st) {
    if (S <= 0 || nh <= 0 || nkv <= 0 || nh % nkv) return hipErrorInvalidValue;
    if (planes) *planes = 0;
    // the matrix-core kernel where it has at least 64 workgroups (1.7B prefill, 512
    // positions: 8.37 ms against 8.72 with the VALU kernel; at 128 positions, 32
    // workgroups, 3.84 against 3.77), else the VALU kernel with 64-, 32- or 16-query
    // workgroups, the largest that still fills the CUs
    const int Sp = qt_pf_spad(S);
    if (P && planes) *planes = 1;
    else P = NULL;
    if ((long long)((S + 63) / 64) * nh >= 64) {
        hipLaunchKernelGGL(k_pf_fattn_mf, dim3((S + 63) / 64, nh), dim3(QT_PF_WG), 0, st, QKV, ld, S, nh, nkv, scale, A, lda,
                           P, Sp);
        return hipGetLastError();
    }
    if ((long long)((S + 63) / 64) * nh >= 256)
        hipLaunchKernelGGL(k_pf_fattn<4>, dim3((S + 63) / 64, nh), dim3(QT_PF_WG), 0, st, QKV, ld, S, nh, nkv, scale, A, lda, P, Sp);
    else if ((long long)((S + 31) / 32) * nh >= 256)
        hipLaunchKernelGGL(k_pf_fattn<2>, dim3((S + 31) / 32, nh), dim3(QT_PF_WG), 0, st, QKV, ld, S, nh, nkv, scale, A, lda, P, Sp);
    else
        hipLaunchKernelGGL(k_pf_fattn<1>, dim3((S + 15) / 16, nh), dim3(QT_PF_WG), 0, st, QKV, ld, S, nh, nkv, scale, A, lda, P, Sp);
    return hipGetLastError();
}

extern "C" hipError_t qt_launch_pf_attn(const float *QKV, int ld, int S, int nh, int nkv, float scale, float *A,
                                        int lda, hipStream_t st) {
    return pf_attn(QKV, ld, S, nh, nkv, scale, A, lda, NULL, NULL, st);
}
extern "C" hipError_t qt_launch_pf_attn_planes(const float *QKV, int ld, int S, int nh, int nkv, float scale, float *A,
                                               int lda, uint16_t *P, int *planes, hipStream_t st) {
    return pf_attn(QKV, ld, S, nh, nkv, scale, A, lda, P, planes, st);
}
