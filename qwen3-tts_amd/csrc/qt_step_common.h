// qt_step_common.h — helpers shared by the persistent decode-step kernels (qt_pstep.hip,
// qt_rstep.hip): explicit global loads, LDS layouts of activations, the exact int8
// activation pieces and their MFMA / v_dot4 dot products, bf16 / q4_0 row tiles.
#pragma once
#include "qt_attn_mf.h"
#include <type_traits>

namespace ps {
constexpr int NB = 256;          // workgroups (one per CU)
constexpr int NWB = 4;           // waves that run the attention chunk (B) and the merge (M)
constexpr int HD = 128, NH = 16, NKV = 8, HPK = 2, QD = NH * HD, KVD = NKV * HD, QKVR = QD + 2 * KVD;
constexpr int G = NB / NKV;      // attention chunks per kv head (32)
constexpr int CHMAX = 256;       // keys per chunk at most (kv_max <= G * CHMAX)
constexpr int PS = 2 + HD;       // partial record per head: max, sum, o[HD]
constexpr unsigned POLL_LIMIT = 1u << 17;
constexpr int MAXL = 64;         // layers whose table fits the LDS copy
constexpr int KVB = 128;         // keys of a chunk staged in LDS at once (K and V: 64 KiB)
static_assert(NWB * 32 == KVB, "each attention wave takes two 16-key tiles of a block");

// Loads through pointers read from memory are made explicitly global (address space
// 1): a generic (flat) load would also count against the LDS counter, so every later
// LDS wait would stall on HBM.
template <typename T>
__device__ __forceinline__ T ldg(const T *p) { return *(const __attribute__((address_space(1))) T *)p; }
// A pointer read from LDS lands in VGPRs; declaring it wave-uniform (readfirstlane)
// lets loads use a scalar base plus a 32-bit lane offset instead of 64-bit per-lane
// addresses that would otherwise be kept live in VGPRs.
template <typename T>
__device__ __forceinline__ T *uni(T *p) {
    const unsigned long long v = (unsigned long long)p;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v), hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
    return (T *)(((unsigned long long)hi << 32) | lo);
}
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
// 16 bytes per lane from global memory straight into LDS (global_load_lds_dwordx4):
// lane i's bytes land at dst + 16*i, dst wave-uniform.  Counted by vmcnt like a load,
// and a workgroup barrier does not wait for it: other waves may read the bytes only after
// a barrier that the copying wave reached behind a wait covering the copy (the next
// gather's wait, whose loads queue behind it, or an explicit s_waitcnt).
__device__ __forceinline__ void lds_copy16(const void *src, void *dst) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                     (__attribute__((address_space(3))) void *)dst, 16, 0, 0);
}
__device__ __forceinline__ uint4 ldg(const uint4 *p) {
    const u32x4_t v = *(const __attribute__((address_space(1))) u32x4_t *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 ldg(const float4 *p) {
    const u32x4_t v = *(const __attribute__((address_space(1))) u32x4_t *)p;
    return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}

struct Layer {
    const uint8_t *w[4];          // qkv, o, gate_up, down (device encodings, qt_device.h)
    const float *s[4];            // int8 row scales
    const uint16_t *s16[4];       // q4 block scales
    const float *in_norm, *post_norm, *qn, *kn;
};


__device__ __forceinline__ void st_i(int *p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ int ld_i(const int *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ unsigned long long ld_w(const unsigned long long *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_tag(unsigned long long *p, float v, unsigned tag) {
    __hip_atomic_store(p, ((unsigned long long)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned tag_of(unsigned long long w) { return (unsigned)(w >> 32); }
__device__ __forceinline__ float val_of(unsigned long long w) { return __uint_as_float((unsigned)w); }



// ---- activation layout in LDS -------------------------------------------------------------
// A COLS-element activation consumed in EPC-element chunks (one chunk per lane and 16-byte
// weight load: EPC = 16 int8 or 8 bf16 weights) is kept chunk-transposed: float4 q of
// chunk c sits at float4 slot q*(COLS/EPC) + c.  Lanes walk consecutive chunks, so every
// wave-wide float4 read (norm statistics, chunk sums, dot products) is one contiguous
// KiB: no LDS bank conflicts (a row-major layout puts consecutive lanes 4*EPC bytes apart,
// a 4*EPC/16-way conflict).  Values and arithmetic order are unchanged.
template <int EPC, int COLS>
__device__ __forceinline__ int xpos(int i) {
    constexpr int NCH = COLS / EPC;
    const int c = i / EPC, e = i % EPC;
    return ((e >> 2) * NCH + c) * 4 + (e & 3);
}
template <int EPC, int COLS>
__device__ __forceinline__ float4 xchunk4(const float *x, int c, int q) {
    return *reinterpret_cast<const float4 *>(x + (q * (COLS / EPC) + c) * 4);
}
struct PosId { __device__ __forceinline__ int operator()(int i) const { return i; } };
template <int EPC, int COLS>
struct PosChunk { __device__ __forceinline__ int operator()(int i) const { return xpos<EPC, COLS>(i); } };

// ---- waiting for tagged data ------------------------------------------------------------
// Each thread gathers elements i = tid + k*NT (k < K, i < n) whose words addr(i) must
// carry `tag`; all reads are issued before any is checked, then only stale words are
// re-read, one round trip per round.  Values land in dst[i] (LDS); ends with a
// workgroup barrier.  n <= 0 gathers nothing.
// (Issuing the next phase's weight loads between the first reads and their check, so
// the issue overlaps the first round trip, was measured 30 % slower per step than
// issuing them before the gather.)
// Statistics for the int8 pieces, per wave into wst[2*wave], wst[2*wave+1] (read after
// the gather's barrier): gains == nullptr: max|x|; else the RMSNorm partial sum of
// squares (thread t: x[t + NT k]^2 accumulated in k order, then the wave's butterfly)
// and max|x*g| over the thread's elements.
template <int K, int NT, typename PosF>
__device__ __forceinline__ void pc_stats(const float (&x)[K], int n, const float *gains, PosF pos, float *wst) {
    const int tid = threadIdx.x;
    float ss = 0.f, m = 0.f;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int i = tid + k * NT;
        if (i < n) {
            if (gains) {
                ss = fmaf(x[k], x[k], ss);
                m = fmaxf(m, fabsf(x[k] * gains[pos(i)]));
            } else {
                m = fmaxf(m, fabsf(x[k]));
            }
        }
    }
    if (gains) ss = group_sum<64>(ss);
    m = group_max<64>(m);
    if ((tid & 63) == 0) { wst[2 * (tid >> 6)] = ss; wst[2 * (tid >> 6) + 1] = m; }
}

template <int K, int NT, typename AddrF, typename PosF = PosId>
__device__ __forceinline__ void gather(int n, AddrF addr, float *dst, unsigned tag, int *err, PosF pos = PosF(),
                                       float *wst = nullptr, const float *gains = nullptr) {
    const int tid = threadIdx.x;
    unsigned long long v[K];
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int i = tid + k * NT;
        v[k] = (i < n) ? ld_w(addr(i)) : ((unsigned long long)tag << 32);
    }
    for (unsigned it = 0;; it++) {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < K; k++) ok = ok && tag_of(v[k]) == tag;
        if (ok) break;
        if ((it & 31) == 31) {
            if (ld_i(err)) break;
            if (it > POLL_LIMIT) { st_i(err, 1); break; }
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int i = tid + k * NT;
            if (i < n && tag_of(v[k]) != tag) v[k] = ld_w(addr(i));
        }
    }
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int i = tid + k * NT;
        if (i < n) dst[pos(i)] = val_of(v[k]);
    }
    if (wst) {      // int8 pieces: per-wave statistics
        float x[K];
#pragma unroll
        for (int k = 0; k < K; k++) x[k] = val_of(v[k]);
        pc_stats<K, NT>(x, n, gains, pos, wst);
    }
    __syncthreads();
}

// ---- weight tiles -----------------------------------------------------------------------
template <int PREC> struct Epc;
template <> struct Epc<QT_BF16> { static constexpr int v = 8; };
template <> struct Epc<QT_INT8> { static constexpr int v = 16; };
template <> struct Epc<QT_Q4> { static constexpr int v = 32; };

// NR consecutive rows per wave of a [rows][COLS] matrix; each row is split over the 64
// lanes, lane l holding the 16-byte chunks c = l + 64*j (j < CPL).  Also carries the
// int8 row scales (row0w is wave-uniform, so those are scalar loads: SGPRs, counted
// apart from the vector loads in flight) or, for q4_0, the f16 bits of each chunk's
// block scale (one 32-weight block per chunk: [rows][COLS/32] halves, vector loads).
template <int PREC, int COLS, int NR_>
struct Tile {
    static constexpr int NR = NR_;
    static constexpr int EPC = Epc<PREC>::v;
    static constexpr int CPL = COLS / (EPC * 64);
    static constexpr size_t RB = PREC == QT_BF16 ? (size_t)COLS * 2 : PREC == QT_INT8 ? (size_t)COLS : (size_t)COLS / 2;
    static_assert(CPL >= 1 && CPL * EPC * 64 == COLS, "tile shape");
    static constexpr int NQ = PREC == QT_Q4 ? NR : 1, CQ = PREC == QT_Q4 ? CPL : 1;
    uint4 w[NR][CPL];
    float rs[NR];
    uint32_t bs[NQ][CQ];

    // S: int8 row scales (float) or q4 block-scale halves (uint16_t), per precision
    __device__ __forceinline__ void load(const uint8_t *W, const void *S, int row0w) {
        const int lane = threadIdx.x & 63;
        W = uni(W);
#pragma unroll
        for (int r = 0; r < NR; r++)
#pragma unroll
            for (int j = 0; j < CPL; j++)
                w[r][j] = ldg(reinterpret_cast<const uint4 *>(W + (size_t)(row0w + r) * RB + (size_t)(lane + 64 * j) * 16));
        if constexpr (PREC == QT_INT8) {
            const float *Sf = uni(static_cast<const float *>(S));
#pragma unroll
            for (int r = 0; r < NR; r++) rs[r] = ldg(Sf + row0w + r);
        } else {
#pragma unroll
            for (int r = 0; r < NR; r++) rs[r] = 1.0f;
        }
        if constexpr (PREC == QT_Q4) {
            const uint16_t *Sh = uni(static_cast<const uint16_t *>(S));
#pragma unroll
            for (int r = 0; r < NR; r++)
#pragma unroll
                for (int j = 0; j < CPL; j++) bs[r][j] = ldg(Sh + (size_t)(row0w + r) * (COLS / 32) + lane + 64 * j);
        }
    }
};

// scale pointer of projection i in the form this precision's tiles take
template <int PREC>
__device__ __forceinline__ const void *lsc(const Layer &ly, int i) {
    return PREC == QT_Q4 ? static_cast<const void *>(ly.s16[i]) : static_cast<const void *>(ly.s[i]);
}

// acc[r] = dot(row r, x) for the tile's rows (bf16 or q4_0 weights; int8 projections use
// the exact pieces below), x read from LDS chunk by chunk (so no activation slice occupies
// registers), reduced over the wave (valid in every lane).  Same arithmetic, in the same
// order, as k_mv in qt_matvec.hip: q4_0 chunk = one block, dot = d * (sum q*x - 8 sum x)
// with the nibbles in storage order (word m: elements 8m..8m+7, even ones low).
template <int PREC, int COLS, int NR>
__device__ __forceinline__ void tile_dot(const Tile<PREC, COLS, NR> &t, const float *x, float (&acc)[NR]) {
    static_assert(PREC != QT_INT8, "int8 projections take the exact activation pieces");
    using T = Tile<PREC, COLS, NR>;
    constexpr int EPC = T::EPC;
    const int lane = threadIdx.x & 63;
    float s[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) s[r] = 0.f;
#pragma unroll
    for (int j = 0; j < T::CPL; j++) {
        const int ci = lane + 64 * j;
        float xv[EPC];
#pragma unroll
        for (int q = 0; q < EPC / 4; q++) {
            const float4 v = xchunk4<EPC, COLS>(x, ci, q);
            xv[4 * q] = v.x; xv[4 * q + 1] = v.y; xv[4 * q + 2] = v.z; xv[4 * q + 3] = v.w;
        }
        if constexpr (PREC == QT_Q4) {
            float xr[32];
#pragma unroll
            for (int m = 0; m < 4; m++)
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    xr[m * 4 + b] = xv[8 * m + 2 * b];
                    xr[16 + m * 4 + b] = xv[8 * m + 2 * b + 1];
                }
            float xsum = 0.f;
#pragma unroll
            for (int e = 0; e < 32; e++) xsum += xr[e];
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const uint32_t w4[4] = {t.w[r][j].x, t.w[r][j].y, t.w[r][j].z, t.w[r][j].w};
                float u = 0.f;
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    const uint32_t lo = w4[m] & 0x0F0F0F0Fu, hi = (w4[m] >> 4) & 0x0F0F0F0Fu;
                    u = fmaf((float)(lo & 0xFFu), xr[m * 4 + 0], u);
                    u = fmaf((float)((lo >> 8) & 0xFFu), xr[m * 4 + 1], u);
                    u = fmaf((float)((lo >> 16) & 0xFFu), xr[m * 4 + 2], u);
                    u = fmaf((float)(lo >> 24), xr[m * 4 + 3], u);
                    u = fmaf((float)(hi & 0xFFu), xr[16 + m * 4 + 0], u);
                    u = fmaf((float)((hi >> 8) & 0xFFu), xr[16 + m * 4 + 1], u);
                    u = fmaf((float)((hi >> 16) & 0xFFu), xr[16 + m * 4 + 2], u);
                    u = fmaf((float)(hi >> 24), xr[16 + m * 4 + 3], u);
                }
                s[r] = fmaf(ref_f16_to_f32(t.bs[r][j]), fmaf(-8.0f, xsum, u), s[r]);
            }
        } else {
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const uint32_t w4[4] = {t.w[r][j].x, t.w[r][j].y, t.w[r][j].z, t.w[r][j].w};
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    s[r] = fmaf(bf_lo(w4[m]), xv[2 * m], s[r]);
                    s[r] = fmaf(bf_hi(w4[m]), xv[2 * m + 1], s[r]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < NR; r++) acc[r] = group_sum<64>(s[r]);
}

// Norm gains [COLS] copied into LDS by global_load_lds (no registers held between the
// phase that issues the copy and the phase that uses it), one phase ahead, in the
// chunk-transposed layout: LDS float4 slot k = q*NCH + c takes global float4 c*EPC/4 + q.
template <int NW, int EPC, int COLS>
__device__ __forceinline__ void load_gains(const float *src, float *dst) {
    constexpr int NCH = COLS / EPC;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    src = uni(src);
    for (int i = wave; i * 256 < COLS; i += NW) {
        const int k = i * 64 + lane, q = k / NCH, c = k % NCH;
        lds_copy16(src + (c * (EPC / 4) + q) * 4, dst + i * 256);
    }
}

// xn = RMSNorm(x) * g into LDS (bf16 layers, the codec head).  The mean square is
// accumulated exactly as k_mv does (lane l over chunks l + 64 j in element order, then a
// wave butterfly), by every wave redundantly, so no extra barrier is needed; then thread
// c normalises chunk c.  Ends with a workgroup barrier.
template <int PREC, int COLS>
__device__ __forceinline__ void stage_norm(const float *x, const float *gain, float eps, float *xn) {
    constexpr int EPC = Epc<PREC>::v, CPL = COLS / (EPC * 64);
    const int lane = threadIdx.x & 63, c = threadIdx.x;
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; j++)
#pragma unroll
        for (int q = 0; q < EPC / 4; q++) {
            const float4 v = xchunk4<EPC, COLS>(x, lane + 64 * j, q);
            ss = fmaf(v.x, v.x, ss); ss = fmaf(v.y, v.y, ss); ss = fmaf(v.z, v.z, ss); ss = fmaf(v.w, v.w, ss);
        }
    ss = group_sum<64>(ss);
    const float inv = 1.0f / sqrtf(ss / (float)COLS + eps);
    if (c * EPC < COLS) {
#pragma unroll
        for (int q = 0; q < EPC / 4; q++) {
            const float4 xv = xchunk4<EPC, COLS>(x, c, q), gv = xchunk4<EPC, COLS>(gain, c, q);
            const float4 v = make_float4((xv.x * inv) * gv.x, (xv.y * inv) * gv.y, (xv.z * inv) * gv.z, (xv.w * inv) * gv.w);
            *reinterpret_cast<float4 *>(xn + (q * (COLS / EPC) + c) * 4) = v;
        }
    }
    __syncthreads();
}

// ---- int8: exact activation pieces and integer dot products -------------------------------
// Every int8 projection takes its input as the four exact int8 planes of qt_device.h
// (qt_pc8, one power-of-two scale per vector), so the dot products are exact int32 sums
// whatever forms them; the per-kernel matvec (qt_matvec.hip) computes the same integers
// with v_dot4 and the same f64 combination, so the two paths agree to the bit.
//
// Pieces live in LDS, 16 bytes per (16-element chunk c, plane q).  Two layouts:
//  plane-major  q*COLS + 16c: a wave reading plane q of chunks lane + 64j reads one
//               contiguous KiB (the v_dot4 path, one chunk per lane);
//  swizzled     the 64-byte group of chunk c inside its 256-byte block is XORed with the
//               block index, so the 16 lanes of an MFMA B-operand read (4 parts x 4 planes,
//               parts 4 chunks apart) hit 16 different 16-byte bank groups.
template <bool SW, int COLS>
__device__ __forceinline__ int pc_off(int c, int q) {
    if (SW) return ((c >> 2) << 8) | ((((c & 3) ^ ((c >> 2) & 3))) << 6) | (q << 4);
    return q * COLS + 16 * c;
}

// Pieces are made in units of 8 elements (half a 16-element chunk): unit u is half u % 2
// of chunk u / 2, read as two float4 of the chunk-transposed activation and written as
// 8 bytes of each plane.
template <bool SW, int COLS>
__device__ __forceinline__ void pc_put8(uint8_t *pc, int u, const float (&v)[8], float isc) {
    uint2 pl[4];
    qt_pc8(v, isc, pl);
#pragma unroll
    for (int q = 0; q < 4; q++) *reinterpret_cast<uint2 *>(pc + pc_off<SW, COLS>(u >> 1, q) + 8 * (u & 1)) = pl[q];
}

// Pieces of RMSNorm(x)*g (A, D) from the gather's statistics (pc_stats): the mean square
// is the waves' partial sums added in wave order, and the scale comes from
// M = inv * max|x*g| * (1 + 2^-20), an upper bound of max|(x*inv)*g| (two f32 roundings
// lie far inside the margin).  k_mv forms both the same way.  Thread u normalises unit u
// and writes its planes.  Returns s; ends with a barrier.
template <int NW>
__device__ __forceinline__ void pc_norm_scale(const float *wst, int cols, float eps, float &inv, QtPcScale &ps) {
    float ss = wst[0], m = wst[1];
#pragma unroll
    for (int w = 1; w < NW; w++) { ss += wst[2 * w]; m = fmaxf(m, wst[2 * w + 1]); }
    inv = 1.0f / sqrtf(ss / (float)cols + eps);
    ps = qt_pc_scale((inv * m) * (1.0f + 0x1p-20f));
}
template <bool SW, int COLS, int NT>
__device__ __forceinline__ float stage_norm_pc(const float *x, const float *gain, float eps, uint8_t *pc, const float *wst) {
    constexpr int EPC = 16, NU = COLS / 8;
    float inv;
    QtPcScale ps;
    pc_norm_scale<NT / 64>(wst, COLS, eps, inv, ps);
    for (int u = threadIdx.x; u < NU; u += NT) {
        float v[8];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const float4 xv = xchunk4<EPC, COLS>(x, u >> 1, 2 * (u & 1) + h);
            const float4 g = xchunk4<EPC, COLS>(gain, u >> 1, 2 * (u & 1) + h);
            v[4 * h] = (xv.x * inv) * g.x; v[4 * h + 1] = (xv.y * inv) * g.y;
            v[4 * h + 2] = (xv.z * inv) * g.z; v[4 * h + 3] = (xv.w * inv) * g.w;
        }
        pc_put8<SW, COLS>(pc, u, v, ps.isc);
    }
    __syncthreads();
    return ps.s;
}

// Pieces of x (C, E): m = max|x| from the gather's statistics.  Returns s; ends with a
// barrier.
template <bool SW, int COLS, int NT>
__device__ __forceinline__ float stage_pc(const float *x, const float *wst, uint8_t *pc) {
    constexpr int EPC = 16, NU = COLS / 8;
    float m = wst[1];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) m = fmaxf(m, wst[2 * w + 1]);
    const QtPcScale ps = qt_pc_scale(m);
    // unrolled over the thread's units: every LDS read is issued before the first convert
    constexpr int NK = (NU + NT - 1) / NT;
    float v[NK][8];
#pragma unroll
    for (int k = 0; k < NK; k++) {
        const int u = threadIdx.x + k * NT;
        if (NU % NT == 0 || u < NU) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const float4 xv = xchunk4<EPC, COLS>(x, u >> 1, 2 * (u & 1) + h);
                v[k][4 * h] = xv.x; v[k][4 * h + 1] = xv.y; v[k][4 * h + 2] = xv.z; v[k][4 * h + 3] = xv.w;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < NK; k++) {
        const int u = threadIdx.x + k * NT;
        if (NU % NT == 0 || u < NU) pc_put8<SW, COLS>(pc, u, v[k], ps.isc);
    }
    __syncthreads();
    return ps.s;
}

// v_dot4 path (rows per wave, lanes over chunks, plane-major pieces): acc[r] = the dot of
// row r (valid in every lane), before the row scale.
template <int COLS, int NR>
__device__ __forceinline__ void tile_dot_pc(const Tile<QT_INT8, COLS, NR> &t, const uint8_t *pc, float s, float (&acc)[NR]) {
    using T = Tile<QT_INT8, COLS, NR>;
    const int lane = threadIdx.x & 63;
    int d[NR][4];
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
        for (int q = 0; q < 4; q++) d[r][q] = 0;
#pragma unroll
    for (int j = 0; j < T::CPL; j++) {
        const int c = lane + 64 * j;
        uint4 p[4];
#pragma unroll
        for (int q = 0; q < 4; q++) p[q] = *reinterpret_cast<const uint4 *>(pc + pc_off<false, COLS>(c, q));
#pragma unroll
        for (int r = 0; r < NR; r++)
#pragma unroll
            for (int q = 0; q < 4; q++) d[r][q] = qt_dot16(t.w[r][j], p[q], d[r][q]);
    }
#pragma unroll
    for (int r = 0; r < NR; r++) {
#pragma unroll
        for (int q = 0; q < 4; q++) d[r][q] = group_sum_i<64>(d[r][q]);
        acc[r] = qt_pc_dot(d[r][0], d[r][1], d[r][2], d[r][3], s);
    }
}

// MFMA path (hidden 2048).  v_mfma_i32_16x16x64_i8 (wave64): lane l supplies 16 bytes of
// A row (l % 16) and of B column (l % 16) for k group kg = l / 16, and receives D rows
// 4*(l/16)+i (i < 4) of column l % 16.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 mfma_i8(uint4 w, uint4 p, i32x4 acc) {
    const i32x4 A = i32x4{(int)w.x, (int)w.y, (int)w.z, (int)w.w};
    const i32x4 B = i32x4{(int)p.x, (int)p.y, (int)p.z, (int)p.w};
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, acc, 0, 0, 0);
}

// 4 rows per wave (the wave's rows row0w..row0w+3) over all COLS: MFMA row m = row m % 4
// of part m / 4; step s covers columns s*256 + part*64 + 16*kg .. +15, so one load
// instruction reads 256 contiguous bytes of each of the 4 rows.  B column n = plane n % 4
// of part n / 4.  D[4p+j][4p+q] (lane 20p+q, register j) is the part-p, plane-q sum of
// row j.
// Row scales are loaded per lane for the lanes that finish the rows (a lane-dependent
// pick among wave-uniform values would make the compiler index an array in scratch):
// PAIR = false: rs[0] = scale of row lane % 4; PAIR = true (gate|up pieces): rs[0], rs[1] =
// scales of rows 2i, 2i+1 with i = lane % 2.
template <int COLS, bool PAIR>
struct TileM4 {
    static constexpr int S = COLS / 256;
    static_assert(S * 256 == COLS, "tile shape");
    uint4 w[S];
    float rs[2];
    __device__ __forceinline__ void load(const uint8_t *W, const void *Sv, int row0w) {
        const float *Sc = static_cast<const float *>(Sv);   // int8 row scales
        const int lane = threadIdx.x & 63, m = lane & 15, kg = lane >> 4;
        W = uni(W);
        const uint8_t *p = W + (size_t)(row0w + (m & 3)) * COLS + (m >> 2) * 64 + kg * 16;
#pragma unroll
        for (int s = 0; s < S; s++) w[s] = ldg(reinterpret_cast<const uint4 *>(p + s * 256));
        if (PAIR) {
            rs[0] = ldg(Sc + row0w + 2 * (lane & 1));
            rs[1] = ldg(Sc + row0w + 2 * (lane & 1) + 1);
        } else {
            rs[0] = ldg(Sc + row0w + (lane & 3));
            rs[1] = 0.f;
        }
    }
};
// The B fragment of step s is read one step ahead; a single tile alternates two
// accumulator chains (summed exactly at the end), three tiles share each B fragment.
template <int COLS>
__device__ __forceinline__ uint4 mf_b4(const uint8_t *pc, int s) {
    const int lane = threadIdx.x & 63, n = lane & 15, kg = lane >> 4;
    return *reinterpret_cast<const uint4 *>(pc + pc_off<true, COLS>(16 * s + 4 * (n >> 2) + kg, n & 3));
}
template <int COLS, bool PAIR>
__device__ __forceinline__ i32x4 mf_dot4(const TileM4<COLS, PAIR> &t, const uint8_t *pc) {
    constexpr int S = TileM4<COLS, PAIR>::S;
    i32x4 acc[2] = {i32x4{0, 0, 0, 0}, i32x4{0, 0, 0, 0}};
    uint4 b = mf_b4<COLS>(pc, 0);
#pragma unroll
    for (int s = 0; s < S; s++) {
        const uint4 bn = mf_b4<COLS>(pc, s + 1 < S ? s + 1 : s);
        acc[s & 1] = mfma_i8(t.w[s], b, acc[s & 1]);
        b = bn;
    }
    return acc[0] + acc[1];
}
template <int COLS, bool PAIR>
__device__ __forceinline__ void mf_dot4x3(const TileM4<COLS, PAIR> &t0, const TileM4<COLS, PAIR> &t1,
                                          const TileM4<COLS, PAIR> &t2, const uint8_t *pc, i32x4 (&acc)[3]) {
    constexpr int S = TileM4<COLS, PAIR>::S;
#pragma unroll
    for (int i = 0; i < 3; i++) acc[i] = i32x4{0, 0, 0, 0};
    uint4 b = mf_b4<COLS>(pc, 0);
#pragma unroll
    for (int s = 0; s < S; s++) {
        const uint4 bn = mf_b4<COLS>(pc, s + 1 < S ? s + 1 : s);
        acc[0] = mfma_i8(t0.w[s], b, acc[0]);
        acc[1] = mfma_i8(t1.w[s], b, acc[1]);
        acc[2] = mfma_i8(t2.w[s], b, acc[2]);
        b = bn;
    }
}
// Part sums of a TileM4 result through 64 ints of the wave's own LDS scratch: the 16
// lanes that hold same-part entries store them (mf_store4); then any lane may sum row j's
// four parts per plane (mf_rowsum).  One wave writes and reads its own scratch, in order.
__device__ __forceinline__ void mf_store4(i32x4 acc, int *red) {
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    if ((n >> 2) == g) *reinterpret_cast<i32x4 *>(red + (g * 4 + (n & 3)) * 4) = acc;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}
__device__ __forceinline__ void mf_rowsum(const int *red, int j, int (&d)[4]) {
#pragma unroll
    for (int q = 0; q < 4; q++)
        d[q] = red[(0 * 4 + q) * 4 + j] + red[(1 * 4 + q) * 4 + j] + red[(2 * 4 + q) * 4 + j] + red[(3 * 4 + q) * 4 + j];
}

// 8 rows per workgroup (row0..row0+7) with the columns split over the 4 waves (wave w:
// columns w*COLS/4 ..): MFMA row m = row m % 8 of part m / 8; step s covers slice
// columns s*128 + part*64 + 16*kg.  B column n < 8 = plane n % 4 of part n / 4.  The
// useful entries D[8p+r][4p+q] sit in lanes 16*(2p + r/4) + 4p + q, register r % 4.
template <int COLS>
struct TileK8 {
    static constexpr int S = COLS / 512;
    static_assert(S * 512 == COLS, "tile shape");
    uint4 w[S];
    float rs;                // lane t < 8: scale of row row0 + t
    __device__ __forceinline__ void load(const uint8_t *W, const void *Sv, int row0, int wave) {
        const float *Sc = static_cast<const float *>(Sv);   // int8 row scales
        const int lane = threadIdx.x & 63, m = lane & 15, kg = lane >> 4;
        W = uni(W);
        const uint8_t *p = W + (size_t)(row0 + (m & 7)) * COLS + wave * (COLS / 4) + (m >> 3) * 64 + kg * 16;
#pragma unroll
        for (int s = 0; s < S; s++) w[s] = ldg(reinterpret_cast<const uint4 *>(p + s * 128));
        rs = ldg(Sc + row0 + (lane & 7));
    }
};
template <int COLS>
__device__ __forceinline__ uint4 mf_b8(const uint8_t *pc, int wave, int s) {
    const int lane = threadIdx.x & 63, n = lane & 15, kg = lane >> 4;
    uint4 b = make_uint4(0, 0, 0, 0);
    if (n < 8) b = *reinterpret_cast<const uint4 *>(pc + pc_off<true, COLS>(wave * (COLS / 64) + 8 * s + 4 * (n >> 2) + kg, n & 3));
    return b;
}
template <int COLS>
__device__ __forceinline__ i32x4 mf_dot8(const TileK8<COLS> &t, const uint8_t *pc, int wave) {
    constexpr int S = TileK8<COLS>::S;
    i32x4 acc[2] = {i32x4{0, 0, 0, 0}, i32x4{0, 0, 0, 0}};
    uint4 b = mf_b8<COLS>(pc, wave, 0);
#pragma unroll
    for (int s = 0; s < S; s++) {
        const uint4 bn = mf_b8<COLS>(pc, wave, s + 1 < S ? s + 1 : s);
        acc[s & 1] = mfma_i8(t.w[s], b, acc[s & 1]);
        b = bn;
    }
    return acc[0] + acc[1];
}
// Cross-wave sum of TileK8 results: each wave stores its 16 useful lanes into red[wave]
// (64 ints), barrier, then thread t < 8 sums row t over waves and parts per plane.
template <int NW>
__device__ __forceinline__ void mf_rows8(i32x4 acc, int *red, int wave, int (&d)[4]) {
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    if (n < 8 && (n >> 2) == (g >> 1)) *reinterpret_cast<i32x4 *>(red + wave * 64 + (g * 4 + (n & 3)) * 4) = acc;
    __syncthreads();
    const int t = threadIdx.x & 7, rh = t >> 2, i = t & 3;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        int v = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) v += red[w * 64 + (rh * 4 + q) * 4 + i] + red[w * 64 + ((2 + rh) * 4 + q) * 4 + i];
        d[q] = v;
    }
}
}  // namespace ps
