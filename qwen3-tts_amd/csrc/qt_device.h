// qt_device.h — device-side helpers shared by the gfx950 decode kernels.
//
// Weight storage on the device (set up once by qwen_tts_hip.c at init):
//   bf16  rows of 2*cols bytes, the reference's row-major bits unchanged;
//   int8  rows of cols signed bytes q, the reference's quantizer output unchanged
//         (the integer dot products take them as they are).  Scale f32 per row.
//   q4_0  the reference's 18-byte blocks split into qs rows (cols/2 bytes) and a
//         [rows][cols/32] array of f16 scale bits, so qs rows are 16-byte aligned
//         and one 128-bit load covers exactly one block.
// Every matvec streams weights with 128-bit loads: one 16-byte "chunk" per lane per
// load, consecutive lanes on consecutive chunks of a row, so a wave reads 1 KiB of a
// row per load instruction.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define QT_WG 256          // threads per workgroup in every matvec/attention kernel
#define QT_WAVES 4

enum { QT_BF16 = 0, QT_INT8 = 1, QT_Q4 = 2 };
enum { QT_EPI_STORE = 0, QT_EPI_RESID = 1, QT_EPI_SWIGLU = 2, QT_EPI_BIAS = 3 };

struct QtMat {
    const uint8_t *w;      // chunk rows (see above)
    const float *scale;    // int8 per-row scale
    const uint16_t *s16;   // q4 per-block f16 scale bits [rows][cols/32]
    int rows, cols;
};

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ float bf16f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ uint16_t f2bf_trunc(float f) { return (uint16_t)(__float_as_uint(f) >> 16); }

// binary16 -> f32 exactly as the reference's portable branch (qwen_tts_kernels.h:162-179),
// including its subnormal mapping (exponent field 112 - shift).
__device__ __forceinline__ float ref_f16_to_f32(uint32_t h) {
    uint32_t sign = (h & 0x8000u) << 16;
    uint32_t em = h & 0x7FFFu, bits;
    if (em >= 0x7C00u) bits = sign | 0x7F800000u | ((em & 0x3FFu) << 13);
    else if (em >= 0x0400u) bits = sign | ((em + (112u << 10)) << 13);
    else if (em == 0) bits = sign;
    else {
        uint32_t sh = __clz(em) - 21;          // shifts until bit 10 is set
        uint32_t m = em << sh;
        bits = sign | ((112u - sh) << 23) | ((m & 0x3FFu) << 13);
    }
    return __uint_as_float(bits);
}

// Reductions over W-lane groups (W = 16, 32 or 64) with DPP lane moves (VALU, no LDS
// round trip).  Inside a 16-lane row the steps are symmetric exchanges (quad xor 1,
// quad xor 2, half-row mirror, row mirror), so every lane of a row ends with the same
// bits; rows are then combined with row_bcast15/31 and the group's last lane is
// broadcast, so every lane of a group returns the identical value.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_mov_keep(float v) {   // lanes outside ROW_MASK keep v
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}
constexpr int DPP_QXOR1 = 0xB1, DPP_QXOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140,
              DPP_BCAST15 = 0x142, DPP_BCAST31 = 0x143;

__device__ __forceinline__ float lane_bcast(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

template <int W>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(W == 16 || W == 32 || W == 64, "group width");
    v += dpp_mov<DPP_QXOR1>(v);
    v += dpp_mov<DPP_QXOR2>(v);
    v += dpp_mov<DPP_HALF_MIRROR>(v);
    v += dpp_mov<DPP_MIRROR>(v);
    if (W == 16) return v;
    v += dpp_mov<DPP_BCAST15, 0xa>(v);           // rows 1, 3: + row 0, row 2
    if (W == 32) {
        const float lo = lane_bcast(v, 31), hi = lane_bcast(v, 63);
        return (threadIdx.x & 32) ? hi : lo;
    }
    v += dpp_mov<DPP_BCAST31, 0xc>(v);           // rows 2, 3: + lane 31 (rows 0+1)
    return lane_bcast(v, 63);
}
template <int W>
__device__ __forceinline__ float group_max(float v) {
    static_assert(W == 16 || W == 32 || W == 64, "group width");
    v = fmaxf(v, dpp_mov_keep<DPP_QXOR1>(v));
    v = fmaxf(v, dpp_mov_keep<DPP_QXOR2>(v));
    v = fmaxf(v, dpp_mov_keep<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_mov_keep<DPP_MIRROR>(v));
    if (W == 16) return v;
    v = fmaxf(v, dpp_mov_keep<DPP_BCAST15, 0xa>(v));
    if (W == 32) {
        const float lo = lane_bcast(v, 31), hi = lane_bcast(v, 63);
        return (threadIdx.x & 32) ? hi : lo;
    }
    v = fmaxf(v, dpp_mov_keep<DPP_BCAST31, 0xc>(v));
    return lane_bcast(v, 63);
}

// Block-wide sum over QT_WG threads; every thread gets the result.  `red` >= QT_WAVES floats.
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = group_sum<64>(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < QT_WAVES; i++) t += red[i];
    return t;
}

// Merge of split-K softmax partials, one key chunk per lane of a 32-lane half-wave:
// lane cc holds the chunk's running max m (in base-2 units: scores scaled by log2(e)),
// exp-sum l and unnormalised output o (valid for cc < nch).  out = sum_cc o_cc f_cc /
// sum_cc l_cc f_cc with f_cc = 2^(m_cc - M), M = max_cc m_cc; both sums are half-wave reductions, so every merge of the same
// partials (per-kernel attention or the fused step) rounds identically.  A single
// chunk reduces exactly to o / l.
__device__ __forceinline__ float softmax_merge32(float m, float l, float o, bool valid) {
    const float M = group_max<32>(valid ? m : -INFINITY);
    const float f = valid ? __builtin_amdgcn_exp2f(m - M) : 0.f;
    const float L = group_sum<32>(valid ? l * f : 0.f);
    const float V = group_sum<32>(valid ? o * f : 0.f);
    return V * (1.0f / L);
}

template <int W>
__device__ __forceinline__ int group_sum_i(int v) {        // exact: integer adds
    static_assert(W == 16 || W == 32 || W == 64, "group width");
    v += __builtin_amdgcn_update_dpp(0, v, DPP_QXOR1, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, DPP_QXOR2, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, DPP_HALF_MIRROR, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, DPP_MIRROR, 0xf, 0xf, false);
    if (W == 16) return v;
    v += __builtin_amdgcn_update_dpp(0, v, DPP_BCAST15, 0xa, 0xf, false);
    if (W == 32) {
        const int lo = __builtin_amdgcn_readlane(v, 31), hi = __builtin_amdgcn_readlane(v, 63);
        return (threadIdx.x & 32) ? hi : lo;
    }
    v += __builtin_amdgcn_update_dpp(0, v, DPP_BCAST31, 0xc, 0xf, false);
    return __builtin_amdgcn_readlane(v, 63);
}

// One reduce-scatter step over the first N values: the lane and its DPP partner differ
// in one lane bit (`hi`); each keeps the half of the N values that bit selects and adds
// the partner's copy of that half, so the first N/2 entries then hold pair sums.
template <int CTRL, int N, int V>
__device__ __forceinline__ void qt_scatter_step(int (&v)[V], bool hi) {
#pragma unroll
    for (int k = 0; k < N / 2; k++) {
        const int send = hi ? v[k] : v[k + N / 2], keep = hi ? v[k + N / 2] : v[k];
        v[k] = keep + __builtin_amdgcn_update_dpp(0, send, CTRL, 0xf, 0xf, false);
    }
}
// Exact wave-wide sums of V = 4, 8 or 16 integers per lane, returned uniform.  Inside
// each 16-lane row a reduce-scatter over the partners lane^15 (row mirror), lane^7
// (half-row mirror), lane^2 and lane^1 leaves value i's row sum in the lanes whose bits
// 3..0 spell i (in the top log2 V of them); the four rows are then added with the
// row-pair and half-wave swaps, and value i is read from lane i*16/V.  About 3V lane
// moves and selects instead of the 6V of V separate reductions; integer adds, so the
// result does not depend on the order.
template <int V>
__device__ __forceinline__ void wave_sum_i_scatter(int (&v)[V], int (&out)[V]) {
    static_assert(V == 4 || V == 8 || V == 16, "values");
    const int lane = threadIdx.x & 63;
    qt_scatter_step<DPP_MIRROR, V>(v, lane & 8);
    qt_scatter_step<DPP_HALF_MIRROR, V / 2>(v, lane & 4);
    if constexpr (V >= 8) qt_scatter_step<DPP_QXOR2, V / 4>(v, lane & 2);
    else v[0] += __builtin_amdgcn_update_dpp(0, v[0], DPP_QXOR2, 0xf, 0xf, false);
    if constexpr (V >= 16) qt_scatter_step<DPP_QXOR1, V / 8>(v, lane & 1);
    else v[0] += __builtin_amdgcn_update_dpp(0, v[0], DPP_QXOR1, 0xf, 0xf, false);
    const auto p = __builtin_amdgcn_permlane16_swap(v[0], v[0], false, false);   // rows 0+1, 2+3
    const int t = (int)p[0] + (int)p[1];
    const auto q = __builtin_amdgcn_permlane32_swap(t, t, false, false);         // halves
    const int u = (int)q[0] + (int)q[1];
#pragma unroll
    for (int i = 0; i < V; i++) out[i] = __builtin_amdgcn_readlane(u, i * (16 / V));
}

// ---- exact int8 activation pieces (every int8 matvec) ----------------------------------
// An f32 activation vector v is written as one 30-bit integer per element with one
// power-of-two scale: s = 2^(e-29), 2^e <= m = max|v| < 2^(e+1), Y = rint(v/s), so
// |Y| <= 2^30 and |v - s*Y| <= s/2 <= m*2^-30 (Y is exact wherever |v| >= m*2^-6, since
// v/s is then already an integer).  Y is split into four balanced base-256 digits, the
// bytes of t = Y + 0x80808080 each minus 128 (int8 p0..p3, Y = p0 + 2^8 p1 + 2^16 p2 +
// 2^24 p3), giving four int8 planes.  Their products with the int8 weights q are summed
// exactly in int32 (|sum| <= 128*128*K < 2^31 for K < 131072), so the four dot products
// D0..D3 depend neither on summation order nor on the instruction forming them (MFMA in
// the fused step, v_dot4 in the matvec kernel).  The dot is
// s*(D0 + 2^8 D1 + 2^16 D2 + 2^24 D3), formed exactly in f64 and rounded once to f32; the
// row scale is then applied once in f32 as the reference does
// (qwen_tts_kernels.c:2350-2351).  m < 2^-90 or not finite: s = 0, every piece 0.
struct QtPcScale { float s, isc; };
__device__ __forceinline__ QtPcScale qt_pc_scale(float m) {
    const bool ok = m >= 0x1p-90f && m <= 3.0e38f;
    const int e = ok ? ilogbf(m) : 0;
    return {ok ? ldexpf(1.0f, e - 29) : 0.f, ok ? ldexpf(1.0f, 29 - e) : 0.f};
}
// biased word t = Y + 0x80808080 of one value
__device__ __forceinline__ uint32_t qt_pc_word(float v, float isc) {
    return (uint32_t)(int)rintf(v * isc) + 0x80808080u;
}
// 4x4 byte transpose of four biased words into the four planes of those values (plane
// q, byte e = digit q of value e, as a signed int8)
__device__ __forceinline__ void qt_pc_t4(uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3, uint32_t (&pl)[4]) {
    const uint32_t a = __builtin_amdgcn_perm(t1, t0, 0x05010400u), b = __builtin_amdgcn_perm(t3, t2, 0x05010400u);
    const uint32_t c = __builtin_amdgcn_perm(t1, t0, 0x07030602u), d = __builtin_amdgcn_perm(t3, t2, 0x07030602u);
    pl[0] = __builtin_amdgcn_perm(b, a, 0x05040100u) ^ 0x80808080u;
    pl[1] = __builtin_amdgcn_perm(b, a, 0x07060302u) ^ 0x80808080u;
    pl[2] = __builtin_amdgcn_perm(d, c, 0x05040100u) ^ 0x80808080u;
    pl[3] = __builtin_amdgcn_perm(d, c, 0x07060302u) ^ 0x80808080u;
}
// the four planes of 8 consecutive values (plane q: 8 bytes)
__device__ __forceinline__ void qt_pc8(const float (&v)[8], float isc, uint2 (&pl)[4]) {
    uint32_t lo[4], hi[4];
    qt_pc_t4(qt_pc_word(v[0], isc), qt_pc_word(v[1], isc), qt_pc_word(v[2], isc), qt_pc_word(v[3], isc), lo);
    qt_pc_t4(qt_pc_word(v[4], isc), qt_pc_word(v[5], isc), qt_pc_word(v[6], isc), qt_pc_word(v[7], isc), hi);
#pragma unroll
    for (int q = 0; q < 4; q++) pl[q] = make_uint2(lo[q], hi[q]);
}
// the four planes of 16 consecutive values (plane q: 16 bytes)
__device__ __forceinline__ void qt_pc16(const float (&v)[16], float isc, uint4 (&pl)[4]) {
    uint32_t w[4][4];
#pragma unroll
    for (int g = 0; g < 4; g++) {
        uint32_t t[4];
        qt_pc_t4(qt_pc_word(v[4 * g], isc), qt_pc_word(v[4 * g + 1], isc), qt_pc_word(v[4 * g + 2], isc),
                 qt_pc_word(v[4 * g + 3], isc), t);
#pragma unroll
        for (int q = 0; q < 4; q++) w[q][g] = t[q];
    }
#pragma unroll
    for (int q = 0; q < 4; q++) pl[q] = make_uint4(w[q][0], w[q][1], w[q][2], w[q][3]);
}
// the dot product from the four exact plane sums
__device__ __forceinline__ float qt_pc_dot(int d0, int d1, int d2, int d3, float s) {
    const double c = (double)d0 + (double)d1 * 0x1p8 + (double)d2 * 0x1p16 + (double)d3 * 0x1p24;
    return (float)(c * (double)s);
}
// q . p for 16 weight bytes q and 16 piece bytes of one plane
__device__ __forceinline__ int qt_dot16(uint4 w, uint4 p, int acc) {
    acc = __builtin_amdgcn_sdot4((int)w.x, (int)p.x, acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.y, (int)p.y, acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.z, (int)p.z, acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.w, (int)p.w, acc, false);
    return acc;
}

// Agent-scope relaxed accesses: compiled to global_load/store with the sc1 bit, so they
// go to the device coherence point instead of a (per-XCD, non-coherent) L2 line.  Used
// for the few values one workgroup publishes to workgroups on other XCDs inside one
// kernel; ordering is by s_waitcnt + a device-scope atomic, no L2 write-back/invalidate.
__device__ __forceinline__ void st_agent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint4 ld_chunk(const uint8_t *p) {
    return *reinterpret_cast<const uint4 *>(p);
}
