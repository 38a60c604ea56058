// qt_attn_mf.h — an attention chunk's q.k and P.V on the bf16 matrix cores (gfx950),
// shared by the per-kernel attention (qt_attn.hip) and the fused step's attention phase
// (qt_pstep.hip), so both compute every score and every partial output the same way.
//
// Operands.  v_mfma_f32_16x16x32_bf16: lane l supplies row l%16 of A and column l%16 of
// B, each as the 8 consecutive k of group l/16 (16 bytes); D[4*(l/16)+i][l%16] is lane
// l's accumulator i.  An f32 value x is split into three bf16 pieces whose sum is x
// exactly (x truncated to bf16, the truncated rest, the remaining <= 8 significant
// bits); a bf16 x bf16 product is exact in f32, so the matrix core adds, in f32, exact
// products of the f32 query (probabilities) with the bf16 keys (values).
//   scores: A = query pieces (row 4h+p = piece p of head h; p == 3 and h >= HPK rows
//           zero), B = 16 key rows (key = column): lane l ends with the three piece
//           sums of head l/16, key l%16, and the score is (D0 + D1) + D2.
//   P.V:    A = probability pieces (same rows) over 32 keys, B = those keys' value rows
//           for 16 dims, read with the transposing LDS load: lane l ends with head
//           l/16, dim l%16, again as (D0 + D1) + D2 after the last key tile.
//
// LDS layout of a staged key block (row j = 128 bf16 = 16 chunks of 16 bytes):
//   K: chunk c of row j at slot c ^ (j & 15)   — the 16 keys of a score tile read one
//      chunk index each from 16 different bank groups;
//   V: chunk c of row j at slot c ^ vsw(j), vsw(j) = 2*((j & 3) | ((j >> 1) & 4)) —
//      a transposing read covers rows {b..b+3, b+8..b+11} x 32 bytes per half-wave,
//      which land on 8 different 32-byte bank groups.
// The global->LDS copies pick their source chunk so that lane L of a 1-KiB copy (block
// row 4i + L/16, slot L%16) fetches the chunk that belongs in that slot.
#pragma once
#include "qt_device.h"

typedef __bf16 qt_bf16x8 __attribute__((ext_vector_type(8)));
typedef float qt_f32x4 __attribute__((ext_vector_type(4)));
typedef short qt_i16x4 __attribute__((ext_vector_type(4)));
typedef unsigned qt_u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int qt_kslot(int row, int c) { return c ^ (row & 15); }
__device__ __forceinline__ int qt_vslot(int row, int c) { return c ^ (2 * ((row & 3) | ((row >> 1) & 4))); }

__device__ __forceinline__ qt_f32x4 qt_mfma_bf16(qt_u32x4 a, qt_u32x4 b, qt_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(qt_bf16x8, a), __builtin_bit_cast(qt_bf16x8, b),
                                                   c, 0, 0, 0);
}
__device__ __forceinline__ qt_u32x4 qt_lds16(const void *p) { return *reinterpret_cast<const qt_u32x4 *>(p); }
__device__ __forceinline__ qt_u32x4 qt_lds_tr8x2(const uint16_t *p0, const uint16_t *p1) {
    const qt_i16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) qt_i16x4 *)p0);
    const qt_i16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) qt_i16x4 *)p1);
    const uint2 ua = __builtin_bit_cast(uint2, a), ub = __builtin_bit_cast(uint2, b);
    return qt_u32x4{ua.x, ua.y, ub.x, ub.y};
}

// The three bf16 pieces of x, stored at dst[0], dst[stride], dst[2*stride]:
// piece0 + piece1 + piece2 == x exactly
__device__ __forceinline__ void qt_put_pieces(uint16_t *dst, int stride, float x) {
    const uint32_t u0 = __float_as_uint(x) & 0xFFFF0000u;
    const float r1 = x - __uint_as_float(u0);
    const uint32_t u1 = __float_as_uint(r1) & 0xFFFF0000u;
    const float r2 = r1 - __uint_as_float(u1);
    dst[0] = (uint16_t)(u0 >> 16);
    dst[stride] = (uint16_t)(u1 >> 16);
    dst[2 * stride] = (uint16_t)(__float_as_uint(r2) >> 16);
}

// A operand (row 4h+p = piece p of head h, rows with p == 3 or h >= HPK zero) for the
// 8 consecutive k at column k0 + 8(l/16) of piece rows pc[(3h + p) * stride] (LDS)
template <int HPK>
__device__ __forceinline__ qt_u32x4 qt_att_rowpiece(const uint16_t *pc, int stride, int k0, int lane) {
    const int m = lane & 15, h = m >> 2, p = m & 3;
    const bool on = h < HPK && p < 3;
    const qt_u32x4 v = qt_lds16(pc + ((h < HPK ? h : HPK - 1) * 3 + (p < 3 ? p : 2)) * stride + k0 + 8 * (lane >> 4));
    return on ? v : qt_u32x4{0u, 0u, 0u, 0u};
}

// Unscaled scores of T 16-key tiles (block rows r0[t] .. r0[t]+15 of the staged K block
// kb): lane l gets the score of head l/16 with key row r0[t] + l%16 in sc[t].  qp: query
// pieces [HPK][3][128] (LDS).  Row nrow (the key appended by this step, not staged) is
// read from knew.  Every LDS read is issued before the first MFMA.
template <int HPK, int T>
__device__ __forceinline__ void qt_att_qk(const uint16_t *qp, const uint16_t *kb, const uint16_t *knew,
                                          const int (&r0)[T], int nrow, int lane, float (&sc)[T]) {
    const int kg = lane >> 4;
    qt_u32x4 qa[4], kv[T][4];
#pragma unroll
    for (int s = 0; s < 4; s++) qa[s] = qt_att_rowpiece<HPK>(qp, 128, 32 * s, lane);
#pragma unroll
    for (int t = 0; t < T; t++) {
        const int row = r0[t] + (lane & 15);
        const bool nw = row == nrow;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int c = 4 * s + kg;
            kv[t][s] = qt_lds16(nw ? knew + c * 8 : kb + row * 128 + qt_kslot(row, c) * 8);
        }
    }
    // one empty asm that takes every operand: all reads are issued before it, and it
    // waits once for all of them
    static_assert(T == 1 || T == 2, "one or two score tiles");
    if constexpr (T == 1)
        asm volatile("" : "+v"(qa[0]), "+v"(qa[1]), "+v"(qa[2]), "+v"(qa[3]), "+v"(kv[0][0]), "+v"(kv[0][1]),
                     "+v"(kv[0][2]), "+v"(kv[0][3]));
    else
        asm volatile("" : "+v"(qa[0]), "+v"(qa[1]), "+v"(qa[2]), "+v"(qa[3]), "+v"(kv[0][0]), "+v"(kv[0][1]),
                     "+v"(kv[0][2]), "+v"(kv[0][3]), "+v"(kv[T - 1][0]), "+v"(kv[T - 1][1]), "+v"(kv[T - 1][2]),
                     "+v"(kv[T - 1][3]));
#pragma unroll
    for (int t = 0; t < T; t++) {
        qt_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; s++) acc = qt_mfma_bf16(qa[s], kv[t][s], acc);
        sc[t] = (acc[0] + acc[1]) + acc[2];
    }
}

// ---- a staged block of NWV*32 keys in two steps, one workgroup barrier between ----
// Step 1 (qt_att_tiles), wave w: scores of its 16-key tiles w and w + NWV (block rows
// 16w .. +15 and 16(w+NWV) .. +15 = k-tile w), their max m_w per head, p = e^(s - m_w)
// as pieces into column 32w + k of pp, and l_w = sum p; (m_w, l_w) into ml.
// Step 2 (qt_att_pv), wave w: dims d0 .. d0+31 of every head over all NWV k-tiles, one
// MFMA per (k-tile, 16 dims), then o = sum_t e^(m_t - M) o_t with M = max_t m_t, and
// l = sum_t e^(m_t - M) l_t.  Lane l works on head l/16 throughout.
__device__ __forceinline__ void qt_wave_lds_sync() {   // this wave's LDS stores before its loads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int HPK, int NWV>
__device__ __forceinline__ void qt_att_tiles(const uint16_t *qp, const uint16_t *kblk, const uint16_t *knew,
                                             uint16_t *pp, int pstride, float *ml, int w, int nk, int nrow,
                                             float scale, int lane) {
    const int r0[2] = {16 * w, 16 * (w + NWV)};
    float sv[2];
    qt_att_qk<HPK, 2>(qp, kblk, knew, r0, nrow, lane, sv);   // rows past nk: discarded
    const int h = lane >> 4, key = lane & 15;
    const bool va = r0[0] + key < nk, vb = r0[1] + key < nk;
    const float sa = va ? sv[0] * scale : -INFINITY, sb = vb ? sv[1] * scale : -INFINITY;
    const float m = group_max<16>(fmaxf(sa, sb));            // -inf: no keys in this k-tile
    const float pa = va ? expf(sa - m) : 0.f, pb = vb ? expf(sb - m) : 0.f;
    const float ls = group_sum<16>(pa + pb);
    if (h < HPK) {
        qt_put_pieces(pp + 3 * h * pstride + 32 * w + key, pstride, pa);
        qt_put_pieces(pp + 3 * h * pstride + 32 * w + 16 + key, pstride, pb);
        if (key == 0) { ml[(w * HPK + h) * 2] = m; ml[(w * HPK + h) * 2 + 1] = ls; }
    }
}

template <int HPK, int NWV>
__device__ __forceinline__ void qt_att_pv(const uint16_t *pp, int pstride, const float *ml, const uint16_t *vblk,
                                          const uint16_t *vnew, const uint16_t *zeros, int d0, int nk, int nrow,
                                          int lane, float (&o)[2], float &M, float &l) {
    const int kg = lane >> 4, j = lane & 15, h = lane >> 4;
    const int hc = h < HPK ? h : HPK - 1;
    qt_u32x4 pa[NWV], vv[NWV][2];
    float mw[NWV], lw[NWV];
#pragma unroll
    for (int t = 0; t < NWV; t++) {
        pa[t] = qt_att_rowpiece<HPK>(pp, pstride, 32 * t, lane);
        mw[t] = ml[(t * HPK + hc) * 2];
        lw[t] = ml[(t * HPK + hc) * 2 + 1];
#pragma unroll
        for (int dt = 0; dt < 2; dt++) {
            const int col = d0 + 16 * dt + 4 * (j & 3);
            const uint16_t *p[2];
#pragma unroll
            for (int r2 = 0; r2 < 2; r2++) {
                const int kk = 8 * kg + 4 * r2 + (j >> 2);
                const int row = kk < 16 ? 16 * t + kk : 16 * (t + NWV) + kk - 16;
                p[r2] = row == nrow ? vnew + col
                      : row >= nk   ? zeros
                                    : vblk + row * 128 + qt_vslot(row, col >> 3) * 8 + (col & 7);
            }
            vv[t][dt] = qt_lds_tr8x2(p[0], p[1]);
        }
    }
    static_assert(NWV == 4, "four k-tiles");
    asm volatile("" : "+v"(pa[0]), "+v"(pa[1]), "+v"(pa[2]), "+v"(pa[3]), "+v"(vv[0][0]), "+v"(vv[0][1]),
                 "+v"(vv[1][0]), "+v"(vv[1][1]), "+v"(vv[2][0]), "+v"(vv[2][1]), "+v"(vv[3][0]), "+v"(vv[3][1]));
    qt_f32x4 acc[NWV][2];
#pragma unroll
    for (int t = 0; t < NWV; t++)
#pragma unroll
        for (int dt = 0; dt < 2; dt++) acc[t][dt] = qt_mfma_bf16(pa[t], vv[t][dt], qt_f32x4{0.f, 0.f, 0.f, 0.f});
    M = -INFINITY;
#pragma unroll
    for (int t = 0; t < NWV; t++) M = fmaxf(M, mw[t]);
    o[0] = o[1] = 0.f;
    l = 0.f;
#pragma unroll
    for (int t = 0; t < NWV; t++) {
        const float f = mw[t] == -INFINITY ? 0.f : expf(mw[t] - M);
        l = fmaf(lw[t], f, l);
#pragma unroll
        for (int dt = 0; dt < 2; dt++) o[dt] = fmaf((acc[t][dt][0] + acc[t][dt][1]) + acc[t][dt][2], f, o[dt]);
    }
}

// Running (max, sum, output) across the blocks of a chunk longer than one block.
struct QtAttRun {
    float m, l, o[2];
};
__device__ __forceinline__ void qt_att_run_init(QtAttRun &r) { r.m = -INFINITY; r.l = 0.f; r.o[0] = r.o[1] = 0.f; }
__device__ __forceinline__ void qt_att_run_add(QtAttRun &r, const float (&o)[2], float M, float l) {
    const float mn = fmaxf(r.m, M);
    const float fr = r.m == -INFINITY ? 0.f : expf(r.m - mn), fb = expf(M - mn);
    r.l = fmaf(r.l, fr, l * fb);
    r.o[0] = fmaf(r.o[0], fr, o[0] * fb);
    r.o[1] = fmaf(r.o[1], fr, o[1] * fb);
    r.m = mn;
}
