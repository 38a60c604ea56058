// qt_attn_mf.h — an attention chunk's q.k and P.V on the bf16 matrix cores (gfx950),
// shared by the per-kernel attention (qt_attn.hip) and the fused step's attention phase
// (qt_pstep.hip), so both compute every score and every partial output the same way.
//
// Operands.  v_mfma_f32_16x16x32_bf16: lane l supplies row l%16 of A and column l%16 of
// B, each as the 8 consecutive k of group l/16 (16 bytes); D[4*(l/16)+i][l%16] is lane
// l's accumulator i.  An f32 value x is split into three bf16 pieces whose sum is x
// exactly (x truncated to bf16, the truncated rest, the remaining <= 8 significant
// bits); a bf16 x bf16 product is exact in f32, so the matrix core adds, in f32, exact
// products of the f32 query (probabilities) with the bf16 keys (values).  The pieces
// live in LDS as 16 rows, row 4h+p = piece p of head h; rows with p == 3 and heads >=
// HPK stay zero (qt_att_zero_rows), so every lane reads its A operand unconditionally.
//   scores: A = query pieces, B = 16 key rows (key = column): lane l ends with the three
//           piece sums of head l/16, key l%16, and the score is (D0 + D1) + D2.
//   P.V:    A = probability pieces over 32 keys, B = those keys' value rows for 16 dims,
//           read with the transposing LDS load: lane l ends with head l/16, dim l%16.
// Softmax runs in base 2: scores are scaled by scale*log2(e), so e^(s - m) is
// 2^(s' - m') (v_exp_f32), and chunk maxima are published in those units.
//
// LDS layout of a staged key block (row j = 128 bf16 = 16 chunks of 16 bytes):
//   K: chunk c of row j at slot c ^ (j & 15)   — the 16 keys of a score tile read one
//      chunk index each from 16 different bank groups;
//   V: chunk c of row j at slot c ^ vsw(j), vsw(j) = 2*((j & 3) | ((j >> 1) & 4)) —
//      a transposing read covers rows {b..b+3, b+8..b+11} x 32 bytes per half-wave,
//      which land on 8 different 32-byte bank groups.
// The global->LDS copies pick their source chunk so that lane L of a 1-KiB copy (block
// row 4i + L/16, slot L%16) fetches the chunk that belongs in that slot.  The key
// appended by this step is written into its row by the workgroup (qt_kidx/qt_vidx,
// qt_att_put_kv), and value rows past the chunk are zeroed (qt_att_zero_vrows): their
// probabilities are 0, and stale bits could be NaN.
#pragma once
#include "qt_device.h"

typedef __bf16 qt_bf16x8 __attribute__((ext_vector_type(8)));
typedef float qt_f32x4 __attribute__((ext_vector_type(4)));
typedef short qt_i16x4 __attribute__((ext_vector_type(4)));
typedef unsigned qt_u32x4 __attribute__((ext_vector_type(4)));

#define QT_LOG2E 1.4426950408889634f

__device__ __forceinline__ int qt_kslot(int row, int c) { return c ^ (row & 15); }
__device__ __forceinline__ int qt_vslot(int row, int c) { return c ^ (2 * ((row & 3) | ((row >> 1) & 4))); }
__device__ __forceinline__ float qt_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

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

// Zero the rows of a [16][cols] piece array that no head writes (p == 3, h >= HPK).
template <int HPK>
__device__ __forceinline__ void qt_att_zero_rows(uint16_t *pc, int cols, int tid, int nt) {
    for (int i = tid; i < 16 * cols / 8; i += nt) {
        const int row = i / (cols / 8);
        if ((row & 3) == 3 || (row >> 2) >= HPK) *reinterpret_cast<uint4 *>(pc + 8 * i) = make_uint4(0u, 0u, 0u, 0u);
    }
}

// Zero the value rows [nk, rows) of a staged V block (any slot order); rows =
// 32 * ceil(nk / 32), the rows the P.V k-tiles read.
__device__ __forceinline__ void qt_att_zero_vrows(uint16_t *vblk, int nk, int rows, int tid, int nt) {
    for (int i = nk * 16 + tid; i < rows * 16; i += nt) *reinterpret_cast<uint4 *>(vblk + 8 * i) = make_uint4(0u, 0u, 0u, 0u);
}

// Element d (0..127) of block row `row`, at its swizzled place.
__device__ __forceinline__ int qt_kidx(int row, int d) { return row * 128 + qt_kslot(row, d >> 3) * 8 + (d & 7); }
__device__ __forceinline__ int qt_vidx(int row, int d) { return row * 128 + qt_vslot(row, d >> 3) * 8 + (d & 7); }

// Block row `row` of K and V from the bf16 rows knew / vnew (lanes 0..31 of one wave).
__device__ __forceinline__ void qt_att_put_kv(uint16_t *kblk, uint16_t *vblk, int row, const uint16_t *knew,
                                              const uint16_t *vnew, int lane) {
    if (lane < 16)
        *reinterpret_cast<uint4 *>(kblk + row * 128 + qt_kslot(row, lane) * 8) = *reinterpret_cast<const uint4 *>(knew + 8 * lane);
    else if (lane < 32)
        *reinterpret_cast<uint4 *>(vblk + row * 128 + qt_vslot(row, lane - 16) * 8) =
            *reinterpret_cast<const uint4 *>(vnew + 8 * (lane - 16));
}

// Scores of two 16-key tiles (block rows r0[t] .. r0[t]+15 of the staged K block kb):
// lane l gets the q.k sum of head l/16 with key row r0[t] + l%16 in sc[t].  qp: query
// pieces [16][128] (LDS).  Every LDS read is issued before the first MFMA.
__device__ __forceinline__ void qt_att_qk2(const uint16_t *qp, const uint16_t *kb, const int (&r0)[2], int lane,
                                           float (&sc)[2]) {
    const int kg = lane >> 4, key = lane & 15;
    qt_u32x4 qa[4], kv[2][4];
#pragma unroll
    for (int s = 0; s < 4; s++) qa[s] = qt_lds16(qp + key * 128 + 32 * s + 8 * kg);
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int s = 0; s < 4; s++) kv[t][s] = qt_lds16(kb + (r0[t] + key) * 128 + ((4 * s + kg) ^ key) * 8);
    // one empty asm that takes every operand: all reads are issued before it, and it
    // waits once for all of them
    asm volatile("" : "+v"(qa[0]), "+v"(qa[1]), "+v"(qa[2]), "+v"(qa[3]), "+v"(kv[0][0]), "+v"(kv[0][1]),
                 "+v"(kv[0][2]), "+v"(kv[0][3]), "+v"(kv[1][0]), "+v"(kv[1][1]), "+v"(kv[1][2]), "+v"(kv[1][3]));
#pragma unroll
    for (int t = 0; t < 2; t++) {
        qt_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; s++) acc = qt_mfma_bf16(qa[s], kv[t][s], acc);
        sc[t] = (acc[0] + acc[1]) + acc[2];
    }
}

// ---- a staged block of up to 128 keys in two steps, one workgroup barrier between ----
// k-tile t = block rows 32t .. 32t+31; only the nkt = ceil(nk/32) k-tiles holding keys
// take part, and value rows [nk, 32*nkt) are zeroed before step 2.
// Step 1 (qt_att_tiles), wave w < nkt: scores (base 2) of k-tile w as two 16-key score
// tiles, their max m_w per head, p = 2^(s - m_w) as pieces into columns 32w .. 32w+31 of
// pp, l_w = sum p; (m_w, l_w) into ml.
// Step 2 (qt_att_pv), every wave: dims d0 .. d0+31 of every head over the NKT k-tiles,
// one MFMA per (k-tile, 16 dims), then o = sum_t 2^(m_t - M) o_t with M = max_t m_t,
// and l = sum_t 2^(m_t - M) l_t.  Lane l works on head l/16 throughout.
template <int HPK>
__device__ __forceinline__ void qt_att_tiles(const uint16_t *qp, const uint16_t *kblk, uint16_t *pp, int pstride,
                                             float *ml, int w, int nk, float scale2, int lane) {
    const int r0[2] = {32 * w, 32 * w + 16};
    float sv[2];
    qt_att_qk2(qp, kblk, r0, lane, sv);                    // rows past nk: discarded
    const int h = lane >> 4, key = lane & 15;
    const float sa = r0[0] + key < nk ? sv[0] * scale2 : -INFINITY;
    const float sb = r0[1] + key < nk ? sv[1] * scale2 : -INFINITY;
    const float m = group_max<16>(fmaxf(sa, sb));         // finite: row 32w < nk
    const float pa = qt_exp2(sa - m), pb = qt_exp2(sb - m);     // 2^-inf == 0
    const float ls = group_sum<16>(pa + pb);
    if (h < HPK) {
        qt_put_pieces(pp + 4 * h * pstride + r0[0] + key, pstride, pa);
        qt_put_pieces(pp + 4 * h * pstride + r0[1] + key, pstride, pb);
        if (key == 0) { ml[(w * HPK + h) * 2] = m; ml[(w * HPK + h) * 2 + 1] = ls; }
    }
}

template <int HPK, int NKT>
__device__ __forceinline__ void qt_att_pv(const uint16_t *pp, int pstride, const float *ml, const uint16_t *vblk,
                                          int d0, int lane, float (&o)[2], float &M, float &l) {
    static_assert(NKT >= 1 && NKT <= 4, "one to four k-tiles");
    const int kg = lane >> 4, j = lane & 15, h = lane >> 4;
    const int hc = h < HPK ? h : HPK - 1;
    qt_u32x4 pa[4], vv[4][2];
    float mw[NKT], lw[NKT];
    // transposed value reads: lane (kg, j) points at k-tile rows 8kg + 4r2 + j/4, dims
    // col .. col+3; the k-tile offset 32t leaves the swizzle (row bits 0, 1, 3) unchanged
    int vb[2][2];
#pragma unroll
    for (int dt = 0; dt < 2; dt++)
#pragma unroll
        for (int r2 = 0; r2 < 2; r2++) vb[dt][r2] = qt_vidx(8 * kg + 4 * r2 + (j >> 2), d0 + 16 * dt + 4 * (j & 3));
#pragma unroll
    for (int t = 0; t < NKT; t++) {
        pa[t] = qt_lds16(pp + (lane & 15) * pstride + 32 * t + 8 * kg);
        mw[t] = ml[(t * HPK + hc) * 2];
        lw[t] = ml[(t * HPK + hc) * 2 + 1];
#pragma unroll
        for (int dt = 0; dt < 2; dt++)
            vv[t][dt] = qt_lds_tr8x2(vblk + vb[dt][0] + 32 * t * 128, vblk + vb[dt][1] + 32 * t * 128);
    }
    // one empty asm over every operand: all reads issued before it, one wait
    if constexpr (NKT == 1)
        asm volatile("" : "+v"(pa[0]), "+v"(vv[0][0]), "+v"(vv[0][1]));
    else if constexpr (NKT == 2)
        asm volatile("" : "+v"(pa[0]), "+v"(vv[0][0]), "+v"(vv[0][1]), "+v"(pa[1]), "+v"(vv[1][0]), "+v"(vv[1][1]));
    else if constexpr (NKT == 3)
        asm volatile("" : "+v"(pa[0]), "+v"(vv[0][0]), "+v"(vv[0][1]), "+v"(pa[1]), "+v"(vv[1][0]), "+v"(vv[1][1]),
                     "+v"(pa[2]), "+v"(vv[2][0]), "+v"(vv[2][1]));
    else
        asm volatile("" : "+v"(pa[0]), "+v"(vv[0][0]), "+v"(vv[0][1]), "+v"(pa[1]), "+v"(vv[1][0]), "+v"(vv[1][1]),
                     "+v"(pa[2]), "+v"(vv[2][0]), "+v"(vv[2][1]), "+v"(pa[3]), "+v"(vv[3][0]), "+v"(vv[3][1]));
    qt_f32x4 acc[NKT][2];
#pragma unroll
    for (int t = 0; t < NKT; t++)
#pragma unroll
        for (int dt = 0; dt < 2; dt++) acc[t][dt] = qt_mfma_bf16(pa[t], vv[t][dt], qt_f32x4{0.f, 0.f, 0.f, 0.f});
    M = mw[0];                                              // finite: k-tile 0 holds key 0
#pragma unroll
    for (int t = 1; t < NKT; t++) M = fmaxf(M, mw[t]);
    o[0] = o[1] = 0.f;
    l = 0.f;
#pragma unroll
    for (int t = 0; t < NKT; t++) {
        const float f = qt_exp2(mw[t] - M);
        l = fmaf(lw[t], f, l);
#pragma unroll
        for (int dt = 0; dt < 2; dt++) o[dt] = fmaf((acc[t][dt][0] + acc[t][dt][1]) + acc[t][dt][2], f, o[dt]);
    }
}
// step 2 for the block's k-tile count (uniform)
template <int HPK>
__device__ __forceinline__ void qt_att_pv_n(int nkt, const uint16_t *pp, int pstride, const float *ml,
                                            const uint16_t *vblk, int d0, int lane, float (&o)[2], float &M, float &l) {
    if (nkt <= 1) qt_att_pv<HPK, 1>(pp, pstride, ml, vblk, d0, lane, o, M, l);
    else if (nkt == 2) qt_att_pv<HPK, 2>(pp, pstride, ml, vblk, d0, lane, o, M, l);
    else if (nkt == 3) qt_att_pv<HPK, 3>(pp, pstride, ml, vblk, d0, lane, o, M, l);
    else qt_att_pv<HPK, 4>(pp, pstride, ml, vblk, d0, lane, o, M, l);
}

// Running (max, sum, output) across the blocks of a chunk longer than one block.
struct QtAttRun {
    float m, l, o[2];
};
__device__ __forceinline__ void qt_att_run_init(QtAttRun &r) { r.m = -INFINITY; r.l = 0.f; r.o[0] = r.o[1] = 0.f; }
__device__ __forceinline__ void qt_att_run_add(QtAttRun &r, const float (&o)[2], float M, float l) {
    const float mn = fmaxf(r.m, M);
    const float fr = qt_exp2(r.m - mn), fb = qt_exp2(M - mn);   // first block: fr = 0, fb = 1
    r.l = fmaf(r.l, fr, l * fb);
    r.o[0] = fmaf(r.o[0], fr, o[0] * fb);
    r.o[1] = fmaf(r.o[1], fr, o[1] * fb);
    r.m = mn;
}

// ---- one-pass chunks under the chunk maximum ------------------------------------------
// A chunk of up to 512 keys (k-tiles t = 0 .. ceil(n/32) - 1 of 32 keys; k-tile t =
// 4b + w belongs to wave w, block b) is one softmax with no running state:
//   1. every wave scores its k-tiles (two 16-key score tiles each, s' = s * scale * log2 e,
//      keys >= n at -inf) and takes its maximum per head, m_w;
//   2. M = max_w m_w (one workgroup barrier; a maximum is exact in any order);
//   3. p = 2^(s' - M) as pieces into the chunk's probability columns, l_w = sum over the
//      wave's k-tiles in block order of group_sum<16>(p_a + p_b);
//   4. (barrier) P.V: dims d0 .. d0 + 31 of every head, one accumulator per 16 dims,
//      chained over the k-tiles in order t = 0, 1, ..; o = (D0 + D1) + D2 (the pieces);
//      l = ((l_0 + l_1) + l_2) + l_3.
// Every float operation and its order is fixed by this list, so the per-kernel attention
// and the fused step, which stage keys differently, give the same bits.
//
// Step 3 for one k-tile of this wave: the pieces of p into rows 4h+p, columns col ..
// col + 31 of pp (row stride pstride), and the k-tile's sum of p per head.
template <int HPK>
__device__ __forceinline__ float qt_cm_probs(float sa, float sb, float M, uint16_t *pp, int pstride, int col, int lane) {
    const int h = lane >> 4, key = lane & 15;
    const float pa = qt_exp2(sa - M), pb = qt_exp2(sb - M);     // 2^-inf == 0
    if (h < HPK) {
        qt_put_pieces(pp + 4 * h * pstride + col + key, pstride, pa);
        qt_put_pieces(pp + 4 * h * pstride + col + 16 + key, pstride, pb);
    }
    return group_sum<16>(pa + pb);
}
// Step 4's operands for one k-tile: probability pieces of columns col .. col + 31 and the
// transposed value rows of the k-tile starting at vtile, dims d0 .. d0 + 31.
__device__ __forceinline__ void qt_cm_operands(const uint16_t *pp, int pstride, int col, const uint16_t *vtile, int d0,
                                               int lane, qt_u32x4 &pa, qt_u32x4 (&vv)[2]) {
    const int kg = lane >> 4, j = lane & 15;
    pa = qt_lds16(pp + (lane & 15) * pstride + col + 8 * kg);
#pragma unroll
    for (int dt = 0; dt < 2; dt++)
        vv[dt] = qt_lds_tr8x2(vtile + qt_vidx(8 * kg + j / 4, d0 + 16 * dt + 4 * (j & 3)),
                              vtile + qt_vidx(8 * kg + 4 + j / 4, d0 + 16 * dt + 4 * (j & 3)));
}
__device__ __forceinline__ void qt_cm_mfma(const qt_u32x4 &pa, const qt_u32x4 (&vv)[2], qt_f32x4 (&acc)[2]) {
    acc[0] = qt_mfma_bf16(pa, vv[0], acc[0]);
    acc[1] = qt_mfma_bf16(pa, vv[1], acc[1]);
}
