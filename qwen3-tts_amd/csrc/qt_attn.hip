// qt_attn.hip — single-query GQA attention over a bf16 KV cache (gfx950).
//
// Semantics of qwen_causal_attention_bf16kv (qwen_tts_kernels.c:3704-3846) for one
// query row: for head h (kv head g = h / HPK) over keys j < L,
//   s_j = (q . k_j) * scale,  o = sum_j softmax(s)_j v_j.
// Split-K (flash-decoding): grid (G chunks, n_kv).  Workgroup (c, g) takes keys
// [c*CH, c*CH+CH) with CH = roundup16(ceil(L/G)), so the grid is fixed while L grows
// (graph-replay safe) and every workgroup reads K/V of ONE kv head once for all HPK
// query heads that share it.  Per chunk it keeps (m, l, o[128]) per head; the last
// workgroup of a kv head to finish (device-scope counter) merges the chunks:
//   M = max m_c,  l = sum l_c e^(m_c-M),  o = sum o_c e^(m_c-M) / l.
//
// PREP (decode step) additionally does, from the raw QKV projection output:
//   per-head RMSNorm of q and k with the shared [128] gains (qwen_tts_kernels.c:486-577),
//   NeoX split-half RoPE from the uploaded cos/sin tables (qwen_tts_talker.c:203-251),
//   and the KV append at `pos` with f32->bf16 TRUNCATION (qwen_tts_talker.c:612-615),
//   done by the one workgroup whose chunk holds `pos`.
// Latency: the chunk's K and V rows (up to 128 keys) are copied into LDS with
// global_load_lds at kernel entry, before the q/k preparation, so one HBM round trip
// overlaps the prologue; the key at `pos` (appended by this workgroup) is not read from
// memory but taken from LDS (knew/vnew).  The merging workgroup reuses that LDS for the
// chunk partials, so a workgroup needs ~72 KB and two fit on a CU.
#include "qt_attn_mf.h"

#define QT_HD 128
#define QT_CH_MAX 256
#define QT_ATT_G 32

struct QtAttnArgs {
    const float *q;          // PREP: raw [q | k | v]; else rotated q rows (this query row)
    const float *qn, *kn;    // PREP: per-head gains
    const float *rc, *rs;    // PREP: rope tables [rope_len][64]
    float eps;
    const int *d_pos;        // PREP: device position; L = pos + 1
    int Lval;                // !PREP: number of keys
    uint16_t *K, *V;         // layer cache base
    long long pos_stride;    // elements between consecutive positions of one head
    long long head_stride;   // elements between kv heads
    int n_heads, n_kv;
    float scale;
    float *part;             // [n_kv][G][HPK][2 + 128]
    unsigned *cnt;           // [n_kv]
    float *out;              // [n_heads * 128]
    // independent streams (grid z): element offsets of stream z's q, K/V cache, output,
    // partials and counters; d_pos + z is its position (batched step)
    long long q_bs, kv_bs, out_bs, part_bs;
    int min_chunk;           // chunks hold at least this many keys (0: ceil(L/G) rounded to 16)
    int onepass;             // !BATCH, chunks <= 512 keys: one softmax over the chunk under its
                             // maximum (qt_attn_mf.h) instead of a running state across blocks
};

#define QT_KVB 128   // keys of a chunk staged in LDS at once

// The same copy issued from inline assembly: the compiler does not see it write LDS, so
// it inserts no vmcnt(0) before later LDS reads (it cannot tell the K copies from the V
// copies across the key loop); the caller waits for it with qt_wait_vm.  M0 holds the
// LDS address (wave-uniform), one wait state after it is written.
__device__ __forceinline__ void qt_lds_copy16_u(const void *src, void *dst) {
    const unsigned lds = (unsigned)(uintptr_t)(__attribute__((address_space(3))) void *)dst;
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}

// s_waitcnt on one counter only, as assembly with a memory clobber so that no LDS access
// moves across it
template <int N>
__device__ __forceinline__ void qt_wait_vm() {
    static_assert(N == 0 || N == 8, "vmcnt");
    if (N == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
__device__ __forceinline__ void qt_wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
#define QT_B_MIN_CHUNK 1536  // batched step: minimum keys per chunk

// 16 bytes per lane from global memory straight into LDS (global_load_lds_dwordx4):
// lane i's bytes land at dst + 16*i, dst wave-uniform.  Counted by vmcnt like a load.
__device__ __forceinline__ void qt_lds_copy16(const void *src, void *dst) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                     (__attribute__((address_space(3))) void *)dst, 16, 0, 0);
}

// BATCH (many streams, throughput): grid (n_kv, streams, G) so the workgroups of chunk 0
// of every stream and head are dispatched first and idle chunks last (a kv head per XCD
// under round-robin dispatch); the merging workgroup computes each output as one
// weighted sum over the chunks (one thread per output) instead of a half-wave reduction
// per output.  In a BATCH workgroup each wave streams its own 32-key tiles of the chunk
// (tiles w, w + 4, ...: its own block rows, its own copies, its own running softmax) with
// no workgroup barrier in the key loop, and the four wave states are merged at the end;
// !BATCH keeps the arithmetic order of the fused step's attention phase, which it must
// match bit for bit (waves share each 128-key block: scores, barrier, P.V per 32 dims).
template <int HPK, bool PREP, bool BATCH, bool ONEPASS>
__global__ __launch_bounds__(QT_WG) void k_attn(QtAttnArgs a) {
    static_assert(!(BATCH && ONEPASS), "one-pass chunks are single-stream");
    const int z = BATCH ? blockIdx.y : blockIdx.z;
    if (z) {
        a.q += z * a.q_bs; a.K += z * a.kv_bs; a.V += z * a.kv_bs; a.out += z * a.out_bs;
        a.part += z * a.part_bs; a.cnt += (size_t)z * a.n_kv; a.d_pos += z;
    }
    const int g = BATCH ? blockIdx.x : blockIdx.y, c = BATCH ? blockIdx.z : blockIdx.x;
    const int G = BATCH ? gridDim.z : gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pos = PREP ? *a.d_pos : a.Lval - 1;
    const int L = pos + 1;
    int CH = (L + G - 1) / G;
    CH = (CH + 15) & ~15;
    CH = max(CH, a.min_chunk);
    const int nch = (L + CH - 1) / CH;
    if (c >= nch) return;
    const int j0 = c * CH;
    const int n = min(CH, L - j0);
    const bool append = PREP && (pos >= j0 && pos < j0 + n);

    constexpr int PS = 2 + QT_HD;
    // keys staged per block (BATCH: wave w's 32-key tiles in block rows 32w .. 32w+31)
    constexpr int KVB = QT_KVB;
    constexpr int KVBYTES = 2 * KVB * QT_HD * 2, MBYTES = QT_ATT_G * HPK * PS * 4;
    static_assert(KVB % 32 == 0 && KVB <= QT_WAVES * 32, "each wave scores at most one 32-key tile of a block");
    __shared__ __align__(16) uint16_t qp[16][QT_HD];            // query pieces, row 4h+p (qt_attn_mf.h)
    // probability pieces of a block (k-tile w: wave w); ONEPASS: of the whole chunk
    constexpr int PPC = ONEPASS ? 4 * KVB : KVB;
    __shared__ __align__(16) uint16_t pp[16][PPC];
    __shared__ float ml[QT_WAVES][HPK][2];                      // per-k-tile (max, exp-sum)
    __shared__ __align__(16) uint16_t knew[QT_HD];
    __shared__ __align__(16) uint16_t vnew[QT_HD];
    // K rows and V rows of a key block, two LDS objects so that the compiler's wait for the
    // copies into one (global_load_lds, counted by vmcnt) leaves copies into the other in
    // flight; the V object is also the merge staging
    __shared__ __align__(16) uint16_t s_k[KVB * QT_HD];
    __shared__ __align__(16) uint16_t s_vbuf[(KVBYTES / 2 > MBYTES ? KVBYTES / 2 : MBYTES) / 2];
    uint16_t *const s_v = s_vbuf;
    __shared__ int last_flag;

    const uint16_t *Kg = a.K + (long long)g * a.head_stride;
    const uint16_t *Vg = a.V + (long long)g * a.head_stride;
    const int sub = lane & 15, pg = lane >> 4;

    // K and/or V rows of keys [kb, kb + min(KVB, n - kb)) of the chunk into s_k / s_v, in
    // the swizzled slot order of qt_attn_mf.h (lane (pg, sub) fills slot sub of block row
    // 4i + pg); the appended key (PREP) is not read from memory, it comes from knew/vnew.
    auto stage = [&](int kb, bool doK, bool doV) {
        const int nk = min(KVB, n - kb);
        const int ninst = (nk + 3) >> 2;
        for (int i = wave; i < ninst; i += QT_WAVES) {
            const int jl = i * 4 + pg, jj = kb + jl;
            if (jj < n && !(PREP && j0 + jj == pos)) {
                const long long row = (long long)(j0 + jj) * a.pos_stride;
                if (doK) qt_lds_copy16(Kg + row + qt_kslot(jl, sub) * 8, &s_k[i * 4 * QT_HD]);
                if (doV) qt_lds_copy16(Vg + row + qt_vslot(jl, sub) * 8, &s_v[i * 4 * QT_HD]);
            }
        }
    };
    // BATCH: the K (doK) or V rows of 32-key tile tix of the chunk (keys 32 tix .. +31) into
    // this wave's block rows 32w .. 32w+31 (same swizzle: it depends on the row's low bits
    // only), eight 1-KiB copies.  Every lane issues all eight, so the wave's vmcnt counts
    // eight per staging: rows past the chunk copy its last row (their scores are masked and
    // their value rows zeroed), and the appended key's row is copied too and then
    // overwritten from knew / vnew once the copy has landed.
    auto stage_w = [&](int tix, bool doK) {
        const int kb = 32 * tix;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int jl = i * 4 + pg;
            const long long row = (long long)(j0 + min(kb + jl, n - 1)) * a.pos_stride;
            if (doK) qt_lds_copy16_u(Kg + row + qt_kslot(jl, sub) * 8, &s_k[(32 * wave + i * 4) * QT_HD]);
            else qt_lds_copy16_u(Vg + row + qt_vslot(jl, sub) * 8, &s_v[(32 * wave + i * 4) * QT_HD]);
        }
    };
    // LDS written by global_load_lds is counted by vmcnt, and a workgroup barrier does
    // not wait for it: every staging is followed by an explicit full wait before the
    // barrier that publishes the block to the other waves.
    // ---- 0. K/V of the first key block (BATCH: each wave's first tile) in flight first ----
    if (BATCH) {
        if (32 * wave < n) { stage_w(wave, true); stage_w(wave, false); }
    } else {
        stage(0, true, true);
    }

    // ---- 1. query heads (and the new key/value) ----
    if (PREP) {
        const int ntask = HPK + (append ? 1 : 0);
        for (int t = wave; t < ntask; t += QT_WAVES) {
            const bool isk = (t == HPK);
            const float *src = isk ? a.q + a.n_heads * QT_HD + g * QT_HD
                                   : a.q + (g * HPK + t) * QT_HD;
            const float *w = isk ? a.kn : a.qn;
            float x0 = src[lane], x1 = src[lane + 64];
            float ss = group_sum<64>(x0 * x0 + x1 * x1);
            float inv = 1.0f / sqrtf(ss / (float)QT_HD + a.eps);
            float n0 = (x0 * inv) * w[lane], n1 = (x1 * inv) * w[lane + 64];
            float cs = a.rc[(size_t)pos * 64 + lane], sn = a.rs[(size_t)pos * 64 + lane];
            float r0 = fmaf(n0, cs, -(n1 * sn));
            float r1 = fmaf(n1, cs, n0 * sn);
            if (!isk) {
                qt_put_pieces(&qp[4 * t][lane], QT_HD, r0);
                qt_put_pieces(&qp[4 * t][lane + 64], QT_HD, r1);
            } else {
                const float *vs = a.q + a.n_heads * QT_HD + a.n_kv * QT_HD + g * QT_HD;
                const uint16_t k0 = f2bf_trunc(r0), k1 = f2bf_trunc(r1);
                const uint16_t v0 = f2bf_trunc(vs[lane]), v1 = f2bf_trunc(vs[lane + 64]);
                uint16_t *kd = a.K + (long long)g * a.head_stride + (long long)pos * a.pos_stride;
                uint16_t *vd = a.V + (long long)g * a.head_stride + (long long)pos * a.pos_stride;
                kd[lane] = k0; kd[lane + 64] = k1;
                vd[lane] = v0; vd[lane + 64] = v1;
                knew[lane] = k0; knew[lane + 64] = k1;
                vnew[lane] = v0; vnew[lane + 64] = v1;
                const int r = pos - j0;            // its row in the first staged block
                if (!BATCH && r < KVB) {
                    s_k[qt_kidx(r, lane)] = k0; s_k[qt_kidx(r, lane + 64)] = k1;
                    s_v[qt_vidx(r, lane)] = v0; s_v[qt_vidx(r, lane + 64)] = v1;
                }
            }
        }
    } else {
        for (int i = tid; i < HPK * QT_HD; i += QT_WG)
            qt_put_pieces(&qp[4 * (i / QT_HD)][i % QT_HD], QT_HD, a.q[(g * HPK + i / QT_HD) * QT_HD + i % QT_HD]);
    }
    qt_att_zero_rows<HPK>(&qp[0][0], QT_HD, tid, QT_WG);
    qt_att_zero_rows<HPK>(&pp[0][0], PPC, tid, QT_WG);
    if (!BATCH) qt_att_zero_vrows(s_v, min(KVB, n), (min(KVB, n) + 31) & ~31, tid, QT_WG);
    if (!BATCH) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();   // (also, !BATCH: every wave's LDS copies of the first block have landed)

    // ---- 2. per block (qt_attn_mf.h): wave w scores its k-tile (block rows 32w .. +31),
    // barrier, then takes dims [32w, 32w + 32) of P.V over the k-tiles holding keys ----
    const float scale2 = a.scale * QT_LOG2E;
    QtAttRun run;
    qt_att_run_init(run);
    if constexpr (BATCH) {
        // ---- 2b. each wave streams its own 32-key tiles (tix = w, w + 4, ...) with no
        // workgroup barrier: wait for the tile's keys, put the appended key, score
        // (qt_att_tiles on k-tile w), then the next tile's keys go in flight while this
        // tile's values are waited for (the appended value put, the value rows past the
        // chunk zeroed) and P.V runs over all 128 dims of the k-tile (four 32-dim slices);
        // then the next tile's values go in flight and the tile folds into the wave's
        // running (m, l, o).  vmcnt counts eight per staging (stage_w), in issue order. ----
        float wm = -INFINITY, wl = 0.f, wo[4][2];
#pragma unroll
        for (int sl = 0; sl < 4; sl++) wo[sl][0] = wo[sl][1] = 0.f;
        const int ntile = (n + 31) >> 5;
        __builtin_amdgcn_s_waitcnt(0);                // the first tile (and phase 1's stores)
        for (int tix = wave; tix < ntile; tix += QT_WAVES) {
            const int kb = 32 * tix, nk = min(32, n - kb), row = 32 * wave + (pos - j0 - kb);
            const bool more = tix + QT_WAVES < ntile, put = PREP && pos - j0 - kb >= 0 && pos - j0 - kb < nk;
            qt_wait_vm<8>();                          // keys of tile tix (its values may be in flight)
            if (put && lane < 16)
                *reinterpret_cast<uint4 *>(s_k + row * QT_HD + qt_kslot(row, lane) * 8) =
                    *reinterpret_cast<const uint4 *>(knew + 8 * lane);
            qt_att_tiles<HPK>(&qp[0][0], s_k, &pp[0][0], KVB, &ml[0][0][0], wave, 32 * wave + nk, scale2, lane);
            qt_wait_lgkm0();                          // every LDS read of the keys has returned
            if (more) { stage_w(tix + QT_WAVES, true); qt_wait_vm<8>(); }
            else qt_wait_vm<0>();                     // values of tile tix
            if (put && lane < 16)
                *reinterpret_cast<uint4 *>(s_v + row * QT_HD + qt_vslot(row, lane) * 8) =
                    *reinterpret_cast<const uint4 *>(vnew + 8 * lane);
            if (nk < 32) qt_att_zero_vrows(s_v + 32 * wave * QT_HD, nk, 32, lane, 64);
            float to[4][2], tM = 0.f, tl = 0.f;
#pragma unroll
            for (int sl = 0; sl < 4; sl++)
                qt_att_pv<HPK, 1>(&pp[0][0] + 32 * wave, KVB, &ml[wave][0][0], s_v + 32 * wave * QT_HD, 32 * sl, lane,
                                  to[sl], tM, tl);
            qt_wait_lgkm0();                          // every LDS read of the values has returned
            if (more) stage_w(tix + QT_WAVES, false);
            const float mn = fmaxf(wm, tM);
            const float fr = qt_exp2(wm - mn), fb = qt_exp2(tM - mn);   // first tile: fr = 0, fb = 1
            wl = fmaf(wl, fr, tl * fb);
#pragma unroll
            for (int sl = 0; sl < 4; sl++) {
                wo[sl][0] = fmaf(wo[sl][0], fr, to[sl][0] * fb);
                wo[sl][1] = fmaf(wo[sl][1], fr, to[sl][1] * fb);
            }
            wm = mn;
        }
        // ---- merge the four waves' states, waves in order, into the per-lane form of
        // the epilogue (head pg, dims 32 wave + sub and + 16) ----
        __syncthreads();                              // every wave is done with s_k and s_v
        float *ws = reinterpret_cast<float *>(s_vbuf);  // [wave][lane][10]: m, l, o[4][2]
        {
            float *me = ws + (wave * 64 + lane) * 10;
            me[0] = wm; me[1] = wl;
#pragma unroll
            for (int sl = 0; sl < 4; sl++) { me[2 + 2 * sl] = wo[sl][0]; me[3 + 2 * sl] = wo[sl][1]; }
        }
        __syncthreads();
#pragma unroll
        for (int w2 = 0; w2 < QT_WAVES; w2++) {
            const float *src = ws + (w2 * 64 + lane) * 10;   // same lane: same head pg, same sub
            const float o2[2] = {src[2 + 2 * wave], src[3 + 2 * wave]};
            if (src[0] != -INFINITY) qt_att_run_add(run, o2, src[0], src[1]);
        }
    } else if constexpr (ONEPASS) {
        // ---- 2c. one pass under the chunk maximum (qt_attn_mf.h), the arithmetic of the
        // fused role-specialised step (qt_rstep.hip): the K blocks staged in turn and
        // scored into registers, the chunk maximum, the probabilities, then the V blocks in
        // turn for P.V (block 0's values were staged with its keys) ----
        constexpr int NB1 = 4;                    // 128-key blocks (chunks <= 512 keys)
        const int nblk = (n + KVB - 1) / KVB;
        const int hc = pg < HPK ? pg : HPK - 1;
        float sv[NB1][2];
        float wm = -INFINITY;
#pragma unroll
        for (int b = 0; b < NB1; b++) {
            sv[b][0] = sv[b][1] = -INFINITY;
            if (b >= nblk) continue;
            const int kb = KVB * b, nk = min(KVB, n - kb);
            if (b > 0) {
                __syncthreads();                  // every wave is done with the previous keys
                stage(kb, true, false);
                __builtin_amdgcn_s_waitcnt(0);
                const int nrow = pos - j0 - kb;
                if (PREP && wave == 0 && nrow >= 0 && nrow < nk && lane < 16)
                    *reinterpret_cast<uint4 *>(&s_k[nrow * QT_HD + qt_kslot(nrow, lane) * 8]) =
                        *reinterpret_cast<const uint4 *>(knew + 8 * lane);
                __syncthreads();
            }
            if (kb + 32 * wave < n) {
                const int rr[2] = {32 * wave, 32 * wave + 16};
                float sc[2];
                qt_att_qk2(&qp[0][0], s_k, rr, lane, sc);
                sv[b][0] = rr[0] + sub < nk ? sc[0] * scale2 : -INFINITY;
                sv[b][1] = rr[1] + sub < nk ? sc[1] * scale2 : -INFINITY;
                wm = fmaxf(wm, group_max<16>(fmaxf(sv[b][0], sv[b][1])));
            }
        }
        if (pg < HPK && sub == 0) ml[wave][pg][0] = wm;
        __syncthreads();
        const float M = fmaxf(fmaxf(ml[0][hc][0], ml[1][hc][0]), fmaxf(ml[2][hc][0], ml[3][hc][0]));
        float lw = 0.f;
#pragma unroll
        for (int b = 0; b < NB1; b++)
            if (b < nblk && KVB * b + 32 * wave < n)
                lw += qt_cm_probs<HPK>(sv[b][0], sv[b][1], M, &pp[0][0], PPC, KVB * b + 32 * wave, lane);
        if (pg < HPK && sub == 0) ml[wave][pg][1] = lw;
        __syncthreads();
        const int nt = (n + 31) >> 5;
        qt_f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        for (int b = 0; b < nblk; b++) {
            const int kb = KVB * b, nk = min(KVB, n - kb);
            if (b > 0) {
                __syncthreads();                  // every wave is done with the previous values
                stage(kb, false, true);
                __builtin_amdgcn_s_waitcnt(0);
                const int nrow = pos - j0 - kb;
                if (PREP && wave == 0 && nrow >= 0 && nrow < nk && lane < 16)
                    *reinterpret_cast<uint4 *>(&s_v[nrow * QT_HD + qt_vslot(nrow, lane) * 8]) =
                        *reinterpret_cast<const uint4 *>(vnew + 8 * lane);
                qt_att_zero_vrows(s_v, nk, (nk + 31) & ~31, tid, QT_WG);
                __syncthreads();
            }
#pragma unroll
            for (int t = 0; t < 4; t++) {
                if (4 * b + t >= nt) break;
                qt_u32x4 pa, vv[2];
                qt_cm_operands(&pp[0][0], PPC, kb + 32 * t, s_v + 32 * t * QT_HD, 32 * wave, lane, pa, vv);
                qt_cm_mfma(pa, vv, acc);
            }
        }
#pragma unroll
        for (int dt = 0; dt < 2; dt++) run.o[dt] = (acc[dt][0] + acc[dt][1]) + acc[dt][2];
        run.m = M;
        run.l = ((ml[0][hc][1] + ml[1][hc][1]) + ml[2][hc][1]) + ml[3][hc][1];
    } else
    for (int kb = 0; kb < n; kb += KVB) {
        const int nk = min(KVB, n - kb);
        if (kb > 0) {   // chunks longer than one block (caches beyond G*KVB keys)
            __syncthreads();
            stage(kb, true, true);
            __builtin_amdgcn_s_waitcnt(0);
            const int nrow = pos - j0 - kb;   // the appended key's row, if in this block
            if (PREP && wave == 0 && nrow >= 0 && nrow < nk) qt_att_put_kv(s_k, s_v, nrow, knew, vnew, lane);
            qt_att_zero_vrows(s_v, nk, (nk + 31) & ~31, tid, QT_WG);
            __syncthreads();
        }
        if (32 * wave < nk)
            qt_att_tiles<HPK>(&qp[0][0], s_k, &pp[0][0], KVB, &ml[0][0][0], wave, nk, scale2, lane);
        __syncthreads();
        float o[2], M, l;
        qt_att_pv_n<HPK>((nk + 31) >> 5, &pp[0][0], KVB, &ml[0][0][0], s_v, 32 * wave, lane, o, M, l);
        qt_att_run_add(run, o, M, l);
    }
    // lane: head pg, dims 32*wave + sub and + 16
    const int od = 32 * wave + sub;

    // ---- 3. write (single chunk) or publish partial and merge in the last workgroup ----
    if (nch == 1) {
        if (pg < HPK) {
            const float r = 1.0f / run.l;
            a.out[(g * HPK + pg) * QT_HD + od] = run.o[0] * r;
            a.out[(g * HPK + pg) * QT_HD + od + 16] = run.o[1] * r;
        }
        return;
    }
    // Publish the partial with agent-scope (L2-bypassing) stores, wait for them to be
    // acknowledged, then count arrivals with a relaxed device-scope atomic.  This avoids
    // __threadfence(), whose L2 write-back + invalidate on every XCD costs ~17 us for a
    // 256-workgroup grid on MI355X; the merging workgroup reads with agent-scope loads.
    float *mypart = a.part + ((size_t)(g * G + c) * HPK) * PS;
    if (pg < HPK) {
        st_agent(mypart + pg * PS + 2 + od, run.o[0]);
        st_agent(mypart + pg * PS + 2 + od + 16, run.o[1]);
        if (wave == 0 && sub == 0) { st_agent(mypart + pg * PS, run.m); st_agent(mypart + pg * PS + 1, run.l); }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
        last_flag = (__hip_atomic_fetch_add(&a.cnt[g], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                     (unsigned)(nch - 1));
    __syncthreads();
    if (!last_flag) return;
    // Merge: all chunk partials into LDS (the K/V buffer, free now) with one parallel
    // load round, then each half-wave merges one (head, dim) output over the chunks
    // (softmax_merge32, lane = chunk).
    float *mpart = reinterpret_cast<float *>(s_vbuf);
    const float *gp = a.part + (size_t)g * G * HPK * PS;
    {
        // all loads issued before any is consumed (one round trip, not one per element)
        constexpr int MK = (QT_ATT_G * HPK * PS + QT_WG - 1) / QT_WG;
        const int np = nch * HPK * PS;
        float t[MK];
#pragma unroll
        for (int k = 0; k < MK; k++) t[k] = (tid + k * QT_WG < np) ? ld_agent(gp + tid + k * QT_WG) : 0.f;
#pragma unroll
        for (int k = 0; k < MK; k++)
            if (tid + k * QT_WG < np) mpart[tid + k * QT_WG] = t[k];
    }
    __syncthreads();
    if (BATCH) {
        // one output (head h, dim d) per thread: M = max_c m_c, f_c = e^(m_c - M),
        // out = sum_c o_c[d] f_c / sum_c l_c f_c, chunks in order
        for (int i = tid; i < HPK * QT_HD; i += QT_WG) {
            const int h = i / QT_HD, d = i % QT_HD;
            float M = -INFINITY;
            for (int cc = 0; cc < nch; cc++) M = fmaxf(M, mpart[(cc * HPK + h) * PS]);
            float Lsum = 0.f, V = 0.f;
            for (int cc = 0; cc < nch; cc++) {
                const float *pr = mpart + (size_t)(cc * HPK + h) * PS;
                const float f = qt_exp2(pr[0] - M);
                Lsum = fmaf(pr[1], f, Lsum);
                V = fmaf(pr[2 + d], f, V);
            }
            a.out[(g * HPK + h) * QT_HD + d] = V * (1.0f / Lsum);
        }
    } else {
        const int half = lane >> 5, cc = lane & 31;
        const bool valid = cc < nch;
        for (int i = wave * 2 + half; i < HPK * QT_HD; i += QT_WAVES * 2) {
            const int h = i / QT_HD, d = i % QT_HD;
            const float *pr = mpart + (size_t)(cc * HPK + h) * PS;
            const float r = softmax_merge32(valid ? pr[0] : 0.f, valid ? pr[1] : 0.f, valid ? pr[2 + d] : 0.f, valid);
            if (cc == 0) a.out[(g * HPK + h) * QT_HD + d] = r;
        }
    }
    if (tid == 0) __hip_atomic_store(&a.cnt[g], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

static hipError_t attn_launch(const QtAttnArgs &a, int prep, int head_dim, int G, int nz, hipStream_t st) {
    if (head_dim != QT_HD || a.n_kv <= 0 || a.n_heads % a.n_kv) return hipErrorInvalidValue;
    if (G <= 0 || G > QT_ATT_G || nz <= 0 || nz > 65535) return hipErrorInvalidValue;
    if (!prep && (a.Lval <= 0 || a.Lval > G * QT_CH_MAX)) return hipErrorInvalidValue;
    if (a.onepass && a.min_chunk > 0) return hipErrorInvalidValue;
    const int hpk = a.n_heads / a.n_kv;
    const bool batch = a.min_chunk > 0;
    const dim3 grid = batch ? dim3(a.n_kv, nz, G) : dim3(G, a.n_kv, nz);
#define QT_ATT_CASE(H) \
    if (batch && prep) hipLaunchKernelGGL((k_attn<H, true, true, false>), grid, dim3(QT_WG), 0, st, a); \
    else if (a.onepass && prep) hipLaunchKernelGGL((k_attn<H, true, false, true>), grid, dim3(QT_WG), 0, st, a); \
    else if (a.onepass) hipLaunchKernelGGL((k_attn<H, false, false, true>), grid, dim3(QT_WG), 0, st, a); \
    else if (prep) hipLaunchKernelGGL((k_attn<H, true, false, false>), grid, dim3(QT_WG), 0, st, a); \
    else hipLaunchKernelGGL((k_attn<H, false, false, false>), grid, dim3(QT_WG), 0, st, a);
    if (hpk == 1) { QT_ATT_CASE(1) }
    else if (hpk == 2) { QT_ATT_CASE(2) }
    else if (hpk == 4) { QT_ATT_CASE(4) }
    else return hipErrorInvalidValue;
#undef QT_ATT_CASE
    return hipGetLastError();
}

extern "C" hipError_t qt_launch_attn(int prep, const float *q, const float *qn, const float *kn,
                                     const float *rc, const float *rs, float eps, const int *d_pos,
                                     int Lval, uint16_t *K, uint16_t *V, long long pos_stride,
                                     long long head_stride, int n_heads, int n_kv, int head_dim,
                                     float scale, float *part, unsigned *cnt, int G, float *out,
                                     hipStream_t st) {
    QtAttnArgs a;
    a.q = q; a.qn = qn; a.kn = kn; a.rc = rc; a.rs = rs; a.eps = eps; a.d_pos = d_pos; a.Lval = Lval;
    a.K = K; a.V = V; a.pos_stride = pos_stride; a.head_stride = head_stride;
    a.n_heads = n_heads; a.n_kv = n_kv; a.scale = scale; a.part = part; a.cnt = cnt; a.out = out;
    a.q_bs = a.kv_bs = a.out_bs = a.part_bs = 0;
    a.min_chunk = 0;
    a.onepass = 0;
    return attn_launch(a, prep, head_dim, G, 1, st);
}

// The same with each chunk as one softmax over its keys (chunks of at most 512 keys:
// G * 512 >= the cache length): the arithmetic of the role-specialised fused step.
extern "C" hipError_t qt_launch_attn_onepass(int prep, const float *q, const float *qn, const float *kn,
                                             const float *rc, const float *rs, float eps, const int *d_pos,
                                             int Lval, uint16_t *K, uint16_t *V, long long pos_stride,
                                             long long head_stride, int n_heads, int n_kv, int head_dim,
                                             float scale, float *part, unsigned *cnt, int G, float *out,
                                             hipStream_t st) {
    QtAttnArgs a;
    a.q = q; a.qn = qn; a.kn = kn; a.rc = rc; a.rs = rs; a.eps = eps; a.d_pos = d_pos; a.Lval = Lval;
    a.K = K; a.V = V; a.pos_stride = pos_stride; a.head_stride = head_stride;
    a.n_heads = n_heads; a.n_kv = n_kv; a.scale = scale; a.part = part; a.cnt = cnt; a.out = out;
    a.q_bs = a.kv_bs = a.out_bs = a.part_bs = 0;
    a.min_chunk = 0;
    a.onepass = 1;
    return attn_launch(a, prep, head_dim, G, 1, st);
}

// B independent streams in one launch (the batched step): stream z uses q + z*q_bs,
// K/V + z*kv_bs (its own cache), position d_pos[z], partials part + z*part_bs, counters
// cnt + z*n_kv, output out + z*out_bs.  Ragged positions are fine: each stream's chunks
// follow its own length.  Chunks hold at least QT_B_MIN_CHUNK keys: short streams use few
// workgroups, fewer partials are merged, and each wave streams a dozen tiles; throughput,
// not single-stream latency, is what the batch needs.  Measured on the whole batched step
// (32 ragged streams of 128..4096 keys, 1.7B int8, MI355X), wave-streamed tiles with a
// minimum of 256 / 384 / 768 / 1536 / 2048 / 3072 / 4096 keys: 3.30 / 3.20 / 3.17 / 3.08 /
// 3.20 / 3.41 / 3.59 ms/step.  Shared 128-key blocks (scores, barrier, P.V) had given 3.76 /
// 3.49 / 3.43 / 3.58 at 128 / 256 / 512 / 1024, and shared 64-key blocks (four workgroups
// per CU) 3.16 / 3.13 / 3.13 / 3.22 / 3.24 / 3.20 / 3.28 at 256 / 320 / 384 / 448 / 512 /
// 768 / 1024.
extern "C" hipError_t qt_launch_attn_b(const float *q, long long q_bs, const float *qn, const float *kn,
                                       const float *rc, const float *rs, float eps, const int *d_pos,
                                       uint16_t *K, uint16_t *V, long long kv_bs, long long pos_stride,
                                       long long head_stride, int n_heads, int n_kv, int head_dim, float scale,
                                       float *part, long long part_bs, unsigned *cnt, int G, float *out,
                                       long long out_bs, int B, hipStream_t st) {
    QtAttnArgs a;
    a.q = q; a.qn = qn; a.kn = kn; a.rc = rc; a.rs = rs; a.eps = eps; a.d_pos = d_pos; a.Lval = 0;
    a.K = K; a.V = V; a.pos_stride = pos_stride; a.head_stride = head_stride;
    a.n_heads = n_heads; a.n_kv = n_kv; a.scale = scale; a.part = part; a.cnt = cnt; a.out = out;
    a.q_bs = q_bs; a.kv_bs = kv_bs; a.out_bs = out_bs; a.part_bs = part_bs;
    a.min_chunk = QT_B_MIN_CHUNK;
    a.onepass = 0;
    return attn_launch(a, 1, head_dim, G, B, st);
}

// Split-K grid: QT_ATT_G chunks per kv head (256 workgroups for 8 kv heads); a chunk
// holds at most QT_CH_MAX keys, so the grid serves caches up to 8192 positions.
// Returns -1 when max_len does not fit.
extern "C" int qt_attn_grid(int max_len) {
    return max_len <= QT_ATT_G * QT_CH_MAX ? QT_ATT_G : -1;
}
