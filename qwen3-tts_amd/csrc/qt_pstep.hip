// qt_pstep.hip — the whole Talker decode step (optionally many greedy steps) as ONE
// persistent cooperative kernel for gfx950.
//
// Why: a decode step is ~141 dependent phases (5 per layer x 28 + head).  As separate
// kernels each phase costs at least the ~2.4 us launch cycle, which alone exceeds the
// HBM time of the step (1.65 GB at 8 TB/s = 206 us).  Here 256 workgroups (one per CU,
// co-resident by cooperative launch) run all phases and meet at device-wide barriers
// (~1.8 us), and every workgroup issues the NEXT phase's weight loads into registers
// before it waits at the barrier, so HBM streaming overlaps the synchronisation.
//
// Phases of layer l (same math as qwen_tts_talker.c:580-690, kernels in qt_matvec.hip /
// qt_attn.hip):
//   A  q|k|v = W_qkv . RMSNorm(x)                  16 rows per workgroup
//   B  attention item (kv head g, chunk c), 8 x 32 items, one per workgroup: q/k norm,
//      RoPE, KV append (bf16 truncation), split-K partial; the last item of each kv
//      head merges the 32 partials
//   C  xa = x + W_o . attn                          H/256 rows per workgroup
//   D  h = SwiGLU(W_gu . RMSNorm(xa))               2F/256 rows per workgroup
//   E  xb = xa + W_dn . h                           H/256 rows per workgroup
// and per greedy step the codec head (RMSNorm(xb) with the final norm, 12 rows per
// workgroup, masked local argmax) and a global argmax over the 256 local winners.
//
// Memory coherence across XCDs without L2 write-back/invalidate:
//   * every activation is written once per (step parity, layer, phase) into its own
//     slot of an activation ring, with agent-scope (sc1, write-through) stores, so no
//     L2 can hold a stale copy of an address when it is first read in this launch;
//     reads are ordinary vector loads;
//   * a phase's stores are acknowledged (s_waitcnt vmcnt(0)) before its workgroup
//     arrives at the barrier; the barrier itself is agent-scope relaxed atomics;
//   * at the start of each additional step of a multi-step launch every workgroup
//     invalidates its L1/L2 (acquire fence) because the ring parities repeat.
// Every spin-wait is bounded: on timeout the kernel records an error and all
// workgroups run to the end, so a launch always terminates.
#include "qt_device.h"

namespace ps {
constexpr int NB = 256;          // workgroups (one per CU)
constexpr int NW = 4;            // waves per workgroup
constexpr int HD = 128, NH = 16, NKV = 8, HPK = 2, QD = NH * HD, KVD = NKV * HD, QKVR = QD + 2 * KVD;
constexpr int G = 32;            // attention chunks per kv head: NKV * G == NB items
constexpr int CHMAX = 256;       // keys per chunk at most (kv_max <= G * CHMAX)
constexpr int GS = 16;           // barrier: workgroups per first-level counter
constexpr int NGRP = NB / GS;
constexpr unsigned SPIN_LIMIT = 1u << 22;
constexpr int BAR_BLOCK = 1024;  // unsigned words per barrier counter block

struct Layer {
    const uint8_t *w[4];          // qkv, o, gate_up, down (device encodings, qt_device.h)
    const float *s[4];            // int8 row scales
    const uint16_t *s16[4];       // q4 block scales
    const float *in_norm, *post_norm, *qn, *kn;
};

struct Args {
    const Layer *layers;
    int n_layers;
    const float *final_norm, *rope_cos, *rope_sin;
    uint16_t *kc, *vc;            // [L][NKV][kv_max][HD]
    int kv_max;
    float eps, scale;
    float *ring;                  // [2][L][per-layer block] + x_in[2][H]
    float *part;                  // [NKV][G][HPK][2+HD]
    unsigned *cnt;                // [NKV] merge counters (self-resetting)
    float *hid;                   // [H] final normed hidden of the last step
    float *xin;                   // [H] step-0 input (host embed)
    int *d_pos;                   // position of step 0; advanced by n_steps
    unsigned *bar;                // [2][BAR_BLOCK] counter blocks + [2*BAR_BLOCK] launch index
    int *err;
    int n_steps;
    // greedy head (with_head != 0)
    int with_head;
    const uint8_t *head_w;        // bf16 [vocab][H]
    const uint16_t *emb;          // bf16 [vocab][H]
    int vocab;
    float *slots;                 // [NB][2] local winners (value, index)
    int *d_frame, *hist;
    int hist_len;
};

__device__ __forceinline__ unsigned ld_u(const unsigned *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_u(unsigned *p, unsigned v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ unsigned add_u(unsigned *p, unsigned v) { return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_i(int *p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ int ld_i(const int *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// Optional phase trace (build with -DQT_PSTEP_TRACE): s_memrealtime (100 MHz) of every
// workgroup when it has finished a phase (w=0) and when it leaves the barrier (w=1),
// indexed by the barrier's number in the launch; qt_pstep_trace_read copies it out.
#ifdef QT_PSTEP_TRACE
constexpr int TRACE_BARS = 1024;
__device__ unsigned long long ps_trace[TRACE_BARS * 2 * NB];
#define PS_MARK(k, w)                                                                        \
    do {                                                                                     \
        if (threadIdx.x == 0 && (k) < (unsigned)TRACE_BARS)                                  \
            ps_trace[((size_t)(k) * 2 + (w)) * NB + blockIdx.x] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define PS_MARK(k, w) do { } while (0)
#endif

// ---- device-wide barrier: two-level counter tree, monotonic within a launch ----------
struct Bar {
    unsigned *blk;   // this launch's counter block: [0] release, [32] top, [64+32g] groups
    unsigned k;      // barriers completed in this launch
    int *err;
};

// All threads: make this workgroup's stores visible, then thread 0 arrives.
__device__ __forceinline__ void bar_arrive(Bar &b) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    PS_MARK(b.k, 0);
    if (threadIdx.x == 0) {
        const unsigned t = b.k + 1;
        unsigned *gc = b.blk + 64 + 32 * (blockIdx.x / GS);
        if (add_u(gc, 1u) == t * GS - 1) {
            if (add_u(b.blk + 32, 1u) == t * NGRP - 1) st_u(b.blk, t);
        }
    }
}
// Thread 0 spins until every workgroup arrived (bounded), then the workgroup proceeds.
__device__ __forceinline__ void bar_wait(Bar &b) {
    const unsigned t = b.k + 1;
    if (threadIdx.x == 0) {
        unsigned it = 0;
        while (ld_u(b.blk) < t) {
            if (++it > SPIN_LIMIT) { st_i(b.err, 1); break; }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
    PS_MARK(b.k, 1);
    b.k = t;
}

// ---- weight tiles -----------------------------------------------------------------------
template <int PREC> struct Epc;
template <> struct Epc<QT_BF16> { static constexpr int v = 8; };
template <> struct Epc<QT_INT8> { static constexpr int v = 16; };
template <> struct Epc<QT_Q4> { static constexpr int v = 32; };

// RPW rows per wave of a [rows][COLS] matrix, lanes split every row's 16-byte chunks.
template <int PREC, int COLS, int RPW>
struct Tile {
    static constexpr int EPC = Epc<PREC>::v;
    static constexpr int LPR = (COLS / EPC >= 64) ? 64 : 32;
    static constexpr int CPL = COLS / (EPC * LPR);
    static constexpr int NR = RPW / (64 / LPR);
    static constexpr size_t RB = PREC == QT_BF16 ? (size_t)COLS * 2 : PREC == QT_INT8 ? (size_t)COLS : (size_t)COLS / 2;
    static_assert(CPL >= 1 && NR >= 1 && NR * (64 / LPR) == RPW, "tile shape");
    uint4 w[NR][CPL];
    float s[NR][CPL];

    // rows of this lane's group: row0w + grp*NR + r, row0w = first row of the wave
    __device__ __forceinline__ void load(const uint8_t *W, const uint16_t *S16, int row0w) {
        const int lane = threadIdx.x & 63, grp = lane / LPR, sub = lane % LPR;
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const int row = row0w + grp * NR + r;
#pragma unroll
            for (int j = 0; j < CPL; j++) {
                const int c = sub + LPR * j;
                w[r][j] = *reinterpret_cast<const uint4 *>(W + (size_t)row * RB + (size_t)c * 16);
                if (PREC == QT_Q4) s[r][j] = ref_f16_to_f32(S16[(size_t)row * (COLS / 32) + c]);
            }
        }
    }
};

// The activation slice a lane's chunks multiply, in element order, optionally
// RMS-normalised (group reduction over LPR lanes, which together cover the vector).
template <int PREC, int COLS>
struct Slice {
    static constexpr int EPC = Epc<PREC>::v;
    static constexpr int LPR = (COLS / EPC >= 64) ? 64 : 32;
    static constexpr int CPL = COLS / (EPC * LPR);
    float x[CPL][EPC];
    float xsum[CPL];

    __device__ __forceinline__ void load(const float *v) {
        const int sub = (threadIdx.x & 63) % LPR;
#pragma unroll
        for (int j = 0; j < CPL; j++)
#pragma unroll
            for (int q = 0; q < EPC / 4; q++) {
                const float4 t = *reinterpret_cast<const float4 *>(v + (sub + LPR * j) * EPC + 4 * q);
                x[j][4 * q] = t.x; x[j][4 * q + 1] = t.y; x[j][4 * q + 2] = t.z; x[j][4 * q + 3] = t.w;
            }
    }
    // bf16 source (embedding row) -> f32
    __device__ __forceinline__ void load_bf16(const uint16_t *v) {
        const int sub = (threadIdx.x & 63) % LPR;
#pragma unroll
        for (int j = 0; j < CPL; j++)
#pragma unroll
            for (int q = 0; q < EPC / 8; q++) {
                const uint4 t = *reinterpret_cast<const uint4 *>(v + (sub + LPR * j) * EPC + 8 * q);
                const uint32_t u[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
                for (int m = 0; m < 4; m++) { x[j][8 * q + 2 * m] = bf_lo(u[m]); x[j][8 * q + 2 * m + 1] = bf_hi(u[m]); }
            }
    }
    __device__ __forceinline__ void norm(const float *g, float eps) {
        const int sub = (threadIdx.x & 63) % LPR;
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; j++)
#pragma unroll
            for (int e = 0; e < EPC; e++) ss = fmaf(x[j][e], x[j][e], ss);
        ss = group_sum<LPR>(ss);
        const float inv = 1.0f / sqrtf(ss / (float)COLS + eps);
#pragma unroll
        for (int j = 0; j < CPL; j++)
#pragma unroll
            for (int q = 0; q < EPC / 4; q++) {
                const float4 t = *reinterpret_cast<const float4 *>(g + (sub + LPR * j) * EPC + 4 * q);
                x[j][4 * q] = (x[j][4 * q] * inv) * t.x;
                x[j][4 * q + 1] = (x[j][4 * q + 1] * inv) * t.y;
                x[j][4 * q + 2] = (x[j][4 * q + 2] * inv) * t.z;
                x[j][4 * q + 3] = (x[j][4 * q + 3] * inv) * t.w;
            }
    }
    // write the (normalised) vector: every lane of group 0 writes its own chunks
    __device__ __forceinline__ void store(float *dst) {
        const int lane = threadIdx.x & 63, sub = lane % LPR;
        if (lane / LPR) return;
#pragma unroll
        for (int j = 0; j < CPL; j++)
#pragma unroll
            for (int e = 0; e < EPC; e++) dst[(sub + LPR * j) * EPC + e] = x[j][e];
    }
    __device__ __forceinline__ void sums() {
#pragma unroll
        for (int j = 0; j < CPL; j++) {
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < EPC; e++) s += x[j][e];
            xsum[j] = s;
        }
    }
};

// acc[r] = row dot products of the tile with the slice (group-reduced; valid in every
// lane of the group).  Same arithmetic as k_mv in qt_matvec.hip.
template <int PREC, int COLS, int RPW>
__device__ __forceinline__ void tile_dot(const Tile<PREC, COLS, RPW> &t, const Slice<PREC, COLS> &sl,
                                         float acc[Tile<PREC, COLS, RPW>::NR]) {
    using T = Tile<PREC, COLS, RPW>;
#pragma unroll
    for (int r = 0; r < T::NR; r++) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < T::CPL; j++) {
            const uint32_t w4[4] = {t.w[r][j].x, t.w[r][j].y, t.w[r][j].z, t.w[r][j].w};
            if (PREC == QT_BF16) {
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    s = fmaf(bf_lo(w4[m]), sl.x[j][2 * m], s);
                    s = fmaf(bf_hi(w4[m]), sl.x[j][2 * m + 1], s);
                }
            } else if (PREC == QT_INT8) {
                float u = 0.f;
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    const uint32_t w = w4[m];
                    u = fmaf((float)(w & 0xFFu), sl.x[j][4 * m + 0], u);
                    u = fmaf((float)((w >> 8) & 0xFFu), sl.x[j][4 * m + 1], u);
                    u = fmaf((float)((w >> 16) & 0xFFu), sl.x[j][4 * m + 2], u);
                    u = fmaf((float)(w >> 24), sl.x[j][4 * m + 3], u);
                }
                s += fmaf(-128.0f, sl.xsum[j], u);
            } else {
                float u = 0.f;
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    const uint32_t lo = w4[m] & 0x0F0F0F0Fu, hi = (w4[m] >> 4) & 0x0F0F0F0Fu;
                    u = fmaf((float)(lo & 0xFFu), sl.x[j][8 * m + 0], u);
                    u = fmaf((float)((lo >> 8) & 0xFFu), sl.x[j][8 * m + 2], u);
                    u = fmaf((float)((lo >> 16) & 0xFFu), sl.x[j][8 * m + 4], u);
                    u = fmaf((float)(lo >> 24), sl.x[j][8 * m + 6], u);
                    u = fmaf((float)(hi & 0xFFu), sl.x[j][8 * m + 1], u);
                    u = fmaf((float)((hi >> 8) & 0xFFu), sl.x[j][8 * m + 3], u);
                    u = fmaf((float)((hi >> 16) & 0xFFu), sl.x[j][8 * m + 5], u);
                    u = fmaf((float)(hi >> 24), sl.x[j][8 * m + 7], u);
                }
                s = fmaf(t.s[r][j], fmaf(-8.0f, sl.xsum[j], u), s);
            }
        }
        acc[r] = group_sum<T::LPR>(s);
    }
}

// Per-wave row results: lane sub==0 of every group holds NR consecutive rows' values;
// gather all RPW of them into LDS `res[wave][RPW]` so any lane can run the epilogue.
template <int RPW, int LPR, int NR>
__device__ __forceinline__ void publish(float (*res)[64], const float acc[NR]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane % LPR == 0) {
#pragma unroll
        for (int r = 0; r < NR; r++) res[wave][(lane / LPR) * NR + r] = acc[r];
    }
}

// ---- per-layer activation ring --------------------------------------------------------
template <int H, int F>
struct Ring {
    static constexpr int OQKV = 0, OATT = QKVR, OXA = OATT + QD, OH = OXA + H, OXB = OH + F, P = OXB + H;
    float *base;   // ring base
    int L;
    __device__ __forceinline__ float *blk(int par, int l) const { return base + ((size_t)par * L + l) * P; }
};

// ---- the kernel -------------------------------------------------------------------------
template <int PREC, int H, int F>
__global__ __launch_bounds__(256, 1) void k_pstep(Args a) {
    constexpr int RPW_QKV = QKVR / (NB * NW);      // 4
    constexpr int RPW_O = H / (NB * NW);           // 1 or 2
    constexpr int RPW_GU = 2 * F / (NB * NW);      // 6 or 12
    constexpr int RPW_DN = H / (NB * NW);          // 1 or 2
    constexpr int RPW_HEAD = 3;                    // 3072-row codec head
    using TQKV = Tile<PREC, H, RPW_QKV>;
    using TO = Tile<PREC, QD, RPW_O>;
    using TGU = Tile<PREC, H, RPW_GU>;
    using TDN = Tile<PREC, F, RPW_DN>;
    using THEAD = Tile<QT_BF16, H, RPW_HEAD>;

    __shared__ float res[NW][64];
    __shared__ float qs[HPK][HD];
    __shared__ float sc[HPK][CHMAX];
    __shared__ float ored[NW][HPK][HD];
    __shared__ float stat[HPK][2];
    __shared__ __align__(16) uint16_t knew[HD];
    __shared__ __align__(16) uint16_t vnew[HD];
    __shared__ float mst[G * HPK][2];
    __shared__ int last_flag;
    __shared__ float wbest_v[NW];
    __shared__ int wbest_i[NW];

    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    Bar bar;
    {
        const unsigned li = ld_u(a.bar + 2 * BAR_BLOCK);
        bar.blk = a.bar + (li & 1u) * BAR_BLOCK;
        bar.k = 0;
        bar.err = a.err;
    }
    PS_MARK(1023u, 1);   // launch entry (trace builds)
    Ring<H, F> ring{a.ring, a.n_layers};
    const int pos0 = *a.d_pos;
    const int frame0 = a.with_head ? *a.d_frame : 0;
    const int L = a.n_layers;
    int tok = -1;   // greedy token of the previous step (-1: input from a.xin)

    // attention item of this workgroup
    const int ag = b / G, ac = b % G;

    // prefetch of layer 0 QKV weights
    TQKV tq;
    tq.load(a.layers[0].w[0], a.layers[0].s16[0], b * (RPW_QKV * NW) + wave * RPW_QKV);

    for (int step = 0; step < a.n_steps; step++) {
        const int par = step & 1;
        const int pos = pos0 + step;
        const int Lk = pos + 1;
        if (step > 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");   // ring parities repeat
        int CH = (Lk + G - 1) / G;
        CH = (CH + 15) & ~15;
        const int nch = (Lk + CH - 1) / CH;
        const int j0 = ac * CH;
        const int n = (ac < nch) ? min(CH, Lk - j0) : 0;

        for (int l = 0; l < L; l++) {
            const Layer &ly = a.layers[l];
            float *blk = ring.blk(par, l);
            const float *xprev = (l == 0) ? nullptr : ring.blk(par, l - 1) + Ring<H, F>::OXB;

            // ---------------- A: q|k|v rows -----------------
            {
                Slice<PREC, H> sl;
                if (l > 0) sl.load(xprev);
                else if (tok < 0) sl.load(a.xin);
                else sl.load_bf16(a.emb + (size_t)tok * H);
                sl.norm(ly.in_norm, a.eps);
                sl.sums();
                float acc[TQKV::NR];
                tile_dot<PREC, H, RPW_QKV>(tq, sl, acc);
                publish<RPW_QKV, TQKV::LPR, TQKV::NR>(res, acc);
                __syncthreads();
                if (lane < RPW_QKV) {
                    const int row = b * (RPW_QKV * NW) + wave * RPW_QKV + lane;
                    float v = res[wave][lane];
                    if (PREC == QT_INT8) v = __fmul_rn(v, ly.s[0][row]);
                    st_agent(blk + Ring<H, F>::OQKV + row, v);
                }
            }
            bar_arrive(bar);
            // prefetch: K/V of this workgroup's attention chunk (first 64 keys)
            const uint16_t *Kg = a.kc + (((size_t)l * NKV + ag) * a.kv_max) * HD;
            const uint16_t *Vg = a.vc + (((size_t)l * NKV + ag) * a.kv_max) * HD;
            const int sub = lane & 15, pg = lane >> 4;
            uint4 kpre[4], vpre[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int jj = wave * 4 + pg + 16 * u;
                if (jj < n && j0 + jj != pos) {
                    kpre[u] = *reinterpret_cast<const uint4 *>(Kg + (size_t)(j0 + jj) * HD + sub * 8);
                    vpre[u] = *reinterpret_cast<const uint4 *>(Vg + (size_t)(j0 + jj) * HD + sub * 8);
                } else {
                    kpre[u] = make_uint4(0, 0, 0, 0);
                    vpre[u] = make_uint4(0, 0, 0, 0);
                }
            }
            bar_wait(bar);

            // ---------------- B: attention item -----------------
            if (n > 0) {
                const bool append = (pos >= j0 && pos < j0 + n);
                const float *qkv = blk + Ring<H, F>::OQKV;
                const int ntask = HPK + (append ? 1 : 0);
                for (int t = wave; t < ntask; t += NW) {
                    const bool isk = (t == HPK);
                    const float *src = isk ? qkv + QD + ag * HD : qkv + (ag * HPK + t) * HD;
                    const float *w = isk ? ly.kn : ly.qn;
                    const float x0 = src[lane], x1 = src[lane + 64];
                    const float ss = group_sum<64>(x0 * x0 + x1 * x1);
                    const float inv = 1.0f / sqrtf(ss / (float)HD + a.eps);
                    const float n0 = (x0 * inv) * w[lane], n1 = (x1 * inv) * w[lane + 64];
                    const float cs = a.rope_cos[(size_t)pos * 64 + lane], sn = a.rope_sin[(size_t)pos * 64 + lane];
                    const float r0 = fmaf(n0, cs, -(n1 * sn)), r1 = fmaf(n1, cs, n0 * sn);
                    if (!isk) {
                        qs[t][lane] = r0;
                        qs[t][lane + 64] = r1;
                    } else {
                        const float *vs = qkv + QD + KVD + ag * HD;
                        knew[lane] = f2bf_trunc(r0); knew[lane + 64] = f2bf_trunc(r1);
                        vnew[lane] = f2bf_trunc(vs[lane]); vnew[lane + 64] = f2bf_trunc(vs[lane + 64]);
                    }
                }
                __syncthreads();
                if (append && wave == NW - 1) {
                    // KV append: agent-scope 32-bit stores of adjacent bf16 pairs
                    uint32_t *kd = reinterpret_cast<uint32_t *>(a.kc + (((size_t)l * NKV + ag) * a.kv_max + pos) * HD);
                    uint32_t *vd = reinterpret_cast<uint32_t *>(a.vc + (((size_t)l * NKV + ag) * a.kv_max + pos) * HD);
                    const uint32_t kk = (uint32_t)knew[2 * lane] | ((uint32_t)knew[2 * lane + 1] << 16);
                    const uint32_t vv = (uint32_t)vnew[2 * lane] | ((uint32_t)vnew[2 * lane + 1] << 16);
                    __hip_atomic_store(kd + lane, kk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(vd + lane, vv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                float qv[HPK][8];
#pragma unroll
                for (int h = 0; h < HPK; h++)
#pragma unroll
                    for (int e = 0; e < 8; e++) qv[h][e] = qs[h][sub * 8 + e];
                for (int blk0 = 0; blk0 < n; blk0 += 64) {
                    uint4 kw[4];
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const int jj = blk0 + wave * 4 + pg + 16 * u;
                        if (blk0 == 0) kw[u] = kpre[u];
                        else kw[u] = (jj < n && j0 + jj != pos) ? *reinterpret_cast<const uint4 *>(Kg + (size_t)(j0 + jj) * HD + sub * 8)
                                                               : make_uint4(0, 0, 0, 0);
                        if (j0 + jj == pos && jj < n) kw[u] = *reinterpret_cast<const uint4 *>(knew + sub * 8);
                    }
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const uint32_t w4[4] = {kw[u].x, kw[u].y, kw[u].z, kw[u].w};
                        float kf[8];
#pragma unroll
                        for (int m = 0; m < 4; m++) { kf[2 * m] = bf_lo(w4[m]); kf[2 * m + 1] = bf_hi(w4[m]); }
                        const int jj = blk0 + wave * 4 + pg + 16 * u;
#pragma unroll
                        for (int h = 0; h < HPK; h++) {
                            float s = 0.f;
#pragma unroll
                            for (int e = 0; e < 8; e++) s = fmaf(qv[h][e], kf[e], s);
                            s = group_sum<16>(s);
                            if (sub == 0 && jj < n) sc[h][jj] = s * a.scale;
                        }
                    }
                }
                __syncthreads();
                for (int h = wave; h < HPK; h += NW) {
                    float m = -INFINITY;
                    for (int j = lane; j < n; j += 64) m = fmaxf(m, sc[h][j]);
                    m = group_max<64>(m);
                    float lsum = 0.f;
                    for (int j = lane; j < n; j += 64) {
                        const float p = expf(sc[h][j] - m);
                        sc[h][j] = p;
                        lsum += p;
                    }
                    lsum = group_sum<64>(lsum);
                    if (lane == 0) { stat[h][0] = m; stat[h][1] = lsum; }
                }
                __syncthreads();
                float o[HPK][8];
#pragma unroll
                for (int h = 0; h < HPK; h++)
#pragma unroll
                    for (int e = 0; e < 8; e++) o[h][e] = 0.f;
                for (int blk0 = 0; blk0 < n; blk0 += 64) {
                    uint4 vw[4];
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const int jj = blk0 + wave * 4 + pg + 16 * u;
                        if (blk0 == 0) vw[u] = vpre[u];
                        else vw[u] = (jj < n && j0 + jj != pos) ? *reinterpret_cast<const uint4 *>(Vg + (size_t)(j0 + jj) * HD + sub * 8)
                                                               : make_uint4(0, 0, 0, 0);
                        if (j0 + jj == pos && jj < n) vw[u] = *reinterpret_cast<const uint4 *>(vnew + sub * 8);
                    }
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const int jj = blk0 + wave * 4 + pg + 16 * u;
                        if (jj < n) {
                            const uint32_t w4[4] = {vw[u].x, vw[u].y, vw[u].z, vw[u].w};
                            float vf[8];
#pragma unroll
                            for (int m = 0; m < 4; m++) { vf[2 * m] = bf_lo(w4[m]); vf[2 * m + 1] = bf_hi(w4[m]); }
#pragma unroll
                            for (int h = 0; h < HPK; h++) {
                                const float p = sc[h][jj];
#pragma unroll
                                for (int e = 0; e < 8; e++) o[h][e] = fmaf(p, vf[e], o[h][e]);
                            }
                        }
                    }
                }
#pragma unroll
                for (int h = 0; h < HPK; h++)
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        float v = o[h][e];
                        v += __shfl_xor(v, 16, 64);
                        v += __shfl_xor(v, 32, 64);
                        o[h][e] = v;
                    }
                if (pg == 0) {
#pragma unroll
                    for (int h = 0; h < HPK; h++)
#pragma unroll
                        for (int e = 0; e < 8; e++) ored[wave][h][sub * 8 + e] = o[h][e];
                }
                __syncthreads();
                float *attn = blk + Ring<H, F>::OATT;
                if (nch == 1) {
                    for (int i = tid; i < HPK * HD; i += NW * 64) {
                        const int h = i / HD, d = i % HD;
                        const float v = ored[0][h][d] + ored[1][h][d] + ored[2][h][d] + ored[3][h][d];
                        st_agent(attn + (ag * HPK + h) * HD + d, v * (1.0f / stat[h][1]));
                    }
                } else {
                    constexpr int PS = 2 + HD;
                    float *mypart = a.part + ((size_t)(ag * G + ac) * HPK) * PS;
                    for (int i = tid; i < HPK * HD; i += NW * 64) {
                        const int h = i / HD, d = i % HD;
                        st_agent(mypart + h * PS + 2 + d, ored[0][h][d] + ored[1][h][d] + ored[2][h][d] + ored[3][h][d]);
                    }
                    if (tid < HPK) { st_agent(mypart + tid * PS, stat[tid][0]); st_agent(mypart + tid * PS + 1, stat[tid][1]); }
                    __builtin_amdgcn_s_waitcnt(0);
                    __syncthreads();
                    if (tid == 0) last_flag = (add_u(a.cnt + ag, 1u) == (unsigned)(nch - 1));
                    __syncthreads();
                    if (last_flag) {
                        const float *gp = a.part + (size_t)ag * G * HPK * PS;
                        for (int i = tid; i < nch * HPK; i += NW * 64) {
                            mst[i][0] = ld_agent(gp + (size_t)i * PS);
                            mst[i][1] = ld_agent(gp + (size_t)i * PS + 1);
                        }
                        __syncthreads();
                        for (int i = tid; i < HPK * HD; i += NW * 64) {
                            const int h = i / HD, d = i % HD;
                            float pv[G];
#pragma unroll
                            for (int cc = 0; cc < G; cc++) pv[cc] = (cc < nch) ? ld_agent(gp + (size_t)(cc * HPK + h) * PS + 2 + d) : 0.f;
                            float M = -INFINITY;
                            for (int cc = 0; cc < nch; cc++) M = fmaxf(M, mst[cc * HPK + h][0]);
                            float lsum = 0.f, v = 0.f;
#pragma unroll
                            for (int cc = 0; cc < G; cc++) {
                                if (cc < nch) {
                                    const float f = expf(mst[cc * HPK + h][0] - M);
                                    lsum = fmaf(mst[cc * HPK + h][1], f, lsum);
                                    v = fmaf(pv[cc], f, v);
                                }
                            }
                            st_agent(attn + (ag * HPK + h) * HD + d, v * (1.0f / lsum));
                        }
                        if (tid == 0) st_u(a.cnt + ag, 0u);
                    }
                }
            }
            bar_arrive(bar);
            TO to;
            to.load(ly.w[1], ly.s16[1], b * (RPW_O * NW) + wave * RPW_O);
            bar_wait(bar);

            // ---------------- C: xa = x + W_o . attn -----------------
            {
                Slice<PREC, QD> sl;
                sl.load(blk + Ring<H, F>::OATT);
                sl.sums();
                float acc[TO::NR];
                tile_dot<PREC, QD, RPW_O>(to, sl, acc);
                publish<RPW_O, TO::LPR, TO::NR>(res, acc);
                __syncthreads();
                if (lane < RPW_O) {
                    const int row = b * (RPW_O * NW) + wave * RPW_O + lane;
                    float v = res[wave][lane];
                    if (PREC == QT_INT8) v = __fmul_rn(v, ly.s[1][row]);
                    const float xo = (l > 0) ? xprev[row] : (tok < 0 ? a.xin[row] : bf16f(a.emb[(size_t)tok * H + row]));
                    st_agent(blk + Ring<H, F>::OXA + row, __fadd_rn(xo, v));
                }
            }
            bar_arrive(bar);
            TGU tg;
            tg.load(ly.w[2], ly.s16[2], b * (RPW_GU * NW) + wave * RPW_GU);
            bar_wait(bar);

            // ---------------- D: h = SwiGLU(W_gu . RMSNorm(xa)) -----------------
            {
                Slice<PREC, H> sl;
                sl.load(blk + Ring<H, F>::OXA);
                sl.norm(ly.post_norm, a.eps);
                sl.sums();
                float acc[TGU::NR];
                tile_dot<PREC, H, RPW_GU>(tg, sl, acc);
                publish<RPW_GU, TGU::LPR, TGU::NR>(res, acc);
                __syncthreads();
                if (lane < RPW_GU / 2) {
                    const int row = b * (RPW_GU * NW) + wave * RPW_GU + 2 * lane;
                    float g = res[wave][2 * lane], u = res[wave][2 * lane + 1];
                    if (PREC == QT_INT8) { g = __fmul_rn(g, ly.s[2][row]); u = __fmul_rn(u, ly.s[2][row + 1]); }
                    st_agent(blk + Ring<H, F>::OH + (row >> 1), g / (1.0f + expf(-g)) * u);
                }
            }
            bar_arrive(bar);
            TDN td;
            td.load(ly.w[3], ly.s16[3], b * (RPW_DN * NW) + wave * RPW_DN);
            bar_wait(bar);

            // ---------------- E: xb = xa + W_dn . h -----------------
            {
                Slice<PREC, F> sl;
                sl.load(blk + Ring<H, F>::OH);
                sl.sums();
                float acc[TDN::NR];
                tile_dot<PREC, F, RPW_DN>(td, sl, acc);
                publish<RPW_DN, TDN::LPR, TDN::NR>(res, acc);
                __syncthreads();
                if (lane < RPW_DN) {
                    const int row = b * (RPW_DN * NW) + wave * RPW_DN + lane;
                    float v = res[wave][lane];
                    if (PREC == QT_INT8) v = __fmul_rn(v, ly.s[3][row]);
                    st_agent(blk + Ring<H, F>::OXB + row, __fadd_rn(blk[Ring<H, F>::OXA + row], v));
                }
            }
            bar_arrive(bar);
            if (l + 1 < L) tq.load(a.layers[l + 1].w[0], a.layers[l + 1].s16[0], b * (RPW_QKV * NW) + wave * RPW_QKV);
            bar_wait(bar);
        }

        const float *xfin = ring.blk(par, L - 1) + Ring<H, F>::OXB;
        if (!a.with_head) {
            // final norm of the residual -> hid (workgroup 0)
            if (b == 0 && wave == 0) {
                Slice<QT_BF16, H> sl;
                sl.load(xfin);
                sl.norm(a.final_norm, a.eps);
                sl.store(a.hid);
            }
        } else {
            // ---------------- head: logits rows + masked local argmax -----------------
            THEAD th;
            th.load(a.head_w, nullptr, b * (RPW_HEAD * NW) + wave * RPW_HEAD);
            Slice<QT_BF16, H> sl;
            sl.load(xfin);
            sl.norm(a.final_norm, a.eps);
            if (b == 0 && wave == 0) sl.store(a.hid);
            float acc[THEAD::NR];
            tile_dot<QT_BF16, H, RPW_HEAD>(th, sl, acc);
            publish<RPW_HEAD, THEAD::LPR, THEAD::NR>(res, acc);
            __syncthreads();
            const int frame = frame0 + step;
            if (lane == 0) {
                float bv = -INFINITY; int bi = 0x7FFFFFFF;
                for (int r = 0; r < RPW_HEAD; r++) {
                    const int i = b * (RPW_HEAD * NW) + wave * RPW_HEAD + r;
                    if (i >= a.vocab) break;
                    float v = fminf(fmaxf(res[wave][r], -100.0f), 100.0f);
                    if (i >= 2048 && i != 2150) v = -1e30f;
                    if (i == 2150 && frame < 2) v = -1e30f;
                    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
                }
                wbest_v[wave] = bv; wbest_i[wave] = bi;
            }
            __syncthreads();
            if (tid == 0) {
                float bv = wbest_v[0]; int bi = wbest_i[0];
                for (int w = 1; w < NW; w++)
                    if (wbest_v[w] > bv || (wbest_v[w] == bv && wbest_i[w] < bi)) { bv = wbest_v[w]; bi = wbest_i[w]; }
                st_agent(a.slots + 2 * b, bv);
                st_agent(a.slots + 2 * b + 1, __int_as_float(bi));
            }
            bar_arrive(bar);
            if (step + 1 < a.n_steps)
                tq.load(a.layers[0].w[0], a.layers[0].s16[0], b * (RPW_QKV * NW) + wave * RPW_QKV);
            bar_wait(bar);
            // global argmax over the 256 local winners (every workgroup, redundantly)
            {
                float bv = -INFINITY; int bi = 0x7FFFFFFF;
                for (int i = tid; i < NB; i += NW * 64) {
                    const float v = ld_agent(a.slots + 2 * i);
                    const int ix = __float_as_int(ld_agent(a.slots + 2 * i + 1));
                    if (v > bv || (v == bv && ix < bi)) { bv = v; bi = ix; }
                }
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) {
                    const float ov = __shfl_xor(bv, o, 64);
                    const int oi = __shfl_xor(bi, o, 64);
                    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
                }
                if (lane == 0) { wbest_v[wave] = bv; wbest_i[wave] = bi; }
                __syncthreads();
                float gv = wbest_v[0]; int gi = wbest_i[0];
                for (int w = 1; w < NW; w++)
                    if (wbest_v[w] > gv || (wbest_v[w] == gv && wbest_i[w] < gi)) { gv = wbest_v[w]; gi = wbest_i[w]; }
                if (gi == 0x7FFFFFFF) gi = 0;
                tok = gi;
                if (b == 0 && tid == 0) a.hist[frame % a.hist_len] = gi;
                __syncthreads();   // wbest_* reused next step
            }
        }
    }
    // epilogue: position/frame advance, next launch's barrier block
    if (b == 0 && tid == 0) {
        *a.d_pos = pos0 + a.n_steps;
        if (a.with_head) *a.d_frame = frame0 + a.n_steps;
    }
    if (a.with_head && b == 0) {
        // next input embedding (for a following launch / the host)
        for (int i = tid; i < H; i += NW * 64) a.xin[i] = bf16f(a.emb[(size_t)tok * H + i]);
    }
    // the counter block of this launch is dirty; zero the other one for the next launch
    bar_arrive(bar);
    bar_wait(bar);
    if (b == 0) {
        const unsigned li = ld_u(a.bar + 2 * BAR_BLOCK);
        unsigned *other = a.bar + ((li + 1u) & 1u) * BAR_BLOCK;
        for (int i = tid; i < BAR_BLOCK; i += NW * 64) st_u(other + i, 0u);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) st_u(a.bar + 2 * BAR_BLOCK, li + 1u);
    }
}
}  // namespace ps

#ifdef QT_PSTEP_TRACE
extern "C" hipError_t qt_pstep_trace_read(unsigned long long *out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(ps::ps_trace), sizeof(ps::ps_trace), 0, hipMemcpyDeviceToHost);
}
#endif

template <int PREC, int H, int F>
static hipError_t ps_launch(const ps::Args &a, hipStream_t st) {
    void *args[] = {(void *)&a};
    return hipLaunchCooperativeKernel((const void *)ps::k_pstep<PREC, H, F>, dim3(ps::NB), dim3(ps::NW * 64), args, 0, st);
}

extern "C" int qt_pstep_supported(int prec, int hidden, int inter, int n_heads, int n_kv, int head_dim, int kv_max) {
    if (n_heads != ps::NH || n_kv != ps::NKV || head_dim != ps::HD) return 0;
    if (kv_max > ps::G * ps::CHMAX) return 0;
    if (prec != QT_BF16 && prec != QT_INT8) return 0;
    if (!((hidden == 1024 && inter == 3072) || (hidden == 2048 && inter == 6144))) return 0;
    int dev = 0, cus = 0, coop = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess) return 0;
    if (!coop || cus < ps::NB) return 0;
    return 1;
}

// ring floats needed for n_layers layers (2 parities) of a model
extern "C" size_t qt_pstep_ring_floats(int hidden, int inter, int n_layers) {
    const size_t P = (size_t)ps::QKVR + ps::QD + 2 * (size_t)hidden + inter;
    return 2 * (size_t)n_layers * P;
}
extern "C" size_t qt_pstep_bar_words(void) { return 2 * ps::BAR_BLOCK + 64; }
extern "C" size_t qt_pstep_layer_bytes(void) { return sizeof(ps::Layer); }

// Layer table entry, filled on the host in this exact order.
extern "C" void qt_pstep_fill_layer(void *dst, const uint8_t *const w[4], const float *const s[4],
                                    const uint16_t *const s16[4], const float *in_norm, const float *post_norm,
                                    const float *qn, const float *kn) {
    ps::Layer *L = (ps::Layer *)dst;
    for (int i = 0; i < 4; i++) { L->w[i] = w[i]; L->s[i] = s[i]; L->s16[i] = s16[i]; }
    L->in_norm = in_norm; L->post_norm = post_norm; L->qn = qn; L->kn = kn;
}

extern "C" hipError_t qt_launch_pstep(int prec, int hidden, const void *layers_dev, int n_layers,
                                      const float *final_norm, const float *rope_cos, const float *rope_sin,
                                      uint16_t *kc, uint16_t *vc, int kv_max, float eps, float scale, float *ring,
                                      float *part, unsigned *cnt, float *hid, float *xin, int *d_pos,
                                      unsigned *bar, int *err, int n_steps, int with_head, const uint16_t *head_w,
                                      const uint16_t *emb, int vocab, float *slots, int *d_frame, int *hist,
                                      int hist_len, hipStream_t st) {
    ps::Args a;
    a.layers = (const ps::Layer *)layers_dev; a.n_layers = n_layers;
    a.final_norm = final_norm; a.rope_cos = rope_cos; a.rope_sin = rope_sin;
    a.kc = kc; a.vc = vc; a.kv_max = kv_max; a.eps = eps; a.scale = scale;
    a.ring = ring; a.part = part; a.cnt = cnt; a.hid = hid; a.xin = xin; a.d_pos = d_pos;
    a.bar = bar; a.err = err; a.n_steps = n_steps; a.with_head = with_head;
    a.head_w = (const uint8_t *)head_w; a.emb = emb; a.vocab = vocab; a.slots = slots;
    a.d_frame = d_frame; a.hist = hist; a.hist_len = hist_len;
    if (n_steps <= 0 || n_layers <= 0) return hipErrorInvalidValue;
    if (with_head && (vocab != ps::NB * ps::NW * 3 || !head_w || !emb || !slots || !d_frame || !hist)) return hipErrorInvalidValue;
    if (prec == QT_INT8 && hidden == 2048) return ps_launch<QT_INT8, 2048, 6144>(a, st);
    if (prec == QT_INT8 && hidden == 1024) return ps_launch<QT_INT8, 1024, 3072>(a, st);
    if (prec == QT_BF16 && hidden == 2048) return ps_launch<QT_BF16, 2048, 6144>(a, st);
    if (prec == QT_BF16 && hidden == 1024) return ps_launch<QT_BF16, 1024, 3072>(a, st);
    return hipErrorInvalidValue;
}
