// qt_rstep.hip — the Talker decode step of the 1.7B geometry with int8 weights (hidden
// 2048, intermediate 6144, 16 query / 8 kv heads of 128) as ONE persistent cooperative
// kernel whose workgroups each own ONE phase of the layer.
//
// Same math as qwen_talker_step (qwen_tts_talker.c:537-699), same arithmetic per output
// as the per-kernel path (qt_matvec.hip, qt_attn.hip with 8 key chunks per kv head), so
// the two agree to the bit.
//
// Why roles.  A decode layer is a chain of six dependent hand-offs (x -> q|k|v ->
// attention partials -> attention output -> xa -> h -> x'), and each hand-off between
// workgroups costs a trip through the device coherence point.  On a CU, every load
// waits behind the loads issued before it (the CU's memory pipeline is in order across
// its waves), so a workgroup that streams its next weight tile while it polls for its
// next input pays the tile's arrival time on every hand-off (measured: 32 KB of tile
// loads in flight add 0.5-1.0 us to a 2048-word exchange, 64 KB add 1.5-1.9 us).  Here a
// workgroup takes part in one phase per layer (attention takes two: the chunk and the
// merge), streams its tile for the next layer right after its phase, waits until the
// tile has landed and only then polls for its next input — which comes most of a layer
// later, so the tile is in registers by then and the poll sees an empty pipeline.  Each
// workgroup's tile is ~256 KB (int8 rows in VGPR/AGPR) or its attention chunk's keys
// (K in registers, V in LDS), so the weights still stream at the full HBM rate, spread
// over the whole layer instead of in bursts in front of every hand-off.
//
// Workgroup b runs on XCD b % 8 (round-robin dispatch) as slot b / 8 of that XCD:
//   slots  0..3   Q    q|k|v rows of kv group x (head 2x, head 2x+1, k head x, v head x:
//                      128 rows each), RMSNorm fused (exact int8 pieces, MFMA)
//   slots  4..11  ATT  attention chunk c = slot-4 of kv head x (ceil(L/8) keys rounded to
//                      16: per-head q/k norm, RoPE, KV append, scores, softmax, P.V), then
//                      MRG: merge of the group's 8 chunk partials for 32 outputs
//   slots 12..13  O    xa = x + W_o . attn, 128 rows
//   slots 14..25  GU   h = SwiGLU(W_gu . RMSNorm(xa)), 128 interleaved rows = 64 h values
//   slots 26..31  DN   x' = xa + W_dn . h, 48 or 40 rows
// and after the last layer every workgroup but ATT takes 16 rows of the codec head
// (final RMSNorm, masked local argmax) and the global argmax over their 192 winners.
//
// Hand-offs use 4-byte words in a region that holds a sentinel (0xFFFFFFFF, a NaN no
// arithmetic produces) until the producer writes the value: consumers read with
// agent-scope 16-byte loads and re-read groups that still hold a sentinel.  There is one
// region per step parity; during step s the head workgroups clear the region of step
// s-1 (every read of it is done: all of that step's reads precede its winner exchange),
// each fences its clears before publishing its next winner, and after the launch's last
// winner exchange they clear the last step's region, so both regions are clean between
// launches.  The winners themselves use tagged 8-byte words (step number | value).
// Every wait is bounded: on timeout the kernel sets an error flag, the others see it and
// stop waiting, and the launch runs to its end.
#include "qt_step_common.h"

namespace ps {
namespace rs {
constexpr int H = 2048, F = 6144, NT = 256;
constexpr unsigned SENT = 0xFFFFFFFFu;
constexpr int XQ = 4, XATT = 8, XO = 2, XG = 12, XD = 6;                 // workgroups per XCD and role
constexpr int SQ0 = 0, SA0 = SQ0 + XQ, SO0 = SA0 + XATT, SG0 = SO0 + XO, SD0 = SG0 + XG;
static_assert(SD0 + XD == NB / 8, "32 workgroups per XCD");
constexpr int NQ = 8 * XQ, NO = 8 * XO, NG = 8 * XG, ND = 8 * XD;
constexpr int NHEAD = NQ + NO + NG + ND;         // 192: every role but attention
constexpr int ACH = XATT;                        // attention chunks per kv head
constexpr int QROWS = QKVR / NQ, OROWS = H / NO, GROWS = 2 * F / NG;
static_assert(QROWS == 128 && OROWS == 128 && GROWS == 128, "128 rows per projection workgroup");
constexpr int HEADR = 3072 / NHEAD;              // codec-head rows per workgroup (16)
constexpr int ABLK = 4;                          // 128-key blocks of a chunk held resident (512 keys)
constexpr int MAXLR = 32;
// words of one layer's hand-off block
constexpr int R_QKV = 0, R_PO = R_QKV + QKVR, R_PML = R_PO + NKV * HPK * 4 * ACH * 32,
              R_ATT = R_PML + NKV * HPK * ACH * 2, R_XA = R_ATT + QD, R_H = R_XA + H, R_X = R_H + F, LW = R_X + H;
constexpr int CLR16 = LW / (4 * NHEAD);          // 16-byte groups of a layer block each head workgroup clears
static_assert(CLR16 * 4 * NHEAD == LW && CLR16 <= NT, "clear shares");
constexpr int SC1 = 16;                          // buffer cache policy: agent scope (sc1)

// Optional phase trace (build with -DQT_RSTEP_TRACE): s_memrealtime (100 MHz) of each
// workgroup at marks k of (step, layer) — 0 its input wait starts, 1 the input has
// arrived, 2 its output is published, 3 its next tile has landed; attention adds 4 (merge
// input arrived) and 5 (merge output published); layer index L is the head (0 wait starts,
// 1 x arrived, 2 winner published, 4 winners arrived).  Steps past TR_STEPS are not kept.
#ifdef QT_RSTEP_TRACE
constexpr int TR_STEPS = 8, TR_L = 33;
__device__ unsigned long long rs_trace[NB][TR_STEPS * TR_L][8];
#define RS_MARK(st, l, k)                                                                             \
    do {                                                                                              \
        if (threadIdx.x == 0 && (st) < TR_STEPS)                                                      \
            rs_trace[blockIdx.x][(st) * TR_L + (l)][k] = __builtin_amdgcn_s_memrealtime();            \
    } while (0)
#else
#define RS_MARK(st, l, k) do { } while (0)
#endif

struct RArgs {
    const Layer *layers;
    int n_layers;
    const float *final_norm, *rope_cos, *rope_sin;
    uint16_t *kc, *vc;            // [L][NKV][kv_max][HD]
    int kv_max;
    float eps, scale;
    unsigned *reg;                // [2][L][LW] hand-off words (sentinel when empty)
    unsigned long long *slots;    // [2][NHEAD][2] tagged winner words
    float *hid, *decx, *xin;
    int *d_pos;
    unsigned *epoch;
    int *err;
    int n_steps, with_head;
    const uint8_t *head_w;        // bf16 [vocab][H]
    const uint16_t *emb;          // bf16 [vocab][H]
    int vocab;
    int *d_frame, *hist;
    int hist_len;
    float *layer_out;             // optional [L][H]: every layer's output x of the last step
};

// ---- hand-off words ---------------------------------------------------------------------
__device__ __forceinline__ __amdgpu_buffer_rsrc_t brsrc(const void *p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, 0x7FFFFFFF, 0x00020000);
}
__device__ __forceinline__ uint4 ld16a(__amdgpu_buffer_rsrc_t r, unsigned byte_off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, SC1);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ unsigned ld4a(__amdgpu_buffer_rsrc_t r, unsigned byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, SC1);
}
__device__ __forceinline__ void put(unsigned *p, float v) {
    __hip_atomic_store(p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool stale16(const uint4 &v) { return v.x == SENT || v.y == SENT || v.z == SENT || v.w == SENT; }
__device__ __forceinline__ void land() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Waits until the 16-byte groups i = tid + NT*k < n16 (byte offset off(i) in r) hold no
// sentinel; stale groups are re-read after a short pause.  Bounded.
// A consumer usually waits most of a layer for its input, and re-reading all of it every
// round trip would load the fabric with ~36 MB of polls per layer.  So each wave first
// polls a sparse sample (groups PST*j, j = lane*4 + wave: every producer's range holds
// some) until any sampled group is fresh — the producers then finish within a fraction of
// a microsecond — and only then reads the whole input.
template <int K, int PST, typename OffF>
__device__ __forceinline__ void wait16(__amdgpu_buffer_rsrc_t r, int n16, OffF off, uint4 (&v)[K], int *err) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (PST > 0) {
        const int j = lane * 4 + wave, np = (n16 + PST - 1) / PST;
        const bool act = j < np;
        for (unsigned it = 0;; it++) {
            const bool fresh = act && !stale16(ld16a(r, off(act ? j * PST : 0)));
            if (__builtin_amdgcn_ballot_w64(fresh) != 0) break;
            if ((it & 31) == 31) {
                if (ld_i(err)) break;
                if (it > POLL_LIMIT) { st_i(err, 1); break; }
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
#pragma unroll
    for (int k = 0; k < K; k++) v[k] = (tid + NT * k < n16) ? ld16a(r, off(tid + NT * k)) : make_uint4(0, 0, 0, 0);
    for (unsigned it = 0;; it++) {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < K; k++) ok = ok && !stale16(v[k]);
        if (ok) break;
        if ((it & 31) == 31) {
            if (ld_i(err)) break;
            if (it > POLL_LIMIT) { st_i(err, 1); break; }
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int k = 0; k < K; k++)
            if (stale16(v[k])) v[k] = ld16a(r, off(tid + NT * k));
    }
}
// Same for K single words per thread, element i = tid + NT*k at byte offset off(i): the
// element-to-thread map of the RMSNorm statistics (pc_stats), so the sums keep their order.
// The sparse first poll samples words PST*j.
template <int K, int PST, typename OffF>
__device__ __forceinline__ void wait4(__amdgpu_buffer_rsrc_t r, int n, OffF off, unsigned (&v)[K], int *err) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (PST > 0) {
        const int j = lane * 4 + wave, np = (n + PST - 1) / PST;
        const bool act = j < np;
        for (unsigned it = 0;; it++) {
            const bool fresh = act && ld4a(r, off(act ? j * PST : 0)) != SENT;
            if (__builtin_amdgcn_ballot_w64(fresh) != 0) break;
            if ((it & 31) == 31) {
                if (ld_i(err)) break;
                if (it > POLL_LIMIT) { st_i(err, 1); break; }
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
#pragma unroll
    for (int k = 0; k < K; k++) v[k] = ld4a(r, off(tid + NT * k));
    for (unsigned it = 0;; it++) {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < K; k++) ok = ok && v[k] != SENT;
        if (ok) break;
        if ((it & 31) == 31) {
            if (ld_i(err)) break;
            if (it > POLL_LIMIT) { st_i(err, 1); break; }
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int k = 0; k < K; k++)
            if (v[k] == SENT) v[k] = ld4a(r, off(tid + NT * k));
    }
}
// 4 consecutive elements e0..e0+3 (e0 % 4 == 0) of a COLS-wide activation into its
// chunk-transposed LDS layout (xpos): they stay consecutive there.
template <int EPC, int COLS>
__device__ __forceinline__ void put4(float *x, int e0, const uint4 &v) {
    *reinterpret_cast<float4 *>(x + xpos<EPC, COLS>(e0)) =
        make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}

// ---- MFMA row tiles (4 rows per MFMA: row m % 4 of column part m / 4, TileM4 layout) ----
// NQ quads of 4 consecutive rows per wave over COLS columns: w[q][s] covers rows
// row0 + 4q .. +3, columns s*256 + part*64 + 16*kg.
template <int COLS, int NQD>
struct RTile {
    static constexpr int S = COLS / 256;
    uint4 w[NQD][S];
    // buffer loads: one 32-bit lane offset shared by every load, the row and step parts in
    // scalar registers (64-bit per-lane addresses would hold two VGPRs per load in flight)
    __device__ __forceinline__ void load(const uint8_t *W, int row0, int nq) {
        const int lane = threadIdx.x & 63, m = lane & 15, kg = lane >> 4;
        const __amdgpu_buffer_rsrc_t r = brsrc(uni(W));
        const unsigned voff = (unsigned)((m & 3) * COLS + (m >> 2) * 64 + kg * 16);
#pragma unroll
        for (int q = 0; q < NQD; q++)
            if (q < nq) {
#pragma unroll
                for (int s = 0; s < S; s++) {
                    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(
                        r, voff, __builtin_amdgcn_readfirstlane((row0 + 4 * q) * COLS + s * 256), 0);
                    w[q][s] = make_uint4(v.x, v.y, v.z, v.w);
                }
            }
    }
};
// acc[q] = the TileM4 result of quad q against the pieces (B fragment of step s read one
// step ahead, shared by the quads); quads >= nq are skipped.  Two accumulator chains per
// quad when there are few quads, so no MFMA waits for the previous one of its chain.
template <int COLS, int NQD>
__device__ __forceinline__ void rdot(const RTile<COLS, NQD> &t, const uint8_t *pc, int nq, i32x4 (&acc)[NQD]) {
    constexpr int S = COLS / 256;
    constexpr int CH = NQD >= 4 ? 1 : 2;
    i32x4 a[NQD][CH];
#pragma unroll
    for (int q = 0; q < NQD; q++)
#pragma unroll
        for (int c = 0; c < CH; c++) a[q][c] = i32x4{0, 0, 0, 0};
    uint4 b = mf_b4<COLS>(pc, 0);
#pragma unroll
    for (int s = 0; s < S; s++) {
        const uint4 bn = mf_b4<COLS>(pc, s + 1 < S ? s + 1 : s);
#pragma unroll
        for (int q = 0; q < NQD; q++)
            if (q < nq) a[q][s % CH] = mfma_i8(t.w[q][s], b, a[q][s % CH]);
        b = bn;
    }
#pragma unroll
    for (int q = 0; q < NQD; q++) {
        acc[q] = a[q][0];
#pragma unroll
        for (int c = 1; c < CH; c++) acc[q] += a[q][c];
    }
}

// ---- LDS --------------------------------------------------------------------------------
struct HeadLds {
    float x[H];                  // x of the last layer, chunk-transposed (EPC 8)
    float xn[H];                 // final-normed
    float gain[H];               // final norm gains (EPC 8 layout)
    float wbv[4];
    int wbi[4];
    float win[2 * NHEAD];
};
struct LdsP {                    // Q, O, GU (2048-column projections)
    float x[H];                  // gathered input, chunk-transposed (EPC 16)
    float gain[H];
    uint8_t pc[4 * H];
    int red[4][8 * 64];
    float resid[OROWS];
    float wst[8];
    HeadLds hd;
};
struct LdsD {                    // DN
    uint8_t pc[4 * F];
    uint4 tw[4][F / 256][64];    // row-quad 2 of each wave's rows (when it has one): [wave][step][lane]
    int red[4][3 * 64];
    float resid[48];
    float wst[8];
    HeadLds hd;
};
struct LdsA {                    // ATT + MRG
    uint16_t v[ABLK][KVB * HD];  // value rows of the chunk (qt_attn_mf.h swizzle), per 128-key block
    uint16_t qp[16][HD];
    uint16_t pp[2][16][KVB];     // probability pieces, by block parity
    float ml[2][4][HPK][2];
    float qkv[HPK * HD + 2 * HD];
    uint16_t knew[HD], vnew[HD];
    float mo[ACH][32];           // merge inputs
    float mml[ACH][2];
};
constexpr size_t LDS_BYTES = sizeof(LdsA) > sizeof(LdsD) ? (sizeof(LdsA) > sizeof(LdsP) ? sizeof(LdsA) : sizeof(LdsP))
                                                          : (sizeof(LdsD) > sizeof(LdsP) ? sizeof(LdsD) : sizeof(LdsP));

// per-step geometry of the attention chunks (the per-kernel attention's rule with 8 chunks)
struct Geo {
    int pos, CH, nch;
    __device__ __forceinline__ Geo(int p) : pos(p) {
        const int Lk = p + 1;
        CH = ((Lk + ACH - 1) / ACH + 15) & ~15;
        nch = (Lk + CH - 1) / CH;
    }
};

// ---- role context -----------------------------------------------------------------------
struct Ctx {
    RArgs a;
    const Layer *ly;              // layer table (LDS)
    __amdgpu_buffer_rsrc_t rr;    // hand-off region
    int L, pos0, frame0;
    unsigned tag0;
    int hc;                       // head workgroup index (-1: attention)
    __device__ __forceinline__ unsigned blk(int par, int l) const { return (unsigned)((par * L + l) * LW); }   // word offset
    __device__ __forceinline__ unsigned *wp(int par, int l, int off) const { return a.reg + blk(par, l) + off; }
};

// the 43 16-byte groups of this head workgroup's share of layer l's block, parity par
__device__ __forceinline__ void clear_share(const Ctx &c, int par, int l) {
    const int tid = threadIdx.x;
    if (tid < CLR16) {
        const u32x4_t s = {SENT, SENT, SENT, SENT};
        __builtin_amdgcn_raw_buffer_store_b128(s, c.rr, (c.blk(par, l) + (unsigned)(c.hc * CLR16 + tid) * 4u) * 4u, 0, SC1);
    }
}

// Layer-0 input element i of a step: the embedding of the previous step's token, or xin.
__device__ __forceinline__ float x0_elem(const RArgs &a, int tok, int i) {
    return tok < 0 ? ldg(a.xin + i) : bf16f(ldg(a.emb + (size_t)tok * H + i));
}

// ---- head (final norm, codec head rows, masked local argmax, global argmax) ------------
using THead = Tile<QT_BF16, H, HEADR / 4>;
__device__ __forceinline__ int head_phase(const Ctx &c, HeadLds &s, const THead &th, int step, bool last) {
    const RArgs &a = c.a;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int par = step & 1;
    const unsigned tag = c.tag0 + (unsigned)step;
    {
        uint4 v[2];
        const unsigned base = (c.blk(par, c.L - 1) + R_X) * 4u;
        RS_MARK(step, c.L, 0);
        wait16<2, 8>(c.rr, H / 4, [&](int i) { return base + (unsigned)i * 16u; }, v, a.err);
        RS_MARK(step, c.L, 1);
#pragma unroll
        for (int k = 0; k < 2; k++) put4<8, H>(s.x, 4 * (tid + NT * k), v[k]);
    }
    __syncthreads();
    stage_norm<QT_BF16, H>(s.x, s.gain, a.eps, s.xn);
    if (last && c.hc == 0)
        for (int i = tid; i < H; i += NT) { a.hid[i] = s.xn[xpos<8, H>(i)]; a.decx[i] = s.x[xpos<8, H>(i)]; }
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    if (a.with_head) {
        float acc[HEADR / 4];
        tile_dot<QT_BF16, H, HEADR / 4>(th, s.xn, acc);
        const int frame = c.frame0 + step;
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < HEADR / 4; r++) {
                const int i = c.hc * HEADR + wave * (HEADR / 4) + r;
                float v = fminf(fmaxf(acc[r], -100.0f), 100.0f);
                if (i >= 2048 && i != 2150) v = -1e30f;
                if (i == 2150 && frame < 2) v = -1e30f;
                if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
            }
            s.wbv[wave] = bv; s.wbi[wave] = bi;
        }
        __syncthreads();
        bv = s.wbv[0]; bi = s.wbi[0];
        for (int w = 1; w < 4; w++)
            if (s.wbv[w] > bv || (s.wbv[w] == bv && s.wbi[w] < bi)) { bv = s.wbv[w]; bi = s.wbi[w]; }
    }
    // every store of this workgroup (the clears of the previous step's region among them)
    // is performed before the winner is visible: they are agent-scope (write-through)
    // stores, so their acknowledgements are the release (a release fence would also write
    // back the XCD's whole L2, several microseconds)
    land();
    __syncthreads();
    unsigned long long *slots = a.slots + (size_t)par * NHEAD * 2;
    if (tid == 0) {
        st_tag(slots + 2 * c.hc, bv, tag);
        st_tag(slots + 2 * c.hc + 1, __int_as_float(bi), tag);
    }
    RS_MARK(step, c.L, 2);
    gather<2, NT>(2 * NHEAD, [&](int i) { return slots + i; }, s.win, tag, a.err);
    RS_MARK(step, c.L, 4);
    float gv = -INFINITY;
    int gi = 0x7FFFFFFF;
    for (int i = tid; i < NHEAD; i += NT) {
        const float v = s.win[2 * i];
        const int ix = __float_as_int(s.win[2 * i + 1]);
        if (v > gv || (v == gv && ix < gi)) { gv = v; gi = ix; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(gv, o, 64);
        const int oi = __shfl_xor(gi, o, 64);
        if (ov > gv || (ov == gv && oi < gi)) { gv = ov; gi = oi; }
    }
    __syncthreads();
    if (lane == 0) { s.wbv[wave] = gv; s.wbi[wave] = gi; }
    __syncthreads();
    gv = s.wbv[0]; gi = s.wbi[0];
    for (int w = 1; w < 4; w++)
        if (s.wbv[w] > gv || (s.wbv[w] == gv && s.wbi[w] < gi)) { gv = s.wbv[w]; gi = s.wbi[w]; }
    if (gi < 0 || gi >= a.vocab) gi = 0;
    if (a.with_head && c.hc == 0 && tid == 0) a.hist[(c.frame0 + step) % a.hist_len] = gi;
    __syncthreads();
    if (last)   // every read of this step's region is done (all of them precede the winners)
        for (int l = 0; l < c.L; l++) clear_share(c, par, l);
    return a.with_head ? gi : -1;
}

// ---- Q: q|k|v rows ------------------------------------------------------------------------
__device__ __forceinline__ void role_q(const Ctx &c, LdsP &s, int grp, int qi) {
    const RArgs &a = c.a;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row0 = qi < 2 ? (2 * grp + qi) * HD : qi == 2 ? QD + grp * HD : QD + KVD + grp * HD;
    const int rw = row0 + wave * 32;
    RTile<H, 8> t;
    float rs = 0.f;
    auto load = [&](int l) {
        t.load(c.ly[l].w[0], rw, 8);
        if (lane < 32) rs = ldg(uni(c.ly[l].s[0]) + rw + lane);
        load_gains<4, 16, H>(c.ly[l].in_norm, s.gain);
    };
    THead th;
    load_gains<4, 8, H>(a.final_norm, s.hd.gain);
    load(0);
    land();
    int tok = -1;
    for (int step = 0; step < a.n_steps; step++) {
        const int par = step & 1;
        const bool last = step + 1 == a.n_steps;
        for (int l = 0; l < c.L; l++) {
            float xv[8];
            if (l == 0) {
#pragma unroll
                for (int k = 0; k < 8; k++) xv[k] = x0_elem(a, tok, tid + NT * k);
            } else {
                unsigned v[8];
                const unsigned base = (c.blk(par, l - 1) + R_X) * 4u;
                RS_MARK(step, l, 0);
                wait4<8, 32>(c.rr, H, [&](int i) { return base + (unsigned)i * 4u; }, v, a.err);
                RS_MARK(step, l, 1);
#pragma unroll
                for (int k = 0; k < 8; k++) xv[k] = __uint_as_float(v[k]);
            }
#pragma unroll
            for (int k = 0; k < 8; k++) s.x[xpos<16, H>(tid + NT * k)] = xv[k];
            __syncthreads();   // the gains' LDS copy has landed for every wave (land() before)
            pc_stats<8, NT>(xv, H, s.gain, PosChunk<16, H>(), s.wst);
            __syncthreads();
            const float sA = stage_norm_pc<true, H, NT>(s.x, s.gain, a.eps, s.pc, s.wst);
            RS_MARK(step, l, 6);
            i32x4 acc[8];
            rdot<H, 8>(t, s.pc, 8, acc);
            RS_MARK(step, l, 7);
            int *red = s.red[wave];
#pragma unroll
            for (int q = 0; q < 8; q++) mf_store4(acc[q], red + q * 64);
            if (lane < 32) {
                int d[4];
                mf_rowsum(red + (lane >> 2) * 64, lane & 3, d);
                put(c.wp(par, l, R_QKV + rw + lane), __fmul_rn(qt_pc_dot(d[0], d[1], d[2], d[3], sA), rs));
            }
            RS_MARK(step, l, 2);
            if (step > 0) clear_share(c, par ^ 1, l);
            __syncthreads();   // the tile registers and the gains buffer are free
            if (l + 1 < c.L) load(l + 1);
            else if (!last) load(0);
            land();
            RS_MARK(step, l, 3);
        }
        // the codec-head tile is loaded here, not inside the layer loop, so that its
        // registers are live only for the head
        if (a.with_head) th.load(a.head_w, nullptr, c.hc * HEADR + wave * (HEADR / 4));
        land();
        tok = head_phase(c, s.hd, th, step, last);
    }
    if (c.hc == 0) {   // workgroup 0: position / frame / tag advance, next launch's input
        if (a.with_head)
            for (int i = tid; i < H; i += NT) a.xin[i] = bf16f(ldg(a.emb + (size_t)tok * H + i));
        if (tid == 0) {
            *a.d_pos = c.pos0 + a.n_steps;
            if (a.with_head) *a.d_frame = c.frame0 + a.n_steps;
            *a.epoch = c.tag0 + (unsigned)a.n_steps;
        }
    }
}

// ---- O: xa = x + W_o . attn -------------------------------------------------------------
// Thread t holds attention outputs 8t .. 8t+7 (16-byte groups 2t, 2t+1) and makes their
// pieces straight from registers (the values, scale and order of stage_pc).
__device__ __forceinline__ void role_o(const Ctx &c, LdsP &s, int oi) {
    const RArgs &a = c.a;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row0 = oi * OROWS, rw = row0 + wave * 32;
    RTile<QD, 8> t;
    float rs = 0.f;
    auto load = [&](int l) {
        t.load(c.ly[l].w[1], rw, 8);
        if (lane < 32) rs = ldg(uni(c.ly[l].s[1]) + rw + lane);
    };
    THead th;
    load_gains<4, 8, H>(a.final_norm, s.hd.gain);
    load(0);
    land();
    int tok = -1;
    for (int step = 0; step < a.n_steps; step++) {
        const int par = step & 1;
        const bool last = step + 1 == a.n_steps;
        for (int l = 0; l < c.L; l++) {
            // attn (2048) and, after layer 0, the residual rows of x (128)
            uint4 v[3];
            {
                const unsigned ba = (c.blk(par, l) + R_ATT) * 4u;
                const unsigned bx = l > 0 ? (c.blk(par, l - 1) + R_X + row0) * 4u : 0u;
                const int n16 = QD / 4 + (l > 0 ? OROWS / 4 : 0);
                RS_MARK(step, l, 0);
                wait16<3, 8>(c.rr, n16, [&](int i) {
                    return i < QD / 4 ? ba + (unsigned)(2 * (i % NT) + i / NT) * 16u : bx + (unsigned)(i - QD / 4) * 16u;
                }, v, a.err);
                RS_MARK(step, l, 1);
            }
            float m = 0.f;
#pragma unroll
            for (int k = 0; k < 2; k++)
                m = fmaxf(m, fmaxf(fmaxf(fabsf(__uint_as_float(v[k].x)), fabsf(__uint_as_float(v[k].y))),
                                   fmaxf(fabsf(__uint_as_float(v[k].z)), fabsf(__uint_as_float(v[k].w)))));
            if (l > 0 && tid < OROWS / 4)
                *reinterpret_cast<float4 *>(s.resid + 4 * tid) = make_float4(
                    __uint_as_float(v[2].x), __uint_as_float(v[2].y), __uint_as_float(v[2].z), __uint_as_float(v[2].w));
            if (l == 0 && tid < OROWS) s.resid[tid] = x0_elem(a, tok, row0 + tid);
            m = group_max<64>(m);
            if (lane == 0) s.wst[wave] = m;
            __syncthreads();
            const QtPcScale ps = qt_pc_scale(fmaxf(fmaxf(s.wst[0], s.wst[1]), fmaxf(s.wst[2], s.wst[3])));
            {
                const float v8[8] = {__uint_as_float(v[0].x), __uint_as_float(v[0].y), __uint_as_float(v[0].z),
                                     __uint_as_float(v[0].w), __uint_as_float(v[1].x), __uint_as_float(v[1].y),
                                     __uint_as_float(v[1].z), __uint_as_float(v[1].w)};
                pc_put8<true, QD>(s.pc, tid, v8, ps.isc);
            }
            __syncthreads();
            RS_MARK(step, l, 6);
            i32x4 acc[8];
            rdot<QD, 8>(t, s.pc, 8, acc);
            RS_MARK(step, l, 7);
            int *red = s.red[wave];
#pragma unroll
            for (int q = 0; q < 8; q++) mf_store4(acc[q], red + q * 64);
            if (lane < 32) {
                int d[4];
                mf_rowsum(red + (lane >> 2) * 64, lane & 3, d);
                const float vv = __fmul_rn(qt_pc_dot(d[0], d[1], d[2], d[3], ps.s), rs);
                put(c.wp(par, l, R_XA + rw + lane), __fadd_rn(s.resid[wave * 32 + lane], vv));
            }
            RS_MARK(step, l, 2);
            if (step > 0) clear_share(c, par ^ 1, l);
            __syncthreads();
            if (l + 1 < c.L) { load(l + 1); land(); }
            RS_MARK(step, l, 3);
        }
        if (a.with_head) th.load(a.head_w, nullptr, c.hc * HEADR + wave * (HEADR / 4));
        land();
        tok = head_phase(c, s.hd, th, step, last);
        if (last) break;   // (so the compiler sees the tile below as the next step's only value)
        load(0);
        land();
    }
}

// ---- GU: h = SwiGLU(W_gu . RMSNorm(xa)) ---------------------------------------------------
__device__ __forceinline__ void role_gu(const Ctx &c, LdsP &s, int gi) {
    const RArgs &a = c.a;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rw = gi * GROWS + wave * 32;
    RTile<H, 8> t;
    float rsg = 0.f, rsu = 0.f;
    auto load = [&](int l) {
        t.load(c.ly[l].w[2], rw, 8);
        if (lane < 16) { const float *S = uni(c.ly[l].s[2]); rsg = ldg(S + rw + 2 * lane); rsu = ldg(S + rw + 2 * lane + 1); }
        load_gains<4, 16, H>(c.ly[l].post_norm, s.gain);
    };
    THead th;
    load_gains<4, 8, H>(a.final_norm, s.hd.gain);
    load(0);
    land();
    for (int step = 0; step < a.n_steps; step++) {
        const int par = step & 1;
        const bool last = step + 1 == a.n_steps;
        for (int l = 0; l < c.L; l++) {
            float xv[8];
            {
                unsigned v[8];
                const unsigned base = (c.blk(par, l) + R_XA) * 4u;
                RS_MARK(step, l, 0);
                wait4<8, 32>(c.rr, H, [&](int i) { return base + (unsigned)i * 4u; }, v, a.err);
                RS_MARK(step, l, 1);
#pragma unroll
                for (int k = 0; k < 8; k++) { xv[k] = __uint_as_float(v[k]); s.x[xpos<16, H>(tid + NT * k)] = xv[k]; }
            }
            __syncthreads();
            pc_stats<8, NT>(xv, H, s.gain, PosChunk<16, H>(), s.wst);
            __syncthreads();
            const float sD = stage_norm_pc<true, H, NT>(s.x, s.gain, a.eps, s.pc, s.wst);
            RS_MARK(step, l, 6);
            i32x4 acc[8];
            rdot<H, 8>(t, s.pc, 8, acc);
            RS_MARK(step, l, 7);
            int *red = s.red[wave];
#pragma unroll
            for (int q = 0; q < 8; q++) mf_store4(acc[q], red + q * 64);
            if (lane < 16) {
                // h element p of the wave: gate row 2p, up row 2p + 1 (quad p/2, rows 2(p%2), +1)
                int dg[4], du[4];
                mf_rowsum(red + (lane >> 1) * 64, 2 * (lane & 1), dg);
                mf_rowsum(red + (lane >> 1) * 64, 2 * (lane & 1) + 1, du);
                const float gt = __fmul_rn(qt_pc_dot(dg[0], dg[1], dg[2], dg[3], sD), rsg);
                const float up = __fmul_rn(qt_pc_dot(du[0], du[1], du[2], du[3], sD), rsu);
                put(c.wp(par, l, R_H + rw / 2 + lane), gt / (1.0f + expf(-gt)) * up);
            }
            RS_MARK(step, l, 2);
            if (step > 0) clear_share(c, par ^ 1, l);
            __syncthreads();
            if (l + 1 < c.L) { load(l + 1); land(); }
            RS_MARK(step, l, 3);
        }
        if (a.with_head) th.load(a.head_w, nullptr, c.hc * HEADR + wave * (HEADR / 4));
        land();
        head_phase(c, s.hd, th, step, last);
        if (last) break;   // (so the compiler sees the tile below as the next step's only value)
        load(0);
        land();
    }
}

// ---- DN: x' = xa + W_dn . h ---------------------------------------------------------------
// Row quads 0 and 1 of a wave's rows in registers, quad 2 (when the wave has one) in LDS,
// copied there straight from memory.  Thread t holds h values 8u .. 8u+7 for u = t + 256k
// and makes their pieces from registers (the values, scale and order of stage_pc).
__device__ __forceinline__ void role_dn(const Ctx &c, LdsD &s, int di) {
    const RArgs &a = c.a;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m16 = lane & 15, kg = lane >> 4;
    // 16 workgroups of 48 rows (12 per wave), 32 of 40 (12, 12, 8, 8)
    const bool big = di < 16;
    const int row0 = big ? 48 * di : 768 + 40 * (di - 16);
    const int nrows = big ? 48 : 40;
    const int woff = wave < 3 ? 12 * wave : (big ? 36 : 32);
    const int nq = (big || wave < 2) ? 3 : 2;
    const int rw = row0 + woff;
    constexpr int S = F / 256;
    RTile<F, 2> t;
    float rs = 0.f;
    auto load = [&](int l) {
        t.load(c.ly[l].w[3], rw, 2);
        if (nq > 2) {
            const __amdgpu_buffer_rsrc_t r = brsrc(uni(c.ly[l].w[3]));
            const unsigned voff = (unsigned)((m16 & 3) * F + (m16 >> 2) * 64 + kg * 16);
#pragma unroll
            for (int st = 0; st < S; st++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)&s.tw[wave][st][0], 16,
                                                         voff, __builtin_amdgcn_readfirstlane((rw + 8) * F + st * 256), 0, 0);
        }
        if (lane < 4 * nq) rs = ldg(uni(c.ly[l].s[3]) + rw + lane);
    };
    THead th;
    load_gains<4, 8, H>(a.final_norm, s.hd.gain);
    load(0);
    land();
    for (int step = 0; step < a.n_steps; step++) {
        const int par = step & 1;
        const bool last = step + 1 == a.n_steps;
        for (int l = 0; l < c.L; l++) {
            uint4 v[7];
            {
                const unsigned bh = (c.blk(par, l) + R_H) * 4u, bx = (c.blk(par, l) + R_XA + row0) * 4u;
                const int n16 = F / 4 + nrows / 4;
                RS_MARK(step, l, 0);
                wait16<7, 16>(c.rr, n16, [&](int i) {
                    if (i >= F / 4) return bx + (unsigned)(i - F / 4) * 16u;
                    const int j = i / NT;                       // slot: unit tid + NT*(j/2), half j%2
                    return bh + (unsigned)(2 * (i % NT + NT * (j >> 1)) + (j & 1)) * 16u;
                }, v, a.err);
                RS_MARK(step, l, 1);
            }
            float m = 0.f;
#pragma unroll
            for (int k = 0; k < 6; k++)
                m = fmaxf(m, fmaxf(fmaxf(fabsf(__uint_as_float(v[k].x)), fabsf(__uint_as_float(v[k].y))),
                                   fmaxf(fabsf(__uint_as_float(v[k].z)), fabsf(__uint_as_float(v[k].w)))));
            if (tid < nrows / 4)
                *reinterpret_cast<float4 *>(s.resid + 4 * tid) = make_float4(
                    __uint_as_float(v[6].x), __uint_as_float(v[6].y), __uint_as_float(v[6].z), __uint_as_float(v[6].w));
            m = group_max<64>(m);
            if (lane == 0) s.wst[wave] = m;
            __syncthreads();
            const QtPcScale ps = qt_pc_scale(fmaxf(fmaxf(s.wst[0], s.wst[1]), fmaxf(s.wst[2], s.wst[3])));
#pragma unroll
            for (int k = 0; k < 3; k++) {
                const float v8[8] = {__uint_as_float(v[2 * k].x), __uint_as_float(v[2 * k].y), __uint_as_float(v[2 * k].z),
                                     __uint_as_float(v[2 * k].w), __uint_as_float(v[2 * k + 1].x), __uint_as_float(v[2 * k + 1].y),
                                     __uint_as_float(v[2 * k + 1].z), __uint_as_float(v[2 * k + 1].w)};
                pc_put8<true, F>(s.pc, tid + NT * k, v8, ps.isc);
            }
            __syncthreads();
            RS_MARK(step, l, 6);
            // quads 0, 1 from registers, quad 2 from LDS; two accumulator chains each
            i32x4 acc[3][2];
#pragma unroll
            for (int q = 0; q < 3; q++) acc[q][0] = acc[q][1] = i32x4{0, 0, 0, 0};
            {
                uint4 b = mf_b4<F>(s.pc, 0);
                uint4 w2 = nq > 2 ? s.tw[wave][0][lane] : make_uint4(0, 0, 0, 0);
#pragma unroll
                for (int st = 0; st < S; st++) {
                    const uint4 bn = mf_b4<F>(s.pc, st + 1 < S ? st + 1 : st);
                    const uint4 w2n = nq > 2 ? s.tw[wave][st + 1 < S ? st + 1 : st][lane] : make_uint4(0, 0, 0, 0);
                    acc[0][st & 1] = mfma_i8(t.w[0][st], b, acc[0][st & 1]);
                    acc[1][st & 1] = mfma_i8(t.w[1][st], b, acc[1][st & 1]);
                    if (nq > 2) acc[2][st & 1] = mfma_i8(w2, b, acc[2][st & 1]);
                    b = bn;
                    w2 = w2n;
                }
            }
            RS_MARK(step, l, 7);
            int *red = s.red[wave];
#pragma unroll
            for (int q = 0; q < 3; q++)
                if (q < nq) mf_store4(acc[q][0] + acc[q][1], red + q * 64);
            if (lane < 4 * nq) {
                int d[4];
                mf_rowsum(red + (lane >> 2) * 64, lane & 3, d);
                const float vv = __fmul_rn(qt_pc_dot(d[0], d[1], d[2], d[3], ps.s), rs);
                const float xo = __fadd_rn(s.resid[woff + lane], vv);
                put(c.wp(par, l, R_X + rw + lane), xo);
                if (a.layer_out && last) a.layer_out[(size_t)l * H + rw + lane] = xo;
            }
            RS_MARK(step, l, 2);
            if (step > 0) clear_share(c, par ^ 1, l);
            __syncthreads();
            if (l + 1 < c.L) { load(l + 1); land(); }
            RS_MARK(step, l, 3);
        }
        if (a.with_head) th.load(a.head_w, nullptr, c.hc * HEADR + wave * (HEADR / 4));
        land();
        head_phase(c, s.hd, th, step, last);
        if (last) break;   // (so the compiler sees the tile below as the next step's only value)
        load(0);
        land();
    }
}

// ---- ATT + MRG -----------------------------------------------------------------------------
__device__ __forceinline__ void role_att(const Ctx &c, LdsA &s, int g, int ch) {
    const RArgs &a = c.a;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kg = lane >> 4, key = lane & 15;
    uint4 kf[ABLK][8];            // key rows of the chunk: block b, this wave's k-tile, [score tile][dim step]
    float qn0 = 0.f, qn1 = 0.f, kn0 = 0.f, kn1 = 0.f, rc = 0.f, rsn = 0.f;
    // K rows (registers, MFMA B-operand layout) and V rows (LDS) of layer lk's chunk
    // under geometry ge; row ge.pos is never loaded (it is this step's append)
    auto prefetch = [&](int lk, const Geo &ge) {
        const int j0 = ch * ge.CH, n = ch < ge.nch ? min(ge.CH, ge.pos + 1 - j0) : 0;
        const uint16_t *Kl = a.kc + (((size_t)lk * NKV + g) * a.kv_max) * HD;
        const uint16_t *Vl = a.vc + (((size_t)lk * NKV + g) * a.kv_max) * HD;
#pragma unroll
        for (int b = 0; b < ABLK; b++) {
            if (128 * b >= n) break;
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++) {
                const int jj = 128 * b + 32 * wave + 16 * t2 + key;
                const bool ok = jj < n && j0 + jj != ge.pos;
                const uint16_t *kr = Kl + (size_t)(j0 + (ok ? jj : 0)) * HD + 8 * kg;
#pragma unroll
                for (int s2 = 0; s2 < 4; s2++)
                    kf[b][t2 * 4 + s2] = ok ? ldg(reinterpret_cast<const uint4 *>(kr + 32 * s2)) : make_uint4(0, 0, 0, 0);
            }
            const int nk = min(KVB, n - 128 * b);
            const int ninst = (nk + 3) >> 2;
            for (int i = wave; i < ninst; i += 4) {
                const int jl = i * 4 + kg, jj = 128 * b + jl;
                if (jj < n && j0 + jj != ge.pos)
                    lds_copy16(Vl + (size_t)(j0 + jj) * HD + qt_vslot(jl, key) * 8, &s.v[b][i * 4 * HD]);
            }
        }
        const float *qnp = uni(c.ly[lk].qn), *knp = uni(c.ly[lk].kn);
        qn0 = ldg(qnp + lane); qn1 = ldg(qnp + lane + 64); kn0 = ldg(knp + lane); kn1 = ldg(knp + lane + 64);
        rc = ldg(a.rope_cos + (size_t)ge.pos * 64 + lane); rsn = ldg(a.rope_sin + (size_t)ge.pos * 64 + lane);
    };
    qt_att_zero_rows<HPK>(&s.qp[0][0], HD, tid, NT);
    qt_att_zero_rows<HPK>(&s.pp[0][0][0], KVB, tid, NT);
    qt_att_zero_rows<HPK>(&s.pp[1][0][0], KVB, tid, NT);
    prefetch(0, Geo(c.pos0));
    land();
    const float scale2 = a.scale * QT_LOG2E;
    for (int step = 0; step < a.n_steps; step++) {
        const int par = step & 1;
        const bool last = step + 1 == a.n_steps;
        const Geo ge(c.pos0 + step);
        const int pos = ge.pos;
        const int j0 = ch * ge.CH, n = ch < ge.nch ? min(ge.CH, pos + 1 - j0) : 0;
        const int nblk = (n + KVB - 1) / KVB;
        const bool append = n > 0 && pos >= j0 && pos < j0 + n;
        for (int l = 0; l < c.L; l++) {
            // ---------------- attention chunk -----------------
            if (n > 0) {
                {
                    uint4 v[1];
                    const unsigned bq = c.blk(par, l) * 4u;
                    RS_MARK(step, l, 0);
                    wait16<1, 0>(c.rr, (HPK * HD + 2 * HD) / 4, [&](int i) {
                        const int w = i < 64 ? R_QKV + HPK * HD * g + 4 * i
                                    : i < 96 ? R_QKV + QD + HD * g + 4 * (i - 64) : R_QKV + QD + KVD + HD * g + 4 * (i - 96);
                        return bq + (unsigned)w * 4u;
                    }, v, a.err);
                    RS_MARK(step, l, 1);
                    if (tid < (HPK * HD + 2 * HD) / 4)
                        *reinterpret_cast<float4 *>(s.qkv + 4 * tid) = make_float4(
                            __uint_as_float(v[0].x), __uint_as_float(v[0].y), __uint_as_float(v[0].z), __uint_as_float(v[0].w));
                }
                __syncthreads();
                const int ntask = HPK + (append ? 1 : 0);
                for (int tk = wave; tk < ntask; tk += 4) {
                    const bool isk = (tk == HPK);
                    const float *srcv = isk ? s.qkv + HPK * HD : s.qkv + tk * HD;
                    const float w0 = isk ? kn0 : qn0, w1 = isk ? kn1 : qn1;
                    const float x0 = srcv[lane], x1 = srcv[lane + 64];
                    const float ss = group_sum<64>(x0 * x0 + x1 * x1);
                    const float inv = 1.0f / sqrtf(ss / (float)HD + a.eps);
                    const float n0 = (x0 * inv) * w0, n1 = (x1 * inv) * w1;
                    const float r0 = fmaf(n0, rc, -(n1 * rsn)), r1 = fmaf(n1, rc, n0 * rsn);
                    if (!isk) {
                        qt_put_pieces(&s.qp[4 * tk][lane], HD, r0);
                        qt_put_pieces(&s.qp[4 * tk][lane + 64], HD, r1);
                    } else {
                        const float *vs = s.qkv + HPK * HD + HD;
                        const uint16_t k0 = f2bf_trunc(r0), k1 = f2bf_trunc(r1);
                        const uint16_t v0 = f2bf_trunc(vs[lane]), v1 = f2bf_trunc(vs[lane + 64]);
                        s.knew[lane] = k0; s.knew[lane + 64] = k1;
                        s.vnew[lane] = v0; s.vnew[lane + 64] = v1;
                        const int r = pos - j0;
                        s.v[r / KVB][qt_vidx(r % KVB, lane)] = v0;
                        s.v[r / KVB][qt_vidx(r % KVB, lane + 64)] = v1;
                    }
                }
                {   // value rows past the chunk end in its last block: probabilities 0, stale bits could be NaN
                    const int nkl = n - KVB * (nblk - 1);
                    qt_att_zero_vrows(s.v[nblk - 1], nkl, (nkl + 31) & ~31, tid, NT);
                }
                __syncthreads();
                if (append) {   // the appended key into the registers of the wave whose k-tile holds it
                    const int r = pos - j0, rb = r / KVB, rr = r % KVB;
                    if (wave == rr / 32 && key == (rr & 15)) {
                        const int t2 = (rr & 31) >> 4;
#pragma unroll
                        for (int b = 0; b < ABLK; b++)
#pragma unroll
                            for (int tt = 0; tt < 2; tt++)
                                if (b == rb && tt == t2)
#pragma unroll
                                    for (int s2 = 0; s2 < 4; s2++)
                                        kf[b][tt * 4 + s2] = *reinterpret_cast<const uint4 *>(s.knew + 32 * s2 + 8 * kg);
                    }
                }
                RS_MARK(step, l, 6);
                QtAttRun run;
                qt_att_run_init(run);
#pragma unroll
                for (int b = 0; b < ABLK; b++) {
                    if (b >= nblk) break;
                    const int nk = min(KVB, n - KVB * b);
                    uint16_t *pp = &s.pp[b & 1][0][0];
                    float *ml = &s.ml[b & 1][0][0][0];
                    if (32 * wave < nk) {
                        // scores of k-tile `wave` (two 16-key score tiles) against the query
                        // pieces: qt_att_tiles with the key rows from registers
                        qt_u32x4 qa[4];
#pragma unroll
                        for (int s2 = 0; s2 < 4; s2++) qa[s2] = qt_lds16(&s.qp[key][32 * s2 + 8 * kg]);
                        float sv[2];
#pragma unroll
                        for (int t2 = 0; t2 < 2; t2++) {
                            qt_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                            for (int s2 = 0; s2 < 4; s2++) {
                                const uint4 kk = kf[b][t2 * 4 + s2];
                                acc = qt_mfma_bf16(qa[s2], qt_u32x4{kk.x, kk.y, kk.z, kk.w}, acc);
                            }
                            sv[t2] = (acc[0] + acc[1]) + acc[2];
                        }
                        const int hh = lane >> 4;
                        const int r00 = 32 * wave, r01 = 32 * wave + 16;
                        const float sa = r00 + key < nk ? sv[0] * scale2 : -INFINITY;
                        const float sb = r01 + key < nk ? sv[1] * scale2 : -INFINITY;
                        const float m = group_max<16>(fmaxf(sa, sb));
                        const float pa = qt_exp2(sa - m), pb = qt_exp2(sb - m);
                        const float ls = group_sum<16>(pa + pb);
                        if (hh < HPK) {
                            qt_put_pieces(pp + 4 * hh * KVB + r00 + key, KVB, pa);
                            qt_put_pieces(pp + 4 * hh * KVB + r01 + key, KVB, pb);
                            if (key == 0) { ml[(wave * HPK + hh) * 2] = m; ml[(wave * HPK + hh) * 2 + 1] = ls; }
                        }
                    }
                    __syncthreads();
                    float o[2], M, lsum;
                    qt_att_pv_n<HPK>((nk + 31) >> 5, pp, KVB, ml, s.v[b], 32 * wave, lane, o, M, lsum);
                    qt_att_run_add(run, o, M, lsum);
                }
                RS_MARK(step, l, 7);
                // partial of this chunk: o (head lane/16, dims 32 wave + lane%16 and +16), m, l
                const int hq = lane >> 4;
                if (hq < HPK) {
                    const int ob = R_PO + (((g * HPK + hq) * 4 + wave) * ACH + ch) * 32 + key;
                    put(c.wp(par, l, ob), run.o[0]);
                    put(c.wp(par, l, ob + 16), run.o[1]);
                    if (wave == 0 && key == 0) {
                        put(c.wp(par, l, R_PML + ((g * HPK + hq) * ACH + ch) * 2), run.m);
                        put(c.wp(par, l, R_PML + ((g * HPK + hq) * ACH + ch) * 2 + 1), run.l);
                    }
                }
                RS_MARK(step, l, 2);
                if (append && wave == 3) {
                    // KV append: agent-scope 32-bit stores of adjacent bf16 pairs
                    uint32_t *kd = reinterpret_cast<uint32_t *>(a.kc + (((size_t)l * NKV + g) * a.kv_max + pos) * HD);
                    uint32_t *vd = reinterpret_cast<uint32_t *>(a.vc + (((size_t)l * NKV + g) * a.kv_max + pos) * HD);
                    const uint32_t kk = (uint32_t)s.knew[2 * lane] | ((uint32_t)s.knew[2 * lane + 1] << 16);
                    const uint32_t vv = (uint32_t)s.vnew[2 * lane] | ((uint32_t)s.vnew[2 * lane + 1] << 16);
                    __hip_atomic_store(kd + lane, kk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(vd + lane, vv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            // ---------------- merge: head 2g + ch/4, dims 32 (ch % 4) .. +31 -----------------
            {
                const int hh = ch >> 2, dblk = ch & 3;
                const int nch = ge.nch;
                {
                    uint4 v[1];
                    const unsigned bo = (c.blk(par, l) + R_PO + ((g * HPK + hh) * 4 + dblk) * ACH * 32) * 4u;
                    wait16<1, 0>(c.rr, 8 * nch, [&](int i) { return bo + (unsigned)i * 16u; }, v, a.err);
                    unsigned long long mlw = 0;
                    if (tid >= 64 && tid < 64 + nch) {
                        const unsigned long long *p = reinterpret_cast<const unsigned long long *>(
                            c.wp(par, l, R_PML + ((g * HPK + hh) * ACH + (tid - 64)) * 2));
                        mlw = ld_w(p);
                        for (unsigned it = 0; (unsigned)mlw == SENT || (unsigned)(mlw >> 32) == SENT; it++) {
                            if ((it & 31) == 31) {
                                if (ld_i(a.err)) break;
                                if (it > POLL_LIMIT) { st_i(a.err, 1); break; }
                            }
                            __builtin_amdgcn_s_sleep(1);
                            mlw = ld_w(p);
                        }
                        s.mml[tid - 64][0] = __uint_as_float((unsigned)mlw);
                        s.mml[tid - 64][1] = __uint_as_float((unsigned)(mlw >> 32));
                    }
                    if (tid < 8 * nch)
                        *reinterpret_cast<float4 *>(&s.mo[tid >> 3][4 * (tid & 7)]) = make_float4(
                            __uint_as_float(v[0].x), __uint_as_float(v[0].y), __uint_as_float(v[0].z), __uint_as_float(v[0].w));
                }
                __syncthreads();
                RS_MARK(step, l, 4);
                // output d = tid / 8 over the chunks cc = tid % 8: softmax_merge32 over 32
                // lanes with lanes >= nch idle adds exact zeros after the 8-lane tree, so the
                // 8-lane tree plus one +0 gives the same bits
                const int d = tid >> 3, cc = tid & 7;
                const bool valid = cc < nch;
                const float m = valid ? s.mml[cc][0] : 0.f, lw = valid ? s.mml[cc][1] : 0.f, ow = valid ? s.mo[cc][d] : 0.f;
                float M = valid ? m : -INFINITY;
                M = fmaxf(M, dpp_mov_keep<DPP_QXOR1>(M));
                M = fmaxf(M, dpp_mov_keep<DPP_QXOR2>(M));
                M = fmaxf(M, dpp_mov_keep<DPP_HALF_MIRROR>(M));
                const float f = valid ? __builtin_amdgcn_exp2f(m - M) : 0.f;
                float Ls = valid ? lw * f : 0.f, Vs = valid ? ow * f : 0.f;
                Ls += dpp_mov<DPP_QXOR1>(Ls); Vs += dpp_mov<DPP_QXOR1>(Vs);
                Ls += dpp_mov<DPP_QXOR2>(Ls); Vs += dpp_mov<DPP_QXOR2>(Vs);
                Ls += dpp_mov<DPP_HALF_MIRROR>(Ls); Vs += dpp_mov<DPP_HALF_MIRROR>(Vs);
                Ls = Ls + 0.0f; Vs = Vs + 0.0f;
                if (cc == 0) put(c.wp(par, l, R_ATT + (2 * g + hh) * HD + 32 * dblk + d), Vs * (1.0f / Ls));
                RS_MARK(step, l, 5);
            }
            __syncthreads();   // the chunk's LDS (values, staging) is free for the next copy
            if (l + 1 < c.L) prefetch(l + 1, ge);
            else if (!last) prefetch(0, Geo(pos + 1));
            land();
            RS_MARK(step, l, 3);
        }
    }
}

__global__ __launch_bounds__(NT, 1) void k_rstep(RArgs a) {
    __shared__ __align__(16) unsigned char lds[LDS_BYTES];
    __shared__ Layer s_layers[MAXLR];
    const int b = blockIdx.x, tid = threadIdx.x;
    const int x = b % 8, slot = b / 8;
    for (int i = tid; i < a.n_layers * (int)(sizeof(Layer) / 8); i += NT)
        reinterpret_cast<unsigned long long *>(s_layers)[i] = ldg(reinterpret_cast<const unsigned long long *>(a.layers) + i);
    __syncthreads();
    int hc = -1;
    if (slot < SA0) hc = (slot - SQ0) * 8 + x;
    else if (slot >= SO0 && slot < SG0) hc = NQ + (slot - SO0) * 8 + x;
    else if (slot >= SG0 && slot < SD0) hc = NQ + NO + (slot - SG0) * 8 + x;
    else if (slot >= SD0) hc = NQ + NO + NG + (slot - SD0) * 8 + x;
    const Ctx c{a, s_layers, brsrc(a.reg), a.n_layers, *a.d_pos, a.with_head ? *a.d_frame : 0, *a.epoch, hc};
    if (slot < SA0) role_q(c, *reinterpret_cast<LdsP *>(lds), x, slot - SQ0);
    else if (slot < SO0) role_att(c, *reinterpret_cast<LdsA *>(lds), x, slot - SA0);
    else if (slot < SG0) role_o(c, *reinterpret_cast<LdsP *>(lds), (slot - SO0) * 8 + x);
    else if (slot < SD0) role_gu(c, *reinterpret_cast<LdsP *>(lds), (slot - SG0) * 8 + x);
    else role_dn(c, *reinterpret_cast<LdsD *>(lds), (slot - SD0) * 8 + x);
}
}  // namespace rs
}  // namespace ps

#ifdef QT_RSTEP_TRACE
extern "C" hipError_t qt_rstep_trace_read(unsigned long long *out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(ps::rs::rs_trace), sizeof(ps::rs::rs_trace), 0, hipMemcpyDeviceToHost);
}
#endif

extern "C" int qt_rstep_supported(int prec, int hidden, int inter, int n_heads, int n_kv, int head_dim, int kv_max,
                                  int n_layers) {
    if (prec != QT_INT8 || hidden != ps::rs::H || inter != ps::rs::F) return 0;
    if (n_heads != ps::NH || n_kv != ps::NKV || head_dim != ps::HD) return 0;
    if (kv_max > ps::rs::ACH * ps::rs::ABLK * ps::KVB || n_layers < 1 || n_layers > ps::rs::MAXLR) return 0;
    int dev = 0, cus = 0, coop = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess) return 0;
    return coop && cus >= ps::NB;
}
// hand-off words (both parities) and winner words
extern "C" size_t qt_rstep_region_words(int n_layers) { return (size_t)2 * n_layers * ps::rs::LW; }
extern "C" size_t qt_rstep_slot_words(void) { return (size_t)2 * ps::rs::NHEAD * 2; }
// attention key chunks per kv head (the per-kernel attention must use the same split)
extern "C" int qt_rstep_chunks(void) { return ps::rs::ACH; }

extern "C" hipError_t qt_launch_rstep(const void *layers_dev, int n_layers, const float *final_norm, const float *rope_cos,
                                      const float *rope_sin, uint16_t *kc, uint16_t *vc, int kv_max, float eps, float scale,
                                      unsigned *reg, unsigned long long *slots, float *hid, float *decx, float *xin,
                                      int *d_pos, unsigned *epoch, int *err, int n_steps, int with_head,
                                      const uint16_t *head_w, const uint16_t *emb, int vocab, int *d_frame, int *hist,
                                      int hist_len, float *layer_out, hipStream_t st) {
    ps::rs::RArgs a;
    a.layers = (const ps::Layer *)layers_dev; a.n_layers = n_layers;
    a.final_norm = final_norm; a.rope_cos = rope_cos; a.rope_sin = rope_sin;
    a.kc = kc; a.vc = vc; a.kv_max = kv_max; a.eps = eps; a.scale = scale;
    a.reg = reg; a.slots = slots; a.hid = hid; a.decx = decx; a.xin = xin; a.d_pos = d_pos; a.epoch = epoch;
    a.err = err; a.n_steps = n_steps; a.with_head = with_head;
    a.head_w = (const uint8_t *)head_w; a.emb = emb; a.vocab = vocab;
    a.d_frame = d_frame; a.hist = hist; a.hist_len = hist_len; a.layer_out = layer_out;
    if (n_steps <= 0 || n_layers <= 0 || n_layers > ps::rs::MAXLR || kv_max > ps::rs::ACH * ps::rs::ABLK * ps::KVB)
        return hipErrorInvalidValue;
    if (!with_head && n_steps != 1) return hipErrorInvalidValue;   // without the head the next input is unknown
    if (with_head && (vocab != ps::rs::NHEAD * ps::rs::HEADR || !head_w || !emb || !d_frame || !hist || hist_len <= 0))
        return hipErrorInvalidValue;
    void *args[] = {(void *)&a};
    return hipLaunchCooperativeKernel((const void *)ps::rs::k_rstep, dim3(ps::NB), dim3(ps::rs::NT), args, 0, st);
}
