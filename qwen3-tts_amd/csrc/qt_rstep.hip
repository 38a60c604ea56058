// qt_rstep.hip — the Talker decode step (16 query / 8 kv heads of 128) as ONE persistent
// cooperative kernel whose workgroups each own ONE phase of the layer.  Built four times:
// the 1.7B geometry with int8 weights (hidden 2048, intermediate 6144; namespace ps::rs,
// entry points qt_rstep_* / qt_launch_rstep); with QT_RS_SMALL (qt_rstep06.hip) the 0.6B
// geometry (hidden 1024, intermediate 3072; ps::rs06, qt_rstep06_*), which has half the O,
// GU and DN workgroups and gives the slots left over to the codec head alone (and runs a
// whole Code Predictor frame as one launch: qt_launch_rstep06_cp); with QT_RS_SMALL and
// QT_RS_BF16 (qt_rstep06b.hip) the 0.6B geometry with bf16 weights (ps::rs06b); with
// QT_RS_Q4 (qt_rstep4.hip) the 1.7B geometry with q4_0 weights (ps::rs4).
//
// Same math as qwen_talker_step (qwen_tts_talker.c:537-699).  With int8 and q4_0 weights
// every output has the per-kernel path's arithmetic (qt_matvec.hip, qt_attn.hip with 8 key
// chunks per kv head), so the two agree to the bit; with bf16 weights the projections sum
// the same exact products in the MFMA's order, so the two agree to f32 rounding.
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
// (0.6B: O slot 12, GU 13..18, DN 19..21 with the same rows per workgroup, 22..31 idle)
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

#if defined(QT_RS_SMALL) && defined(QT_RS_BF16)
#define QT_RS_NS rs06b
#define QT_RS_NAME(a, b) a##06b##b
#elif defined(QT_RS_Q4)
#define QT_RS_NS rs4
#define QT_RS_NAME(a, b) a##4##b
#elif defined(QT_RS_SMALL)
#define QT_RS_NS rs06
#define QT_RS_NAME(a, b) a##06##b
#else
#define QT_RS_NS rs
#define QT_RS_NAME(a, b) a##b
#endif

namespace ps {
namespace QT_RS_NS {
#if defined(QT_RS_SMALL) && defined(QT_RS_BF16)
constexpr int H = 1024, F = 3072, XO = 2, XG = 6, XD = 3;               // bf16 O rows take twice the bytes
#elif defined(QT_RS_SMALL)
constexpr int H = 1024, F = 3072, XO = 1, XG = 6, XD = 3;               // O, GU, DN workgroups per XCD
#else
constexpr int H = 2048, F = 6144, XO = 2, XG = 12, XD = 6;
#endif
constexpr int NT = 256;
constexpr unsigned SENT = 0xFFFFFFFFu;
// Weight type of the build: int8 rows on v_mfma_i32_16x16x64_i8 against four exact int8
// activation planes, or (QT_RS_BF16) bf16 rows on v_mfma_f32_16x16x32_bf16 against three
// exact bf16 planes.  Either way an MFMA step covers 64 bytes of a weight row.
#ifdef QT_RS_BF16
constexpr bool WBF = true;
#else
constexpr bool WBF = false;
#endif
#ifdef QT_RS_Q4
constexpr bool WQ4 = true;                       // q4_0 rows (1.7B geometry only): see QTile16
#else
constexpr bool WQ4 = false;
#endif
constexpr bool RSC = !WBF && !WQ4;               // int8 rows carry a row scale
constexpr int PREC = WBF ? QT_BF16 : WQ4 ? QT_Q4 : QT_INT8;
constexpr int WB = WBF ? 2 : 1;                  // bytes per weight (q4_0: 64 columns per MFMA step too)
constexpr int NPL = WBF ? 3 : 4;                 // activation planes
constexpr int KSTEP = 64 / WB;                   // columns per MFMA step
template <int C> constexpr int steps() { return C * WB / 64; }   // MFMA steps over C columns
constexpr int XQ = 4, XATT = 8, XI = NB / 8 - (XQ + XATT + XO + XG + XD);   // XI: head-only slots
constexpr int SQ0 = 0, SA0 = SQ0 + XQ, SO0 = SA0 + XATT, SG0 = SO0 + XO, SD0 = SG0 + XG, SI0 = SD0 + XD;
static_assert(XI >= 0 && SI0 + XI == NB / 8, "32 workgroups per XCD");
constexpr int NQ = 8 * XQ, NO = 8 * XO, NG = 8 * XG, ND = 8 * XD, NI = 8 * XI;
constexpr int NHEAD = NQ + NO + NG + ND + NI;    // 192: every workgroup but attention
constexpr int ACH = XATT;                        // attention chunks per kv head
constexpr int QROWS = QKVR / NQ, OROWS = H / NO, GROWS = 2 * F / NG;
static_assert(QROWS == 128 && OROWS == 128 / WB && GROWS == 128, "rows per projection workgroup");
constexpr int EH = H / NT;                       // elements of an H-vector per thread (8 or 4)
static_assert(EH == 4 || EH == 8, "H-vector split");
constexpr int UD = F / 768;                      // DN: elements per h unit (three units per lane)
static_assert(UD == 4 || UD == 8, "h split");
constexpr int NDB = (H - 40 * ND) / 8;           // DN workgroups of 48 rows; the others take 40
static_assert(NDB >= 0 && NDB <= ND && 48 * NDB + 40 * (ND - NDB) == H, "DN rows");
constexpr int PCW = H > QD ? H : QD;             // widest input whose pieces LdsP holds
constexpr int HEADR = 3072 / NHEAD;              // codec-head rows per workgroup (16)
constexpr int ABLK = 4;                          // 128-key blocks of a chunk held resident (512 keys)
constexpr int MAXLR = 32;
// words of one layer's hand-off block (padded so that the head workgroups' clear shares
// are equal)
constexpr int R_QKV = 0, R_PO = R_QKV + QKVR, R_PML = R_PO + NKV * HPK * 4 * ACH * 32,
              R_ATT = R_PML + NKV * HPK * ACH * 2, R_XA = R_ATT + QD, R_H = R_XA + H, R_X = R_H + F,
#ifdef QT_RS_SMALL
              R_XIN = R_X + H,           // Code Predictor with the mtp projection: pass input (layer 0's block)
              LW = (R_XIN + H + 4 * NHEAD - 1) / (4 * NHEAD) * (4 * NHEAD);
constexpr int EMB = 2048;                        // mtp projection input (the 1.7B Talker's hidden size)
constexpr int NMTP = H / 16;                     // mtp workgroups (16 rows each, in the head-only slots)
static_assert(NMTP <= NI && NMTP % 8 == 0, "mtp workgroups");
#else
              LW = (R_X + H + 4 * NHEAD - 1) / (4 * NHEAD) * (4 * NHEAD);
#endif
constexpr int CLR16 = LW / (4 * NHEAD);          // 16-byte groups of a layer block each head workgroup clears
static_assert(CLR16 * 4 * NHEAD == LW && CLR16 <= NT, "clear shares");
constexpr int SC1 = 16;                          // buffer cache policy: agent scope (sc1)

// Optional phase trace (build with -DQT_RSTEP_TRACE): s_memrealtime (100 MHz) of each
// workgroup at marks k of (step, layer) — 0 its input wait starts, 1 the input has
// arrived, 2 its output is published, 3 its next tile has landed; attention adds 4 (merge
// input arrived) and 5 (merge output published); layer index L is the head (0 wait starts,
// 1 x arrived, 2 winner published, 4 winners arrived).  Marks 1 and 2 also keep the shader
// clock counter (s_memtime) in slots 13 and 14, and mark 1 of wave w is also kept in slot
// 16 + w.  Steps past TR_STEPS are not kept.
#ifdef QT_RSTEP_TRACE
constexpr int TR_STEPS = 8, TR_L = 33;
__device__ unsigned long long rs_trace[NB][TR_STEPS * TR_L][24];
#define RS_MARK(st, l, k)                                                                             \
    do {                                                                                              \
        if ((st) < TR_STEPS && (k) == 1 && (threadIdx.x & 63) == 0)                                   \
            rs_trace[blockIdx.x][(st) * TR_L + (l)][16 + (threadIdx.x >> 6)] = __builtin_amdgcn_s_memrealtime(); \
        if (threadIdx.x == 0 && (st) < TR_STEPS) {                                                    \
            rs_trace[blockIdx.x][(st) * TR_L + (l)][k] = __builtin_amdgcn_s_memrealtime();            \
            if ((k) == 1 || (k) == 2) rs_trace[blockIdx.x][(st) * TR_L + (l)][12 + (k)] = __builtin_amdgcn_s_memtime(); \
        }                                                                                             \
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
    // Code Predictor frame (0.6B builds only): step s is pass s at position s; the input of
    // pass 0 is xin, of pass s >= 1 row codes[s-1] of table cp_emb[s-1]; after pass s >= 1
    // lm head s-1 (`vocab` rows cp_head[s-1]: int8 with row scales cp_hs[s-1], or bf16) on
    // the final-normed x gives codes[s] (plain argmax, lowest index on ties).  Device arrays
    // of 15 pointers each; codes[0] is the frame's input code.
    int cp;
    const uint8_t *const *cp_head;
    const float *const *cp_hs;
    const uint16_t *const *cp_emb;
    int *cp_codes;
    // with the mtp projection (mtp_w != NULL): every pass input is W.e + b (rows of EMB
    // columns in the build's weight type, int8 with row scales mtp_s; bias), e the table
    // row (EMB wide) or, for pass 0, xin
    const uint8_t *mtp_w;
    const float *mtp_s, *mtp_b;
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
// A wave's LDS accesses complete in program order, so LDS data a wave wrote for itself
// needs no barrier before it reads it back: only the compiler must keep the order.
__device__ __forceinline__ void wave_lds_order() { asm volatile("" ::: "memory"); }

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
    if constexpr (PST > 0) {
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
    if constexpr (PST > 0) {
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

// ---- MFMA row tiles: 16 weight rows x 64 columns per v_mfma_i32_16x16x64_i8 -----------
// A = 16 rows (lane l: row l % 16, columns 16*(l/16) .. +15 of the 64-column step), B =
// the four activation planes of those 64 columns as columns 0..3 (columns 4..15 zero),
// so D[r][n] accumulates the plane-n dot product of row r over the steps: lane l ends
// with rows 4*(l/16) + i (register i) of plane l % 16, and the four planes of a row are
// the four lanes of one quad (DPP quad broadcasts, no LDS round trip).  Exact int32 sums,
// so the values equal every other way of forming the dot products.
//
// Pieces live in plane-major LDS rows of WB*COLS + 16 bytes (the pad puts the planes of
// one column range on different banks).
template <int COLS> constexpr int pcs() { return WB * COLS + 16; }
// unit u: elements E*u .. E*u + E-1 (E = 8 or 4), E elements of each plane (int8: the four
// exact planes of scale isc; bf16: the three exact bf16 planes of qt_put_pieces)
template <int COLS, int E>
__device__ __forceinline__ void pcw_put(uint8_t *pc, int u, const float (&v)[E], float isc) {
    static_assert(E == 8 || E == 4, "unit size");
    if constexpr (WBF) {
        uint16_t p3[3][E];
#pragma unroll
        for (int e = 0; e < E; e++) qt_put_pieces(&p3[0][e], E, v[e]);
#pragma unroll
        for (int q = 0; q < 3; q++) {
            if constexpr (E == 8)
                *reinterpret_cast<uint4 *>(pc + q * pcs<COLS>() + 16 * u) = *reinterpret_cast<const uint4 *>(p3[q]);
            else
                *reinterpret_cast<uint2 *>(pc + q * pcs<COLS>() + 8 * u) = *reinterpret_cast<const uint2 *>(p3[q]);
        }
    } else if constexpr (WQ4) {
        // q4_0: each 16-column group is stored even columns first, then odd ones (the
        // order of a q4_0 byte's low and high nibbles as QTile16's B operand holds them)
        static_assert(E == 8, "q4_0 pieces: 8-element units");
        uint2 pl[4];
        qt_pc8(v, isc, pl);
        const int g = u >> 1, sub = u & 1;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            uint8_t *d = pc + q * pcs<COLS>() + 16 * g + 4 * sub;
            *reinterpret_cast<uint32_t *>(d) = __builtin_amdgcn_perm(pl[q].y, pl[q].x, 0x06040200u);
            *reinterpret_cast<uint32_t *>(d + 8) = __builtin_amdgcn_perm(pl[q].y, pl[q].x, 0x07050301u);
        }
    } else if constexpr (E == 8) {
        uint2 pl[4];
        qt_pc8(v, isc, pl);
#pragma unroll
        for (int q = 0; q < 4; q++) *reinterpret_cast<uint2 *>(pc + q * pcs<COLS>() + 8 * u) = pl[q];
    } else {
        uint32_t pl[4];
        qt_pc_t4(qt_pc_word(v[0], isc), qt_pc_word(v[1], isc), qt_pc_word(v[2], isc), qt_pc_word(v[3], isc), pl);
#pragma unroll
        for (int q = 0; q < 4; q++) *reinterpret_cast<uint32_t *>(pc + q * pcs<COLS>() + 4 * u) = pl[q];
    }
}
// B fragment of columns col0 .. col0 + KSTEP-1 (planes as columns 0 .. NPL-1)
template <int COLS>
__device__ __forceinline__ uint4 pcw_b(const uint8_t *pc, int col0) {
    const int lane = threadIdx.x & 63, n = lane & 15, kg = lane >> 4;
    const uint4 b = *reinterpret_cast<const uint4 *>(pc + (n & 3) * pcs<COLS>() + WB * col0 + 16 * kg);
    return n < NPL ? b : make_uint4(0, 0, 0, 0);
}
// NT16 tiles of 16 rows (row0 + 16t ..) over S 64-column steps from column c0.  Buffer
// loads: one 32-bit lane offset shared by every load, the row and step parts in scalar
// registers (64-bit per-lane addresses would hold two VGPRs per load in flight).  Rows at
// or past row_end are not loaded (their A stays zero).
// NT16 tiles of 16 rows of COLS-wide weight rows (WB bytes each); S MFMA steps of 64 bytes
// from column c0 (elements).
template <int COLS, int NT16, int S>
struct RTile16 {
    uint4 w[NT16][S];
    __device__ __forceinline__ void load(const uint8_t *W, int row0, int c0, int row_end) {
        const int lane = threadIdx.x & 63, m = lane & 15, kg = lane >> 4;
        const __amdgpu_buffer_rsrc_t r = brsrc(uni(W));
        const unsigned voff = (unsigned)(m * WB * COLS + 16 * kg);
#pragma unroll
        for (int t = 0; t < NT16; t++) {
            const bool ok = row0 + 16 * t + m < row_end;
#pragma unroll
            for (int s = 0; s < S; s++) {
                const u32x4_t v = ok ? __builtin_amdgcn_raw_buffer_load_b128(
                                           r, voff, __builtin_amdgcn_readfirstlane(WB * ((row0 + 16 * t) * COLS + c0) + 64 * s), 0)
                                     : u32x4_t{0, 0, 0, 0};
                w[t][s] = make_uint4(v.x, v.y, v.z, v.w);
            }
        }
    }
    __device__ __forceinline__ void load(const uint8_t *W, const uint16_t *, int row0, int c0, int row_end) {
        load(W, row0, c0, row_end);
    }
};
// the build's MFMA: exact int32 plane sums (int8) or f32 sums of exact products (bf16)
using AccT = std::conditional_t<WQ4, float, std::conditional_t<WBF, qt_f32x4, i32x4>>;
using RedT = std::conditional_t<WBF || WQ4, float, int>;
#ifdef QT_RS_BF16
__device__ __forceinline__ AccT mma(uint4 w, uint4 p, AccT acc) {
    return qt_mfma_bf16(qt_u32x4{w.x, w.y, w.z, w.w}, qt_u32x4{p.x, p.y, p.z, p.w}, acc);
}
__device__ __forceinline__ AccT acc_zero() { return qt_f32x4{0.f, 0.f, 0.f, 0.f}; }
#elif defined(QT_RS_Q4)
__device__ __forceinline__ i32x4 mma(uint4 w, uint4 p, i32x4 acc) { return mfma_i8(w, p, acc); }
__device__ __forceinline__ i32x4 acc_zero() { return i32x4{0, 0, 0, 0}; }
#else
__device__ __forceinline__ AccT mma(uint4 w, uint4 p, AccT acc) { return mfma_i8(w, p, acc); }
__device__ __forceinline__ AccT acc_zero() { return i32x4{0, 0, 0, 0}; }
#endif
// acc[t] = tile t against the pieces of columns c0 .. c0 + KSTEP*S; CH accumulator chains
// per tile so that no MFMA waits for the previous one of its chain
template <int COLS, int NT16, int S, int CH>
__device__ __forceinline__ void rdot16(const RTile16<COLS, NT16, S> &t, const uint8_t *pc, int c0, AccT (&acc)[NT16],
                                       const int * = nullptr) {
    AccT a[NT16][CH];
#pragma unroll
    for (int q = 0; q < NT16; q++)
#pragma unroll
        for (int c = 0; c < CH; c++) a[q][c] = acc_zero();
    uint4 b = pcw_b<COLS>(pc, c0);
#pragma unroll
    for (int s = 0; s < S; s++) {
        const uint4 bn = pcw_b<COLS>(pc, c0 + KSTEP * (s + 1 < S ? s + 1 : s));
#pragma unroll
        for (int q = 0; q < NT16; q++) a[q][s % CH] = mma(t.w[q][s], b, a[q][s % CH]);
        b = bn;
    }
#pragma unroll
    for (int q = 0; q < NT16; q++) {
        acc[q] = a[q][0];
#pragma unroll
        for (int c = 1; c < CH; c++) acc[q] += a[q][c];
    }
}
#ifdef QT_RS_Q4
// ---- q4_0 row tiles ------------------------------------------------------------------------
// The reference's q4_0 blocks (32 weights w = (n - 8) d, byte i holding n of weights 2i
// (low nibble) and 2i+1, one f16 scale d; qwen_tts_kernels.c:2815-2816) on the same
// v_mfma_i32_16x16x64_i8 with the operands swapped: A = the activation pieces, row 4h+i =
// plane (0, 2, 1, 3)[i] over block h of the 64-column step (the other block's columns zero,
// rows 8..15 zero: those rows read a zero plane), B = 16 weight rows of unsigned nibbles n (lane l:
// row l%16, the 16 weights 16*(l/16) .. +15 of the step, even ones then odd ones, the
// pieces' storage order).  The accumulator input holds -8 x the block's piece sums (made
// once per input by q4_psum) in planes 0 and 2, so lane l < 32 ends with the exact sums of
// (n - 8)*p for row l%16 over block l/16 of the step; the four planes join in two exact
// 23-bit halves, and the block scale times their f32 value is added to the lane's f32 sum
// over its blocks.
// binary16 bits -> f32 as ref_f16_to_f32 (the reference's portable conversion, its
// subnormal mapping included), with selects instead of branches
__device__ __forceinline__ float f16_ref_sel(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16, em = h & 0x7FFFu;
    const uint32_t sh = ((uint32_t)__clz((int)(em | 1u)) - 21u) & 31u, ms = em << sh;   // (subnormals: 1..10)
    const uint32_t bi = sign | 0x7F800000u | ((em & 0x3FFu) << 13);
    const uint32_t bn = sign | ((em + (112u << 10)) << 13);
    const uint32_t bs = sign | ((112u - sh) << 23) | ((ms & 0x3FFu) << 13);
    return __uint_as_float(em >= 0x7C00u ? bi : em >= 0x0400u ? bn : em == 0 ? sign : bs);
}
template <int COLS, int NT16, int S>
struct QTile16 {
    uint2 w[NT16][S];     // the lane's 8 nibble bytes of each tile and step
    // the block scales go to the wave's LDS area sd[(s*64 + lane)*NT16 + t] (f32; scale of
    // row l%16 of tile t, block 2s + (l/16)%2 of the slice), which keeps the registers for
    // the MFMA results
    static constexpr int SD = S * 64 * NT16;   // floats per wave
    __device__ __forceinline__ void load(const uint8_t *W, const uint16_t *S16, int row0, int c0, int row_end, float *sd) {
        typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
        const int lane = threadIdx.x & 63, m = lane & 15, kg = lane >> 4, h = kg & 1;
        const __amdgpu_buffer_rsrc_t r = brsrc(uni(W)), rq = brsrc(uni(S16));
        const unsigned voff = (unsigned)(m * (COLS / 2) + 8 * kg);
        const unsigned soff = (unsigned)(m * (COLS / 32) * 2);
        static_assert(S % 4 == 0, "scale groups");
        // every load of every tile is issued before the first scale is converted (a
        // conversion waits for its load, and with it for every load issued before it)
        unsigned raw[NT16][S];   // dword s: the f16 scales of blocks 2s, 2s+1 of the slice
#pragma unroll
        for (int t = 0; t < NT16; t++) {
            const bool ok = row0 + 16 * t + m < row_end;
#pragma unroll
            for (int s = 0; s < S; s++) {
                const u32x2_t v = ok ? __builtin_amdgcn_raw_buffer_load_b64(
                                           r, voff, __builtin_amdgcn_readfirstlane(((row0 + 16 * t) * COLS + c0) / 2 + 32 * s), 0)
                                     : u32x2_t{0, 0};
                w[t][s] = make_uint2(v.x, v.y);
            }
#pragma unroll
            for (int j = 0; j < S / 4; j++) {
                const u32x4_t v = ok ? __builtin_amdgcn_raw_buffer_load_b128(
                                           rq, soff, __builtin_amdgcn_readfirstlane(((row0 + 16 * t) * (COLS / 32) + c0 / 32) * 2 + 16 * j), 0)
                                     : u32x4_t{0, 0, 0, 0};
                raw[t][4 * j] = v.x; raw[t][4 * j + 1] = v.y; raw[t][4 * j + 2] = v.z; raw[t][4 * j + 3] = v.w;
            }
        }
#pragma unroll
        for (int s = 0; s < S; s++) {
            float v[NT16];
#pragma unroll
            for (int t = 0; t < NT16; t++) v[t] = f16_ref_sel(h ? raw[t][s] >> 16 : raw[t][s] & 0xFFFFu);
            float *dst = sd + (s * 64 + lane) * NT16;
            if constexpr (NT16 % 4 == 0) {
#pragma unroll
                for (int t = 0; t < NT16; t += 4)
                    *reinterpret_cast<float4 *>(dst + t) = make_float4(v[t], v[t + 1], v[t + 2], v[t + 3]);
            } else {
#pragma unroll
                for (int t = 0; t < NT16; t++) dst[t] = v[t];
            }
        }
    }
};
// -8 x the piece sums of each 32-column block of the wave's slice (KW columns from c0), two
// per block: pq[2b] = -8 (P0 + 2^8 P1), pq[2b+1] = -8 (P2 + 2^8 P3), P_p the sum of plane p
template <int COLS, int KW>
__device__ __forceinline__ void q4_psum(const uint8_t *pc, int c0, int *pq) {
    constexpr int NBK = KW / 32, NI = NBK / 16;
    static_assert(NBK % 16 == 0, "blocks per lane");
    const int lane = threadIdx.x & 63, p = lane & 3;
    // every read first, then the sums (two chains each), then the neighbour plane's sum
    // from the quad (DPP, no LDS round trip), then the stores
    uint4 x[NI][2];
#pragma unroll
    for (int k = 0; k < NI; k++) {
        const int b = (lane >> 2) + 16 * k;
        const uint4 *src = reinterpret_cast<const uint4 *>(pc + p * pcs<COLS>() + c0 + 32 * b);
        x[k][0] = src[0];
        x[k][1] = src[1];
    }
    int sum[NI];
#pragma unroll
    for (int k = 0; k < NI; k++) {
        int s0 = 0, s1 = 0;
        s0 = __builtin_amdgcn_sdot4((int)x[k][0].x, 0x01010101, s0, false);
        s1 = __builtin_amdgcn_sdot4((int)x[k][1].x, 0x01010101, s1, false);
        s0 = __builtin_amdgcn_sdot4((int)x[k][0].y, 0x01010101, s0, false);
        s1 = __builtin_amdgcn_sdot4((int)x[k][1].y, 0x01010101, s1, false);
        s0 = __builtin_amdgcn_sdot4((int)x[k][0].z, 0x01010101, s0, false);
        s1 = __builtin_amdgcn_sdot4((int)x[k][1].z, 0x01010101, s1, false);
        s0 = __builtin_amdgcn_sdot4((int)x[k][0].w, 0x01010101, s0, false);
        s1 = __builtin_amdgcn_sdot4((int)x[k][1].w, 0x01010101, s1, false);
        sum[k] = s0 + s1;
    }
#pragma unroll
    for (int k = 0; k < NI; k++) {
        const int hi = __builtin_amdgcn_mov_dpp(sum[k], 0xB1, 0xF, 0xF, false);   // quad_perm(1,0,3,2): plane p ^ 1
        if ((p & 1) == 0) pq[2 * ((lane >> 2) + 16 * k) + (p >> 1)] = -8 * (sum[k] + 256 * hi);
    }
    wave_lds_order();
}
// Zero the plane after the NPL piece planes of a COLS-column input, once per launch (the
// piece writers never touch it), with a barrier before any wave reads it
template <int COLS>
__device__ __forceinline__ void q4_zero_plane(uint8_t *pc) {
    for (int i = threadIdx.x; i < pcs<COLS>() / 16; i += NT)
        reinterpret_cast<uint4 *>(pc + NPL * pcs<COLS>())[i] = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();
}
template <int COLS, int NT16, int S, int CH>
__device__ __forceinline__ void rdot16(const QTile16<COLS, NT16, S> &t, const uint8_t *pc, int c0, float (&acc)[NT16],
                                       const int *pq, const float *sd) {
    static_assert(S % 2 == 0, "steps are taken in pairs");
    const int lane = threadIdx.x & 63, m = lane & 15, kg = lane >> 4;
    // Steps s, s+1 (s even) share one accumulator: the first MFMA fills rows 0..7 (blocks
    // 2s, 2s+1 of the slice), the second rows 8..15 (blocks 2s+2, 2s+3), so lane group kg
    // ends with block 2s + kg.  Rows that carry no piece in an MFMA read the zero plane
    // after the pieces (q4_zero_plane); row 4h+i holds plane 0, 2, 1, 3 for i = 0..3, so
    // that the two corrections (planes 0 and 2) are the first two entries of the
    // accumulator input.
    const int pl = ((m & 1) << 1) | ((m >> 1) & 1);
    const bool row1 = m < 8 && (m >> 2) == (kg >> 1), row2 = m >= 8 && (m >> 2) - 2 == (kg >> 1);
    const uint8_t *pa1 = pc + (row1 ? pl : NPL) * pcs<COLS>() + c0 + 16 * kg;
    const uint8_t *pa2 = pc + (row2 ? pl : NPL) * pcs<COLS>() + c0 + 64 + 16 * kg;
    auto ld = [](const uint8_t *p, int off) { return *reinterpret_cast<const uint4 *>(p + off); };
    auto ld_d = [&](int s, float (&d)[NT16]) {   // block scales of step s, lanes < 32
        const float *ds = sd + (s * 64 + lane) * NT16;
        if constexpr (NT16 % 4 == 0) {
#pragma unroll
            for (int q = 0; q < NT16; q += 4) {
                const float4 v = *reinterpret_cast<const float4 *>(ds + q);
                d[q] = v.x; d[q + 1] = v.y; d[q + 2] = v.z; d[q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int q = 0; q < NT16; q++) d[q] = ds[q];
        }
    };
    auto nib = [](uint2 w) {
        return make_uint4(w.x & 0x0F0F0F0Fu, w.y & 0x0F0F0F0Fu, (w.x >> 4) & 0x0F0F0F0Fu, (w.y >> 4) & 0x0F0F0F0Fu);
    };
#pragma unroll
    for (int q = 0; q < NT16; q++) acc[q] = 0.f;
    uint4 a1 = ld(pa1, 0), a2 = ld(pa2, 0);
#pragma unroll
    for (int s = 0; s < S; s += 2) {
        const int sn = s + 2 < S ? s + 2 : s;
        const uint4 a1n = ld(pa1, 64 * sn), a2n = ld(pa2, 64 * sn);
        const int2 qc = *reinterpret_cast<const int2 *>(pq + 4 * s + 2 * kg);
        float de[NT16], dd[NT16];
        ld_d(s, de);
        ld_d(s + 1, dd);
        // the correction enters the first MFMA of the pair as its accumulator input
        const i32x4 cq = {qc.x, qc.y, 0, 0};
        i32x4 D[NT16];   // every MFMA of the pair first, then the epilogues (results in flight)
#pragma unroll
        for (int q = 0; q < NT16; q++) D[q] = mfma_i8(a1, nib(t.w[q][s]), cq);
#pragma unroll
        for (int q = 0; q < NT16; q++) D[q] = mfma_i8(a2, nib(t.w[q][s + 1]), D[q]);
#pragma unroll
        for (int q = 0; q < NT16; q++) {
            const int lo = D[q][0] + (D[q][2] << 8), hi = D[q][1] + (D[q][3] << 8);
            const float f = fmaf((float)hi, 65536.f, (float)lo);
            // lanes < 32 take the odd step's value of their row and block from lane + 32
            // (the swap's second result), so each lane's sum still runs over its blocks in
            // step order; the first result keeps f in lanes < 32, and the second operand
            // (lo, dead here) only gives the swap a register to write
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(f), (unsigned)lo, false, false);
            acc[q] = fmaf(dd[q], __uint_as_float(sw[1]), fmaf(de[q], __uint_as_float(sw[0]), acc[q]));
        }
        a1 = a1n;
        a2 = a2n;
        // keep each pair's epilogue here: the sums feed only the lanes < 32 store after the
        // loop, and the compiler would otherwise sink every epilogue down to that store,
        // holding all the MFMA results at once (spills)
#pragma unroll
        for (int q = 0; q < NT16; q++) asm volatile("" : "+v"(acc[q]));
    }
}
template <int COLS, int NT16, int S> using WTile = QTile16<COLS, NT16, S>;
#define RS_PQ(s, w) (&(s).pq[w][0])
#define RS_SD(s, w) , (&(s).sd[w][0])
#else
template <int COLS, int KW> __device__ __forceinline__ void q4_psum(const uint8_t *, int, int *) {}
template <int COLS> __device__ __forceinline__ void q4_zero_plane(uint8_t *) {}
template <int COLS, int NT16, int S> using WTile = RTile16<COLS, NT16, S>;
#define RS_PQ(s, w) nullptr
#define RS_SD(s, w)
#endif
// ---- LDS --------------------------------------------------------------------------------
struct HeadLds {
    float x[H];                  // x of the last layer, chunk-transposed (EPC 8)
    float xn[H];                 // final-normed
    float gain[H];               // final norm gains (EPC 8 layout)
    float wbv[4];
    int wbi[4];
    float win[2 * NHEAD];
#if defined(QT_RS_SMALL) && !defined(QT_RS_BF16)
    float cxs[H];                // Code Predictor int8 lm head: the input in unit order
    float cwst[8];
    uint8_t cpc[4 * pcs<H>()];   // pieces of RMSNorm(x) * final_norm
    int cred[16][4][4];          // partial plane sums [row][wave][plane] (int8 lm head)
    float clg[HEADR];            // the workgroup's logits
#endif
};
struct LdsP {                    // Q, O, GU (and the head-only workgroups)
    float xs[H];                 // the input in element order (RMSNorm: statistics order -> unit order)
    uint8_t pc[(NPL + (WQ4 ? 1 : 0)) * pcs<PCW>()];   // q4_0: plus a zero plane (q4_zero_plane)
#ifdef QT_RS_Q4
    int pq[4][2 * (PCW / 4 / 32)];   // per wave: -8 x its blocks' piece sums (q4_psum)
    float sd[4][(PCW / 4 / 64) * 64 * 8];   // per wave: its tiles' block scales (QTile16)
#endif
    RedT red[8 * 16][4][4];      // partial plane sums [row][wave][plane] (K split over the waves)
    float resid[OROWS];
    float wst[8];
    HeadLds hd;
};
struct LdsD {                    // DN
    uint8_t pc[(NPL + (WQ4 ? 1 : 0)) * pcs<F>()];   // q4_0: plus a zero plane (q4_zero_plane)
#ifdef QT_RS_Q4
    int pq[4][2 * (F / 4 / 32)];     // per wave: -8 x its blocks' piece sums (q4_psum)
    float sd[4][(F / 4 / 64) * 64 * 3];   // per wave: its tiles' block scales (QTile16)
#else
    uint4 tw[4][steps<F / 4>()][64]; // tile 2 (rows 32..47): [wave][step][lane]
#endif
    RedT red[4][3][16][4];       // partial plane sums [wave][tile][row][plane]
    float resid[48];
    float wst[8];
    HeadLds hd;
};
struct LdsA {                    // ATT + MRG
    uint16_t v[ABLK][KVB * HD];  // value rows of the chunk (qt_attn_mf.h swizzle), per 128-key block
    uint16_t qp[16][HD];
    uint16_t pp[16][ABLK * KVB]; // probability pieces of the chunk's keys, row 4h+p
    float ml[4][HPK][2];         // per-wave (max, exp-sum)
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

// Layer-0 input element i of a step: the embedding of the previous step's token, or xin
// (Code Predictor: xin for pass 0, else row tok of that pass's table).
__device__ __forceinline__ float x0_elem(const RArgs &a, int tok, int i, int step) {
#ifdef QT_RS_SMALL
    if (a.cp) return step == 0 ? ldg(a.xin + i) : bf16f(ldg(uni(ldg(a.cp_emb + step - 1)) + (size_t)tok * H + i));
#endif
    return tok < 0 ? ldg(a.xin + i) : bf16f(ldg(a.emb + (size_t)tok * H + i));
}

// K split over the waves: each wave's partial plane sums of its tiles' rows into
// red[row][wave][plane] (the lanes of plane columns 0..3; bf16's column 3 holds exact
// zeros), then a barrier; ksplit_row adds the four waves' sums for one row, waves in order.
template <int NT16, typename A, typename T>
__device__ __forceinline__ void ksplit_store(const A (&acc)[NT16], T (*red)[4][4]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 15, kg = lane >> 4;
    if (n < 4) {
#pragma unroll
        for (int t = 0; t < NT16; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) red[16 * t + 4 * kg + i][wave][n] = acc[t][i];
    }
    __syncthreads();
}
#ifdef QT_RS_Q4
// q4_0: lane l < 32 holds row l%16's f32 sum over block half l/16: red[row][wave][half]
template <int NT16>
__device__ __forceinline__ void ksplit_store(const float (&acc)[NT16], float (*red)[4][4]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane < 32) {
#pragma unroll
        for (int t = 0; t < NT16; t++) red[16 * t + (lane & 15)][wave][lane >> 4] = acc[t];
    }
    __syncthreads();
}
#endif
template <typename T>
__device__ __forceinline__ void ksplit_row(const T (*red)[4][4], int r, T (&d)[4]) {
#pragma unroll
    for (int p = 0; p < 4; p++) d[p] = ((red[r][0][p] + red[r][1][p]) + red[r][2][p]) + red[r][3][p];
}
// a row's dot product from its plane sums: int8 s*(D0 + 2^8 D1 + 2^16 D2 + 2^24 D3) times
// the row scale rs; bf16 the three planes' f32 sums added hi to lo (no row scale)
// (q4_0: the two block halves' f32 sums times the pieces' scale; the block scales are in)
__device__ __forceinline__ float row_dot(const RedT (&d)[4], float s, float rs) {
#if defined(QT_RS_Q4)
    return (d[0] + d[1]) * s;
#else
    if constexpr (WBF) return (d[0] + d[1]) + d[2];
    else return __fmul_rn(qt_pc_dot(d[0], d[1], d[2], d[3], s), rs);
#endif
}

// Pieces of RMSNorm(x)*g: x arrives in the statistics' order (thread t: elements t + NT*k),
// the statistics are summed in that order (thread in k order, wave butterfly, waves in
// order: pc_stats), x goes through LDS to unit order (thread u: elements EH*u .. +EH-1) and
// the pieces are made there from the same values with the same operations as
// stage_norm_pc.  gc: gains of the thread's statistics elements, gu: of its unit.  Returns
// the pieces' scale; ends with a barrier.
__device__ __forceinline__ float norm_pieces(const float (&xv)[EH], const float (&gc)[EH], const float (&gu)[EH], float *xs,
                                             float *wst, uint8_t *pc, float eps) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float ss = 0.f, m = 0.f;
#pragma unroll
    for (int k = 0; k < EH; k++) {
        ss = fmaf(xv[k], xv[k], ss);
        m = fmaxf(m, fabsf(xv[k] * gc[k]));
    }
    ss = group_sum<64>(ss);
    m = group_max<64>(m);
    if (lane == 0) { wst[2 * wave] = ss; wst[2 * wave + 1] = m; }
#pragma unroll
    for (int k = 0; k < EH; k++) xs[tid + NT * k] = xv[k];
    __syncthreads();
    float inv;
    QtPcScale ps;
    pc_norm_scale<4>(wst, H, eps, inv, ps);
    float v[EH];
#pragma unroll
    for (int q = 0; q < EH / 4; q++) {
        const float4 p = *reinterpret_cast<const float4 *>(xs + EH * tid + 4 * q);
        v[4 * q] = (p.x * inv) * gu[4 * q]; v[4 * q + 1] = (p.y * inv) * gu[4 * q + 1];
        v[4 * q + 2] = (p.z * inv) * gu[4 * q + 2]; v[4 * q + 3] = (p.w * inv) * gu[4 * q + 3];
    }
    pcw_put<H, EH>(pc, tid, v, ps.isc);
    wave_lds_order();   // unit tid: wave w makes the pieces of columns (H/4)w .. +H/4-1, its own K slice
    return ps.s;
}
// the RMSNorm gains a thread needs: statistics elements tid + NT*k, unit elements EH tid ..
__device__ __forceinline__ void load_norm_gains(const float *g, float (&gc)[EH], float (&gu)[EH]) {
    const int tid = threadIdx.x;
    g = uni(g);
#pragma unroll
    for (int k = 0; k < EH; k++) gc[k] = ldg(g + tid + NT * k);
#pragma unroll
    for (int q = 0; q < EH / 4; q++) {
        const float4 a = ldg(reinterpret_cast<const float4 *>(g + EH * tid + 4 * q));
        gu[4 * q] = a.x; gu[4 * q + 1] = a.y; gu[4 * q + 2] = a.z; gu[4 * q + 3] = a.w;
    }
}
__device__ __forceinline__ float4 f4(const uint4 &v) {
    return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
__device__ __forceinline__ float amax4(const uint4 &v) {
    return fmaxf(fmaxf(fabsf(__uint_as_float(v.x)), fabsf(__uint_as_float(v.y))),
                 fmaxf(fabsf(__uint_as_float(v.z)), fabsf(__uint_as_float(v.w))));
}

// ---- head (final norm, codec head rows, masked local argmax, global argmax) ------------
using THead = Tile<QT_BF16, H, HEADR / 4>;
// The head rows of a workgroup for the step about to end: the Talker's bf16 codec head, or
// (Code Predictor) 16 rows of the pass's lm head: int8, one 16-row MFMA tile with the
// columns split over the waves as in the projections, or bf16 as the codec head.
struct HeadTile {
    THead th;
#if defined(QT_RS_SMALL) && !defined(QT_RS_BF16)
    RTile16<H, 1, steps<H / 4>()> tc;
    float tcs = 0.f;             // row scale of row hc*HEADR + tid (tid < HEADR)
#endif
    __device__ __forceinline__ void load(const RArgs &a, int hc, int wave, int step) {
        if (a.with_head) th.load(a.head_w, nullptr, hc * HEADR + wave * (HEADR / 4));
#if defined(QT_RS_SMALL) && defined(QT_RS_BF16)
        else if (a.cp && step > 0 && hc * HEADR < a.vocab)   // bf16 lm head rows (the codebook is whole tiles)
            th.load(uni(ldg(a.cp_head + step - 1)), nullptr, hc * HEADR + wave * (HEADR / 4));
#elif defined(QT_RS_SMALL)
        else if (a.cp && step > 0) {
            const int tid = threadIdx.x, r0 = hc * HEADR;
            tc.load(uni(ldg(a.cp_head + step - 1)), r0, wave * (H / 4), a.vocab);
            tcs = (tid < HEADR && r0 + tid < a.vocab) ? ldg(uni(ldg(a.cp_hs + step - 1)) + r0 + tid) : 0.f;
        }
#endif
    }
};
__device__ __forceinline__ int head_phase(const Ctx &c, HeadLds &s, const HeadTile &ht, int step, bool last) {
    const RArgs &a = c.a;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int par = step & 1;
    const unsigned tag = c.tag0 + (unsigned)step;
    {
        constexpr int KX = H / 4 / NT;
        uint4 v[KX];
        const unsigned base = (c.blk(par, c.L - 1) + R_X) * 4u;
        RS_MARK(step, c.L, 0);
        wait16<KX, 8>(c.rr, H / 4, [&](int i) { return base + (unsigned)i * 16u; }, v, a.err);
        RS_MARK(step, c.L, 1);
#pragma unroll
        for (int k = 0; k < KX; k++) put4<8, H>(s.x, 4 * (tid + NT * k), v[k]);
    }
    __syncthreads();
#if defined(QT_RS_SMALL) && !defined(QT_RS_BF16)
    // (a Code Predictor's int8 lm head makes its own pieces of the normed x: xn only for hid)
    if (!a.cp || (last && c.hc == 0))
#endif
        stage_norm<QT_BF16, H>(s.x, s.gain, a.eps, s.xn);
    if (last && c.hc == 0)
        for (int i = tid; i < H; i += NT) { a.hid[i] = s.xn[xpos<8, H>(i)]; a.decx[i] = s.x[xpos<8, H>(i)]; }
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    if (a.with_head) {
        float acc[HEADR / 4];
        tile_dot<QT_BF16, H, HEADR / 4>(ht.th, s.xn, acc);
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
#if defined(QT_RS_SMALL) && defined(QT_RS_BF16)
    else if (a.cp && step > 0) {
        // bf16 lm head rows on the final-normed x (the Talker head's arithmetic, k_mv's bf16
        // order); plain argmax from the start value -1e30, lowest index on ties
        float acc[HEADR / 4];
        tile_dot<QT_BF16, H, HEADR / 4>(ht.th, s.xn, acc);
        if (lane == 0) {
            float b = -1e30f;
            int ix = 0x7FFFFFFF;
#pragma unroll
            for (int r = 0; r < HEADR / 4; r++) {
                const int i = c.hc * HEADR + wave * (HEADR / 4) + r;
                if (i < a.vocab && (acc[r] > b || (acc[r] == b && i < ix))) { b = acc[r]; ix = i; }
            }
            s.wbv[wave] = b; s.wbi[wave] = ix;
        }
        __syncthreads();
        bv = s.wbv[0]; bi = s.wbi[0];
        for (int w = 1; w < 4; w++)
            if (s.wbv[w] > bv || (s.wbv[w] == bv && s.wbi[w] < bi)) { bv = s.wbv[w]; bi = s.wbi[w]; }
    }
#elif defined(QT_RS_SMALL)
    else if (a.cp && step > 0) {
        // the lm head on the pieces of RMSNorm(x) * final_norm, made in k_mv's int8 order
        // (the per-kernel frame's lm-head matvec), so the logits are the same bits; plain
        // argmax from the start value -1e30, lowest index on ties (k_select mode 0)
        float xv[EH], gc[EH], gu[EH];
#pragma unroll
        for (int k = 0; k < EH; k++) {   // the final norm's gains from their LDS copy
            xv[k] = s.x[xpos<8, H>(tid + NT * k)];
            gc[k] = s.gain[xpos<8, H>(tid + NT * k)];
            gu[k] = s.gain[xpos<8, H>(EH * tid + k)];
        }
        const float sA = norm_pieces(xv, gc, gu, s.cxs, s.cwst, s.cpc, a.eps);
        i32x4 acc[1];
        rdot16<H, 1, H / 4 / 64, 1>(ht.tc, s.cpc, wave * (H / 4), acc);
        ksplit_store<1>(acc, s.cred);
        if (tid < HEADR) {
            int d[4];
            ksplit_row(s.cred, tid, d);
            s.clg[tid] = __fmul_rn(qt_pc_dot(d[0], d[1], d[2], d[3], sA), ht.tcs);   // int8 lm head
        }
        __syncthreads();
        bv = -1e30f;
        for (int r = 0; r < HEADR; r++) {
            const int i = c.hc * HEADR + r;
            const float v = s.clg[r];
            if (i < a.vocab && (v > bv || (v == bv && i < bi))) { bv = v; bi = i; }
        }
    }
#endif
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
#ifdef QT_RS_SMALL
    if (a.cp) {
        if (step == 0) gi = ldg(a.cp_codes);   // pass 1 reads the frame's input code
        else if (c.hc == 0 && tid == 0) a.cp_codes[step] = gi;
    }
#endif
    __syncthreads();
    if (last)   // every read of this step's region is done (all of them precede the winners)
        for (int l = 0; l < c.L; l++) clear_share(c, par, l);
    return (a.with_head || a.cp) ? gi : -1;
}

// 16-byte / 8-byte agent-scope stores of hand-off words
__device__ __forceinline__ void put4w(const Ctx &c, unsigned word, float a0, float a1, float a2, float a3) {
    const u32x4_t v = {__float_as_uint(a0), __float_as_uint(a1), __float_as_uint(a2), __float_as_uint(a3)};
    __builtin_amdgcn_raw_buffer_store_b128(v, c.rr, word * 4u, 0, SC1);
}
__device__ __forceinline__ void put2w(const Ctx &c, unsigned word, float a0, float a1) {
    typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
    const u32x2_t v = {__float_as_uint(a0), __float_as_uint(a1)};
    __builtin_amdgcn_raw_buffer_store_b64(v, c.rr, word * 4u, 0, SC1);
}


// ---- Q: q|k|v rows ------------------------------------------------------------------------
__device__ __forceinline__ void role_q(const Ctx &c, LdsP &s, int grp, int qi) {
    const RArgs &a = c.a;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // 128 rows; wave w takes columns (H/4)w .. +H/4-1 of all of them
    const int row0 = qi < 2 ? (2 * grp + qi) * HD : qi == 2 ? QD + grp * HD : QD + KVD + grp * HD;
    WTile<H, 8, steps<H / 4>()> t;
    float rs = WBF ? 1.f : 0.f;   // bf16 rows carry no scale
    float gc[EH], gu[EH];
    auto load = [&](int l) {
        t.load(c.ly[l].w[0], c.ly[l].s16[0], row0, wave * (H / 4), row0 + QROWS RS_SD(s, wave));
        if (RSC && tid < QROWS) rs = ldg(uni(c.ly[l].s[0]) + row0 + tid);
        load_norm_gains(c.ly[l].in_norm, gc, gu);
    };
    HeadTile ht;
    load_gains<4, 8, H>(a.final_norm, s.hd.gain);
    q4_zero_plane<H>(s.pc);
    load(0);
    land();
    int tok = -1;
    for (int step = 0; step < a.n_steps; step++) {
        const int par = step & 1;
        const bool last = step + 1 == a.n_steps;
        for (int l = 0; l < c.L; l++) {
            float xv[EH];
#ifdef QT_RS_SMALL
            const bool x0_direct = l == 0 && !a.mtp_w;   // else the pass input comes through R_XIN
#else
            const bool x0_direct = l == 0;
#endif
            if (x0_direct) {
#pragma unroll
                for (int k = 0; k < EH; k++) xv[k] = x0_elem(a, tok, tid + NT * k, step);
            } else {
                unsigned v[EH];
#ifdef QT_RS_SMALL
                const unsigned base = (l == 0 ? c.blk(par, 0) + R_XIN : c.blk(par, l - 1) + R_X) * 4u;
#else
                const unsigned base = (c.blk(par, l - 1) + R_X) * 4u;
#endif
                RS_MARK(step, l, 0);
                wait4<EH, 32>(c.rr, H, [&](int i) { return base + (unsigned)i * 4u; }, v, a.err);
                RS_MARK(step, l, 1);
#pragma unroll
                for (int k = 0; k < EH; k++) xv[k] = __uint_as_float(v[k]);
            }
            const float sA = norm_pieces(xv, gc, gu, s.xs, s.wst, s.pc, a.eps);
            q4_psum<H, H / 4>(s.pc, wave * (H / 4), RS_PQ(s, wave));
            RS_MARK(step, l, 6);
            AccT acc[8];
            rdot16<H, 8, steps<H / 4>(), 1>(t, s.pc, wave * (H / 4), acc, RS_PQ(s, wave) RS_SD(s, wave));
            RS_MARK(step, l, 7);
            ksplit_store<8>(acc, s.red);
            if (tid < QROWS) {
                RedT d[4];
                ksplit_row(s.red, tid, d);
                put(c.wp(par, l, R_QKV + row0 + tid), row_dot(d, sA, rs));
            }
            RS_MARK(step, l, 2);
            if (step > 0) clear_share(c, par ^ 1, l);
            __syncthreads();   // the LDS of this layer is free
            if (l + 1 < c.L) load(l + 1);
            else if (!last) load(0);
            land();
            RS_MARK(step, l, 3);
        }
        // the codec-head tile is loaded here, not inside the layer loop, so that its
        // registers are live only for the head
        ht.load(a, c.hc, wave, step);
        land();
        tok = head_phase(c, s.hd, ht, step, last);
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
    const int row0 = oi * OROWS;
    constexpr int OT = OROWS / 16;   // row tiles (8 int8, 4 bf16)
    WTile<QD, OT, steps<QD / 4>()> t;
    float rs = WBF ? 1.f : 0.f;   // bf16 rows carry no scale
    auto load = [&](int l) {
        t.load(c.ly[l].w[1], c.ly[l].s16[1], row0, wave * (QD / 4), row0 + OROWS RS_SD(s, wave));
        if (RSC && tid < OROWS) rs = ldg(uni(c.ly[l].s[1]) + row0 + tid);
    };
    HeadTile ht;
    load_gains<4, 8, H>(a.final_norm, s.hd.gain);
    q4_zero_plane<QD>(s.pc);
    load(0);
    land();
    int tok = -1;
    for (int step = 0; step < a.n_steps; step++) {
        const int par = step & 1;
        const bool last = step + 1 == a.n_steps;
        for (int l = 0; l < c.L; l++) {
            // attn (2048) and, after layer 0, the residual rows of x (128)
            uint4 v[3];
#ifdef QT_RS_SMALL
            const bool xres = l > 0 || a.mtp_w;   // residual rows from the hand-off words
            const unsigned bx = l > 0 ? (c.blk(par, l - 1) + R_X + row0) * 4u : (c.blk(par, 0) + R_XIN + row0) * 4u;
#else
            const bool xres = l > 0;
            const unsigned bx = l > 0 ? (c.blk(par, l - 1) + R_X + row0) * 4u : 0u;
#endif
            {
                const unsigned ba = (c.blk(par, l) + R_ATT) * 4u;
                const int n16 = QD / 4 + (xres ? OROWS / 4 : 0);
                RS_MARK(step, l, 0);
                wait16<3, 8>(c.rr, n16, [&](int i) {
                    return i < QD / 4 ? ba + (unsigned)(2 * (i % NT) + i / NT) * 16u : bx + (unsigned)(i - QD / 4) * 16u;
                }, v, a.err);
                RS_MARK(step, l, 1);
            }
            float m = fmaxf(amax4(v[0]), amax4(v[1]));
            if (xres && tid < OROWS / 4) *reinterpret_cast<float4 *>(s.resid + 4 * tid) = f4(v[2]);
            if (!xres && tid < OROWS) s.resid[tid] = x0_elem(a, tok, row0 + tid, step);
            m = group_max<64>(m);
            if (lane == 0) s.wst[wave] = m;
            __syncthreads();
            const QtPcScale ps = qt_pc_scale(fmaxf(fmaxf(s.wst[0], s.wst[1]), fmaxf(s.wst[2], s.wst[3])));
            {
                const float4 p0 = f4(v[0]), p1 = f4(v[1]);
                const float v8[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
                pcw_put<QD, 8>(s.pc, tid, v8, ps.isc);
            }
            wave_lds_order();   // unit tid: wave w makes the pieces of columns 512w .. +511, its own K slice
            q4_psum<QD, QD / 4>(s.pc, wave * (QD / 4), RS_PQ(s, wave));
            RS_MARK(step, l, 6);
            AccT acc[OT];
            rdot16<QD, OT, steps<QD / 4>(), 1>(t, s.pc, wave * (QD / 4), acc, RS_PQ(s, wave) RS_SD(s, wave));
            RS_MARK(step, l, 7);
            ksplit_store<OT>(acc, s.red);
            if (tid < OROWS) {
                RedT d[4];
                ksplit_row(s.red, tid, d);
                put(c.wp(par, l, R_XA + row0 + tid), __fadd_rn(s.resid[tid], row_dot(d, ps.s, rs)));
            }
            RS_MARK(step, l, 2);
            if (step > 0) clear_share(c, par ^ 1, l);
            __syncthreads();
            if (l + 1 < c.L) { load(l + 1); land(); }
            RS_MARK(step, l, 3);
        }
        ht.load(a, c.hc, wave, step);
        land();
        tok = head_phase(c, s.hd, ht, step, last);
        if (last) break;   // (so the compiler sees the tile below as the next step's only value)
        load(0);
        land();
    }
}

// ---- GU: h = SwiGLU(W_gu . RMSNorm(xa)) ---------------------------------------------------
// Rows 2i, 2i+1 of the interleaved matrix are the gate and up rows of h element i.
__device__ __forceinline__ void role_gu(const Ctx &c, LdsP &s, int gi) {
    const RArgs &a = c.a;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row0 = gi * GROWS;
    WTile<H, 8, steps<H / 4>()> t;
    float rsg = WBF ? 1.f : 0.f, rsu = rsg;
    float gc[EH], gu[EH];
    auto load = [&](int l) {
        t.load(c.ly[l].w[2], c.ly[l].s16[2], row0, wave * (H / 4), row0 + GROWS RS_SD(s, wave));
        if (RSC && tid < GROWS / 2) {
            const float *S = uni(c.ly[l].s[2]);
            rsg = ldg(S + row0 + 2 * tid);
            rsu = ldg(S + row0 + 2 * tid + 1);
        }
        load_norm_gains(c.ly[l].post_norm, gc, gu);
    };
    HeadTile ht;
    load_gains<4, 8, H>(a.final_norm, s.hd.gain);
    q4_zero_plane<H>(s.pc);
    load(0);
    land();
    for (int step = 0; step < a.n_steps; step++) {
        const int par = step & 1;
        const bool last = step + 1 == a.n_steps;
        for (int l = 0; l < c.L; l++) {
            float xv[EH];
            {
                unsigned v[EH];
                const unsigned base = (c.blk(par, l) + R_XA) * 4u;
                RS_MARK(step, l, 0);
                wait4<EH, 32>(c.rr, H, [&](int i) { return base + (unsigned)i * 4u; }, v, a.err);
                RS_MARK(step, l, 1);
#pragma unroll
                for (int k = 0; k < EH; k++) xv[k] = __uint_as_float(v[k]);
            }
            const float sD = norm_pieces(xv, gc, gu, s.xs, s.wst, s.pc, a.eps);
            q4_psum<H, H / 4>(s.pc, wave * (H / 4), RS_PQ(s, wave));
            RS_MARK(step, l, 6);
            AccT acc[8];
            rdot16<H, 8, steps<H / 4>(), 1>(t, s.pc, wave * (H / 4), acc, RS_PQ(s, wave) RS_SD(s, wave));
            RS_MARK(step, l, 7);
            ksplit_store<8>(acc, s.red);
            if (tid < GROWS / 2) {
                RedT dg[4], du[4];
                ksplit_row(s.red, 2 * tid, dg);
                ksplit_row(s.red, 2 * tid + 1, du);
                const float gt = row_dot(dg, sD, rsg);
                const float up = row_dot(du, sD, rsu);
                put(c.wp(par, l, R_H + row0 / 2 + tid), gt / (1.0f + expf(-gt)) * up);
            }
            RS_MARK(step, l, 2);
            if (step > 0) clear_share(c, par ^ 1, l);
            __syncthreads();
            if (l + 1 < c.L) { load(l + 1); land(); }
            RS_MARK(step, l, 3);
        }
        ht.load(a, c.hc, wave, step);
        land();
        head_phase(c, s.hd, ht, step, last);
        if (last) break;   // (so the compiler sees the tile below as the next step's only value)
        load(0);
        land();
    }
}

// ---- DN: x' = xa + W_dn . h ---------------------------------------------------------------
// The workgroup's 48 or 40 rows are three 16-row tiles (the third partly empty for 40);
// wave w takes columns (F/4)w .. +F/4-1 of all three (tiles 0, 1 in registers, tile 2 in
// LDS, copied there straight from memory) and the four waves' exact partial sums are
// added through LDS.  Lane l of wave w holds the h units n = 192w + l + 64k (k < 3, UD
// values each, all in the wave's own K slice) and makes their pieces from registers (the
// values, scale and order of stage_pc).
__device__ __forceinline__ void role_dn(const Ctx &c, LdsD &s, int di) {
    const RArgs &a = c.a;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    [[maybe_unused]] const int m16 = lane & 15, kg = lane >> 4;
    const bool big = di < NDB;                 // NDB workgroups of 48 rows, the others 40
    const int row0 = big ? 48 * di : 48 * NDB + 40 * (di - NDB);
    const int nrows = big ? 48 : 40;
    constexpr int KW = F / 4, S = steps<KW>();  // columns and 64-byte MFMA steps per wave
    const int c0 = wave * KW;
#ifdef QT_RS_Q4
    QTile16<F, 3, S> t;           // all three tiles in registers (half the bytes of int8)
    float rs = 0.f;
    auto load = [&](int l) { t.load(c.ly[l].w[3], c.ly[l].s16[3], row0, c0, row0 + nrows, &s.sd[wave][0]); };
#else
    RTile16<F, 2, S> t;
    float rs = WBF ? 1.f : 0.f;   // bf16 rows carry no scale
    auto load = [&](int l) {
        t.load(c.ly[l].w[3], row0, c0, row0 + nrows);
        if (row0 + 32 + m16 < row0 + nrows) {
            const __amdgpu_buffer_rsrc_t r = brsrc(uni(c.ly[l].w[3]));
            const unsigned voff = (unsigned)(m16 * WB * F + 16 * kg);
#pragma unroll
            for (int st = 0; st < S; st++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)&s.tw[wave][st][0], 16,
                                                         voff, __builtin_amdgcn_readfirstlane(WB * ((row0 + 32) * F + c0) + 64 * st), 0, 0);
        }
        if (RSC && tid < nrows) rs = ldg(uni(c.ly[l].s[3]) + row0 + tid);
    };
#endif
    HeadTile ht;
    load_gains<4, 8, H>(a.final_norm, s.hd.gain);
    q4_zero_plane<F>(s.pc);
    load(0);
    land();
    for (int step = 0; step < a.n_steps; step++) {
        const int par = step & 1;
        const bool last = step + 1 == a.n_steps;
        for (int l = 0; l < c.L; l++) {
            // thread (wave w, lane) takes h units 192w + lane + 64k (UD values, UD/4 16-byte
            // groups each), all in the wave's own K slice, and the residual rows of xa
            constexpr int GPU_ = UD / 4, GD = 3 * GPU_;
            uint4 v[GD + 1];
            {
                const unsigned bh = (c.blk(par, l) + R_H) * 4u, bx = (c.blk(par, l) + R_XA + row0) * 4u;
                const int n16 = GD * NT + nrows / 4;
                RS_MARK(step, l, 0);
                wait16<GD + 1, 16>(c.rr, n16, [&](int i) {
                    const int k = i / NT, t = i % NT;
                    if (k < GD)
                        return bh + (unsigned)(GPU_ * (192 * (t >> 6) + (t & 63) + 64 * (k / GPU_)) + (k % GPU_)) * 16u;
                    return bx + (unsigned)t * 16u;
                }, v, a.err);
                RS_MARK(step, l, 1);
            }
            float m = 0.f;
#pragma unroll
            for (int k = 0; k < GD; k++) m = fmaxf(m, amax4(v[k]));
            if (tid < nrows / 4) *reinterpret_cast<float4 *>(s.resid + 4 * tid) = f4(v[GD]);
            m = group_max<64>(m);
            if (lane == 0) s.wst[wave] = m;
            __syncthreads();
            const QtPcScale ps = qt_pc_scale(fmaxf(fmaxf(s.wst[0], s.wst[1]), fmaxf(s.wst[2], s.wst[3])));
#pragma unroll
            for (int k = 0; k < 3; k++) {
                float vu[UD];
#pragma unroll
                for (int g2 = 0; g2 < GPU_; g2++) {
                    const float4 p = f4(v[GPU_ * k + g2]);
                    vu[4 * g2] = p.x; vu[4 * g2 + 1] = p.y; vu[4 * g2 + 2] = p.z; vu[4 * g2 + 3] = p.w;
                }
                pcw_put<F, UD>(s.pc, 192 * wave + lane + 64 * k, vu, ps.isc);
            }
            wave_lds_order();   // the wave's own K slice
#ifdef QT_RS_Q4
            q4_psum<F, KW>(s.pc, c0, RS_PQ(s, wave));
            RS_MARK(step, l, 6);
            {
                float acc[3];
                rdot16<F, 3, S, 1>(t, s.pc, c0, acc, RS_PQ(s, wave), &s.sd[wave][0]);
                RS_MARK(step, l, 7);
                if (lane < 32) {
#pragma unroll
                    for (int q = 0; q < 3; q++) s.red[wave][q][lane & 15][lane >> 4] = acc[q];
                }
            }
            __syncthreads();
#else
            RS_MARK(step, l, 6);
            AccT acc[3];
            {
                AccT ac[3][2];
#pragma unroll
                for (int q = 0; q < 3; q++) ac[q][0] = ac[q][1] = acc_zero();
                uint4 b = pcw_b<F>(s.pc, c0);
                uint4 w2 = s.tw[wave][0][lane];
#pragma unroll
                for (int st = 0; st < S; st++) {
                    const int sn = st + 1 < S ? st + 1 : st;
                    const uint4 bn = pcw_b<F>(s.pc, c0 + KSTEP * sn);
                    const uint4 w2n = s.tw[wave][sn][lane];
                    ac[0][st & 1] = mma(t.w[0][st], b, ac[0][st & 1]);
                    ac[1][st & 1] = mma(t.w[1][st], b, ac[1][st & 1]);
                    ac[2][st & 1] = mma(w2, b, ac[2][st & 1]);
                    b = bn;
                    w2 = w2n;
                }
#pragma unroll
                for (int q = 0; q < 3; q++) acc[q] = ac[q][0] + ac[q][1];
            }
            RS_MARK(step, l, 7);
            // partial plane sums of this wave: red[wave][tile][row][plane]
            if (m16 < 4) {
#pragma unroll
                for (int q = 0; q < 3; q++)
#pragma unroll
                    for (int i = 0; i < 4; i++) s.red[wave][q][4 * kg + i][m16] = acc[q][i];
            }
            __syncthreads();
#endif
            if (tid < nrows) {
                const int q = tid >> 4, rr = tid & 15;
                RedT d[4];
#pragma unroll
                for (int n = 0; n < 4; n++) d[n] = ((s.red[0][q][rr][n] + s.red[1][q][rr][n]) + s.red[2][q][rr][n]) + s.red[3][q][rr][n];
                const float vv = row_dot(d, ps.s, rs);
                const float xo = __fadd_rn(s.resid[tid], vv);
                put(c.wp(par, l, R_X + row0 + tid), xo);
                if (a.layer_out && last) a.layer_out[(size_t)l * H + row0 + tid] = xo;
            }
            RS_MARK(step, l, 2);
            if (step > 0) clear_share(c, par ^ 1, l);
            __syncthreads();
            if (l + 1 < c.L) { load(l + 1); land(); }
            RS_MARK(step, l, 3);
        }
        ht.load(a, c.hc, wave, step);
        land();
        head_phase(c, s.hd, ht, step, last);
        if (last) break;   // (so the compiler sees the tile below as the next step's only value)
        load(0);
        land();
    }
}

// ---- attention chunk (one pass under the chunk maximum, qt_attn_mf.h) --------------------
// NBK 128-key blocks: K rows in kf (wave w holds k-tile w of each block), V rows in LDS.
// k-tiles holding no key are neither scored nor multiplied.
template <int NBK>
__device__ __forceinline__ void att_chunk(LdsA &s, const uint4 (&kf)[ABLK][8], int n, float scale2, QtAttRun &run, int st_, int l_) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kg = lane >> 4, key = lane & 15, hh = lane >> 4;
    const int hc = hh < HPK ? hh : HPK - 1;
    qt_u32x4 qa[4];
#pragma unroll
    for (int s2 = 0; s2 < 4; s2++) qa[s2] = qt_lds16(&s.qp[key][32 * s2 + 8 * kg]);
    // 1. scores and the wave's maximum
    float sv[NBK][2];
    float wm = -INFINITY;
#pragma unroll
    for (int b = 0; b < NBK; b++) {
        const int r0 = KVB * b + 32 * wave;
        sv[b][0] = sv[b][1] = -INFINITY;
        if (r0 < n) {
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++) {
                qt_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s2 = 0; s2 < 4; s2++) {
                    const uint4 kk = kf[b][t2 * 4 + s2];
                    acc = qt_mfma_bf16(qa[s2], qt_u32x4{kk.x, kk.y, kk.z, kk.w}, acc);
                }
                const float sc = (acc[0] + acc[1]) + acc[2];
                sv[b][t2] = r0 + 16 * t2 + key < n ? sc * scale2 : -INFINITY;
            }
            wm = fmaxf(wm, group_max<16>(fmaxf(sv[b][0], sv[b][1])));
        }
    }
    RS_MARK(st_, l_, 8);
    if (hh < HPK && key == 0) s.ml[wave][hh][0] = wm;
    __syncthreads();
    // 2., 3. chunk maximum, probabilities, the wave's sums
    const float M = fmaxf(fmaxf(s.ml[0][hc][0], s.ml[1][hc][0]), fmaxf(s.ml[2][hc][0], s.ml[3][hc][0]));
    float lw = 0.f;
#pragma unroll
    for (int b = 0; b < NBK; b++) {
        const int r0 = KVB * b + 32 * wave;
        if (r0 < n) lw += qt_cm_probs<HPK>(sv[b][0], sv[b][1], M, &s.pp[0][0], ABLK * KVB, r0, lane);
    }
    if (hh < HPK && key == 0) s.ml[wave][hh][1] = lw;
    RS_MARK(st_, l_, 9);
    __syncthreads();
    RS_MARK(st_, l_, 10);
    // 4. P.V over the k-tiles holding keys, operands of up to eight k-tiles read before
    // their MFMAs
    const int nt = (n + 31) >> 5, d0 = 32 * wave;
    qt_f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    constexpr int NTL = NBK * 4, GT = NTL < 8 ? NTL : 8;
#pragma unroll
    for (int g0 = 0; g0 < NTL; g0 += GT) {
        qt_u32x4 pa[GT], vv[GT][2];
#pragma unroll
        for (int u = 0; u < GT; u++) {
            const int t = g0 + u;
            if (t >= nt) break;
            qt_cm_operands(&s.pp[0][0], ABLK * KVB, 32 * t, &s.v[t >> 2][32 * (t & 3) * HD], d0, lane, pa[u], vv[u]);
        }
#pragma unroll
        for (int u = 0; u < GT; u++) {
            const int t = g0 + u;
            if (t >= nt) break;
            qt_cm_mfma(pa[u], vv[u], acc);
        }
    }
    RS_MARK(st_, l_, 11);
#pragma unroll
    for (int dt = 0; dt < 2; dt++) run.o[dt] = (acc[dt][0] + acc[dt][1]) + acc[dt][2];
    run.m = M;
    run.l = ((s.ml[0][hc][1] + s.ml[1][hc][1]) + s.ml[2][hc][1]) + s.ml[3][hc][1];
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
    qt_att_zero_rows<HPK>(&s.pp[0][0], ABLK * KVB, tid, NT);
    // a launch whose every step has all its keys in chunk 0 (at most 16, e.g. a Code
    // Predictor frame): chunk 0 writes the attention output itself and no workgroup merges
    // (the merge of a single partial is o * (1 / l) after +0 terms, done here the same way);
    // the other chunks then have no work at all
    const bool one = Geo(c.pos0 + a.n_steps - 1).nch == 1;
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
                // one pass over the chunk (qt_attn_mf.h), specialised on its block count so
                // that it is straight-line code: every wave scores its k-tile of every block,
                // two barriers (chunk maximum, probabilities), then P.V of its 32 dims over
                // the k-tiles
                QtAttRun run;
                if (nblk == 1) att_chunk<1>(s, kf, n, scale2, run, step, l);
                else if (nblk == 2) att_chunk<2>(s, kf, n, scale2, run, step, l);
                else if (nblk == 3) att_chunk<3>(s, kf, n, scale2, run, step, l);
                else att_chunk<4>(s, kf, n, scale2, run, step, l);
                RS_MARK(step, l, 7);
                // partial of this chunk: o (head lane/16, dims 32 wave + lane%16 and +16), m, l
                const int hq = lane >> 4;
                if (one) {
                    if (hq < HPK) {
                        const float il = 1.0f / run.l;
                        const int ob = R_ATT + (2 * g + hq) * HD + 32 * wave + key;
                        put(c.wp(par, l, ob), (run.o[0] + 0.0f) * il);
                        put(c.wp(par, l, ob + 16), (run.o[1] + 0.0f) * il);
                    }
                } else if (hq < HPK) {
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
            if (!one) {
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
            // (returning here, not falling out of the loops, shows the compiler that the key
            // registers are always reloaded before the next use)
            if (last && l + 1 == c.L) return;
            if (l + 1 < c.L) prefetch(l + 1, ge);
            else prefetch(0, Geo(pos + 1));
            land();
            RS_MARK(step, l, 3);
        }
    }
}

// ---- head only (the slots the 0.6B geometry leaves over) ------------------------------------
// Takes part in every step's head phase; clears its shares of the previous step's region at
// the start of the step (every read of that region came before the previous step's winner
// exchange, which this workgroup has completed).
// mi >= 0 (Code Predictor with the mtp projection): rows 16 mi .. +15 of the projection,
// made for every pass before its layers can start: e's pieces (k_mv's int8 order without a
// norm: the scale from max|e|), one MFMA row tile with the K split over the waves, row
// scale, + bias (the per-kernel projection's arithmetic), published to R_XIN.
__device__ __forceinline__ void role_idle(const Ctx &c, LdsP &s, int mi) {
    const RArgs &a = c.a;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    HeadTile ht;
#ifdef QT_RS_SMALL
    const bool mtp = a.mtp_w && mi >= 0;
    RTile16<EMB, 1, steps<EMB / 4>()> tm;
    float ms = 0.f, mb = 0.f;
    if (mtp) {
        tm.load(a.mtp_w, 16 * mi, wave * (EMB / 4), H);
        if (tid < 16) { ms = WBF ? 1.f : ldg(a.mtp_s + 16 * mi + tid); mb = ldg(a.mtp_b + 16 * mi + tid); }
    }
    int tok = -1;
#endif
    load_gains<4, 8, H>(a.final_norm, s.hd.gain);
    land();
    for (int step = 0; step < a.n_steps; step++) {
        const int par = step & 1;
        const bool last = step + 1 == a.n_steps;
        if (step > 0)
            for (int l = 0; l < c.L; l++) clear_share(c, par ^ 1, l);
#ifdef QT_RS_SMALL
        if (mtp) {
            static_assert(EMB / 8 == NT, "one 8-element unit of e per thread");
            float v[8];
            if (step == 0) {
                const float4 p = ldg(reinterpret_cast<const float4 *>(a.xin + 8 * tid));
                const float4 q = ldg(reinterpret_cast<const float4 *>(a.xin + 8 * tid + 4));
                v[0] = p.x; v[1] = p.y; v[2] = p.z; v[3] = p.w; v[4] = q.x; v[5] = q.y; v[6] = q.z; v[7] = q.w;
            } else {
                const uint4 r = ldg(reinterpret_cast<const uint4 *>(uni(ldg(a.cp_emb + step - 1)) + (size_t)tok * EMB + 8 * tid));
                const unsigned w4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
                for (int k = 0; k < 4; k++) { v[2 * k] = __uint_as_float(w4[k] << 16); v[2 * k + 1] = __uint_as_float(w4[k] & 0xFFFF0000u); }
            }
            float m = 0.f;
#pragma unroll
            for (int k = 0; k < 8; k++) m = fmaxf(m, fabsf(v[k]));
            m = group_max<64>(m);
            if (lane == 0) s.wst[wave] = m;
            __syncthreads();
            const QtPcScale ps = qt_pc_scale(fmaxf(fmaxf(s.wst[0], s.wst[1]), fmaxf(s.wst[2], s.wst[3])));
            pcw_put<EMB, 8>(s.pc, tid, v, ps.isc);
            wave_lds_order();   // unit tid: wave w makes the pieces of columns 512w .. +511, its own K slice
            AccT acc[1];
            rdot16<EMB, 1, steps<EMB / 4>(), 1>(tm, s.pc, wave * (EMB / 4), acc);
            ksplit_store<1>(acc, s.red);
            if (tid < 16) {
                RedT d[4];
                ksplit_row(s.red, tid, d);
                put(c.wp(par, 0, R_XIN + 16 * mi + tid), __fadd_rn(row_dot(d, ps.s, ms), mb));
            }
            __syncthreads();   // s.wst, s.red free for the next pass
        }
#endif
        ht.load(a, c.hc, wave, step);
        land();
#ifdef QT_RS_SMALL
        tok = head_phase(c, s.hd, ht, step, last);
#else
        head_phase(c, s.hd, ht, step, last);
#endif
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
#ifdef QT_RS_SMALL
    // head rows in the order Q, O, GU, head-only, DN: a Code Predictor's 2048-row lm head then
    // leaves DN (the last role of a layer to finish, whose head tile would land after the
    // others are already waiting for it) without rows
    else if (slot >= SD0 && slot < SI0) hc = NQ + NO + NG + NI + (slot - SD0) * 8 + x;
    else if (slot >= SI0) hc = NQ + NO + NG + (slot - SI0) * 8 + x;
#else
    else if (slot >= SD0 && slot < SI0) hc = NQ + NO + NG + (slot - SD0) * 8 + x;
    else if (slot >= SI0) hc = NQ + NO + NG + ND + (slot - SI0) * 8 + x;
#endif
#ifdef QT_RS_SMALL
    const int pos0 = a.cp ? 0 : *a.d_pos;   // a Code Predictor frame starts at position 0
#else
    const int pos0 = *a.d_pos;
#endif
    const Ctx c{a, s_layers, brsrc(a.reg), a.n_layers, pos0, a.with_head ? *a.d_frame : 0, *a.epoch, hc};
    if (slot < SA0) role_q(c, *reinterpret_cast<LdsP *>(lds), x, slot - SQ0);
    else if (slot < SO0) role_att(c, *reinterpret_cast<LdsA *>(lds), x, slot - SA0);
    else if (slot < SG0) role_o(c, *reinterpret_cast<LdsP *>(lds), (slot - SO0) * 8 + x);
    else if (slot < SD0) role_gu(c, *reinterpret_cast<LdsP *>(lds), (slot - SG0) * 8 + x);
    else if (XI == 0 || slot < SI0) role_dn(c, *reinterpret_cast<LdsD *>(lds), (slot - SD0) * 8 + x);
    else {
#ifdef QT_RS_SMALL
        const int mi = slot - SI0 < NMTP / 8 ? (slot - SI0) * 8 + x : -1;   // mtp rows of the first NMTP/8 idle slots
#else
        const int mi = -1;
#endif
        role_idle(c, *reinterpret_cast<LdsP *>(lds), mi);
    }
}
}  // namespace QT_RS_NS
}  // namespace ps

#ifdef QT_RSTEP_TRACE
extern "C" hipError_t QT_RS_NAME(qt_rstep, _trace_read)(unsigned long long *out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(ps::QT_RS_NS::rs_trace), sizeof(ps::QT_RS_NS::rs_trace), 0,
                               hipMemcpyDeviceToHost);
}
#endif

extern "C" int QT_RS_NAME(qt_rstep, _supported)(int prec, int hidden, int inter, int n_heads, int n_kv, int head_dim,
                                                int kv_max, int n_layers) {
    if (prec != ps::QT_RS_NS::PREC || hidden != ps::QT_RS_NS::H || inter != ps::QT_RS_NS::F)
        return 0;
    if (n_heads != ps::NH || n_kv != ps::NKV || head_dim != ps::HD) return 0;
    if (kv_max > ps::QT_RS_NS::ACH * ps::QT_RS_NS::ABLK * ps::KVB || n_layers < 1 || n_layers > ps::QT_RS_NS::MAXLR)
        return 0;
    int dev = 0, cus = 0, coop = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess) return 0;
    return coop && cus >= ps::NB;
}
// hand-off words (both parities) and winner words
extern "C" size_t QT_RS_NAME(qt_rstep, _region_words)(int n_layers) { return (size_t)2 * n_layers * ps::QT_RS_NS::LW; }
extern "C" size_t QT_RS_NAME(qt_rstep, _slot_words)(void) { return (size_t)2 * ps::QT_RS_NS::NHEAD * 2; }
#if !defined(QT_RS_SMALL) && !defined(QT_RS_Q4)
// attention key chunks per kv head, every build (the per-kernel attention must use the
// same split)
extern "C" int qt_rstep_chunks(void) { return ps::rs::ACH; }
#endif

extern "C" hipError_t QT_RS_NAME(qt_launch_rstep, )(const void *layers_dev, int n_layers, const float *final_norm,
                                                    const float *rope_cos, const float *rope_sin, uint16_t *kc,
                                                    uint16_t *vc, int kv_max, float eps, float scale, unsigned *reg,
                                                    unsigned long long *slots, float *hid, float *decx, float *xin,
                                                    int *d_pos, unsigned *epoch, int *err, int n_steps, int with_head,
                                                    const uint16_t *head_w, const uint16_t *emb, int vocab, int *d_frame,
                                                    int *hist, int hist_len, float *layer_out, hipStream_t st) {
    namespace rs = ps::QT_RS_NS;
    rs::RArgs a = {};
    a.layers = (const ps::Layer *)layers_dev; a.n_layers = n_layers;
    a.final_norm = final_norm; a.rope_cos = rope_cos; a.rope_sin = rope_sin;
    a.kc = kc; a.vc = vc; a.kv_max = kv_max; a.eps = eps; a.scale = scale;
    a.reg = reg; a.slots = slots; a.hid = hid; a.decx = decx; a.xin = xin; a.d_pos = d_pos; a.epoch = epoch;
    a.err = err; a.n_steps = n_steps; a.with_head = with_head;
    a.head_w = (const uint8_t *)head_w; a.emb = emb; a.vocab = vocab;
    a.d_frame = d_frame; a.hist = hist; a.hist_len = hist_len; a.layer_out = layer_out;
    if (n_steps <= 0 || n_layers <= 0 || n_layers > rs::MAXLR || kv_max > rs::ACH * rs::ABLK * ps::KVB)
        return hipErrorInvalidValue;
    if (!with_head && n_steps != 1) return hipErrorInvalidValue;   // without the head the next input is unknown
    if (with_head && (vocab != rs::NHEAD * rs::HEADR || !head_w || !emb || !d_frame || !hist || hist_len <= 0))
        return hipErrorInvalidValue;
    void *args[] = {(void *)&a};
    return hipLaunchCooperativeKernel((const void *)rs::k_rstep, dim3(ps::NB), dim3(rs::NT), args, 0, st);
}

#ifdef QT_RS_SMALL
// Code Predictor frame (qwen_tts_code_predictor.c:926-1045) in one launch: n_passes passes
// of the n_layers CP layers at positions 0 .. n_passes-1, pass 0 on xin, the lm head after
// every pass s >= 1 writing codes[s], pass s+1 on row codes[s] of its table.  cp_tab: device
// array of 45 pointers (15 lm heads [vocab][1024] in the build's weight type, their 15 row-
// scale arrays (int8; unused with bf16), the 15 input tables: the Talker's codec embedding,
// then CP embeddings 0 .. 13).  codes[0] is the frame's input code.
extern "C" hipError_t QT_RS_NAME(qt_launch_rstep, _cp)(const void *layers_dev, int n_layers, const float *final_norm,
                                           const float *rope_cos, const float *rope_sin, uint16_t *kc, uint16_t *vc,
                                           int kv_max, float eps, float scale, unsigned *reg, unsigned long long *slots,
                                           float *hid, float *decx, float *xin, int *d_pos, unsigned *epoch, int *err,
                                           int n_passes, const void *const *cp_tab, int vocab, int *codes,
                                           const uint8_t *mtp_w, const float *mtp_s, const float *mtp_b,
                                           hipStream_t st) {
    namespace rs = ps::QT_RS_NS;
    rs::RArgs a = {};
    a.layers = (const ps::Layer *)layers_dev; a.n_layers = n_layers;
    a.final_norm = final_norm; a.rope_cos = rope_cos; a.rope_sin = rope_sin;
    a.kc = kc; a.vc = vc; a.kv_max = kv_max; a.eps = eps; a.scale = scale;
    a.reg = reg; a.slots = slots; a.hid = hid; a.decx = decx; a.xin = xin; a.d_pos = d_pos; a.epoch = epoch;
    a.err = err; a.n_steps = n_passes; a.with_head = 0; a.vocab = vocab;
    a.cp = 1;
    a.cp_head = reinterpret_cast<const uint8_t *const *>(cp_tab);
    a.cp_hs = reinterpret_cast<const float *const *>(cp_tab + 15);
    a.cp_emb = reinterpret_cast<const uint16_t *const *>(cp_tab + 30);
    a.cp_codes = codes;
    a.mtp_w = mtp_w; a.mtp_s = mtp_s; a.mtp_b = mtp_b;
    if (mtp_w && ((!rs::WBF && !mtp_s) || !mtp_b)) return hipErrorInvalidValue;
    if (n_passes < 1 || n_passes > 16 || n_passes > kv_max || n_layers <= 0 || n_layers > rs::MAXLR ||
        kv_max > rs::ACH * rs::ABLK * ps::KVB)
        return hipErrorInvalidValue;
    if (!cp_tab || !codes || !xin || vocab < 1 || vocab > rs::NHEAD * rs::HEADR) return hipErrorInvalidValue;
    if (rs::WBF && vocab % rs::HEADR) return hipErrorInvalidValue;   // bf16 head tiles read whole 16-row tiles
    void *args[] = {(void *)&a};
    return hipLaunchCooperativeKernel((const void *)rs::k_rstep, dim3(ps::NB), dim3(rs::NT), args, 0, st);
}
#endif
