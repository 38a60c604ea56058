// qt_pstep.hip — the whole Talker decode step (optionally many greedy steps) as ONE
// persistent cooperative kernel for gfx950, synchronised by data instead of barriers.
//
// Why: a decode step is ~170 dependent phases (6 per layer x 28 + head).  As separate
// kernels each costs at least the ~2.4 us launch cycle; with device-wide barriers each
// still costs ~3-5 us (store acknowledgement, two atomic round trips, release, reload).
// Here every activation value is stored together with the number of the decode step
// that produced it, as one 64-bit word {tag:32 | f32 bits:32} written with an
// agent-scope (write-through, sc1) store.  A consumer reads the words it needs with
// agent-scope loads and retries only the ones whose tag is not yet the current step's:
// no counters, no barriers, no store acknowledgement on the producer side.  A hop
// costs one write plus one read of the device coherence point (about 1 us).
//
// 256 workgroups (one per CU, co-resident by cooperative launch), 4 waves each.
// Workgroup b has group g = b % 8 (one kv head; workgroups of one group share an XCD
// under round-robin dispatch) and index c = b / 8 within it.  Phases of layer l (same
// math as qwen_tts_talker.c:580-690, per-kernel twins in qt_matvec.hip / qt_attn.hip):
//   A  q|k|v rows of kv group g: 16 rows per workgroup (= RMSNorm(x) . W_qkv)
//   B  attention chunk c of kv head g (2 query heads): q/k per-head norm, RoPE, KV
//      append (bf16 truncation) by the chunk holding pos, scores, softmax, P.V;
//      the chunk's (max, sum, o[2][128]) is published
//   M  merge of the chunk partials for 8 of the 2048 attention outputs
//   C  xa = x + W_o . attn                    H/256 rows per workgroup
//   D  h  = SwiGLU(W_gu . RMSNorm(xa))        2F/256 rows per workgroup
//   E  x' = xa + W_dn . h                     H/256 rows per workgroup
// and per greedy step the codec head (12 rows per workgroup, masked local argmax) and
// the global argmax over the 256 local winners, computed redundantly by everyone.
//
// Every workgroup stages a phase's input once into LDS (one agent-scope load per
// element), so the waves read it from LDS.  The weights (and int8 row scales, norm
// gains) of the NEXT phase are loaded into registers right after the current phase's
// output has been issued: a wave that issues a large tile stalls until much of it has
// arrived (the CU's share of HBM bandwidth is ~31 GB/s), and that stall then overlaps
// the output's trip to the other workgroups instead of delaying it.
//
// Reuse safety: the activation ring has one slot per (step parity, layer, phase).  A
// slot written at step s is rewritten at step s+2 only; no workgroup can be a whole
// step ahead of another, because every step's phase A reads the complete x written by
// all workgroups.  KV rows are read only after they were written (row pos is patched
// from LDS in the step that writes it), so no cache holds a stale copy.
// Every wait is bounded: on timeout the kernel sets an error flag, the others see it
// and stop waiting, and the launch runs to its end.
#include "qt_step_common.h"

namespace ps {
struct Args {
    const Layer *layers;
    int n_layers;
    const float *final_norm, *rope_cos, *rope_sin;
    uint16_t *kc, *vc;            // [L][NKV][kv_max][HD]
    int kv_max;
    float eps, scale;
    unsigned long long *ring;     // tagged words, [2][L][slots] + [2][NB][2] head slots
    float *hid, *decx;            // [H] final normed hidden and residual of the last step
    float *xin;                   // [H] step-0 input when no token is given
    int *d_pos;                   // position of step 0; advanced by n_steps
    unsigned *epoch;              // tag of step 0; advanced by n_steps
    int *err;
    int n_steps;
    int with_head;
    const uint8_t *head_w;        // bf16 [vocab][H]
    const uint16_t *emb;          // bf16 [vocab][H]
    int vocab;
    int *d_frame, *hist;
    int hist_len;
};

// Optional phase trace (build with -DQT_PSTEP_TRACE): s_memrealtime (100 MHz) of every
// workgroup when its input for a phase has arrived (w=0), at two points inside the
// phase (w=2, 3) and when its output and the next loads have been issued (w=1),
// indexed by the phase's number in the launch.  Marks are kept in LDS and
// written out once at the end of the launch (a global store per mark would add its
// acknowledgement to the next vmcnt wait); qt_pstep_trace_read copies them out.
#ifdef QT_PSTEP_TRACE
constexpr int TRACE_PH = 520;
__device__ unsigned long long ps_trace[TRACE_PH * 4 * NB];
#define PS_TRACE_LDS __shared__ unsigned long long s_trace[TRACE_PH * 4];
#define PS_MARK(k, w)                                                                          \
    do {                                                                                       \
        if (threadIdx.x == 0 && (unsigned)(k) < (unsigned)TRACE_PH)                            \
            s_trace[(size_t)(k) * 4 + (w)] = __builtin_amdgcn_s_memrealtime();                 \
    } while (0)
#define PS_TRACE_FLUSH()                                                                       \
    do {                                                                                       \
        __syncthreads();                                                                       \
        for (int i_ = threadIdx.x; i_ < TRACE_PH * 4; i_ += (int)blockDim.x)                   \
            ps_trace[(size_t)i_ * NB + blockIdx.x] = s_trace[i_];                              \
    } while (0)
#define PS_TRACE_CLEAR()                                                                       \
    do {                                                                                       \
        for (int i_ = threadIdx.x; i_ < TRACE_PH * 4; i_ += (int)blockDim.x) s_trace[i_] = 0;  \
    } while (0)
#else
#define PS_TRACE_LDS
#define PS_MARK(k, w) do { } while (0)
#define PS_TRACE_FLUSH() do { } while (0)
#define PS_TRACE_CLEAR() do { } while (0)
#endif


// ---- ring layout (tagged words) -----------------------------------------------------------
template <int H, int F>
struct Ring {
    static constexpr size_t OQKV = 0, OPART = QKVR, OATT = OPART + (size_t)NKV * G * HPK * PS,
                            OXA = OATT + QD, OH = OXA + H, OX = OH + F, P = OX + H;
    unsigned long long *base;
    int L;
    __device__ __forceinline__ unsigned long long *blk(int par, int l) const { return base + ((size_t)par * L + l) * P; }
    __device__ __forceinline__ unsigned long long *slots(int par) const { return base + (size_t)2 * L * P + (size_t)par * NB * 2; }
};

// ---- the kernel ---------------------------------------------------------------------------
// LDS of the attention phase (B) and the merge (M)
template <int HPK>
struct AttLds {
    __attribute__((aligned(16))) uint16_t qp[16][HD];          // rotated queries as bf16 pieces, row 4h+p (qt_attn_mf.h)
    __attribute__((aligned(16))) uint16_t pp[16][KVB];         // probability pieces of a block (k-tile w: wave w)
    float ml[NWB][HPK][2];                                      // per-k-tile (max, exp-sum)
    float mst[G * 10];                                          // merge (M) inputs
    __attribute__((aligned(16))) uint16_t knew[HD], vnew[HD];   // key/value at pos (bf16)
};

template <int PREC, int H, int F, int NW>
__global__ __launch_bounds__(NW * 64, 1) void k_pstep(Args a) {
    constexpr int NT = NW * 64;                    // threads per workgroup
    constexpr int RPW_QKV = QKVR / (NB * NW);      // 4 (NW 4) or 2 (NW 8)
    constexpr int RPW_O = H / (NB * NW);           // rows per wave of W_o
    constexpr int RPW_GU = 2 * F / (NB * NW);      // rows per wave of gate|up
    constexpr int RPW_DN = H / (NB * NW);          // rows per wave of W_down
    constexpr int HEADR = 12;                      // 3072-row codec head: rows per workgroup
    constexpr int RPW_HEAD = (HEADR + NW - 1) / NW;   // 3 (NW 4) or 2 (NW 8; waves 6, 7 idle)
    static_assert(RPW_QKV >= 1 && RPW_O >= 1 && RPW_DN >= 1 && RPW_QKV * NB * NW == QKVR && RPW_O * NB * NW == H &&
                  RPW_GU * NB * NW == 2 * F && RPW_DN * NB * NW == H, "row split");
    // int8: exact activation pieces (PI); at hidden 2048 the dots run on MFMA (MF), with
    // 4 rows per wave for q|k|v and gate|up and 8 rows per workgroup split over the waves'
    // column slices for O and down
    constexpr bool PI = PREC == QT_INT8;
    constexpr bool MF = PI && H == 2048 && NW == 4;
    constexpr int RGU = RPW_GU / 3;                // gate|up rows per piece (4 or 2)
    static_assert(!MF || (RPW_QKV == 4 && RGU == 4 && H / NB == 8), "MFMA tile shapes");
    using TQKV = std::conditional_t<MF, TileM4<H, false>, Tile<PREC, H, RPW_QKV>>;
    using TO = std::conditional_t<MF, TileK8<QD>, Tile<PREC, QD, RPW_O>>;
    using TGU = std::conditional_t<MF, TileM4<H, true>, Tile<PREC, H, RGU>>;
    using TDN = std::conditional_t<MF, TileK8<F>, Tile<PREC, F, RPW_DN>>;
    using THEAD = Tile<QT_BF16, H, RPW_HEAD>;
    using R = Ring<H, F>;
    static_assert(RPW_GU % 3 == 0 && RGU % 2 == 0, "gate/up pairs stay in one piece");
    constexpr int EP = Epc<PREC>::v, EH = Epc<QT_BF16>::v;   // chunk sizes: layers, codec head
    using PH = PosChunk<EP, H>;

    __shared__ __align__(16) float s_x[H];       // layer input (kept for C's residual)
    __shared__ __align__(16) float s_xa[H];      // post-attention residual (kept for E)
    __shared__ __align__(16) float s_xn[H];      // RMS-normalised input of A / D / head
    __shared__ __align__(16) float s_qkv[HPK * HD + 2 * HD];
    __shared__ __align__(16) AttLds<HPK> att;                 // attention chunk (B), merge input (M)
    __shared__ float wbest_v[NW];
    __shared__ int wbest_i[NW];
    __shared__ Layer s_layers[MAXL];
    __shared__ __align__(16) uint16_t s_kv[2][KVB * HD];          // K, V rows of the attention chunk (B)
    // attn (C) / h (E) / head slots share the K/V buffer: B is done with it before C
    // writes, and the next layer's K/V copy is issued after E's dot products
    static_assert((F > QD ? F : QD) * 4 <= 2 * KVB * HD * 2, "s_in fits the K/V buffer");
    float *const s_in = reinterpret_cast<float *>(&s_kv[0][0]);
    __shared__ __align__(16) float s_gain[2][H];                  // norm gains: [0] input (A), [1] post (D) / final
    // int8 pieces: A's in the s_xn space (unused by int8 layers), C/D/E's in the second
    // half of the K/V buffer (free from C until the next layer's K/V copy after E)
    static_assert(4 * H <= H * 4 && 32768 + 4 * (F > QD ? F : QD) <= 2 * KVB * HD * 2, "pieces fit");
    uint8_t *const pcA = reinterpret_cast<uint8_t *>(s_xn);
    uint8_t *const pcB = reinterpret_cast<uint8_t *>(&s_kv[0][0]) + 32768;
    __shared__ __align__(16) int s_red[PI ? NW * 3 * 64 : 1];     // MFMA part sums
    __shared__ float s_wst[2 * NW];                               // per-wave statistics of a gather (pieces)
    PS_TRACE_LDS

    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: row bases are scalar
    const int g = b % NKV, c = b / NKV;            // kv group, index within the group
    R ring{a.ring, a.n_layers};
    const int pos0 = *a.d_pos;
    const unsigned tag0 = *a.epoch;
    const int frame0 = a.with_head ? *a.d_frame : 0;
    const int L = a.n_layers;
    int tok = -1;   // greedy token of the previous step (-1: input from a.xin)
    int ph = 0;     // phase counter (trace index)
    (void)ph;

    // rows this workgroup owns in each projection
    // A: 16 q|k|v rows of group g: c < 16 -> q rows of head 2g + c/8, c < 24 -> k, else v
    const int qkv_row0 = (c < 16) ? (2 * g + (c >> 3)) * HD + (c & 7) * 16
                       : (c < 24) ? QD + g * HD + (c - 16) * 16 : QD + KVD + g * HD + (c - 24) * 16;
    const int rw_qkv = qkv_row0 + wave * RPW_QKV;
    const int rw_o = b * (RPW_O * NW) + wave * RPW_O;
    const int rw_gu = b * (RPW_GU * NW) + wave * RPW_GU;
    const int rw_dn = b * (RPW_DN * NW) + wave * RPW_DN;
    const bool head_on = wave * RPW_HEAD < HEADR;
    const int rw_head = b * HEADR + (head_on ? wave * RPW_HEAD : 0);

    PS_TRACE_CLEAR();
    // the layer table lives in LDS: reading it never waits behind weight loads
    for (int i = tid; i < L * (int)(sizeof(Layer) / 8); i += NT)
        reinterpret_cast<unsigned long long *>(s_layers)[i] = ldg(reinterpret_cast<const unsigned long long *>(a.layers) + i);
    qt_att_zero_rows<HPK>(&att.qp[0][0], HD, tid, NT);
    qt_att_zero_rows<HPK>(&att.pp[0][0], KVB, tid, NT);
    __syncthreads();

    TQKV tq;
    tq.load(s_layers[0].w[0], lsc<PREC>(s_layers[0], 0), rw_qkv);
    load_gains<NW, EP, H>(s_layers[0].in_norm, s_gain[0]);


    for (int step = 0; step < a.n_steps; step++) {
        const int par = step & 1;
        const unsigned tag = tag0 + (unsigned)step;
        const int pos = pos0 + step;
        const int Lk = pos + 1;
        int CH = (Lk + G - 1) / G;
        CH = (CH + 15) & ~15;
        const int nch = (Lk + CH - 1) / CH;
        const int j0 = c * CH;
        const int n = (c < nch) ? min(CH, Lk - j0) : 0;

        // B's operands, loaded one phase ahead: K/V rows of this workgroup's chunk (the
        // first KVB keys) copied straight into LDS by global_load_lds_dwordx4 (no VGPRs
        // held; one wave instruction moves 4 keys = 1 KiB), the q/k norm gains and the
        // RoPE row of pos.  Row pos is never loaded (its stale bits must not enter any
        // cache: it is written by this step's B and read from the next step on); lanes
        // past the chunk end load nothing.
        float qn0 = 0.f, qn1 = 0.f, kn0 = 0.f, kn1 = 0.f, rc = 0.f, rsn = 0.f;
        auto stage_kv = [&](int lk, int kb, bool doK, bool doV) {
            const uint16_t *Kl = a.kc + (((size_t)lk * NKV + g) * a.kv_max) * HD;
            const uint16_t *Vl = a.vc + (((size_t)lk * NKV + g) * a.kv_max) * HD;
            const int nk = min(KVB, n - kb);
            const int ninst = (nk + 3) >> 2;
            const int jq = lane >> 4, js = lane & 15;
            for (int i = wave; i < ninst; i += NW) {
                const int jl = i * 4 + jq, jj = kb + jl;
                if (jj < n && j0 + jj != pos) {   // slot js of block row jl: swizzled source chunk
                    const size_t row = (size_t)(j0 + jj) * HD;
                    if (doK) lds_copy16(Kl + row + qt_kslot(jl, js) * 8, &s_kv[0][i * 4 * HD]);
                    if (doV) lds_copy16(Vl + row + qt_vslot(jl, js) * 8, &s_kv[1][i * 4 * HD]);
                }
            }
        };
        auto prefetch_kv = [&](int lk) {
            if (n > 0) stage_kv(lk, 0, true, true);
            const float *qnp = uni(s_layers[lk].qn), *knp = uni(s_layers[lk].kn);
            qn0 = ldg(qnp + lane); qn1 = ldg(qnp + lane + 64); kn0 = ldg(knp + lane); kn1 = ldg(knp + lane + 64);
            rc = ldg(a.rope_cos + (size_t)pos * 64 + lane); rsn = ldg(a.rope_sin + (size_t)pos * 64 + lane);
        };
        for (int l = 0; l < L; l++) {
            const Layer &ly = s_layers[l];
            unsigned long long *blk = ring.blk(par, l);

            // ---------------- A: q|k|v rows -----------------
            if (l > 0) {
                const unsigned long long *src = ring.blk(par, l - 1) + R::OX;
                gather<H / NT, NT>(H, [&](int i) { return src + i; }, s_x, tag, a.err, PH(), PI ? s_wst : nullptr, s_gain[0]);
            } else {
                float xv[H / NT];
#pragma unroll
                for (int k = 0; k < H / NT; k++) {
                    const int i = tid + k * NT;
                    xv[k] = tok < 0 ? ldg(a.xin + i) : bf16f(ldg(a.emb + (size_t)tok * H + i));
                    s_x[xpos<EP, H>(i)] = xv[k];
                }
                if (PI) {
                    __syncthreads();                 // the gains' LDS copy has landed for every wave
                    pc_stats<H / NT, NT>(xv, H, s_gain[0], PH(), s_wst);
                }
                __syncthreads();
            }
            PS_MARK(ph, 0);
            if constexpr (MF) {
                const float sA = stage_norm_pc<true, H, NT>(s_x, s_gain[0], a.eps, pcA, s_wst);
                PS_MARK(ph, 2);
                int d[4];
                mf_store4(mf_dot4(tq, pcA), s_red + wave * 192);
                mf_rowsum(s_red + wave * 192, lane & 3, d);
                if (lane < 4)
                    st_tag(blk + R::OQKV + rw_qkv + lane, __fmul_rn(qt_pc_dot(d[0], d[1], d[2], d[3], sA), tq.rs[0]), tag);
                PS_MARK(ph, 3);
            } else if constexpr (PI) {
                const float sA = stage_norm_pc<false, H, NT>(s_x, s_gain[0], a.eps, pcA, s_wst);
                PS_MARK(ph, 2);
                float acc[RPW_QKV];
                tile_dot_pc<H, RPW_QKV>(tq, pcA, sA, acc);
#pragma unroll
                for (int r = 0; r < RPW_QKV; r++)
                    if (lane == r) st_tag(blk + R::OQKV + rw_qkv + r, __fmul_rn(acc[r], tq.rs[r]), tag);
                PS_MARK(ph, 3);
            } else {
                stage_norm<PREC, H>(s_x, s_gain[0], a.eps, s_xn);
                PS_MARK(ph, 2);
                float acc[RPW_QKV];
                tile_dot<PREC, H, RPW_QKV>(tq, s_xn, acc);
#pragma unroll
                for (int r = 0; r < RPW_QKV; r++)
                    if (lane == r) st_tag(blk + R::OQKV + rw_qkv + r, PREC == QT_INT8 ? __fmul_rn(acc[r], tq.rs[r]) : acc[r], tag);
                PS_MARK(ph, 3);
            }
            if (l == 0) prefetch_kv(0);
            // next operands (issued after this phase's output): W_o, first gate|up piece, post-norm gains
            TO to;
            if constexpr (MF) to.load(ly.w[1], ly.s[1], b * (H / NB), wave);
            else to.load(ly.w[1], lsc<PREC>(ly, 1), rw_o);
            TGU tg0, tg1, tg2;
            tg0.load(ly.w[2], lsc<PREC>(ly, 2), rw_gu);
            load_gains<NW, EP, H>(ly.post_norm, s_gain[1]);
            PS_MARK(ph, 1); ph++;

            // ---------------- B: attention chunk -----------------
            {
                const unsigned long long *src = blk + R::OQKV;
                gather<2, NT>(n > 0 ? HPK * HD + 2 * HD : 0, [&](int i) {
                    return src + (i < HPK * HD ? g * HPK * HD + i
                                  : i < HPK * HD + HD ? QD + g * HD + (i - HPK * HD) : QD + KVD + g * HD + (i - HPK * HD - HD));
                }, s_qkv, tag, a.err);
            }
            PS_MARK(ph, 0);
            if (n > 0) {
                const bool append = (pos >= j0 && pos < j0 + n);
                const int ntask = HPK + (append ? 1 : 0);
                for (int t = wave; t < ntask; t += NW) {
                    const bool isk = (t == HPK);
                    const float *srcv = isk ? s_qkv + HPK * HD : s_qkv + t * HD;
                    const float w0 = isk ? kn0 : qn0, w1 = isk ? kn1 : qn1;
                    const float x0 = srcv[lane], x1 = srcv[lane + 64];
                    const float ss = group_sum<64>(x0 * x0 + x1 * x1);
                    const float inv = 1.0f / sqrtf(ss / (float)HD + a.eps);
                    const float n0 = (x0 * inv) * w0, n1 = (x1 * inv) * w1;
                    const float r0 = fmaf(n0, rc, -(n1 * rsn)), r1 = fmaf(n1, rc, n0 * rsn);
                    if (!isk) {
                        qt_put_pieces(&att.qp[4 * t][lane], HD, r0);
                        qt_put_pieces(&att.qp[4 * t][lane + 64], HD, r1);
                    } else {
                        const float *vs = s_qkv + HPK * HD + HD;
                        const uint16_t k0 = f2bf_trunc(r0), k1 = f2bf_trunc(r1);
                        const uint16_t v0 = f2bf_trunc(vs[lane]), v1 = f2bf_trunc(vs[lane + 64]);
                        att.knew[lane] = k0; att.knew[lane + 64] = k1;
                        att.vnew[lane] = v0; att.vnew[lane + 64] = v1;
                        const int r = pos - j0;            // its row in the first staged block
                        if (r < KVB) {
                            s_kv[0][qt_kidx(r, lane)] = k0; s_kv[0][qt_kidx(r, lane + 64)] = k1;
                            s_kv[1][qt_vidx(r, lane)] = v0; s_kv[1][qt_vidx(r, lane + 64)] = v1;
                        }
                    }
                }
                qt_att_zero_vrows(s_kv[1], min(KVB, n), (min(KVB, n) + 31) & ~31, tid, NT);
                __syncthreads();
                // per LDS block (qt_attn_mf.h, the same arithmetic as k_attn): wave w scores
                // its k-tile (block rows 32w .. +31), barrier, then takes dims [32w, 32w + 32)
                // of P.V over the k-tiles holding keys
                const float scale2 = a.scale * QT_LOG2E;
                QtAttRun run;
                qt_att_run_init(run);
                for (int kb = 0; kb < n; kb += KVB) {
                    const int nk = min(KVB, n - kb);
                    if (kb > 0) {   // chunks longer than KVB keys (caches beyond G*KVB positions)
                        __syncthreads();
                        stage_kv(l, kb, true, true);
                        __builtin_amdgcn_s_waitcnt(0);     // the barrier does not wait for LDS copies
                        const int nrow = pos - j0 - kb;    // the appended key's row, if in this block
                        if (wave == 0 && nrow >= 0 && nrow < nk) qt_att_put_kv(s_kv[0], s_kv[1], nrow, att.knew, att.vnew, lane);
                        qt_att_zero_vrows(s_kv[1], nk, (nk + 31) & ~31, tid, NT);
                        __syncthreads();
                    }
                    if (wave < NWB && 32 * wave < nk)
                        qt_att_tiles<HPK>(&att.qp[0][0], s_kv[0], &att.pp[0][0], KVB, &att.ml[0][0][0], wave, nk, scale2,
                                          lane);
                    __syncthreads();
                    PS_MARK(ph, 2);
                    if (wave < NWB) {
                        float o[2], M, lsum;
                        qt_att_pv_n<HPK>((nk + 31) >> 5, &att.pp[0][0], KVB, &att.ml[0][0][0], s_kv[1], 32 * wave, lane,
                                         o, M, lsum);
                        qt_att_run_add(run, o, M, lsum);
                    }
                }
                PS_MARK(ph, 3);
                unsigned long long *mypart = blk + R::OPART + (size_t)(g * G + c) * HPK * PS;
                const int hq = lane >> 4, od = 32 * wave + (lane & 15);
                if (wave < NWB && hq < HPK) {
                    st_tag(mypart + hq * PS + 2 + od, run.o[0], tag);
                    st_tag(mypart + hq * PS + 2 + od + 16, run.o[1], tag);
                    if (wave == 0 && (lane & 15) == 0) {
                        st_tag(mypart + hq * PS, run.m, tag);
                        st_tag(mypart + hq * PS + 1, run.l, tag);
                    }
                }
                if (append && wave == NW - 1) {
                    // KV append: agent-scope 32-bit stores of adjacent bf16 pairs (after the
                    // attention, so no wait inside it covers their acknowledgement)
                    uint32_t *kd = reinterpret_cast<uint32_t *>(a.kc + (((size_t)l * NKV + g) * a.kv_max + pos) * HD);
                    uint32_t *vd = reinterpret_cast<uint32_t *>(a.vc + (((size_t)l * NKV + g) * a.kv_max + pos) * HD);
                    const uint32_t kk = (uint32_t)att.knew[2 * lane] | ((uint32_t)att.knew[2 * lane + 1] << 16);
                    const uint32_t vv = (uint32_t)att.vnew[2 * lane] | ((uint32_t)att.vnew[2 * lane + 1] << 16);
                    __hip_atomic_store(kd + lane, kk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(vd + lane, vv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            tg1.load(ly.w[2], lsc<PREC>(ly, 2), rw_gu + RGU);
            PS_MARK(ph, 1); ph++;

            // ---------------- M: merge 8 attention outputs -----------------
            {
                const int hh = c >> 4, d0 = (c & 15) * 8;
                const unsigned long long *gp = blk + R::OPART + (size_t)g * G * HPK * PS + hh * PS;
                // element i: chunk i/10, field i%10 (0 max, 1 sum, 2.. dims d0..d0+7)
                float *st = att.mst;
                gather<2, NT>(nch * 10, [&](int i) {
                    const int cc = i / 10, f = i % 10;
                    return gp + (size_t)cc * HPK * PS + (f < 2 ? f : 2 + d0 + (f - 2));
                }, st, tag, a.err);
                PS_MARK(ph, 0);
                // half-wave per output dim d0 + dd, lane = chunk (waves 0..NWB-1)
                if (wave < NWB) {
                    const int half = lane >> 5, cc = lane & 31, dd = 2 * wave + half;
                    const bool valid = cc < nch;
                    const float r = softmax_merge32(valid ? st[cc * 10] : 0.f, valid ? st[cc * 10 + 1] : 0.f,
                                                    valid ? st[cc * 10 + 2 + dd] : 0.f, valid);
                    if (cc == 0) st_tag(blk + R::OATT + (2 * g + hh) * HD + d0 + dd, r, tag);
                }
            }
            tg2.load(ly.w[2], lsc<PREC>(ly, 2), rw_gu + 2 * RGU);
            PS_MARK(ph, 1); ph++;

            // ---------------- C: xa = x + W_o . attn -----------------
            {
                const unsigned long long *src = blk + R::OATT;
                gather<QD / NT, NT>(QD, [&](int i) { return src + i; }, s_in, tag, a.err, PosChunk<EP, QD>(),
                                    PI ? s_wst : nullptr);
            }
            PS_MARK(ph, 0);
            if constexpr (PI) {
                const float sC = stage_pc<MF, QD, NT>(s_in, s_wst, pcB);
                if constexpr (MF) {
                    int d[4];
                    mf_rows8<NW>(mf_dot8(to, pcB, wave), s_red, wave, d);
                    if (tid < H / NB) {
                        const int r = b * (H / NB) + tid;
                        const float v = __fmul_rn(qt_pc_dot(d[0], d[1], d[2], d[3], sC), to.rs);
                        st_tag(blk + R::OXA + r, __fadd_rn(s_x[xpos<EP, H>(r)], v), tag);
                    }
                } else {
                    float acc[RPW_O];
                    tile_dot_pc<QD, RPW_O>(to, pcB, sC, acc);
#pragma unroll
                    for (int r = 0; r < RPW_O; r++)
                        if (lane == r)
                            st_tag(blk + R::OXA + rw_o + r, __fadd_rn(s_x[xpos<EP, H>(rw_o + r)], __fmul_rn(acc[r], to.rs[r])), tag);
                }
            } else {
                float acc[RPW_O];
                tile_dot<PREC, QD, RPW_O>(to, s_in, acc);
#pragma unroll
                for (int r = 0; r < RPW_O; r++)
                    if (lane == r) {
                        const float v = PREC == QT_INT8 ? __fmul_rn(acc[r], to.rs[r]) : acc[r];
                        st_tag(blk + R::OXA + rw_o + r, __fadd_rn(s_x[xpos<EP, H>(rw_o + r)], v), tag);
                    }
            }
            TDN td;
            if constexpr (MF) td.load(ly.w[3], ly.s[3], b * (H / NB), wave);
            else td.load(ly.w[3], lsc<PREC>(ly, 3), rw_dn);
            PS_MARK(ph, 1); ph++;

            // ---------------- D: h = SwiGLU(W_gu . RMSNorm(xa)) -----------------
            {
                const unsigned long long *src = blk + R::OXA;
                gather<H / NT, NT>(H, [&](int i) { return src + i; }, s_xa, tag, a.err, PH(), PI ? s_wst : nullptr, s_gain[1]);
            }
            PS_MARK(ph, 0);
            if constexpr (MF) {
                const float sD = stage_norm_pc<true, H, NT>(s_xa, s_gain[1], a.eps, pcB, s_wst);
                PS_MARK(ph, 2);
                int *red = s_red + wave * 192;
                i32x4 acc3[3];
                mf_dot4x3(tg0, tg1, tg2, pcB, acc3);
                mf_store4(acc3[0], red);
                mf_store4(acc3[1], red + 64);
                mf_store4(acc3[2], red + 128);
                // lane t < 6: h element (piece t/2, pair t%2) from rows 2i (gate), 2i+1 (up)
                const int pc = lane >> 1, i = lane & 1;
                int dg[4], du[4];
                mf_rowsum(red + (pc < 3 ? pc : 0) * 64, 2 * i, dg);
                mf_rowsum(red + (pc < 3 ? pc : 0) * 64, 2 * i + 1, du);
                if (lane < 6) {
                    const float sg = pc == 0 ? tg0.rs[0] : pc == 1 ? tg1.rs[0] : tg2.rs[0];
                    const float su = pc == 0 ? tg0.rs[1] : pc == 1 ? tg1.rs[1] : tg2.rs[1];
                    const float gt = __fmul_rn(qt_pc_dot(dg[0], dg[1], dg[2], dg[3], sD), sg);
                    const float up = __fmul_rn(qt_pc_dot(du[0], du[1], du[2], du[3], sD), su);
                    st_tag(blk + R::OH + ((rw_gu + pc * RGU) >> 1) + i, gt / (1.0f + expf(-gt)) * up, tag);
                }
            } else if constexpr (PI) {
                const float sD = stage_norm_pc<false, H, NT>(s_xa, s_gain[1], a.eps, pcB, s_wst);
                PS_MARK(ph, 2);
                float acc[3][RGU];
                tile_dot_pc<H, RGU>(tg0, pcB, sD, acc[0]);
                tile_dot_pc<H, RGU>(tg1, pcB, sD, acc[1]);
                tile_dot_pc<H, RGU>(tg2, pcB, sD, acc[2]);
#pragma unroll
                for (int pc = 0; pc < 3; pc++) {
                    const TGU &t = pc == 0 ? tg0 : pc == 1 ? tg1 : tg2;
#pragma unroll
                    for (int i = 0; i < RGU / 2; i++)
                        if (lane == pc * (RGU / 2) + i) {
                            const float gt = __fmul_rn(acc[pc][2 * i], t.rs[2 * i]);
                            const float up = __fmul_rn(acc[pc][2 * i + 1], t.rs[2 * i + 1]);
                            st_tag(blk + R::OH + ((rw_gu + pc * RGU) >> 1) + i, gt / (1.0f + expf(-gt)) * up, tag);
                        }
                }
            } else {
                stage_norm<PREC, H>(s_xa, s_gain[1], a.eps, s_xn);
                PS_MARK(ph, 2);
                float acc[3][RGU];
                tile_dot<PREC, H, RGU>(tg0, s_xn, acc[0]);
                tile_dot<PREC, H, RGU>(tg1, s_xn, acc[1]);
                tile_dot<PREC, H, RGU>(tg2, s_xn, acc[2]);
                // rows 2i, 2i+1 of a piece are the gate and up rows of one h element
#pragma unroll
                for (int pc = 0; pc < 3; pc++) {
                    const TGU &t = pc == 0 ? tg0 : pc == 1 ? tg1 : tg2;
#pragma unroll
                    for (int i = 0; i < RGU / 2; i++)
                        if (lane == pc * (RGU / 2) + i) {
                            const float gt = PREC == QT_INT8 ? __fmul_rn(acc[pc][2 * i], t.rs[2 * i]) : acc[pc][2 * i];
                            const float up = PREC == QT_INT8 ? __fmul_rn(acc[pc][2 * i + 1], t.rs[2 * i + 1]) : acc[pc][2 * i + 1];
                            st_tag(blk + R::OH + ((rw_gu + pc * RGU) >> 1) + i, gt / (1.0f + expf(-gt)) * up, tag);
                        }
                }
            }
            PS_MARK(ph, 3);
            if (l + 1 < L) {
                tq.load(s_layers[l + 1].w[0], lsc<PREC>(s_layers[l + 1], 0), rw_qkv);
                load_gains<NW, EP, H>(s_layers[l + 1].in_norm, s_gain[0]);
            }
            PS_MARK(ph, 1); ph++;

            // ---------------- E: x' = xa + W_dn . h -----------------
            {
                const unsigned long long *src = blk + R::OH;
                gather<F / NT, NT>(F, [&](int i) { return src + i; }, s_in, tag, a.err, PosChunk<EP, F>(),
                                   PI ? s_wst : nullptr);
            }
            PS_MARK(ph, 0);
            if constexpr (PI) {
                const float sE = stage_pc<MF, F, NT>(s_in, s_wst, pcB);
                PS_MARK(ph, 2);
                if constexpr (MF) {
                    int d[4];
                    mf_rows8<NW>(mf_dot8(td, pcB, wave), s_red, wave, d);
                    if (tid < H / NB) {
                        const int r = b * (H / NB) + tid;
                        const float v = __fmul_rn(qt_pc_dot(d[0], d[1], d[2], d[3], sE), td.rs);
                        st_tag(blk + R::OX + r, __fadd_rn(s_xa[xpos<EP, H>(r)], v), tag);
                    }
                } else {
                    float acc[RPW_DN];
                    tile_dot_pc<F, RPW_DN>(td, pcB, sE, acc);
#pragma unroll
                    for (int r = 0; r < RPW_DN; r++)
                        if (lane == r)
                            st_tag(blk + R::OX + rw_dn + r, __fadd_rn(s_xa[xpos<EP, H>(rw_dn + r)], __fmul_rn(acc[r], td.rs[r])), tag);
                }
            } else {
                PS_MARK(ph, 2);
                float acc[RPW_DN];
                tile_dot<PREC, F, RPW_DN>(td, s_in, acc);
#pragma unroll
                for (int r = 0; r < RPW_DN; r++)
                    if (lane == r) {
                        const float v = PREC == QT_INT8 ? __fmul_rn(acc[r], td.rs[r]) : acc[r];
                        st_tag(blk + R::OX + rw_dn + r, __fadd_rn(s_xa[xpos<EP, H>(rw_dn + r)], v), tag);
                    }
            }
            PS_MARK(ph, 3);
            // the next layer's K/V copy lands in the buffer this phase's input and pieces
            // occupy: every wave must be done reading them
            __syncthreads();
            if (l + 1 < L) prefetch_kv(l + 1);
            PS_MARK(ph, 1); ph++;
        }

        const unsigned long long *xfin = ring.blk(par, L - 1) + R::OX;
        const bool last_step = (step + 1 == a.n_steps);
        if (!a.with_head) {
            // final norm of the residual -> hid, residual -> decx (workgroup 0)
            if (b == 0) {
                load_gains<NW, EH, H>(a.final_norm, s_gain[1]);
                gather<H / NT, NT>(H, [&](int i) { return xfin + i; }, s_x, tag, a.err, PosChunk<EH, H>());
                stage_norm<QT_BF16, H>(s_x, s_gain[1], a.eps, s_xn);
                for (int i = tid; i < H; i += NT) { a.hid[i] = s_xn[xpos<EH, H>(i)]; a.decx[i] = s_x[xpos<EH, H>(i)]; }
            }
        } else {
            // ---------------- head: logits rows + masked local argmax -----------------
            // (its tile is loaded here rather than during the last layer: a tile carried
            // through the layer loop would hold its registers for the whole loop)
            THEAD th;
            th.load(a.head_w, nullptr, rw_head);
            load_gains<NW, EH, H>(a.final_norm, s_gain[1]);
            gather<H / NT, NT>(H, [&](int i) { return xfin + i; }, s_x, tag, a.err, PosChunk<EH, H>());
            PS_MARK(ph, 0);
            stage_norm<QT_BF16, H>(s_x, s_gain[1], a.eps, s_xn);
            if (last_step && b == 0)
                for (int i = tid; i < H; i += NT) { a.hid[i] = s_xn[xpos<EH, H>(i)]; a.decx[i] = s_x[xpos<EH, H>(i)]; }
            float acc[RPW_HEAD];
            tile_dot<QT_BF16, H, RPW_HEAD>(th, s_xn, acc);
            const int frame = frame0 + step;
            if (lane == 0) {
                float bv = -INFINITY; int bi = 0x7FFFFFFF;
#pragma unroll
                for (int r = 0; r < RPW_HEAD; r++) {
                    if (!head_on || wave * RPW_HEAD + r >= HEADR) break;
                    const int i = rw_head + r;
                    float v = fminf(fmaxf(acc[r], -100.0f), 100.0f);
                    if (i >= 2048 && i != 2150) v = -1e30f;
                    if (i == 2150 && frame < 2) v = -1e30f;
                    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
                }
                wbest_v[wave] = bv; wbest_i[wave] = bi;
            }
            __syncthreads();
            unsigned long long *slots = ring.slots(par);
            if (tid == 0) {
                float bv = wbest_v[0]; int bi = wbest_i[0];
                for (int w = 1; w < NW; w++)
                    if (wbest_v[w] > bv || (wbest_v[w] == bv && wbest_i[w] < bi)) { bv = wbest_v[w]; bi = wbest_i[w]; }
                st_tag(slots + 2 * b, bv, tag);
                st_tag(slots + 2 * b + 1, __int_as_float(bi), tag);
            }
            if (!last_step) {
                tq.load(s_layers[0].w[0], lsc<PREC>(s_layers[0], 0), rw_qkv);
                load_gains<NW, EP, H>(s_layers[0].in_norm, s_gain[0]);
            }
            PS_MARK(ph, 1); ph++;
            // global argmax over the 256 local winners (every workgroup, redundantly)
            gather<2, NT>(2 * NB, [&](int i) { return slots + i; }, s_in, tag, a.err);
            {
                float bv = -INFINITY; int bi = 0x7FFFFFFF;
                for (int i = tid; i < NB; i += NT) {
                    const float v = s_in[2 * i];
                    const int ix = __float_as_int(s_in[2 * i + 1]);
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
                if (gi < 0 || gi >= a.vocab) gi = 0;
                tok = gi;
                if (b == 0 && tid == 0) a.hist[frame % a.hist_len] = gi;
                __syncthreads();   // wbest_* and s_in are reused in the next step
            }
        }
    }
    // epilogue (workgroup 0): position/frame/tag advance and the next launch's input
    if (b == 0) {
        if (a.with_head)
            for (int i = tid; i < H; i += NT) a.xin[i] = bf16f(ldg(a.emb + (size_t)tok * H + i));
        if (tid == 0) {
            *a.d_pos = pos0 + a.n_steps;
            if (a.with_head) *a.d_frame = frame0 + a.n_steps;
            *a.epoch = tag0 + (unsigned)a.n_steps;
        }
    }
    PS_TRACE_FLUSH();
}
}  // namespace ps

#ifdef QT_PSTEP_TRACE
extern "C" hipError_t qt_pstep_trace_read(unsigned long long *out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(ps::ps_trace), sizeof(ps::ps_trace), 0, hipMemcpyDeviceToHost);
}
#endif

// 4 waves per workgroup (one per SIMD).  The kernel also builds with 8 (two per SIMD, so
// one wave's latency could hide behind the other's work), but at 256 registers per wave
// its tiles spill and the step is slower.
template <int PREC, int H, int F>
static hipError_t ps_launch(const ps::Args &a, hipStream_t st) {
    constexpr int NW = 4;
    void *args[] = {(void *)&a};
    return hipLaunchCooperativeKernel((const void *)ps::k_pstep<PREC, H, F, NW>, dim3(ps::NB), dim3(NW * 64), args, 0, st);
}

extern "C" int qt_pstep_supported(int prec, int hidden, int inter, int n_heads, int n_kv, int head_dim, int kv_max) {
    if (n_heads != ps::NH || n_kv != ps::NKV || head_dim != ps::HD) return 0;
    if (kv_max > ps::G * ps::CHMAX) return 0;
    if (prec != QT_BF16 && prec != QT_INT8 && prec != QT_Q4) return 0;
    if (!((hidden == 1024 && inter == 3072) || (hidden == 2048 && inter == 6144))) return 0;
    if (prec == QT_Q4 && hidden != 2048) return 0;   // a q4 chunk is 32 columns: 64 lanes need 2048
    int dev = 0, cus = 0, coop = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess) return 0;
    if (!coop || cus < ps::NB) return 0;
    return 1;
}

// tagged ring words for n_layers layers (2 parities) plus the head's winner slots
extern "C" size_t qt_pstep_ring_words(int hidden, int inter, int n_layers) {
    const size_t P = (size_t)ps::QKVR + (size_t)ps::NKV * ps::G * ps::HPK * ps::PS + ps::QD + 2 * (size_t)hidden + inter;
    return 2 * (size_t)n_layers * P + 2 * (size_t)ps::NB * 2;
}
extern "C" size_t qt_pstep_layer_bytes(void) { return sizeof(ps::Layer); }
// word offset of layer l's output x (phase E) in the ring block of parity par
extern "C" size_t qt_pstep_ring_x_offset(int hidden, int inter, int n_layers, int par, int l) {
    const size_t OX = (size_t)ps::QKVR + (size_t)ps::NKV * ps::G * ps::HPK * ps::PS + ps::QD + (size_t)hidden + inter;
    const size_t P = OX + hidden;
    return ((size_t)par * n_layers + l) * P + OX;
}

// Layer table entry, filled on the host in this exact order.
extern "C" void qt_pstep_fill_layer(void *dst, const uint8_t *const w[4], const float *const s[4], const uint16_t *const s16[4],
                                    const float *in_norm, const float *post_norm, const float *qn, const float *kn) {
    ps::Layer *L = (ps::Layer *)dst;
    for (int i = 0; i < 4; i++) { L->w[i] = w[i]; L->s[i] = s[i]; L->s16[i] = s16[i]; }
    L->in_norm = in_norm; L->post_norm = post_norm; L->qn = qn; L->kn = kn;
}

extern "C" hipError_t qt_launch_pstep(int prec, int hidden, const void *layers_dev, int n_layers,
                                      const float *final_norm, const float *rope_cos, const float *rope_sin,
                                      uint16_t *kc, uint16_t *vc, int kv_max, float eps, float scale,
                                      unsigned long long *ring, float *hid, float *decx, float *xin, int *d_pos,
                                      unsigned *epoch, int *err, int n_steps, int with_head, const uint16_t *head_w,
                                      const uint16_t *emb, int vocab, int *d_frame, int *hist, int hist_len,
                                      hipStream_t st) {
    ps::Args a;
    a.layers = (const ps::Layer *)layers_dev; a.n_layers = n_layers;
    a.final_norm = final_norm; a.rope_cos = rope_cos; a.rope_sin = rope_sin;
    a.kc = kc; a.vc = vc; a.kv_max = kv_max; a.eps = eps; a.scale = scale;
    a.ring = ring; a.hid = hid; a.decx = decx; a.xin = xin; a.d_pos = d_pos; a.epoch = epoch;
    a.err = err; a.n_steps = n_steps; a.with_head = with_head;
    a.head_w = (const uint8_t *)head_w; a.emb = emb; a.vocab = vocab;
    a.d_frame = d_frame; a.hist = hist; a.hist_len = hist_len;
    if (n_steps <= 0 || n_layers <= 0 || n_layers > ps::MAXL || kv_max > ps::G * ps::CHMAX) return hipErrorInvalidValue;
    if (!with_head && n_steps != 1) return hipErrorInvalidValue;   // without the head the next input is unknown
    if (with_head && (vocab != ps::NB * 12 || !head_w || !emb || !d_frame || !hist || hist_len <= 0))
        return hipErrorInvalidValue;
    if (prec == QT_INT8 && hidden == 2048) return ps_launch<QT_INT8, 2048, 6144>(a, st);
    if (prec == QT_INT8 && hidden == 1024) return ps_launch<QT_INT8, 1024, 3072>(a, st);
    if (prec == QT_BF16 && hidden == 2048) return ps_launch<QT_BF16, 2048, 6144>(a, st);
    if (prec == QT_BF16 && hidden == 1024) return ps_launch<QT_BF16, 1024, 3072>(a, st);
    if (prec == QT_Q4 && hidden == 2048) return ps_launch<QT_Q4, 2048, 6144>(a, st);
    return hipErrorInvalidValue;
}
