/*
 * qwen_tts_hip.h — C ABI of the MI355X (gfx950) decode-step library, libqwen_tts_hip.so.
 *
 * Drop-in for the reference engine's GPU seams (paths relative to the reference root):
 *   level 1  per-op backend vtable  (qwen_tts_backend.h:34-49, qwen_tts_cuda.h:23-35)
 *            and the qwen_tts_kernels.h kernel signatures used as the parity surface;
 *   level 2  resident fused steps   (qwen_tts_cuda.h:62-67, qwen_tts_cuda_talker.cu:313-947,
 *            qwen_tts_metal.m:2246-2277 for the device-side CP frame).
 * The reference's level-2 init functions take a qwen_tts_ctx_t*; this ABI takes plain
 * pointers instead (qwen_hip_talker_desc_t), filled from the ctx by a short glue file
 * on the reference side (qwen3-tts_amd/glue/qwen_tts_hip_glue.c).  Weight pointers may be host or
 * device memory; init copies them to the device and never aliases them.
 *
 * Error convention (mirrors the reference: init NULL -> caller stays on CPU):
 *   init functions return NULL on any failure and print one line to stderr;
 *   a state that hits a HIP error later is marked dead: its step functions return
 *   nonzero, qwen_hip_last_error() describes the failure.
 * Threading: one state = one HIP stream; a state must not be used from two threads
 * at once.  All level-2 calls are synchronous unless named *_async.
 */
#ifndef QWEN_TTS_HIP_H
#define QWEN_TTS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { QWEN_HIP_BF16 = 0, QWEN_HIP_INT8 = 1, QWEN_HIP_Q4_0 = 2 };

/* One weight matrix [rows][cols] in the reference's host layout:
 *   BF16  uint16 bf16 bits, row-major (qwen_tts.h:125-137);
 *   INT8  int8 row-major + f32 scale[rows] (qwen_tts.h:143-155, quantizer k.c:2143);
 *   Q4_0  q4_0_block_t[rows][cols/32] (18 B: u16 f16 scale, u8 qs[16]) (k.h:206-210). */
typedef struct {
    const void *w;
    const float *scale;      /* INT8 only, else NULL */
} qwen_hip_mat_t;

/* One transformer layer: the fields of qwen_talker_layer_t / qwen_cp_layer_t the
 * decode step reads (qwen_tts.h:125-229).  gate_up is the reference's row-interleaved
 * fused matrix [2*inter][hidden] (qwen_tts_talker.c:378-388). */
typedef struct {
    qwen_hip_mat_t q, k, v, o, gate_up, down;
    const float *input_norm, *post_attn_norm;   /* [hidden] */
    const float *q_norm, *k_norm;               /* [head_dim] */
} qwen_hip_layer_t;

/* Everything qwen_cuda_talker_init reads from the ctx (qwen_tts_cuda_talker.cu:313-360). */
typedef struct {
    int hidden, inter, n_heads, n_kv_heads, head_dim, n_layers;
    int kv_max;                 /* device KV capacity (positions) */
    float eps;                  /* rms_norm_eps */
    int prec;                   /* QWEN_HIP_* of the pointers in layers[] */
    int quantize_to;            /* -1: keep; QWEN_HIP_INT8/Q4_0: quantize BF16 weights on device */
    const qwen_hip_layer_t *layers;
    const float *final_norm;    /* talker_norm [hidden]; CP: cp_norm */
    const float *rope_cos, *rope_sin;  /* [rope_len][head_dim/2] (qwen_tts_talker.c:478-495) */
    int rope_len;
} qwen_hip_talker_desc_t;

/* ---- level 2: resident Talker step (qwen_tts_cuda_talker.cu:313-438, 933-947) ---- */

/* replaces qwen_cuda_talker_init(ctx)            (qwen_tts_cuda_talker.cu:313) */
void *qwen_hip_talker_init(const qwen_hip_talker_desc_t *desc);
/* The Talker's layers straight from the model file to the device; no counterpart in the
 * reference, which maps model.safetensors on the host (ingot, qwen_tts_talker.c:105-122)
 * and builds gate|up and the quantized twins there (t.c:286-317, 378-388).  model_path: the
 * safetensors file, or the directory holding model.safetensors.  shape: dimensions,
 * kv_max, eps, quantize_to (-1 keeps bf16; QWEN_HIP_INT8 / QWEN_HIP_Q4_0 quantize on the
 * device, bit-identical to the reference's host quantizers) and the RoPE tables; its prec,
 * layers and final_norm are ignored (read from the file).  Every tensor is checked (name,
 * dtype BF16 -- norms BF16 or F32 --, shape, extent) before the GPU is touched.  Returns
 * the state qwen_hip_talker_init returns, or NULL (qwen_hip_last_error() says why). */
void *qwen_hip_talker_load_file(const char *model_path, const qwen_hip_talker_desc_t *shape);
/* replaces qwen_cuda_talker_step                 (qwen_tts_cuda_talker.cu:395):
 * embed host f32[hidden] in, hidden_out host f32[hidden] (final-normed) out; appends
 * KV at pos.  Returns 0 on success. */
int   qwen_hip_talker_step(void *state, const float *embed, float *hidden_out, int pos);
/* replaces qwen_cuda_talker_get_dec_x            (qwen_tts_cuda_talker.cu:419) */
void  qwen_hip_talker_get_dec_x(void *state, float *out);
/* replaces qwen_cuda_talker_upload_kv(state, ctx, prefill_len) (qwen_tts_cuda_talker.cu:424):
 * kv_k/kv_v are the host bf16 caches [n_layers][host_kv_max][kv_dim] (qwen_tts.h:513-518),
 * ordinary pageable memory.  The call copies them through two pinned buffers that the
 * state made at init: four short-lived host threads fill one buffer while the DMA engine
 * drains the other.  The caches may be reused as soon as the call returns. */
int   qwen_hip_talker_upload_kv(void *state, const uint16_t *kv_k, const uint16_t *kv_v,
                                int host_kv_max, int prefill_len);
/* replaces qwen_cuda_talker_free                 (qwen_tts_cuda_talker.cu:933) */
void  qwen_hip_talker_free(void *state);

/* Talker prefill on the device: the twin of qwen_talker_prefill(ctx, input_embeds,
 * seq_len) (qwen_tts_talker.c:730-1038), which the reference runs on the CPU before
 * qwen_cuda_talker_upload_kv (qwen_tts.c:1454-1476); no GPU counterpart in the reference.
 * input_embeds host f32[seq][hidden].  Writes KV rows [0, seq) of every layer of the
 * state's device cache and dec_x (qwen_hip_talker_get_dec_x) = the last position's
 * residual; the next step runs at pos = seq.  Projections use bf16 weights as the
 * reference's prefill does (t.c:832-839): the state's own when it holds bf16, else
 * bf16_layers (the descriptor's bf16 layer weights, copied to the device on the first
 * call and kept; NULL is allowed after that or for a bf16 state).  Needs hidden, inter
 * and the q|k|v row count divisible by 64.  Returns 0 on success; argument errors
 * leave the state usable. */
int   qwen_hip_talker_prefill(void *state, const qwen_hip_layer_t *bf16_layers, const float *input_embeds, int seq);
/* Benchmark entry (no reference counterpart): enqueue n more prefills of the last
 * prefill's inputs (seq <= the last call's seq) on the state's stream, no host sync. */
int   qwen_hip_talker_prefill_async(void *state, int seq, int n);

/* Reads back the device KV of positions [0, n) in the host layout (checks/tests). */
int   qwen_hip_talker_download_kv(void *state, uint16_t *kv_k, uint16_t *kv_v, int host_kv_max, int n);

/* Device-resident greedy decode (no counterpart in the reference's C engine; it fuses
 * the per-frame glue of qwen_tts.c:1649-1694 + 919-924 with the step): runs n_steps
 * Talker steps starting at pos with input embed (host f32[hidden]); after each step
 * the codec head + greedy rule picks code0 and the next input is
 * codec_embedding[code0].  tokens_out[n_steps], hidden_out (nullable) the last
 * hidden.  frame0 is the frame index of the first step (EOS masked for frames < 2). */
int   qwen_hip_talker_greedy(void *state, const uint16_t *codec_head, const uint16_t *codec_emb,
                             int codec_vocab, const float *embed, int pos, int frame0,
                             int n_steps, int *tokens_out, float *hidden_out);

/* Timing entry for benchmarks: enqueue n_steps steps of the resident greedy loop on the
 * state's stream without host synchronisation (inputs already resident on the device).
 * Call qwen_hip_talker_greedy once first (it uploads the heads and seeds the loop). */
int   qwen_hip_talker_greedy_async(void *state, int n_steps);
int   qwen_hip_talker_sync(void *state);
/* The state's stream (hipStream_t), for callers that time it with events. */
void *qwen_hip_talker_stream(void *state);
/* Diagnostic query (no reference counterpart): 1 when steps run as the single fused
 * persistent kernel, 0 when they run as the per-kernel sequence (shapes or devices the
 * fused kernel does not cover), -1 for a NULL state. */
int   qwen_hip_talker_fused(void *state);
/* replaces kv_cache_grow(ctx, required) (qwen_tts_talker.c:257-280): the device KV cache's
 * capacity doubles until it holds `required` positions (at most 8192, and within the rope
 * table given at init); the rows are copied on the device and the decode keeps its fused
 * kernel.  0 when the capacity already suffices or after growing, -1 with
 * qwen_hip_last_error() set otherwise.  The step, prefill, upload and loop entry points
 * grow the cache themselves when their positions need it (as qwen_talker_step does before
 * its step, qwen_tts_talker.c:574, and qwen_talker_prefill, :773), so a caller only needs
 * this to grow ahead of time. */
int   qwen_hip_talker_grow_kv(void *state, int required);
/* the device KV cache's current capacity in positions (-1 for a NULL state) */
int   qwen_hip_talker_kv_max(void *state);
/* Diagnostic query (no reference counterpart): which fused kernel runs the steps —
 * 2 the role-specialised persistent kernel (qt_rstep.hip), 1 the single-role persistent
 * kernel (qt_pstep.hip), 0 the per-kernel sequence, -1 for a NULL state. */
int   qwen_hip_talker_fused_kernel(void *state);
/* Diagnostic (no reference counterpart; the device twin of the per-layer check the
 * reference's own tests make by truncating num_layers, qwen_tts_talker.c:659-665): one step
 * like qwen_hip_talker_step that also returns the residual after every layer,
 * residuals host f32[n_layers][hidden].  The fused kernel's values are read back from its
 * activation ring (tags checked); the per-kernel path copies x after each layer. */
int   qwen_hip_talker_step_layers(void *state, const float *embed, float *residuals, float *hidden_out, int pos);
/* Same as qwen_hip_talker_step, but the device graph runs with graph capture disabled
 * (one launch per kernel), for profiling and A/B checks. */
int   qwen_hip_talker_step_nograph(void *state, const float *embed, float *hidden_out, int pos);

/* Benchmark/profiling aid (no reference counterpart): enqueue n launches of one kernel
 * of the step on the state's stream, no sync.  kernel: 0 norm+QKV, 1 attention at the
 * current device position, 2 O projection, 3 norm+gate_up+SwiGLU, 4 down projection,
 * 5 final norm.  Kernels 2 and 4 write scratch instead of the residual stream, so
 * repeated launches leave the decode state unchanged (kernel 1 rewrites the KV slot at
 * the current position with the same bits). */
int   qwen_hip_talker_launch_kernel(void *state, int kernel, int layer, int n);

/* ---- level 2: batched Talker step (qwen_tts_cuda_talker.cu:595-648; CPU twin
 * batch_talker_step_impl, qwen_tts_talker.c:1192-1270, qwen_tts_batch.h:87-98) ----
 * B <= 64 streams share the single state's device weights (read once per step for all
 * streams: every precision runs each projection as one GEMM over the B streams on the
 * matrix cores -- int8 and q4_0 on the integer MFMA with exact int8 activation pieces,
 * bf16 on the bf16 MFMA with exact bf16 activation planes); each stream has its
 * own bf16 KV cache (single state's kv_max) and its own position (ragged).  Free the
 * batch before the single state. */

/* replaces qwen_cuda_talker_batch_init(single, B)      (qwen_tts_cuda_talker.cu:595) */
void *qwen_hip_talker_batch_init(void *single, int B);
/* replaces qwen_cuda_talker_batch_step                  (qwen_tts_cuda_talker.cu:618):
 * embeds host f32[B][hidden], pos_arr host int[B] (each stream's position: its KV row
 * written, RoPE and causal length pos+1), hidden_out host f32[B][hidden] final-normed. */
int   qwen_hip_talker_batch_step(void *state, const float *embeds, const int *pos_arr, float *hidden_out);
/* Diagnostic (no reference counterpart; the batched twin of qwen_hip_talker_step_layers):
 * one batched step run without graph capture that also returns every stream's residual after
 * every layer, residuals host f32[n_layers][B][hidden].  Allocates a temporary device buffer. */
int   qwen_hip_talker_batch_step_layers(void *state, const float *embeds, const int *pos_arr, float *residuals,
                                        float *hidden_out);
/* replaces qwen_cuda_talker_batch_upload_slot           (qwen_tts_cuda_talker.cu:629):
 * seeds slot b's device KV from the batch engine's host bf16 caches laid out
 * ((b*n_layers + l)*src_kv_max + pos)*kv_dim (qwen_tts_batch.h:26-27). */
int   qwen_hip_talker_batch_upload_slot(void *state, int b, const uint16_t *kv_k, const uint16_t *kv_v,
                                        int src_kv_max, int prefill_len);
/* replaces qwen_cuda_talker_batch_free                  (qwen_tts_cuda_talker.cu:643);
 * the shared weights stay with the single state. */
void  qwen_hip_talker_batch_free(void *state);
/* Reads slot b's positions [0, n) back in the upload layout (checks/tests; no
 * reference counterpart). */
int   qwen_hip_talker_batch_download_slot(void *state, int b, uint16_t *kv_k, uint16_t *kv_v, int dst_kv_max, int n);
/* Benchmark entries (no reference counterpart): replay n steps of the last batch_step's
 * inputs on the device without host sync; the state's stream. */
int   qwen_hip_talker_batch_step_async(void *state, int n_steps);
int   qwen_hip_talker_batch_sync(void *state);
void *qwen_hip_talker_batch_stream(void *state);
/* Test/measurement switch (no reference counterpart): int8 projections make their
 * activation pieces inside the projection launch (on = 1, the default wherever every
 * projection shape allows it) or in a launch of their own (0); both give the same bytes.
 * Applies to Talker and CP batch states.  Returns the mode in effect, -1 on error. */
int   qwen_hip_batch_fold_pieces(void *state, int on);

/* ---- level 2: Code Predictor (qwen_tts_cuda_talker.cu:751-841; qwen_tts_metal.m:2246) ---- */

typedef struct {
    qwen_hip_talker_desc_t cp;      /* CP layers; final_norm = cp_norm; rope = cp tables */
    int codebook;                   /* 2048 */
    int lm_prec;                    /* precision of lm_head[] (QWEN_HIP_*) */
    qwen_hip_mat_t lm_head[15];     /* [codebook][cp_hidden] */
    const uint16_t *cp_codec_emb[15];  /* bf16 [codebook][emb_dim] */
    const uint16_t *talker_codec_emb;  /* bf16 [codec_vocab][talker_hidden] */
    int codec_vocab, talker_hidden, emb_dim;
    int mtp_prec;                   /* small_to_mtp_projection precision (BF16/INT8) */
    qwen_hip_mat_t mtp;             /* [cp_hidden][emb_dim] or w=NULL (identity) */
    const float *mtp_bias;          /* f32 [cp_hidden] or NULL */
} qwen_hip_cp_desc_t;

/* replaces qwen_cuda_cp_init(ctx)                (qwen_tts_cuda_talker.cu:751) */
void *qwen_hip_cp_init(const qwen_hip_cp_desc_t *desc);
/* replaces qwen_cuda_cp_step(state, x, pos)      (qwen_tts_cuda_talker.cu:796):
 * x host f32[cp_hidden] residual in/out (not normed); one 5-layer pass at pos. */
int   qwen_hip_cp_step(void *state, float *x, int pos);
/* twin of qwen_metal_cp_frame (qwen_tts_metal.m:2246-2277), the device-side version of
 * qwen_cp_predict (qwen_tts_code_predictor.c:926-1045): 16 passes + 15 greedy lm-head
 * picks + embedding gathers, one host sync.  out_codes[15]. */
int   qwen_hip_cp_frame(void *state, const float *talker_hidden, int code0, int *out_codes);
/* benchmark entry: n frames back to back on device inputs already uploaded by a
 * previous qwen_hip_cp_frame call, no host sync. */
int   qwen_hip_cp_frame_async(void *state, int n_frames);
int   qwen_hip_cp_sync(void *state);
void *qwen_hip_cp_stream(void *state);
/* Test/measurement switch (no reference counterpart): frames as one launch of the
 * role-specialised kernel (on = 1, the default where the CP qualifies: 0.6B geometry, one
 * weight type, int8 or bf16, in every layer, lm head and the 2048 -> 1024 mtp projection,
 * two-position prefill off) or as the per-kernel launch graph (0); int8 weights give the
 * same bits both ways, bf16 weights the same codes with K/V within f32 rounding.  Returns
 * the mode in effect, -1 on error. */
int   qwen_hip_cp_fused(void *state, int on);
/* replaces qwen_cuda_cp_free                     (qwen_tts_cuda_talker.cu:917) */
void  qwen_hip_cp_free(void *state);
/* Diagnostic (no reference counterpart; what the reference keeps in ctx->cp_kv_k/cp_kv_v
 * after qwen_cp_predict, qwen_tts_code_predictor.c:926-1045): positions [0, n) of the CP's
 * device KV cache into host bf16 [cp_layers][host_kv_max][kv_heads*head_dim]. */
int   qwen_hip_cp_download_kv(void *state, uint16_t *kv_k, uint16_t *kv_v, int host_kv_max, int n);
/* two-position prefill, twin of cp_prefill2 (qwen_tts_code_predictor.c:816-902) and of
 * its switch cp_prefill2_mode / QWEN_CP_PREFILL2 (:783-807).  set_prefill2(state, 1)
 * needs int8 weights in every CP layer (the reference: quantized CP only) and makes
 * qwen_hip_cp_frame run positions 0 and 1 as one two-column pass (weights read once);
 * 0 restores the sequential passes (the default).  qwen_hip_cp_prefill2 runs that pass
 * alone: x0, x1 host f32[cp_hidden] residuals in/out at positions 0 and 1. */
int   qwen_hip_cp_set_prefill2(void *state, int on);
int   qwen_hip_cp_prefill2(void *state, float *x0, float *x1);
/* CP batch twins (qwen_tts_cuda_talker.cu:879-915): B streams over the single CP state's
 * weights; x host f32[B][cp_hidden] residuals in/out (not normed), one pass per stream
 * at pos_arr[b] on its own CP KV. */
void *qwen_hip_cp_batch_init(void *single, int B);
int   qwen_hip_cp_batch_step(void *state, float *x, const int *pos_arr);
void  qwen_hip_cp_batch_free(void *state);

/* ---- level 1: per-op backend (qwen_tts_cuda.h:23-35, qwen_tts_backend.h:34-49) ---- */

int   qwen_hip_available(void);
void *qwen_hip_init(void);
void  qwen_hip_free(void *ctx);
/* y[rows] = W[rows,cols] @ x[cols] (W bf16; host pointers; W cached on device by
 * host address like qwen_tts_cuda.c:96-112) */
void  qwen_hip_matvec_bf16(void *ctx, float *y, const uint16_t *W, const float *x, int rows, int cols);
/* Y[rows,B] = W[rows,cols] @ X[cols,B] (row-major f32, B<=64); W read once for all B columns
 * (exact bf16 planes of X on the bf16 MFMA) when rows and cols are multiples of 64 */
void  qwen_hip_matmat_bf16(void *ctx, float *Y, const uint16_t *W, const float *X, int rows, int cols, int B);

/* qwen_tts_kernels.h signatures on the HIP kernels (host pointers in and out; every
 * call uploads, computes, downloads).  Return 0 on success. */
int qwen_hip_op_matvec_int8(float *y, const int8_t *W, const float *scale, const float *x, int rows, int cols);
int qwen_hip_op_matvec_q4_0(float *y, const void *W, const float *x, int rows, int cols);
int qwen_hip_op_matvec_bf16(float *y, const uint16_t *W, const float *x, int rows, int cols);
int qwen_hip_op_causal_attention_bf16kv(float *out, const float *Q, const uint16_t *K, const uint16_t *V,
                                        int seq_q, int seq_k, int n_heads, int n_kv_heads, int head_dim,
                                        float scale, int q_offset);
int qwen_hip_op_rms_norm(float *out, const float *x, const float *w, int seq, int dim, float eps);
int qwen_hip_op_rms_norm_per_head(float *x, const float *w, int seq, int n_heads, int head_dim, float eps);
int qwen_hip_op_swiglu(float *out, const float *gate_up, int n);
/* The prefill projection alone (no reference counterpart as one call: the sgemm /
 * qwen_matmat_bf16 of t.c:845-847, 913, 964, 990): Y[S][N] = X[S][K] . W[N][K]^T
 * (epi 0), Y += that (epi 1), or SwiGLU of the interleaved gate|up rows into Y[S][N/2]
 * (epi 2); W bf16, f32 host arrays, N and K multiples of 64. */
int qwen_hip_op_prefill_gemm(float *Y, const uint16_t *W, const float *X, int S, int N, int K, int epi);
/* The prefill's causal attention alone (qwen_causal_attention, k.c:3454-3560, as
 * t.c:904-907 calls it): out f32[S][nh*128] from QKV f32[S][(nh + 2 nkv)*128] holding the
 * normed, rotated q | k | v rows of every position. */
int qwen_hip_op_prefill_attention(float *out, const float *QKV, int S, int nh, int nkv, float scale);
int qwen_hip_op_argmax_matvec(int prec, const float *x, const void *W, const float *scale, int in_dim, int out_dim);
/* Sampling settings of the Talker's frame loop: the fields of qwen_tts_ctx_t that the loop
 * of qwen_tts.c:1649-1721 reads (defaults at qwen_tts.c:559: temperature 0.9, top_k 50,
 * top_p 1.0, rep_penalty 1.05, greedy_warmup 0). */
typedef struct {
    float temperature;      /* ctx->temperature; < 1e-6 = greedy */
    int top_k;              /* ctx->top_k (0 = off) */
    float top_p;            /* ctx->top_p (1.0 = off) */
    float rep_penalty;      /* ctx->rep_penalty (1.0 = off) */
    int greedy_warmup;      /* ctx->greedy_warmup: frames below it draw greedily (temp 0, top_k 1) */
    int text_len;           /* text_content_len: EOS boost 0.5 per frame past 2 x 3 x text_len, capped
                             * at 10 (qwen_tts.c:1666-1675); 0 = no boost */
} qwen_hip_sample_params_t;

/* The Talker's frame loop with sampling on the device (qwen_tts.c:1649-1721 for code0):
 * n_steps x (Talker step at pos + i, final norm + codec head, codec-head rule for frame
 * frame0 + i incl. the EOS boost, qwen_tts_sample with the repetition penalty over
 * prev_tokens and the tokens drawn so far, next input codec_emb[token]).  Same head and
 * embedding arguments as qwen_hip_talker_greedy; *seed is the LCG state in and out
 * (qwen_set_seed / qwen_get_seed, sampling.c:38-49); tokens_out[n_steps]; the last step's
 * normed hidden state in hidden_out (may be NULL).  Like the reference's loop, generation
 * ends at the first EOS (2150): that token is the last one returned, the LCG state and the
 * history stop there, and the remaining steps' results are discarded.  Returns the number
 * of tokens generated (<= n_steps, the last one EOS when EOS was drawn) or -1.
 * n_prev + n_steps < 16384.  Allocates nothing per call.  Afterwards the greedy loop must
 * be re-seeded with qwen_hip_talker_greedy before qwen_hip_talker_greedy_async. */
int qwen_hip_talker_sample(void *state, const uint16_t *codec_head, const uint16_t *codec_emb, int codec_vocab,
                           const float *embed, int pos, int frame0, int n_steps, const qwen_hip_sample_params_t *params,
                           const int *prev_tokens, int n_prev, uint32_t *seed, int *tokens_out, float *hidden_out);
/* The whole frame loop of qwen_tts_generate (qwen_tts.c:1649-1778, non-streaming) on the
 * device, no counterpart as one call in the reference: per frame, codec head over the last
 * normed hidden state -> codec-head rule + qwen_tts_sample (params; the code0 history
 * prev_tokens + the tokens drawn here; *seed the LCG state in and out) -> the CP frame of
 * cp_state for that hidden state and code0 (qwen_cp_predict, cp.c:926-1045) -> next input
 * codec_emb[code0] + sum_g cp_codec_emb[g][code_g] + tts_pad (host f32[hidden], the text
 * side's pad embedding) -> one Talker step at pos + f.  hidden0: the normed hidden state
 * the loop starts from (host f32[hidden]: the prefill's last position, or the previous
 * call's hidden_out).  codes_out[n_frames][16] = code0 then the 15 CP codes.  As in the
 * reference the frame whose code0 is EOS ends the utterance (codes_out[n][0] == 2150 marks
 * it when n < n_frames).  Returns the number of frames generated, or -1.  One host sync per
 * call; allocates nothing; the CP state must not be used elsewhere meanwhile. */
int qwen_hip_generate(void *talker_state, void *cp_state, const uint16_t *codec_head, const uint16_t *codec_emb,
                      int codec_vocab, const float *tts_pad, const float *hidden0, int pos, int frame0, int n_frames,
                      const qwen_hip_sample_params_t *params, const int *prev_tokens, int n_prev, uint32_t *seed,
                      int *codes_out, float *hidden_out);
/* Token sampling on the device: qwen_tts_sample (qwen_tts_sampling.c:160-202; repetition
 * penalty, temperature softmax, top-k, top-p, renormalisation, LCG draw) with the
 * thread-local LCG state of qwen_set_seed / qwen_get_seed (sampling.c:38-49) passed as
 * *seed and advanced as the reference advances it (once per non-greedy draw).  vocab <= 4096.
 * Returns the token, or -1 on error (see qwen_hip_last_error). */
int qwen_hip_op_sample(const float *logits, int vocab, float temp, int top_k, float top_p, float rep_penalty,
                       const int *prev_tokens, int n_prev, uint32_t *seed);
/* The codec-head rule of the Talker's frame loop (qwen_tts.c:1652-1679: clip to +-100,
 * tokens >= 2048 except EOS 2150 masked, EOS masked for frames < 2, eos_boost added to
 * the EOS logit) followed by qwen_hip_op_sample (qwen_tts.c:1689-1691). */
int qwen_hip_op_codec_sample(const float *logits, int vocab, int frame, float eos_boost, float temp, int top_k,
                             float top_p, float rep_penalty, const int *prev_tokens, int n_prev, uint32_t *seed);
/* qwen_matmat_int8 (qwen_tts_kernels.h:121-122): Y[rows][B] = (W*scale) @ X[cols][B]
 * (row-major f32, B <= 64, cols a multiple of 64) on the batched MFMA kernel. */
int qwen_hip_op_matmat_int8(float *Y, const int8_t *W, const float *scale, const float *X, int rows, int cols, int B);
/* qwen_matmat_q4_0 (qwen_tts_kernels.h:226-227): Y[rows][B] = dequant(W) @ X[cols][B] with W
 * in the reference's 18-byte q4_0 blocks (row-major f32 X/Y, B <= 64, cols a multiple of 64,
 * <= 8192): the weights are read once for all B columns, each 32-block's dot product is an
 * exact integer sum of the nibbles against exact int8 pieces of X, scaled by the block's f16
 * scale in f32. */
int qwen_hip_op_matmat_q4_0(float *Y, const void *W, const float *X, int rows, int cols, int B);
/* No counterpart in the reference: qwen_hip_op_matmat_int8 for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that forbid
 * hipMalloc).  All pointers are the caller's DEVICE buffers: Y[B][rows] and X[B][cols]
 * stream-major f32 (row b is stream b), W int8 [rows][cols] + scale f32[rows] in the
 * reference's encoding; launched on `stream` (a hipStream_t; NULL = the null stream),
 * asynchronous.  The activation pieces live in a file-scope device array of
 * 8192*3*64 + 256 bytes per GPU (held until the process ends), so cols <= 8192 (a multiple
 * of 64) and 1 <= B <= 64; larger shapes return -1 with qwen_hip_last_error() set.
 * The array used is the one of the device `stream` belongs to (the current device for the
 * null stream).  Allocates nothing.  Calls that overlap on one GPU share that array and
 * race: callers must serialise them on one stream per GPU. */
int qwen_hip_op_matmat_int8_noalloc(float *Y, const int8_t *W, const float *scale, const float *X, int rows, int cols,
                                    int B, void *stream);
/* qwen_quantize_bf16_to_int8 / _q4_0 (k.c:2143, k.c:2662) run on the device; output in
 * the reference's host layout. */
int qwen_hip_op_quantize_int8(const uint16_t *src, int rows, int cols, int8_t *dst, float *scale);
int qwen_hip_op_quantize_q4_0(const uint16_t *src, int rows, int cols, void *dst_blocks);
/* Dequantise rows of a resident Talker weight (layer, which: 0 q 1 k 2 v 3 o 4 gate_up
 * 5 down) to f32, from the device copy: proves upload/repack is bit-exact. */
int qwen_hip_talker_dequant(void *state, int layer, int which, int r0, int n, float *out);

/* ---- speech decoder: codes -> 24 kHz audio (qwen_tts_speech_decoder.c) ---- */
/* Tensor lookup by the reference's names (the role of get_f32 over ctx->speech_safetensors,
 * sd.c:77-80): a host pointer to n_elems contiguous f32 values, or NULL if the tensor is
 * missing or has another size.  The pointer need only stay valid until the next call. */
typedef const float *(*qwen_hip_sd_get_fn)(void *user, const char *name, long long n_elems);
/* replaces qwen_speech_decoder_load (sd.c:372-578): uploads the decoder's weights (the
 * codebooks dequantised from their EMA sums on the device) and returns a state, or NULL
 * (qwen_hip_last_error() names the missing tensor). */
void *qwen_hip_sd_init(qwen_hip_sd_get_fn get, void *user);
/* The same from the speech tokenizer's safetensors file (F32 tensors; a directory is taken
 * to hold speech_decoder.safetensors), read straight from the file. */
void *qwen_hip_sd_load_file(const char *path);
/* replaces qwen_speech_decoder_decode (sd.c:579-1290, the one-shot decode): codes
 * [n_frames][16] (code0, then the 15 CP codes; values outside [0, 2048) contribute
 * nothing) -> audio_out[1920 n_frames] in [-1, 1].  1 <= n_frames <= 8000.  Returns the
 * sample count (1920 n_frames), or -1 (audio_out too small: max_samples). */
int qwen_hip_sd_decode(void *state, const int *codes, int n_frames, float *audio_out, int max_samples);
/* No counterpart in the reference: the same on device buffers (d_codes int[n][16],
 * d_audio f32[1920 n]), enqueued on qwen_hip_sd_stream(state) without a host sync, for
 * callers whose codes are already on the device (qwen_hip_generate's output). */
int qwen_hip_sd_decode_device(void *state, const int *d_codes, int n_frames, float *d_audio);
/* No counterpart in the reference as one call: the VQ lookup and the pre-transformer alone
 * (sd.c:599-1044, what the reference's streaming decode caches per frame): latent_out
 * [n_frames][1024], time-major. */
int qwen_hip_sd_latent(void *state, const int *codes, int n_frames, float *latent_out);
void *qwen_hip_sd_stream(void *state);
void qwen_hip_sd_free(void *state);
/* Streaming decode (qwen_speech_decoder_decode_streaming_st, sd.c:1881-2389: the same
 * contract -- new frames in, exactly their samples out -- with the one-shot decode's
 * arithmetic, so its ConvNeXt LayerNorm is E[x^2] - mean^2 where the reference's streaming
 * path uses a two-pass one, sd.c:1343-1352): a stream state over a decoder state (weights shared; several streams may share one
 * decoder, calls on them are serialised on its stream).  Each call decodes new_frames more
 * frames of the utterance and returns exactly their 1920 new_frames samples, equal to that
 * slice of the one-shot decode of all frames so far (qwen_hip_sd_decode); at most 8000 frames
 * per utterance.  reset starts a new utterance (qwen_sd_stream_init). */
void *qwen_hip_sd_stream_new(void *sd_state);
int qwen_hip_sd_stream_decode(void *stream_state, const int *new_codes, int new_frames, float *audio_out,
                              int max_samples);
int qwen_hip_sd_stream_reset(void *stream_state);
void qwen_hip_sd_stream_free(void *stream_state);
/* The decoder's layers one at a time, on time-major host arrays (X [T][Cin], Y [T][Cout]):
 * causal_conv1d (sd.c:98-119; W [Cout][Cin][kernel], left pad (kernel-1) dilation) and
 * causal_conv_transpose1d (sd.c:122-160; W [Cin][Cout][kernel], kernel <= 2 stride, Y
 * [Tin stride][Cout]); the conv's kernel is at most 8.  bias may be NULL.  tile: 0 = as the decoder picks it, 16, 32,
 * 64 or 128 = force the implicit GEMM's row tile (every tile gives the same bits).  Cin a multiple of 16, Cout of 4. */
int qwen_hip_op_sd_conv(float *Y, const float *X, const float *W, const float *bias, int T, int Cin, int Cout,
                        int kernel, int dilation, int tile);
int qwen_hip_op_sd_conv_transpose(float *Y, const float *X, const float *W, const float *bias, int Tin, int Cin,
                                  int Cout, int kernel, int stride, int tile);

const char *qwen_hip_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* QWEN_TTS_HIP_H */
