/*
 * qwen_tts_hip_glue.h — the reference side of the drop-in: functions the reference
 * engine calls at its GPU hook points, built into the reference (make hip) together
 * with qwen_tts_hip_glue.c and linked against libqwen_tts_hip.so.  They take the
 * reference's qwen_tts_ctx_t (qwen_tts.h) and translate it into the library's plain
 * descriptors (include/qwen_tts_hip.h).
 */
#ifndef QWEN_TTS_HIP_GLUE_H
#define QWEN_TTS_HIP_GLUE_H

#include <stdint.h>

#include "qwen_tts.h"
#include "qwen_tts_backend.h"
#include "qwen_tts_hip.h"

/* The HIP kind of the reference's backend vtable (qwen_tts_backend.h:28-32 lists CPU 0,
 * METAL 1, CUDA 2): the value a maintainer adds to qwen_backend_kind_t. */
#define QWEN_BACKEND_HIP ((qwen_backend_kind_t)3)

/* What qwen_backend_init(QWEN_BACKEND_HIP) returns (qwen_tts_backend.c:106-150, the CUDA
 * branch's shape): a qwen_backend_t of kind QWEN_BACKEND_HIP, name "hip", whose
 * matvec_bf16 / matmat_bf16 are qwen_hip_matvec_bf16 / qwen_hip_matmat_bf16 on a
 * qwen_hip_init() context and whose free releases both.  NULL when no HIP device is
 * present or the context cannot be made: the caller then keeps the CPU backend, as
 * qwen_backend_init does.  qwen_backend_install_global(b) routes qwen_matvec_bf16 (and the
 * fused bf16 QKV matvec) and qwen_matmat_bf16 through it unchanged. */
qwen_backend_t *qwen_hip_glue_backend_new(void);

/* qwen_cuda_talker_init(ctx) (qwen_tts_cuda_talker.cu:313): the Talker layers at the
 * precision their pointers carry (q4 > int8 > bf16, qwen_tts_talker.c:587-600); a device
 * KV cache of kv_max positions (0: ctx->kv_max).  NULL: stay on the CPU path. */
void *qwen_hip_glue_talker_init(qwen_tts_ctx_t *ctx, int kv_max);
/* the delegation at the top of qwen_talker_step (qwen_tts_talker.c:552-563): one step at
 * pos = ctx->kv_len, ctx->dec_x refreshed, kv_len advanced.  0 on success. */
int qwen_hip_glue_talker_step(void *state, qwen_tts_ctx_t *ctx, float *embed, float *hidden_out);
/* the hand-off after the CPU prefill (qwen_tts.c:1466-1476) */
int qwen_hip_glue_upload_kv(void *state, qwen_tts_ctx_t *ctx, int prefill_len);
/* the prefill itself on the device, in place of qwen_talker_prefill + upload
 * (qwen_tts.c:1454-1476): KV rows [0, seq) and dec_x; ctx->kv_len = seq. */
int qwen_hip_glue_talker_prefill(void *state, qwen_tts_ctx_t *ctx, float *embeds, int seq);

/* qwen_cuda_cp_init(ctx) (qwen_tts_cuda_talker.cu:751) */
void *qwen_hip_glue_cp_init(qwen_tts_ctx_t *ctx);
/* the device frame in front of qwen_cp_predict's CPU loop (qwen_tts_code_predictor.c:931-941) */
int qwen_hip_glue_cp_predict(void *state, float *talker_hidden, int code0, int *out_codes);
/* the per-pass delegation of cp_transformer_step (qwen_tts_code_predictor.c:742-747) */
int qwen_hip_glue_cp_step(void *state, qwen_tts_ctx_t *ctx, float *x, int pos);

/* code0 of frame `frame` from ctx->logits (the codec head's output): the codec-head rule
 * with the EOS boost for text_content_len, greedy warmup, qwen_tts_sample with the
 * context's settings and history (qwen_tts.c:1652-1691), on the device.  *lcg is the
 * sampler state (seeded from ctx->seed as qwen_set_seed seeds the CPU sampler).
 * Returns the token, or -1 (then the caller samples on the CPU). */
int qwen_hip_glue_codec_sample(qwen_tts_ctx_t *ctx, int frame, int text_content_len, uint32_t *lcg);

/* qwen_speech_decoder_load(ctx) (qwen_tts_speech_decoder.c:372): the decoder's F32 tensors
 * from ctx->speech_safetensors by name, as get_f32 finds them (sd.c:77-80), onto the
 * device.  NULL: stay on the CPU decoder. */
void *qwen_hip_glue_sd_init(qwen_tts_ctx_t *ctx);
/* qwen_speech_decoder_decode's contract (sd.c:579): codes [n_frames][16] -> *audio_out
 * (malloc'd, the caller frees it as it frees the CPU decoder's) of *n_samples samples.
 * 0 on success. */
int qwen_hip_glue_sd_decode(void *state, const int *codes, int n_frames, float **audio_out, int *n_samples);

#endif
