/* qt_launch.h — C declarations of the kernel launchers defined in the .hip files. */
#ifndef QT_LAUNCH_H
#define QT_LAUNCH_H
#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* sets the text qwen_hip_last_error() returns (and prints it) */
void qt_seterr(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

enum { QT_BF16 = 0, QT_INT8 = 1, QT_Q4 = 2 };
enum { QT_EPI_STORE = 0, QT_EPI_RESID = 1, QT_EPI_SWIGLU = 2, QT_EPI_BIAS = 3 };
/* token history of the device sampled loop: previous tokens + tokens drawn in one call */
enum { QT_SAMPLE_HIST_MAX = 16384 };

hipError_t qt_launch_mv(int prec, int epi, int norm, const float *vin, const float *nw, float eps,
                        const uint8_t *w, const float *scale, const uint16_t *s16, int rows, int cols,
                        float *out, float *resid, const float *bias, float *nout, hipStream_t st);
hipError_t qt_launch_attn(int prep, const float *q, const float *qn, const float *kn, const float *rc,
                          const float *rs, float eps, const int *d_pos, int Lval, uint16_t *K, uint16_t *V,
                          long long pos_stride, long long head_stride, int n_heads, int n_kv, int head_dim,
                          float scale, float *part, unsigned *cnt, int G, float *out, hipStream_t st);
hipError_t qt_launch_attn_onepass(int prep, const float *q, const float *qn, const float *kn, const float *rc,
                          const float *rs, float eps, const int *d_pos, int Lval, uint16_t *K, uint16_t *V,
                          long long pos_stride, long long head_stride, int n_heads, int n_kv, int head_dim,
                          float scale, float *part, unsigned *cnt, int G, float *out, hipStream_t st);
hipError_t qt_launch_attn_b(const float *q, long long q_bs, const float *qn, const float *kn, const float *rc,
                            const float *rs, float eps, const int *d_pos, uint16_t *K, uint16_t *V, long long kv_bs,
                            long long pos_stride, long long head_stride, int n_heads, int n_kv, int head_dim,
                            float scale, float *part, long long part_bs, unsigned *cnt, int G, float *out,
                            long long out_bs, int B, hipStream_t st);
int qt_attn_grid(int max_len);
/* batched projections (qt_batch.hip) */
hipError_t qt_launch_bpieces(const float *x, long long xstride, const float *norm_w, float eps, int K, int B, int Bp,
                             int8_t *P, float *S, hipStream_t st);
hipError_t qt_launch_bgemm_i8(int epi, const uint8_t *w, const float *scale, int rows, int K, const int8_t *P,
                              const float *S, int B, int Bp, float *out, long long ostride, hipStream_t st);
int qt_bgemm2_plan(int rows, int K, int Bp, int *kb, int *S, int *rt, size_t *part_ints, int *n_cnt);
hipError_t qt_launch_bgemm2_i8(int epi, const uint8_t *w, const float *scale, int rows, int K, const int8_t *P,
                               const float *S, int B, int Bp, float *out, long long ostride, int *part, unsigned *cnt,
                               hipStream_t st);
hipError_t qt_launch_bgemm2_i8_px(int epi, const uint8_t *w, const float *scale, int rows, int K, const float *x,
                                  long long xstride, const float *norm_w, float eps, int8_t *P, float *S, int B, int Bp,
                                  float *out, long long ostride, int *part, unsigned *cnt, unsigned *sync,
                                  int sync_wgs, unsigned *err, hipStream_t st);
int qt_bgemm2_px_wgs(int rows, int K, int Bp);
hipError_t qt_launch_bgemm_q4(int epi, const uint8_t *w, const uint16_t *s16, int rows, int K, const int8_t *P,
                              const float *S, int B, int Bp, float *out, long long ostride, hipStream_t st);
hipError_t qt_launch_advance_pos(int *pos, int n, hipStream_t st);
hipError_t qt_launch_rmsnorm(const float *x, const float *w, float *out, int n, float eps, int *d_pos,
                             hipStream_t st);
hipError_t qt_launch_rmsnorm_rows(float *x, const float *w, int rows, int n, float eps, hipStream_t st);
hipError_t qt_launch_rmsnorm_rows_to(const float *x, float *out, const float *w, int rows, int n, float eps,
                                    int *pos, hipStream_t st);
hipError_t qt_launch_swiglu(const float *gu, float *out, int n, hipStream_t st);
hipError_t qt_launch_sample(const float *logits, int n, int rule, int frame, float eos_boost, float temp,
                            int top_k, float top_p, float rep, const int *prev, int n_prev, uint32_t *seed, int *tok,
                            int *done, hipStream_t st);
hipError_t qt_launch_select(const float *logits, int n, int mode, int *d_frame, int advance, int *tok,
                            int *hist, int hist_len, const uint16_t *emb, int emb_dim, float *out,
                            int *d_pos, hipStream_t st);
hipError_t qt_launch_gather(const int *tok, int tok_max, const uint16_t *table, int dim, float *out,
                            hipStream_t st);
hipError_t qt_launch_copy_f32(const float *src, float *dst, int n, hipStream_t st);
hipError_t qt_launch_quant_int8(const uint16_t *src, int rows, int cols, uint8_t *dst, float *scale,
                                hipStream_t st);
hipError_t qt_launch_repack_q4(const uint8_t *blocks, size_t nblocks, uint8_t *qs, uint16_t *s16,
                               hipStream_t st);
hipError_t qt_launch_quant_q4(const uint16_t *src, int rows, int cols, uint8_t *qs, uint16_t *s16,
                              hipStream_t st);
hipError_t qt_launch_dequant(int prec, const uint8_t *w, const float *scale, const uint16_t *s16, int cols,
                             int r0, int n, float *out, hipStream_t st);
hipError_t qt_launch_zero_u32(uint32_t *p, size_t n, hipStream_t st);
/* next Talker input of the frame loop: codec_emb[codes[0]] + sum_g cp_emb[g][codes[g+1]] + pad */
hipError_t qt_launch_frame_embed(const int *codes, int vocab, int codebook, const uint16_t *codec_emb,
                                 const uint16_t *const cp_emb[15], const float *pad, int H, float *out, hipStream_t st);
/* out rows 2r = gate row r, 2r+1 = up row r (bf16, cols % 8 == 0) */
hipError_t qt_launch_interleave_rows(const uint16_t *gate, const uint16_t *up, uint16_t *out, int rows, int cols,
                                     hipStream_t st);
/* KV rows [n][nkv*hd] (host order) <-> head-major [nkv][kv_max][hd] (device cache) */
hipError_t qt_launch_kv_relayout(const uint16_t *src, uint16_t *dst, int n, int nkv, int hd, int kv_max, int to_heads,
                                 hipStream_t st);

/* role-specialised persistent decode step (qt_rstep.hip), int8 weights: the 1.7B geometry
 * (qt_rstep_* / qt_launch_rstep) and the 0.6B one (qt_rstep06_* / qt_launch_rstep06, built
 * from the same source by qt_rstep06.hip); qt_rstep_chunks holds for both */
int qt_rstep_supported(int prec, int hidden, int inter, int n_heads, int n_kv, int head_dim, int kv_max, int n_layers);
size_t qt_rstep_region_words(int n_layers);
size_t qt_rstep_slot_words(void);
int qt_rstep_chunks(void);
hipError_t qt_launch_rstep(const void *layers_dev, int n_layers, const float *final_norm, const float *rope_cos,
                           const float *rope_sin, uint16_t *kc, uint16_t *vc, int kv_max, float eps, float scale,
                           unsigned *reg, unsigned long long *slots, float *hid, float *decx, float *xin, int *d_pos,
                           unsigned *epoch, int *err, int n_steps, int with_head, const uint16_t *head_w,
                           const uint16_t *emb, int vocab, int *d_frame, int *hist, int hist_len, float *layer_out,
                           hipStream_t st);
hipError_t qt_launch_rstep06_cp(const void *layers_dev, int n_layers, const float *final_norm, const float *rope_cos,
                                const float *rope_sin, uint16_t *kc, uint16_t *vc, int kv_max, float eps, float scale,
                                unsigned *reg, unsigned long long *slots, float *hid, float *decx, float *xin,
                                int *d_pos, unsigned *epoch, int *err, int n_passes, const void *const *cp_tab,
                                int vocab, int *codes, const uint8_t *mtp_w, const float *mtp_s, const float *mtp_b,
                                hipStream_t st);
int qt_rstep06_supported(int prec, int hidden, int inter, int n_heads, int n_kv, int head_dim, int kv_max, int n_layers);
size_t qt_rstep06_region_words(int n_layers);
size_t qt_rstep06_slot_words(void);
hipError_t qt_launch_rstep06(const void *layers_dev, int n_layers, const float *final_norm, const float *rope_cos,
                             const float *rope_sin, uint16_t *kc, uint16_t *vc, int kv_max, float eps, float scale,
                             unsigned *reg, unsigned long long *slots, float *hid, float *decx, float *xin, int *d_pos,
                             unsigned *epoch, int *err, int n_steps, int with_head, const uint16_t *head_w,
                             const uint16_t *emb, int vocab, int *d_frame, int *hist, int hist_len, float *layer_out,
                             hipStream_t st);
/* the same kernel's 0.6B build with bf16 weights (qt_rstep06b.hip): bf16 MFMA on three exact
 * bf16 pieces of every activation; lm heads of the Code Predictor frame bf16 (cp_tab's scale
 * entries unused), mtp projection bf16 (mtp_s unused) */
int qt_rstep06b_supported(int prec, int hidden, int inter, int n_heads, int n_kv, int head_dim, int kv_max, int n_layers);
size_t qt_rstep06b_region_words(int n_layers);
size_t qt_rstep06b_slot_words(void);
hipError_t qt_launch_rstep06b(const void *layers_dev, int n_layers, const float *final_norm, const float *rope_cos,
                              const float *rope_sin, uint16_t *kc, uint16_t *vc, int kv_max, float eps, float scale,
                              unsigned *reg, unsigned long long *slots, float *hid, float *decx, float *xin, int *d_pos,
                              unsigned *epoch, int *err, int n_steps, int with_head, const uint16_t *head_w,
                              const uint16_t *emb, int vocab, int *d_frame, int *hist, int hist_len, float *layer_out,
                              hipStream_t st);
hipError_t qt_launch_rstep06b_cp(const void *layers_dev, int n_layers, const float *final_norm, const float *rope_cos,
                                 const float *rope_sin, uint16_t *kc, uint16_t *vc, int kv_max, float eps, float scale,
                                 unsigned *reg, unsigned long long *slots, float *hid, float *decx, float *xin,
                                 int *d_pos, unsigned *epoch, int *err, int n_passes, const void *const *cp_tab,
                                 int vocab, int *codes, const uint8_t *mtp_w, const float *mtp_s, const float *mtp_b,
                                 hipStream_t st);
/* the same kernel's 1.7B build with q4_0 weights (qt_rstep4.hip): integer MFMA on the exact
 * int8 activation planes, each block's f16 scale applied to its exact sums; layer tables
 * point at the qs rows (w) and the [rows][cols/32] f16 scales (s16) */
int qt_rstep4_supported(int prec, int hidden, int inter, int n_heads, int n_kv, int head_dim, int kv_max, int n_layers);
size_t qt_rstep4_region_words(int n_layers);
size_t qt_rstep4_slot_words(void);
hipError_t qt_launch_rstep4(const void *layers_dev, int n_layers, const float *final_norm, const float *rope_cos,
                            const float *rope_sin, uint16_t *kc, uint16_t *vc, int kv_max, float eps, float scale,
                            unsigned *reg, unsigned long long *slots, float *hid, float *decx, float *xin, int *d_pos,
                            unsigned *epoch, int *err, int n_steps, int with_head, const uint16_t *head_w,
                            const uint16_t *emb, int vocab, int *d_frame, int *hist, int hist_len, float *layer_out,
                            hipStream_t st);
/* persistent decode step (qt_pstep.hip) */
int qt_pstep_supported(int prec, int hidden, int inter, int n_heads, int n_kv, int head_dim, int kv_max);
size_t qt_pstep_ring_words(int hidden, int inter, int n_layers);
size_t qt_pstep_layer_bytes(void);
size_t qt_pstep_ring_x_offset(int hidden, int inter, int n_layers, int par, int l);
void qt_pstep_fill_layer(void *dst, const uint8_t *const w[4], const float *const s[4], const uint16_t *const s16[4],
                         const float *in_norm, const float *post_norm, const float *qn, const float *kn);
hipError_t qt_launch_pstep(int prec, int hidden, const void *layers_dev, int n_layers, const float *final_norm,
                           const float *rope_cos, const float *rope_sin, uint16_t *kc, uint16_t *vc, int kv_max,
                           float eps, float scale, unsigned long long *ring, float *hid, float *decx, float *xin,
                           int *d_pos, unsigned *epoch, int *err, int n_steps, int with_head, const uint16_t *head_w,
                           const uint16_t *emb, int vocab, int *d_frame, int *hist, int hist_len, hipStream_t st);

/* Talker prefill (qt_prefill.hip) */
enum { QT_PF_STORE = 0, QT_PF_RESID = 1, QT_PF_SWIGLU = 2 };
int qt_pf_spad(int S);
hipError_t qt_launch_pf_pieces(const float *X, int ldx, int S, int K, const float *gain, float eps, uint16_t *P,
                               hipStream_t st);
/* part: split-K partials (part_cap floats; NULL: never split) */
hipError_t qt_launch_pf_gemm(int epi, const uint16_t *W, const uint16_t *P, int S, int N, int K, float *Y, int ldy,
                             float *part, long long part_cap, hipStream_t st);
/* SwiGLU projection whose h goes out as the next projection's three input planes (S*N <= part_cap) */
hipError_t qt_launch_pf_gemm_swiglu_planes(const uint16_t *W, const uint16_t *P, int S, int N, int K, uint16_t *Pout,
                                           float *part, long long part_cap, hipStream_t st);
/* residual projection (Y += W . x) whose updated rows, RMS-normalised with gain, go out as the next
 * projection's input planes Pout (S*N <= part_cap) */
/* q|k|v projection whose rows are finished as qt_launch_pf_qkv_post does (per-head norm, RoPE,
 * KV store) by the split-K reduce itself (S*N <= part_cap) */
hipError_t qt_launch_pf_gemm_qkv_post(const uint16_t *W, const uint16_t *P, int S, int N, int K, float *QKV, int ld, int nh,
                                      int nkv, const float *qn, const float *kn, const float *rc, const float *rs, float eps,
                                      uint16_t *kc, uint16_t *vc, long long kv_max, float *part, long long part_cap,
                                      hipStream_t st);
hipError_t qt_launch_pf_gemm_resid_planes(const uint16_t *W, const uint16_t *P, int S, int N, int K, float *Y, int ldy,
                                          const float *gain, float eps, uint16_t *Pout, float *part, long long part_cap,
                                          hipStream_t st);
hipError_t qt_launch_pf_qkv_post(float *QKV, int ld, int S, int nh, int nkv, const float *qn, const float *kn,
                                 const float *rc, const float *rs, float eps, uint16_t *kc, uint16_t *vc,
                                 long long kv_max, hipStream_t st);
hipError_t qt_launch_pf_attn(const float *QKV, int ld, int S, int nh, int nkv, float scale, float *A, int lda,
                             hipStream_t st);
/* as qt_launch_pf_attn, the output going out as the O projection's input planes P instead
 * (*planes = 1) */
hipError_t qt_launch_pf_attn_planes(const float *QKV, int ld, int S, int nh, int nkv, float scale, float *A, int lda,
                                    uint16_t *P, int *planes, hipStream_t st);

/* speech decoder (qt_sd.hip) */
hipError_t qt_launch_sd_gemm(const float *X, int ldx, int Tx, int xlo, const float *W, int K, int N, int ntap, const int *off,
                             int phases, int T, float *Y, int ldy, const float *bias, const float *cscale,
                             const float *R, const float *sa, const float *sib, float *Y2, int epi, int tile,
                             hipStream_t st);
hipError_t qt_launch_sd_cb_dequant(const float *es, const float *cu, float *cb, int rows, int dim, hipStream_t st);
hipError_t qt_launch_sd_snake_params(const float *la, const float *lb, float *a, float *ib, int n, hipStream_t st);
hipError_t qt_launch_sd_vq(const int *codes, const float *cb, float *E, int n, int cbsize, hipStream_t st);
hipError_t qt_launch_sd_rmsnorm(const float *x, const float *w, float *out, int T, int C, float eps, hipStream_t st);
hipError_t qt_launch_sd_rope(float *qkv, const float *cs, const float *sn, int T, int row0, int pos0, hipStream_t st);
hipError_t qt_launch_sd_attn(const float *qkv, float *out, int T, int q0, int kmin, int window, float scale,
                             hipStream_t st);
hipError_t qt_launch_sd_swiglu(const float *gu, float *m, int T, int C, hipStream_t st);
hipError_t qt_launch_sd_dwln(const float *x, const float *dw, const float *db, const float *lw, const float *lb,
                             float *out, int T, int C, int xlo, hipStream_t st);
hipError_t qt_launch_sd_final(const float *x, const float *w, const float *b, float *audio, int T, int C, int xlo,
                              hipStream_t st);
hipError_t qt_launch_sd_shift(float *buf, int H, int T, int C, hipStream_t st);
#ifdef __cplusplus
}
#endif
#endif
