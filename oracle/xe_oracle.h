/*
 * xe_oracle.h -- CPU restatement of atassis/xdna-engine's decode arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP product
 * path: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it.  The product library (libxdna_engine.so) never links or calls
 * it, and has no CPU fallback.
 *
 * Every function cites the reference file:line whose arithmetic it restates
 * (paths relative to the reference root).  Pins (what checks each function
 * against something other than its own formula) are listed per function;
 * "parity unpinned" marks a function nothing but its own restatement backs.
 *
 * Conventions
 *   - Weight matrices are [M, K] row-major (output-major, one row per output
 *     channel).  The reference CPU OPT path stores [K, N] with per-column
 *     scales (opt125m_decode.rs:30-62); that is the transpose with identical
 *     per-output arithmetic, and every accumulation below runs k = 0..K-1 in
 *     order exactly as the reference's k-outer loops do.
 *   - Compiled with -ffp-contract=off: no fused multiply-add unless written.
 */
#ifndef XE_ORACLE_H
#define XE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/xdna_engine.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 (npu-xrt/src/lib.rs:809-822, npu-asr-host/src/lib.rs:12-19) ---- */
uint16_t xo_f32_to_bf16_bits(float x);
float xo_bf16_bits_to_f32(uint16_t b);
float xo_bf16_round(float x);
void xo_pack_bf16(const float *src, uint16_t *dst, size_t n);
void xo_unpack_bf16(const uint16_t *src, float *dst, size_t n);

/* ---- norms / activations ---- */
void xo_layer_norm(const float *x, int rows, int d, const float *gamma,
                   const float *beta, float eps, float *out);
void xo_layer_norm_normalize(const float *x, int rows, int d, float eps,
                             float *out);
void xo_rmsnorm(const float *x, int n, const float *w, float eps, float *out);
float xo_erf_as(float x);
float xo_gelu_erf(float x);
float xo_gelu_tanh(float x);
float xo_fast_exp_nonpos(float x);

/* ---- int8 quantisation (opt125m_decode.rs:45-62, ctx2.rs:1352-1435) ---- */
int8_t xo_quant_i8(float x, float scale);
float xo_quant_scale(const float *a, size_t n);
void xo_quant_rows_i8(const float *w, int m, int k, int8_t *q, float *s);
void xo_quant_cols_i8(const float *w_kn, int k, int n, int8_t *q_kn,
                      float *s);
/* gen_decode.py qrow (:158-165): half-even rounding, bf16-stored scale. */
void xo_quant_rows_i8_elf(const float *w, int m, int k, int8_t *q, float *s_out);
void xo_dequant_epi(const int32_t *acc, int mp, int n, float scale_a,
                    const float *ws, const float *bias, float *out);

/* ---- weight-only GEMV / linear (opt125m_decode.rs:106-125) ---- */
void xo_gemv_i8(const float *x, int b, int k, int m, const int8_t *q,
                const float *s, const float *bias, float *y);
/* xo_gemv_i8 computed from a k-major copy in blocks of 8 rows (the form
 * the decoder models use); bit-identical to xo_gemv_i8. */
void xo_gemv_i8_rowblocked(const float *x, int b, int k, int m, const int8_t *q,
                           const float *s, const float *bias, float *y);
void xo_lin_fwd_i8_kn(const float *x, int b, int k, int n, const int8_t *q_kn,
                      const float *s, const float *bias, float *y);
/* ---- int4 weights (opt125m_decode.rs:63-105) ---- */
void xo_quant_cols_i4(const float *w_kn, int k, int n, uint8_t *packed_kn, float *s);
void xo_lin_fwd_i4_kn(const float *x, int b, int k, int n, const uint8_t *packed_kn,
                      const float *s, const float *bias, float *y);
void xo_quant_rows_i4(const float *w, int m, int k, uint8_t *packed, float *s);
void xo_gemv_i4(const float *x, int b, int k, int m, const uint8_t *packed,
                const float *s, const float *bias, float *y);
void xo_gemv_f32(const float *x, int b, int k, int m, const float *w,
                 const float *bias, float *y);
void xo_gemv_bf16w(const float *x, int b, int k, int m, const uint16_t *w,
                   const float *bias, float *y);

/* ---- bfp16ebs8 block format (ffn_bfp16/golden_ffn_gemm.py:21-49) ---- */
void xo_bfp16_encode(const float *w, int m, int k, int8_t *mant,
                     uint8_t *exps);
void xo_bfp16_decode(const int8_t *mant, const uint8_t *exps, int m, int k,
                     float *w);
void xo_gemv_bfp16(const float *x, int b, int k, int m, const int8_t *mant,
                   const uint8_t *exps, const float *bias, float *y);

/* ---- W8A8 (ctx2.rs:771-830, 1352-1435) ---- */
void xo_gemm_i8i8_i32(const int8_t *a, int mp, int k, const int8_t *w, int m,
                      int32_t *acc);
void xo_w8a8_linear(const float *a, int mp, int k, const int8_t *wq,
                    const float *ws, int m, const float *bias, float *out,
                    float *scale_a_out);
/* dequant epilogues of ctx2.rs Epi (None / Bias / SiluBias). */
enum { XO_EPI_NONE = 0, XO_EPI_BIAS = 1, XO_EPI_SILU_BIAS = 2 };
float xo_fast_sigmoid(float x);
void xo_w8a8_linear_epi(const float *a, int mp, int k, const int8_t *wq,
                        const float *ws, int m, const float *bias, int epi, float *out,
                        float *scale_a_out);

/* ---- fused norm + GEMV (ctx_decode.rs:566-643) ---- */
enum { XO_NORM_NONE = 0, XO_NORM_LN = 1, XO_NORM_RMS = 2, XO_NORM_RMS1P = 3 };
void xo_norm_row(const float *x, int k, int norm, const float *gamma,
                 const float *beta, float eps, float *out);
void xo_fold_weight(const float *w, int m, int k, const float *gamma,
                    const float *beta, const float *bias, float *w_fold,
                    float *bias_fold);

/* ---- attention (whisper_decoder.rs:242-278, mha_decode.cc:90-168) ---- */
void xo_attend_one(const float *q, const float *k_flat, const float *v_flat,
                   int s, int n_heads, int head_dim, float *ctx);
void xo_attn_decode(const float *q, const uint16_t *kc, const uint16_t *vc,
                    const int *lens, int batch, int hq, int hkv, int hd,
                    int max_ctx, float scale, float *out);
void xo_attn_online(const float *q, const uint16_t *kc, const uint16_t *vc,
                    int len, int hd, float scale, float *out);

void xo_rope(const float *x, int rows, int n_heads, int head_dim,
             const float *cos_t, const float *sin_t, float *out);

/* ---- argmax (opt125m_decode.rs:303 last-max; whisper.rs:749-757 first) -- */
int xo_argmax_first(const float *v, int n);
int xo_argmax_last(const float *v, int n);

/* ---- synthetic weights: counter-based, bit-reproducible on CPU and GPU ---- */
uint64_t xo_synth_base(uint64_t seed, uint32_t tensor);
float xo_synth_value(uint64_t base, uint64_t idx, float mean, float stdv);
void xo_synth_fill(uint64_t seed, uint32_t tensor, float mean, float stdv,
                   float *out, size_t n);
void xo_synth_fill_range(uint64_t seed, uint32_t tensor, float mean, float stdv,
                         uint64_t start, float *out, size_t n);

/* ---- decoder models (configs 1, 4, 5) ----
 * The config struct and tensor kinds are the public ones of
 * include/xdna_engine.h, so both sides key the synthetic weights alike. */
typedef struct xo_model xo_model;
xo_model *xo_model_create(const xe_model_config *cfg, uint64_t seed,
                          int batch);
void xo_model_free(xo_model *m);
void xo_model_reset(xo_model *m);
/* fp32 K/V caches instead of bf16 (the reference CPU decoders' choice);
 * clears them.  Used to compare the composition with fp32 implementations. */
int xo_model_set_kv_f32(xo_model *m, int on);
/* Planted composition mistakes, for tests that show the decoder fixtures
 * catch them (0 = none). */
enum {
  XO_MUT_NONE = 0,
  XO_MUT_OPT_POS_OFFSET = 1,       /* OPT position row pos + 1, not pos + 2 */
  XO_MUT_GEMMA_SWAP_POST_NORMS = 2,/* post-attention norm with the post-FFN weight */
  XO_MUT_GEMMA_NO_EMB_SCALE = 3,   /* no sqrt(d) embedding scale */
  XO_MUT_ROPE_THETA = 4,           /* RoPE theta 1e4 instead of the config's */
  XO_MUT_WHISPER_CROSS_SCALE = 5,  /* cross-attention scores without 1/sqrt(hd) */
  XO_MUT_OPT_NO_Q_SCALE = 6        /* OPT q not scaled by hd^-0.5 */
};
int xo_model_set_mutation(xo_model *m, int code);
/* int8 linears through the reference's k-outer [K, N] loop (same values). */
int xo_model_set_kouter(xo_model *m, int on);
/* Synthetic bf16 K/V rows [0, n_pos) for stream b (timing at long contexts). */
int xo_model_prime_kv(xo_model *m, int b, int n_pos, uint64_t seed);
/* int8 per-utterance cross K and/or V (the fused decode ELF's int8_cross_k /
 * int8_cross_v); takes effect at the next xo_model_set_cross. */
int xo_model_set_cross_i8(xo_model *m, int k_int8, int v_int8);
/* enc [n_cross, d]; NULL = the synthetic XE_T_ENC_OUT tensor. */
int xo_model_set_cross(xo_model *m, const float *enc);
/* Per-channel int8 of one layer's cross K or V (whisper_decoder.rs:1186-1219,
 * write_buf_i8 :1110-1134): x fp32 [T, H*hd] (the projection's rows), channel
 * (h, d) scale s = max_t |x| / 127 (1.0 for an all-zero channel), q = clamp(
 * round_half_away(x * (1/s)), -127, 127) stored head-major [H, T, hd]. */
void xo_quant_cross_i8(const float *x, int T, int H, int hd, int8_t *q, float *s);
/* One head's attention over int8 and/or bf16 cross K/V: with k8, scores
 * (sum_d (q[d] s_k[d]) k8[t][d]) * scale (gen_decode.py:263-272: the channel
 * scale applied to q); with v8, out[d] = s_v[d] * sum_t p_t v8[t][d]
 * (:273-279: applied after the sum); kb / vb (bf16) otherwise. */
void xo_head_attend_x8(const float *qh, const int8_t *k8, const float *sk, const uint16_t *kb,
                       const int8_t *v8, const float *sv, const uint16_t *vb, int len, int hd,
                       float scale, float *sc, float *oh);
/* One step for every stream b < batch: tokens[b] at pos[b]. */
void xo_model_step(xo_model *m, const int *tokens, const int *pos, int batch,
                   float *logits);
int xo_model_argmax(const xo_model *m, const float *logits);
size_t xo_model_tensor_numel(const xo_model *m, int kind, int layer);
int xo_model_tensor_f32(const xo_model *m, int kind, int layer, float *out);
int xo_model_tensor_q8(const xo_model *m, int kind, int layer, int8_t *q,
                       float *s);
/* prompt [batch, n_prompt] -> out [batch, n_new]; margins [batch, n_new]
 * receives top1 - top2 logit per emitted token (may be NULL). */
int xo_model_generate(xo_model *m, const int *prompt, int n_prompt, int batch,
                      int n_new, int *out, float *margins);
/* xo_model_generate with the EOT rule: stream b ends at its first emitted
 * token equal to stop (stop < 0: never); out holds stop from there on and
 * n_out[b] (may be NULL) the number of tokens before it. */
int xo_model_generate_until(xo_model *m, const int *prompt, int n_prompt, int batch, int n_new,
                            int stop, int *out, int *n_out, float *margins);
void xo_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
