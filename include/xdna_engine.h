/*
 * xdna_engine.h -- C ABI of the MI355X (gfx950) decode backend.
 *
 * Drop-in for xdna-engine's fused decode hot path: the device layer replaces
 * the XRT shim (rust/npu-xrt/shim/xrt_shim.h:16-113), the op layer replaces
 * CtxDecode (rust/npu-asr/src/ctx_decode.rs:142-694) and the decoder layer
 * replaces the decode-backend contract of HostDecoder / FusedDecoder /
 * BatchedFusedDecoder (rust/npu-engine/src/asr/whisper_decoder.rs:204-1831)
 * and Opt::step/generate (rust/npu-whisper/src/bin/opt125m_decode.rs:252-315).
 *
 * Conventions (mirroring rust/npu-capi/src/lib.rs:11-41 and
 * rust/npu-xrt/shim/xrt_shim.cpp:42-56):
 *   - Every entry point catches all C++ exceptions; failures return NULL or a
 *     negative value and set a thread-local message read by xe_last_error().
 *   - Handles are opaque; the caller destroys what it creates.
 *   - Host buffers passed in are only read (or written) during the call.
 *   - A handle is not thread-safe; one decode context per stream.
 *   - Weight matrices are [M, K] row-major (out-major, nn.Linear layout)
 *     unless XE_LAYOUT_KN is given, which is the reference's [K, N] layout
 *     (opt125m_decode.rs:30-31, ctx_decode.rs:269-317).
 */
#ifndef XDNA_ENGINE_H
#define XDNA_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XE_ABI_VERSION 1

typedef struct xe_device xe_device;
typedef struct xe_buf xe_buf;
typedef struct xe_ctx xe_ctx;
typedef struct xe_weight xe_weight;
typedef struct xe_decoder xe_decoder;

/* element types */
enum xe_dtype {
  XE_F32 = 0,
  XE_BF16 = 1,
  XE_I8 = 2,    /* int8 symmetric, per-output-row fp32 scale */
  XE_BFP16 = 3, /* 8 int8 mantissas per block + one biased 8-bit exponent */
  XE_I32 = 4,
  XE_I4 = 5     /* int4 symmetric (+-7), per-output-row fp32 scale; two
                   nibbles a byte along k (k = 2j low, 2j+1 high) */
};

/* pre-norm of the fused norm+GEMV (ctx_decode.rs:74-79 Norm) */
enum xe_norm {
  XE_NORM_NONE = 0,
  XE_NORM_LN = 1,    /* LayerNorm(gamma, beta, eps), population variance */
  XE_NORM_RMS = 2,   /* RMSNorm: x * inv_rms * gamma */
  XE_NORM_RMS1P = 3  /* Gemma RMSNorm: x * inv_rms * (1 + w) */
};

enum xe_layout { XE_LAYOUT_MK = 0, XE_LAYOUT_KN = 1 };

/* ------------------------------------------------------------------------ */
/* errors / version                                                         */
/* ------------------------------------------------------------------------ */

/* Thread-local message of the last failed call (xrt_shim.cpp:42-56,
 * npu-capi/src/lib.rs:11-16).  Never NULL; "" when no error. */
const char *xe_last_error(void);
int xe_abi_version(void);

/* ------------------------------------------------------------------------ */
/* device layer (xrt_shim.h:16-113)                                         */
/* ------------------------------------------------------------------------ */

/* Number of visible GPUs (0 when none). */
int xe_device_count(void);
/* shim_device_open(index) (xrt_shim.h:20). */
xe_device *xe_device_open(int ordinal);
/* shim_device_close (xrt_shim.h:21). */
void xe_device_close(xe_device *dev);
/* Wait for all work queued on the device's stream. */
int xe_device_synchronize(xe_device *dev);
/* Device name (e.g. "gfx950") into buf; returns bytes written or -1. */
int xe_device_name(xe_device *dev, char *buf, int cap);

/* shim_bo_alloc (xrt_shim.h:30-33): device memory of nbytes. */
xe_buf *xe_buf_alloc(xe_device *dev, size_t nbytes);
/* shim_bo_free (xrt_shim.h:34). */
void xe_buf_free(xe_buf *buf);
/* shim_bo_write + sync_to_device (xrt_shim.h:37-40): host -> device. */
int xe_buf_write(xe_buf *buf, const void *src, size_t nbytes, size_t offset);
/* sync_from_device + shim_bo_read (xrt_shim.h:38-41): device -> host. */
int xe_buf_read(xe_buf *buf, void *dst, size_t nbytes, size_t offset);
/* Device address of the buffer (for the *_dev entry points). */
void *xe_buf_device_ptr(xe_buf *buf);
size_t xe_buf_size(xe_buf *buf);
/* Fill count elements at byte offset of buf with elements [start, start +
 * count) of the counter-based synthetic stream (seed, stream) that
 * xe_decoder_init_synthetic uses for weights: value = mean + stdv * z, z an
 * Irwin-Hall (n=4) approximately normal variate; stored as XE_F32, XE_BF16
 * (RNE) or XE_I8 (rounded half away from zero, clamped to +-127).
 * Deterministic and bit-identical to the CPU generator, so multi-GB test and
 * benchmark inputs are made in HBM without a host copy.  No counterpart in
 * the reference (its inputs come from files). */
int xe_buf_fill_synthetic(xe_buf *buf, size_t offset, int dtype, uint64_t seed,
                          uint32_t stream, uint64_t start, float mean,
                          float stdv, size_t count);
/* Device-to-device copy by a streaming kernel (one read, one write per
 * byte); sizes and offsets multiples of 16 bytes.  Also the known-size copy
 * that calibrates the HBM byte counters. */
int xe_buf_copy(xe_buf *dst, size_t dst_off, const xe_buf *src, size_t src_off,
                size_t nbytes);

/* ------------------------------------------------------------------------ */
/* op layer (CtxDecode, ctx_decode.rs:142-694)                              */
/* ------------------------------------------------------------------------ */

/* CtxDecode::new (ctx_decode.rs:174-200). */
xe_ctx *xe_ctx_create(xe_device *dev);
void xe_ctx_destroy(xe_ctx *ctx);
/* Kernel launches issued so far / reset (ctx_decode.rs:148-172). */
uint64_t xe_ctx_dispatches(xe_ctx *ctx);
void xe_ctx_reset_dispatches(xe_ctx *ctx);

/* CtxDecode::register_weight (ctx_decode.rs:269-317): copy W (fp32, layout
 * MK [m,k] or KN [k,m]) to the device, quantised to wdtype (XE_I8: per-row
 * symmetric int8, scale = amax/127, round half away from zero, clamp +-127 --
 * opt125m_decode.rs:45-62; XE_I4: scale = amax/7, clamp +-7 --
 * opt125m_decode.rs:63-79; XE_BFP16; XE_BF16 RNE).  bias may be NULL. */
xe_weight *xe_register_weight(xe_ctx *ctx, int wdtype, int m, int k,
                              const float *w, int layout, const float *bias);
/* int8 quantisation rules of the reference:
 *   XE_Q8_LIN  Lin::load (opt125m_decode.rs:45-62): fp32 scale amax/127,
 *              round half away from zero (xe_register_weight's rule);
 *   XE_Q8_ELF  the fused decode ELF's static rows (route_b_kernels/
 *              decode_fused/gen_decode.py:158-165, 291-298): numpy round
 *              half to even of w / (amax/127), the scale stored as bf16. */
enum xe_q8_rule { XE_Q8_LIN = 0, XE_Q8_ELF = 1 };
/* xe_register_weight with XE_I8 under the given rule (enum xe_q8_rule). */
xe_weight *xe_register_weight_q8_rule(xe_ctx *ctx, int m, int k,
                                      const float *w, int layout,
                                      const float *bias, int rule);
/* Pre-quantised int8 weight: q [m,k] row-major, scales [m] (fp32). */
xe_weight *xe_register_weight_q8(xe_ctx *ctx, int m, int k, const int8_t *q,
                                 const float *scales, const float *bias);
/* Pre-quantised int4 weight (Lin int4 branch, opt125m_decode.rs:63-105):
 * packed uint8 [m, k/2], byte j of row r holding k = 2j in the low nibble
 * and k = 2j+1 in the high one (two's complement, -7..7), scales [m] fp32.
 * The reference's own packing ([K, N/2], two output columns a byte) is taken
 * by xe_register_weight_q4_kn. */
xe_weight *xe_register_weight_q4(xe_ctx *ctx, int m, int k, const uint8_t *packed,
                                 const float *scales, const float *bias);
/* The reference's int4 layout as Lin::load builds it: packed_kn [k, m/2]
 * (row r = input k, byte c2 = output columns 2*c2 (low) and 2*c2+1 (high)),
 * scales [m]; repacked along k at registration.  m even. */
xe_weight *xe_register_weight_q4_kn(xe_ctx *ctx, int m, int k, const uint8_t *packed_kn,
                                    const float *scales, const float *bias);
/* Pre-encoded bfp16 weight: mant [m,k] int8, exps [m,k/8] biased (e+127). */
xe_weight *xe_register_weight_bfp16(xe_ctx *ctx, int m, int k,
                                    const int8_t *mant, const uint8_t *exps,
                                    const float *bias);
/* Pre-rounded bf16 weight: bits [m,k]. */
xe_weight *xe_register_weight_bf16(xe_ctx *ctx, int m, int k,
                                   const uint16_t *bits, const float *bias);
/* A weight over device memory the caller owns (no copy; freeing the view
 * leaves the memory alone): w_dev in the layout of the dtype above,
 * scale_dev [m] fp32 (XE_I8), exps_dev [m, k/8] (XE_BFP16), bias_dev [m] or
 * NULL.  The register-once form of DecodeWeight (ctx_decode.rs:82-140) for
 * weights already resident, e.g. in a loaded arena (npu-weights/src/
 * arena.rs:14-99). */
xe_weight *xe_register_weight_view(xe_ctx *ctx, int wdtype, int m, int k,
                                   const void *w_dev, const float *scale_dev,
                                   const uint8_t *exps_dev,
                                   const float *bias_dev);
/* CtxDecode::register_fused (ctx_decode.rs:566-612): a weight plus a pre-norm
 * (enum xe_norm) applied to x on the device before the GEMV.  gamma/beta have
 * k elements (beta only for XE_NORM_LN). */
xe_weight *xe_register_fused(xe_ctx *ctx, int wdtype, int m, int k,
                             const float *w, int layout, int norm,
                             const float *gamma, const float *beta, float eps,
                             const float *bias);
/* Attach a pre-norm to an already registered weight (q8/bfp16/bf16). */
int xe_weight_set_norm(xe_weight *w, int norm, const float *gamma,
                       const float *beta, float eps);
void xe_weight_free(xe_weight *w);
int xe_weight_shape(const xe_weight *w, int *m, int *k, int *wdtype);

/* CtxDecode::gemv (ctx_decode.rs:325-366), batched: y[b,m] = W x[b,k]
 * (+ bias), fp32 out.  x_dtype XE_F32 or XE_BF16 (host pointer).  batch
 * 1..512 (the reference's batched tiles go to Mp = 512, ctx2.rs:46-55): up
 * to 8 rows run the bandwidth GEMV, more the MFMA GEMM (bf16-split fp32
 * activations, fp32 accumulate). */
int xe_gemv(xe_ctx *ctx, const xe_weight *w, const void *x, int x_dtype,
            int batch, float *y);
/* CtxDecode::fused_norm_gemv (ctx_decode.rs:617-643). */
int xe_fused_norm_gemv(xe_ctx *ctx, const xe_weight *w, const void *x,
                       int x_dtype, int batch, float *y);
/* Device-pointer form of xe_gemv / xe_fused_norm_gemv (no host copies; the
 * weight's pre-norm, if any, is applied).  Asynchronous on the ctx stream.
 * More than 8 rows need XE_F32 x. */
int xe_gemv_dev(xe_ctx *ctx, const xe_weight *w, const void *x_dev,
                int x_dtype, int batch, float *y_dev);

/* int8 activations x int8 weights -> int32 (ctx2.rs:771-830 device part):
 * acc[b,m] = sum_k xq[b,k] * q[m,k], exact.  w must be XE_I8; batch 1..512
 * (<= 8 rows an sdot4 GEMV, more the int8 MFMA GEMM). */
int xe_gemv_i8act(xe_ctx *ctx, const xe_weight *w, const int8_t *xq,
                  int batch, int32_t *acc);
int xe_gemv_i8act_dev(xe_ctx *ctx, const xe_weight *w, const int8_t *xq_dev,
                      int batch, int32_t *acc_dev);
/* W8A8 dynamic linear (ctx2.rs:771-830, 1352-1435): per-tensor activation
 * scale amax/127, int8 x int8 -> i32, dequant in the order
 * (acc * scale_a) * ws[c] (+ bias[c]) -- all on the device; batch 1..512
 * (<= 8 rows an sdot4 GEMV, more the int8 MFMA GEMM).  Epi::Bias when the
 * weight has a bias, Epi::None otherwise.  scale_a_out may be NULL. */
int xe_w8a8_linear(xe_ctx *ctx, const xe_weight *w, const float *x,
                   int batch, float *y, float *scale_a_out);
/* dequant epilogues of the reference's Epi (ctx2.rs:1386-1435). */
enum xe_epi {
  XE_EPI_NONE = 0,      /* (acc * scale_a) * ws[c] */
  XE_EPI_BIAS = 1,      /* ... + bias[c] */
  XE_EPI_SILU_BIAS = 2  /* z = ... + bias[c]; z * fast_sigmoid(z) (:1338-1348) */
};
/* Device-pointer form (asynchronous on the ctx stream): x_dev fp32
 * [batch, k], y_dev fp32 [batch, m], scale_a_dev (a device float, may be
 * NULL) receives scale_a.  epi is enum xe_epi. */
int xe_w8a8_linear_dev(xe_ctx *ctx, const xe_weight *w, const float *x_dev,
                       int batch, int epi, float *y_dev, float *scale_a_dev);

/* Single-query attention over a bf16 KV cache (CtxDecode::attn,
 * ctx_decode.rs:468-555; mha_decode.cc:90-175), generalised to GQA,
 * per-sequence lengths and long contexts.
 *   q     fp32 [batch, hq, hd]
 *   kc,vc bf16 [batch, hkv, max_ctx, hd]
 *   lens  int32 [batch] (1 <= lens[i] <= max_ctx)
 *   out   fp32 [batch, hq, hd]
 * scores = (q . k) * scale; softmax over positions [0, lens[i]). */
int xe_attn_decode(xe_ctx *ctx, const float *q, const uint16_t *kc,
                   const uint16_t *vc, const int32_t *lens, int batch, int hq,
                   int hkv, int hd, int max_ctx, float scale, float *out);
int xe_attn_decode_dev(xe_ctx *ctx, const float *q_dev, const uint16_t *kc_dev,
                       const uint16_t *vc_dev, const int32_t *lens_dev,
                       int batch, int hq, int hkv, int hd, int max_ctx,
                       float scale, float *out_dev);
/* xe_attn_decode_dev without any allocation.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * split partials go to a static per-GPU workspace of 4 Mi floats (16 MB)
 * instead of the ctx's own; a call needing more (batch * hq * splits *
 * (hd + 2) floats, splits <= 64) fails with -1.  Same kernels and results
 * as xe_attn_decode_dev.  Calls that overlap on one GPU (any ctx, any
 * thread) share the workspace and race: serialise them. */
int xe_attn_decode_dev_static(xe_ctx *ctx, const float *q_dev,
                              const uint16_t *kc_dev, const uint16_t *vc_dev,
                              const int32_t *lens_dev, int batch, int hq,
                              int hkv, int hd, int max_ctx, float scale,
                              float *out_dev);

/* Wait for the ctx stream; returns 0 or -1. */
int xe_ctx_synchronize(xe_ctx *ctx);

/* ---- asynchronous submission (xrt_shim.h:47-54: shim_run_*_start returns
 * a run handle without waiting, shim_run_wait blocks, shim_run_free) ----
 * The *_dev entry points queue their work on the ctx stream and return at
 * once; xe_ctx_record then takes a handle on everything queued so far, so
 * shim_run_matmul8_start maps to xe_gemv_dev + xe_ctx_record.  Buffers the
 * work reads or writes must stay alive until the handle completes. */
typedef struct xe_run xe_run;
xe_run *xe_ctx_record(xe_ctx *ctx);
/* 1 = complete, 0 = still running, -1 = error (xe_last_error). */
int xe_run_query(xe_run *run);
/* Block until complete: 0, or -1 (for a resident dispatch, also when its
 * step reported a failure). */
int xe_run_wait(xe_run *run);
/* Free a handle (waits for its work first). */
void xe_run_free(xe_run *run);

/* Kernel probes (the reference's decode_gemv_probe.rs / mha_decode_probe.rs
 * timing runs): the launches of one xe_gemv_dev per weight in ws (same
 * shape; rotating copies defeat the 256 MB last-level cache) or of one
 * xe_attn_decode_dev call, repeated reps times; the device time (HIP events
 * on the ctx stream) per launch / per call is returned in microseconds.
 * flags 0: the launches are captured in a HIP graph and the graph replayed
 * (no host gaps); XE_PROBE_EAGER: plain launches (for runs under a kernel
 * tracer, which reports the kernel durations itself). */
enum { XE_PROBE_EAGER = 1 };
int xe_probe_gemv(xe_ctx *ctx, const xe_weight *const *ws, int n_weights,
                  const void *x_dev, int x_dtype, int batch, float *y_dev,
                  int reps, int flags, double *us_per_launch);
int xe_probe_attn(xe_ctx *ctx, const float *q_dev, const uint16_t *kc_dev,
                  const uint16_t *vc_dev, const int32_t *lens_dev, int batch,
                  int hq, int hkv, int hd, int max_ctx, float scale,
                  float *out_dev, int reps, int flags, double *us_per_call);

/* ------------------------------------------------------------------------ */
/* decoder layer (decode-backend contract)                                  */
/* ------------------------------------------------------------------------ */

enum xe_family { XE_OPT = 0, XE_WHISPER = 1, XE_GEMMA3 = 2 };

typedef struct xe_model_config {
  int family;      /* enum xe_family */
  int n_layers;
  int d_model;
  int n_heads;     /* query heads */
  int n_kv_heads;
  int head_dim;
  int ffn;
  int vocab;
  int max_pos;     /* learned position rows (OPT table has max_pos + 2) */
  int max_ctx;     /* KV capacity per sequence */
  int wdtype;      /* XE_I8 / XE_BF16 / XE_BFP16 for linears + embedding */
  float eps;
  float rope_theta;
  int n_cross;     /* Whisper encoder frames (0 otherwise) */
} xe_model_config;

/* Tensor kinds of a decoder (names follow the reference weight files:
 * opt125m_decode.rs:155-181, whisper_decoder.rs LayerWeights, HF Gemma3).
 * Layer tensors are addressed with (kind, layer); global ones use layer -1.
 * Matrices are [out, in]. */
enum xe_tensor {
  XE_T_TOK_EMB = 0, /* [vocab, d]; also the tied lm-head */
  XE_T_POS_EMB = 1, /* [max_pos(+2 for OPT), d] learned positions */
  XE_T_LNF_W = 2,   /* final norm (OPT ln_final, Whisper ln_post, Gemma norm) */
  XE_T_LNF_B = 3,
  XE_T_ENC_OUT = 4, /* synthetic Whisper encoder output [n_cross, d] */
  XE_T_LN1_W = 8,   /* self-attn pre-norm */
  XE_T_LN1_B = 9,
  XE_T_Q_W = 10,
  XE_T_Q_B = 11,
  XE_T_K_W = 12,
  XE_T_K_B = 13,
  XE_T_V_W = 14,
  XE_T_V_B = 15,
  XE_T_O_W = 16,
  XE_T_O_B = 17,
  XE_T_LN2_W = 18,  /* FFN pre-norm (Gemma pre_feedforward_layernorm) */
  XE_T_LN2_B = 19,
  XE_T_FC1_W = 20,  /* fc1 / Gemma gate_proj */
  XE_T_FC1_B = 21,
  XE_T_UP_W = 22,   /* Gemma up_proj */
  XE_T_FC2_W = 23,  /* fc2 / Gemma down_proj */
  XE_T_FC2_B = 24,
  XE_T_QNORM_W = 25,
  XE_T_KNORM_W = 26,
  XE_T_POST_ATTN_W = 27,
  XE_T_POST_FFN_W = 28,
  XE_T_LNX_W = 29,  /* Whisper cross-attn pre-norm */
  XE_T_LNX_B = 30,
  XE_T_XQ_W = 31,
  XE_T_XQ_B = 32,
  XE_T_XK_W = 33,
  XE_T_XV_W = 34,
  XE_T_XV_B = 35,
  XE_T_XO_W = 36,
  XE_T_XO_B = 37,
  XE_T_COUNT = 38
};

/* Synthetic-weight stream id of a tensor (the counter-based generator keys
 * every element by (seed, id, index)). */
#define XE_SYNTH_ID(kind, layer) \
  ((uint32_t)((layer) < 0 ? (kind) : 64 * ((layer) + 1) + (kind)))

/* Create a decoder (weights uninitialised).  max_batch streams. */
xe_decoder *xe_decoder_create(xe_device *dev, const xe_model_config *cfg,
                              int max_batch);
void xe_decoder_destroy(xe_decoder *dec);
/* Fill every weight with the seeded synthetic generator, on the device. */
int xe_decoder_init_synthetic(xe_decoder *dec, uint64_t seed);
/* Upload one fp32 tensor ([out,in] for matrices); quantised like
 * xe_register_weight.  Returns 0 or -1 (unknown kind / wrong size). */
int xe_decoder_set_tensor(xe_decoder *dec, int kind, int layer,
                          const float *data, size_t count);
/* Shape [rows, cols] of tensor (kind, layer) of a model ([out, in] for
 * matrices; vectors are 1 x n); -1 when the family has no such tensor.
 * Host only (the tensor table of npu-weights/src/spec.rs, per family). */
int xe_model_tensor_shape(const xe_model_config *cfg, int kind, int layer,
                          int *rows, int *cols);
/* The decoder's model configuration. */
int xe_decoder_config(xe_decoder *dec, xe_model_config *out);
/* Load a decoder's weights from a safetensors file (the reference's weight
 * arena loader, npu-weights/src/arena.rs:14-99, and its Hugging Face
 * sources): either a baked OPT arena (metadata arch "opt", format_version
 * 1; names and [in, out] linears of arch/opt.rs:1-20) or a Hugging Face
 * checkpoint of the model family (OPTForCausalLM, the Whisper decoder,
 * Gemma3ForCausalLM names; [out, in] linears).  F32 / BF16 / F16 tensors;
 * each is quantised like xe_decoder_set_tensor.  Tensors the model does not
 * use (encoder weights, a tied lm_head) are skipped; a tied lm_head /
 * proj_out stands in for a missing token embedding.  Every tensor the model
 * needs must be present.  Returns the number of tensors loaded, or -1. */
int xe_decoder_load_safetensors(xe_decoder *dec, const char *path);
/* Host-only dry run of the loader for a config: the number of tensors that
 * map, and (report, may be NULL) one line per tensor "name -> kind layer
 * [T]" or "name -> skipped" after a first line "arena" / "hf".  -1 (with
 * the loader's message) when the file would not load. */
int xe_safetensors_plan(const char *path, const xe_model_config *cfg,
                        char *report, int cap);
/* Read back a quantised int8 tensor (q [rows*cols], scales [rows]). */
int xe_decoder_get_tensor_q8(xe_decoder *dec, int kind, int layer, int8_t *q,
                             float *scales);
/* reset() (whisper_decoder.rs:1235-1243): clear every stream's KV cache. */
int xe_decoder_reset(xe_decoder *dec);
/* Fill positions [0, n_pos) of one stream's self-attention K / V cache
 * (every layer and KV head) with the counter-based synthetic stream, bf16
 * N(0, 1): element (pos, e) of (layer l, head h) is value pos * head_dim + e
 * of stream id 2 (l n_kv_heads + h) (K) or that + 1 (V) under `seed`, and
 * the stream's next position becomes n_pos.  A decode can then start at a
 * long context without feeding a prompt of that length (parity tests and
 * benchmarks at the contexts of BASELINE config 5).  No counterpart in the
 * reference, whose decoders always start from an empty cache (reset(),
 * whisper_decoder.rs:1235-1243); the oracle's xo_model_prime_kv fills the
 * same values. */
int xe_decoder_prime_kv(xe_decoder *dec, int stream, int n_pos, uint64_t seed);
/* precompute_cross (whisper_decoder.rs:1143-1232): enc [n_cross, d] fp32, or
 * NULL to use the synthetic XE_T_ENC_OUT tensor of the last init. */
int xe_decoder_set_cross(xe_decoder *dec, const float *enc);
/* Per-utterance int8 cross K and/or V (the fused decode ELF's int8_cross_k /
 * int8_cross_v, whisper_decoder.rs:951-960, quantised as :1186-1219 and
 * applied as route_b_kernels/decode_fused/gen_decode.py:263-282): channel
 * scale s = max_t|x| / 127, q = round(x / s); scores use q * s_k, the
 * attention output is scaled by s_v.  Half the cross-attention bytes per
 * token.  Takes effect at the next xe_decoder_set_cross (call it again
 * after switching).  With K and V both int8 the low-latency executor reads
 * the int8 rows inside its step; K or V alone steps on the phase kernels
 * (graph executor). */
int xe_decoder_set_cross_int8(xe_decoder *dec, int k_int8, int v_int8);
/* step(tok, pos) -> logits (whisper_decoder.rs:1293-1349) for `batch`
 * streams with per-stream positions.  logits [batch, vocab] may be NULL;
 * next [batch] receives the greedy token (argmax with the family's tie
 * rule: OPT last max, Whisper/Gemma first max) and may be NULL. */
int xe_decoder_step(xe_decoder *dec, const int32_t *tokens,
                    const int32_t *pos, int batch, float *logits,
                    int32_t *next);
/* Greedy generation (Opt::generate, opt125m_decode.rs:296-315): feed
 * prompt [batch, n_prompt] from position 0, then emit n_new tokens per
 * stream into out [batch, n_new].  The token loop runs in a HIP graph. */
int xe_decoder_generate(xe_decoder *dec, const int32_t *prompt, int n_prompt,
                        int batch, int n_new, int32_t *out);
/* Split form of generate: feed() resets positions to 0 and runs the prompt
 * (the last prompt step emits the first new token); decode() runs n_steps
 * more greedy steps from the device state, returning the tokens they emit
 * (out [batch, n_steps], may be NULL) and the device time of the whole run
 * measured with HIP events on the decoder stream (device_us, may be NULL). */
int xe_decoder_feed(xe_decoder *dec, const int32_t *prompt, int n_prompt, int batch);
/* decode() returns the number of steps that ran (n_steps unless a stop
 * token ended the run early, below), or -1. */
int xe_decoder_decode(xe_decoder *dec, int batch, int n_steps, int32_t *out,
                      double *device_us);
/* Stop rule of the reference's greedy loops (EOT, whisper.rs:371-380 and,
 * batched, :618-668): from the next feed() on, a stream whose generated
 * token is stop_id has stopped; it is fed stop_id at its following positions
 * (its KV cache advances, its output is ignored) and, in out rows of
 * decode() / generate(), every token after its stop is stop_id.  A
 * low-latency launch ends at the step where every stream has stopped; the
 * phase-kernel executors launch no further steps after the next check
 * (every 8 steps).  Prompt tokens never stop a stream; the argmax after the
 * last prompt token can.  stop_id -1 (the default) removes the rule
 * (Opt::generate, opt125m_decode.rs:296-315, has none). */
int xe_decoder_set_stop(xe_decoder *dec, int32_t stop_id);
/* greedy_decode_fused[_batch] (whisper.rs:344-389, 618-668): feed prompt
 * [batch, n_prompt], then generate until every stream has emitted stop_id or
 * max_new tokens (MAX_DECODE, whisper.rs:36).  out [batch, max_new] holds
 * each stream's tokens, the stop token excluded, then stop_id; n_out [batch]
 * (may be NULL) the number of tokens before the stop.  The decoder's own
 * stop setting is restored afterwards. */
int xe_decoder_generate_until(xe_decoder *dec, const int32_t *prompt, int n_prompt,
                              int batch, int max_new, int32_t stop_id,
                              int32_t *out, int32_t *n_out);
/* One eager decode step with a HIP event after every launch (the step
 * advances the streams like decode).  Per launch: a label (32-byte slots in
 * labels), device microseconds and algorithmic bytes.  Returns the number of
 * launches recorded (<= max_entries) or -1.  Phase-timing aid, the
 * counterpart of FUSED_PHASE_TIMING (whisper_decoder.rs:741-779). */
int xe_decoder_profile_step(xe_decoder *dec, int batch, int max_entries, char *labels,
                            double *us, double *bytes);
/* Executor a decode step of `batch` streams runs on.  XE_EXEC_LL is the
 * default wherever its plan supports the model and batch: one cooperative
 * launch per token run, workgroups exchanging activations through HBM.  The
 * others launch one kernel per phase: replayed from a HIP graph (the
 * default beyond the low-latency plan, or XE_STEP=graph) or launched eagerly
 * (XE_STEP=eager).  Value 1 is retired (a persistent phase kernel with grid
 * barriers, removed: it was slower than both).  No counterpart in the
 * reference (its executors are fixed per backend); returns -1 on error. */
enum { XE_EXEC_GRAPH = 0, XE_EXEC_EAGER = 2, XE_EXEC_LL = 3 };
int xe_decoder_executor(xe_decoder *dec, int batch);
/* Resident decode step (ElfResident, npu-xrt/src/lib.rs:591-629 and
 * xrt_shim.h:95-111: a constant program bound once, per-token parameters
 * written to a host-mapped scratchpad, then dispatched).  open() builds the
 * decoder's step for `batch` streams once (its HIP graph, or the low-latency
 * kernel's plan); write() puts tokens [batch] and positions [batch] into
 * pinned host memory (no device work); dispatch() copies them to the
 * device, runs the step and waits; dispatch_start() returns a run handle
 * instead (xe_run_wait / xe_run_query; write() and read() refuse while it
 * is in flight); read() gives the last completed dispatch's greedy tokens
 * [batch] and/or logits [batch, vocab] (either may be NULL).  The step is
 * the one xe_decoder_step runs; the streams' cache positions advance alike.
 * Close the resident step before the decoder. */
typedef struct xe_resident xe_resident;
xe_resident *xe_resident_open(xe_decoder *dec, int batch);
void xe_resident_close(xe_resident *res);
int xe_resident_write(xe_resident *res, const int32_t *tokens,
                      const int32_t *pos);
int xe_resident_dispatch(xe_resident *res);
xe_run *xe_resident_dispatch_start(xe_resident *res);
int xe_resident_read(xe_resident *res, int32_t *next, float *logits);
/* Mean device time (microseconds) of the last generate's decode steps. */
double xe_decoder_last_step_us(xe_decoder *dec);
/* Bytes of weights one decode step streams (int8/bf16/bfp16 + scales). */
uint64_t xe_decoder_weight_bytes(xe_decoder *dec);

#ifdef __cplusplus
}
#endif
#endif
