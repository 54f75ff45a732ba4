/*
 * oracle.h — CPU restatement of the reference's Stories110M / Qwen3-shaped token loop.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker or the timed CPU
 * baseline. The product (libstories_hip.so) never links, loads or calls it.
 *
 * Every function restates a reference function, cited file:line (paths relative to the
 * reference tree). Float semantics follow the reference's Go code on a non-FMA target:
 * float32 arithmetic evaluated left to right, float64 where the reference converts to
 * float64, compiled with -ffp-contract=off so no multiply-add is fused.
 */
#ifndef STORIES_ORACLE_H
#define STORIES_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Storage rounding applied to K/V when they enter the cache. */
enum { OR_KV_F32 = 0, OR_KV_F16 = 1, OR_KV_BF16 = 2 };

typedef struct or_config {
    int32_t dim, hidden, n_layers, n_heads, n_kv_heads, head_dim, vocab, max_seq;
    double rope_theta;     /* 10000 in infer.go:102 / rope.go:13 */
    double norm_eps;       /* 1e-5 in infer.go:307, accel_other.go:21, cpu.go:104 */
    double qk_norm_eps;    /* per-head Q/K RMSNorm eps (used when qk_norm != 0) */
    float residual_scale;  /* alpha: 1 for infer.go:227,238; 1/sqrt(2L) for residual.go:9 */
    int32_t qk_norm;       /* 1: RMSNorm each q/k head before RoPE */
    int32_t kv_dtype;      /* OR_KV_* */
    int32_t w8a8;          /* 1: int8 weights per output row + per-tensor int8 activations */
} or_config;

typedef struct or_layer {
    const float *wq, *wk, *wv, *wo;   /* [H*hd, D], [KVH*hd, D], [KVH*hd, D], [D, H*hd] */
    const float *w1, *w2, *w3;        /* [F, D], [D, F], [F, D] */
    const float *rms_att, *rms_ffn;   /* [D] */
    const float *q_norm, *k_norm;     /* [hd] (qk_norm only) */
} or_layer;

typedef struct or_weights {
    const or_layer *layers;   /* n_layers entries */
    const float *embed;       /* [V, D] row-major, weights.go:22 */
    const float *rms_final;   /* [D] */
    const float *cls;         /* [V, D] classifier rows; equals embed when tied */
} or_weights;

typedef struct or_decoder or_decoder;

/* ---- scalar building blocks (exported so tests can pin them one by one) ---- */
float or_half_round(float x);   /* float32 -> fp16 (round to nearest even) -> float32 */
float or_bf16_round(float x);   /* float32 -> bf16 (round to nearest even) -> float32 */
void or_rms_norm_vec(float *out, const float *x, const float *w, int n, double eps);
void or_mat_vec(float *out, const float *mat, const float *in, int rows, int cols, int threads);
float or_silu(float x);
void or_softmax_prefix(float *dst, const float *src, int n);
int32_t or_argmax(const float *v, int n);
void or_rope_tables(float *cos_out, float *sin_out, int max_seq, int head_dim, double theta);

/* ---- W8A8 quantizer (bridge/ane_bridge.m:374-399) ---- */
int8_t or_quantize_value(float v_over_scale);
float or_absmax_scale(const float *src, size_t n);
void or_quantize_tensor(const float *src, size_t n, int8_t *dst, float *scale_out);
void or_quantize_rows(const float *src, int rows, int cols, int8_t *dst, float *scales);
void or_dequantize_rows(const int8_t *q, const float *scales, int rows, int cols, float *dst);
void or_mat_vec_w8a8(float *out, const int8_t *wq, const float *wscale, const float *in,
                     int rows, int cols, int threads);

/* ---- KV-cache decoder (ane/stories/infer.go) ---- */
or_decoder *or_decoder_new(const or_config *cfg, const or_weights *w, int threads);
void or_decoder_free(or_decoder *d);
void or_decoder_reset(or_decoder *d);
/* forwardOne (infer.go:204-245). logits_out may be NULL. Returns 0 or -1. */
int or_forward_one(or_decoder *d, int token, int pos, float *logits_out);
/* Prompt ids tokens[0, n) at positions pos0.. in one layer-major pass; the K/V cache and the
 * last token's logits (logits_out, may be NULL) equal n calls of or_forward_one bit for bit.
 * Returns 0 or -1 (ids or positions out of range). */
int or_prompt_forward(or_decoder *d, const int32_t *tokens, int n, int pos0, float *logits_out);
/* sampleFromLogits (infer.go:347-371) with the uniform draw u in [0, 1) given; *slack = the
 * draw's distance from the chosen index's CDF interval ends over the total (0 for argmax). */
int or_sample_from_logits(const float *logits, int n, float temperature, double u, double *slack);
int or_prompt_forward_logits(or_decoder *d, const int32_t *tokens, int n, int pos0, int first,
                             float *logits_out);
/* Decode with temperature 0 (infer.go:136-202). out_tokens holds prompt + generated
 * (capacity max_seq). margins (optional, capacity max_new) receives top1-top2 gaps. */
int or_greedy_decode(or_decoder *d, const int32_t *prompt, int n_prompt, int max_new,
                     int32_t *out_tokens, int32_t *n_out, int32_t *stopped_eos,
                     float *margins);
/* Debug taps of the last forward_one (last layer): 0 x (residual out), 1 q and 2 k (after
 * QK-norm and RoPE), 3 v, 4 att, 5 gate, 6 x2 (residual after attention), 7 q and 8 k as
 * projected (before QK-norm and RoPE). */
const float *or_decoder_tap(const or_decoder *d, int which);

/* ---- full-sequence channel-first forward (ane/storiesane/engine.go:804-842) ---- */
void or_embed_lookup_cf(float *out, const float *embed, int vocab, const uint16_t *tokens,
                        int dim, int seq);
void or_eval_logits_cf(const or_config *cfg, const or_weights *w, const uint16_t *tokens,
                       int seq, float *logits_cf, int threads);
/* or_eval_logits_cf with the reference's threading (linearCF and attention serial, the
 * vocabulary product over `threads`): the same values, for timing. */
void or_eval_logits_cf_ref_threads(const or_config *cfg, const or_weights *w, const uint16_t *tokens,
                                   int seq, float *logits_cf, int threads);
/* One layer of the channel-first forward (engine.go:815-838), x_cf [D,S] -> out_cf [D,S]. */
void or_layer_forward_cf(const or_config *cfg, const or_layer *L, const float *x_cf, int seq,
                         float *out_cf, int threads);
/* The same layer with its intermediates, channel-first: sdpa_taps [D + 2*H*hd + 2*KVH*hd, S] =
 * concat(x2, q_rope, k_rope, v, att) (stories_dynamic.go:162), ffn_taps [D + 2F, S] =
 * concat(x_next, h1, h3) (stories_dynamic.go:222). Either may be NULL. */
void or_layer_forward_cf_taps(const or_config *cfg, const or_layer *L, const float *x_cf, int seq,
                              float *out_cf, float *sdpa_taps, float *ffn_taps, int threads);
/* cpu.go:97-111 RMSNorm (final form) over channel-first [dim, seq]. */
void or_rms_norm_final_cf(float *out, const float *x, const float *w, int dim, int seq,
                          double eps);
/* cpu.go:276-300 MatMulVocabSeq: logits [vocab, seq] = embed [vocab, dim] . x [dim, seq]. */
void or_matmul_vocab_seq(float *logits, const float *embed, const float *x, int vocab, int dim,
                         int seq, int threads);
/* forward_common.go:35-46 linearCF: out [out_ch, seq] = W [out_ch, in_ch] . in [in_ch, seq]. */
void or_linear_cf(float *out, const float *w, const float *in, int out_ch, int in_ch, int seq,
                  int threads);
void or_fill_decode_window(uint16_t *dst, int seq, const int32_t *tokens, int n);

/* ---- training step (ane/storiesane/train_full.go CPU path; MHA Stories-shaped models) ---- */
typedef struct or_train_layer {
    float *wq, *wk, *wv, *wo, *w1, *w2, *w3, *rms_att, *rms_ffn;
} or_train_layer;
typedef struct or_train_params {
    or_train_layer *layers;   /* n_layers entries */
    float *embed;             /* [V, D], also the classifier (tied) */
    float *rms_final;         /* [D] */
} or_train_params;
typedef struct or_train_hparams {
    float lr, beta1, beta2, eps, weight_decay, grad_clip, loss_scale;
} or_train_hparams;
/* rmsnorm.go:32-47 rmsNormBackwardWithRRMS over channel-first [d, s] with the forward's
 * per-token rrms; dw accumulates. */
void or_rms_norm_backward_cf(float *dx, float *dw, const float *dy, const float *x,
                             const float *w, const float *rrms, int d, int s, int threads);
/* cpu.go:74-95 EmbedBackward: dembed [vocab, dim] += dx [dim, seq] at each in-range token row. */
void or_embed_backward(float *dembed, const float *dx, const uint16_t *tokens, int vocab,
                       int dim, int seq);
/* cpu.go:173-253 CrossEntropyLoss over logits [v, s] channel-first; dlogits may equal logits. */
float or_cross_entropy_loss(float *dlogits, const float *logits, const uint16_t *targets,
                            int v, int s);
/* One Engine.Step body without the window choice: forwardTrainingCPU, runFinalHead (CPU
 * path), backwardAndApply (CPU path, accumulation 1). p holds the fp32 weights (updated in
 * place when apply != 0), m and v the Adam moments, grads receives the gradients Adam applies
 * (after the loss-scale undo and clipping); step_t is the 1-based Adam step. Returns the loss. */
float or_train_step(const or_config *cfg, or_train_params *p, or_train_params *m,
                    or_train_params *v, or_train_params *grads, const or_train_hparams *hp,
                    int step_t, const uint16_t *input, const uint16_t *target, int seq,
                    int apply, int threads);
/* One Engine.Step body with AccumSteps > 1 before the flush (backwardAndAccumulate,
 * train_full.go:709-774, CPU path): this window's gradients (still multiplied by the loss scale)
 * are added onto accum. Returns the loss. */
float or_train_accumulate(const or_config *cfg, const or_train_params *p, or_train_params *accum,
                          const or_train_hparams *hp, const uint16_t *input,
                          const uint16_t *target, int seq, int threads);
/* flushPending (engine.go:540-565) after `pending` accumulated windows: accum scaled by
 * float32(1/pending) / loss scale, clipped, then Adam at 1-based step step_t. On return accum
 * holds the gradients Adam applied; the reference clears it next (clearModelGrad), which is
 * left to the caller. pending <= 0 does nothing. */
void or_train_flush(const or_config *cfg, or_train_params *p, or_train_params *m,
                    or_train_params *v, or_train_params *accum, const or_train_hparams *hp,
                    int step_t, int pending);
/* engine.go:725-732 and :307-316: drand48 state from a seed, its next float64, and the start
 * of the next training window. */
uint64_t or_drand48_seed(int64_t seed);
double or_drand48_next(uint64_t *state);
uint64_t or_train_window(uint64_t *state, int64_t n_tokens, int seq);

#ifdef __cplusplus
}
#endif
#endif
