/*
 * stories_hip.h — C ABI of libstories_hip.so, the MI355X (gfx950) token loop for
 * Stories110M- and Qwen3-shaped Llama models.
 *
 * This is the drop-in boundary. Each entry point names the reference interface it replaces
 * (paths relative to the reference tree). The conventions follow the reference's own C ABI,
 * bridge/ane_bridge.h: opaque handle types (:17-18), int status 0 on success / negative on
 * failure (:27), NULL from constructors on failure (:38-42), caller-owned input and output
 * buffers, and the error text of the calling thread's last failure via sh_last_error
 * (stories_trainer_bridge.h:36). Plain pointers and sizes only; no C++ or torch types.
 *
 * Threading: a model handle is single-threaded, like stories.Decoder (infer.go:30-59); two
 * threads must not call into one handle at the same time. Distinct handles are independent.
 * Host pointers are read or written only during the call (cgo pointer rules).
 */
#ifndef STORIES_HIP_H
#define STORIES_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sh_model sh_model;

/* Weight storage types. Host weights are always fp32; upload rounds them on the device. */
enum {
    SH_DTYPE_F16 = 1,   /* fp16 weights (round to nearest even), fp32 activations */
    SH_DTYPE_BF16 = 2,  /* bf16 weights (round to nearest even), fp32 activations */
    SH_DTYPE_W8A8 = 3   /* int8 weights per output row + int8 per-tensor activations */
};

/* KV-cache storage types. */
enum { SH_KV_F32 = 0, SH_KV_F16 = 1, SH_KV_BF16 = 2 };

/* Model shape and numerics. Replaces the compile-time constants of ane/stories/config.go:3-18
 * (and training/training_dynamic/models/qwen3_06b.h:6-16) with a runtime description. */
typedef struct sh_config {
    int32_t dim;          /* D: residual width (config.go:4 Dim) */
    int32_t hidden;       /* F: SwiGLU width (config.go:5 Hidden) */
    int32_t n_layers;     /* config.go:8 NLayers */
    int32_t n_heads;      /* query heads (config.go:6 Heads) */
    int32_t n_kv_heads;   /* key/value heads; q head h reads kv head h / (H/KVH) */
    int32_t head_dim;     /* hd; Stories D/H = 64 */
    int32_t vocab;        /* config.go:9 Vocab */
    int32_t max_seq;      /* KV-cache positions (infer.go:84-89 clamps Stories to 256) */
    double rope_theta;    /* infer.go:102 (10000) */
    double norm_eps;      /* infer.go:307 (1e-5) */
    double qk_norm_eps;   /* per-head Q/K RMSNorm eps, when qk_norm != 0 */
    float residual_scale; /* alpha in x + alpha*branch: 1 (infer.go:227,238) or
                             1/sqrt(2L) (ane/storiesane/residual.go:9) */
    int32_t qk_norm;      /* 1: RMSNorm every q and k head before RoPE */
    int32_t tied_embed;   /* 1: classifier rows are the embedding (weights.go:22) */
    int32_t kv_dtype;     /* SH_KV_* */
    int32_t max_batch;    /* sequences for the batched entry points (>= 1) */
} sh_config;

/* Timing of the last decode / prefill call, from HIP events on the library's stream. */
typedef struct sh_timing {
    double gpu_ms;          /* device time of the last call's timed region */
    int64_t forwards;       /* token forwards (one per position) in that region */
    int64_t tokens_out;     /* tokens produced (greedy) in that region */
    double bytes_per_forward_mean; /* algorithmic bytes per forward, averaged */
    int32_t persistent;     /* 1: the persistent decode kernel ran; 0: per-stage kernels */
    int32_t grid;           /* workgroups of the persistent kernel */
    double prefill_ms;      /* device time of the prompt's full-sequence forward: part of
                               gpu_ms for sh_greedy_decode (every dtype) and
                               sh_prefill_logits, apart from it for sh_batch_greedy_decode
                               (whose gpu_ms is the decode steps); 0 if none */
} sh_timing;

/* ---- library ------------------------------------------------------------------------ */
/* bridge/ane_bridge.h:27 ane_bridge_init: 0 on success, -1 on failure. Selects the device
 * this thread's subsequent sh_model_create calls use. */
int sh_init(int32_t device);
/* stories_trainer_bridge.h:36: copies this thread's last error text into buf (NUL-ended,
 * truncated to len) and returns the full length. */
size_t sh_last_error(char *buf, size_t len);
/* Default shapes: ane/stories/config.go:3-10 (Stories110M, alpha 1, fp32 KV) and
 * training/training_dynamic/models/qwen3_06b.h:6-16 (theta 1e6, QK-norm, tied, bf16 KV). */
int sh_config_stories110m(sh_config *cfg);
int sh_config_qwen3_06b(sh_config *cfg);

/* ---- model -------------------------------------------------------------------------- */
/* stories.NewDecoder (ane/stories/infer.go:80-133) / storiesane.Open (engine.go:149):
 * allocates device weights, KV cache and RoPE tables. NULL on failure. */
sh_model *sh_model_create(const sh_config *cfg, int32_t dtype);
/* Uploads one layer of stories.LayerWeights (ane/stories/weights.go:13-17), fp32 row-major
 * [out, in]: wq [H*hd, D], wk/wv [KVH*hd, D], wo [D, H*hd], w1/w3 [F, D], w2 [D, F],
 * rms_att/rms_ffn [D], q_norm/k_norm [hd] (NULL unless cfg.qk_norm). */
int sh_model_upload_layer(sh_model *m, int32_t layer, const float *wq, const float *wk,
                          const float *wv, const float *wo, const float *w1, const float *w2,
                          const float *w3, const float *rms_att, const float *rms_ffn,
                          const float *q_norm, const float *k_norm);
/* ModelWeights.Embed [V, D] and RMSFinal [D] (weights.go:19-24); cls [V, D] or NULL when
 * cfg.tied_embed (the Embed rows are the classifier, infer.go:243). */
int sh_model_upload_globals(sh_model *m, const float *embed, const float *rms_final,
                            const float *cls);
/* A tensor as the device stores it, for checking the upload's conversion (the reference
 * converts weights to fp16 blobs on the host, ane/mil/generator.go:151-219; here the device
 * rounds): layer >= 0 with name wq wk wv wo w1 w2 w3, or layer -1 with "embed" (the 16-bit
 * lookup table) or "cls" (classifier rows when untied or W8A8). dst receives the raw rows:
 * fp16 / bf16 bits (2 bytes each) or int8 (W8A8); "<name>.scale" gives a W8A8 tensor's fp32
 * row scales. bytes must equal the tensor's size. No reference counterpart. */
int sh_model_read_weights(const sh_model *m, int32_t layer, const char *name, void *dst, size_t bytes);
/* (*Decoder).ResetCache (infer.go:61-70). */
int sh_reset_cache(sh_model *m);
/* (*Decoder).EvalNextLogits (infer.go:72-77) = forwardOne (infer.go:204-245): one token
 * at one position through the KV cache. logits (V floats) may be NULL; argmax_out (first
 * maximum, infer.go:373-383) may be NULL. */
int sh_decode_step(sh_model *m, int32_t token, int32_t pos, float *logits,
                   int32_t *argmax_out);
/* (*Decoder).Decode with Temperature 0 (infer.go:136-202): clears the cache, feeds the
 * prompt (last max_seq ids; [BOS] if empty), generates up to max_new tokens (64 if <= 0),
 * stops after EOS=2 or at max_seq tokens. out_tokens (capacity max_seq) receives prompt +
 * generated ids, *n_out their count, *stopped_eos whether EOS ended the loop. The whole
 * loop runs on the device; the host sees only the final ids. The prompt's first n-1 positions
 * run as one full-sequence forward that fills the cache as the token-by-token feed would (for
 * W8A8 bit for bit, on its int8 matrix-core form); sh_stats then counts only the forwards after
 * it, and reports that forward's device time as prefill_ms. */
int sh_greedy_decode(sh_model *m, const int32_t *prompt, int32_t n_prompt, int32_t max_new,
                     int32_t *out_tokens, int32_t *n_out, int32_t *stopped_eos);
/* (*Engine).EvalLogits (ane/storiesane/engine.go:363-376) = evalLogitsCPUInto
 * (engine.go:804-842): the full causal forward of `seq` tokens (seq <= max_seq), logits
 * channel-first [V, seq] (logits[v*seq + t]). Out-of-range ids give a zero embedding
 * column (cpu.go:41-72). Residual scale = cfg.residual_scale. An fp16 model's matrix
 * products take the activations as one fp16 plane (the logits agree with the fp32 path to
 * about 1e-3); bf16 models carry them as a hi/lo pair. A W8A8 model runs it on the int8
 * matrix cores with each token's activations quantized on their own and the decode's float
 * order wherever a value feeds a quantizer, so its logits equal forwardOne's at every
 * position. */
int sh_prefill_logits(sh_model *m, const uint16_t *tokens, int32_t seq, float *logits_cf);
/* ---- storiesane plugin seams over channel-first data (the _other.go stubs' HIP side) ---- */
/* compileStoriesLayerForwardFunc + (*layerForward).run (ane/storiesane/layer_other.go:27-37,
 * called per layer from engine.go:784): one transformer layer of the uploaded model over
 * x_cf [dim, seq] (x_cf[d*seq + t]) at positions 0..seq-1, result out_cf [dim, seq]; the
 * numerics of evalLogitsCPUInto's layer body (engine.go:815-838: rmsNormCF, q/k/v, RoPE,
 * causal attention, Wo, x2 = x + a*o, rmsNormCF, W1/W3, SiLU gate, W2, x = x2 + a*ff with
 * a = cfg.residual_scale). The KV cache is not touched. out_cf may equal x_cf. Needs the
 * model's layers uploaded, not its globals: a model with n_layers = 1 holding one layer is
 * the counterpart of one compiled layerForward. */
int sh_layer_forward_cf(sh_model *m, int32_t layer, const float *x_cf, int32_t seq,
                        float *out_cf);
/* sh_layer_forward_cf plus the layer's intermediates, as the reference's fused ANE layer
 * programs return them (GenStoriesSDPAForwardDynamicTaps, ane/mil/stories_dynamic.go:71-165,
 * output concat at :162; GenStoriesFFNForwardDynamicTaps, :176-225, concat at :222), all
 * channel-first [rows, seq] fp32:
 *   sdpa_cf [dim + 2*H*hd + 2*KVH*hd, seq] = x2 (x + a*Wo.att), q after QK-norm and RoPE,
 *           k after QK-norm and RoPE, v, att (the attention output Wo consumes);
 *   ffn_cf  [dim + 2*hidden, seq] = x_next (= out_cf), h1 = W1.n, h3 = W3.n with n the
 *           RMSNorm of x2.
 * Either may be NULL. The layer's own output is the same as sh_layer_forward_cf's. */
int sh_layer_forward_cf_taps(sh_model *m, int32_t layer, const float *x_cf, int32_t seq,
                             float *out_cf, float *sdpa_cf, float *ffn_cf);
/* offload.runRMSForward (offload_other.go:22-24; offload_darwin.go:345-356): the final
 * RMSNorm with the model's rms_final over x_cf [dim, seq] (stories.RMSNorm numerics,
 * cpu.go:97-111) into out_cf [dim, seq]. out_cf may equal x_cf. */
int sh_rms_final_cf(sh_model *m, const float *x_cf, int32_t seq, float *out_cf);
/* offload.runClassifierForward (offload_other.go:25-27; offload_darwin.go:358-):
 * logits_cf [vocab, seq] = classifier [vocab, dim] . xnorm_cf [dim, seq] (MatMulVocabSeq's
 * product, cpu.go:276-300) with the model's classifier rows. */
int sh_classifier_cf(sh_model *m, const float *xnorm_cf, int32_t seq, float *logits_cf);
/* matMulVocabSeqAccelerate (ane/stories/gemm_stub.go:5-7, called by MatMulVocabSeq at
 * cpu.go:276-278; "true = handled" there, 0 here): logits [vocab, seq] = embed [vocab, dim] .
 * x [dim, seq], channel-first, from host fp32 arrays. No model is needed: embed is rounded to
 * fp16 on the device for each call (x keeps ~22 significant bits as hi/lo operand planes).
 * Needs dim % 32 == 0 and vocab % 64 == 0; otherwise -1 and the caller keeps its CPU loop. */
int sh_matmul_vocab_seq(const float *embed, const float *x_cf, int32_t vocab, int32_t dim,
                        int32_t seq, float *logits_cf);
/* forward.ConvEval (ane/forward/conv.go:11-52) over a compiled 1x1-conv kernel
 * (model.Kernel, ane/model/model_other.go:41-93): sh_conv_create uploads w [out_dim, in_dim]
 * (rounded to fp16) and returns NULL on failure; sh_conv_eval takes x row-major [s, in_dim]
 * and writes out row-major [s, out_dim], out[t*out_dim + o] = sum_i w[o, i] x[t*in_dim + i]
 * (ConvEval's channel-first transposes are folded into the product). Needs in_dim % 32 == 0
 * and out_dim % 64 == 0. sh_conv_destroy accepts NULL. */
typedef struct sh_conv sh_conv;
sh_conv *sh_conv_create(const float *w, int32_t out_dim, int32_t in_dim);
int sh_conv_eval(sh_conv *c, const float *x, int32_t s, float *out);
void sh_conv_destroy(sh_conv *c);
/* sh_conv_eval without any allocation, for callers that cannot allocate device memory: code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc. No
 * reference counterpart (ConvEval allocates its IOSurfaces per kernel). x [s, in_dim] and out
 * [s, out_dim] are device pointers the caller owns; the work is enqueued on `stream` (a
 * hipStream_t; NULL = the null stream) and the call returns without waiting. The input's
 * operand planes and the product's K-range partials live in a static 16 MiB device array
 * per GPU (resolved at sh_init); a call needing more (4*s*in_dim bytes of planes plus the
 * partials of the split product) fails with a message saying how much. Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (two streams, two threads) race, so
 * a caller must order them. Results equal sh_conv_eval's bit for bit. */
int sh_conv_eval_noalloc(sh_conv *c, const float *x, int32_t s, float *out, void *stream);
/* (*Engine).Decode with Temperature 0 (ane/storiesane/decode.go:18-94): every step runs the
 * full causal forward (as sh_prefill_logits) over the last `seq` tokens left-padded with BOS
 * (fillDecodeWindow, :83-94) and appends the argmax of the last position's logits. The prompt
 * is [BOS] if empty and its last `seq` ids are kept; max_new <= 0 means 64; stops after EOS=2
 * (there is no max_seq stop: the window slides). seq <= cfg.max_seq.
 * out_tokens (capacity min(n_prompt, seq) + max_new, or 1 + max_new for an empty prompt)
 * receives prompt + generated ids. The loop runs on the device. */
int sh_window_greedy_decode(sh_model *m, const int32_t *prompt, int32_t n_prompt, int32_t seq,
                            int32_t max_new, int32_t *out_tokens, int32_t *n_out,
                            int32_t *stopped_eos);
/* Batched greedy decode: n_seqs independent (*Decoder).Decode runs with Temperature 0
 * (infer.go:136-202 each), stepped together on the device. No single reference entry point
 * does this; it is n_seqs decoders sharing one weight stream per step. prompts: n_seqs rows of
 * prompt_len ids (1 <= prompt_len <= max_seq, ids in [0, vocab)); max_new <= 0 means 64. The
 * first prompt_len - 1 ids of every row go through one causal forward that fills the KV
 * caches; then each step feeds every sequence's latest token, so step i yields token
 * prompt_len + i of every row. A row stops after EOS=2 or at max_seq tokens. out_tokens holds
 * n_seqs rows of stride prompt_len + (max_new > 0 ? max_new : 64); n_out[s] is row s's count.
 * Needs n_seqs <= min(32, cfg.max_batch) (W8A8: dim, n_heads*head_dim and hidden multiples
 * of 128, as for its full-sequence forward). sh_stats then reports the
 * decode steps (forwards = steps, tokens_out = tokens kept) and the prefill time. */
int sh_batch_greedy_decode(sh_model *m, const int32_t *prompts, int32_t n_seqs,
                           int32_t prompt_len, int32_t max_new, int32_t *out_tokens,
                           int32_t *n_out);
/* sh_batch_greedy_decode that also returns the logits of sequences rows[0, n_rows) at every
 * step: logits_out[(i * n_rows + k) * vocab + v] for step i (the forward at position
 * prompt_len - 1 + i, whose argmax is token prompt_len + i), for every step the call runs
 * (min(max_new, max_seq - prompt_len)). The counterpart of reading EvalNextLogits
 * (infer.go:72-77) at each step of those sequences' decodes; an inspection and testing aid
 * (the steps run as eager launches rather than the captured step graph, so sh_stats' times
 * are not the batched decode's). */
int sh_batch_greedy_decode_logits(sh_model *m, const int32_t *prompts, int32_t n_seqs,
                                  int32_t prompt_len, int32_t max_new, int32_t *out_tokens,
                                  int32_t *n_out, const int32_t *rows, int32_t n_rows,
                                  float *logits_out);
/* Human-readable description of the decode path this model runs (persistent kernel or
 * per-stage kernels) and why; returns the full length. No reference counterpart: the
 * reference reports its ANE/CPU choice through Diagnostics (ane/storiesane/diagnostics.go). */
size_t sh_model_describe(const sh_model *m, char *buf, size_t len);
/* Testing aids (no reference counterpart): sh_debug_option(m, option, value), 0 or -1.
 * SH_DEBUG_FAIL_NEXT_LAUNCH exercises the persistent decode kernel's failure handling, whose
 * contract is the reference's fallback on an accelerator failure (ane/storiesane/engine.go:
 * 739-746): the next persistent launch ends at once in every workgroup, as if value 2: a
 * bounded wait expired before the whole grid was resident (the model then switches to the
 * per-stage graph path for good and the call is repeated there; W8A8, which has no such path,
 * returns -1), or value 1: a wait expired with every workgroup running (the call returns -1 and
 * the model keeps its path); 0 disarms; -1 when the model does not run the persistent kernel.
 * SH_DEBUG_PROMPT_PREFILL 0: sh_greedy_decode feeds the prompt through the token loop (one
 * forward per position, as infer.go:175-177 does) instead of one full-sequence forward; 1
 * restores the default. */
enum { SH_DEBUG_FAIL_NEXT_LAUNCH = 1, SH_DEBUG_PROMPT_PREFILL = 2 };
int sh_debug_option(sh_model *m, int32_t option, int32_t value);
/* Stage trace of the persistent decode kernel (a tracing aid like the reference's per-step
 * metrics, ane/storiesane/metrics.go:13-60): arm with the index of a forward within the next
 * decode launch (-1 disarms); after it, sh_trace_read returns grid x 2 x (5*n_layers + 3)
 * constant-clock timestamps, one row pair per workgroup (grid = sh_timing.grid). The first
 * row: forward start, then after each layer's qkv, attention, wo, w13 and w2 stages, after the
 * classifier, after the argmax (a workgroup that owns no rows in a stage stamps it as soon as
 * it skips it). The second row, same columns: when the workgroup had that stage's whole input
 * (0 where it waited for none).
 * -1 when the model does not run the persistent kernel. */
int sh_trace_forward(sh_model *m, int32_t forward);
int sh_trace_read(sh_model *m, int64_t *out, int32_t cap, int32_t *n_out, double *ticks_per_s);
/* Intermediate vectors of the last layer of the last token forward (the counterpart of the
 * reference engine's cache taps, ane/storiesane/engine_test.go:154-239, which compare the
 * engine's x2/q/k/v/att outputs with the CPU functions). which: SH_TAP_X the layer output
 * (D), SH_TAP_QKV the q|k|v projection before QK-norm and RoPE (H*hd + 2*KVH*hd),
 * SH_TAP_ATT attention output (H*hd), SH_TAP_GATE silu(W1 x) * W3 x (F), SH_TAP_X2 the
 * residual after attention (D). n must equal that length. */
enum { SH_TAP_X = 0, SH_TAP_QKV = 1, SH_TAP_ATT = 4, SH_TAP_GATE = 5, SH_TAP_X2 = 6 };
int sh_decode_tap(const sh_model *m, int32_t which, float *out, int32_t n);
/* Timing of the last sh_greedy_decode / sh_decode_step / sh_prefill_logits / batched or
 * window decode / channel-first seam call. */
int sh_stats(const sh_model *m, sh_timing *out);
/* (*Engine).Close (engine.go:480): frees device memory. NULL is allowed. */
void sh_model_destroy(sh_model *m);

/* ---- training: ane/storiesane Engine.Step (engine.go:295-361, train_full.go) ------------ */
/* Options (storiesane.Options, engine.go:15-32); zero / negative fields take Open's defaults
 * (engine.go:153-186): seq 256, lr 3e-4, beta1 0.9, beta2 0.999, eps 1e-8, loss_scale 256,
 * seed 42, accum_steps 1; grad_clip 0 = off; weight_decay 0. accum_steps > 1 accumulates the
 * gradients of that many windows and applies Adam to their mean (backwardAndAccumulate,
 * train_full.go:709-774; flushPending, engine.go:540-565). */
typedef struct sh_train_options {
    int32_t seq;
    float lr, beta1, beta2, eps, weight_decay, grad_clip, loss_scale;
    int64_t seed;
    int32_t accum_steps;
} sh_train_options;
/* storiesane.State (engine.go:35-44) without the wall-clock totals, plus the last step's
 * device time. */
typedef struct sh_train_state {
    uint64_t token_pos;
    float last_loss;
    uint32_t cum_steps, adam_t;
    double last_step_ms;
    uint32_t cum_batches, pending_steps;
} sh_train_state;
typedef struct sh_trainer sh_trainer;
enum { SH_TRAIN_PARAMS = 0, SH_TRAIN_GRADS = 1, SH_TRAIN_ADAM_M = 2, SH_TRAIN_ADAM_V = 3 };
/* Open (engine.go:149-270) for a Stories-shaped model (MHA, no QK-norm, tied classifier):
 * fp32 weights, gradients and Adam moments on the device; residual branches scaled by
 * cfg->residual_scale (layerResidualScale, residual.go:9, for the reference's engine). NULL
 * on failure. Weights are uploaded with the two calls below (fp32, reference layouts). */
sh_trainer *sh_trainer_create(const sh_config *cfg, const sh_train_options *opt);
int sh_trainer_upload_layer(sh_trainer *t, int32_t layer, const float *wq, const float *wk,
                            const float *wv, const float *wo, const float *w1, const float *w2,
                            const float *w3, const float *rms_att, const float *rms_ffn);
int sh_trainer_upload_globals(sh_trainer *t, const float *embed, const float *rms_final);
/* Options.Tokens: the training stream (copied). */
int sh_trainer_set_tokens(sh_trainer *t, const uint16_t *tokens, int64_t n);
/* (*Engine).Step (engine.go:295-361): picks the window with drand48 (engine.go:307-316,
 * :725-732), runs forwardTraining, runFinalHead and backwardAndUpdate on the device (the
 * reference's CPU-path numerics) and returns the loss. "not enough tokens" when the stream is
 * shorter than seq + 1. */
int sh_trainer_step(sh_trainer *t, float *loss);
/* The same step on a given (input, target) window of seq ids, without the window choice. */
int sh_trainer_step_window(sh_trainer *t, const uint16_t *input, const uint16_t *target,
                           float *loss);
/* (*Engine).Flush (engine.go:398-410): applies the pending accumulated gradients, if any
 * (scaled by 1/pending, loss scale undone, clipped, Adam). */
int sh_trainer_flush(sh_trainer *t);
/* Copies one tensor of a set (SH_TRAIN_PARAMS / GRADS / ADAM_M / ADAM_V) to dst. GRADS holds
 * the gradients Adam last applied, or, while accumulated windows are pending, their sum (still
 * multiplied by the loss scale). name is "embed", "rms_final" or "layers.<l>.<key>"
 * with key wq wk wv wo w1 w2 w3 rms_att rms_ffn; n must be its element count. No reference
 * counterpart (the engine's weights are Go slices the caller reads directly). */
int sh_trainer_read(const sh_trainer *t, int32_t which, const char *name, float *dst, size_t n);
int sh_trainer_state(const sh_trainer *t, sh_train_state *out);
/* (*Engine).Close (engine.go:480). NULL is allowed. */
void sh_trainer_destroy(sh_trainer *t);

/* ---- W8A8 quantizer (bridge/ane_bridge.m:374-399), run on the device --------------- */
/* per_row == 0: one scale for the whole tensor, exactly the bridge formula
 * (scale = max|x|/127, 0 -> 1; q = (int8)(clamp(x/scale, -128, 127) +- 0.5)).
 * per_row != 0: the same formula applied to each row on its own; scales has `rows`
 * entries. Bit-exact with the bridge's C code. */
int sh_quantize_i8(const float *src, int32_t rows, int32_t cols, int8_t *dst, float *scales,
                   int32_t per_row);
/* dst[r, c] = (float)q[r, c] * scale(r) (constexpr_affine_dequantize with zero point 0,
 * ane_int8_bench.m:62-70). */
int sh_dequantize_i8(const int8_t *q, const float *scales, int32_t rows, int32_t cols,
                     int32_t per_row, float *dst);

/* ---- measurement --------------------------------------------------------------------- */
/* No reference counterpart. Copies `bytes` (a multiple of 16) between two fresh device
 * buffers with a plain 16-byte-per-lane copy kernel (k_copy_calibrate), `reps` times after
 * one untimed run, and reports the mean kernel time. The read + write bytes of that kernel
 * are known exactly, so profiler byte counters read over it give the scale that turns the
 * same counters over another kernel into bytes; *gbps is the measured copy bandwidth, a
 * practical HBM ceiling beside the datasheet figure. */
int sh_copy_calibrate(size_t bytes, int32_t reps, double *ms_per_copy, double *gbps);
/* No reference counterpart. The read-only companion of sh_copy_calibrate: a plain kernel
 * (k_read_calibrate) streams `bytes` (a multiple of 16) of one fresh device buffer, 16 bytes
 * per lane and four loads in flight, and writes nothing; `reps` timed runs after one untimed
 * run. *gbps is the measured read bandwidth: the practical ceiling for kernels whose HBM
 * traffic is almost all reads (the decodes' weight and KV streams). */
int sh_read_calibrate(size_t bytes, int32_t reps, double *ms_per_read, double *gbps);

/* ---- host helpers (no device work) -------------------------------------------------- */
/* Deterministic synthetic weights, replacing stories.RandomInit (weights.go:124-153) for
 * the N(0, std) configurations: element i of tensor `tensor_id` is a Box-Muller normal of
 * two splitmix64 draws keyed by (seed, tensor_id, i). Same values on every host. */
int sh_synth_normal(float *dst, size_t n, uint64_t seed, uint64_t tensor_id, float std);
/* Uniform token ids in [0, vocab) keyed by seed (prompts of the synthetic configs). */
int sh_synth_tokens(int32_t *dst, size_t n, uint64_t seed, int32_t vocab);
/* Rounds fp32 data in place to the values a dtype stores (SH_DTYPE_F16 / SH_DTYPE_BF16:
 * round to nearest even), so a CPU check can consume exactly the device's weights. */
int sh_round_dtype(float *data, size_t n, int32_t dtype);

#ifdef __cplusplus
}
#endif
#endif
