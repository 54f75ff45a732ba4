// sh_internal.hpp — device-side data layout of a model and the kernel launchers shared by
// the C ABI (sh_api.hip) and the kernels (sh_kernels.hip). gfx950 only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "stories_hip.h"

namespace sh {

constexpr int kBlock = 256;          // threads per workgroup (4 wave64)
constexpr int kMaxCols = 4096;       // widest GEMV input staged in LDS
constexpr int kMaxSeqLds = 4096;     // attention scores kept in LDS
constexpr int kBos = 1;              // infer.go:10
constexpr int kEos = 2;              // infer.go:11

// Per-layer device tensors. Row-major [out, in] weights in the storage type (fp16 / bf16
// bits, or int8 with one fp32 scale per row for W8A8).
struct LayerDev {
    void *wqkv;      // [H*hd + 2*KVH*hd, D]: Wq rows, then Wk rows, then Wv rows
    void *wo;        // [D, H*hd]
    void *w13;       // [2F, D]: row 2r = W1 row r, row 2r+1 = W3 row r
    void *w2;        // [D, F]
    float *s_qkv, *s_o, *s_13, *s_2;   // W8A8 row scales (NULL otherwise)
    float *rms_att, *rms_ffn;          // [D]
    float *q_norm, *k_norm;            // [hd] (qk_norm only)
};

// Device-resident decode state (one sequence).
struct DecodeState {
    int32_t pos;        // position of the token the next forward consumes
    int32_t n_prompt;   // tokens[0, n_prompt) are prompt ids, later ones are generated
    int32_t pad[2];
};

// How a persistent decode launch ended early (its error word): a bounded wait expired with
// every workgroup started (kErrTimeout), or before every workgroup had started, i.e. the grid
// was not all resident (kErrAbsent).
constexpr int kErrTimeout = 1;
constexpr int kErrAbsent = 2;

struct ArgmaxPartial {
    float v;
    int32_t i;
};

// Rows of one GEMV stage of the persistent decode kernel: workgroup off + i (mod grid), for
// i < n, owns rows [i*per, (i+1)*per), so the hand-over words it writes are contiguous.
struct StageOwn {
    int off, n, per;
    int row0;   // first row of rank 0's block (blocks start at row0 + rank * per)
};

}  // namespace sh

struct sh_model {
    sh_config cfg;
    int32_t dtype;
    int device;
    hipStream_t stream;
    int qdim, kvdim, qkv_rows;

    void *arena;          // one allocation holding every weight tensor
    size_t arena_bytes;
    sh::LayerDev *layers; // host array of n_layers
    void *embed;          // [V, D] fp16/bf16 bits (lookup; W8A8 keeps fp16 here)
    void *cls;            // [V, D] classifier rows in the storage type (== embed when tied
                          // and not W8A8)
    float *s_cls;         // W8A8 classifier row scales
    float *rms_final;     // [D]
    int uploaded_layers;
    bool globals_uploaded;

    void *kcache, *vcache;   // [L][max_seq][KVH*hd] in kv_dtype
    size_t kv_elems;
    float *rope_cos, *rope_sin;  // [max_seq][hd/2]

    // activations (fp32)
    float *x, *x2, *qkv, *att, *gate, *logits;
    sh::ArgmaxPartial *partials;
    int n_partials;
    int32_t *tokens;       // [max_seq + 1]
    int32_t *argmax_hist;  // [max_seq + 1]: argmax produced by the forward at each position
    sh::DecodeState *state;

    hipGraphExec_t step_exec;
    bool step_ready;
    hipEvent_t ev0, ev1, ev_mid;   // ev_mid: end of a greedy decode's prompt forward
    sh_timing last;

    // persistent decode kernel (sh_persistent.hip); unused when `persistent` is false
    bool persistent;
    int p_grid;
    // GEMV stage ownership (qkv, wo, w13, w2, classifier): workgroups off .. off+n-1 (mod
    // grid) own row blocks of `per` rows in order
    sh::StageOwn p_own[5];
    int p_ostride[5];       // hand-over words between consecutive workgroups' output blocks
    // classifier split when its rows fit: the attention workgroups own p_own_cls_a (their
    // register tile), the others p_own[4] whose last p_cls_lds_rows rows stay in LDS for the
    // launch; p_own_cls_a.n == 0: p_own[4] for every workgroup
    sh::StageOwn p_own_cls_a;
    int p_cls_lds_rows;
    bool p_argmax_every;    // w13 not on every workgroup: the next-token exchange every forward
    void *p_layers;         // device array of per-layer weight pointers
    uint64_t *ll_qkv, *ll_att, *ll_x2, *ll_gate, *ll_x, *ll_pv, *ll_pi;
    int *p_err;             // device: [0] how a persistent launch ended early, [1] workgroups started
    int fail_next;          // testing aid: the next persistent launch ends at once with this code
    bool no_prompt_prefill; // testing aid: a greedy decode feeds its prompt through the token loop
    uint32_t epoch;         // next unused hand-over epoch
    long long spin_ticks;   // wait bound in constant-clock ticks
    char path_note[512];    // which decode path runs, and why
    long long *trace_buf;   // device: grid x 2 x (5L + 3) stage timestamps (ends, inputs ready)
    int trace_f;            // forward index traced in the next launch, -1 = off

    // full-sequence forward (sh_prefill.hip): token-major scratch for up to pf_cap tokens
    void *pf_arena;
    int pf_cap;
    int32_t *pf_tokens;                        // [S]
    float *pf_x, *pf_x2, *pf_qkv, *pf_logits;  // [S,D] [S,D] [S,qkv_rows] [V,S]
    int32_t *pf_rowpos, *pf_rowseq;            // [S] position and sequence of each row
    float *pf_part;                            // K-range partials of split GEMMs
    size_t pf_part_cap;                        // elements of pf_part
    float *pf_q, *pf_k, *pf_v;                 // roped q, k and v: [S,qdim] [S,kvdim] x2
    float *pf_cf;                              // [D,S] channel-first staging of the seams
    uint16_t *pf_xn, *pf_att, *pf_gate;        // GEMM operands: hi plane, then lo plane
    int8_t *pf_a8;                             // W8A8: A operand quantized per row [S, <= 4096]
    float *pf_sa;                              //       and its row scales [S]
    float *tap_buf;                            // layer taps: channel-first outputs + [S, 2F]
    size_t tap_cap;                            // elements of tap_buf

    // batched decode (sh_prefill.hip): B sequences stepped together, state on the device
    void *bt_arena;
    int bt_cap, bt_nch;
    int32_t *bt_tok, *bt_pos, *bt_seq;         // [B] next token, its position, sequence index
    int32_t *bt_hist;                          // [B][max_seq + 1] token history
    float *bt_x, *bt_x2, *bt_qkv, *bt_q, *bt_k, *bt_v, *bt_logits;
    uint16_t *bt_xn, *bt_att, *bt_gate;        // GEMM operand planes
    float *bt_pm, *bt_pl, *bt_pacc;            // attention chunk partials
    float *bt_part;                            // skinny-GEMM K-range partials
    size_t bt_part_cap;                        // elements of bt_part
    float *bt_apv;                             // argmax partials (value, index)
    int32_t *bt_api;
    int8_t *bt_a8;                             // W8A8: quantized A operand [B, <= 4096]
    float *bt_sa;                              //       and its row scales [B]
    uint64_t *bt_tm, *bt_tl, *bt_tacc;         // streaming attention: tagged split partials
    int32_t *bt_cnt;                           // [B][KVH] split-merge counters
    int32_t *bt_err;                           // set when a split partial never arrived
    uint32_t *bt_gen;                          // device copy of the call generation (tag part)
    uint32_t bt_gen_host;
    hipGraphExec_t bt_exec;                    // one captured step for bt_graph_b sequences
    bool bt_ready;
    int bt_graph_b;

    // window decode (sh_prefill.hip): the window lives in pf_tokens
    void *wd_arena;
    int wd_cap;                                // tokens wd_hist holds
    uint16_t *wd_xn;                           // last row, normalised (operand planes)
    float *wd_logits, *wd_part, *wd_apv;
    size_t wd_part_cap;
    int32_t *wd_api, *wd_hist, *wd_count;
    hipGraphExec_t wd_exec;                    // one captured step for window length wd_seq
    bool wd_ready;
    int wd_seq;
    // sh_prefill_logits: the whole forward captured for pf_graph_seq rows (its kernels point
    // into the prefill scratch, so reallocating that drops it)
    hipGraphExec_t pf_exec;
    bool pf_one_plane;  // the full-sequence products take A's hi plane only (EvalLogits, fp16)
    bool pf_ready;
    int pf_graph_seq;
};

namespace sh {

void set_error(const std::string &msg);
bool hip_ok(hipError_t e, const char *what);

// Launchers (sh_kernels.hip). All enqueue on m->stream.
// Source row r (of `cols` values) lands in destination row r * dst_row_step + dst_row_offset,
// both counted in rows of `cols` elements (a plain contiguous copy is step 1, offset 0).
hipError_t launch_convert_rows(const float *src, void *dst, int rows, int cols, int dtype,
                               int dst_row_step, int dst_row_offset, hipStream_t s);
hipError_t launch_quantize_rows(const float *src, int8_t *dst, float *scales, int rows,
                                int cols, int dst_row_stride, int dst_row_offset,
                                int scale_stride, int scale_offset, hipStream_t s);
hipError_t launch_quantize_tensor(const float *src, int8_t *dst, float *scale, size_t n,
                                  float *work, hipStream_t s);
hipError_t launch_dequantize(const int8_t *q, const float *scales, int rows, int cols,
                             int per_row, float *dst, hipStream_t s);
hipError_t launch_copy_calibrate(const void *src, void *dst, size_t bytes, hipStream_t s);
hipError_t launch_read_calibrate(const void *src, size_t bytes, uint32_t never, uint32_t *out, hipStream_t s);
// One token forward at the device-resident position (DecodeState.pos), then argmax and
// state advance.
hipError_t enqueue_decode_step(sh_model *m);
int gemv_partials(const sh_model *m);

bool persistent_supported(const sh_model *m);
hipError_t persistent_plan(sh_model *m, std::string *why);
constexpr int kArgSlot = 16;  // hand-over words per argmax partial slot (one 128-byte line)
hipError_t launch_persistent(sh_model *m, int pos0, int n_forwards, int n_prompt);
size_t persistent_layer_ptr_bytes(int n_layers);
bool prefill_supported(const sh_model *m, std::string *why);
hipError_t prefill_alloc(sh_model *m, int S, bool logits);
// Causal forward of the rows pf_tokens[0, S) (positions pf_rowpos, sequences pf_rowseq,
// at most seg_max rows per sequence): logits [V, S] into pf_logits when `logits`; fill_kv
// writes every row's K/V into its sequence's cache (decode numerics).
hipError_t enqueue_prefill(sh_model *m, int S, int seg_max, bool logits, bool fill_kv);
// Plugin seams over channel-first [D, S] data in pf_cf (rows at positions 0..S-1 of one
// sequence in pf_rowpos / pf_rowseq): one layer (result back in pf_cf), the final RMSNorm
// (result in pf_cf), the classifier (logits [V, S] in pf_logits).
hipError_t enqueue_layer_cf(sh_model *m, int l, int S);
// The intermediates of the layer enqueue_layer_cf just ran, channel-first: sdpa (x2, q_rope,
// k_rope, v, att) and ffn (x_next, h1, h3), either NULL; h13 is [S, 2F] scratch.
hipError_t enqueue_layer_taps_cf(sh_model *m, int l, int S, float *sdpa, float *ffn, float *h13);
hipError_t enqueue_rms_final_cf(sh_model *m, int S);
hipError_t enqueue_classifier_cf(sh_model *m, int S);
// Model-free products for the stateless seams: partial elements the split GEMM needs, and
// out = x [M, K] . w [N, K]^T (w in the 16-bit type dt; x converted to operand planes in
// `planes`, 2*M*K elements), written [M, N] or channel-first [N, M].
size_t gemm_partial_elems(int M, int N, int K);
// One-time set-up of the GEMM kernels (their LDS limit); called before any capture.
hipError_t gemm_setup();
hipError_t enqueue_linear_rows(const float *x, int M, int K, const uint16_t *w, int N, int dt,
                               uint16_t *planes, float *out, bool cf, float *partial,
                               size_t part_cap, hipStream_t s);
hipError_t enqueue_transpose(const float *src, int rows, int cols, float *dst, hipStream_t s);
bool batch_supported(const sh_model *m, int B, std::string *why);
hipError_t batch_alloc(sh_model *m, int B);
// Before a batched decode's steps: the next tag generation of the attention's split partials.
hipError_t batch_new_generation(sh_model *m);
// One greedy step of B sequences (token bt_tok at bt_pos each), argmax into bt_hist.
hipError_t enqueue_batch_step(sh_model *m, int B);
hipError_t window_alloc(sh_model *m, int max_new);
// One full-window decode step over pf_tokens[0, seq): next token into wd_hist, window shift.
hipError_t enqueue_window_step(sh_model *m, int seq);
void persistent_fill_layer_ptrs(const sh_model *m, void *host);

}  // namespace sh
