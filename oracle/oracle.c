/*
 * oracle.c — CPU restatement of the reference's Stories110M / Qwen3-shaped token loop.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h). Build: oracle/Makefile
 * (gcc -O2 -ffp-contract=off -fopenmp). Nothing here is shipped or measured as the product.
 *
 * Reference files restated (paths relative to the reference tree):
 *   ane/stories/infer.go            KV-cache Decoder: forwardOne, attend, rmsNormVec, matVec,
 *                                   silu, softmaxPrefix, argmax, RoPE tables, Decode loop
 *   ane/stories/cpu.go              EmbedLookup (CF), RMSNorm (CF, float64 product),
 *                                   MatMulVocabSeq
 *   ane/storiesane/engine.go        evalLogitsCPUInto (the full-sequence forward)
 *   ane/storiesane/forward_common.go, accel_other.go, rope.go, residual.go, decode.go
 *   bridge/ane_bridge.m:374-399     symmetric int8 quantizer
 *   training/training_dynamic/io.h:437-457  GQA head mapping kv = h / (H/KVH)
 *
 * Extensions beyond the reference (each switched off for the Stories configuration):
 * GQA, per-head Q/K RMSNorm, configurable RoPE theta / eps / residual scale, K/V storage
 * rounding, and per-output-row W8A8 projections.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define OR_BOS 1
#define OR_EOS 2

/* ------------------------------------------------------------------------------------ */
/* dtype rounding (IEEE round-to-nearest-even, the rounding of v_cvt_f16_f32 and of      */
/* numpy/torch casts). The reference's own converter (ane/mil/generator.go:151-184) only */
/* feeds the ANE path; both sides here consume the same RNE-rounded values.              */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float or_half_round(float x) {
    uint32_t u = f2u(x);
    uint32_t sign = u & 0x80000000u;
    uint32_t absu = u & 0x7fffffffu;
    if (absu >= 0x7f800000u) return x;                       /* inf / nan pass through */
    float a = u2f(absu);
    if (a >= 65520.0f) return u2f(sign | 0x7f800000u);       /* rounds to inf */
    if (a < 6.103515625e-05f) {                              /* fp16 subnormal range */
        /* quantum 2^-24: round-to-nearest-even of a / 2^-24 */
        double q = (double)a * 16777216.0;
        double r = nearbyint(q);                             /* default mode: ties to even */
        float m = (float)(r / 16777216.0);
        return sign ? -m : m;
    }
    /* normal: keep 10 mantissa bits, RNE on the 13 dropped bits */
    uint32_t lsb = (absu >> 13) & 1u;
    uint32_t rounded = absu + 0x0fffu + lsb;
    rounded &= ~0x1fffu;
    return u2f(sign | rounded);
}

float or_bf16_round(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return x;          /* nan */
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    u &= 0xffff0000u;
    return u2f(u);
}

static float kv_round(int kv_dtype, float v) {
    if (kv_dtype == OR_KV_F16) return or_half_round(v);
    if (kv_dtype == OR_KV_BF16) return or_bf16_round(v);
    return v;
}

/* ------------------------------------------------------------------------------------ */
/* infer.go:301-311 rmsNormVec: float64 sum of squares, float32 rrms, (x*rrms)*w float32 */
void or_rms_norm_vec(float *out, const float *x, const float *w, int n, double eps) {
    double sum = 0;
    for (int i = 0; i < n; i++) {
        double v = (double)x[i];
        sum += v * v;
    }
    float rrms = (float)(1.0 / sqrt(sum / (double)n + eps));
    for (int i = 0; i < n; i++) out[i] = x[i] * rrms * w[i];
}

/* infer.go:313-322 matVec: out[r] = sum over c in order of row[c]*in[c], float32.
 * Four rows are walked together so the CPU overlaps their independent add chains; each
 * row's own sum keeps the reference order. */
static void mat_vec_range(float *out, const float *mat, const float *in, int r0, int r1,
                          int cols) {
    int r = r0;
    for (; r + 4 <= r1; r += 4) {
        const float *a = mat + (size_t)r * cols;
        const float *b = a + cols, *c = b + cols, *d = c + cols;
        float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
        for (int k = 0; k < cols; k++) {
            float xv = in[k];
            s0 += a[k] * xv;
            s1 += b[k] * xv;
            s2 += c[k] * xv;
            s3 += d[k] * xv;
        }
        out[r] = s0; out[r + 1] = s1; out[r + 2] = s2; out[r + 3] = s3;
    }
    for (; r < r1; r++) {
        const float *a = mat + (size_t)r * cols;
        float s = 0;
        for (int k = 0; k < cols; k++) s += a[k] * in[k];
        out[r] = s;
    }
}

void or_mat_vec(float *out, const float *mat, const float *in, int rows, int cols,
                int threads) {
    if (threads <= 1 || rows < 256) {
        mat_vec_range(out, mat, in, 0, rows, cols);
        return;
    }
    int chunks = (rows + 63) / 64;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int ch = 0; ch < chunks; ch++) {
        int r0 = ch * 64, r1 = r0 + 64 > rows ? rows : r0 + 64;
        mat_vec_range(out, mat, in, r0, r1, cols);
    }
}

/* infer.go:324-326 silu: x / (1 + float32(exp(float64(-x)))) */
float or_silu(float x) { return x / (1.0f + (float)exp((double)(-x))); }

/* infer.go:328-345 softmaxPrefix: float32 max, float32(exp(float64(s-mx))), float64 sum of
 * the rounded terms, float32 inverse, float32 scale. */
void or_softmax_prefix(float *dst, const float *src, int n) {
    float mx = src[0];
    for (int i = 1; i < n; i++)
        if (src[i] > mx) mx = src[i];
    double sum = 0;
    for (int i = 0; i < n; i++) {
        float e = (float)exp((double)(src[i] - mx));
        dst[i] = e;
        sum += (double)e;
    }
    float inv = (float)(1.0 / sum);
    for (int i = 0; i < n; i++) dst[i] *= inv;
}

/* infer.go:373-383 argmax: first maximum (strict >) */
int32_t or_argmax(const float *v, int n) {
    int32_t best = 0;
    float bv = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > bv) { bv = v[i]; best = i; }
    return best;
}

/* infer.go:97-107 / rope.go:5-24: freq = pos / theta^(2i/hd) in float64, float32 cos/sin,
 * table [max_seq][hd/2] */
void or_rope_tables(float *cos_out, float *sin_out, int max_seq, int head_dim, double theta) {
    int half = head_dim / 2;
    for (int pos = 0; pos < max_seq; pos++)
        for (int i = 0; i < half; i++) {
            double freq = (double)pos / pow(theta, (double)(2 * i) / (double)head_dim);
            cos_out[pos * half + i] = (float)cos(freq);
            sin_out[pos * half + i] = (float)sin(freq);
        }
}

/* ------------------------------------------------------------------------------------ */
/* bridge/ane_bridge.m:374-399: scale = max|x|/127 (0 -> 1); v = x/scale; clamp to        */
/* [-128,127]; q = (int8)(v + (v >= 0 ? 0.5 : -0.5)) (round half away, then truncate).    */
int8_t or_quantize_value(float v) {
    if (v > 127.0f) v = 127.0f;
    if (v < -128.0f) v = -128.0f;
    return (int8_t)(v + (v >= 0 ? 0.5f : -0.5f));
}

float or_absmax_scale(const float *src, size_t n) {
    float max_abs = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float a = src[i] < 0 ? -src[i] : src[i];
        if (a > max_abs) max_abs = a;
    }
    float scale = max_abs / 127.0f;
    if (scale == 0.0f) scale = 1.0f;
    return scale;
}

void or_quantize_tensor(const float *src, size_t n, int8_t *dst, float *scale_out) {
    float scale = or_absmax_scale(src, n);
    for (size_t i = 0; i < n; i++) dst[i] = or_quantize_value(src[i] / scale);
    *scale_out = scale;
}

/* The bridge formula applied to each output row on its own (one row = the bridge call). */
void or_quantize_rows(const float *src, int rows, int cols, int8_t *dst, float *scales) {
    for (int r = 0; r < rows; r++)
        or_quantize_tensor(src + (size_t)r * cols, (size_t)cols, dst + (size_t)r * cols,
                           &scales[r]);
}

void or_dequantize_rows(const int8_t *q, const float *scales, int rows, int cols,
                        float *dst) {
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < cols; c++)
            dst[(size_t)r * cols + c] = (float)q[(size_t)r * cols + c] * scales[r];
}

/* W8A8 projection: per-tensor activation quantization of `in`, exact int32 dot product per
 * row, y = (float)acc * (s_w[r] * s_a). */
void or_mat_vec_w8a8(float *out, const int8_t *wq, const float *wscale, const float *in,
                     int rows, int cols, int threads) {
    int8_t *qa = (int8_t *)malloc((size_t)cols);
    float sa;
    or_quantize_tensor(in, (size_t)cols, qa, &sa);
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static) if (threads > 1 && rows >= 256)
    for (int r = 0; r < rows; r++) {
        const int8_t *row = wq + (size_t)r * cols;
        int32_t acc = 0;
        for (int c = 0; c < cols; c++) acc += (int32_t)row[c] * (int32_t)qa[c];
        out[r] = (float)acc * (wscale[r] * sa);
    }
    free(qa);
}

/* ------------------------------------------------------------------------------------ */
/* KV-cache decoder: ane/stories/infer.go                                                */

enum { P_WQ, P_WK, P_WV, P_WO, P_W1, P_W2, P_W3, P_N };

struct or_decoder {
    or_config cfg;
    or_layer *layers;
    const float *embed, *rms_final, *cls;
    int threads;
    int qdim, kvdim, hd;
    float *kc, *vc;           /* [L][max_seq][kvdim] */
    float *rcos, *rsin;       /* [max_seq][hd/2] */
    float *x, *xn, *q, *k, *v, *att, *x2, *x2n, *h1, *h3, *ff, *scores, *probs, *logits;
    float *qpre, *kpre;       /* q and k of the last layer before QK-norm and RoPE (taps) */
    /* W8A8 */
    int8_t *q8[64][P_N];
    float *s8[64][P_N];
    int8_t *cls8;
    float *cls_s;
};

static const float *layer_mat(const or_layer *l, int p) {
    switch (p) {
    case P_WQ: return l->wq;
    case P_WK: return l->wk;
    case P_WV: return l->wv;
    case P_WO: return l->wo;
    case P_W1: return l->w1;
    case P_W2: return l->w2;
    default: return l->w3;
    }
}

static void mat_shape(const or_decoder *d, int p, int *rows, int *cols) {
    const or_config *c = &d->cfg;
    switch (p) {
    case P_WQ: *rows = d->qdim; *cols = c->dim; break;
    case P_WK: case P_WV: *rows = d->kvdim; *cols = c->dim; break;
    case P_WO: *rows = c->dim; *cols = d->qdim; break;
    case P_W1: case P_W3: *rows = c->hidden; *cols = c->dim; break;
    default: *rows = c->dim; *cols = c->hidden; break;
    }
}

or_decoder *or_decoder_new(const or_config *cfg, const or_weights *w, int threads) {
    if (!cfg || !w || cfg->n_layers > 64 || cfg->n_layers <= 0) return NULL;
    if (cfg->n_kv_heads <= 0 || cfg->n_heads % cfg->n_kv_heads) return NULL;
    or_decoder *d = (or_decoder *)calloc(1, sizeof(*d));
    d->cfg = *cfg;
    d->threads = threads < 1 ? 1 : threads;
    d->hd = cfg->head_dim;
    d->qdim = cfg->n_heads * cfg->head_dim;
    d->kvdim = cfg->n_kv_heads * cfg->head_dim;
    d->layers = (or_layer *)malloc(sizeof(or_layer) * cfg->n_layers);
    memcpy(d->layers, w->layers, sizeof(or_layer) * cfg->n_layers);
    d->embed = w->embed;
    d->rms_final = w->rms_final;
    d->cls = w->cls ? w->cls : w->embed;
    size_t kvn = (size_t)cfg->n_layers * cfg->max_seq * d->kvdim;
    d->kc = (float *)calloc(kvn, sizeof(float));
    d->vc = (float *)calloc(kvn, sizeof(float));
    int half = d->hd / 2;
    d->rcos = (float *)malloc(sizeof(float) * cfg->max_seq * half);
    d->rsin = (float *)malloc(sizeof(float) * cfg->max_seq * half);
    or_rope_tables(d->rcos, d->rsin, cfg->max_seq, d->hd, cfg->rope_theta);
    int big = cfg->dim > d->qdim ? cfg->dim : d->qdim;
    d->x = (float *)calloc(cfg->dim, sizeof(float));
    d->xn = (float *)calloc(cfg->dim, sizeof(float));
    d->q = (float *)calloc(d->qdim, sizeof(float));
    d->k = (float *)calloc(d->kvdim, sizeof(float));
    d->v = (float *)calloc(d->kvdim, sizeof(float));
    d->qpre = (float *)calloc(d->qdim, sizeof(float));
    d->kpre = (float *)calloc(d->kvdim, sizeof(float));
    d->att = (float *)calloc(big, sizeof(float));
    d->x2 = (float *)calloc(cfg->dim, sizeof(float));
    d->x2n = (float *)calloc(cfg->dim, sizeof(float));
    d->h1 = (float *)calloc(cfg->hidden, sizeof(float));
    d->h3 = (float *)calloc(cfg->hidden, sizeof(float));
    d->ff = (float *)calloc(cfg->dim, sizeof(float));
    d->scores = (float *)calloc(cfg->max_seq, sizeof(float));
    d->probs = (float *)calloc(cfg->max_seq, sizeof(float));
    d->logits = (float *)calloc(cfg->vocab, sizeof(float));
    if (cfg->w8a8) {
        for (int l = 0; l < cfg->n_layers; l++)
            for (int p = 0; p < P_N; p++) {
                int rows, cols;
                mat_shape(d, p, &rows, &cols);
                d->q8[l][p] = (int8_t *)malloc((size_t)rows * cols);
                d->s8[l][p] = (float *)malloc(sizeof(float) * rows);
                or_quantize_rows(layer_mat(&d->layers[l], p), rows, cols, d->q8[l][p],
                                 d->s8[l][p]);
            }
        d->cls8 = (int8_t *)malloc((size_t)cfg->vocab * cfg->dim);
        d->cls_s = (float *)malloc(sizeof(float) * cfg->vocab);
        or_quantize_rows(d->cls, cfg->vocab, cfg->dim, d->cls8, d->cls_s);
    }
    return d;
}

void or_decoder_free(or_decoder *d) {
    if (!d) return;
    if (d->cfg.w8a8) {
        for (int l = 0; l < d->cfg.n_layers; l++)
            for (int p = 0; p < P_N; p++) { free(d->q8[l][p]); free(d->s8[l][p]); }
        free(d->cls8);
        free(d->cls_s);
    }
    free(d->layers); free(d->kc); free(d->vc); free(d->rcos); free(d->rsin);
    free(d->x); free(d->xn); free(d->q); free(d->k); free(d->v); free(d->att);
    free(d->qpre); free(d->kpre);
    free(d->x2); free(d->x2n); free(d->h1); free(d->h3); free(d->ff);
    free(d->scores); free(d->probs); free(d->logits);
    free(d);
}

/* infer.go:61-70 ResetCache */
void or_decoder_reset(or_decoder *d) {
    size_t kvn = (size_t)d->cfg.n_layers * d->cfg.max_seq * d->kvdim;
    memset(d->kc, 0, kvn * sizeof(float));
    memset(d->vc, 0, kvn * sizeof(float));
}

static void project(or_decoder *d, int l, int p, float *out, const float *in) {
    int rows, cols;
    mat_shape(d, p, &rows, &cols);
    if (d->cfg.w8a8)
        or_mat_vec_w8a8(out, d->q8[l][p], d->s8[l][p], in, rows, cols, d->threads);
    else
        or_mat_vec(out, layer_mat(&d->layers[l], p), in, rows, cols, d->threads);
}

/* infer.go:247-265 applyRoPE on n_heads heads of vec (interleaved pairs 2i, 2i+1) */
static void apply_rope(const or_decoder *d, float *vec, int n_heads, int pos) {
    int stride = d->hd / 2;
    for (int h = 0; h < n_heads; h++) {
        int base = h * d->hd;
        int rb = pos * stride;
        for (int i = 0; i < stride; i++) {
            float c = d->rcos[rb + i], s = d->rsin[rb + i];
            float e = vec[base + 2 * i], o = vec[base + 2 * i + 1];
            vec[base + 2 * i] = e * c - o * s;
            vec[base + 2 * i + 1] = e * s + o * c;
        }
    }
}

/* infer.go:273-299 attend; q head h reads kv head h / (H/KVH) (io.h:437-457 mapping).
 * q, att, scores and probs are the caller's (the decoder's own vectors for forwardOne, one
 * token's rows and per-thread buffers for the prompt pass). */
static void attend_into(const or_decoder *d, int layer, int pos, const float *q, float *att,
                        float *scores, float *probs) {
    const or_config *c = &d->cfg;
    int hd = d->hd;
    int group = c->n_heads / c->n_kv_heads;
    float inv_sqrt_hd = (float)(1.0 / sqrt((double)hd));
    for (int h = 0; h < c->n_heads; h++) {
        int qb = h * hd;
        int kb0 = (h / group) * hd;
        for (int t = 0; t <= pos; t++) {
            const float *kr = d->kc + ((size_t)layer * c->max_seq + t) * d->kvdim + kb0;
            float dot = 0;
            for (int i = 0; i < hd; i++) dot += q[qb + i] * kr[i];
            scores[t] = dot * inv_sqrt_hd;
        }
        or_softmax_prefix(probs, scores, pos + 1);
        for (int i = 0; i < hd; i++) {
            float sum = 0;
            for (int t = 0; t <= pos; t++) {
                const float *vr = d->vc + ((size_t)layer * c->max_seq + t) * d->kvdim + kb0;
                sum += probs[t] * vr[i];
            }
            att[qb + i] = sum;
        }
    }
}

static void attend(or_decoder *d, int layer, int pos) {
    attend_into(d, layer, pos, d->q, d->att, d->scores, d->probs);
}

/* infer.go:204-245 forwardOne */
int or_forward_one(or_decoder *d, int token, int pos, float *logits_out) {
    const or_config *c = &d->cfg;
    if (token < 0 || token >= c->vocab) return -1;
    if (pos < 0 || pos >= c->max_seq) return -1;
    int D = c->dim, F = c->hidden, hd = d->hd;
    float alpha = c->residual_scale;
    memcpy(d->x, d->embed + (size_t)token * D, sizeof(float) * D);
    for (int l = 0; l < c->n_layers; l++) {
        const or_layer *L = &d->layers[l];
        or_rms_norm_vec(d->xn, d->x, L->rms_att, D, c->norm_eps);
        project(d, l, P_WQ, d->q, d->xn);
        project(d, l, P_WK, d->k, d->xn);
        project(d, l, P_WV, d->v, d->xn);
        memcpy(d->qpre, d->q, sizeof(float) * d->qdim);
        memcpy(d->kpre, d->k, sizeof(float) * d->kvdim);
        if (c->qk_norm) {
            for (int h = 0; h < c->n_heads; h++)
                or_rms_norm_vec(d->q + h * hd, d->q + h * hd, L->q_norm, hd, c->qk_norm_eps);
            for (int h = 0; h < c->n_kv_heads; h++)
                or_rms_norm_vec(d->k + h * hd, d->k + h * hd, L->k_norm, hd, c->qk_norm_eps);
        }
        apply_rope(d, d->q, c->n_heads, pos);
        apply_rope(d, d->k, c->n_kv_heads, pos);
        /* infer.go:267-271 storeKV (rounded to the cache's storage type) */
        size_t base = ((size_t)l * c->max_seq + pos) * d->kvdim;
        for (int i = 0; i < d->kvdim; i++) {
            d->kc[base + i] = kv_round(c->kv_dtype, d->k[i]);
            d->vc[base + i] = kv_round(c->kv_dtype, d->v[i]);
        }
        attend(d, l, pos);
        project(d, l, P_WO, d->x2, d->att);
        for (int i = 0; i < D; i++) d->x2[i] = d->x[i] + alpha * d->x2[i];
        or_rms_norm_vec(d->x2n, d->x2, L->rms_ffn, D, c->norm_eps);
        project(d, l, P_W1, d->h1, d->x2n);
        project(d, l, P_W3, d->h3, d->x2n);
        for (int i = 0; i < F; i++) d->h1[i] = or_silu(d->h1[i]) * d->h3[i];
        project(d, l, P_W2, d->ff, d->h1);
        for (int i = 0; i < D; i++) d->x[i] = d->x2[i] + alpha * d->ff[i];
    }
    or_rms_norm_vec(d->xn, d->x, d->rms_final, D, c->norm_eps);
    if (c->w8a8)
        or_mat_vec_w8a8(d->logits, d->cls8, d->cls_s, d->xn, c->vocab, D, d->threads);
    else
        or_mat_vec(d->logits, d->cls, d->xn, c->vocab, D, d->threads);
    if (logits_out) memcpy(logits_out, d->logits, sizeof(float) * c->vocab);
    return 0;
}

/* matVec (infer.go:313-322) for n tokens at once: out[t*rows + r] = sum over c in order of
 * mat[r*cols + c] * in[t*cols + c]. Eight tokens ride in the lanes of two 4-float vectors,
 * so each lane adds its own token's products in the reference order (multiply, then add:
 * -ffp-contract=off keeps them apart), and four weight rows share each block of tokens. */
typedef float or_v4 __attribute__((vector_size(16)));

static void mat_tokens(float *out, const float *mat, const float *in, int rows, int cols, int n,
                       int threads) {
    int nb = (n + 7) / 8;
    or_v4 *xt = (or_v4 *)aligned_alloc(16, sizeof(or_v4) * 2 * (size_t)cols * nb);
    float *xf = (float *)xt;
    for (int b = 0; b < nb; b++)
        for (int c = 0; c < cols; c++)
            for (int j = 0; j < 8; j++) {
                int t = b * 8 + j;
                xf[((size_t)b * cols + c) * 8 + j] = t < n ? in[(size_t)t * cols + c] : 0.0f;
            }
    int groups = (rows + 3) / 4;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int g = 0; g < groups; g++) {
        int r0 = g * 4, nr = rows - r0 < 4 ? rows - r0 : 4;
        const float *w[4];
        for (int i = 0; i < 4; i++) w[i] = mat + (size_t)(r0 + (i < nr ? i : 0)) * cols;
        for (int b = 0; b < nb; b++) {
            const or_v4 *x = xt + (size_t)b * cols * 2;
            or_v4 s[4][2];
            memset(s, 0, sizeof(s));
            for (int c = 0; c < cols; c++) {
                or_v4 x0 = x[2 * c], x1 = x[2 * c + 1];
                for (int i = 0; i < 4; i++) {
                    float wv = w[i][c];
                    or_v4 wb = {wv, wv, wv, wv};
                    s[i][0] += wb * x0;
                    s[i][1] += wb * x1;
                }
            }
            for (int i = 0; i < nr; i++)
                for (int j = 0; j < 8 && b * 8 + j < n; j++)
                    out[(size_t)(b * 8 + j) * rows + r0 + i] = s[i][j >> 2][j & 3];
        }
    }
    free(xt);
}

/* or_mat_vec_w8a8 for n tokens: each token's activation quantized on its own, then the exact
 * int32 dot per row and y = (float)acc * (s_w[r] * s_a[t]). */
static void mat_tokens_w8a8(float *out, const int8_t *wq, const float *wscale, const float *in,
                            int rows, int cols, int n, int threads) {
    int8_t *qa = (int8_t *)malloc((size_t)n * cols);
    float *sa = (float *)malloc(sizeof(float) * (size_t)n);
    for (int t = 0; t < n; t++)
        or_quantize_tensor(in + (size_t)t * cols, (size_t)cols, qa + (size_t)t * cols, &sa[t]);
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int r = 0; r < rows; r++) {
        const int8_t *row = wq + (size_t)r * cols;
        for (int t = 0; t < n; t++) {
            const int8_t *a = qa + (size_t)t * cols;
            int32_t acc = 0;
            for (int c = 0; c < cols; c++) acc += (int32_t)row[c] * (int32_t)a[c];
            out[(size_t)t * rows + r] = (float)acc * (wscale[r] * sa[t]);
        }
    }
    free(qa);
    free(sa);
}

static void project_tokens(const or_decoder *d, int l, int p, float *out, const float *in,
                           int n) {
    int rows, cols;
    mat_shape(d, p, &rows, &cols);
    if (d->cfg.w8a8)
        mat_tokens_w8a8(out, d->q8[l][p], d->s8[l][p], in, rows, cols, n, d->threads);
    else
        mat_tokens(out, layer_mat(&d->layers[l], p), in, rows, cols, n, d->threads);
}

/* The prompt part of Decode (infer.go:136-202 feeds the prompt ids to forwardOne one
 * position at a time) with the loops turned layer-major: tokens[0, n) at positions
 * pos0 .. pos0+n-1. Every token gets forwardOne's values at its position: the same ordered
 * float32 sums, RMSNorms, RoPE and K/V rounding, and attention over the positions up to its
 * own, whose K/V the layer pass has stored before any token of it attends. The K/V cache it
 * leaves and the last token's logits therefore equal those of n calls of or_forward_one, bit
 * for bit. The classifier runs for the last token only; the taps are not updated. */
static int prompt_forward(or_decoder *d, const int32_t *tokens, int n, int pos0, int first, float *logits_out);

int or_prompt_forward(or_decoder *d, const int32_t *tokens, int n, int pos0, float *logits_out) {
    return prompt_forward(d, tokens, n, pos0, n - 1, logits_out);
}

/* or_prompt_forward keeping the logits of every token from `first` on: logits_out[(t - first)
 * * vocab + v] for t in [first, n), each equal, bit for bit, to or_forward_one's at position
 * pos0 + t (the final RMSNorm per token, then the classifier rows summed in the same order). */
int or_prompt_forward_logits(or_decoder *d, const int32_t *tokens, int n, int pos0, int first,
                             float *logits_out) {
    if (first < 0 || first >= n || !logits_out) return -1;
    return prompt_forward(d, tokens, n, pos0, first, logits_out);
}

static int prompt_forward(or_decoder *d, const int32_t *tokens, int n, int pos0, int first, float *logits_out) {
    const or_config *c = &d->cfg;
    if (n <= 0 || pos0 < 0 || pos0 + n > c->max_seq) return -1;
    for (int t = 0; t < n; t++)
        if (tokens[t] < 0 || tokens[t] >= c->vocab) return -1;
    int D = c->dim, F = c->hidden, hd = d->hd, qd = d->qdim, kvd = d->kvdim;
    int thr = d->threads;
    float alpha = c->residual_scale;
    size_t N = (size_t)n;
    float *x = (float *)malloc(sizeof(float) * N * D);
    float *xn = (float *)malloc(sizeof(float) * N * D);
    float *q = (float *)malloc(sizeof(float) * N * qd);
    float *k = (float *)malloc(sizeof(float) * N * kvd);
    float *v = (float *)malloc(sizeof(float) * N * kvd);
    float *att = (float *)malloc(sizeof(float) * N * qd);
    float *x2 = (float *)malloc(sizeof(float) * N * D);
    float *h1 = (float *)malloc(sizeof(float) * N * F);
    float *h3 = (float *)malloc(sizeof(float) * N * F);
    for (int t = 0; t < n; t++)
        memcpy(x + (size_t)t * D, d->embed + (size_t)tokens[t] * D, sizeof(float) * D);
    for (int l = 0; l < c->n_layers; l++) {
        const or_layer *L = &d->layers[l];
        for (int t = 0; t < n; t++)
            or_rms_norm_vec(xn + (size_t)t * D, x + (size_t)t * D, L->rms_att, D, c->norm_eps);
        project_tokens(d, l, P_WQ, q, xn, n);
        project_tokens(d, l, P_WK, k, xn, n);
        project_tokens(d, l, P_WV, v, xn, n);
        for (int t = 0; t < n; t++) {
            float *qt = q + (size_t)t * qd, *kt = k + (size_t)t * kvd, *vt = v + (size_t)t * kvd;
            if (c->qk_norm) {
                for (int h = 0; h < c->n_heads; h++)
                    or_rms_norm_vec(qt + h * hd, qt + h * hd, L->q_norm, hd, c->qk_norm_eps);
                for (int h = 0; h < c->n_kv_heads; h++)
                    or_rms_norm_vec(kt + h * hd, kt + h * hd, L->k_norm, hd, c->qk_norm_eps);
            }
            apply_rope(d, qt, c->n_heads, pos0 + t);
            apply_rope(d, kt, c->n_kv_heads, pos0 + t);
            size_t base = ((size_t)l * c->max_seq + pos0 + t) * kvd;
            for (int i = 0; i < kvd; i++) {
                d->kc[base + i] = kv_round(c->kv_dtype, kt[i]);
                d->vc[base + i] = kv_round(c->kv_dtype, vt[i]);
            }
        }
#pragma omp parallel num_threads(thr)
        {
            float *sc = (float *)malloc(sizeof(float) * c->max_seq);
            float *pr = (float *)malloc(sizeof(float) * c->max_seq);
#pragma omp for schedule(dynamic, 4)
            for (int t = 0; t < n; t++)
                attend_into(d, l, pos0 + t, q + (size_t)t * qd, att + (size_t)t * qd, sc, pr);
            free(sc);
            free(pr);
        }
        project_tokens(d, l, P_WO, x2, att, n);
        for (size_t i = 0; i < N * D; i++) x2[i] = x[i] + alpha * x2[i];
        for (int t = 0; t < n; t++)
            or_rms_norm_vec(xn + (size_t)t * D, x2 + (size_t)t * D, L->rms_ffn, D, c->norm_eps);
        project_tokens(d, l, P_W1, h1, xn, n);
        project_tokens(d, l, P_W3, h3, xn, n);
        for (size_t i = 0; i < N * F; i++) h1[i] = or_silu(h1[i]) * h3[i];
        project_tokens(d, l, P_W2, x, h1, n);
        for (size_t i = 0; i < N * D; i++) x[i] = x2[i] + alpha * x[i];
    }
    or_rms_norm_vec(d->xn, x + (N - 1) * D, d->rms_final, D, c->norm_eps);
    if (c->w8a8)
        or_mat_vec_w8a8(d->logits, d->cls8, d->cls_s, d->xn, c->vocab, D, thr);
    else
        or_mat_vec(d->logits, d->cls, d->xn, c->vocab, D, thr);
    if (logits_out && first == n - 1) {
        memcpy(logits_out, d->logits, sizeof(float) * c->vocab);
    } else if (logits_out) {
        int nk = n - first;
        for (int t = first; t < n; t++)
            or_rms_norm_vec(xn + (size_t)(t - first) * D, x + (size_t)t * D, d->rms_final, D, c->norm_eps);
        if (c->w8a8)
            mat_tokens_w8a8(logits_out, d->cls8, d->cls_s, xn, c->vocab, D, nk, thr);
        else
            mat_tokens(logits_out, d->cls, xn, c->vocab, D, nk, thr);
    }
    free(x); free(xn); free(q); free(k); free(v); free(att); free(x2); free(h1); free(h3);
    return 0;
}

const float *or_decoder_tap(const or_decoder *d, int which) {
    switch (which) {
    case 0: return d->x;
    case 1: return d->q;
    case 2: return d->k;
    case 3: return d->v;
    case 4: return d->att;
    case 5: return d->h1;
    case 6: return d->x2;
    case 7: return d->qpre;
    case 8: return d->kpre;
    default: return d->logits;
    }
}

static float top2_margin(const float *v, int n) {
    float a = -INFINITY, b = -INFINITY;
    for (int i = 0; i < n; i++) {
        if (v[i] > a) { b = a; a = v[i]; }
        else if (v[i] > b) b = v[i];
    }
    return a - b;
}

/* sampleFromLogits (infer.go:347-371) with the uniform draw given: temperature <= 1e-6 takes
 * the first maximum (argmax, infer.go:373-383); otherwise mx = the first maximum's value,
 * terms exp((float64(l) - float64(mx)) * float64(1/T)) (1/T in float32, as the reference's
 * invT := float64(1 / temperature)), total their float64 sum in index order, target = u * total,
 * and the first index whose running float64 sum reaches target (the last index if none does).
 * *slack (may be NULL) receives the target's distance from the nearer end of the chosen index's
 * CDF interval, divided by total (0 for the argmax rule). */
int or_sample_from_logits(const float *logits, int n, float temperature, double u, double *slack) {
    if (slack) *slack = 0.0;
    if (temperature <= 1e-6f) {
        int best = 0;
        for (int i = 1; i < n; i++)
            if (logits[i] > logits[best]) best = i;
        return best;
    }
    float mx = logits[0];
    for (int i = 1; i < n; i++)
        if (logits[i] > mx) mx = logits[i];
    double inv_t = (double)(1.0f / temperature);
    double total = 0.0;
    for (int i = 0; i < n; i++) total += exp(((double)logits[i] - (double)mx) * inv_t);
    double target = u * total, acc = 0.0;
    for (int i = 0; i < n; i++) {
        double lo = acc;
        acc += exp(((double)logits[i] - (double)mx) * inv_t);
        if (acc >= target) {
            if (slack) *slack = fmin(target - lo, acc - target) / total;
            return i;
        }
    }
    return n - 1;
}

/* infer.go:136-202 Decode with temperature <= 1e-6 (argmax sampling, infer.go:347-350) */
int or_greedy_decode(or_decoder *d, const int32_t *prompt, int n_prompt, int max_new,
                     int32_t *out_tokens, int32_t *n_out, int32_t *stopped_eos,
                     float *margins) {
    const or_config *c = &d->cfg;
    if (max_new <= 0) max_new = 64;
    int32_t bos = OR_BOS;
    if (n_prompt <= 0) { prompt = &bos; n_prompt = 1; }
    if (n_prompt > c->max_seq) { prompt += n_prompt - c->max_seq; n_prompt = c->max_seq; }
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= c->vocab) return -1;
    or_decoder_reset(d);
    int n = 0;
    for (int i = 0; i < n_prompt; i++) out_tokens[n++] = prompt[i];
    if (n_prompt > 1 && or_prompt_forward(d, prompt, n_prompt - 1, 0, NULL)) return -1;
    *stopped_eos = 0;
    for (int step = 0; step < max_new && n < c->max_seq; step++) {
        int pos = n - 1;
        if (or_forward_one(d, out_tokens[pos], pos, NULL)) return -1;
        int32_t next = or_argmax(d->logits, c->vocab);
        if (margins) margins[step] = top2_margin(d->logits, c->vocab);
        out_tokens[n++] = next;
        if (next == OR_EOS) { *stopped_eos = 1; break; }
    }
    *n_out = n;
    return 0;
}

/* ------------------------------------------------------------------------------------ */
/* Full-sequence channel-first forward: ane/storiesane/engine.go:804-842                 */

/* cpu.go:41-72 EmbedLookup: out[d*S+t] = embed[tok*D+d]; out-of-range token -> zero column */
void or_embed_lookup_cf(float *out, const float *embed, int vocab, const uint16_t *tokens,
                        int dim, int seq) {
    for (int t = 0; t < seq; t++) {
        int tok = tokens[t];
        for (int d = 0; d < dim; d++)
            out[(size_t)d * seq + t] =
                (tok < 0 || tok >= vocab) ? 0.0f : embed[(size_t)tok * dim + d];
    }
}

/* accel_other.go:11-28 rmsNormCFWithRRMSImpl: float64 sum, float32 scale, x*scale*w */
static void rms_norm_cf(float *out, const float *x, const float *w, int dim, int seq,
                        double eps) {
    for (int t = 0; t < seq; t++) {
        double sum = 0;
        for (int i = 0; i < dim; i++) {
            double v = (double)x[(size_t)i * seq + t];
            sum += v * v;
        }
        float scale = (float)(1.0 / sqrt(sum / (double)dim + eps));
        for (int i = 0; i < dim; i++)
            out[(size_t)i * seq + t] = x[(size_t)i * seq + t] * scale * w[i];
    }
}

/* forward_common.go:35-46 linearCF: out[o*S+t] = sum over i in order of W[o,i]*in[i*S+t].
 * The input is first transposed to [S][in] (pure data movement) so the ordered sums read
 * contiguous memory. */
static void linear_cf(float *out, const float *wts, const float *in, int out_ch, int in_ch,
                      int seq, int threads) {
    float *inT = (float *)malloc(sizeof(float) * (size_t)in_ch * seq);
    for (int i = 0; i < in_ch; i++)
        for (int t = 0; t < seq; t++) inT[(size_t)t * in_ch + i] = in[(size_t)i * seq + t];
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int o = 0; o < out_ch; o++) {
        const float *row = wts + (size_t)o * in_ch;
        int t = 0;
        for (; t + 4 <= seq; t += 4) {
            const float *a = inT + (size_t)t * in_ch;
            const float *b = a + in_ch, *c = b + in_ch, *e = c + in_ch;
            float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
            for (int i = 0; i < in_ch; i++) {
                float wv = row[i];
                s0 += wv * a[i];
                s1 += wv * b[i];
                s2 += wv * c[i];
                s3 += wv * e[i];
            }
            out[(size_t)o * seq + t] = s0;
            out[(size_t)o * seq + t + 1] = s1;
            out[(size_t)o * seq + t + 2] = s2;
            out[(size_t)o * seq + t + 3] = s3;
        }
        for (; t < seq; t++) {
            const float *a = inT + (size_t)t * in_ch;
            float s = 0;
            for (int i = 0; i < in_ch; i++) s += row[i] * a[i];
            out[(size_t)o * seq + t] = s;
        }
    }
    free(inT);
}

/* rope.go:26-46 applyRoPECFInPlace: e' = e*c - o*s, o' = o*c + e*s */
static void rope_cf(float *x, int heads, int hd, int seq, const float *rc, const float *rs) {
    int half = hd / 2;
    for (int h = 0; h < heads; h++)
        for (int i = 0; i < half; i++) {
            size_t even = (size_t)(h * hd + 2 * i) * seq, odd = even + seq;
            for (int t = 0; t < seq; t++) {
                float c = rc[t * half + i], s = rs[t * half + i];
                float e = x[even + t], o = x[odd + t];
                x[even + t] = e * c - o * s;
                x[odd + t] = o * c + e * s;
            }
        }
}

/* Per-head RMSNorm of q or k in channel-first layout (extension: Qwen3-shaped QK-norm),
 * the rmsNormVec arithmetic (infer.go:301-311) over each head's hd values at each t. */
static void qk_norm_cf(float *x, int heads, int hd, int seq, const float *g, double eps) {
    for (int h = 0; h < heads; h++)
        for (int t = 0; t < seq; t++) {
            double sum = 0;
            for (int i = 0; i < hd; i++) {
                double v = (double)x[(size_t)(h * hd + i) * seq + t];
                sum += v * v;
            }
            float rr = (float)(1.0 / sqrt(sum / (double)hd + eps));
            for (int i = 0; i < hd; i++) {
                size_t o = (size_t)(h * hd + i) * seq + t;
                x[o] = x[o] * rr * g[i];
            }
        }
}

/* accel_other.go:190-207 softmaxRowAccel: float64 exp terms summed unrounded */
static void softmax_row(float *out, const float *in, int n) {
    float maxv = in[0];
    for (int i = 1; i < n; i++)
        if (in[i] > maxv) maxv = in[i];
    double sum = 0;
    for (int i = 0; i < n; i++) {
        double e = exp((double)(in[i] - maxv));
        out[i] = (float)e;
        sum += e;
    }
    float inv = (float)(1.0 / sum);
    for (int i = 0; i < n; i++) out[i] *= inv;
}

/* forward_common.go:5-33 causalAttentionCF: masked scores = -65504, softmax over the whole
 * row, P.V over the whole row. q head h reads kv head h / (H/KVH). */
static void causal_attention_cf(float *out, const float *qf, const float *kf,
                                const float *vf, int heads, int kv_heads, int hd, int seq,
                                int threads) {
    float scale = (float)(1.0 / sqrt((double)hd));
    int group = heads / kv_heads;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int h = 0; h < heads; h++) {
        float *scores = (float *)malloc(sizeof(float) * seq);
        float *probs = (float *)malloc(sizeof(float) * seq);
        int qb = h * hd, kb = (h / group) * hd;
        for (int t = 0; t < seq; t++) {
            for (int j = 0; j < seq; j++) {
                if (j > t) { scores[j] = -65504.0f; continue; }
                float sum = 0;
                for (int i = 0; i < hd; i++)
                    sum += qf[(size_t)(qb + i) * seq + t] * kf[(size_t)(kb + i) * seq + j];
                scores[j] = sum * scale;
            }
            softmax_row(probs, scores, seq);
            for (int i = 0; i < hd; i++) {
                float sum = 0;
                for (int j = 0; j < seq; j++) sum += probs[j] * vf[(size_t)(kb + i) * seq + j];
                out[(size_t)(qb + i) * seq + t] = sum;
            }
        }
        free(scores);
        free(probs);
    }
}

/* cpu.go:97-111 RMSNorm: float64 rrms and a float64 product rounded once */
static void rms_norm_final_cf(float *out, const float *x, const float *w, int d, int s,
                              double eps) {
    for (int t = 0; t < s; t++) {
        double sum = 0;
        for (int i = 0; i < d; i++) {
            double v = (double)x[(size_t)i * s + t];
            sum += v * v;
        }
        double rrms = 1.0 / sqrt(sum / (double)d + eps);
        for (int i = 0; i < d; i++)
            out[(size_t)i * s + t] = (float)((double)x[(size_t)i * s + t] * rrms * (double)w[i]);
    }
}

/* cpu.go:276-300 MatMulVocabSeq: logits[v*S+t] = sum over d in order of E[v,d]*x[d*S+t] */
static void matmul_vocab_seq(float *logits, const float *embed, const float *x, int vocab,
                             int dim, int seq, int threads) {
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int v = 0; v < vocab; v++) {
        float *acc = logits + (size_t)v * seq;
        const float *eb = embed + (size_t)v * dim;
        for (int t = 0; t < seq; t++) acc[t] = 0;
        for (int d = 0; d < dim; d++) {
            float wv = eb[d];
            const float *xd = x + (size_t)d * seq;
            for (int t = 0; t < seq; t++) acc[t] += wv * xd[t];
        }
    }
}

/* One layer of evalLogitsCPUInto (engine.go:815-838): x_cf [D,S] -> out_cf [D,S] at
 * positions 0..S-1. out_cf may not alias x_cf. */
void or_layer_forward_cf(const or_config *cfg, const or_layer *L, const float *x_cf, int seq,
                         float *out_cf, int threads) {
    or_layer_forward_cf_taps(cfg, L, x_cf, seq, out_cf, NULL, NULL, threads);
}

/* The layer above, also copying its intermediates out channel-first, in the output order of
 * the reference's fused ANE programs: sdpa_taps = concat(x2, q_rope, k_rope, v, att_out)
 * (GenStoriesSDPAForwardDynamicTaps, ane/mil/stories_dynamic.go:162), ffn_taps =
 * concat(x_next, h1, h3) (GenStoriesFFNForwardDynamicTaps, :222). Either may be NULL. */
void or_layer_forward_cf_taps(const or_config *cfg, const or_layer *L, const float *x_cf, int seq,
                              float *out_cf, float *sdpa_taps, float *ffn_taps, int threads) {
    int D = cfg->dim, F = cfg->hidden, H = cfg->n_heads, KVH = cfg->n_kv_heads;
    int hd = cfg->head_dim, qd = H * hd, kvd = KVH * hd;
    size_t S = (size_t)seq;
    float alpha = cfg->residual_scale;
    float *xn = (float *)malloc(sizeof(float) * D * S);
    float *qf = (float *)malloc(sizeof(float) * qd * S);
    float *kf = (float *)malloc(sizeof(float) * kvd * S);
    float *vf = (float *)malloc(sizeof(float) * kvd * S);
    float *att = (float *)malloc(sizeof(float) * qd * S);
    float *x2 = (float *)malloc(sizeof(float) * D * S);
    float *h1 = (float *)malloc(sizeof(float) * F * S);
    float *h3 = (float *)malloc(sizeof(float) * F * S);
    float *gate = (float *)malloc(sizeof(float) * F * S);
    float *ff = (float *)malloc(sizeof(float) * D * S);
    float *rc = (float *)malloc(sizeof(float) * S * (hd / 2));
    float *rs = (float *)malloc(sizeof(float) * S * (hd / 2));
    or_rope_tables(rc, rs, seq, hd, cfg->rope_theta);            /* engine.go:218 */
    rms_norm_cf(xn, x_cf, L->rms_att, D, seq, cfg->norm_eps);
    linear_cf(qf, L->wq, xn, qd, D, seq, threads);
    linear_cf(kf, L->wk, xn, kvd, D, seq, threads);
    if (cfg->qk_norm) {
        qk_norm_cf(qf, H, hd, seq, L->q_norm, cfg->qk_norm_eps);
        qk_norm_cf(kf, KVH, hd, seq, L->k_norm, cfg->qk_norm_eps);
    }
    rope_cf(qf, H, hd, seq, rc, rs);
    rope_cf(kf, KVH, hd, seq, rc, rs);
    linear_cf(vf, L->wv, xn, kvd, D, seq, threads);
    causal_attention_cf(att, qf, kf, vf, H, KVH, hd, seq, threads);
    linear_cf(x2, L->wo, att, D, qd, seq, threads);
    for (size_t i = 0; i < D * S; i++) x2[i] = x_cf[i] + alpha * x2[i];   /* residual.go:19 */
    rms_norm_cf(xn, x2, L->rms_ffn, D, seq, cfg->norm_eps);
    linear_cf(h1, L->w1, xn, F, D, seq, threads);
    linear_cf(h3, L->w3, xn, F, D, seq, threads);
    for (size_t i = 0; i < F * S; i++) {                    /* accel_other.go:128-133 */
        float sig = (float)(1.0 / (1.0 + exp((double)(-h1[i]))));
        gate[i] = (h1[i] * sig) * h3[i];
    }
    linear_cf(ff, L->w2, gate, D, F, seq, threads);
    for (size_t i = 0; i < D * S; i++) out_cf[i] = x2[i] + alpha * ff[i];
    if (sdpa_taps) {
        float *t = sdpa_taps;
        memcpy(t, x2, sizeof(float) * D * S); t += D * S;
        memcpy(t, qf, sizeof(float) * qd * S); t += qd * S;
        memcpy(t, kf, sizeof(float) * kvd * S); t += kvd * S;
        memcpy(t, vf, sizeof(float) * kvd * S); t += kvd * S;
        memcpy(t, att, sizeof(float) * qd * S);
    }
    if (ffn_taps) {
        memcpy(ffn_taps, out_cf, sizeof(float) * D * S);
        memcpy(ffn_taps + D * S, h1, sizeof(float) * F * S);
        memcpy(ffn_taps + (D + (size_t)F) * S, h3, sizeof(float) * F * S);
    }
    free(xn); free(qf); free(kf); free(vf); free(att); free(x2);
    free(h1); free(h3); free(gate); free(ff); free(rc); free(rs);
}

void or_rms_norm_final_cf(float *out, const float *x, const float *w, int dim, int seq,
                          double eps) {
    rms_norm_final_cf(out, x, w, dim, seq, eps);
}

void or_matmul_vocab_seq(float *logits, const float *embed, const float *x, int vocab, int dim,
                         int seq, int threads) {
    matmul_vocab_seq(logits, embed, x, vocab, dim, seq, threads);
}

void or_linear_cf(float *out, const float *w, const float *in, int out_ch, int in_ch, int seq,
                  int threads) {
    linear_cf(out, w, in, out_ch, in_ch, seq, threads);
}

static void eval_logits_cf(const or_config *cfg, const or_weights *w, const uint16_t *tokens, int seq,
                           float *logits_cf, int layer_threads, int threads);

void or_eval_logits_cf(const or_config *cfg, const or_weights *w, const uint16_t *tokens,
                       int seq, float *logits_cf, int threads) {
    eval_logits_cf(cfg, w, tokens, seq, logits_cf, threads, threads);
}

/* The same forward with the reference's threading, for timing it as the reference runs:
 * linearCF and causalAttentionCF serial (forward_common.go:5-46), the vocabulary product over
 * `threads` (MatMulVocabSeq's parallelFor over V, cpu.go:276-300). (RMSNorm, which the reference
 * also spreads over GOMAXPROCS, stays serial here: under 0.1% of the forward's work.) */
void or_eval_logits_cf_ref_threads(const or_config *cfg, const or_weights *w, const uint16_t *tokens,
                                   int seq, float *logits_cf, int threads) {
    eval_logits_cf(cfg, w, tokens, seq, logits_cf, 1, threads);
}

static void eval_logits_cf(const or_config *cfg, const or_weights *w, const uint16_t *tokens, int seq,
                           float *logits_cf, int layer_threads, int threads) {
    int D = cfg->dim;
    size_t S = (size_t)seq;
    float *x = (float *)malloc(sizeof(float) * D * S);
    float *next = (float *)malloc(sizeof(float) * D * S);
    or_embed_lookup_cf(x, w->embed, cfg->vocab, tokens, D, seq);
    for (int l = 0; l < cfg->n_layers; l++) {
        or_layer_forward_cf(cfg, &w->layers[l], x, seq, next, layer_threads);
        float *tmp = x; x = next; next = tmp;   /* cur and next swap every layer */
    }
    rms_norm_final_cf(next, x, w->rms_final, D, seq, cfg->norm_eps);
    matmul_vocab_seq(logits_cf, w->cls ? w->cls : w->embed, next, cfg->vocab, D, seq, threads);
    free(x); free(next);
}

/* decode.go:83-94 fillDecodeWindow: BOS-left-pad the last `seq` tokens */
void or_fill_decode_window(uint16_t *dst, int seq, const int32_t *tokens, int n) {
    for (int i = 0; i < seq; i++) dst[i] = OR_BOS;
    if (n >= seq) { tokens += n - seq; n = seq; }
    int start = seq - n;
    for (int i = 0; i < n; i++) dst[start + i] = (uint16_t)tokens[i];
}

/* ------------------------------------------------------------------------------------ */
/* Training step: ane/storiesane/train_full.go (CPU path), loss.go, rmsnorm.go,          */
/* accel_other.go, ane/stories/cpu.go. Channel-first [C, S] like the reference.          */

/* cpu.go:74-95 EmbedBackward: dEmbed[tok*D+d] += dx[d*S+t] for in-range ids */
void or_embed_backward(float *dembed, const float *dx, const uint16_t *tokens, int vocab,
                       int dim, int seq) {
    for (int t = 0; t < seq; t++) {
        int tok = tokens[t];
        if (tok >= vocab) continue;
        for (int d = 0; d < dim; d++) dembed[(size_t)tok * dim + d] += dx[(size_t)d * seq + t];
    }
}

/* accel_other.go:11-28 rmsNormCFWithRRMSImpl, keeping the per-token scale */
static void rms_norm_cf_rrms(float *out, float *rrms, const float *x, const float *w, int dim,
                             int seq, double eps) {
    for (int t = 0; t < seq; t++) {
        double sum = 0;
        for (int i = 0; i < dim; i++) {
            double v = (double)x[(size_t)i * seq + t];
            sum += v * v;
        }
        float scale = (float)(1.0 / sqrt(sum / (double)dim + eps));
        rrms[t] = scale;
        for (int i = 0; i < dim; i++)
            out[(size_t)i * seq + t] = x[(size_t)i * seq + t] * scale * w[i];
    }
}

/* train_full.go:228-245 linearBackwardDXCF: dx[i*S+t] = sum over o in order of W[o,i]*dy[o*S+t] */
static void linear_backward_dx_cf(float *dx, const float *w, const float *dy, int out_ch,
                                  int in_ch, int seq, int threads) {
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int i = 0; i < in_ch; i++) {
        float *row = dx + (size_t)i * seq;
        for (int t = 0; t < seq; t++) row[t] = 0;
        for (int o = 0; o < out_ch; o++) {
            float wt = w[(size_t)o * in_ch + i];
            const float *dyr = dy + (size_t)o * seq;
            for (int t = 0; t < seq; t++) row[t] += wt * dyr[t];
        }
    }
}

/* train_full.go:199-217 accumLinearGradCF: dW[o,i] += sum over t in order of dy[o*S+t]*x[i*S+t] */
static void accum_linear_grad_cf(float *dw, const float *dy, const float *x, int out_ch,
                                 int in_ch, int seq, int threads) {
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int o = 0; o < out_ch; o++) {
        const float *dyr = dy + (size_t)o * seq;
        for (int i = 0; i < in_ch; i++) {
            const float *xr = x + (size_t)i * seq;
            float sum = 0;
            for (int t = 0; t < seq; t++) sum += dyr[t] * xr[t];
            dw[(size_t)o * in_ch + i] += sum;
        }
    }
}

/* train_full.go:247-301 causalAttentionBackwardCF. Gradients of the post-RoPE q and k (the
 * reference does not rotate them back); heads are independent, so they run in parallel. */
static void causal_attention_backward_cf(float *dq, float *dk, float *dv, const float *dout,
                                         const float *q, const float *k, const float *v,
                                         int heads, int hd, int seq, int threads) {
    size_t n = (size_t)heads * hd * seq;
    memset(dq, 0, sizeof(float) * n);
    memset(dk, 0, sizeof(float) * n);
    memset(dv, 0, sizeof(float) * n);
    float scale = (float)(1.0 / sqrt((double)hd));
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int h = 0; h < heads; h++) {
        float *scores = (float *)malloc(sizeof(float) * seq);
        float *probs = (float *)malloc(sizeof(float) * seq);
        float *dscores = (float *)malloc(sizeof(float) * seq);
        int base = h * hd;
        for (int t = 0; t < seq; t++) {
            float maxv = -INFINITY;
            for (int s = 0; s <= t; s++) {
                float sum = 0;
                for (int i = 0; i < hd; i++)
                    sum += q[(size_t)(base + i) * seq + t] * k[(size_t)(base + i) * seq + s];
                scores[s] = sum * scale;
                if (scores[s] > maxv) maxv = scores[s];
            }
            double total = 0;
            for (int s = 0; s <= t; s++) {
                double e = exp((double)(scores[s] - maxv));
                probs[s] = (float)e;
                total += e;
            }
            float inv_total = (float)(1.0 / total);
            for (int s = 0; s <= t; s++) probs[s] *= inv_total;
            float ds_sum = 0;
            for (int s = 0; s <= t; s++) {
                float dot = 0;
                for (int i = 0; i < hd; i++)
                    dot += dout[(size_t)(base + i) * seq + t] * v[(size_t)(base + i) * seq + s];
                dscores[s] = dot;
                ds_sum += probs[s] * dot;
            }
            for (int s = 0; s <= t; s++) {
                float ds = probs[s] * (dscores[s] - ds_sum) * scale;
                for (int i = 0; i < hd; i++) {
                    size_t qi = (size_t)(base + i) * seq;
                    dq[qi + t] += ds * k[qi + s];
                    dk[qi + s] += ds * q[qi + t];
                    dv[qi + s] += probs[s] * dout[qi + t];
                }
            }
        }
        free(scores);
        free(probs);
        free(dscores);
    }
}

/* accel_other.go:77-84 siluBackwardAccel */
static void silu_backward(float *dh1, float *dh3, const float *dgate, const float *h1,
                          const float *h3, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float sig = (float)(1.0 / (1.0 + exp((double)(-h1[i]))));
        float silu_grad = sig * (1 + h1[i] * (1 - sig));
        dh1[i] = dgate[i] * h3[i] * silu_grad;
        dh3[i] = dgate[i] * (h1[i] * sig);
    }
}

/* rmsnorm.go:32-47 rmsNormBackwardWithRRMS: dx[i,t] = (dy - x*dot*r^2/d) * r * w (float64),
 * dot = sum_i dy*x*w, dw[i] += float32(float64(dy*x) * r), t in order for each i. The exact
 * gradient's second term carries no w[i] factor: this form equals it for unit gains only. */
void or_rms_norm_backward_cf(float *dx, float *dw, const float *dy, const float *x,
                             const float *w, const float *rrms, int d, int s, int threads);
static void rms_norm_backward_cf(float *dx, float *dw, const float *dy, const float *x,
                                 const float *w, const float *rrms, int d, int s, int threads) {
    or_rms_norm_backward_cf(dx, dw, dy, x, w, rrms, d, s, threads);
}
void or_rms_norm_backward_cf(float *dx, float *dw, const float *dy, const float *x,
                             const float *w, const float *rrms, int d, int s, int threads) {
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int t = 0; t < s; t++) {
        double r = (double)rrms[t];
        double r2 = (r * r) / (double)d;
        double dot = 0;
        for (int i = 0; i < d; i++)
            dot += (double)(dy[(size_t)i * s + t] * x[(size_t)i * s + t] * w[i]);
        for (int i = 0; i < d; i++) {
            double v = (double)dy[(size_t)i * s + t] - (double)x[(size_t)i * s + t] * dot * r2;
            dx[(size_t)i * s + t] = (float)(v * r * (double)w[i]);
        }
    }
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int i = 0; i < d; i++)
        for (int t = 0; t < s; t++)
            dw[i] += (float)((double)(dy[(size_t)i * s + t] * x[(size_t)i * s + t]) * (double)rrms[t]);
}

/* cpu.go:173-253 CrossEntropyLoss: column softmax (float32 exp terms summed in float64),
 * loss -= log(max(p, 1e-10)) at the target, dLogits = probs - onehot, columns of invalid
 * targets zeroed, valid columns scaled by 1/valid. Returns the mean loss. */
float or_cross_entropy_loss(float *dlogits, const float *logits, const uint16_t *targets,
                            int v, int s) {
    double loss = 0;
    int valid = 0;
    for (int t = 0; t < s; t++) {
        float mx = logits[t];
        for (int i = 1; i < v; i++)
            if (logits[(size_t)i * s + t] > mx) mx = logits[(size_t)i * s + t];
        double sum = 0;
        for (int i = 0; i < v; i++) {
            float e = (float)exp((double)(logits[(size_t)i * s + t] - mx));
            dlogits[(size_t)i * s + t] = e;
            sum += (double)e;
        }
        float inv = (float)(1.0 / sum);
        int tgt = targets[t];
        for (int i = 0; i < v; i++) dlogits[(size_t)i * s + t] *= inv;
        if (tgt < 0 || tgt >= v) {
            for (int i = 0; i < v; i++) dlogits[(size_t)i * s + t] = 0;
            continue;
        }
        float p = dlogits[(size_t)tgt * s + t];
        if (p < 1e-10f) p = 1e-10f;
        loss -= log((double)p);
        dlogits[(size_t)tgt * s + t] -= 1;
        valid++;
    }
    if (valid == 0) return 0;
    float inv_valid = (float)(1.0 / (double)valid);
    for (int t = 0; t < s; t++) {
        int tgt = targets[t];
        if (tgt < 0 || tgt >= v) continue;
        for (int i = 0; i < v; i++) dlogits[(size_t)i * s + t] *= inv_valid;
    }
    return (float)(loss / (double)valid);
}

/* cpu.go:306-333 MatMulEmbedTScale: dx[d*S+t] = (sum over v in order of E[v,d]*dL[v*S+t]) * scale */
static void matmul_embed_t_scale(float *dx, const float *embed, const float *dl, int vocab,
                                 int dim, int seq, float scale, int threads) {
    if (scale == 0) {
        memset(dx, 0, sizeof(float) * (size_t)dim * seq);
        return;
    }
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int d = 0; d < dim; d++) {
        float *acc = dx + (size_t)d * seq;
        for (int t = 0; t < seq; t++) acc[t] = 0;
        for (int vv = 0; vv < vocab; vv++) {
            float wv = embed[(size_t)vv * dim + d];
            const float *dlv = dl + (size_t)vv * seq;
            for (int t = 0; t < seq; t++) acc[t] += wv * dlv[t];
        }
        for (int t = 0; t < seq; t++) acc[t] = acc[t] * scale;
    }
}

/* train_full.go:525-587 compactEmbedGrad with cpu.go:339-358 MatMulGradEmbedScale: the
 * classifier's embedding gradient, rows of the distinct in-range target ids only,
 * g[v,d] = (sum over t in order of dL[v*S+t]*x[d*S+t]) * scale; every other row 0. The full
 * product replaces it when the distinct ids exceed half of stories.Vocab (32000). */
static void compact_embed_grad(float *gembed, const float *dl, const float *xnorm,
                               const uint16_t *targets, int vocab, int dim, int seq,
                               float scale, int threads) {
    memset(gembed, 0, sizeof(float) * (size_t)vocab * dim);
    if (scale == 0) return;
    unsigned char *seen = (unsigned char *)calloc((size_t)vocab, 1);
    int *rows = (int *)malloc(sizeof(int) * (size_t)(seq > 0 ? seq : 1));
    int n = 0;
    for (int t = 0; t < seq; t++) {
        int tok = targets[t];
        if (tok >= vocab || seen[tok]) continue;
        seen[tok] = 1;
        rows[n++] = tok;
    }
    int full = n <= 0 || n > 32000 / 2;
    int nr = full ? vocab : n;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int r = 0; r < nr; r++) {
        int vv = full ? r : rows[r];
        for (int d = 0; d < dim; d++) {
            float sum = 0;
            for (int t = 0; t < seq; t++)
                sum += dl[(size_t)vv * seq + t] * xnorm[(size_t)d * seq + t];
            gembed[(size_t)vv * dim + d] = sum * scale;
        }
    }
    free(seen);
    free(rows);
}

/* train_full.go:926-969 adamBiasCorrectionInv + adamUpdateCFWithInv */
static void adam_update(float *w, const float *g, float *m, float *v, size_t n, float lr,
                        float b1, float b2, float eps, float wd, float inv_bc1, float inv_bc2) {
    for (size_t i = 0; i < n; i++) {
        m[i] = b1 * m[i] + (1 - b1) * g[i];
        v[i] = b2 * v[i] + (1 - b2) * g[i] * g[i];
        float mh = m[i] * inv_bc1;
        float vh = v[i] * inv_bc2;
        float update = mh / ((float)sqrt((double)vh) + eps);
        if (wd != 0) update += wd * w[i];
        w[i] -= lr * update;
    }
}

static void scale_slice(float *v, size_t n, float s) {
    for (size_t i = 0; i < n; i++) v[i] *= s;
}

static double sum_squares(const float *v, size_t n) {
    double s = 0;
    for (size_t i = 0; i < n; i++) s += (double)v[i] * (double)v[i];
    return s;
}

/* Tensors of one layer in the order or_train_layer lists them, with their element counts. */
static void train_layer_tensors(const or_config *cfg, or_train_layer *l, float **p, size_t *n) {
    size_t D = cfg->dim, F = cfg->hidden;
    p[0] = l->wq; n[0] = D * D;
    p[1] = l->wk; n[1] = D * D;
    p[2] = l->wv; n[2] = D * D;
    p[3] = l->wo; n[3] = D * D;
    p[4] = l->w1; n[4] = F * D;
    p[5] = l->w2; n[5] = D * F;
    p[6] = l->w3; n[6] = F * D;
    p[7] = l->rms_att; n[7] = D;
    p[8] = l->rms_ffn; n[8] = D;
}

/* Forward, final head and backward of one window (train_full.go:368-396, :435-523 and the
 * layer loops of :709-774 / :776-848, CPU path). accumulate == 0: grads receives this window's
 * gradients (clearLayerGrad, train_full.go:783). accumulate != 0: grads is the accumulator;
 * layer gradients add onto it in place, the final-gain and embedding gradients of the window are
 * formed on their own and then added (addSlice, train_full.go:767-768). Returns the loss. */
static float train_gradients(const or_config *cfg, const or_train_params *p, or_train_params *grads,
                             const or_train_hparams *hp, const uint16_t *input,
                             const uint16_t *target, int seq, int accumulate, int threads) {
    const int D = cfg->dim, F = cfg->hidden, H = cfg->n_heads, hd = cfg->head_dim;
    const int V = cfg->vocab, L = cfg->n_layers;
    const size_t S = (size_t)seq, DS = (size_t)D * S, FS = (size_t)F * S;
    const float alpha = cfg->residual_scale;
    const double eps = cfg->norm_eps;
    /* per-layer caches (train_full.go:46-70 newLayerCache) */
    float *cache = (float *)malloc(sizeof(float) * (size_t)L * (11 * DS + 3 * FS + 2 * S));
    float *c = cache;
#define TAKE(n) (c += (n), c - (n))
    float *rc = (float *)malloc(sizeof(float) * S * (hd / 2));
    float *rs = (float *)malloc(sizeof(float) * S * (hd / 2));
    or_rope_tables(rc, rs, seq, hd, cfg->rope_theta);   /* rope.go:5-24 buildRoPETables */
    typedef struct { float *x, *xn, *q, *k, *v, *att, *x2, *x2n, *h1, *h3, *gate, *ra, *rf; } lc;
    lc *lcs = (lc *)malloc(sizeof(lc) * L);
    float *cur = (float *)malloc(sizeof(float) * DS), *next = (float *)malloc(sizeof(float) * DS);
    float *tmp = (float *)malloc(sizeof(float) * DS);
    /* forwardTrainingCPU (train_full.go:368-396) */
    or_embed_lookup_cf(cur, p->embed, V, input, D, seq);
    for (int l = 0; l < L; l++) {
        lc *C = &lcs[l];
        or_train_layer *W = &p->layers[l];
        C->x = TAKE(DS); C->xn = TAKE(DS); C->q = TAKE(DS); C->k = TAKE(DS); C->v = TAKE(DS);
        C->att = TAKE(DS); C->x2 = TAKE(DS); C->x2n = TAKE(DS); C->h1 = TAKE(FS); C->h3 = TAKE(FS);
        C->gate = TAKE(FS); C->ra = TAKE(S); C->rf = TAKE(S);
        memcpy(C->x, cur, sizeof(float) * DS);
        rms_norm_cf_rrms(C->xn, C->ra, C->x, W->rms_att, D, seq, eps);
        linear_cf(C->q, W->wq, C->xn, D, D, seq, threads);
        linear_cf(C->k, W->wk, C->xn, D, D, seq, threads);
        rope_cf(C->q, H, hd, seq, rc, rs);
        rope_cf(C->k, H, hd, seq, rc, rs);
        linear_cf(C->v, W->wv, C->xn, D, D, seq, threads);
        causal_attention_cf(C->att, C->q, C->k, C->v, H, H, hd, seq, threads);
        linear_cf(next, W->wo, C->att, D, D, seq, threads);
        for (size_t i = 0; i < DS; i++) C->x2[i] = C->x[i] + alpha * next[i];   /* residual.go:19 */
        rms_norm_cf_rrms(C->x2n, C->rf, C->x2, W->rms_ffn, D, seq, eps);
        linear_cf(C->h1, W->w1, C->x2n, F, D, seq, threads);
        linear_cf(C->h3, W->w3, C->x2n, F, D, seq, threads);
        for (size_t i = 0; i < FS; i++) {                    /* accel_other.go:70-75 */
            float sig = (float)(1.0 / (1.0 + exp((double)(-C->h1[i]))));
            C->gate[i] = (C->h1[i] * sig) * C->h3[i];
        }
        linear_cf(next, W->w2, C->gate, D, F, seq, threads);
        for (size_t i = 0; i < DS; i++) next[i] = C->x2[i] + alpha * next[i];
        float *sw = cur; cur = next; next = sw;
    }
    /* runFinalHead, CPU path (train_full.go:435-523) */
    float *xnf = (float *)malloc(sizeof(float) * DS), *rfin = (float *)malloc(sizeof(float) * S);
    float *logits = (float *)malloc(sizeof(float) * (size_t)V * S);
    rms_norm_cf_rrms(xnf, rfin, cur, p->rms_final, D, seq, eps);
    matmul_vocab_seq(logits, p->embed, xnf, V, D, seq, threads);
    float loss = or_cross_entropy_loss(logits, logits, target, V, seq);
    const float grad_scale = hp->loss_scale;   /* scale = 1 (logits already scaled) x loss scale */
    float *dy = (float *)malloc(sizeof(float) * DS), *dcur = (float *)malloc(sizeof(float) * DS);
    float *dprev = (float *)malloc(sizeof(float) * DS);
    or_train_params *g = grads;
    /* the window's own final-gain and embedding gradients (e.gRMS, e.gEmbed) */
    float *g_rms = accumulate ? (float *)malloc(sizeof(float) * D) : g->rms_final;
    float *g_emb = accumulate ? (float *)malloc(sizeof(float) * (size_t)V * D) : g->embed;
    memset(g_rms, 0, sizeof(float) * D);
    matmul_embed_t_scale(dy, p->embed, logits, V, D, seq, grad_scale, threads);
    compact_embed_grad(g_emb, logits, xnf, target, V, D, seq, grad_scale, threads);
    rms_norm_backward_cf(dcur, g_rms, dy, cur, p->rms_final, rfin, D, seq, threads);
    /* backwardAndApply, CPU path (train_full.go:776-848) */
    float *dout = (float *)malloc(sizeof(float) * DS), *gx2 = (float *)malloc(sizeof(float) * DS);
    float *dx2s = (float *)malloc(sizeof(float) * DS), *gxn = (float *)malloc(sizeof(float) * DS);
    float *ggate = (float *)malloc(sizeof(float) * FS), *gh1 = (float *)malloc(sizeof(float) * FS);
    float *gh3 = (float *)malloc(sizeof(float) * FS), *gatt = (float *)malloc(sizeof(float) * DS);
    float *gq = (float *)malloc(sizeof(float) * DS), *gk = (float *)malloc(sizeof(float) * DS);
    float *gv = (float *)malloc(sizeof(float) * DS);
    for (int l = L - 1; l >= 0; l--) {
        lc *C = &lcs[l];
        or_train_layer *W = &p->layers[l], *G = &g->layers[l];
        float *gt[9];
        size_t gn[9];
        train_layer_tensors(cfg, G, gt, gn);
        if (!accumulate)
            for (int i = 0; i < 9; i++) memset(gt[i], 0, sizeof(float) * gn[i]);   /* clearLayerGrad */
        for (size_t i = 0; i < DS; i++) dout[i] = dcur[i] * alpha;           /* scaleInto */
        /* backwardFFNCPU (train_full.go:618-627) */
        memcpy(gx2, dcur, sizeof(float) * DS);
        linear_backward_dx_cf(ggate, W->w2, dout, D, F, seq, threads);
        silu_backward(gh1, gh3, ggate, C->h1, C->h3, FS);
        linear_backward_dx_cf(gxn, W->w1, gh1, F, D, seq, threads);
        linear_backward_dx_cf(dprev, W->w3, gh3, F, D, seq, threads);
        for (size_t i = 0; i < DS; i++) gxn[i] += dprev[i];
        rms_norm_backward_cf(dprev, G->rms_ffn, gxn, C->x2, W->rms_ffn, C->rf, D, seq, threads);
        for (size_t i = 0; i < DS; i++) gx2[i] += dprev[i];
        accum_linear_grad_cf(G->w2, dout, C->gate, D, F, seq, threads);
        accum_linear_grad_cf(G->w1, gh1, C->x2n, F, D, seq, threads);
        accum_linear_grad_cf(G->w3, gh3, C->x2n, F, D, seq, threads);
        for (size_t i = 0; i < DS; i++) dx2s[i] = gx2[i] * alpha;
        /* backwardAttentionCPU (train_full.go:674-693) */
        linear_backward_dx_cf(gatt, W->wo, dx2s, D, D, seq, threads);
        causal_attention_backward_cf(gq, gk, gv, gatt, C->q, C->k, C->v, H, hd, seq, threads);
        linear_backward_dx_cf(gxn, W->wq, gq, D, D, seq, threads);
        linear_backward_dx_cf(dprev, W->wk, gk, D, D, seq, threads);
        for (size_t i = 0; i < DS; i++) gxn[i] += dprev[i];
        linear_backward_dx_cf(dprev, W->wv, gv, D, D, seq, threads);
        for (size_t i = 0; i < DS; i++) gxn[i] += dprev[i];
        rms_norm_backward_cf(dprev, G->rms_att, gxn, C->x, W->rms_att, C->ra, D, seq, threads);
        for (size_t i = 0; i < DS; i++) dprev[i] += gx2[i];
        accum_linear_grad_cf(G->wo, dx2s, C->att, D, D, seq, threads);
        accum_linear_grad_cf(G->wq, gq, C->xn, D, D, seq, threads);
        accum_linear_grad_cf(G->wk, gk, C->xn, D, D, seq, threads);
        accum_linear_grad_cf(G->wv, gv, C->xn, D, D, seq, threads);
        float *sw = dcur; dcur = dprev; dprev = sw;
    }
    or_embed_backward(g_emb, dcur, input, V, D, seq);
    if (accumulate) {
        for (int i = 0; i < D; i++) g->rms_final[i] += g_rms[i];
        for (size_t i = 0; i < (size_t)V * D; i++) g->embed[i] += g_emb[i];
        free(g_rms);
        free(g_emb);
    }
#undef TAKE
    free(cache); free(rc); free(rs); free(lcs); free(cur); free(next); free(tmp); free(xnf);
    free(rfin); free(logits); free(dy); free(dcur); free(dprev); free(dout); free(gx2); free(dx2s);
    free(gxn); free(ggate); free(gh1); free(gh3); free(gatt); free(gq); free(gk); free(gv);
    return loss;
}

/* Every gradient tensor of the model scaled by s (scaleModelGrad, train_full.go:133-139). */
static void scale_all(const or_config *cfg, or_train_params *g, float s) {
    for (int l = 0; l < cfg->n_layers; l++) {
        float *gt[9];
        size_t gn[9];
        train_layer_tensors(cfg, &g->layers[l], gt, gn);
        for (int i = 0; i < 9; i++) scale_slice(gt[i], gn[i], s);
    }
    scale_slice(g->rms_final, cfg->dim, s);
    scale_slice(g->embed, (size_t)cfg->vocab * cfg->dim, s);
}

/* clipLayerGradients (train_full.go:149-181), then Adam at 1-based step step_t
 * (adamBiasCorrectionInv / adamUpdateCFWithInv, :926-969; applyLayerAdamAll, :875-924). */
static void clip_and_adam(const or_config *cfg, or_train_params *p, or_train_params *m,
                          or_train_params *v, or_train_params *g, const or_train_hparams *hp,
                          int step_t, int apply) {
    const int D = cfg->dim, V = cfg->vocab, L = cfg->n_layers;
    if (hp->grad_clip > 0) {
        double norm2 = 0;
        for (int l = 0; l < L; l++) {
            float *gt[9];
            size_t gn[9];
            train_layer_tensors(cfg, &g->layers[l], gt, gn);
            for (int i = 0; i < 9; i++) norm2 += sum_squares(gt[i], gn[i]);
        }
        norm2 += sum_squares(g->rms_final, D);
        norm2 += sum_squares(g->embed, (size_t)V * D);
        if (norm2 > 0) {
            float norm = (float)sqrt(norm2);
            if (norm > hp->grad_clip) scale_all(cfg, g, hp->grad_clip / norm);
        }
    }
    if (!apply) return;
    float inv_bc1 = 1 / (float)(1.0 - pow((double)hp->beta1, (double)step_t));
    float inv_bc2 = 1 / (float)(1.0 - pow((double)hp->beta2, (double)step_t));
    for (int l = 0; l < L; l++) {
        float *pw[9], *gw[9], *mw[9], *vw[9];
        size_t n[9];
        train_layer_tensors(cfg, &p->layers[l], pw, n);
        train_layer_tensors(cfg, &g->layers[l], gw, n);
        train_layer_tensors(cfg, &m->layers[l], mw, n);
        train_layer_tensors(cfg, &v->layers[l], vw, n);
        for (int i = 0; i < 9; i++)
            adam_update(pw[i], gw[i], mw[i], vw[i], n[i], hp->lr, hp->beta1, hp->beta2, hp->eps,
                        i < 7 ? hp->weight_decay : 0, inv_bc1, inv_bc2);
    }
    adam_update(p->rms_final, g->rms_final, m->rms_final, v->rms_final, D, hp->lr, hp->beta1,
                hp->beta2, hp->eps, 0, inv_bc1, inv_bc2);
    adam_update(p->embed, g->embed, m->embed, v->embed, (size_t)V * D, hp->lr, hp->beta1,
                hp->beta2, hp->eps, hp->weight_decay, inv_bc1, inv_bc2);
}

float or_train_step(const or_config *cfg, or_train_params *p, or_train_params *m,
                    or_train_params *v, or_train_params *grads, const or_train_hparams *hp,
                    int step_t, const uint16_t *input, const uint16_t *target, int seq,
                    int apply, int threads) {
    float loss = train_gradients(cfg, p, grads, hp, input, target, seq, 0, threads);
    /* loss-scale undo (train_full.go:826-835) */
    if (hp->loss_scale != 0 && hp->loss_scale != 1)
        scale_all(cfg, grads, (float)(1.0 / (double)hp->loss_scale));
    clip_and_adam(cfg, p, m, v, grads, hp, step_t, apply);
    return loss;
}

float or_train_accumulate(const or_config *cfg, const or_train_params *p, or_train_params *accum,
                          const or_train_hparams *hp, const uint16_t *input,
                          const uint16_t *target, int seq, int threads) {
    return train_gradients(cfg, p, accum, hp, input, target, seq, 1, threads);
}

void or_train_flush(const or_config *cfg, or_train_params *p, or_train_params *m,
                    or_train_params *v, or_train_params *accum, const or_train_hparams *hp,
                    int step_t, int pending) {
    if (pending <= 0) return;
    /* engine.go:544-547: float32(1/pending), then divided by the loss scale in float32 */
    float s = (float)(1.0 / (double)pending);
    if (hp->loss_scale > 0) s /= hp->loss_scale;
    scale_all(cfg, accum, s);
    clip_and_adam(cfg, p, m, v, accum, hp, step_t, 1);
}

/* engine.go:725-732 drand48Seed / nextFloat64, and Step's window choice (engine.go:307-316):
 * returns the start of the next (input, target) window of `seq` tokens in a stream of n. */
uint64_t or_drand48_seed(int64_t seed) { return (((uint64_t)seed & 0xffffffffull) << 16) | 0x330E; }
double or_drand48_next(uint64_t *state) {
    *state = (0x5DEECE66Dull * *state + 0xBull) & ((1ull << 48) - 1);
    return (double)*state / (double)(1ull << 48);
}
uint64_t or_train_window(uint64_t *state, int64_t n_tokens, int seq) {
    uint64_t limit = (uint64_t)(n_tokens - seq - 1), pos = 0;
    if (limit > 0) {
        pos = (uint64_t)(or_drand48_next(state) * (double)limit);
        if (pos >= limit) pos = limit - 1;
    }
    return pos;
}
