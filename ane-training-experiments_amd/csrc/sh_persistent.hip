// sh_persistent.hip — the whole greedy decode loop as one persistent kernel for gfx950.
//
// Why: one token forward (ane/stories/infer.go:204-245) is ~5 dependent GEMV-sized stages
// per layer. Launched as separate kernels, even inside a HIP graph, each stage pays ~1.6 us
// of dispatch; a grid-wide atomic barrier costs more. Here every workgroup stays resident
// for all forwards and the stages hand data over through "LL" words: each element of an
// inter-stage vector is one 64-bit word (float bits | 32-bit epoch) written with a single
// agent-scope store, so a consumer that reads the expected epoch also holds the value; no
// fences or counters are needed. Epochs are unique per (forward, layer), so buffers are
// never cleared.
//
// Stages of one forward (each GEMV stage on its own range of workgroups, which own blocks
// of consecutive rows; persistent_plan places them):
//   per layer l (epoch e):
//     qkv   rows of [Wq;Wk;Wv] . rmsnorm(x)          -> ll_qkv
//     attn  per kv head g: QK-norm, RoPE, KV append, softmax, P.V for its q heads
//           (the 16-bit 128-dim-head shape: per q head)  -> ll_att      (workgroups 0..NA-1)
//     wo    x2 = x + alpha * Wo . att                -> ll_x2
//     w13   gate = silu(W1 . n) * (W3 . n), n = rmsnorm(x2) -> ll_gate (every workgroup)
//     w2    x = x2 + alpha * W2 . gate               -> ll_x
//   classifier: logits = Cls . rmsnorm(x), per-workgroup (max, first index) -> ll_pv/ll_pi
//   argmax: every workgroup reduces the partials itself and knows the next token.
// Layer 0 reads x straight from the embedding row, so it needs no hand-over.
//
// Weight tiles of a stage are loaded into registers before the stage's input is polled,
// so HBM streaming overlaps the hand-over latency. Each kv head's cache rows are written
// and read by the same workgroup (same CU), so the cache needs no cross-CU coherence.
// A consumer polls only when it has outputs to produce in that stage; every produced
// element is consumed downstream, so no buffer is overwritten before all its pollers read
// it. Every wait is bounded (spin_limit ticks of the constant-rate clock): on expiry the
// kernel sets *err and all workgroups exit.
#include <hip/hip_fp16.h>
#include <math.h>

#include <algorithm>
#include <string>

#include "sh_internal.hpp"
#include "sh_wave.hpp"

namespace sh {
namespace {

// Address-space-qualified pointers: weights and caches are global memory, staged rows are
// LDS. Without the qualifier, pointers fetched from memory compile to FLAT accesses.
#define SH_GLOBAL __attribute__((address_space(1)))
#define SH_LDS __attribute__((address_space(3)))

// Plain clang vectors: loadable through address-space-qualified pointers.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kPB = 512;           // threads per workgroup
constexpr int kPW = kPB / 64;      // waves per workgroup
constexpr int kXs = 4096;          // staged input vector
constexpr int kScores = 4096;      // attention scores: group * max_seq
constexpr int kMaxGroup = 2;       // q heads per kv head
constexpr int kMaxRes = 32;        // residual rows a workgroup owns in a residual stage
constexpr int kMaxPer = 256;       // rows a workgroup owns in a GEMV stage with hand-over output
constexpr int kKvStage = 96 * 1024; // LDS bytes for one kv head's cached K and V rows

struct LayerPtrs {
    const void *wqkv, *wo, *w13, *w2;          // fp16 / bf16 bits, or int8 (W8A8)
    const float *s_qkv, *s_o, *s_13, *s_2;     // W8A8 per-row weight scales
    const float *rms_att, *rms_ffn, *q_norm, *k_norm;
};

// The layer table is written by the host before the launch and only read by the kernel, so
// it is read through the constant address space: uniform scalar loads, which do not join the
// in-order vector memory counter. Read as vector loads, a pointer fetched after a stage's
// early weight loads would make the stage wait for those weights before its first poll.
__device__ __forceinline__ LayerPtrs layer_ptrs(const LayerPtrs *table, int l) {
#ifdef __HIP_DEVICE_COMPILE__
    return ((const __attribute__((address_space(4))) LayerPtrs *)table)[l];
#else
    return table[l];  // the host pass only parses device functions
#endif
}

struct PParams {
    int D, F, H, KVH, hd, V, max_seq, L, qdim, kvdim, qkv_rows;
    int NA;               // attention workgroups [0, NA): one per kv head, or per q head (split)
    float alpha, inv_sqrt_hd;
    double eps, qk_eps;
    int qk_norm;
    const LayerPtrs *layers;
    const uint16_t *embed;
    const void *cls;
    const float *s_cls;                        // W8A8 classifier row scales
    const float *rms_final;
    void *kcache, *vcache;
    const float *rope_cos, *rope_sin;
    uint64_t *ll_qkv, *ll_att, *ll_x2, *ll_gate, *ll_x, *ll_pv, *ll_pi;
    float *logits;
    int32_t *tokens, *hist;
    int pos0, n_forwards, n_prompt;
    uint32_t epoch0;
    // err[0]: 0, or how the launch ended early: kErrTimeout (a wait expired with every
    // workgroup started), kErrAbsent (a wait expired before every workgroup had started: not
    // all of the grid was resident); err[1]: workgroups started so far
    int *err;
    int fail_mode;     // testing aid: nonzero ends every workgroup at once with err[0] = fail_mode
    long long spin_limit;
    long long quiet;   // ticks a wait runs before it also reads the abort flag (20 us)
    long long *trace;  // forward trace_f: per workgroup 5L+3 stage-end stamps, then as many
                       // input-ready stamps (the stage's whole input staged on the workgroup)
    int trace_f;
    StageOwn own[5];   // qkv, wo, w13, w2, classifier
    StageOwn own_cls_a;   // classifier rows of the attention workgroups (n == 0: own[4])
    int cls_lds_rows;     // classifier rows a non-attention workgroup keeps in LDS (0: none)
    int argmax_every;     // the next-token exchange after every forward (w13 not on every workgroup)
    int ostride[5];    // words between consecutive workgroups' output blocks, per stage
    uint32_t omagic[5];  // ceil(2^31 / elements per output block), per stage
};

__device__ __forceinline__ float h2f(uint32_t b) {
    return __half2float(__ushort_as_half((unsigned short)b));
}
// 16-bit value of a lookup table (embedding rows): fp16 for F16 and W8A8 models, bf16 for BF16.
template <int WT>
__device__ __forceinline__ float w2f(uint32_t b) {
    if constexpr (WT == SH_DTYPE_BF16) return __uint_as_float(b << 16);
    else return h2f(b);
}
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }
__device__ __forceinline__ uint16_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

template <int WT>
__device__ __forceinline__ void unpack8(const u32x4 &v, float *f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if constexpr (WT == SH_DTYPE_F16) {
            f[2 * i] = h2f(w[i] & 0xffffu);
            f[2 * i + 1] = h2f(w[i] >> 16);
        } else {
            f[2 * i] = __uint_as_float(w[i] << 16);
            f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
}

template <int KVT>
__device__ __forceinline__ float kv_ld(const void *b, size_t i) {
    if constexpr (KVT == SH_KV_F32) return ((const float *)b)[i];
    else if constexpr (KVT == SH_KV_F16) return h2f(((const uint16_t *)b)[i]);
    else return __uint_as_float((uint32_t)((const uint16_t *)b)[i] << 16);
}
template <int KVT>
__device__ __forceinline__ float kv_rnd(float v) {
    if constexpr (KVT == SH_KV_F32) return v;
    else if constexpr (KVT == SH_KV_F16) return h2f(f2h(v));
    else return __uint_as_float((uint32_t)f2bf(v) << 16);
}
template <int KVT>
__device__ __forceinline__ void kv_st(void *b, size_t i, float v) {
    if constexpr (KVT == SH_KV_F32) ((float *)b)[i] = v;
    else if constexpr (KVT == SH_KV_F16) ((uint16_t *)b)[i] = f2h(v);
    else ((uint16_t *)b)[i] = f2bf(v);
}

// Eight consecutive cache elements starting at a multiple of 8.
template <int KVT>
__device__ __forceinline__ void kv_ld8(const void *b, size_t i, float *out) {
    if constexpr (KVT == SH_KV_F32) {
        const float4 a = ((const float4 *)b)[i / 4], c = ((const float4 *)b)[i / 4 + 1];
        out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
        out[4] = c.x; out[5] = c.y; out[6] = c.z; out[7] = c.w;
    } else {
        const uint4 v = ((const uint4 *)b)[i / 8];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if constexpr (KVT == SH_KV_F16) {
                out[2 * k] = h2f(w[k] & 0xffffu);
                out[2 * k + 1] = h2f(w[k] >> 16);
            } else {
                out[2 * k] = __uint_as_float(w[k] << 16);
                out[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
            }
        }
    }
}

// Workgroup barrier that orders LDS traffic only. __syncthreads() also waits for every
// outstanding global store of the wave (loads and stores share one counter on this
// architecture), which would stall each barrier behind the write-through acknowledgement of
// the hand-over stores. Global data is never exchanged between waves of one workgroup
// inside a forward, so LDS ordering is all the barriers here need.
__device__ __forceinline__ void lds_barrier() {
    __asm__ __volatile__("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Workgroup-wide AND of a per-thread flag, over LDS (two barriers, so the flag array can be
// reused by the next call).
__device__ __forceinline__ bool block_and(bool ok) {
    __shared__ int flags[kPW];
    const bool w = __all(ok);
    if ((threadIdx.x & 63) == 0) flags[threadIdx.x >> 6] = w;
    lds_barrier();
    bool r = true;
#pragma unroll
    for (int i = 0; i < kPW; i++) r = r && flags[i];
    lds_barrier();
    return r;
}

// Workgroup maximum in one barrier, through an array of its own: the next write to it comes
// after the next stage's barriers, when every thread has read this one.
__device__ __forceinline__ float block_max(float v) {
    __shared__ float wmx[kPW];
    v = wmax<64>(v);
    if ((threadIdx.x & 63) == 0) wmx[threadIdx.x >> 6] = v;
    lds_barrier();
    float m = wmx[0];
#pragma unroll
    for (int w = 1; w < kPW; w++) m = fmaxf(m, wmx[w]);
    return m;
}

// Elements per 16-byte weight chunk and bytes per weight element.
template <int WT> constexpr int chunk_elems() { return WT == SH_DTYPE_W8A8 ? 16 : 8; }
template <int WT> constexpr int elem_bytes() { return WT == SH_DTYPE_W8A8 ? 1 : 2; }

// The bridge quantizer for one value (ane_bridge.m:390-396): x / scale with IEEE division,
// clamp to [-128, 127], round half away from zero by +-0.5 and truncation.
__device__ __forceinline__ uint32_t quant8(float x, float scale) {
    float v = __fdiv_rn(x, scale);
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    return (uint32_t)(int)(v >= 0.0f ? v + 0.5f : v - 0.5f) & 0xffu;
}
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

// ---- LL hand-over ---------------------------------------------------------------------------
__device__ __forceinline__ void ll_put(uint64_t *p, float v, uint32_t e) {
    __hip_atomic_store(p, ((uint64_t)e << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_put_u(uint64_t *p, uint32_t v, uint32_t e) {
    __hip_atomic_store(p, ((uint64_t)e << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ll_get(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool aborted(const PParams &p) {
    return __hip_atomic_load(p.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// The bound of a wait, taken once per poll round: false once the wait has to end (its time
// limit passed, which sets *p.err, or, after the quiet period, *p.err set by another wave).
// The clock is read every eighth round. Each round re-requests every missing word once, after
// the shortest sleep: on rings of stages one request per word per round costs 1.33 us per
// hand-over without a sleep and 1.36 us with one, two or four requests in flight per word
// (staggered by sleeps) 1.50 to 1.93 us; in the full decode the sleep is neutral at 768 wide
// and 0.6% faster at 1024 wide, where the polls of 256 workgroups contend for the L2.
// The expiry branches are marked unlikely so that they are laid out after the hot code: the
// whole decode loop runs out of the instruction cache, and the larger shapes' kernels slow
// down by about 12 us per forward for every KB of code added to it.
struct WaitBound {
    long long t0 = 0;
    unsigned rounds = 0;
    __device__ __forceinline__ bool more(const PParams &p) {
        __builtin_amdgcn_s_sleep(1);
        if (__builtin_expect((rounds++ & 7u) != 0, 1)) return true;
        const long long now = wall_clock64();
        if (!t0) {
            t0 = now;
            return true;
        }
        if (__builtin_expect(now - t0 > p.spin_limit, 0)) {
            const int started = __hip_atomic_load(p.err + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_max(p.err, started < (int)gridDim.x ? kErrAbsent : kErrTimeout, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
        return !(now - t0 > p.quiet && aborted(p));
    }
};

// Block-wide wait: once every word j < n (located by map.src(j)) carries epoch map.ep(j),
// its value is in *map.dst(j). Starts with a workgroup barrier, after the first requests
// are issued: the LDS a stage writes is free once every wave has passed it. Each thread requests all of its K words at once and, while any is
// missing, re-requests the missing ones together, so a poll costs one memory round trip
// whatever the number of words. Returns false for the whole block on timeout/abort.
template <int K, typename Map>
__device__ __forceinline__ bool ll_wait_batch(int n, const PParams &p, const Map &map) {
    uint64_t v[K];
    unsigned need = 0;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int j = threadIdx.x + k * kPB;
        if (j < n) {
            v[k] = ll_get(map.src(j));
            need |= 1u << k;
        }
    }
    // every wave is done with the destination's previous contents (stages end without a
    // barrier; this one overlaps the first round trip)
    lds_barrier();
    bool ok = true;
    WaitBound wb;
    while (true) {
#pragma unroll
        for (int k = 0; k < K; k++) {
            if ((need >> k) & 1u) {
                if ((uint32_t)(v[k] >> 32) == map.ep(threadIdx.x + k * kPB)) {
                    *map.dst(threadIdx.x + k * kPB) = __uint_as_float((uint32_t)v[k]);
                    need &= ~(1u << k);
                }
            }
        }
        if (!need) break;
        if (!wb.more(p)) {
            ok = false;
            break;
        }
#pragma unroll
        for (int k = 0; k < K; k++)
            if ((need >> k) & 1u) v[k] = ll_get(map.src(threadIdx.x + k * kPB));
    }
    return block_and(ok);
}

struct VecMap {
    const uint64_t *s;
    float *d;
    uint32_t e;
    __device__ const uint64_t *src(int j) const { return s + j; }
    __device__ float *dst(int j) const { return d + j; }
    __device__ uint32_t ep(int) const { return e; }
};

// Hand-over vectors are written in producer blocks: the workgroup of rank r in a stage
// writes its `per` consecutive elements at words [r * stride, r * stride + per), stride a
// multiple of 16, so each producer's block sits on 128-byte lines of its own. Element i of
// the vector is word (i / per) * stride + i % per. A dense vector is one block (per =
// stride = kDense). i / per is taken as mulhi(2i, magic), magic = ceil(2^31 / per): with
// e = magic * per - 2^31 < per the quotient is exact while i * per < 2^31 (every index and
// block here is below 2^16); per = 1 gives magic = 2^31, per = kDense gives 2.
constexpr int kDense = 1 << 30;
__device__ __forceinline__ int ll_index(int i, int per, int stride, uint32_t magic) {
    const int q = (int)__umulhi((uint32_t)i << 1, magic);
    return q * stride + (i - q * per);
}

// A stage input staged in LDS: elements [0, n) of the input vector (epoch e), then the
// stage's residual rows r0 .. r0 + (count - n) - 1 of the residual vector (epoch er), polled
// together so the residual costs no round trip of its own. (Both sources are addressed from
// one base, without a select between two pointers: that form trips an instruction-
// selection error in the gfx950 backend.)
struct InputMap {
    const uint64_t *s;            // input vector words
    ptrdiff_t roff;               // residual vector words, relative to s
    float *d;
    int n, per, stride;
    int r0, rper, rstride;
    uint32_t magic, rmagic;
    uint32_t e, er;
    __device__ const uint64_t *src(int j) const {
        return s + (j < n ? (ptrdiff_t)ll_index(j, per, stride, magic)
                          : roff + ll_index(r0 + j - n, rper, rstride, rmagic));
    }
    __device__ float *dst(int j) const { return d + j; }
    __device__ uint32_t ep(int j) const { return j < n ? e : er; }
};

// Block-wide: dst[i] = value of src[i] once every word of src[0, n) carries epoch e;
// n <= K * kPB.
template <int K>
__device__ __forceinline__ bool ll_wait_vec(const uint64_t *src, int n, uint32_t e, float *dst, const PParams &p) {
    return ll_wait_batch<K>(n, p, VecMap{src, dst, e});
}

// This thread's words j = threadIdx.x + k*kPB (k < K, j < n) of an input map, into
// registers once each carries its epoch (other entries of val are left as they are).
// `pre` runs right after the first requests are issued (the stage's weight loads go there:
// queued behind the first requests, they hold up none of them). Then a workgroup barrier
// (the LDS the stage writes next is free after it). *ok is this thread's outcome; the caller
// combines it over the workgroup.
template <int K, typename Pre>
__device__ __forceinline__ void ll_poll_regs(int n, const PParams &p, const InputMap &map, float (&val)[K], bool &ok,
                                             Pre &&pre) {
    // The word addresses are worked out once, and every round requests all of the thread's
    // words (a word beyond n re-reads word n-1): a fixed set of loads per round with no
    // branch around them, so a round's examination waits for that round's loads and no
    // others (measured 5 us per Stories110M forward and 100 us per Qwen3-shaped forward
    // faster than re-requesting only the missing words).
    const uint64_t *src[K];
    uint64_t v[K];
    unsigned need = 0;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int j = threadIdx.x + k * kPB;
        src[k] = map.src(j < n ? j : n - 1);
        if (j < n) need |= 1u << k;
        v[k] = ll_get(src[k]);
    }
    pre();
    lds_barrier();
    ok = true;
    WaitBound wb;
    while (true) {
#pragma unroll
        for (int k = 0; k < K; k++) {
            if (((need >> k) & 1u) && (uint32_t)(v[k] >> 32) == map.ep(threadIdx.x + k * kPB)) {
                val[k] = __uint_as_float((uint32_t)v[k]);
                need &= ~(1u << k);
            }
        }
        if (!need) break;
        if (!wb.more(p)) {
            ok = false;
            break;
        }
#pragma unroll
        for (int k = 0; k < K; k++) v[k] = ll_get(src[k]);
    }
}

// Stage this stage's input in LDS: xs[0, n) from an LL vector (map) or, when emb_row is
// given, from an embedding row; xs[n, count) receives the residual rows polled with it.
// With NORM (the stage's `gain`), rmsNormVec (infer.go:301-311): ss = sum of x^2 in float64, rrms =
// float32(1 / sqrt(ss/n + eps)); the fp16/bf16 models take ss and rrms in float (rsqrt).
//   fp16 / bf16: xs = x * gain and *rscale = rrms, applied by the caller to each finished
//                dot product (sum w*(x*g) * rrms instead of sum w*((x*rrms)*g): the float
//                rounding of each term differs, by about 1 ulp).
//   W8A8:        the reference's order, xs = (x * rrms) * gain, then the per-tensor int8
//                quantization (its boundaries must see the reference's values).
// Barriers: the poll's first (frees LDS), one after the partial sums (and the ok flags), and
// for W8A8 two more around the quantization (one: a stage without a norm carries max|x| in the
// partial-sum barrier).
template <int WT, int COLS, bool NORM, typename Pre>
__device__ __forceinline__ bool stage_input(float *xs, int n, const InputMap &map, int count,
                            const uint16_t *emb_row, const uint16_t *res_emb, const float *gain,
                            double eps, double *red, int *okw, const PParams &p, uint32_t *xq,
                            float *sa, float *rscale, Pre &&pre) {
    constexpr int K = (COLS + kMaxRes + kPB - 1) / kPB;
    constexpr bool Q8 = WT == SH_DTYPE_W8A8;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // the gain is loaded into registers before the input is polled, so its memory latency
    // overlaps the hand-over instead of following it
    float gr[NORM ? K : 1];
    if constexpr (NORM) {
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int i = threadIdx.x + k * kPB;
            gr[k] = i < n ? gain[i] : 1.f;
        }
    }
    // residual rows from the embedding row (layer 0) instead of a hand-over vector
    float val[K];
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int j = threadIdx.x + k * kPB;
        val[k] = res_emb && j >= n && j < count ? w2f<WT>(res_emb[map.r0 + j - n]) : 0.f;
    }
    bool ok = true;
    if (emb_row) {
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int i = threadIdx.x + k * kPB;
            if (i < n) val[k] = w2f<WT>(emb_row[i]);
        }
        pre();
        lds_barrier();
    } else {
        ll_poll_regs<K>(res_emb ? n : count, p, map, val, ok, pre);
    }
    // sum of squares: float64 as the reference for W8A8, float for the fp16/bf16 models. W8A8
    // without a norm needs only max|x| for its scale, which rides on the same barrier.
    double ss = 0;
    float ssf = 0.f, mx0 = 0.f;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int j = threadIdx.x + k * kPB;
        if (j < n) {
            if constexpr (NORM && Q8) ss += (double)val[k] * (double)val[k];
            if constexpr (NORM && !Q8) ssf += val[k] * val[k];
            if constexpr (!NORM && Q8) mx0 = fmaxf(mx0, fabsf(val[k]));
            if constexpr (!Q8) xs[j] = NORM ? val[k] * gr[NORM ? k : 0] : val[k];
        } else if (j < count) {
            xs[j] = val[k];   // residual rows
        }
    }
    if constexpr (NORM && Q8) ss = wsum_d64(ss);
    if constexpr (NORM && !Q8) ss = (double)wsum<64>(ssf);
    if constexpr (!NORM && Q8) ss = (double)wmax<64>(mx0);
    const bool wok = __all(ok);
    if (lane == 0) {
        red[wave] = ss;
        okw[wave] = wok;
    }
    lds_barrier();
    bool all_ok = true;
    double tot = 0;
#pragma unroll
    for (int w = 0; w < kPW; w++) {
        all_ok = all_ok && okw[w];
        if constexpr (!NORM && Q8) tot = fmax(tot, red[w]);
        else tot += red[w];
    }
    if (!all_ok) return false;
    float rrms = 1.f;
    if constexpr (NORM && Q8) rrms = (float)(1.0 / sqrt(tot / (double)n + eps));
    if constexpr (NORM && !Q8) rrms = rsqrtf((float)tot / (float)n + (float)eps);
    if constexpr (!Q8) {
        *rscale = rrms;
    } else {
        *rscale = 1.f;
        // xs = (x * rrms) * g in the reference's order; s_a = max|xs| / 127 (0 -> 1);
        // each element quantized on its own thread into a byte of xq (ane_bridge.m:374-399)
        float mx = 0.f;
        if constexpr (NORM) {
#pragma unroll
            for (int k = 0; k < K; k++) {
                const int j = threadIdx.x + k * kPB;
                if (j < n) {
                    val[k] = val[k] * rrms * gr[k];
                    mx = fmaxf(mx, fabsf(val[k]));
                }
            }
            mx = block_max(mx);
        } else {
            mx = (float)tot;   // the workgroup's max|x|, exact through float64
        }
        float s = __fdiv_rn(mx, 127.0f);
        if (s == 0.0f) s = 1.0f;
        *sa = s;
        SH_LDS uint8_t *xb = (SH_LDS uint8_t *)xq;
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int j = threadIdx.x + k * kPB;
            if (j < n) xb[j] = (uint8_t)quant8(val[k], s);
        }
        lds_barrier();
    }
    return true;
}

enum { E_STORE = 0, E_RESID = 1, E_GATE = 2, E_CLS = 3 };

struct StageIO {
    const uint64_t *in_ll;      // input vector (LL) or NULL when emb_row is used
    const uint16_t *emb_row;
    const float *gain;
    uint64_t *out_ll;           // LL output (E_STORE / E_RESID / E_GATE)
    const uint64_t *res_ll;     // E_RESID residual from an LL vector
    const uint16_t *res_emb;    // E_RESID residual from the embedding row (layer 0)
    uint32_t e_in, e_res, e_out;
    int in_per, in_stride;      // input vector layout (in_per 0: dense)
    int res_per, res_stride;    // residual vector layout
    uint32_t in_magic, res_magic;   // ceil(2^31 / per) of the two layouts
    int out_stride;             // words between consecutive workgroups' output blocks
    float *logits;              // E_CLS: logits output, or NULL when not read back
};

// Register tile of a GEMV stage: the weight chunks this lane needs for the first U row groups
// of its wave (CPL 16-byte chunks per row).
template <int U, int CPL>
struct WTile {
    u32x4 w[U][CPL];
};

// This workgroup's row block [r0, r1) in a stage and its rank among the stage's owners;
// false when it owns no rows.
__device__ __forceinline__ bool own_block(const StageOwn o, int rows, int &rank, int &r0, int &r1) {
    rank = (int)blockIdx.x - o.off;
    if (rank < 0) rank += gridDim.x;
    if (rank >= o.n) return false;
    r0 = o.row0 + rank * o.per;
    r1 = min(rows, r0 + o.per);
    return r0 < r1;
}

// What a stage's arithmetic needs from its input poll.
struct StageCtx {
    int rank, r0, r1;
    float sa;       // W8A8: the input's per-tensor scale
    float rscale;   // fp16/bf16 with RMSNorm: rrms, applied to each finished dot product
};

// Loads the tile of the owner's rows [c.r0, c.r1) in a stage: row group k of the block
// belongs to wave k % kPW, G = 64/LPR rows per group, LPR lanes per row. A lane past the
// block's end re-reads row r0, so every entry of the tile is written.
template <int LPR, int CPL, int WT, int U>
__device__ __forceinline__ void tile_load(WTile<U, CPL> &t, const StageCtx &c, const void *__restrict__ W,
                                          int cols) {
    constexpr int G = 64 / LPR;
    const SH_GLOBAL uint8_t *Wb = (const SH_GLOBAL uint8_t *)W;
    const size_t row_bytes = (size_t)cols * elem_bytes<WT>();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, grp = lane / LPR;
    const int r0 = c.r0, r1 = c.r1;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int row = r0 + (wave + u * kPW) * G + grp;
        const SH_GLOBAL u32x4 *src = (const SH_GLOBAL u32x4 *)(Wb + (size_t)(row < r1 ? row : r0) * row_bytes);
#pragma unroll
        for (int j = 0; j < CPL; j++) t.w[u][j] = src[sub + j * LPR];
    }
}

// First half of one GEMV stage over W [rows, cols]: the workgroup owns the row block of its
// rank in the stage's ownership `o` (blocks of consecutive rows keep each hand-over line
// written by one workgroup). An owner polls the stage's input (and residual rows) into LDS
// and normalises it. Returns 0 for a workgroup owning no rows (it polls nothing), 1 once the
// input is staged, -1 on timeout/abort. An owner runs `pre(c)` right after issuing its first
// poll requests: the stage's weight loads go there. Loads complete in issue order, so weight
// loads issued ahead of the poll would hold up its first answer, while these travel beside
// the hand-over they wait for.
template <int LPR, int CPL, int WT, bool NORM, typename Pre>
__device__ __forceinline__ int stage_poll(const PParams &p, const StageOwn o, int rows, int cols, int epi,
                                          const StageIO &io, float *xs, uint32_t *xq, double *red, int *okw,
                                          StageCtx &c, Pre &&pre) {
    constexpr int EPC = chunk_elems<WT>();
    if (!own_block(o, rows, c.rank, c.r0, c.r1)) return 0;
    c.sa = 1.0f;
    c.rscale = 1.f;
    // residual rows, polled with the input (or read from the embedding row in layer 0), land
    // in xs[cols, cols + r1 - r0)
    const int nres = epi == E_RESID ? c.r1 - c.r0 : 0;
    InputMap im{};
    im.s = io.in_ll;
    im.roff = io.res_ll ? io.res_ll - io.in_ll : 0;
    im.d = xs;
    im.n = cols;
    im.per = io.in_per > 0 ? io.in_per : kDense;
    im.stride = io.in_per > 0 ? io.in_stride : kDense;
    im.magic = io.in_per > 0 ? io.in_magic : 2u;   // ceil(2^31 / kDense)
    im.r0 = c.r0;
    im.rper = io.res_per > 0 ? io.res_per : kDense;
    im.rstride = io.res_per > 0 ? io.res_stride : kDense;
    im.rmagic = io.res_per > 0 ? io.res_magic : 2u;
    im.e = io.e_in;
    im.er = io.e_res;
    if (!stage_input<WT, LPR * CPL * EPC, NORM>(xs, cols, im, cols + nres, io.emb_row,
                                                epi == E_RESID ? io.res_emb : nullptr, io.gain, p.eps,
                                                red, okw, p, xq, &c.sa, &c.rscale, [&] { pre(c); }))
        return -1;
    return 1;
}

// Taken at the end of a stage on both paths: after the owner's arithmetic (every load of the
// stage has been used by then) and where a workgroup that owns no rows skips it. The compiler
// cannot tell that the skipping workgroup never loaded the stage's tile, nor that the owner's
// row loop issues no load in its last pass, so without it the registers of those loads would
// count as in flight after the join, and the next stage reusing them would wait there for
// every later request as well (the vector memory counter is in order): for its own stores
// and, behind them, its first poll. Here nothing is in flight but earlier hand-over stores.
__device__ __forceinline__ void settle_loads() {
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0), expcnt and lgkmcnt left alone
}

// Second half: the dot products of the owner's rows against the staged input, the tile `t`
// holding the first U row groups of each wave (further groups stream through it), then the
// epilogue and the block's hand-over stores. For E_CLS, *best_v/*best_i receive this wave's
// (max, first index).
// Rows from lrow0 on, when lrows is given, are read from LDS (lrows: those rows back to back)
// instead of W.
template <int LPR, int CPL, int WT, int U>
__device__ __forceinline__ void stage_compute(const PParams &p, const void *__restrict__ W,
                                              const float *__restrict__ wscale, int cols, int epi,
                                              const StageIO &io, float *xs, uint32_t *xq, float *ostage,
                                              float &best_v, int &best_i, const StageCtx &c,
                                              WTile<U, CPL> &t, const SH_LDS uint8_t *lrows = nullptr,
                                              int lrow0 = 0) {
    constexpr int G = 64 / LPR;
    constexpr bool Q8 = WT == SH_DTYPE_W8A8;
    const SH_GLOBAL uint8_t *Wb = (const SH_GLOBAL uint8_t *)W;
    const size_t row_bytes = (size_t)cols * elem_bytes<WT>();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, grp = lane / LPR;
    const int r0 = c.r0, r1 = c.r1;
    const float sa = c.sa, rscale = c.rscale;
    // first row of this wave's k-th group (wave-uniform)
    auto gbase = [&](int k) { return r0 + (wave + k * kPW) * G; };
    auto &w = t.w;
    // this lane's slice of the input: floats, or packed int8 words for W8A8
    float xr[Q8 ? 1 : CPL * 8];
    uint32_t xr8[Q8 ? CPL * 4 : 1];
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        if constexpr (Q8) {
#pragma unroll
            for (int e = 0; e < 4; e++) xr8[j * 4 + e] = xq[(sub + j * LPR) * 4 + e];
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) xr[j * 8 + e] = xs[(sub + j * LPR) * 8 + e];
        }
    }

    for (int k0 = 0; gbase(k0) < r1; k0 += U) {
        float acc[U];
        int acci[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            acc[u] = 0.f;
            acci[u] = 0;
            const int row = gbase(k0 + u) + grp;
            if (row < r1) {
                // four partial sums per row (a dependent chain a quarter as long), added in a
                // fixed order
                float a4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < CPL; j++) {
                    if constexpr (Q8) {
                        const uint32_t ww[4] = {w[u][j].x, w[u][j].y, w[u][j].z, w[u][j].w};
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            acci[u] = __builtin_amdgcn_sdot4((int)ww[e], (int)xr8[j * 4 + e], acci[u], false);
                    } else {
                        float f[8];
                        unpack8<WT>(w[u][j], f);
#pragma unroll
                        for (int e = 0; e < 8; e++) a4[e & 3] = fmaf(f[e], xr[j * 8 + e], a4[e & 3]);
                    }
                }
                if constexpr (!Q8) acc[u] = (a4[0] + a4[1]) + (a4[2] + a4[3]);
            }
        }
        // next tiles are issued before this batch's reductions and stores
        if (gbase(k0 + U) < r1) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int row = gbase(k0 + U + u) + grp;
                if (row < r1) {
                    if (lrows && gbase(k0 + U + u) >= lrow0) {   // wave-uniform
                        const SH_LDS u32x4 *src = (const SH_LDS u32x4 *)(lrows + (size_t)(row - lrow0) * row_bytes);
#pragma unroll
                        for (int j = 0; j < CPL; j++) w[u][j] = src[sub + j * LPR];
                    } else {
                        const SH_GLOBAL u32x4 *src = (const SH_GLOBAL u32x4 *)(Wb + (size_t)row * row_bytes);
#pragma unroll
                        for (int j = 0; j < CPL; j++) w[u][j] = src[sub + j * LPR];
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int row = gbase(k0 + u) + grp;
            float a;
            if constexpr (Q8) {
                // exact int32 dot, then (float)acc * (s_w[r] * s_a) (one fixed order)
                const int ai = wsum_i<LPR>(acci[u]);
                a = row < r1 ? (float)ai * (wscale[row] * sa) : 0.0f;
            } else {
                a = wsum<LPR>(acc[u]) * rscale;
            }
            if (epi == E_GATE) {
                // rows (2i, 2i+1) = (W1 row i, W3 row i) sit in adjacent lane groups; the
                // owner's gate block starts at rank * out_stride
                float h3 = 0.f;
                if constexpr (LPR < 64) h3 = from_lane_up<LPR>(a);
                if (sub == 0 && (grp & 1) == 0 && row < r1) {
                    // infer.go:324-326: float64 exp for W8A8 (its quantizer sees these values);
                    // the 16-bit models use the hardware exp2 and reciprocal (a few ulp)
                    const float s = Q8 ? a / (1.0f + (float)exp(-(double)a))
                                       : a * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(a * -1.4426950408889634f));
                    ostage[(row - r0) >> 1] = s * h3;
                }
            } else if (sub == 0 && row < r1) {
                if (epi == E_STORE) {
                    ostage[row - r0] = a;
                } else if (epi == E_RESID) {
                    ostage[row - r0] = xs[cols + row - r0] + p.alpha * a;
                } else {  // E_CLS
                    if (io.logits) io.logits[row] = a;
                    if (a > best_v) {
                        best_v = a;
                        best_i = row;
                    }
                }
            }
        }
    }
    settle_loads();
    // The block's outputs leave in one store instruction per 64 words: a hand-over line
    // written by one wave instruction becomes visible as a whole, about a microsecond
    // sooner than the same line written word by word from several waves.
    if (epi != E_CLS) {
        lds_barrier();
        const int nout = epi == E_GATE ? (r1 - r0) >> 1 : r1 - r0;
        uint64_t *out = io.out_ll + (size_t)c.rank * io.out_stride;
        for (int i = threadIdx.x; i < nout; i += kPB) ll_put(out + i, ostage[i], io.e_out);
    }
    // no closing barrier: the next stage's poll starts with one before it writes LDS
}

// Three LL segments (q heads, k, v of one kv head) waited for as one vector.
struct QkvMap {
    const uint64_t *base;       // ll_qkv (dense: qkv blocks are whole lines)
    float *d;                   // q heads, k, v staged contiguously
    size_t qo, ko, vo;          // word offsets of the group's q heads, k and v in ll_qkv
    int nq, hd;
    uint32_t e;
    __device__ const uint64_t *src(int j) const {
        return base + (j < nq ? qo + j : (j < nq + hd ? ko + (j - nq) : vo + (j - nq - hd)));
    }
    __device__ float *dst(int j) const { return d + j; }
    __device__ uint32_t ep(int) const { return e; }
};

// Asynchronous copy of cached rows [0, rows) of one kv head into LDS (global_load_lds:
// each lane moves 16 bytes; one wave instruction fills 1 KB of LDS). Row t of the head
// starts at element base + t*stride; rows are RB bytes long and land contiguously. With SWZ
// the 16-byte chunk c of row t lands in slot c ^ (t mod chunks per row): threads that each
// read their own row chunk by chunk in order then hit distinct LDS banks.
template <int RB, bool SWZ = false>
__device__ __forceinline__ void kv_rows_to_lds(const uint8_t *cache, size_t base_bytes, size_t stride_bytes,
                                               int rows, uint8_t *lds) {
    constexpr int LPRW = RB / 16;            // lanes per row
    constexpr int RPI = 64 / LPRW;           // rows per wave instruction
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r_in = lane / LPRW, slot = lane % LPRW;
    for (int r0 = wave * RPI; r0 < rows; r0 += kPW * RPI) {
        const int r = r0 + r_in < rows ? r0 + r_in : r0;   // a spare lane re-reads a valid row
        const int c = SWZ ? slot ^ ((r0 + r_in) & (LPRW - 1)) : slot;   // chunk for this slot
        const uint8_t *g = cache + base_bytes + (size_t)r * stride_bytes + c * 16;
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)g,
                                         (__attribute__((address_space(3))) void *)(lds + (size_t)r0 * RB),
                                         16, 0, 0);
    }
}

// Rows of one kv head's cache that live in LDS during its attention stage.
template <int KVT, int HD>
struct KvStage {
    static constexpr int EB = KVT == SH_KV_F32 ? 4 : 2;   // bytes per cache element
    static constexpr int RB = HD * EB;                     // bytes per row
    static constexpr int ROWS = kKvStage / (2 * RB);       // K rows, then as many V rows
};

// Starts the asynchronous copy of kv head g's cached rows [0, min(pos, ROWS)) of layer l
// into LDS. Issued at the start of the layer, so it overlaps the qkv stage. KSWZ: the K rows
// in the swizzled chunk order (kv_rows_to_lds), for the one-thread-per-row scores.
template <int KVT, int HD, bool KSWZ = false>
__device__ __forceinline__ void attn_prefetch(const PParams &p, int l, int g, int pos, uint8_t *kvlds) {
    using S = KvStage<KVT, HD>;
    const size_t lbase = (size_t)l * p.max_seq * p.kvdim + (size_t)g * HD;
    const int nst = pos < S::ROWS ? pos : S::ROWS;
    kv_rows_to_lds<S::RB, KSWZ>((const uint8_t *)p.kcache, lbase * S::EB, (size_t)p.kvdim * S::EB, nst, kvlds);
    kv_rows_to_lds<S::RB>((const uint8_t *)p.vcache, lbase * S::EB, (size_t)p.kvdim * S::EB, nst,
                          kvlds + (size_t)S::ROWS * S::RB);
}

template <int KVT>
__device__ __forceinline__ float kv_get(const SH_LDS uint8_t *row, int e) {
    if constexpr (KVT == SH_KV_F32) return ((const SH_LDS float *)row)[e];
    else if constexpr (KVT == SH_KV_F16) return h2f(((const SH_LDS uint16_t *)row)[e]);
    else return __uint_as_float((uint32_t)((const SH_LDS uint16_t *)row)[e] << 16);
}
template <int KVT>
__device__ __forceinline__ void kv_put(SH_LDS uint8_t *row, int e, float v) {
    if constexpr (KVT == SH_KV_F32) ((SH_LDS float *)row)[e] = v;
    else if constexpr (KVT == SH_KV_F16) ((SH_LDS uint16_t *)row)[e] = f2h(v);
    else ((SH_LDS uint16_t *)row)[e] = f2bf(v);
}
// 16 bytes of a cache row as floats: 4 (fp32) or 8 (fp16 / bf16) elements.
template <int KVT>
__device__ __forceinline__ void kv_unpack16(const u32x4 &v, float *f) {
    if constexpr (KVT == SH_KV_F32) {
        f[0] = __uint_as_float(v.x); f[1] = __uint_as_float(v.y);
        f[2] = __uint_as_float(v.z); f[3] = __uint_as_float(v.w);
    } else {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if constexpr (KVT == SH_KV_F16) {
                f[2 * k] = h2f(w[k] & 0xffffu);
                f[2 * k + 1] = h2f(w[k] >> 16);
            } else {
                f[2 * k] = __uint_as_float(w[k] << 16);
                f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
            }
        }
    }
}

// Attention for kv head g (one workgroup) and its `group` query heads (infer.go:273-299) in
// the reference's float summation order, each product and sum rounded on its own: a score
// is the sequential sum over i of q[i]*k[i] (infer.go:284-286), an output element the
// sequential sum over t of p[t]*v[t][i] (:292-295). The W8A8 model uses it: its activations
// are re-quantized after attention, and a last-bit difference that moves x/s across a
// rounding boundary would change an int8 input. q, k and v arrive through one batched poll;
// the cached rows were copied into LDS by attn_prefetch (K rows swizzled), rows beyond the
// LDS capacity are read from the cache. Softmax: one wave per head.
template <int KVT, int HD>
__device__ __forceinline__ bool attn_stage(const PParams &p, int l, int g, int pos, uint32_t e, float *qs,
                           float *sc, float *part, uint8_t *kvlds, double *red, float *redf, long long *tin) {
    using S = KvStage<KVT, HD>;
    constexpr int hd = HD;
    const int group = p.H / p.KVH, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const LayerPtrs Lp = layer_ptrs(p.layers, l);
    const size_t lbase = (size_t)l * p.max_seq * p.kvdim + (size_t)g * hd;
    SH_LDS uint8_t *kst = (SH_LDS uint8_t *)kvlds;
    SH_LDS uint8_t *vst = kst + (size_t)S::ROWS * S::RB;
    const SH_LDS float *qsl = (const SH_LDS float *)qs;

    // qs holds the group's q heads, then k (at kofs), then v (at vofs): one LDS array
    // addressed by offsets, so no pointer ever selects between two LDS arrays
    const int kofs = group * hd, vofs = kofs + hd;
    float *ks = qs + kofs, *vs = qs + vofs;
    QkvMap qm{p.ll_qkv, qs, (size_t)g * group * hd, p.qdim + (size_t)g * hd,
              p.qdim + p.kvdim + (size_t)g * hd, group * hd, hd, e};
    if (!ll_wait_batch<(kMaxGroup + 2) * 256 / kPB>(group * hd + 2 * hd, p, qm)) return false;
    if (__builtin_expect(tin != nullptr, 0)) *tin = wall_clock64();
    if (p.qk_norm) {
        // per-head RMSNorm: wave w < group normalises q head w, wave `group` normalises k
        if (wave <= group) {
            float *v = qs + (wave < group ? wave : group) * hd;
            const float *gn = wave < group ? Lp.q_norm : Lp.k_norm;
            double ss = 0;
            for (int i = lane; i < hd; i += 64) ss += (double)v[i] * (double)v[i];
            ss = wsum_d64(ss);
            const float rr = (float)(1.0 / sqrt(ss / (double)hd + p.qk_eps));
            for (int i = lane; i < hd; i += 64) v[i] = v[i] * rr * gn[i];
        }
        lds_barrier();
    }
    // infer.go:247-265 RoPE, interleaved pairs, on every q head and on k
    const int half = hd / 2;
    for (int i = tid; i < (group + 1) * half; i += kPB) {
        const int h = i / half, pi = i % half;
        float *v = qs + h * hd;   // h == group: k
        const float c = p.rope_cos[pos * half + pi], s = p.rope_sin[pos * half + pi];
        const float ev = v[2 * pi], ov = v[2 * pi + 1];
        // each product rounded before the sum, as the reference computes it
        v[2 * pi] = __fsub_rn(__fmul_rn(ev, c), __fmul_rn(ov, s));
        v[2 * pi + 1] = __fadd_rn(__fmul_rn(ev, s), __fmul_rn(ov, c));
    }
    __builtin_amdgcn_s_waitcnt(0);   // the LDS copies of the cached rows have landed
    lds_barrier();
    // infer.go:267-271 storeKV in the cache's storage type; row pos also joins the LDS rows
    for (int i = tid; i < hd; i += kPB) {
        ks[i] = kv_rnd<KVT>(ks[i]);
        vs[i] = kv_rnd<KVT>(vs[i]);
        kv_st<KVT>(p.kcache, lbase + (size_t)pos * p.kvdim + i, ks[i]);
        kv_st<KVT>(p.vcache, lbase + (size_t)pos * p.kvdim + i, vs[i]);
        if (pos < S::ROWS) {
            // K rows sit in the swizzled chunk order (attn_prefetch<..., true>)
            constexpr int NCH = S::RB / 16, EPC = 16 / S::EB;
            const int ik = ((i / EPC) ^ (pos & (NCH - 1))) * EPC + i % EPC;
            kv_put<KVT>(kst + (size_t)pos * S::RB, ik, ks[i]);
            kv_put<KVT>(vst + (size_t)pos * S::RB, i, vs[i]);
        }
    }
    lds_barrier();
    // scores (infer.go:280-288): one thread per position, the row's 16-byte chunks in order
    // (the reference's summation order), positions beyond the LDS stage read from the cache
    for (int t = tid; t <= pos; t += kPB) {
        float d[kMaxGroup];
#pragma unroll
        for (int h = 0; h < kMaxGroup; h++) d[h] = 0.f;
        if (t < S::ROWS) {
            constexpr int NCH = S::RB / 16, EPC = 16 / S::EB;
            const SH_LDS u32x4 *row = (const SH_LDS u32x4 *)(kst + (size_t)t * S::RB);
            const int swz = t & (NCH - 1);   // chunk c of the row sits in slot c ^ swz
#pragma unroll 4
            for (int c = 0; c < NCH; c++) {
                float kf[EPC];
                const u32x4 kv4 = row[c ^ swz];
                kv_unpack16<KVT>(kv4, kf);
#pragma unroll
                for (int h = 0; h < kMaxGroup; h++) {
                    if (h >= group) continue;
                    const SH_LDS f32x4 *q4 = (const SH_LDS f32x4 *)(qsl + h * hd + c * EPC);
#pragma unroll
                    for (int e4 = 0; e4 < EPC / 4; e4++) {
                        const f32x4 qv = q4[e4];
                        d[h] = __fadd_rn(d[h], __fmul_rn(qv.x, kf[4 * e4 + 0]));
                        d[h] = __fadd_rn(d[h], __fmul_rn(qv.y, kf[4 * e4 + 1]));
                        d[h] = __fadd_rn(d[h], __fmul_rn(qv.z, kf[4 * e4 + 2]));
                        d[h] = __fadd_rn(d[h], __fmul_rn(qv.w, kf[4 * e4 + 3]));
                    }
                }
            }
        } else {
            const size_t rb = lbase + (size_t)t * p.kvdim;
#pragma unroll 8
            for (int k = 0; k < hd; k++) {
                const float kv = t == pos ? ks[k] : kv_ld<KVT>(p.kcache, rb + k);
#pragma unroll
                for (int h = 0; h < kMaxGroup; h++) {
                    if (h >= group) continue;
                    d[h] = __fadd_rn(d[h], __fmul_rn(qs[h * hd + k], kv));
                }
            }
        }
#pragma unroll
        for (int h = 0; h < kMaxGroup; h++)
            if (h < group) sc[h * p.max_seq + t] = __fmul_rn(d[h], p.inv_sqrt_hd);
    }
    lds_barrier();
    // infer.go:328-345 softmaxPrefix: wave h handles head h; sc then holds probabilities.
    // The float64 sum of the exp terms is combined in lane/tree order; that reorders float64
    // additions only, a relative difference near 1e-16 before the sum is rounded to float.
    if (wave < group) {
        float *s = sc + wave * p.max_seq;
        float mx = -INFINITY;
        for (int t = lane; t <= pos; t += 64) mx = fmaxf(mx, s[t]);
        mx = wmax<64>(mx);
        double sum = 0;
        for (int t = lane; t <= pos; t += 64) {
            const float ev = (float)exp((double)(s[t] - mx));
            s[t] = ev;
            sum += (double)ev;
        }
        sum = wsum_d64(sum);
        const float inv = (float)(1.0 / sum);
        for (int t = lane; t <= pos; t += 64) s[t] = s[t] * inv;
    }
    lds_barrier();
    // P.V in the reference's order: thread (h, i) sums p[t] * v[t][i] over t = 0..pos
    for (int k = tid; k < group * hd; k += kPB) {
        const int h = k / hd, ii = k % hd;
        const float *ph = sc + h * p.max_seq;
        const SH_LDS float *phl = (const SH_LDS float *)ph;
        const int tl = pos < S::ROWS ? pos : S::ROWS - 1;
        float sum = 0.f;
        // One wave does this chain for all 64 dims of a head, so it is bound by the wave's
        // instruction issue: four positions per trip, each a read of p, a read of v, a
        // rounded product and a rounded sum; the reads of a trip issue together at fixed
        // offsets from one address, the adds stay in position order.
        const SH_LDS uint8_t *vcol = vst + (size_t)ii * S::EB;
        int t = 0;
#pragma unroll 2
        for (; t + 4 <= tl + 1; t += 4) {
            float pp[4], vv[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                pp[u] = phl[t + u];
                vv[u] = kv_get<KVT>(vcol + (size_t)(t + u) * S::RB, 0);
            }
#pragma unroll
            for (int u = 0; u < 4; u++) sum = __fadd_rn(sum, __fmul_rn(pp[u], vv[u]));
        }
        for (; t <= tl; t++) sum = __fadd_rn(sum, __fmul_rn(phl[t], kv_get<KVT>(vcol + (size_t)t * S::RB, 0)));
#pragma unroll 8
        for (int t = tl + 1; t <= pos; t++) {
            const float vv = t == pos ? vs[ii] : kv_ld<KVT>(p.vcache, lbase + (size_t)t * p.kvdim + ii);
            sum = __fadd_rn(sum, __fmul_rn(ph[t], vv));
        }
        ll_put(p.ll_att + (size_t)(g * group + h) * hd + ii, sum, e);
    }
    lds_barrier();
    return true;
}


// attn_stage<KVT, 64> for one q head per kv head (the Stories110M W8A8 model): every
// float operation, and its order, as there; what moves is which wave does it and how often
// the workgroup waits. A 64-dim head is one wave wide, so wave 0 polls q and k and wave 1
// polls v (no workgroup barrier around the poll); wave 0 applies the QK-norm (float64 sums
// over the wave) and RoPE (the two elements of a pair sit in adjacent lanes, swapped by DPP),
// appends k and wave 1 appends v. One barrier, the scores (one thread per position, as
// there), a second barrier; then wave 0 alone runs the softmax and P.V, so nothing waits
// between them, and P.V issues the LDS reads of its next 8 positions before it adds the
// current 8 (the adds stay in position order). The closing barrier keeps the other waves
// from the next layer's cache prefetch into the rows P.V reads; they have nothing else to
// do until the head's output is out.
template <int KVT, int HD>
__device__ __forceinline__ void attn_exact1_tail(const PParams &p, int g, int pos, uint32_t e, size_t lbase,
                                                 float *qs, float *sc, const SH_LDS uint8_t *vst);
template <int KVT, int HD>
__device__ __forceinline__ bool attn_stage_exact1(const PParams &p, int l, int g, int pos, uint32_t e, float *qs,
                                                  float *sc, uint8_t *kvlds, int *okw, long long *tin) {
    static_assert(HD == 64, "one wave per head vector");
    using S = KvStage<KVT, HD>;
    constexpr int NCH = S::RB / 16, EPC = 16 / S::EB;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const LayerPtrs Lp = layer_ptrs(p.layers, l);
    const size_t lbase = (size_t)l * p.max_seq * p.kvdim + (size_t)g * HD;
    SH_LDS uint8_t *kst = (SH_LDS uint8_t *)kvlds;
    SH_LDS uint8_t *vst = kst + (size_t)S::ROWS * S::RB;
    const SH_LDS float *qsl = (const SH_LDS float *)qs;
    float *ks = qs + HD, *vs = qs + 2 * HD;
    bool ok = true;
    if (wave <= 1) {
        // wave 0: q and k words; wave 1: v
        const uint64_t *sq = p.ll_qkv + (wave == 0 ? (size_t)g * HD : (size_t)p.qdim + p.kvdim + (size_t)g * HD) + lane;
        const uint64_t *sk = p.ll_qkv + (size_t)p.qdim + (size_t)g * HD + lane;
        // RoPE factors of this lane's pair and the QK-norm gains, before the poll
        const int half = HD / 2, pi = lane >> 1;
        const float rc = p.rope_cos[pos * half + pi], rs = p.rope_sin[pos * half + pi];
        const float gq = p.qk_norm ? Lp.q_norm[lane] : 1.f, gk = p.qk_norm ? Lp.k_norm[lane] : 1.f;
        uint64_t a = ll_get(sq), b = wave == 0 ? ll_get(sk) : ((uint64_t)e << 32);
        WaitBound wb;
        while (!__all((uint32_t)(a >> 32) == e && (uint32_t)(b >> 32) == e)) {
            if (!wb.more(p)) {
                ok = false;
                break;
            }
            a = ll_get(sq);
            if (wave == 0) b = ll_get(sk);
        }
        if (__builtin_expect(tin != nullptr, 0) && tid == 0) *tin = wall_clock64();
        float x = __uint_as_float((uint32_t)a), y = __uint_as_float((uint32_t)b);
        // the cached rows of this wave's share have landed (waited for before the append's
        // stores: the counter would otherwise also wait for their write-back)
        __builtin_amdgcn_s_waitcnt(0);
        if (ok && wave == 0) {
            // per-head RMSNorm (float64 sum of squares), then RoPE (infer.go:247-265)
            auto norm_rope = [&](float v, float gn) {
                if (p.qk_norm) {
                    const double ss = wsum_d64((double)v * (double)v);
                    const float rr = (float)(1.0 / sqrt(ss / (double)HD + p.qk_eps));
                    v = v * rr * gn;
                }
                const float o = __uint_as_float(dpp_u<kDppXor1>(__float_as_uint(v)));   // the pair's other element
                const float ev = (lane & 1) ? o : v, ov = (lane & 1) ? v : o;
                return (lane & 1) ? __fadd_rn(__fmul_rn(ev, rs), __fmul_rn(ov, rc))
                                  : __fsub_rn(__fmul_rn(ev, rc), __fmul_rn(ov, rs));
            };
            qs[lane] = norm_rope(x, gq);
            const float kr = kv_rnd<KVT>(norm_rope(y, gk));
            ks[lane] = kr;
            kv_st<KVT>(p.kcache, lbase + (size_t)pos * p.kvdim + lane, kr);
            // K rows sit in the swizzled chunk order (attn_prefetch<..., true>)
            if (pos < S::ROWS) kv_put<KVT>(kst + (size_t)pos * S::RB, ((lane / EPC) ^ (pos & (NCH - 1))) * EPC + lane % EPC, kr);
        } else if (ok) {
            const float vr = kv_rnd<KVT>(x);
            vs[lane] = vr;
            kv_st<KVT>(p.vcache, lbase + (size_t)pos * p.kvdim + lane, vr);
            if (pos < S::ROWS) kv_put<KVT>(vst + (size_t)pos * S::RB, lane, vr);
        }
        if (lane == 0) okw[wave] = __all(ok);
    } else {
        __builtin_amdgcn_s_waitcnt(0);   // this wave's share of the cached rows has landed
    }
    lds_barrier();
    if (!(okw[0] && okw[1])) return false;
    // scores (infer.go:280-288): one thread per position, the row's chunks in order,
    // requested eight at a time ahead of their adds; q[i] reaches every lane of the wave from
    // lane i's register (readlane: a scalar operand, no LDS read per element). readlane reads
    // lanes whatever the branch, so q is loaded in every lane before anything diverges, and a
    // wave takes the LDS path only when all of its positions are LDS rows (lanes past pos
    // score row pos and store nothing); a wave reaching past them reads every row of its
    // positions from the cache, lane by lane.
    float qme = qsl[lane];
    __asm__ __volatile__("" : "+v"(qme));
    for (int t0 = wave * 64; t0 <= pos; t0 += kPB) {
        const int t = t0 + lane;
        float d = 0.f;
        if ((t0 + 63 < pos ? t0 + 63 : pos) < S::ROWS) {
            const int te = t < pos ? t : pos;
            const SH_LDS u32x4 *row = (const SH_LDS u32x4 *)(kst + (size_t)te * S::RB);
            const int swz = te & (NCH - 1);   // chunk c of the row sits in slot c ^ swz
            constexpr int R = NCH < 8 ? NCH : 8;   // chunks requested at once (registers)
#pragma unroll
            for (int c0 = 0; c0 < NCH; c0 += R) {
                u32x4 kc[R];
#pragma unroll
                for (int c = 0; c < R; c++) kc[c] = row[(c0 + c) ^ swz];
#pragma unroll
                for (int c = 0; c < R; c++) {
                    float kf[EPC];
                    kv_unpack16<KVT>(kc[c], kf);
#pragma unroll
                    for (int k = 0; k < EPC; k++) {
                        const float qi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qme), (c0 + c) * EPC + k));
                        d = __fadd_rn(d, __fmul_rn(qi, kf[k]));
                    }
                }
            }
        } else if (t <= pos) {
            const size_t rb = lbase + (size_t)t * p.kvdim;
#pragma unroll 8
            for (int k = 0; k < HD; k++) {
                const float kv = t == pos ? ks[k] : kv_ld<KVT>(p.kcache, rb + k);
                d = __fadd_rn(d, __fmul_rn(qs[k], kv));
            }
        }
        if (t <= pos) sc[t] = __fmul_rn(d, p.inv_sqrt_hd);
    }
    lds_barrier();
    if (wave == 0) attn_exact1_tail<KVT, HD>(p, g, pos, e, lbase, qs, sc, vst);
    lds_barrier();
    return true;
}

// attn_stage_exact1's wave 0 after the scores: softmax, P.V and the head's output words.
template <int KVT, int HD>
__device__ __forceinline__ void attn_exact1_tail(const PParams &p, int g, int pos, uint32_t e, size_t lbase,
                                                 float *qs, float *sc, const SH_LDS uint8_t *vst) {
    using S = KvStage<KVT, HD>;
    const int lane = threadIdx.x & 63;
    const float *vs = qs + 2 * HD;
    // infer.go:328-345 softmaxPrefix, as attn_stage computes it: float max, float64 exp
    // terms, a float64 sum per lane in position order, then over the lanes; the first four
    // positions of a lane are read at once and their exp terms computed side by side
    constexpr int kU = 4;
    float sv[kU];
#pragma unroll
    for (int k = 0; k < kU; k++) sv[k] = lane + 64 * k <= pos ? sc[lane + 64 * k] : -INFINITY;
    float mx = sv[0];
#pragma unroll
    for (int k = 1; k < kU; k++) mx = fmaxf(mx, sv[k]);
    for (int t = lane + 64 * kU; t <= pos; t += 64) mx = fmaxf(mx, sc[t]);
    mx = wmax<64>(mx);
    float ev[kU];
#pragma unroll
    for (int k = 0; k < kU; k++) ev[k] = (float)exp((double)(sv[k] - mx));
    double sum = 0;
#pragma unroll
    for (int k = 0; k < kU; k++)
        if (lane + 64 * k <= pos) sum += (double)ev[k];
    for (int t = lane + 64 * kU; t <= pos; t += 64) {
        const float x = (float)exp((double)(sc[t] - mx));
        sc[t] = x;
        sum += (double)x;
    }
    sum = wsum_d64(sum);
    const float inv = (float)(1.0 / sum);
#pragma unroll
    for (int k = 0; k < kU; k++)
        if (lane + 64 * k <= pos) sc[lane + 64 * k] = ev[k] * inv;
    for (int t = lane + 64 * kU; t <= pos; t += 64) sc[t] = sc[t] * inv;
    __asm__ __volatile__("s_waitcnt lgkmcnt(0)" ::: "memory");   // every lane's p[t] in LDS
    // P.V (infer.go:290-297): lane i sums p[t] * v[t][i] over t = 0..pos in order. The reads
    // of the next 8 positions (p as two broadcast reads, V one element per lane and row) are
    // issued before the current 8 are added, into two register sets used in turn
    const SH_LDS float *phl = (const SH_LDS float *)sc;
    const SH_LDS uint8_t *vcol = vst + (size_t)lane * S::EB;
    const int tl = pos < S::ROWS ? pos : S::ROWS - 1;
    constexpr int PB = 8;
    const int nfull = (tl + 1) / PB;
    float acc = 0.f;
    struct Chunk {
        f32x4 p[PB / 4];
        float v[PB];
    };
    auto cload = [&](int t0, Chunk &ch) {
#pragma unroll
        for (int j = 0; j < PB / 4; j++) ch.p[j] = ((const SH_LDS f32x4 *)(phl + t0))[j];
#pragma unroll
        for (int u = 0; u < PB; u++) ch.v[u] = kv_get<KVT>(vcol + (size_t)(t0 + u) * S::RB, 0);
    };
    auto cmac = [&](const Chunk &ch) {
#pragma unroll
        for (int u = 0; u < PB; u++) {
            const f32x4 q = ch.p[u / 4];
            const float pt = u % 4 == 0 ? q.x : u % 4 == 1 ? q.y : u % 4 == 2 ? q.z : q.w;
            acc = __fadd_rn(acc, __fmul_rn(pt, ch.v[u]));
        }
    };
    const int tf = nfull * PB;
    if (tf > 0) {
        Chunk ca, cb;
        cload(0, ca);
        int t0 = 0;
        for (; t0 + 2 * PB <= tf; t0 += 2 * PB) {
            cload(t0 + PB, cb);
            cmac(ca);
            cload(min(t0 + 2 * PB, tf - PB), ca);   // the last trip re-reads the last chunk
            cmac(cb);
        }
        if (t0 < tf) cmac(ca);
    }
    for (int t = nfull * PB; t <= tl; t++) acc = __fadd_rn(acc, __fmul_rn(phl[t], kv_get<KVT>(vcol + (size_t)t * S::RB, 0)));
#pragma unroll 8
    for (int t = tl + 1; t <= pos; t++) {
        const float vv = t == pos ? vs[lane] : kv_ld<KVT>(p.vcache, lbase + (size_t)t * p.kvdim + lane);
        acc = __fadd_rn(acc, __fmul_rn(sc[t], vv));
    }
    ll_put(p.ll_att + (size_t)g * HD + lane, acc, e);
}

// Attention for the fp16 / bf16 models with two q heads per kv head (the Qwen3 shape: 128-dim
// heads; attn_stage_wave serves one q head per kv head, the W8A8 model attn_stage_exact1 with
// one q head per kv head and 64-dim heads, attn_stage<...> otherwise):
// the same mathematics in fewer dependent steps, rounded differently in the last bits. (The
// per-wave form measured slower at this shape: 736 against 658 us per Qwen3-shaped forward,
// each of its waves polling 512 words.)
//  - RoPE factors are loaded before the poll; QK-norm and the softmax use float math;
//  - scores are lane-sliced dot products over the cached rows (LDS rows two blocks per trip,
//    rows beyond the LDS stage read from the cache the same way), each wave tracking the
//    running maximum of its scores;
//  - the softmax runs on all waves; the exp terms are left unnormalised and the P.V sums are
//    scaled by 1/sum at the end (p.v/sum instead of (p/sum).v);
//  - three workgroup barriers after the cache append, none at the end (the next stage's poll
//    starts with one).
template <int KVT, int HD, int GROUP, bool SPLIT = false>
__device__ __forceinline__ bool attn_stage_fast(const PParams &p, int l, int g, int pos, uint32_t e, float *qs,
                                                float *sc, float *part, uint8_t *kvlds, float *redf,
                                                long long *tin) {
    using S = KvStage<KVT, HD>;
    constexpr int hd = HD, ngr = kPB / HD;
    constexpr int LPK = S::RB / 16, EPC = 16 / S::EB, PPW = 64 / LPK;
    constexpr int group = GROUP;   // q heads of this workgroup, known at compile time so the
                                   // loops below carry no per-row branches
    static_assert(!SPLIT || GROUP == 1, "a split workgroup takes one q head");
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    // SPLIT: workgroup g takes q head g of kv head g / (H / KVH) (the two workgroups of a kv
    // head both finish its k and v and both append them, the same values to the same cache
    // row, so each reads back only rows it wrote itself); otherwise kv head g, q heads
    // g * GROUP ..
    const int qh0 = SPLIT ? g : g * GROUP;   // first q head
    g = SPLIT ? g / (p.H / p.KVH) : g;
    const int ms = p.max_seq;
    const LayerPtrs Lp = layer_ptrs(p.layers, l);
    const size_t lbase = (size_t)l * ms * p.kvdim + (size_t)g * hd;
    SH_LDS uint8_t *kst = (SH_LDS uint8_t *)kvlds;
    SH_LDS uint8_t *vst = kst + (size_t)S::ROWS * S::RB;
    const int kofs = group * hd, vofs = kofs + hd;
    float *ks = qs + kofs, *vs = qs + vofs;
    const int half = hd / 2;
    // this thread's RoPE pair (q heads, then k) and its factors, before the poll
    const bool rope_t = tid < (group + 1) * half;
    const int rpi = tid % half;
    float rc = 0.f, rs = 0.f;
    if (rope_t) {
        rc = p.rope_cos[pos * half + rpi];
        rs = p.rope_sin[pos * half + rpi];
    }
    // QK-norm gains of this wave's head (wave w < group: q head w, wave group: k)
    constexpr int GPL = (HD + 63) / 64;
    float gq[GPL];
#pragma unroll
    for (int q = 0; q < GPL; q++) gq[q] = 0.f;
    if (p.qk_norm && wave <= group) {
        const float *gn = wave < group ? Lp.q_norm : Lp.k_norm;
#pragma unroll
        for (int q = 0; q < GPL; q++)
            if (lane + 64 * q < hd) gq[q] = gn[lane + 64 * q];
    }
    QkvMap qm{p.ll_qkv, qs, (size_t)qh0 * hd, p.qdim + (size_t)g * hd,
              p.qdim + p.kvdim + (size_t)g * hd, group * hd, hd, e};
    if (!ll_wait_batch<(GROUP + 2) * 256 / kPB>(group * hd + 2 * hd, p, qm)) return false;
    if (__builtin_expect(tin != nullptr, 0)) *tin = wall_clock64();
    if (p.qk_norm) {
        // per-head RMSNorm: wave w < group normalises q head w, wave `group` normalises k
        if (wave <= group) {
            float *v = qs + (wave < group ? wave : group) * hd;
            float ss = 0.f;
            for (int i = lane; i < hd; i += 64) ss += v[i] * v[i];
            ss = wsum<64>(ss);
            const float rr = rsqrtf(ss / (float)hd + (float)p.qk_eps);
#pragma unroll
            for (int q = 0; q < GPL; q++)
                if (lane + 64 * q < hd) v[lane + 64 * q] = v[lane + 64 * q] * rr * gq[q];
        }
        lds_barrier();
    }
    if (rope_t) {   // infer.go:247-265, interleaved pairs
        float *v = qs + (tid / half) * hd;
        const float ev = v[2 * rpi], ov = v[2 * rpi + 1];
        v[2 * rpi] = ev * rc - ov * rs;
        v[2 * rpi + 1] = ev * rs + ov * rc;
    }
    __builtin_amdgcn_s_waitcnt(0);   // the LDS copies of the cached rows have landed
    lds_barrier();
    // infer.go:267-271 storeKV in the cache's storage type; row pos also joins the LDS rows
    for (int i = tid; i < hd; i += kPB) {
        ks[i] = kv_rnd<KVT>(ks[i]);
        vs[i] = kv_rnd<KVT>(vs[i]);
        kv_st<KVT>(p.kcache, lbase + (size_t)pos * p.kvdim + i, ks[i]);
        kv_st<KVT>(p.vcache, lbase + (size_t)pos * p.kvdim + i, vs[i]);
        if (pos < S::ROWS) {
            kv_put<KVT>(kst + (size_t)pos * S::RB, i, ks[i]);
            kv_put<KVT>(vst + (size_t)pos * S::RB, i, vs[i]);
        }
    }
    lds_barrier();
    // scores (infer.go:280-288) and each wave's maximum
    const int sl = lane % LPK, rin = lane / LPK;
    float qr[GROUP][EPC];
#pragma unroll
    for (int h = 0; h < GROUP; h++)
#pragma unroll
        for (int q = 0; q < EPC; q++) qr[h][q] = h < group ? qs[h * hd + sl * EPC + q] : 0.f;
    float mx[GROUP];
#pragma unroll
    for (int h = 0; h < GROUP; h++) mx[h] = -INFINITY;
    auto score_row = [&](const float (&kf)[EPC], int t, bool valid) {
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            if (h >= group) continue;
            float d = 0.f;
#pragma unroll
            for (int q = 0; q < EPC; q++) d = fmaf(qr[h][q], kf[q], d);
            d = wsum<LPK>(d) * p.inv_sqrt_hd;
            if (valid) {
                if (sl == 0) sc[h * ms + t] = d;
                mx[h] = fmaxf(mx[h], d);
            }
        }
    };
    const int tl = pos < S::ROWS ? pos : S::ROWS - 1;   // last position held in LDS
    for (int t0 = wave * PPW; t0 <= tl; t0 += 2 * kPW * PPW) {
        const int ta = t0 + rin, tb = t0 + kPW * PPW + rin;
        const bool va = ta <= tl, vb = tb <= tl;
        const u32x4 ka = ((const SH_LDS u32x4 *)(kst + (size_t)(va ? ta : tl) * S::RB))[sl];
        const u32x4 kb = ((const SH_LDS u32x4 *)(kst + (size_t)(vb ? tb : tl) * S::RB))[sl];
        float fa[EPC], fb[EPC];
        kv_unpack16<KVT>(ka, fa);
        kv_unpack16<KVT>(kb, fb);
        score_row(fa, ta, va);
        score_row(fb, tb, vb);
    }
    if (pos > tl) {
        // rows beyond the LDS stage, from the cache (row pos from the staged k)
        float kpos[EPC];
#pragma unroll
        for (int q = 0; q < EPC; q++) kpos[q] = ks[sl * EPC + q];
        // four row blocks per trip, their cache reads in flight together
        const SH_GLOBAL uint8_t *kc = (const SH_GLOBAL uint8_t *)p.kcache;
        for (int tb = tl + 1 + wave * PPW; tb <= pos; tb += 4 * kPW * PPW) {
            u32x4 kv4[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int t = tb + u * kPW * PPW + rin;
                const int tr = t < pos ? t : tl;   // a row in the cache (row pos is not read)
                kv4[u] = ((const SH_GLOBAL u32x4 *)(kc + (lbase + (size_t)tr * p.kvdim) * S::EB))[sl];
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                if (tb + u * kPW * PPW > pos) continue;   // uniform over the wave
                const int t = tb + u * kPW * PPW + rin;
                float kf[EPC];
                kv_unpack16<KVT>(kv4[u], kf);
                if (t == pos) {
#pragma unroll
                    for (int q = 0; q < EPC; q++) kf[q] = kpos[q];
                }
                score_row(kf, t, t <= pos);
            }
        }
    }
#pragma unroll
    for (int h = 0; h < GROUP; h++) {
        const float m = wmax<64>(mx[h]);
        if (lane == 0 && h < group) redf[wave * GROUP + h] = m;
    }
    lds_barrier();
    // softmax (infer.go:328-345) on every wave: unnormalised exp terms and their sums
    float gmx[GROUP], sum[GROUP];
#pragma unroll
    for (int h = 0; h < GROUP; h++) {
        gmx[h] = -INFINITY;
        sum[h] = 0.f;
        if (h < group)
            for (int w = 0; w < kPW; w++) gmx[h] = fmaxf(gmx[h], redf[w * GROUP + h]);
    }
    for (int t = tid; t <= pos; t += kPB) {
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            if (h >= group) continue;
            const float ev = expf(sc[h * ms + t] - gmx[h]);
            sc[h * ms + t] = ev;
            sum[h] += ev;
        }
    }
#pragma unroll
    for (int h = 0; h < GROUP; h++) {
        const float sw = wsum<64>(sum[h]);
        if (lane == 0 && h < group) redf[(kPW + wave) * GROUP + h] = sw;
    }
    lds_barrier();
    // P.V (infer.go:290-297): thread (position group tg, dim vi), partials through LDS; the
    // LDS rows are read four at a time (clamped indices, zero weights past the end), so the
    // reads of a batch are in flight together
    const int vi = tid % hd, tg = tid / hd;
    float acc[GROUP];
#pragma unroll
    for (int h = 0; h < GROUP; h++) acc[h] = 0.f;
    for (int t = tg; t <= tl; t += 4 * ngr) {
        float vv[4], pw[GROUP][4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int tt = t + u * ngr;
            const int tc = tt <= tl ? tt : tl;
            vv[u] = kv_get<KVT>(vst + (size_t)tc * S::RB, vi);
#pragma unroll
            for (int h = 0; h < GROUP; h++) {
                const float w = sc[h * ms + tc];
                pw[h][u] = tt <= tl ? w : 0.f;
            }
        }
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int h = 0; h < GROUP; h++) acc[h] = fmaf(pw[h][u], vv[u], acc[h]);
    }
    // rows beyond the LDS stage: cache reads eight at a time (row pos from the staged v)
    for (int t = tl + 1 + ((tg - (tl + 1) % ngr + ngr) % ngr); t <= pos; t += 8 * ngr) {
        float vc[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int tt = t + u * ngr;
            vc[u] = kv_ld<KVT>(p.vcache, lbase + (size_t)(tt < pos ? tt : tl) * p.kvdim + vi);
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int tt = t + u * ngr;
            if (tt > pos) continue;
            const float vv = tt == pos ? vs[vi] : vc[u];
#pragma unroll
            for (int h = 0; h < GROUP; h++) acc[h] = fmaf(sc[h * ms + tt], vv, acc[h]);
        }
    }
#pragma unroll
    for (int h = 0; h < GROUP; h++) part[(h * ngr + tg) * hd + vi] = acc[h];
    lds_barrier();
    for (int k = tid; k < group * hd; k += kPB) {
        const int h = k / hd, ii = k % hd;
        float tot = 0.f, o = 0.f;
        for (int w = 0; w < kPW; w++) tot += redf[(kPW + w) * GROUP + h];
        for (int r = 0; r < ngr; r++) o += part[(h * ngr + r) * hd + ii];
        ll_put(p.ll_att + (size_t)(qh0 + h) * hd + ii, o / tot, e);
    }
    return true;
}

// Cross-group sum: lanes l, l + N, l + 2N, ... (N = 4, 8, 16, 32) added, the result the same
// on all of them (every step adds two values equal on both partners). Within a 16-lane row
// the groups are combined by rotations (row_ror:8, then row_ror:4: the sum over all rotations
// by multiples of N), then rows by the permlane swaps.
constexpr int kDppRor8 = 0x128;   // row_ror:8 (lane i <- (i + 8) mod 16 within a row)
constexpr int kDppRor4 = 0x124;   // row_ror:4
template <int N>
__device__ __forceinline__ float gsum(float v) {
    static_assert(N == 4 || N == 8 || N == 16 || N == 32, "groups of 4..32 lanes");
    if constexpr (N <= 8) v += __uint_as_float(dpp_u<kDppRor8>(__float_as_uint(v)));
    if constexpr (N <= 4) v += __uint_as_float(dpp_u<kDppRor4>(__float_as_uint(v)));
    if constexpr (N <= 16) {
        const SwapPair s = swap16(__float_as_uint(v));
        v = __uint_as_float(s.a) + __uint_as_float(s.b);
    }
    const SwapPair s = swap32(__float_as_uint(v));
    return __uint_as_float(s.a) + __uint_as_float(s.b);
}
template <int N>
__device__ __forceinline__ float gmax(float v) {
    static_assert(N == 4 || N == 8 || N == 16 || N == 32, "groups of 4..32 lanes");
    if constexpr (N <= 8) v = fmaxf(v, __uint_as_float(dpp_u<kDppRor8>(__float_as_uint(v))));
    if constexpr (N <= 4) v = fmaxf(v, __uint_as_float(dpp_u<kDppRor4>(__float_as_uint(v))));
    if constexpr (N <= 16) {
        const SwapPair s = swap16(__float_as_uint(v));
        v = fmaxf(__uint_as_float(s.a), __uint_as_float(s.b));
    }
    const SwapPair s = swap32(__float_as_uint(v));
    return fmaxf(__uint_as_float(s.a), __uint_as_float(s.b));
}

// Attention for the fp16 / bf16 models (infer.go:273-299): kv head g on this workgroup, its
// GROUP q heads; the W8A8 model keeps attn_stage<...>. Every wave works on its own
// slice of positions and meets the others once, at the end:
//  - each wave polls q|k|v itself (no workgroup barrier after the hand-over), stages the words
//    in its own LDS region and reads them back lane-sliced: lane (r, s) of the wave serves row r
//    of each 64-lane row block and holds elements [EPC*s, EPC*s + EPC) of every vector, so a
//    cache row is one 16-byte LDS read per lane and a block of PPW rows one wave instruction;
//  - QK-norm and RoPE on those registers (RoPE pairs sit inside a lane's slice);
//  - wave w owns rows (8j + w)*PPW + r: the rows its own share of attn_prefetch copied into
//    LDS (kv_rows_to_lds deals rows to waves the same way), so a wave only waits for its own
//    copies; row pos comes from the registers; rows beyond the LDS stage from the cache;
//  - scores with the wave's maximum, then exp(s - max) and the P.V sums over the same rows;
//  - one workgroup barrier: the waves' (max, sum, P.V) combine as in split softmax,
//    out = sum_w e^(m_w - M) o_w / sum_w e^(m_w - M) l_w.
template <int KVT, int HD, int GROUP>
__device__ __forceinline__ bool attn_stage_wave(const PParams &p, int l, int g, int pos, uint32_t e,
                                                float *wst, float *mls, int *okw, uint8_t *kvlds,
                                                long long *tin) {
    using S = KvStage<KVT, HD>;
    constexpr int LPK = S::RB / 16, EPC = 16 / S::EB, PPW = 64 / LPK;
    constexpr int NW = (GROUP + 2) * HD;              // q heads, k, v words
    constexpr int KW = (NW + 63) / 64;                // words a lane polls
    constexpr int WREG = kMaxGroup * 256;             // floats of a wave's LDS region
    static_assert(NW <= WREG && GROUP * HD + 2 * GROUP <= WREG, "wave region");
    static_assert(EPC % 2 == 0, "RoPE pairs inside a lane's slice");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane / LPK, s = lane % LPK;
    const int ms = p.max_seq;
    const LayerPtrs Lp = layer_ptrs(p.layers, l);
    const size_t lbase = (size_t)l * ms * p.kvdim + (size_t)g * HD;
    const SH_LDS uint8_t *kst = (const SH_LDS uint8_t *)kvlds;
    const SH_LDS uint8_t *vst = kst + (size_t)S::ROWS * S::RB;
    float *wr = wst + wave * WREG;   // this wave's LDS region
    // RoPE factors of this lane's pairs and the QK-norm gains of its elements, before the poll
    const int half = HD / 2;
    float rc[EPC / 2], rs[EPC / 2];
#pragma unroll
    for (int j = 0; j < EPC / 2; j++) {
        rc[j] = p.rope_cos[pos * half + s * (EPC / 2) + j];
        rs[j] = p.rope_sin[pos * half + s * (EPC / 2) + j];
    }
    float gqn[EPC], gkn[EPC];
#pragma unroll
    for (int i = 0; i < EPC; i++) {
        gqn[i] = p.qk_norm ? Lp.q_norm[s * EPC + i] : 1.f;
        gkn[i] = p.qk_norm ? Lp.k_norm[s * EPC + i] : 1.f;
    }
    // poll: lane polls words lane + 64k of [q heads | k | v]
    const size_t qo = (size_t)g * GROUP * HD, ko = p.qdim + (size_t)g * HD, vo = (size_t)p.qdim + p.kvdim + (size_t)g * HD;
    const uint64_t *src[KW];
    uint64_t v[KW];
#pragma unroll
    for (int k = 0; k < KW; k++) {
        const int j0 = lane + 64 * k, j = j0 < NW ? j0 : NW - 1;
        src[k] = p.ll_qkv + (j < GROUP * HD ? qo + j : (j < GROUP * HD + HD ? ko + (j - GROUP * HD)
                                                                            : vo + (j - GROUP * HD - HD)));
        v[k] = ll_get(src[k]);
    }
    bool ok = true;
    {
        WaitBound wb;
        while (true) {
            bool have = true;
#pragma unroll
            for (int k = 0; k < KW; k++) have = have && (uint32_t)(v[k] >> 32) == e;
            if (__all(have)) break;
            if (!wb.more(p)) {
                ok = false;
                break;
            }
#pragma unroll
            for (int k = 0; k < KW; k++) v[k] = ll_get(src[k]);
        }
    }
    if (__builtin_expect(tin != nullptr, 0) && wave == 0) *tin = wall_clock64();
    float mw[GROUP], lw[GROUP], acc[GROUP][EPC];
#pragma unroll
    for (int h = 0; h < GROUP; h++) {
        mw[h] = -INFINITY;
        lw[h] = 0.f;
#pragma unroll
        for (int i = 0; i < EPC; i++) acc[h][i] = 0.f;
    }
    if (ok) {
        // lane-sliced copies of q, k, v through the wave's own LDS region
#pragma unroll
        for (int k = 0; k < KW; k++)
            if (lane + 64 * k < NW) wr[lane + 64 * k] = __uint_as_float((uint32_t)v[k]);
        __asm__ __volatile__("s_waitcnt lgkmcnt(0)" ::: "memory");
        float q[GROUP][EPC], kk[EPC], vv[EPC];
#pragma unroll
        for (int i = 0; i < EPC; i++) {
#pragma unroll
            for (int h = 0; h < GROUP; h++) q[h][i] = wr[h * HD + s * EPC + i];
            kk[i] = wr[GROUP * HD + s * EPC + i];
            vv[i] = wr[GROUP * HD + HD + s * EPC + i];
        }
        // per-head RMSNorm (float) and RoPE (infer.go:247-265, interleaved pairs) of q and k
        auto norm_rope = [&](float (&x)[EPC], const float (&gn)[EPC]) {
            if (p.qk_norm) {
                float ss = 0.f;
#pragma unroll
                for (int i = 0; i < EPC; i++) ss += x[i] * x[i];
                ss = wsum<LPK>(ss);
                const float rr = rsqrtf(ss / (float)HD + (float)p.qk_eps);
#pragma unroll
                for (int i = 0; i < EPC; i++) x[i] = x[i] * rr * gn[i];
            }
#pragma unroll
            for (int j = 0; j < EPC / 2; j++) {
                const float ev = x[2 * j], ov = x[2 * j + 1];
                x[2 * j] = ev * rc[j] - ov * rs[j];
                x[2 * j + 1] = ev * rs[j] + ov * rc[j];
            }
        };
#pragma unroll
        for (int h = 0; h < GROUP; h++) norm_rope(q[h], gqn);
        norm_rope(kk, gkn);
        // infer.go:267-271 storeKV in the cache's storage type: row pos as the scores see it
#pragma unroll
        for (int i = 0; i < EPC; i++) {
            kk[i] = kv_rnd<KVT>(kk[i]);
            vv[i] = kv_rnd<KVT>(vv[i]);
        }
        u32x4 kw, vw;   // this lane's 16 bytes of row pos in the cache's storage form
        if constexpr (KVT == SH_KV_F32) {
            kw = u32x4{__float_as_uint(kk[0]), __float_as_uint(kk[1]), __float_as_uint(kk[2]), __float_as_uint(kk[3])};
            vw = u32x4{__float_as_uint(vv[0]), __float_as_uint(vv[1]), __float_as_uint(vv[2]), __float_as_uint(vv[3])};
        } else {
            uint32_t a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t k0 = KVT == SH_KV_F16 ? f2h(kk[2 * i]) : f2bf(kk[2 * i]);
                const uint32_t k1 = KVT == SH_KV_F16 ? f2h(kk[2 * i + 1]) : f2bf(kk[2 * i + 1]);
                const uint32_t v0 = KVT == SH_KV_F16 ? f2h(vv[2 * i]) : f2bf(vv[2 * i]);
                const uint32_t v1 = KVT == SH_KV_F16 ? f2h(vv[2 * i + 1]) : f2bf(vv[2 * i + 1]);
                a[i] = k0 | (k1 << 16);
                b[i] = v0 | (v1 << 16);
            }
            kw = u32x4{a[0], a[1], a[2], a[3]};
            vw = u32x4{b[0], b[1], b[2], b[3]};
        }
        // this wave's share of the cached rows has landed in LDS (waited for before the append's
        // stores: the counter would otherwise also wait for their write-back)
        __builtin_amdgcn_s_waitcnt(0);
        const int pwave = (pos / PPW) % kPW;   // the wave whose row blocks hold row pos
        if (r == 0) {
            if (wave == 0) {
                const size_t o = (lbase + (size_t)pos * p.kvdim) * S::EB + s * 16;
                *(SH_GLOBAL u32x4 *)((uint8_t *)p.kcache + o) = kw;
                *(SH_GLOBAL u32x4 *)((uint8_t *)p.vcache + o) = vw;
            }
            // row pos also joins the LDS stage, written and read by the same wave
            if (wave == pwave && pos < S::ROWS) {
                ((SH_LDS u32x4 *)(kst + (size_t)pos * S::RB))[s] = kw;
                ((SH_LDS u32x4 *)(vst + (size_t)pos * S::RB))[s] = vw;
            }
        }
        // Online softmax per lane group over this wave's rows, NB row blocks per pass
        // (branch-free, so the blocks' dependent chains interleave): the group's running
        // (max m, sum l, P.V acc) is rescaled when its maximum grows. Scores are kept in the
        // base-2 domain (scaled by log2 e) so each softmax term is one exp2.
        constexpr int NB = EPC == 4 ? 4 : 2;   // blocks per pass (two for 16-bit caches: registers)
        const float qscale = p.inv_sqrt_hd * 1.4426950408889634f;
        float m[GROUP];
#pragma unroll
        for (int h = 0; h < GROUP; h++) m[h] = -INFINITY;
        // ALL: rows [0, pos] all in LDS (a row past pos reads row pos's slot and weighs nothing).
        // Otherwise rows [S::ROWS, pos) come from the cache (pos > S::ROWS, so a block of PPW
        // rows never straddles the LDS stage's end) and row pos from the registers.
        auto pass_rows = [&](auto all) {
            constexpr bool ALL = decltype(all)::value;
            const SH_GLOBAL uint8_t *kcg = (const SH_GLOBAL uint8_t *)p.kcache;
            const SH_GLOBAL uint8_t *vcg = (const SH_GLOBAL uint8_t *)p.vcache;
            for (int b0 = wave * PPW; b0 <= pos; b0 += NB * kPW * PPW) {
                float kf[NB][EPC], vf[NB][EPC];
                int t[NB];
#pragma unroll
                for (int i = 0; i < NB; i++) {
                    const int t0 = b0 + i * kPW * PPW;
                    t[i] = t0 + r;
                    u32x4 kr, vr;
                    if (ALL || t0 < S::ROWS) {
                        const int tr = ALL ? (t[i] < pos ? t[i] : pos) : (t[i] < pos ? t[i] : 0);
                        kr = ((const SH_LDS u32x4 *)(kst + (size_t)tr * S::RB))[s];
                        vr = ((const SH_LDS u32x4 *)(vst + (size_t)tr * S::RB))[s];
                    } else {
                        const size_t o = (lbase + (size_t)(t[i] < pos ? t[i] : 0) * p.kvdim) * S::EB + s * 16;
                        kr = *(const SH_GLOBAL u32x4 *)(kcg + o);
                        vr = *(const SH_GLOBAL u32x4 *)(vcg + o);
                    }
                    kv_unpack16<KVT>(kr, kf[i]);
                    kv_unpack16<KVT>(vr, vf[i]);
                    if constexpr (ALL) {
                        // rows past pos weigh nothing (row pos was written by another wave, so
                        // its bytes as this wave sees them may be anything, NaN included)
#pragma unroll
                        for (int e2 = 0; e2 < EPC; e2++) vf[i][e2] = t[i] <= pos ? vf[i][e2] : 0.f;
                    } else {
                        // row pos from the registers; rows past pos weigh nothing (their bytes
                        // may be anything, NaN included)
#pragma unroll
                        for (int e2 = 0; e2 < EPC; e2++) {
                            kf[i][e2] = t[i] == pos ? kk[e2] : kf[i][e2];
                            vf[i][e2] = t[i] == pos ? vv[e2] : (t[i] < pos ? vf[i][e2] : 0.f);
                        }
                    }
                }
#pragma unroll
                for (int h = 0; h < GROUP; h++) {
                    // scores (infer.go:280-288), times log2 e
                    float sc4[NB];
#pragma unroll
                    for (int i = 0; i < NB; i++) {
                        float d0 = 0.f, d1 = 0.f;
#pragma unroll
                        for (int e2 = 0; e2 < EPC; e2 += 2) {
                            d0 = fmaf(q[h][e2], kf[i][e2], d0);
                            d1 = fmaf(q[h][e2 + 1], kf[i][e2 + 1], d1);
                        }
                        sc4[i] = d0 + d1;
                    }
#pragma unroll
                    for (int i = 0; i < NB; i++) sc4[i] = wsum<LPK>(sc4[i]) * qscale;
                    float mn = m[h];
#pragma unroll
                    for (int i = 0; i < NB; i++) mn = t[i] <= pos ? fmaxf(mn, sc4[i]) : mn;
                    // softmax terms (infer.go:328-345) against the running maximum
                    // 0 from a -inf running maximum, 1 while the group has seen no row
                    const float f = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m[h] - mn);
                    float pw[NB];
#pragma unroll
                    for (int i = 0; i < NB; i++) pw[i] = t[i] <= pos ? __builtin_amdgcn_exp2f(sc4[i] - mn) : 0.f;
                    m[h] = mn;
                    float ls = pw[0];
#pragma unroll
                    for (int i = 1; i < NB; i++) ls += pw[i];
                    lw[h] = fmaf(lw[h], f, ls);
                    // P.V (infer.go:290-297)
#pragma unroll
                    for (int e2 = 0; e2 < EPC; e2++) {
                        float a = pw[0] * vf[0][e2];
#pragma unroll
                        for (int i = 1; i < NB; i++) a = fmaf(pw[i], vf[i][e2], a);
                        acc[h][e2] = fmaf(acc[h][e2], f, a);
                    }
                }
            }
        };
        if (pos < S::ROWS) pass_rows(std::true_type{});
        else pass_rows(std::false_type{});
        // the wave's groups combined: maximum over groups, each group's sums rescaled to it
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            const float M = gmax<LPK>(m[h]);
            const float f = m[h] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[h] - M);
            mw[h] = M;
            lw[h] = gsum<LPK>(lw[h] * f);
#pragma unroll
            for (int e2 = 0; e2 < EPC; e2++) acc[h][e2] = gsum<LPK>(acc[h][e2] * f);
        }
        // P.V into the wave's region (its q|k|v copies were read above); the wave's maximum
        // and sum into mls, [head][max | sum][wave], so the combine reads them in a few
        // vector reads
        if (r == 0) {
#pragma unroll
            for (int h = 0; h < GROUP; h++)
#pragma unroll
                for (int i = 0; i < EPC; i++) wr[h * HD + s * EPC + i] = acc[h][i];
        }
        if (lane == 0) {
#pragma unroll
            for (int h = 0; h < GROUP; h++) {
                mls[(2 * h) * kPW + wave] = mw[h];
                mls[(2 * h + 1) * kPW + wave] = lw[h];
            }
        }
    }
    if (lane == 0) okw[wave] = ok;
    lds_barrier();
    bool all_ok = true;
#pragma unroll
    for (int w = 0; w < kPW; w++) all_ok = all_ok && okw[w];
    if (!all_ok) return false;
    // combine the waves: thread (h, d), every LDS read issued before the first is used (wave
    // 0 holds row 0, so the maximum M is finite; a wave without rows weighs exp2(-inf) = 0)
    for (int k = tid; k < GROUP * HD; k += kPB) {
        const int h = k / HD;
        float mv[kPW], lv[kPW], ov[kPW];
#pragma unroll
        for (int w = 0; w < kPW; w++) {
            mv[w] = mls[(2 * h) * kPW + w];
            lv[w] = mls[(2 * h + 1) * kPW + w];
            ov[w] = wst[w * WREG + k];
        }
        float M = mv[0];
#pragma unroll
        for (int w = 1; w < kPW; w++) M = fmaxf(M, mv[w]);
        float tot = 0.f, o = 0.f;
#pragma unroll
        for (int w = 0; w < kPW; w++) {
            const float f = __builtin_amdgcn_exp2f(mv[w] - M);
            tot = fmaf(f, lv[w], tot);
            o = fmaf(f, ov[w], o);
        }
        ll_put(p.ll_att + (size_t)g * GROUP * HD + k, o * __builtin_amdgcn_rcpf(tot), e);
    }
    return true;
}

// Asynchronous copy of bytes [0, nbytes) from src (nbytes a multiple of 16, at most kKvStage)
// into LDS, 1 KB per wave instruction (global_load_lds, 16 bytes per lane); a lane past the
// end re-reads the last 16 bytes, so every read stays in bounds.
__device__ __forceinline__ void bytes_to_lds(const uint8_t *src, int nbytes, uint8_t *lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = nbytes / 16;
    for (int base = wave * 64; base < n; base += kPW * 64) {
        const int c = min(base + lane, n - 1);
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(src + (size_t)c * 16),
                                         (__attribute__((address_space(3))) void *)(lds + (size_t)base * 16), 16, 0,
                                         0);
    }
}

template <int WT, int KVT, int HD, int LD, int CD, int LQ, int CQ, int LF, int CF>
__global__ __launch_bounds__(kPB, 1) void k_decode_persistent(PParams p) {
    __shared__ float xs[kXs];
    __shared__ __attribute__((aligned(16))) uint32_t xq[WT == SH_DTYPE_W8A8 ? kXs / 4 : 1];
    __shared__ __attribute__((aligned(16))) float qs[(kMaxGroup + 2) * 256];   // q heads, k, v
    __shared__ __attribute__((aligned(16))) float sc[kScores];
    __shared__ float part[kPW * kMaxGroup * 256];
    __shared__ __attribute__((aligned(16))) uint8_t kvlds[kKvStage];
    __shared__ double red[kPW];
    __shared__ int okw[kPW];
    __shared__ float ostage[kMaxPer];   // a GEMV stage's output block, before its stores
    __shared__ __attribute__((aligned(16))) float redf[2 * kPW * kMaxGroup];
    __shared__ ArgmaxPartial cand[kPW];
    __shared__ int next_tok;

    const int L = p.L;
    const int n_stamps = 5 * L + 3;
    int tok_next = 0;
    if (__builtin_expect(p.fail_mode != 0, 0)) {
        if (threadIdx.x == 0) __hip_atomic_fetch_max(p.err, p.fail_mode, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (threadIdx.x == 0) __hip_atomic_fetch_add(p.err + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Classifier rows: the attention workgroups own what their register tile holds; with
    // cls_lds_rows the others own twice as many and keep the second half in the attention
    // cache's LDS (unused outside attention) for the whole launch, copied here once.
    // (Instantiated for the 16-bit 64-dim-head shapes only: elsewhere the vocabulary does not
    // split so, and the branch would cost the larger shapes registers.)
    constexpr bool kClsLds = WT != SH_DTYPE_W8A8 && HD == 64;
    // the 16-bit 128-dim-head shape (two q heads per kv head) runs attention on one workgroup
    // per q head
    constexpr bool kSplitAttn = WT != SH_DTYPE_W8A8 && HD == 128;
    constexpr int kClsTileRows = 4 * kPW * (64 / LD);   // rows of the classifier's WTile<4>
    const StageOwn cown = p.own_cls_a.n && (int)blockIdx.x < p.KVH ? p.own_cls_a : p.own[4];
    const SH_LDS uint8_t *cls_lds = nullptr;
    int cls_lrow0 = 0;
    if (kClsLds && p.cls_lds_rows && (int)blockIdx.x >= p.KVH) {
        int rk, a0, a1;
        if (own_block(cown, p.V, rk, a0, a1) && a1 > a0 + kClsTileRows) {
            const int row_bytes = p.D * elem_bytes<WT>();
            cls_lrow0 = a0 + kClsTileRows;
            bytes_to_lds((const uint8_t *)p.cls + (size_t)cls_lrow0 * row_bytes, (a1 - cls_lrow0) * row_bytes, kvlds);
            cls_lds = (const SH_LDS uint8_t *)kvlds;
        }
    }
    // Each GEMV stage keeps the weights of its first row groups in registers (qkv and w13: two
    // per wave, wo and w2: one, the classifier: four), loaded inside the stage's poll right
    // after its first requests.
    for (int f = 0; f < p.n_forwards; f++) {
        const int pos = p.pos0 + f;
        const bool tracing = p.trace && f == p.trace_f && threadIdx.x == 0;
        long long *tr = p.trace + (size_t)blockIdx.x * 2 * n_stamps;
        int ts = 0;
        auto stamp = [&]() {
            if (__builtin_expect(tracing, 0)) tr[ts] = wall_clock64();
            ts++;
        };
        // input ready for the stage whose end stamp comes next
        auto stamp_in = [&]() {
            if (__builtin_expect(tracing, 0)) tr[n_stamps + ts] = wall_clock64();
        };
        stamp();
        const int tok = pos < p.n_prompt ? p.tokens[pos] : tok_next;
        const bool tok_ok = tok >= 0 && tok < p.V;
        const uint16_t *emb_row = p.embed + (size_t)(tok_ok ? tok : 0) * p.D;
        const uint32_t base = p.epoch0 + (uint32_t)f * (uint32_t)(L + 1);
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        // one layer
        auto layer = [&](int l) -> bool {
            const uint32_t e = base + (uint32_t)l + 1;
            const LayerPtrs Lp = layer_ptrs(p.layers, l);
            if ((int)blockIdx.x < p.NA)
                attn_prefetch<KVT, HD, WT == SH_DTYPE_W8A8>(p, l, kSplitAttn ? (int)blockIdx.x / (p.H / p.KVH) : (int)blockIdx.x,
                                                           pos, kvlds);
            StageIO io{};
            StageCtx c{};
            int r;
            // qkv
            io.in_ll = l ? p.ll_x : nullptr;
            io.in_per = p.own[3].per;
            io.in_stride = p.ostride[3];
            io.in_magic = p.omagic[3];
            io.emb_row = l ? nullptr : emb_row;
            io.gain = Lp.rms_att;
            io.out_ll = p.ll_qkv;
            io.out_stride = p.ostride[0];
            io.e_in = e - 1;
            io.e_out = e;
            {
                WTile<2, CD> t;
                if ((r = stage_poll<LD, CD, WT, true>(p, p.own[0], p.qkv_rows, p.D, E_STORE, io, xs, xq, red, okw, c,
                        [&](const StageCtx &cc) { tile_load<LD, CD, WT, 2>(t, cc, Lp.wqkv, p.D); })) < 0)
                    return false;
                if (r) {
                    stamp_in();
                    stage_compute<LD, CD, WT, 2>(p, Lp.wqkv, Lp.s_qkv, p.D, E_STORE, io, xs, xq, ostage, bv, bi, c, t);
                } else {
                    settle_loads();
                }
            }
            stamp();
            // attention
            if ((int)blockIdx.x < p.NA) {
                long long *tin = tracing ? tr + n_stamps + ts : nullptr;
                bool aok;
                // (each instance compiles only the forms its shapes can take: a kernel's register
                // allocation is the largest any of its paths needs)
                if constexpr (WT == SH_DTYPE_W8A8 && HD == 64)
                    aok = p.H == p.KVH
                              ? attn_stage_exact1<KVT, HD>(p, l, blockIdx.x, pos, e, qs, sc, kvlds, okw, tin)
                              : attn_stage<KVT, HD>(p, l, blockIdx.x, pos, e, qs, sc, part, kvlds, red, redf, tin);
                else if constexpr (WT == SH_DTYPE_W8A8)
                    aok = attn_stage<KVT, HD>(p, l, blockIdx.x, pos, e, qs, sc, part, kvlds, red, redf, tin);
                else if constexpr (kSplitAttn)   // 128-dim heads, two q heads per kv head: one per workgroup
                    aok = attn_stage_fast<KVT, HD, 1, true>(p, l, blockIdx.x, pos, e, qs, sc, part, kvlds, redf, tin);
                else if (p.H == p.KVH)
                    aok = attn_stage_wave<KVT, HD, 1>(p, l, blockIdx.x, pos, e, part, redf, okw, kvlds, tin);
                else
                    aok = attn_stage_fast<KVT, HD, 2>(p, l, blockIdx.x, pos, e, qs, sc, part, kvlds, redf, tin);
                if (!aok) return false;
            }
            stamp();
            // wo + residual
            io = StageIO{};
            io.in_ll = p.ll_att;
            io.out_ll = p.ll_x2;
            io.out_stride = p.ostride[1];
            io.res_ll = l ? p.ll_x : nullptr;
            io.res_per = p.own[3].per;
            io.res_stride = p.ostride[3];
            io.res_magic = p.omagic[3];
            io.res_emb = l ? nullptr : emb_row;
            io.e_in = e;
            io.e_res = e - 1;
            io.e_out = e;
            {
                WTile<1, CQ> t;
                if ((r = stage_poll<LQ, CQ, WT, false>(p, p.own[1], p.D, p.qdim, E_RESID, io, xs, xq, red, okw, c,
                        [&](const StageCtx &cc) { tile_load<LQ, CQ, WT, 1>(t, cc, Lp.wo, p.qdim); })) < 0)
                    return false;
                if (r) {
                    stamp_in();
                    stage_compute<LQ, CQ, WT, 1>(p, Lp.wo, Lp.s_o, p.qdim, E_RESID, io, xs, xq, ostage, bv, bi, c, t);
                } else {
                    settle_loads();
                }
            }
            stamp();
            // w1/w3 + silu gate
            io = StageIO{};
            io.in_ll = p.ll_x2;
            io.in_per = p.own[1].per;
            io.in_stride = p.ostride[1];
            io.in_magic = p.omagic[1];
            io.gain = Lp.rms_ffn;
            io.out_ll = p.ll_gate;
            io.out_stride = p.ostride[2];
            io.e_in = e;
            io.e_out = e;
            {
                WTile<2, CD> t;
                if ((r = stage_poll<LD, CD, WT, true>(p, p.own[2], 2 * p.F, p.D, E_GATE, io, xs, xq, red, okw, c,
                        [&](const StageCtx &cc) { tile_load<LD, CD, WT, 2>(t, cc, Lp.w13, p.D); })) < 0)
                    return false;
                if (r) {
                    stamp_in();
                    stage_compute<LD, CD, WT, 2>(p, Lp.w13, Lp.s_13, p.D, E_GATE, io, xs, xq, ostage, bv, bi, c, t);
                } else {
                    settle_loads();
                }
            }
            stamp();
            // w2 + residual
            io = StageIO{};
            io.in_ll = p.ll_gate;
            io.in_per = p.own[2].per / 2;
            io.in_stride = p.ostride[2];
            io.in_magic = p.omagic[2];
            io.out_ll = p.ll_x;
            io.out_stride = p.ostride[3];
            io.res_ll = p.ll_x2;
            io.res_per = p.own[1].per;
            io.res_stride = p.ostride[1];
            io.res_magic = p.omagic[1];
            io.e_in = e;
            io.e_res = e;
            io.e_out = e;
            {
                WTile<1, CF> t;
                if ((r = stage_poll<LF, CF, WT, false>(p, p.own[3], p.D, p.F, E_RESID, io, xs, xq, red, okw, c,
                        [&](const StageCtx &cc) { tile_load<LF, CF, WT, 1>(t, cc, Lp.w2, p.F); })) < 0)
                    return false;
                if (r) {
                    stamp_in();
                    stage_compute<LF, CF, WT, 1>(p, Lp.w2, Lp.s_2, p.F, E_RESID, io, xs, xq, ostage, bv, bi, c, t);
                } else {
                    settle_loads();
                }
            }
            stamp();
            return true;
        };
        for (int l = 0; l < L; l++)
            if (!layer(l)) return;
        // classifier over rmsnorm(x) (infer.go:242-243)
        const uint32_t ec = base + (uint32_t)L + 1;
        {
            StageIO io{};
            StageCtx c{};
            io.in_ll = p.ll_x;
            io.in_per = p.own[3].per;
            io.in_stride = p.ostride[3];
            io.in_magic = p.omagic[3];
            io.gain = p.rms_final;
            // only the launch's last forward leaves its logits: the host reads them after a
            // one-forward launch, and stores queued ahead of the argmax poll delay it
            io.logits = f == p.n_forwards - 1 ? p.logits : nullptr;
            io.e_in = base + (uint32_t)L;
            // the classifier's tile (four row groups) is loaded before its poll: loaded inside
            // it, beside the poll's registers, it would spill. Every workgroup loads one (a
            // workgroup owning no rows reads row 0), so the tile is defined on every path and
            // the compiler keeps no copy of it alive around the loop.
            WTile<4, CD> t;
            {
                StageCtx ct{};
                if (!own_block(cown, p.V, ct.rank, ct.r0, ct.r1)) ct.r0 = ct.r1 = 0;
                tile_load<LD, CD, WT, 4>(t, ct, p.cls, p.D);
            }
            const int r = stage_poll<LD, CD, WT, true>(p, cown, p.V, p.D, E_CLS, io, xs, xq, red, okw, c,
                                                       [](const StageCtx &) {});
            if (r < 0) return;
            stamp_in();
            if (r)
                stage_compute<LD, CD, WT, 4>(p, p.cls, p.s_cls, p.D, E_CLS, io, xs, xq, ostage, bv, bi, c, t, cls_lds,
                                             cls_lrow0);
        }
        stamp();
        // this workgroup's (max, first index)
        {
            float v = bv;
            int idx = bi;
            wargmax(v, idx);
            if ((threadIdx.x & 63) == 0) cand[threadIdx.x >> 6] = ArgmaxPartial{v, idx};
            lds_barrier();
            if (threadIdx.x == 0) {
                ArgmaxPartial b = cand[0];
                for (int w = 1; w < kPW; w++)
                    if (better(cand[w].v, cand[w].i, b.v, b.i)) b = cand[w];
                const size_t slot = ((size_t)(f & 1) * gridDim.x + blockIdx.x) * kArgSlot;
                ll_put(p.ll_pv + slot, b.v, ec);
                ll_put_u(p.ll_pi + slot, (uint32_t)b.i, ec);
            }
        }
        // next token: needed to generate, and always after the last forward of a launch. When the
        // w13 stage does not span every workgroup the exchange runs after every forward: it is
        // what keeps a slow workgroup's classifier poll of x ahead of the next forward's w2
        // stores.
        if (p.argmax_every || pos + 1 >= p.n_prompt || f == p.n_forwards - 1) {
            bool ok = true;
            float v = -INFINITY;
            int idx = 0x7fffffff;
            const int n = gridDim.x;
            const uint64_t *pv = p.ll_pv + (size_t)(f & 1) * n * kArgSlot;
            const uint64_t *pi = p.ll_pi + (size_t)(f & 1) * n * kArgSlot;
            // one partial per thread (n <= kPB); its value and index words polled together
            if ((int)threadIdx.x < n) {
                const size_t o = (size_t)threadIdx.x * kArgSlot;
                uint64_t a = ll_get(pv + o), b = ll_get(pi + o);
                WaitBound wb;
                while ((uint32_t)(a >> 32) != ec || (uint32_t)(b >> 32) != ec) {
                    if (!wb.more(p)) {
                        ok = false;
                        break;
                    }
                    if ((uint32_t)(a >> 32) != ec) a = ll_get(pv + o);
                    if ((uint32_t)(b >> 32) != ec) b = ll_get(pi + o);
                }
                v = __uint_as_float((uint32_t)a);
                idx = (int)(uint32_t)b;
            }
            if (!block_and(ok)) return;
            stamp_in();
            wargmax(v, idx);
            if ((threadIdx.x & 63) == 0) cand[threadIdx.x >> 6] = ArgmaxPartial{v, idx};
            lds_barrier();
            if (threadIdx.x == 0) {
                ArgmaxPartial b = cand[0];
                for (int w = 1; w < kPW; w++)
                    if (better(cand[w].v, cand[w].i, b.v, b.i)) b = cand[w];
                const int nt = b.i == 0x7fffffff ? 0 : b.i;
                next_tok = nt;
                if (blockIdx.x == 0) {
                    p.hist[pos] = nt;
                    if (pos + 1 <= p.max_seq && pos + 1 >= p.n_prompt) p.tokens[pos + 1] = nt;
                }
            }
            lds_barrier();
            tok_next = next_tok;
        }
        stamp();
    }
}

typedef void (*PersistentKernel)(PParams);

template <int WT, int KVT>
PersistentKernel pick_shape(int D, int Q, int F, int HDv) {
    if constexpr (WT == SH_DTYPE_W8A8) {
        if (D == 768 && Q == 768 && F == 2048 && HDv == 64)
            return &k_decode_persistent<WT, KVT, 64, 16, 3, 16, 3, 32, 4>;
        if (D == 1024 && Q == 2048 && F == 3072 && HDv == 128)
            return &k_decode_persistent<WT, KVT, 128, 32, 2, 32, 4, 64, 3>;
        if (D == 128 && Q == 128 && F == 256 && HDv == 32)
            return &k_decode_persistent<WT, KVT, 32, 8, 1, 8, 1, 16, 1>;
    } else {
        if (D == 768 && Q == 768 && F == 2048 && HDv == 64)
            return &k_decode_persistent<WT, KVT, 64, 32, 3, 32, 3, 64, 4>;
        if (D == 1024 && Q == 2048 && F == 3072 && HDv == 128)
            return &k_decode_persistent<WT, KVT, 128, 32, 4, 64, 4, 64, 6>;
        if (D == 128 && Q == 128 && F == 256 && HDv == 32)
            return &k_decode_persistent<WT, KVT, 32, 16, 1, 16, 1, 32, 1>;
    }
    return nullptr;
}

// Lanes per weight row of the model-dim stages (qkv, w13, classifier) in pick_shape's
// instances: their LD parameter.
int shape_ld(int dtype, int D) {
    if (dtype == SH_DTYPE_W8A8) return D == 1024 ? 32 : (D == 768 ? 16 : 8);
    return D == 128 ? 16 : 32;
}

PersistentKernel pick_persistent(int dtype, int kv, int D, int Q, int F, int HDv) {
    if (dtype == SH_DTYPE_F16) {
        if (kv == SH_KV_F32) return pick_shape<SH_DTYPE_F16, SH_KV_F32>(D, Q, F, HDv);
        if (kv == SH_KV_F16) return pick_shape<SH_DTYPE_F16, SH_KV_F16>(D, Q, F, HDv);
        return pick_shape<SH_DTYPE_F16, SH_KV_BF16>(D, Q, F, HDv);
    }
    if (dtype == SH_DTYPE_BF16) {
        if (kv == SH_KV_F32) return pick_shape<SH_DTYPE_BF16, SH_KV_F32>(D, Q, F, HDv);
        if (kv == SH_KV_F16) return pick_shape<SH_DTYPE_BF16, SH_KV_F16>(D, Q, F, HDv);
        return pick_shape<SH_DTYPE_BF16, SH_KV_BF16>(D, Q, F, HDv);
    }
    if (dtype == SH_DTYPE_W8A8) {
        if (kv == SH_KV_F32) return pick_shape<SH_DTYPE_W8A8, SH_KV_F32>(D, Q, F, HDv);
        if (kv == SH_KV_F16) return pick_shape<SH_DTYPE_W8A8, SH_KV_F16>(D, Q, F, HDv);
        return pick_shape<SH_DTYPE_W8A8, SH_KV_BF16>(D, Q, F, HDv);
    }
    return nullptr;
}

}  // namespace

bool persistent_supported(const sh_model *m) {
    const sh_config &c = m->cfg;
    const int group = c.n_heads / c.n_kv_heads;
    if (!pick_persistent(m->dtype, c.kv_dtype, c.dim, m->qdim, c.hidden, c.head_dim)) return false;
    if (group > kMaxGroup || group * c.max_seq > kScores || c.head_dim > 256) return false;
    if (c.head_dim == 128 && m->dtype != SH_DTYPE_W8A8 && group != 2) return false;   // the one form compiled
    // staged input plus the residual rows polled with it
    if (c.dim + kMaxRes > kXs || m->qdim + kMaxRes > kXs || c.hidden + kMaxRes > kXs) return false;
    if (kPB % c.head_dim) return false;
    return true;
}

// Grid and stage ownership. The grid is one workgroup per CU (at most kPB, one argmax
// partial per thread), shrunk until row blocks of the w13 stage can cover every workgroup.
// qkv takes blocks of 16 rows over as many workgroups as that needs, after the attention
// workgroups [0, NA) when it fits; wo takes about 24 KB of weights per workgroup, placed
// after qkv when it fits (its workgroups then idle through qkv and attention, so their weight
// tiles arrive before att does). w13 and w2 then take one of two layouts: on every
// workgroup (w2 a few rows each, so the weight tiles it loads after the w13 stage stay
// small; w13 spanning the grid makes it depend on every workgroup having finished the
// previous forward's classifier, which keeps the single-buffered ll_x safe while prompt
// forwards run without an argmax exchange), or, where the blocks fit, w13 on half the grid
// and w2 after the qkv block (below; the exchange then runs after every forward).
// Attention workgroups: one per q head for the 16-bit 128-dim-head shape (the kernel's split
// form), else one per kv head.
int attn_workgroups(const sh_model *m) {
    return m->cfg.head_dim == 128 && m->dtype != SH_DTYPE_W8A8 ? m->cfg.n_heads : m->cfg.n_kv_heads;
}

hipError_t persistent_plan(sh_model *m, std::string *why) {
    const sh_config &c = m->cfg;
    PersistentKernel k = pick_persistent(m->dtype, c.kv_dtype, c.dim, m->qdim, c.hidden, c.head_dim);
    if (!k) return hipErrorInvalidValue;
    int cus = 0, per_cu = 0;
    hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, m->device);
    if (e != hipSuccess) return e;
    hipFuncAttributes fa{};
    if (hipFuncGetAttributes(&fa, (const void *)k) == hipSuccess)
        *why = "k_decode_persistent: " + std::to_string(fa.numRegs) + " VGPRs, " +
               std::to_string(fa.sharedSizeBytes) + " B LDS, " + std::to_string(fa.localSizeBytes) +
               " B scratch, max " + std::to_string(fa.maxThreadsPerBlock) + " threads";
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)k, kPB, 0);
    if (e != hipSuccess) return e;
    *why += "; " + std::to_string(per_cu) + " workgroup(s) of " + std::to_string(kPB) + " per CU";
    if (per_cu < 1) return hipErrorInvalidConfiguration;
    auto cdiv = [](int a, int b) { return (a + b - 1) / b; };
    auto up = [&](int a, int b) { return cdiv(a, b) * b; };
    const int rows13 = 2 * c.hidden;
    int grid = std::min(cus, kPB);
    grid = std::min(grid, rows13 / 2);
    auto per13_for = [&](int g) { return up(cdiv(rows13, g), 2); };
    while (grid > 1 && cdiv(rows13, per13_for(grid)) != grid) grid--;
    const int KVH = c.n_kv_heads, NA = attn_workgroups(m);
    if (grid < NA) return hipErrorInvalidConfiguration;
    const int wbytes = m->dtype == SH_DTYPE_W8A8 ? 1 : 2;   // bytes per weight
    // w2 on every workgroup (its weights are the second largest; a few rows each keeps the
    // weight tiles loaded after the w13 stage small), unless the layout below applies
    int per_w2 = cdiv(c.dim, grid);
    int n_w2 = cdiv(c.dim, per_w2);
    // qkv: blocks of 16 rows (whole lines of the dense qkv vector) spread over the grid,
    // after the attention workgroups when they fit
    const int per_qkv = up(cdiv(m->qkv_rows, grid), 16);
    const int n_qkv = cdiv(m->qkv_rows, per_qkv);
    // wo: about 24 KB of weights per workgroup (its workgroups are idle through qkv and
    // attention, so their tiles arrive long before att), at most kMaxRes rows
    int per_wo = std::max(1, std::min(kMaxRes, 24576 / (m->qdim * wbytes)));
    if (cdiv(c.dim, per_wo) > grid) per_wo = cdiv(c.dim, grid);
    const int n_wo = cdiv(c.dim, per_wo);
    const int off_qkv = NA + n_qkv <= grid ? NA : 0;
    int off_wo = off_qkv + n_qkv;
    if (off_wo + n_wo > grid) off_wo = NA + n_wo <= grid ? NA : 0;
    int per13 = per13_for(grid), n13 = grid, off_w2 = 0;
    // Where it fits: w13 on the first half of the grid with blocks its register tile holds
    // whole (those workgroups are idle through wo, which sits after qkv), and w2 on the
    // workgroups after the qkv block, so neither w2 nor the next layer's qkv workgroups are
    // busy with the stage before theirs when its input arrives. Stories110M fp16: 158.5 against
    // 170.3 us per forward with w13 and w2 on every workgroup. w13 then no longer spans the
    // grid, so the next-token exchange runs after every forward (argmax_every).
    {
        const int tile13 = 2 * kPW * (64 / shape_ld(m->dtype, c.dim));   // rows of w13's WTile<2>
        const int h13 = grid / 2, p13 = up(cdiv(rows13, std::max(h13, 1)), 2);
        const int o2 = off_qkv + n_qkv, p2 = o2 < grid ? cdiv(c.dim, grid - o2) : kMaxRes + 1;
        if (h13 >= 1 && p13 <= tile13 && p2 <= kMaxRes) {
            per13 = p13;
            n13 = cdiv(rows13, p13);
            per_w2 = p2;
            n_w2 = cdiv(c.dim, p2);
            off_w2 = o2;
        }
    }
    m->p_argmax_every = n13 < grid;
    m->p_grid = grid;
    m->p_own[0] = StageOwn{off_qkv, n_qkv, per_qkv};
    m->p_own[1] = StageOwn{off_wo, n_wo, per_wo};
    m->p_own[2] = StageOwn{0, n13, per13};
    m->p_own[3] = StageOwn{off_w2, n_w2, per_w2};
    m->p_own[4] = StageOwn{0, grid, cdiv(c.vocab, grid)};
    // classifier: the attention workgroups keep only their register tile's rows (their LDS
    // holds the attention cache); the others twice that, the second half resident in LDS for
    // the launch, where the vocabulary splits so and those rows fit the cache stage
    m->p_own_cls_a = StageOwn{0, 0, 0, 0};
    m->p_cls_lds_rows = 0;
    {
        const int rt = 4 * kPW * (64 / shape_ld(m->dtype, c.dim));
        const int row_bytes = c.dim * wbytes;
        const int rest = c.vocab - KVH * rt;
        const int per_b = rest > 0 && grid > KVH ? cdiv(rest, grid - KVH) : 0;
        if (m->dtype != SH_DTYPE_W8A8 && c.head_dim == 64 && per_b > rt && per_b <= 2 * rt &&
            (per_b - rt) * row_bytes <= kKvStage) {
            m->p_own_cls_a = StageOwn{0, KVH, rt, 0};
            m->p_own[4] = StageOwn{KVH, grid - KVH, per_b, KVH * rt};
            m->p_cls_lds_rows = per_b - rt;
        }
    }
    if (per_wo > kMaxRes || per_w2 > kMaxRes) return hipErrorInvalidConfiguration;
    if (per_qkv > kMaxPer || per13 > kMaxPer) return hipErrorInvalidConfiguration;
    m->p_ostride[0] = per_qkv;   // a multiple of 16: qkv stays dense for the attention stage
    m->p_ostride[1] = up(per_wo, 16);
    m->p_ostride[2] = up(per13 / 2, 16);
    m->p_ostride[3] = up(per_w2, 16);
    m->p_ostride[4] = 0;
    *why += "; rows/workgroups qkv " + std::to_string(per_qkv) + "x" + std::to_string(n_qkv) + " wo " +
            std::to_string(per_wo) + "x" + std::to_string(n_wo) + " w13 " + std::to_string(per13) + "x" +
            std::to_string(n13) + " w2 " + std::to_string(per_w2) + "x" + std::to_string(n_w2) +
            (off_w2 ? " from workgroup " + std::to_string(off_w2) : std::string("")) +
            (m->p_cls_lds_rows ? " classifier " + std::to_string(m->p_own_cls_a.per) + "x" +
                                     std::to_string(m->p_own_cls_a.n) + " + " + std::to_string(m->p_own[4].per) +
                                     "x" + std::to_string(m->p_own[4].n) + " (" +
                                     std::to_string(m->p_cls_lds_rows) + " rows each resident in LDS)"
                               : std::string(""));
    return hipSuccess;
}

hipError_t launch_persistent(sh_model *m, int pos0, int n_forwards, int n_prompt) {
    const sh_config &c = m->cfg;
    PersistentKernel k = pick_persistent(m->dtype, c.kv_dtype, c.dim, m->qdim, c.hidden, c.head_dim);
    if (!k) return hipErrorInvalidValue;
    PParams p{};
    p.D = c.dim;
    p.F = c.hidden;
    p.H = c.n_heads;
    p.KVH = c.n_kv_heads;
    p.NA = attn_workgroups(m);
    p.hd = c.head_dim;
    p.V = c.vocab;
    p.max_seq = c.max_seq;
    p.L = c.n_layers;
    p.qdim = m->qdim;
    p.kvdim = m->kvdim;
    p.qkv_rows = m->qkv_rows;
    p.alpha = c.residual_scale;
    p.inv_sqrt_hd = (float)(1.0 / sqrt((double)c.head_dim));
    p.eps = c.norm_eps;
    p.qk_eps = c.qk_norm_eps;
    p.qk_norm = c.qk_norm;
    p.layers = (const LayerPtrs *)m->p_layers;
    p.embed = (const uint16_t *)m->embed;
    p.cls = m->cls;
    p.s_cls = m->s_cls;
    p.rms_final = m->rms_final;
    p.kcache = m->kcache;
    p.vcache = m->vcache;
    p.rope_cos = m->rope_cos;
    p.rope_sin = m->rope_sin;
    p.ll_qkv = m->ll_qkv;
    p.ll_att = m->ll_att;
    p.ll_x2 = m->ll_x2;
    p.ll_gate = m->ll_gate;
    p.ll_x = m->ll_x;
    p.ll_pv = m->ll_pv;
    p.ll_pi = m->ll_pi;
    p.logits = m->logits;
    p.tokens = m->tokens;
    p.hist = m->argmax_hist;
    p.pos0 = pos0;
    p.n_forwards = n_forwards;
    p.n_prompt = n_prompt;
    p.epoch0 = m->epoch;
    p.err = m->p_err;
    p.fail_mode = m->fail_next;
    m->fail_next = 0;
    p.spin_limit = m->spin_ticks;
    // The abort flag is an agent-scope load, a full round trip to the memory side: read on
    // every retry it doubles a retry's period, so a hand-over is noticed half a round trip
    // later on average. A wait reads it only once it has lasted 20 us (no hand-over of a
    // running decode takes that long), which still ends every wave soon after an abort.
    p.quiet = m->spin_ticks / 100000;
    p.trace = m->trace_f >= 0 ? m->trace_buf : nullptr;
    p.trace_f = m->trace_f;
    p.own_cls_a = m->p_own_cls_a;
    p.cls_lds_rows = m->p_cls_lds_rows;
    p.argmax_every = m->p_argmax_every;
    for (int i = 0; i < 5; i++) {
        p.own[i] = m->p_own[i];
        p.ostride[i] = m->p_ostride[i];
        // elements per output block: rows, or row pairs for the gate vector
        const int per = i == 2 ? m->p_own[i].per / 2 : m->p_own[i].per;
        p.omagic[i] = per > 0 ? (uint32_t)((0x80000000ull + (uint64_t)per - 1) / (uint64_t)per) : 0u;
    }
    m->epoch += (uint32_t)n_forwards * (uint32_t)(c.n_layers + 1);
    // A plain launch: the kernel needs its workgroups co-resident (persistent_plan keeps the
    // grid within CUs x resident workgroups per CU) but never synchronises the whole grid, so
    // the cooperative-launch path is not needed. Should a workgroup not become resident (another
    // process holding CUs), the bounded waits end the launch with *err set.
    void *args[] = {&p};
    return hipLaunchKernel((const void *)k, dim3(m->p_grid), dim3(kPB), args, 0, m->stream);
}

size_t persistent_layer_ptr_bytes(int n_layers) { return sizeof(LayerPtrs) * (size_t)n_layers; }

void persistent_fill_layer_ptrs(const sh_model *m, void *host) {
    LayerPtrs *lp = (LayerPtrs *)host;
    for (int l = 0; l < m->cfg.n_layers; l++) {
        const LayerDev &L = m->layers[l];
        lp[l].wqkv = L.wqkv;
        lp[l].wo = L.wo;
        lp[l].w13 = L.w13;
        lp[l].w2 = L.w2;
        lp[l].s_qkv = L.s_qkv;
        lp[l].s_o = L.s_o;
        lp[l].s_13 = L.s_13;
        lp[l].s_2 = L.s_2;
        lp[l].rms_att = L.rms_att;
        lp[l].rms_ffn = L.rms_ffn;
        lp[l].q_norm = L.q_norm;
        lp[l].k_norm = L.k_norm;
    }
}

}  // namespace sh
