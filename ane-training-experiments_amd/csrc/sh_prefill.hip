// sh_prefill.hip — the full-sequence causal forward (ane/storiesane/engine.go:804-842,
// evalLogitsCPUInto) for gfx950.
//
// Activations are token-major ([S, C], row t = token t); the reference's channel-first
// [C, S] layout (forward_common.go:35-46) only appears in the logits output. Every
// projection is an "NT" product Y[S, N] = X[S, K] . W[N, K]^T: activation rows and weight
// rows are both contiguous in K, which is exactly the operand layout of
// v_mfma_f32_16x16x32_{f16,bf16} (lane l holds row l%16, k = 8*(l/16) .. +7), so each wave
// feeds its MFMAs with plain 16-byte loads. The activation operand is carried as two planes
// of the weight type, hi = round(a) and lo = round(a - hi), and each block is two MFMAs
// (hi.W + lo.W): about 16 significant bits of the fp32 activation reach the product, so the
// result tracks the reference's fp32 CPU path instead of a 8- or 11-bit rounding of it.
// Accumulation, q/k/v, attention, the residual stream and every normalisation stay
// fp32/fp64 as in the reference.
//
// Per layer: rmsnorm -> qkv GEMM -> qk-norm/RoPE (+ optional KV-cache fill) -> causal
// attention -> Wo GEMM (+residual) -> rmsnorm -> W1/W3 GEMM (+silu gate) -> W2 GEMM
// (+residual). Then the final RMSNorm and the classifier GEMM writing logits [V, S].
#include <hip/hip_fp16.h>
#include <math.h>

#include "sh_internal.hpp"

namespace sh {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kT = 256;   // threads per workgroup of the row kernels and GEMM

__device__ __forceinline__ float bits_to_f(uint16_t b, int dt) {
    return dt == SH_DTYPE_BF16 ? __uint_as_float((uint32_t)b << 16)
                               : __half2float(__ushort_as_half(b));
}
__device__ __forceinline__ uint16_t f_to_bits(float f, int dt) {
    if (dt == SH_DTYPE_BF16) {
        uint32_t u = __float_as_uint(f);
        if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
        u += 0x7fffu + ((u >> 16) & 1u);
        return (uint16_t)(u >> 16);
    }
    return __half_as_ushort(__float2half_rn(f));
}

// Writes v as a GEMM operand: the hi plane at idx, the lo plane `plane` elements further.
__device__ __forceinline__ void store_op(uint16_t *base, size_t idx, size_t plane, float v,
                                         int dt) {
    const uint16_t hi = f_to_bits(v, dt);
    base[idx] = hi;
    base[plane + idx] = f_to_bits(v - bits_to_f(hi, dt), dt);
}

__device__ __forceinline__ double block_sum(double v, double *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double s = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) s += red[w];
    return s;
}

// cpu.go:41-72 EmbedLookup in token-major form: out-of-range ids give a zero row.
__global__ __launch_bounds__(kT) void k_embed_rows(const uint16_t *embed, const int32_t *tokens,
                                                   int vocab, int dim, int dt, float *x) {
    const int t = blockIdx.x;
    const int tok = tokens[t];
    const bool ok = tok >= 0 && tok < vocab;
    for (int i = threadIdx.x; i < dim; i += blockDim.x)
        x[(size_t)t * dim + i] = ok ? bits_to_f(embed[(size_t)tok * dim + i], dt) : 0.f;
}

// One token row per workgroup. final_form = 0: rmsNormCFWithRRMSImpl (accel_other.go:11-28,
// float32 scale, x*scale*w in float32); 1: stories.RMSNorm (cpu.go:97-111, float64 product
// rounded once). The normalised row is written as a GEMM operand (hi/lo planes).
__global__ __launch_bounds__(kT) void k_rmsnorm_rows(const float *x, const float *w, int dim,
                                                     double eps, int final_form, int dt,
                                                     uint16_t *out, size_t plane) {
    __shared__ double red[kT / 64];
    const float *row = x + (size_t)blockIdx.x * dim;
    double ss = 0;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) ss += (double)row[i] * (double)row[i];
    const double tot = block_sum(ss, red);
    const double rr = 1.0 / sqrt(tot / (double)dim + eps);
    const float scale = (float)rr;
    const size_t o = (size_t)blockIdx.x * dim;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) {
        const float v = final_form ? (float)((double)row[i] * rr * (double)w[i]) : row[i] * scale * w[i];
        store_op(out, o + i, plane, v, dt);
    }
}

enum { G_STORE = 0, G_RESID = 1, G_GATE = 2, G_LOGITS_CF = 3 };

struct GemmArgs {
    const uint16_t *A;   // [M, K] activations, hi plane; the lo plane follows at M*K
    const uint16_t *B;   // [N, K] weight rows
    int M, N, K;
    int epi;
    float *out;          // G_STORE / G_RESID: [M, N]; G_LOGITS_CF: [N, M]
    const float *resid;  // G_RESID
    float alpha;
    uint16_t *out16;     // G_GATE: [M, N/2] operand planes (lo at M*N/2)
    int dt;
};

template <int DT>
__device__ __forceinline__ f32x4 mfma16(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
    if constexpr (DT == SH_DTYPE_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a),
                                                      __builtin_bit_cast(half8, b), c, 0, 0, 0);
}

// Workgroup tile 64 x 64 (4 waves of 32 x 32 = 2 x 2 MFMA blocks), K step 32.
// Requires K % 32 == 0 and N % 64 == 0; rows >= M read zeros and are not written.
template <int DT>
__global__ __launch_bounds__(kT) void k_gemm_nt(GemmArgs g) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m0 = blockIdx.x * 64 + (wave >> 1) * 32;
    const int n0 = blockIdx.y * 64 + (wave & 1) * 32;
    const int lr = lane & 15, lk = (lane >> 4) * 8;
    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
    const uint16_t *arow[2], *brow[2];
    const size_t lo = (size_t)g.M * g.K;
    bool aok[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int m = m0 + i * 16 + lr;
        aok[i] = m < g.M;
        arow[i] = g.A + (size_t)(aok[i] ? m : 0) * g.K + lk;
        brow[i] = g.B + (size_t)(n0 + i * 16 + lr) * g.K + lk;
    }
    for (int k0 = 0; k0 < g.K; k0 += 64) {
        u32x4 a[2][2], al[2][2], b[2][2];
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int k = k0 + s * 32;
            const bool kin = k < g.K;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                a[s][i] = (aok[i] && kin) ? *(const u32x4 *)(arow[i] + k) : zero;
                al[s][i] = (aok[i] && kin) ? *(const u32x4 *)(arow[i] + lo + k) : zero;
                b[s][i] = kin ? *(const u32x4 *)(brow[i] + k) : zero;
            }
        }
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    acc[i][j] = mfma16<DT>(a[s][i], b[s][j], acc[i][j]);
                    acc[i][j] = mfma16<DT>(al[s][i], b[s][j], acc[i][j]);
                }
    }
    // D layout: lane holds column lr of the 16x16 block, rows 4*(lane/16) + r
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + j * 16 + lr;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + i * 16 + (lane >> 4) * 4 + r;
                const float v = acc[i][j][r];
                if (g.epi == G_GATE) {
                    // rows 2q (W1) and 2q+1 (W3) of the weight are adjacent columns here
                    const float h3 = __shfl_xor(v, 1, 64);
                    if ((n & 1) == 0 && m < g.M) {
                        // accel_other.go:128-133 siluGateForwardAccel
                        const float sig = (float)(1.0 / (1.0 + exp(-(double)v)));
                        store_op(g.out16, (size_t)m * (g.N / 2) + (n >> 1), (size_t)g.M * (g.N / 2),
                                 (v * sig) * h3, g.dt);
                    }
                } else if (m < g.M) {
                    if (g.epi == G_STORE) g.out[(size_t)m * g.N + n] = v;
                    else if (g.epi == G_RESID)
                        g.out[(size_t)m * g.N + n] = g.resid[(size_t)m * g.N + n] + g.alpha * v;
                    else g.out[(size_t)n * g.M + m] = v;   // logits[v*S + t]
                }
            }
        }
}

// Per token: optional per-head RMSNorm of q and k, RoPE on q and k (rope.go:26-46:
// e' = e*c - o*s, o' = o*c + e*s); q, k, v written fp32 token-major; optionally the roped k
// and v also enter the KV cache (kcache/vcache point at this sequence's layer slab).
template <int KVT>
__global__ __launch_bounds__(kT) void k_qk_rope(const float *qkv, int qdim, int kvdim, int hd,
                                                int qk_norm, const float *q_norm,
                                                const float *k_norm, double qk_eps,
                                                const float *rope_cos, const float *rope_sin,
                                                float *qo, float *ko, float *vo,
                                                void *kcache, void *vcache, int write_cache) {
    __shared__ float row[4096];
    const int t = blockIdx.x;
    const int n = qdim + 2 * kvdim;
    for (int i = threadIdx.x; i < n; i += blockDim.x) row[i] = qkv[(size_t)t * n + i];
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int heads = (qdim + kvdim) / hd;   // q heads, then k heads
    if (qk_norm) {
        for (int h = wave; h < heads; h += nw) {
            float *v = row + h * hd;
            const float *g = h < qdim / hd ? q_norm : k_norm;
            double ss = 0;
            for (int i = lane; i < hd; i += 64) ss += (double)v[i] * (double)v[i];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
            const float rr = (float)(1.0 / sqrt(ss / (double)hd + qk_eps));
            for (int i = lane; i < hd; i += 64) v[i] = v[i] * rr * g[i];
        }
        __syncthreads();
    }
    const int half = hd / 2;
    for (int p = threadIdx.x; p < (qdim + kvdim) / 2; p += blockDim.x) {
        const int pi = p % half;
        const float c = rope_cos[t * half + pi], s = rope_sin[t * half + pi];
        const float e = row[2 * p], o = row[2 * p + 1];
        row[2 * p] = e * c - o * s;
        row[2 * p + 1] = o * c + e * s;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = row[i];
        if (i < qdim) {
            qo[(size_t)t * qdim + i] = v;
        } else if (i < qdim + kvdim) {
            const int j = i - qdim;
            ko[(size_t)t * kvdim + j] = v;
            if (write_cache) {
                const size_t o = (size_t)t * kvdim + j;
                if (KVT == SH_KV_F32) ((float *)kcache)[o] = v;
                else ((uint16_t *)kcache)[o] = f_to_bits(v, KVT == SH_KV_BF16 ? SH_DTYPE_BF16 : SH_DTYPE_F16);
            }
        } else {
            const int j = i - qdim - kvdim;
            vo[(size_t)t * kvdim + j] = v;
            if (write_cache) {
                const size_t o = (size_t)t * kvdim + j;
                if (KVT == SH_KV_F32) ((float *)vcache)[o] = v;
                else ((uint16_t *)vcache)[o] = f_to_bits(v, KVT == SH_KV_BF16 ? SH_DTYPE_BF16 : SH_DTYPE_F16);
            }
        }
    }
}

// Causal attention (forward_common.go:5-33): one wave per (query t, head h). Lanes walk the
// keys j <= t in blocks of 64; scores are kept in LDS, then the softmax of
// accel_other.go:190-207 (float64 exp terms summed unrounded, p = float32(e) * float32(1/sum);
// masked keys contribute exactly 0) and P.V with lanes over the head dims.
__global__ __launch_bounds__(kT) void k_attn_prefill(const float *qf, const float *kf,
                                                     const float *vf, int S, int H, int KVH,
                                                     int hd, float scale, int dt,
                                                     uint16_t *att, size_t plane) {
    extern __shared__ float sh_scores[];   // [waves][S]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x * (blockDim.x >> 6) + wave;
    const int h = blockIdx.y;
    if (t >= S) return;
    const int qdim = H * hd, kvdim = KVH * hd, kvh = h / (H / KVH);
    float *sc = sh_scores + (size_t)wave * S;
    const float *q = qf + (size_t)t * qdim + h * hd;
    float mx = -INFINITY;
    for (int j0 = 0; j0 <= t; j0 += 64) {
        const int j = j0 + lane;
        float s = -INFINITY;
        if (j <= t) {
            const float *k = kf + (size_t)j * kvdim + kvh * hd;
            float d = 0.f;
            for (int i = 0; i < hd; i += 4) {
                const f32x4 qa = *(const f32x4 *)(q + i), ka = *(const f32x4 *)(k + i);
#pragma unroll
                for (int w = 0; w < 4; w++) d = fmaf(qa[w], ka[w], d);
            }
            s = d * scale;
            sc[j] = s;
        }
        mx = fmaxf(mx, s);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    double sum = 0;
    for (int j = lane; j <= t; j += 64) {
        const double e = exp((double)(sc[j] - mx));
        sc[j] = (float)e;
        sum += e;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    const float inv = (float)(1.0 / sum);
    __builtin_amdgcn_wave_barrier();
    for (int i = lane; i < hd; i += 64) {
        float a = 0.f;
        for (int j = 0; j <= t; j++)
            a = fmaf(sc[j] * inv, vf[(size_t)j * kvdim + kvh * hd + i], a);
        store_op(att, (size_t)t * qdim + h * hd + i, plane, a, dt);
    }
}

hipError_t gemm(const GemmArgs &g, int dt, hipStream_t s) {
    if (g.K % 32 || g.N % 64) return hipErrorInvalidValue;
    dim3 grid((g.M + 63) / 64, g.N / 64);
    if (dt == SH_DTYPE_BF16) hipLaunchKernelGGL(k_gemm_nt<SH_DTYPE_BF16>, grid, dim3(kT), 0, s, g);
    else hipLaunchKernelGGL(k_gemm_nt<SH_DTYPE_F16>, grid, dim3(kT), 0, s, g);
    return hipGetLastError();
}

}  // namespace

bool prefill_supported(const sh_model *m, std::string *why) {
    const sh_config &c = m->cfg;
    if (m->dtype != SH_DTYPE_F16 && m->dtype != SH_DTYPE_BF16) {
        *why = "full-sequence forward needs fp16 or bf16 weights";
        return false;
    }
    if (c.dim % 64 || m->qdim % 64 || c.hidden % 64 || c.vocab % 64 || m->qkv_rows % 64 ||
        (2 * c.hidden) % 64) {
        *why = "full-sequence forward needs dims that are multiples of 64";
        return false;
    }
    if (m->qkv_rows > 4096) {
        *why = "q/k/v width above 4096";
        return false;
    }
    return true;
}

hipError_t prefill_alloc(sh_model *m, int S) {
    if (m->pf_cap >= S) return hipSuccess;
    const sh_config &c = m->cfg;
    (void)hipFree(m->pf_arena);
    m->pf_arena = nullptr;
    m->pf_cap = 0;
    const size_t D = c.dim, F = c.hidden, Q = m->qdim, KV = m->kvdim, R = m->qkv_rows, V = c.vocab;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += (bytes + 255) / 256 * 256;
        return o;
    };
    const size_t o_tok = take(4 * S), o_x = take(4 * S * D), o_x2 = take(4 * S * D),
                 o_xn = take(4 * S * D), o_qkv = take(4 * S * R), o_q = take(4 * S * Q),
                 o_k = take(4 * S * KV), o_v = take(4 * S * KV), o_att = take(4 * S * Q),
                 o_gate = take(4 * S * F), o_log = take(4 * V * S);
    hipError_t e = hipMalloc(&m->pf_arena, off);
    if (e != hipSuccess) return e;
    uint8_t *A = (uint8_t *)m->pf_arena;
    m->pf_tokens = (int32_t *)(A + o_tok);
    m->pf_x = (float *)(A + o_x);
    m->pf_x2 = (float *)(A + o_x2);
    m->pf_xn = (uint16_t *)(A + o_xn);
    m->pf_qkv = (float *)(A + o_qkv);
    m->pf_q = (float *)(A + o_q);
    m->pf_k = (float *)(A + o_k);
    m->pf_v = (float *)(A + o_v);
    m->pf_att = (uint16_t *)(A + o_att);
    m->pf_gate = (uint16_t *)(A + o_gate);
    m->pf_logits = (float *)(A + o_log);
    m->pf_cap = S;
    return hipSuccess;
}

// Enqueues the whole forward for pf_tokens[0, S); logits (if wanted) land in pf_logits as
// [V, S]. kv_seq >= 0 fills that sequence's KV cache rows [0, S) on the way.
hipError_t enqueue_prefill(sh_model *m, int S, bool logits, int kv_seq) {
    const sh_config &c = m->cfg;
    const int dt = m->dtype;
    const int D = c.dim, F = c.hidden;
    hipStream_t s = m->stream;
    hipError_t e;
    hipLaunchKernelGGL(k_embed_rows, dim3(S), dim3(kT), 0, s, (const uint16_t *)m->embed,
                       m->pf_tokens, c.vocab, D, dt, m->pf_x);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const float scale = (float)(1.0 / sqrt((double)c.head_dim));
    const size_t kv_layer = (size_t)c.max_seq * m->kvdim;
    const size_t kv_seq_stride = kv_layer * c.n_layers;
    const size_t kvb = c.kv_dtype == SH_KV_F32 ? 4 : 2;
    for (int l = 0; l < c.n_layers; l++) {
        const LayerDev &L = m->layers[l];
        hipLaunchKernelGGL(k_rmsnorm_rows, dim3(S), dim3(kT), 0, s, m->pf_x, L.rms_att, D,
                           c.norm_eps, 0, dt, m->pf_xn, (size_t)S * D);
        GemmArgs g{};
        g.A = m->pf_xn; g.B = (const uint16_t *)L.wqkv; g.M = S; g.N = m->qkv_rows; g.K = D;
        g.epi = G_STORE; g.out = m->pf_qkv; g.dt = dt;
        if ((e = gemm(g, dt, s)) != hipSuccess) return e;
        void *kc = nullptr, *vc = nullptr;
        if (kv_seq >= 0) {
            const size_t o = ((size_t)kv_seq * kv_seq_stride + (size_t)l * kv_layer) * kvb;
            kc = (uint8_t *)m->kcache + o;
            vc = (uint8_t *)m->vcache + o;
        }
#define SH_QKR(KVT)                                                                           \
    hipLaunchKernelGGL(k_qk_rope<KVT>, dim3(S), dim3(kT), 0, s, m->pf_qkv, m->qdim, m->kvdim,  \
                       c.head_dim, c.qk_norm, L.q_norm, L.k_norm, c.qk_norm_eps, m->rope_cos,  \
                       m->rope_sin, m->pf_q, m->pf_k, m->pf_v, kc, vc, kv_seq >= 0 ? 1 : 0)
        if (c.kv_dtype == SH_KV_F32) SH_QKR(SH_KV_F32);
        else if (c.kv_dtype == SH_KV_F16) SH_QKR(SH_KV_F16);
        else SH_QKR(SH_KV_BF16);
#undef SH_QKR
        const int wpb = kT / 64;
        hipLaunchKernelGGL(k_attn_prefill, dim3((S + wpb - 1) / wpb, c.n_heads), dim3(kT),
                           sizeof(float) * wpb * S, s, m->pf_q, m->pf_k, m->pf_v, S, c.n_heads,
                           c.n_kv_heads, c.head_dim, scale, dt, m->pf_att, (size_t)S * m->qdim);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        g = GemmArgs{};
        g.A = m->pf_att; g.B = (const uint16_t *)L.wo; g.M = S; g.N = D; g.K = m->qdim;
        g.epi = G_RESID; g.out = m->pf_x2; g.resid = m->pf_x; g.alpha = c.residual_scale; g.dt = dt;
        if ((e = gemm(g, dt, s)) != hipSuccess) return e;
        hipLaunchKernelGGL(k_rmsnorm_rows, dim3(S), dim3(kT), 0, s, m->pf_x2, L.rms_ffn, D,
                           c.norm_eps, 0, dt, m->pf_xn, (size_t)S * D);
        g = GemmArgs{};
        g.A = m->pf_xn; g.B = (const uint16_t *)L.w13; g.M = S; g.N = 2 * F; g.K = D;
        g.epi = G_GATE; g.out16 = m->pf_gate; g.dt = dt;
        if ((e = gemm(g, dt, s)) != hipSuccess) return e;
        g = GemmArgs{};
        g.A = m->pf_gate; g.B = (const uint16_t *)L.w2; g.M = S; g.N = D; g.K = F;
        g.epi = G_RESID; g.out = m->pf_x; g.resid = m->pf_x2; g.alpha = c.residual_scale; g.dt = dt;
        if ((e = gemm(g, dt, s)) != hipSuccess) return e;
    }
    if (!logits) return hipSuccess;
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(S), dim3(kT), 0, s, m->pf_x, m->rms_final, D,
                       c.norm_eps, 1, dt, m->pf_xn, (size_t)S * D);
    GemmArgs g{};
    g.A = m->pf_xn; g.B = (const uint16_t *)m->cls; g.M = S; g.N = c.vocab; g.K = D;
    g.epi = G_LOGITS_CF; g.out = m->pf_logits; g.dt = dt;
    return gemm(g, dt, s);
}

}  // namespace sh
