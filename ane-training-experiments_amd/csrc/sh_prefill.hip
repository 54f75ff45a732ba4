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

#include <algorithm>
#include <vector>

#include "sh_internal.hpp"
#include "sh_tiles.hpp"
#include "sh_wave.hpp"

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
// Round to nearest even in the hardware conversions (v_cvt_pk_bf16_f32 / v_cvt_f16_f32).
__device__ __forceinline__ uint16_t f_to_bits(float f, int dt) {
    if (dt == SH_DTYPE_BF16) return __builtin_bit_cast(uint16_t, (__bf16)f);
    return __half_as_ushort(__float2half_rn(f));
}

// Writes v as a 16-bit GEMM operand: the hi plane at idx, the lo plane `plane` elements
// further (dt fp16 or bf16).
__device__ __forceinline__ void store_op16(uint16_t *base, size_t idx, size_t plane, float v,
                                           int dt) {
    const uint16_t hi = f_to_bits(v, dt);
    base[idx] = hi;
    base[plane + idx] = f_to_bits(v - bits_to_f(hi, dt), dt);
}

// store_op16 for the kernels a W8A8 model also runs (row kernels, the plane conversion):
// W8A8 carries the operand as fp32 instead (element idx of the same buffer viewed as float,
// whose 2 * plane 16-bit slots hold exactly `plane` floats), so the per-row quantizer sees
// the value itself, as the reference's quantizer does.
__device__ __forceinline__ void store_op(uint16_t *base, size_t idx, size_t plane, float v, int dt) {
    if (dt == SH_DTYPE_W8A8) ((float *)base)[idx] = v;
    else store_op16(base, idx, plane, v, dt);
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
// rounded once). The normalised row is written as a GEMM operand (hi/lo planes), or as fp32
// rows into out32 when that is given.
__global__ __launch_bounds__(kT) void k_rmsnorm_rows(const float *x, const float *w, int dim,
                                                     double eps, int final_form, int dt,
                                                     uint16_t *out, size_t plane,
                                                     float *out32 = nullptr) {
    __shared__ double red[kT / 64];
    const float *row = x + (size_t)blockIdx.x * dim;
    double ss = 0;
    for (int i4 = threadIdx.x; i4 < dim / 4; i4 += blockDim.x) {   // dim % 4 == 0
        const f32x4 v = *(const f32x4 *)(row + 4 * i4);
        ss += (double)v.x * (double)v.x + (double)v.y * (double)v.y +
              (double)v.z * (double)v.z + (double)v.w * (double)v.w;
    }
    const double tot = block_sum(ss, red);
    const double rr = 1.0 / sqrt(tot / (double)dim + eps);
    const float scale = (float)rr;
    const size_t o = (size_t)blockIdx.x * dim;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) {
        const float v = final_form ? (float)((double)row[i] * rr * (double)w[i]) : row[i] * scale * w[i];
        if (out32) out32[o + i] = v;
        else store_op(out, o + i, plane, v, dt);
    }
}

// dst [cols, rows] = src [rows, cols]^T, fp32, through 32 x 33 LDS tiles (the channel-first
// <-> token-major conversion at the plugin-seam entry points).
__global__ __launch_bounds__(kT) void k_transpose(const float *src, int rows, int cols, float *dst) {
    __shared__ float tile[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int j = ty; j < 32; j += kT / 32) {
        const int r = r0 + j, c = c0 + tx;
        if (r < rows && c < cols) tile[j][tx] = src[(size_t)r * cols + c];
    }
    __syncthreads();
    for (int j = ty; j < 32; j += kT / 32) {
        const int c = c0 + j, r = r0 + tx;
        if (c < cols && r < rows) dst[(size_t)c * rows + r] = tile[tx][j];
    }
}

// fp32 values as GEMM operand planes (hi at i, lo `plane` further).
__global__ __launch_bounds__(kT) void k_to_planes(const float *x, size_t n, int dt, uint16_t *out,
                                                  size_t plane) {
    const size_t i = (size_t)blockIdx.x * kT + threadIdx.x;
    if (i < n) store_op(out, i, plane, x[i], dt);
}

// dst [count, S] (channel-first) = columns col0, col0 + cstep, ... of the token-major src
// [S, ncols]: dst[c*S + t] = src[t*ncols + col0 + c*cstep]. The layer taps' layout change.
__global__ __launch_bounds__(kT) void k_cf_gather(const float *src, int S, int ncols, int col0,
                                                  int cstep, int count, float *dst) {
    const size_t i = (size_t)blockIdx.x * kT + threadIdx.x;
    if (i >= (size_t)count * S) return;
    const int c = (int)(i / S), t = (int)(i % S);
    dst[i] = src[(size_t)t * ncols + col0 + (size_t)c * cstep];
}

// fp32 value of operand planes: hi + lo (hi at i, lo `plane` further); W8A8: the fp32 operand.
__global__ __launch_bounds__(kT) void k_planes_f32(const uint16_t *in, size_t n, size_t plane, int dt,
                                                   float *out) {
    const size_t i = (size_t)blockIdx.x * kT + threadIdx.x;
    if (i < n)
        out[i] = dt == SH_DTYPE_W8A8 ? ((const float *)in)[i]
                                     : bits_to_f(in[i], dt) + bits_to_f(in[plane + i], dt);
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
    int decode_forms;    // G_GATE: 1 = infer.go:324-326 silu, 0 = accel_other.go:128-133
    int partial_only;    // skinny GEMM: always leave K-range partials, no epilogue
    int one_plane;       // pipelined fp16 GEMMs: A's hi plane only (lo neither read nor used)
    // W8A8 models: B holds int8 rows with fp32 row scales sw [N]; A is the fp32 operand
    // [M, K], which the product quantizes per row into a8 [M, K] with scales sa [M] first
    const float *sw;
    int8_t *a8;
    float *sa;
};

// silu(h1) * h3: decode form x / (1 + float32(exp(-x))) (infer.go:324-326), or the
// full-sequence form (h1 * float32(1 / (1 + exp(-h1)))) * h3 (accel_other.go:128-133).
// EXACT (the W8A8 products, whose gate values feed a quantizer): the reference's float64
// exp, rounded as it rounds. Otherwise (the 16-bit models) float expf, the form their decode
// kernel computes: within an ulp or so of the float64 form, at a fraction of its cost.
template <bool EXACT>
__device__ __forceinline__ float silu_gate(float h1, float h3, int decode_forms) {
    if constexpr (EXACT) {
        if (decode_forms) return (h1 / (1.0f + (float)exp(-(double)h1))) * h3;
        const float sig = (float)(1.0 / (1.0 + exp(-(double)h1)));
        return (h1 * sig) * h3;
    } else {
        if (decode_forms) return (h1 / (1.0f + expf(-h1))) * h3;
        const float sig = 1.0f / (1.0f + expf(-h1));
        return (h1 * sig) * h3;
    }
}

template <int DT>
__device__ __forceinline__ f32x4 mfma16(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
    if constexpr (DT == SH_DTYPE_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a),
                                                      __builtin_bit_cast(half8, b), c, 0, 0, 0);
}

// Epilogue of one output element pair (columns n, n+1 of row m) is shared with the skinny
// GEMM (skinny_epilogue); the tiled GEMM applies it per element with the same forms. Q8: the
// W8A8 product, whose gate operand is fp32 (store_op's W8A8 form).
template <bool Q8>
__device__ __forceinline__ void tile_epilogue(const GemmArgs &g, int m, int n, float v, float v_right) {
    if (g.epi == G_GATE) {
        if ((n & 1) == 0 && Q8)
            ((float *)g.out16)[(size_t)m * (g.N / 2) + (n >> 1)] = silu_gate<true>(v, v_right, g.decode_forms);
        else if ((n & 1) == 0)
            store_op16(g.out16, (size_t)m * (g.N / 2) + (n >> 1), (size_t)g.M * (g.N / 2),
                     silu_gate<Q8>(v, v_right, g.decode_forms), g.dt);
    } else if (g.epi == G_STORE) {
        g.out[(size_t)m * g.N + n] = v;
    } else if (g.epi == G_RESID) {
        g.out[(size_t)m * g.N + n] = g.resid[(size_t)m * g.N + n] + g.alpha * v;
    } else {
        g.out[(size_t)n * g.M + m] = v;   // logits[v*S + t]
    }
}

// A wave's FM x FN blocks of 16 x 16 results (rows from mb, columns from nb) to the K-range
// partials (more than one range) or through the epilogue. D layout: lane holds column
// lane%16 of each block, rows 4*(lane/16) + r. The gate epilogue pairs lanes n and n ^ 1
// (the W1 and W3 columns of one gate value, for the same four rows): after swapping their
// values, the even lane finishes rows 0-1 and the odd lane rows 2-3, so every lane computes
// two gate values instead of half the lanes computing four.
template <int FM, int FN>
__device__ __forceinline__ void tile_out(const GemmArgs &g, float *partial, const f32x4 (&acc)[FM][FN], int mb,
                                         int nb, int lane) {
    if (gridDim.z > 1) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int n = nb + j * 16 + (lane & 15);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = mb + i * 16 + (lane >> 4) * 4 + r;
                    if (m < g.M) partial[((size_t)blockIdx.z * g.M + m) * g.N + n] = acc[i][j][r];
                }
            }
        return;
    }
    if (g.epi == G_GATE) {
        const bool odd = lane & 1;
        const size_t plane = (size_t)g.M * (g.N / 2);
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int q = (nb + j * 16 + (lane & 15)) >> 1;
                // own and partner values of rows k and k + 2, chosen with a per-lane select
                // mask (a select of two array elements can become a dynamic index, in scratch)
                const uint32_t sel = odd ? ~0u : 0u;
                auto pick = [&](float lo_row, float hi_row) {
                    return __builtin_bit_cast(float, (__builtin_bit_cast(uint32_t, hi_row) & sel) |
                                                         (__builtin_bit_cast(uint32_t, lo_row) & ~sel));
                };
                const f32x4 av = acc[i][j];
                float vx[4];
#pragma unroll
                for (int r = 0; r < 4; r++) vx[r] = __shfl_xor(av[r], 1, 64);
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    const float own = pick(av[k], av[k + 2]);
                    const float oth = pick(vx[k], vx[k + 2]);
                    const int m = mb + i * 16 + (lane >> 4) * 4 + (odd ? k + 2 : k);
                    if (m < g.M)
                        store_op16(g.out16, (size_t)m * (g.N / 2) + q, plane,
                                   silu_gate<false>(odd ? oth : own, odd ? own : oth, g.decode_forms), g.dt);
                }
            }
        return;
    }
    if (g.epi == G_LOGITS_CF && (g.M & 3) == 0) {
        // channel-first logits: a lane's four rows are consecutive in memory, one 16-byte store
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int n = nb + j * 16 + (lane & 15), m = mb + i * 16 + (lane >> 4) * 4;
                if (m < g.M) *(f32x4 *)(g.out + (size_t)n * g.M + m) = acc[i][j];
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int n = nb + j * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = mb + i * 16 + (lane >> 4) * 4 + r;
                if (m < g.M) tile_epilogue<false>(g, m, n, acc[i][j][r], 0.f);
            }
        }
}

// Tiled MFMA GEMM: C[M, N] = A[M, K] . W[N, K]^T, A as hi/lo operand planes. Workgroup tile
// BM x BN (2 x 2 waves of BM/2 x BN/2, 16 x 16 x 32 MFMA blocks), K in steps of 32 through
// two LDS buffers: the next step's A hi, A lo and W rows are loaded into registers while
// the MFMAs of this step read the other buffer. LDS rows are 64 data bytes padded to 80, so
// the 16 rows x 4 chunks a wave reads for one fragment spread over the banks. Workgroup z
// covers K range [z*kc, (z+1)*kc); with more than one range the tile goes to `partial`
// ([ranges][M][N]) and k_gemm_skinny_reduce finishes it. Needs N % BN == 0, kc % 32 == 0.
template <int DT, int BM, int BN>
__global__ __launch_bounds__(kT) void k_gemm_tiled(GemmArgs g, float *partial, int kc) {
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 16, FN = WN / 16;
    constexpr int RS = 80;                       // LDS bytes per tile row (64 + 16 pad)
    constexpr int R = 2 * BM + BN;               // tile rows: A hi, A lo, W
    constexpr int PER = R * 4 / kT;              // 16-byte chunks per thread per step
    static_assert(R * 4 % kT == 0, "tile chunks must split evenly over the workgroup");
    __shared__ __attribute__((aligned(16))) uint8_t lds[2][R * RS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * WM, wn = (wave & 1) * WN;
    const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
    const int kbeg = blockIdx.z * kc, kend = kbeg + kc;
    const size_t lo = (size_t)g.M * g.K;
    const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
    u32x4 stage[PER];
    auto gload = [&](int k) {
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int ci = tid + j * kT, r = ci >> 2, c = ci & 3;
            if (r < 2 * BM) {
                const int m = m0 + (r < BM ? r : r - BM);
                const uint16_t *src = g.A + (r < BM ? 0 : lo) + (size_t)m * g.K + k + c * 8;
                stage[j] = m < g.M ? *(const u32x4 *)src : zero;
            } else {
                stage[j] = *(const u32x4 *)(g.B + (size_t)(n0 + r - 2 * BM) * g.K + k + c * 8);
            }
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int ci = tid + j * kT;
            *(u32x4 *)(&lds[buf][(ci >> 2) * RS + (ci & 3) * 16]) = stage[j];
        }
    };
    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    gload(kbeg);
    lstore(0);
    __syncthreads();
    int buf = 0;
    const int fr = lane & 15, fc = (lane >> 4) * 16;   // fragment row, byte offset of k chunk
    for (int k = kbeg; k < kend; k += 32) {
        const bool more = k + 32 < kend;
        if (more) gload(k + 32);
        const uint8_t *L = lds[buf];
        u32x4 bfr[FN];
#pragma unroll
        for (int j = 0; j < FN; j++) bfr[j] = *(const u32x4 *)(L + (2 * BM + wn + j * 16 + fr) * RS + fc);
#pragma unroll
        for (int i = 0; i < FM; i++) {
            const u32x4 ah = *(const u32x4 *)(L + (wm + i * 16 + fr) * RS + fc);
            const u32x4 al = *(const u32x4 *)(L + (BM + wm + i * 16 + fr) * RS + fc);
#pragma unroll
            for (int j = 0; j < FN; j++) {
                acc[i][j] = mfma16<DT>(ah, bfr[j], acc[i][j]);
                acc[i][j] = mfma16<DT>(al, bfr[j], acc[i][j]);
            }
        }
        if (more) lstore(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }
    tile_out<FM, FN>(g, partial, acc, m0 + wm, n0 + wn, lane);
}

// Burst form of k_gemm_tiled for K ranges that are a multiple of 32*NB: each burst issues
// the global loads of NB consecutive K steps at once and then feeds them through the two LDS
// buffers a step at a time, so a workgroup waits out one load latency per burst rather than
// one per step (short K ranges of small-M products are latency-bound, not MFMA-bound). The
// LDS tiles, fragments and epilogue are k_gemm_tiled's. One barrier per step suffices: a
// buffer is rewritten two steps after it was read, and every wave has passed the barrier
// between.
// Byte offset of 16-byte chunk c (0..3) of row r in an LDS tile of unpadded 64-byte rows, the
// chunks XOR-swizzled by row: 8 or 16 lanes reading one chunk of 16 consecutive rows, and
// 4 lanes per row writing whole rows, then fall on distinct banks (32- or 64-bank LDS).
__device__ __forceinline__ int swz64(int r, int c) { return r * 64 + ((c ^ (((r >> 1) ^ (r >> 3)) & 3)) << 4); }

template <int DT, int BM, int BN, int NB, int PL = 2>
__global__ __launch_bounds__(kT) void k_gemm_burst(GemmArgs g, float *partial, int kc) {
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 16, FN = WN / 16;
    constexpr int RS = 64;            // unpadded rows, chunks placed by swz64
    constexpr int R = PL * BM + BN;   // A hi (and A lo) rows, then W rows
    constexpr int PER = R * 4 / kT;
    static_assert(kT == 256 && BM % 64 == 0 && NB % 2 == 0, "64 rows per chunk index; bursts of even length");
    __shared__ __attribute__((aligned(16))) uint8_t lds[2][R * RS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * WM, wn = (wave & 1) * WN;
    int tx, ty;
    gemm_tile(tx, ty);
    const int m0 = tx * BM, n0 = ty * BN;
    const int kbeg = blockIdx.z * kc, kend = kbeg + kc;
    const size_t lo = (size_t)g.M * g.K;
    const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
    u32x4 stage[NB][PER];
    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int fr = lane & 15, fq = lane >> 4;
    for (int kb = kbeg; kb < kend; kb += NB * 32) {
        // chunk j of a thread is row 64*j + tid/4 of the tile (A hi, A lo or W by j alone, as
        // BM is a multiple of 64), 16 bytes at k + 8*(tid%4); rows past M load row M-1 and
        // are zeroed, so no load sits under a branch and the waits count loads in order
#pragma unroll
        for (int st = 0; st < NB; st++) {
            const int k = kb + st * 32 + (tid & 3) * 8;
#pragma unroll
            for (int j = 0; j < PER; j++) {
                const int rr = j * 64 + (tid >> 2);
                if (j * 64 < PL * BM) {
                    const int m = m0 + (j * 64 < BM ? rr : rr - BM);
                    const uint16_t *src = g.A + (j * 64 < BM ? 0 : lo) + (size_t)min(m, g.M - 1) * g.K + k;
                    const u32x4 v = *(const u32x4 *)src;
                    stage[st][j] = m < g.M ? v : zero;
                } else {
                    stage[st][j] = *(const u32x4 *)(g.B + (size_t)(n0 + rr - PL * BM) * g.K + k);
                }
            }
        }
#pragma unroll
        for (int st = 0; st < NB; st++) {
            uint8_t *L = lds[st & 1];
#pragma unroll
            for (int j = 0; j < PER; j++) {
                const int ci = tid + j * kT;
                *(u32x4 *)(&L[swz64(ci >> 2, ci & 3)]) = stage[st][j];
            }
            __syncthreads();
            u32x4 bfr[FN];
#pragma unroll
            for (int j = 0; j < FN; j++) bfr[j] = *(const u32x4 *)(L + swz64(PL * BM + wn + j * 16 + fr, fq));
#pragma unroll
            for (int i = 0; i < FM; i++) {
                const u32x4 ah = *(const u32x4 *)(L + swz64(wm + i * 16 + fr, fq));
                u32x4 al = ah;
                if constexpr (PL == 2) al = *(const u32x4 *)(L + swz64(BM + wm + i * 16 + fr, fq));
#pragma unroll
                for (int j = 0; j < FN; j++) {
                    acc[i][j] = mfma16<DT>(ah, bfr[j], acc[i][j]);
                    if constexpr (PL == 2) acc[i][j] = mfma16<DT>(al, bfr[j], acc[i][j]);
                }
            }
        }
    }
    tile_out<FM, FN>(g, partial, acc, m0 + wm, n0 + wn, lane);
}

// s_waitcnt immediate that waits until at most n vector memory operations of the wave are
// outstanding (gfx9 encoding: vmcnt bits 3:0 and 15:14; expcnt and lgkmcnt left at their
// maxima, i.e. not waited for).
constexpr int vm_wait_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Pipelined MFMA GEMM for short inputs: the same product and epilogue as k_gemm_burst, with
// the operand tiles streamed into an NS-deep LDS ring by global_load_lds (each lane moves 16
// bytes straight into LDS, one wave instruction fills 1 KB; no staging registers and no LDS
// stores), so NS - 1 K steps of BK are always in flight and a workgroup waits out one memory
// latency per product rather than one per burst. One barrier per K step:
//   wait for this wave's loads of step s; barrier (every wave's loads of step s have landed
//   and every wave has finished step s - 1); issue step s + NS - 1 into the slot step s - 1
//   used; MFMAs of step s.
// The waits are explicit s_waitcnt vmcnt(n) with a plain s_barrier: __syncthreads' release
// fence would wait for every outstanding load, collapsing the ring to one step.
// Tile rows (A hi, A lo, W; BK 16-bit elements each) are stored unpadded with their 16-byte
// chunks XOR-swizzled by row (chunk c of row r in slot c ^ swz(r)), which is how each lane
// picks its global chunk; a wave's fragment reads (16 rows x one chunk) then spread over the
// LDS banks. Workgroup tile BM x BN of 2 x 2 waves, each FM x FN 16 x 16 blocks; the hi and
// lo products accumulate separately (independent MFMA chains) and are added at the end.
// Needs N % BN == 0, kc % BK == 0 and kc / BK >= NS - 1; rows past M re-read row M - 1.
template <int DT, int BM, int BN, int BK, int NS, int PL = 2>
__device__ __forceinline__ void pipe_product(const GemmArgs &g, int kc, uint8_t *lds,
                                             f32x4 (&acc)[BM / 32][BN / 32], int m0, int n0) {
    constexpr int FM = BM / 32, FN = BN / 32;
    constexpr int CPR = BK / 8;                 // 16-byte chunks per tile row
    constexpr int RB = BK * 2;                  // bytes per tile row
    constexpr int RPI = 1024 / RB;              // tile rows per wave instruction
    constexpr int ROWS = PL * BM + BN;          // A hi (and A lo) rows, then W rows
    constexpr int IPW = ROWS / RPI / 4;         // wave instructions per step, per wave
    constexpr int SB = ROWS * RB;               // bytes per ring slot
    static_assert(kT == 256 && ROWS % (4 * RPI) == 0 && BM % RPI == 0 && BN % RPI == 0 && CPR >= 4,
                  "each step's rows must split evenly over the four waves");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int kbeg = blockIdx.z * kc;
    const int nsteps = kc / BK;
    const size_t lo = (size_t)g.M * g.K;
    auto swz = [](int r) { return CPR == 4 ? (r >> 1) & 3 : r & 7; };
    const uint16_t *src[IPW];
#pragma unroll
    for (int i = 0; i < IPW; i++) {
        const int gi = wave * IPW + i;
        const int r = gi * RPI + lane / CPR;
        const int c = (lane % CPR) ^ swz(r);
        const uint16_t *p;
        if (r < BM) p = g.A + (size_t)min(m0 + r, g.M - 1) * g.K;
        else if (r < PL * BM) p = g.A + lo + (size_t)min(m0 + r - BM, g.M - 1) * g.K;
        else p = g.B + (size_t)(n0 + r - PL * BM) * g.K;
        src[i] = p + kbeg + c * 8;
    }
    auto issue = [&](int st) {
        uint8_t *base = lds + (st % NS) * SB + wave * IPW * 1024;
#pragma unroll
        for (int i = 0; i < IPW; i++)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(src[i] + st * BK),
                                             (__attribute__((address_space(3))) void *)(base + i * 1024), 16, 0, 0);
    };
    const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * (BN / 2);
    const int fr = lane & 15, fq = lane >> 4;
    f32x4 acl[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) {
            acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
            acl[i][j] = acc[i][j];
        }
    auto compute = [&](int st) {
        const uint8_t *L = lds + (st % NS) * SB;
#pragma unroll
        for (int ks = 0; ks < BK / 32; ks++) {
            const int c = ks * 4 + fq;
            u32x4 ah[FM], al[FM], b[FN];
#pragma unroll
            for (int i = 0; i < FM; i++) {
                const int r = wm + i * 16 + fr, r2 = BM + r;
                ah[i] = *(const u32x4 *)(L + r * RB + ((c ^ swz(r)) << 4));
                if constexpr (PL == 2) al[i] = *(const u32x4 *)(L + r2 * RB + ((c ^ swz(r2)) << 4));
            }
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int r = PL * BM + wn + j * 16 + fr;
                b[j] = *(const u32x4 *)(L + r * RB + ((c ^ swz(r)) << 4));
            }
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++) acc[i][j] = mfma16<DT>(ah[i], b[j], acc[i][j]);
            if constexpr (PL == 2) {
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++) acl[i][j] = mfma16<DT>(al[i], b[j], acl[i][j]);
            }
        }
    };
#pragma unroll
    for (int st = 0; st < NS - 1; st++) issue(st);
    int s = 0;
    for (; s < nsteps - (NS - 1); s++) {
        __builtin_amdgcn_s_waitcnt(vm_wait_imm((NS - 2) * IPW));
        __builtin_amdgcn_s_barrier();
        issue(s + NS - 1);
        compute(s);
    }
    __builtin_amdgcn_s_waitcnt(vm_wait_imm(0));
    __builtin_amdgcn_s_barrier();
    for (; s < nsteps; s++) compute(s);
    if constexpr (PL == 2) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) acc[i][j] += acl[i][j];
    }
}

template <int DT, int BM, int BN, int BK, int NS, int PL = 2>
__global__ __launch_bounds__(kT) void k_gemm_pipe(GemmArgs g, float *partial, int kc) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    f32x4 acc[BM / 32][BN / 32];
    int tx, ty;
    gemm_tile<4>(tx, ty);
    pipe_product<DT, BM, BN, BK, NS, PL>(g, kc, lds, acc, tx * BM, ty * BN);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    tile_out<BM / 32, BN / 32>(g, partial, acc, tx * BM + (wave >> 1) * (BM / 2),
                               ty * BN + (wave & 1) * (BN / 2), lane);
}

// The pipelined GEMM's shapes: 64 x 64 tiles with 6 slots of K 64 (147,456 bytes of LDS, one
// workgroup per CU) where the tiles alone fill the chip, else 32 x 32 tiles with 4 slots
// (49,152 bytes) and up to four K ranges.
constexpr int kPipeBigLds = 6 * (3 * 64) * 128;
constexpr int kPipeSmallLds = 4 * (3 * 32) * 128;
constexpr int kPipeWideLds = 4 * (2 * 32 + 64) * 128;   // 32 x 64 tiles (65,536 bytes)

// ---- W8A8 products on the int8 matrix cores --------------------------------------------

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// The bridge quantizer for one value (ane_bridge.m:386-396): x / scale with IEEE division,
// clamp to [-128, 127], round half away from zero by +-0.5 and truncation.
__device__ __forceinline__ int8_t quant_i8(float x, float scale) {
    float v = __fdiv_rn(x, scale);
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    return (int8_t)(int)(v >= 0.0f ? v + 0.5f : v - 0.5f);
}

// Per-token activation quantization: the bridge formula (ane_bridge.m:374-399) applied to
// each row on its own, as the W8A8 decode quantizes its one token. Row m of the fp32 A
// operand [M, K] -> int8 row m of a8 and sa[m] = max|x| / 127 (0 -> 1), q = quantize(x / sa[m]).
__global__ __launch_bounds__(kT) void k_quant_rows_i8(const float *x, int K, int8_t *a8,
                                                       float *sa) {
    __shared__ float red[kT / 64];
    const int m = blockIdx.x;
    const float *row = x + (size_t)m * K;
    float mx = 0.f;
    for (int i = threadIdx.x; i < K; i += kT) mx = fmaxf(mx, fabsf(row[i]));
    mx = wmax<64>(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kT / 64; w++) mx = fmaxf(mx, red[w]);
    float scale = __fdiv_rn(mx, 127.0f);
    if (scale == 0.0f) scale = 1.0f;
    for (int i = threadIdx.x; i < K; i += kT) a8[(size_t)m * K + i] = quant_i8(row[i], scale);
    if (threadIdx.x == 0) sa[m] = scale;
}

// W8A8 causal attention in the decode's float order (infer.go:273-299 attend with the
// softmaxPrefix of infer.go:328-345), so the attention output the Wo quantizer sees is the
// W8A8 decode's: per (row t, head h) workgroup, score j = (sum over i in order of
// q[i] * k[j][i]) * (1 / sqrt(hd)) for the keys j <= rowpos[t] of the row's sequence, their
// float maximum, e_j = float(exp(double(s_j - max))), the float64 sum of the e_j in key order,
// p_j = e_j * float(1 / sum), and att[i] = sum over j in key order of p_j * v[j][i]. Keys are
// the rows t - rowpos[t] .. t of the token-major k / v arrays (values already rounded to the
// cache type) or, with from_cache, rows 0 .. rowpos[t] of the sequence's KV cache slab
// (rowseq[t] * seq_stride elements in). att is the fp32 operand [rows, qdim].
template <int KVT>
__global__ __launch_bounds__(kT) void k_attn_exact(const float *q, int qdim, const void *kb,
                                                   const void *vb, size_t seq_stride, int kvdim,
                                                   int from_cache, const int32_t *rowpos,
                                                   const int32_t *rowseq, int n_heads,
                                                   int n_kv_heads, int hd, float inv_sqrt_hd,
                                                   float *att) {
    __shared__ float sc[kMaxSeqLds];
    __shared__ float qs[256];
    __shared__ float red[kT / 64];
    __shared__ float inv_s;
    const int t = blockIdx.x, h = blockIdx.y;
    const int pos = rowpos[t], L = pos + 1;
    const int g = h / (n_heads / n_kv_heads);
    const size_t r0 = (from_cache ? (size_t)rowseq[t] * seq_stride : (size_t)(t - pos) * kvdim) + (size_t)g * hd;
    auto kv = [&](const void *base, int j, int i) -> float {
        const size_t o = r0 + (size_t)j * kvdim + i;
        if constexpr (KVT == SH_KV_F32) return ((const float *)base)[o];
        else return bits_to_f(((const uint16_t *)base)[o], KVT == SH_KV_BF16 ? SH_DTYPE_BF16 : SH_DTYPE_F16);
    };
    for (int i = threadIdx.x; i < hd; i += kT) qs[i] = q[(size_t)t * qdim + (size_t)h * hd + i];
    __syncthreads();
    float mx = -INFINITY;
    for (int j = threadIdx.x; j < L; j += kT) {
        float dot = 0.f;
        for (int i = 0; i < hd; i++) dot += qs[i] * kv(kb, j, i);
        const float sj = dot * inv_sqrt_hd;
        sc[j] = sj;
        mx = fmaxf(mx, sj);
    }
    mx = wmax<64>(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kT / 64; w++) mx = fmaxf(mx, red[w]);
    for (int j = threadIdx.x; j < L; j += kT) sc[j] = (float)exp((double)(sc[j] - mx));
    __syncthreads();
    if (threadIdx.x == 0) {
        double sum = 0;
        for (int j = 0; j < L; j++) sum += (double)sc[j];
        inv_s = (float)(1.0 / sum);
    }
    __syncthreads();
    const float inv = inv_s;
    for (int j = threadIdx.x; j < L; j += kT) sc[j] *= inv;
    __syncthreads();
    for (int i = threadIdx.x; i < hd; i += kT) {
        float a = 0.f;
        for (int j = 0; j < L; j++) a += sc[j] * kv(vb, j, i);
        att[(size_t)t * qdim + (size_t)h * hd + i] = a;
    }
}

// W8A8 projection: C[m, n] = (float)(sum over k of a8[m, k] * W[n, k]) * (sw[n] * sa[m]),
// the int32 sum exact (or_mat_vec_w8a8's dequantization: the int32 dot product, then the
// row scale times the activation scale). v_mfma_i32_16x16x64_i8 over 64 x 64 workgroup tiles
// of 2 x 2 waves; K in steps of 64 (one 64-byte LDS row per tile row, padded to 80 bytes),
// NB steps' loads issued per burst as in k_gemm_burst. A and W fragments are read with the
// same lane pattern (row lane % 16, 16 bytes at k + 16 * (lane / 16)), so each MFMA sums
// the same 64 products whatever the instruction's k order. No K split: one workgroup
// finishes its tile and applies the epilogue (the same forms as the 16-bit GEMM).
template <int BM, int BN, int NB>
__global__ __launch_bounds__(kT) void k_gemm_i8(GemmArgs g) {
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 16, FN = WN / 16;
    constexpr int RS = 80;
    constexpr int R = BM + BN;                   // tile rows: A, then W
    constexpr int PER = R * 4 / kT;              // 16-byte chunks per thread per step
    static_assert(kT == 256 && BM % 64 == 0 && BN % 64 == 0 && NB % 2 == 0,
                  "64 rows per chunk index; bursts of even length");
    __shared__ __attribute__((aligned(16))) uint8_t lds[2][R * RS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * WM, wn = (wave & 1) * WN;
    const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
    const int8_t *A = g.a8, *W = (const int8_t *)g.B;
    const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
    u32x4 stage[NB][PER];
    i32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = i32x4{0, 0, 0, 0};
    const int fr = lane & 15, fc = (lane >> 4) * 16;
    for (int kb = 0; kb < g.K; kb += NB * 64) {
        // chunk j of a thread: row 64*j + tid/4 of the tile (A rows, then W rows), 16 bytes
        // at k + 16*(tid%4); A rows past M load row M-1 and are zeroed (no load under a branch)
#pragma unroll
        for (int st = 0; st < NB; st++) {
            const int k = kb + st * 64 + (tid & 3) * 16;
#pragma unroll
            for (int j = 0; j < PER; j++) {
                const int rr = j * 64 + (tid >> 2);
                if (j * 64 < BM) {
                    const int m = m0 + rr;
                    const u32x4 v = *(const u32x4 *)(A + (size_t)min(m, g.M - 1) * g.K + k);
                    stage[st][j] = m < g.M ? v : zero;
                } else {
                    stage[st][j] = *(const u32x4 *)(W + (size_t)(n0 + rr - BM) * g.K + k);
                }
            }
        }
#pragma unroll
        for (int st = 0; st < NB; st++) {
            uint8_t *L = lds[st & 1];
#pragma unroll
            for (int j = 0; j < PER; j++) {
                const int ci = tid + j * kT;
                *(u32x4 *)(&L[(ci >> 2) * RS + (ci & 3) * 16]) = stage[st][j];
            }
            __syncthreads();
            i32x4 bfr[FN];
#pragma unroll
            for (int j = 0; j < FN; j++)
                bfr[j] = __builtin_bit_cast(i32x4, *(const u32x4 *)(L + (BM + wn + j * 16 + fr) * RS + fc));
#pragma unroll
            for (int i = 0; i < FM; i++) {
                const i32x4 a = __builtin_bit_cast(i32x4, *(const u32x4 *)(L + (wm + i * 16 + fr) * RS + fc));
#pragma unroll
                for (int j = 0; j < FN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bfr[j], acc[i][j], 0, 0, 0);
            }
        }
    }
    // D layout as the 16-bit GEMM's: lane holds column lane % 16, rows 4 * (lane / 16) + r
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int n = n0 + wn + j * 16 + (lane & 15);
            const float sw = g.sw[n];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm + i * 16 + (lane >> 4) * 4 + r;
                const float v = (float)acc[i][j][r] * (sw * g.sa[min(m, g.M - 1)]);
                const float vr = __shfl_xor(v, 1, 64);   // column n ^ 1, same row
                if (m < g.M) tile_epilogue<true>(g, m, n, v, vr);
            }
        }
}

template <int KVT>
__device__ __forceinline__ float kv_round(float v) {
    if constexpr (KVT == SH_KV_F32) return v;
    else if constexpr (KVT == SH_KV_F16) return bits_to_f(f_to_bits(v, SH_DTYPE_F16), SH_DTYPE_F16);
    else return bits_to_f(f_to_bits(v, SH_DTYPE_BF16), SH_DTYPE_BF16);
}
template <int KVT>
__device__ __forceinline__ void kv_store(void *base, size_t o, float v) {
    if constexpr (KVT == SH_KV_F32) ((float *)base)[o] = v;
    else ((uint16_t *)base)[o] = f_to_bits(v, KVT == SH_KV_BF16 ? SH_DTYPE_BF16 : SH_DTYPE_F16);
}

// Row t of the token-major activations is token rowpos[t] of sequence rowseq[t].
// Per row: optional per-head RMSNorm of q and k, RoPE at the row's position (rope.go:26-46:
// e' = e*c - o*s, o' = o*c + e*s); q written fp32 token-major, k and v too when ko/vo are
// given. With write_cache the roped k and v also enter the cache at (rowseq[t], layer,
// rowpos[t]) — kcache/vcache point at sequence 0's slab of this layer, kv_seq_stride
// elements apart per sequence — and ko/vo then carry the values as the cache stores them,
// so attention sees what a token-by-token decode would see (infer.go:267-271 stores k and v
// before attending).
struct QkRopeArgs {
    int qdim, kvdim, hd, qk_norm;
    const float *q_norm, *k_norm;
    double qk_eps;
    const float *rope_cos, *rope_sin;
    const int32_t *rowpos, *rowseq;
    float *qo, *ko, *vo;
    void *kcache, *vcache;
    size_t kv_seq_stride;
    int write_cache;
    int round_kv;        // ko / vo rounded to the cache type even without a cache write
    int kv16;            // k_gemm_pipe_qkv64: ko / vo as fp16 values (uint16_t), for the
                         // one-plane fp16 attention that reads them as they are
};

// Finishes row t held in LDS (q | k | v, qdim + 2*kvdim floats).
template <int KVT>
__device__ __forceinline__ void qk_rope_row(float *row, int t, const QkRopeArgs &a) {
    const int tp = a.rowpos[t];
    const size_t kv_row = (size_t)a.rowseq[t] * a.kv_seq_stride + (size_t)tp * a.kvdim;
    const int qdim = a.qdim, kvdim = a.kvdim, hd = a.hd, n = qdim + 2 * kvdim;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int heads = (qdim + kvdim) / hd;   // q heads, then k heads
    if (a.qk_norm) {
        for (int h = wave; h < heads; h += nw) {
            float *v = row + h * hd;
            const float *g = h < qdim / hd ? a.q_norm : a.k_norm;
            double ss = 0;
            for (int i = lane; i < hd; i += 64) ss += (double)v[i] * (double)v[i];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
            const float rr = (float)(1.0 / sqrt(ss / (double)hd + a.qk_eps));
            for (int i = lane; i < hd; i += 64) v[i] = v[i] * rr * g[i];
        }
        __syncthreads();
    }
    const int half = hd / 2;
    for (int p = threadIdx.x; p < (qdim + kvdim) / 2; p += blockDim.x) {
        const int pi = p % half;
        const float c = a.rope_cos[tp * half + pi], s = a.rope_sin[tp * half + pi];
        const float e = row[2 * p], o = row[2 * p + 1];
        row[2 * p] = e * c - o * s;
        row[2 * p + 1] = o * c + e * s;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = row[i];
        if (i < qdim) {
            a.qo[(size_t)t * qdim + i] = v;
        } else if (i < qdim + kvdim) {
            const int j = i - qdim;
            if (a.write_cache) kv_store<KVT>(a.kcache, kv_row + j, v);
            if (a.ko) a.ko[(size_t)t * kvdim + j] = a.write_cache || a.round_kv ? kv_round<KVT>(v) : v;
        } else {
            const int j = i - qdim - kvdim;
            if (a.write_cache) kv_store<KVT>(a.vcache, kv_row + j, v);
            if (a.vo) a.vo[(size_t)t * kvdim + j] = a.write_cache || a.round_kv ? kv_round<KVT>(v) : v;
        }
    }
}

template <int KVT>
__global__ __launch_bounds__(kT) void k_qk_rope(const float *qkv, QkRopeArgs a) {
    __shared__ __attribute__((aligned(16))) float row[4096];
    const int t = blockIdx.x;
    const int n = a.qdim + 2 * a.kvdim;
#pragma unroll 4
    for (int i4 = threadIdx.x; i4 < n / 4; i4 += blockDim.x)   // n % 4 == 0
        *(f32x4 *)(row + 4 * i4) = *(const f32x4 *)(qkv + (size_t)t * n + 4 * i4);
    __syncthreads();
    qk_rope_row<KVT>(row, t, a);
}

// The q|k|v projection of a model with 64-dim heads, its row epilogue fused (qk_rope_row's
// QK-norm, RoPE and KV-cache fill, in the same operations and order): with BM x 64 tiles of
// the pipelined GEMM a tile is BM rows of exactly one q, k or v head. The tile goes through
// LDS (the ring is free once the product is done); wave w then finishes its BM / 4 rows with
// lane = head dim: the QK-norm sum is a butterfly over the wave, the RoPE partner of dim
// 2p / 2p+1 the neighbouring lane. Saves the separate k_qk_rope launch. BM = 32 serves
// inputs of at most 32 rows.
template <int BM, int PL>
constexpr int qkv64_lds() { return 6 * (PL * BM + 64) * 128; }
template <int DT, int KVT, int PL = 2, int BM = 64>
__global__ __launch_bounds__(kT) void k_gemm_pipe_qkv64(GemmArgs g, QkRopeArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int RPW = BM / 4;   // rows finished per wave
    static_assert(BM == 32 || BM == 64, "32- or 64-row tiles");
    f32x4 acc[BM / 32][2];
    int tx, ty;
    gemm_tile<4>(tx, ty);
    pipe_product<DT, BM, 64, 64, 6, PL>(g, g.K, lds, acc, tx * BM, ty * 64);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * 32;
    __syncthreads();   // every wave is done reading the ring
    float *T = (float *)lds;   // [BM][65]
#pragma unroll
    for (int i = 0; i < BM / 32; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                T[(wm + i * 16 + (lane >> 4) * 4 + r) * 65 + wn + j * 16 + (lane & 15)] = acc[i][j][r];
    __syncthreads();
    const int m0 = tx * BM, n0 = ty * 64;
    const int region = n0 < a.qdim ? 0 : n0 < a.qdim + a.kvdim ? 1 : 2;   // q, k or v head
    const float gn = a.qk_norm && region < 2 ? (region == 0 ? a.q_norm : a.k_norm)[lane] : 1.f;
    void *cache = region == 1 ? a.kcache : a.vcache;
    float *kvo = region == 1 ? a.ko : a.vo;
    const int j = n0 - a.qdim - (region == 2 ? a.kvdim : 0) + lane;
    // positions and sequences of the wave's RPW rows (lane r holds row r's), then every row's
    // RoPE factors, all requested before the first is used
    const int r0 = m0 + wave * RPW, nrows = min(RPW, g.M - r0);
    int tpl = 0, sql = 0;
    if (lane < nrows) {
        tpl = a.rowpos[r0 + lane];
        sql = a.rowseq[r0 + lane];
    }
    float cs[RPW], sn[RPW];
    if (region < 2) {
#pragma unroll
        for (int rr = 0; rr < RPW; rr++) {
            const int tp = __shfl(tpl, rr, 64);
            cs[rr] = a.rope_cos[tp * 32 + (lane >> 1)];
            sn[rr] = a.rope_sin[tp * 32 + (lane >> 1)];
        }
    }
#pragma unroll
    for (int rr = 0; rr < RPW; rr++) {
        const int t = r0 + rr;
        const int tp = __shfl(tpl, rr, 64), sq = __shfl(sql, rr, 64);
        if (rr >= nrows) break;   // uniform over the wave
        float v = T[(wave * RPW + rr) * 65 + lane];
        if (region < 2) {
            if (a.qk_norm) {
                double ss = (double)v * (double)v;
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
                const float rn = (float)(1.0 / sqrt(ss / 64.0 + a.qk_eps));
                v = v * rn * gn;
            }
            const float o = __shfl_xor(v, 1, 64);   // the other element of the pair
            v = (lane & 1) ? v * cs[rr] + o * sn[rr] : v * cs[rr] - o * sn[rr];
        }
        if (region == 0) {
            a.qo[(size_t)t * a.qdim + n0 + lane] = v;
        } else {
            if (a.write_cache) kv_store<KVT>(cache, (size_t)sq * a.kv_seq_stride + (size_t)tp * a.kvdim + j, v);
            if (kvo) {
                const float kv = a.write_cache || a.round_kv ? kv_round<KVT>(v) : v;
                if (a.kv16) ((uint16_t *)kvo)[(size_t)t * a.kvdim + j] = f_to_bits(kv, SH_DTYPE_F16);
                else kvo[(size_t)t * a.kvdim + j] = kv;
            }
        }
    }
}

// Batched decode: row m of the q|k|v projection is the sum of the skinny GEMM's K-range
// partials ([ranges][M][n], added in range order), then qk_rope_row.
template <int KVT>
__global__ __launch_bounds__(1024) void k_row_qkv(const float *partial, int ranges, int M, QkRopeArgs a) {
    __shared__ __attribute__((aligned(16))) float row[4096];
    const int m = blockIdx.x;
    const int n = a.qdim + 2 * a.kvdim;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float v = 0.f;
        for (int r = 0; r < ranges; r++) v += partial[((size_t)r * M + m) * n + i];
        row[i] = v;
    }
    __syncthreads();
    qk_rope_row<KVT>(row, m, a);
}

// Row m of a residual projection, x_out = resid + alpha * (sum of the K-range partials, in
// range order), then x_out normalised with `gain` as a GEMM operand row: final_form 0 is
// rmsNormVec / rmsNormCFWithRRMSImpl (infer.go:301-311, accel_other.go:11-28: float32 scale,
// x*scale*w), 1 is stories.RMSNorm (cpu.go:97-111: the float64 product rounded once).
__global__ __launch_bounds__(1024) void k_row_resid_norm(const float *partial, int ranges, int M,
                                                         int D, const float *resid, float alpha,
                                                         float *x_out, const float *gain,
                                                         double eps, int final_form, int dt,
                                                         uint16_t *xn) {
    __shared__ float row[4096];
    __shared__ double red[1024 / 64];
    const int m = blockIdx.x;
    double ss = 0;
    for (int i = threadIdx.x; i < D; i += blockDim.x) {
        float v = 0.f;
        for (int r = 0; r < ranges; r++) v += partial[((size_t)r * M + m) * D + i];
        const float x = resid[(size_t)m * D + i] + alpha * v;
        x_out[(size_t)m * D + i] = x;
        row[i] = x;
        ss += (double)x * (double)x;
    }
    const double tot = block_sum(ss, red);
    const double rr = 1.0 / sqrt(tot / (double)D + eps);
    const float scale = (float)rr;
    for (int i = threadIdx.x; i < D; i += blockDim.x)
        store_op(xn, (size_t)m * D + i, (size_t)M * D,
                 final_form ? (float)((double)row[i] * rr * (double)gain[i]) : row[i] * scale * gain[i], dt);
}

// k_row_resid_norm for rows of at most 1024 elements: one 256-thread workgroup per row, each
// thread owning one 16-byte chunk. The same operations (the K ranges added in range order,
// x = resid + alpha * sum, the float64 sum of squares, the same normalised forms), but a
// thread issues the loads of up to eight ranges together before it adds them, and the sum
// of squares crosses the workgroup through one barrier (the block form's 1024 threads load
// one range per round trip and reduce through LDS twice).
__global__ __launch_bounds__(256) void k_row_resid_norm_v(const float *partial, int ranges, int M, int D,
                                                          const float *resid, float alpha, float *x_out,
                                                          const float *gain, double eps, int final_form, int dt,
                                                          uint16_t *xn) {
    __shared__ double red[4];
    const int m = blockIdx.x, i = threadIdx.x * 4;
    const bool own = i < D;
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    double ss = 0;
    if (own) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int r0 = 0; r0 < ranges; r0 += 8) {
            float4 q[8];
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (r0 + j < ranges) q[j] = *(const float4 *)(partial + ((size_t)(r0 + j) * M + m) * D + i);
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (r0 + j < ranges) {
                    v.x += q[j].x; v.y += q[j].y; v.z += q[j].z; v.w += q[j].w;
                }
        }
        const float4 rs = *(const float4 *)(resid + (size_t)m * D + i);
        x = make_float4(rs.x + alpha * v.x, rs.y + alpha * v.y, rs.z + alpha * v.z, rs.w + alpha * v.w);
        *(float4 *)(x_out + (size_t)m * D + i) = x;
        ss = (double)x.x * (double)x.x;
        ss += (double)x.y * (double)x.y;
        ss += (double)x.z * (double)x.z;
        ss += (double)x.w * (double)x.w;
    }
    ss = wsum_d64(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const double tot = red[0] + red[1] + red[2] + red[3];
    if (!own) return;
    const double rr = 1.0 / sqrt(tot / (double)D + eps);
    const float scale = (float)rr;
    const float4 g4 = *(const float4 *)(gain + i);
    const float x4[4] = {x.x, x.y, x.z, x.w}, gg[4] = {g4.x, g4.y, g4.z, g4.w};
    const size_t plane = (size_t)M * D;
#pragma unroll
    for (int e = 0; e < 4; e++)
        store_op(xn, (size_t)m * D + i + e, plane,
                 final_form ? (float)((double)x4[e] * rr * (double)gg[e]) : x4[e] * scale * gg[e], dt);
}

// The residual + RMSNorm row kernel for M rows of D: the chunk-per-thread form where a row
// fits one 256-thread workgroup.
hipError_t launch_row_resid_norm(const float *partial, int ranges, int M, int D, const float *resid, float alpha,
                                 float *x_out, const float *gain, double eps, int final_form, int dt,
                                 uint16_t *xn, hipStream_t s) {
    if (D % 4 == 0 && D <= 1024)
        hipLaunchKernelGGL(k_row_resid_norm_v, dim3(M), dim3(256), 0, s, partial, ranges, M, D, resid, alpha, x_out,
                           gain, eps, final_form, dt, xn);
    else
        hipLaunchKernelGGL(k_row_resid_norm, dim3(M), dim3(1024), 0, s, partial, ranges, M, D, resid, alpha, x_out,
                           gain, eps, final_form, dt, xn);
    return hipGetLastError();
}

// Two 16-bit operand values packed as the MFMA expects (element 2i in the low half).
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return (uint32_t)f_to_bits(a, DT) | ((uint32_t)f_to_bits(b, DT) << 16);
}
// hi = round(v), lo = round(v - hi) for 8 consecutive values, as two MFMA operands.
template <int DT>
__device__ __forceinline__ void split8(const float *f, u32x4 &hi, u32x4 &lo) {
    float r[8];
#pragma unroll
    for (int e = 0; e < 8; e++) r[e] = f[e] - bits_to_f(f_to_bits(f[e], DT), DT);
    hi = u32x4{pack2<DT>(f[0], f[1]), pack2<DT>(f[2], f[3]), pack2<DT>(f[4], f[5]), pack2<DT>(f[6], f[7])};
    lo = u32x4{pack2<DT>(r[0], r[1]), pack2<DT>(r[2], r[3]), pack2<DT>(r[4], r[5]), pack2<DT>(r[6], r[7])};
}
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
// pack2 by the hardware conversion of a pair (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32: round to
// nearest even, the same bits as f_to_bits for every value but NaN payloads): one instruction
// per pair where the bf16 bit arithmetic takes about six per value.
template <int DT>
__device__ __forceinline__ uint32_t pack2_hw(float a, float b) {
    const f32x2 v = {a, b};
    if constexpr (DT == SH_DTYPE_BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
    else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}
// split8 with pack2_hw; the residual is taken against the rounded pair's values.
template <int DT>
__device__ __forceinline__ void split8_hw(const float *f, u32x4 &hi, u32x4 &lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        h[i] = pack2_hw<DT>(f[2 * i], f[2 * i + 1]);
        l[i] = pack2_hw<DT>(f[2 * i] - bits_to_f((uint16_t)h[i], DT), f[2 * i + 1] - bits_to_f((uint16_t)(h[i] >> 16), DT));
    }
    hi = u32x4{h[0], h[1], h[2], h[3]};
    lo = u32x4{l[0], l[1], l[2], l[3]};
}
// Two values that are exact in the 16-bit type DT (K and V rounded to the cache type by the
// cache fill), packed without rounding: bf16 keeps each float's high half (one byte permute
// per pair), fp16 converts exactly.
template <int DT>
__device__ __forceinline__ uint32_t pack2_exact(float a, float b) {
    if constexpr (DT == SH_DTYPE_BF16) return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
    else return pack2_hw<DT>(a, b);
}

// max / sum over the four lanes l, l^16, l^32, l^48 (the four row groups of a wave)
__device__ __forceinline__ float max_rows(float v) {
    SwapPair s = swap16(__float_as_uint(v));
    v = fmaxf(__uint_as_float(s.a), __uint_as_float(s.b));
    s = swap32(__float_as_uint(v));
    return fmaxf(__uint_as_float(s.a), __uint_as_float(s.b));
}
__device__ __forceinline__ float sum_rows(float v) {
    SwapPair s = swap16(__float_as_uint(v));
    v = __uint_as_float(s.a) + __uint_as_float(s.b);
    s = swap32(__float_as_uint(v));
    return __uint_as_float(s.a) + __uint_as_float(s.b);
}

// Causal attention of the full-sequence forward on MFMA (forward_common.go:5-33, flash
// style). Workgroup = 16 query rows x one head; row t is position rowpos[t] of its sequence,
// whose keys are j in [t - rowpos[t], t]. The key blocks (BK keys) that some row of the tile
// can see are dealt round-robin to the four waves, each with its own LDS slice, so a short
// tile's blocks run side by side rather than one after another; the waves' softmax states
// (running max, sum, unnormalised O) are merged through LDS at the end. S/16 x H workgroups
// keep the CUs busy at S = 256, where S/64 x H did not.
//
// Per key block a wave stages K ([key][dim]) and V transposed ([dim][key]) in its LDS slice as
// 16-bit operand planes, then computes S^T = K . Q^T with v_mfma_f32_16x16x32 (A = K rows,
// B = the 16 queries), so a lane holds one query (lane % 16) and 16 of the block's keys: key
// 16j + 4(lane/16) + r of tile j, register r. An online softmax per query (running max
// uniform over the query's four lanes, per-lane partial sums) gives P, which is already in
// the B-operand layout of O^T = V^T . P^T (lane = query, k slots = the lane's 8 keys of a
// 32-key step), and V^T rows are read in the same key order. O^T accumulates per lane as
// query lane % 16, dims 16i + 4(lane/16) + r, so the softmax rescale is per lane. Scores are
// kept in the base-2 domain (scaled by log2 e), so each softmax term is one exp2, and the
// 16-bit operands are rounded by the hardware pair conversions.
//
// Operands are hi/lo pairs of the model's 16-bit type: Q and P always; K and V too (LO) when
// they are fp32 rather than values already rounded to this type by the KV cache. The products
// hi.hi + lo.hi + hi.lo keep about 16 (bf16) or 22 (fp16) significant bits, fp32 accumulate.
template <int HD> constexpr int attn_bk() { return HD >= 128 ? 32 : 64; }
template <int HD> constexpr size_t attn_lds_bytes() {
    // per wave: K rows (HD*2 + 16 bytes) and V^T rows (BK*2 + 8 bytes), hi and lo planes
    return (size_t)4 * 2 * (attn_bk<HD>() * (HD * 2 + 16) + HD * (attn_bk<HD>() * 2 + 8));
}
template <int DT, int HD, bool LO, int QP = 2, bool KV16 = false>
__global__ __launch_bounds__(kT) void k_attn_prefill_mfma(const float *qf, const float *kf,
                                                          const float *vf, int S,
                                                          const int32_t *rowpos, int H, int KVH,
                                                          float scale, uint16_t *att, size_t plane) {
    constexpr int BQ = 16, BK = attn_bk<HD>(), NP = LO ? 2 : 1, NW = kT / 64;
    constexpr int KRS = HD * 2 + 16;              // LDS bytes per K row (16-byte pad)
    constexpr int VRS = BK * 2 + 8;               // LDS bytes per V^T row (8-byte pad)
    constexpr int KPT = BK * HD / 8 / 64;         // K staging tasks (key, 8 dims) per lane
    constexpr int VPT = (BK / 4) * (HD / 4) / 64; // V staging tasks (4 keys, 4 dims) per lane
    constexpr int NS = HD / 32, NO = HD / 16;     // QK k-steps, O^T tiles
    constexpr int KSL = BK * KRS, VSL = HD * VRS; // one plane of a wave's K / V^T slice
    constexpr int OLD = HD + 4;                   // merge: floats per (wave, query) O row
    static_assert(KPT * 64 * 8 == BK * HD && VPT * 64 * 16 == BK * HD, "staging splits evenly");
    static_assert((size_t)NW * (BQ * OLD + 2 * BQ) * 4 <= attn_lds_bytes<HD>(), "merge fits");
    __shared__ __attribute__((aligned(16))) uint8_t lds[attn_lds_bytes<HD>()];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g4 = lane >> 4, ql = lane & 15;
    const int q0 = blockIdx.x * BQ, h = blockIdx.y;
    const int qdim = H * HD, kvdim = KVH * HD, kvh = h / (H / KVH);
    const int qlast = min(q0 + BQ, S) - 1;
    // rowpos null: row t is position t of one sequence (the EvalLogits forward)
    const int kb0 = rowpos ? (q0 - rowpos[q0]) & ~(BK - 1) : 0;
    uint8_t *ksl = lds + (size_t)wave * NP * (KSL + VSL);   // this wave's K planes, then V^T
    uint8_t *vsl = ksl + NP * KSL;

    // this lane's query and its Q operand planes (B operand: dims 32s + 8*g4 .. +7)
    const int t = q0 + ql;
    const bool tok = t < S;
    const int jlo = tok ? (rowpos ? t - rowpos[t] : 0) : 0x7fffffff;
    u32x4 qh[NS], qlo[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        float f[8];
        if (tok) {
            const f32x4 a = *(const f32x4 *)(qf + (size_t)t * qdim + h * HD + 32 * s + 8 * g4);
            const f32x4 b = *(const f32x4 *)(qf + (size_t)t * qdim + h * HD + 32 * s + 8 * g4 + 4);
            f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) f[e] = 0.f;
        }
        split8<DT>(f, qh[s], qlo[s]);
    }

    // staging registers for the wave's next key block (KV16: K and V already the model's
    // 16-bit values, as the fused q|k|v epilogue wrote them, copied without conversion)
    f32x4 kst[KV16 ? 1 : KPT][2], vst[KV16 ? 1 : VPT][4];
    u32x4 k16[KV16 ? KPT : 1];
    uint2 v16[KV16 ? VPT : 1][4];
    auto gload16 = [&](int kb) {
        const uint16_t *kh = (const uint16_t *)kf, *vh = (const uint16_t *)vf;
#pragma unroll
        for (int u = 0; u < KPT; u++) {
            const int c = lane + u * 64;
            const int r = c / (HD / 8), d = (c % (HD / 8)) * 8, j = kb + r;
            const u32x4 a = *(const u32x4 *)(kh + (size_t)min(j, S - 1) * kvdim + kvh * HD + d);
            k16[u] = j < S ? a : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < VPT; u++) {
            const int c = lane + u * 64;
            const int kq = c / (HD / 4), d = (c % (HD / 4)) * 4;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int j = kb + 4 * kq + i;
                const uint2 a = *(const uint2 *)(vh + (size_t)min(j, S - 1) * kvdim + kvh * HD + d);
                v16[u][i] = j < S ? a : uint2{0u, 0u};
            }
        }
    };
    auto lstore16 = [&]() {
#pragma unroll
        for (int u = 0; u < KPT; u++) {
            const int c = lane + u * 64;
            const int r = c / (HD / 8), d = (c % (HD / 8)) * 8;
            *(u32x4 *)&ksl[r * KRS + d * 2] = k16[u];
        }
#pragma unroll
        for (int u = 0; u < VPT; u++) {
            const int c = lane + u * 64;
            const int kq = c / (HD / 4), d = (c % (HD / 4)) * 4;
            // dim d + i of keys 4kq .. 4kq+3: half i of each key's four dims
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int sh = 16 * (i & 1);
                uint32_t e[4];
#pragma unroll
                for (int q = 0; q < 4; q++) e[q] = ((i < 2 ? v16[u][q].x : v16[u][q].y) >> sh) & 0xffffu;
                *(uint2 *)&vsl[(d + i) * VRS + 8 * kq] = uint2{e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
            }
        }
    };
    auto gload = [&](int kb) {
#pragma unroll
        for (int u = 0; u < KPT; u++) {
            const int c = lane + u * 64;
            const int r = c / (HD / 8), d = (c % (HD / 8)) * 8, j = kb + r;
            const float *src = kf + (size_t)min(j, S - 1) * kvdim + kvh * HD + d;
            const f32x4 a = *(const f32x4 *)src, b = *(const f32x4 *)(src + 4);
            kst[u][0] = j < S ? a : f32x4{0.f, 0.f, 0.f, 0.f};
            kst[u][1] = j < S ? b : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < VPT; u++) {
            const int c = lane + u * 64;
            const int kq = c / (HD / 4), d = (c % (HD / 4)) * 4;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int j = kb + 4 * kq + i;
                const f32x4 a = *(const f32x4 *)(vf + (size_t)min(j, S - 1) * kvdim + kvh * HD + d);
                vst[u][i] = j < S ? a : f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
    };
    auto lstore = [&]() {
#pragma unroll
        for (int u = 0; u < KPT; u++) {
            const int c = lane + u * 64;
            const int r = c / (HD / 8), d = (c % (HD / 8)) * 8;
            const float f[8] = {kst[u][0].x, kst[u][0].y, kst[u][0].z, kst[u][0].w,
                                kst[u][1].x, kst[u][1].y, kst[u][1].z, kst[u][1].w};
            u32x4 hi, lo;
            split8_hw<DT>(f, hi, lo);
            *(u32x4 *)&ksl[r * KRS + d * 2] = hi;
            if constexpr (LO) *(u32x4 *)&ksl[KSL + r * KRS + d * 2] = lo;
        }
#pragma unroll
        for (int u = 0; u < VPT; u++) {
            const int c = lane + u * 64;
            const int kq = c / (HD / 4), d = (c % (HD / 4)) * 4;
#pragma unroll
            for (int i = 0; i < 4; i++) {   // dim d + i: keys 4kq .. 4kq+3
                const float a0 = vst[u][0][i], a1 = vst[u][1][i], a2 = vst[u][2][i], a3 = vst[u][3][i];
                const uint32_t h01 = pack2_hw<DT>(a0, a1), h23 = pack2_hw<DT>(a2, a3);
                *(uint2 *)&vsl[(d + i) * VRS + 8 * kq] = uint2{h01, h23};
                if constexpr (LO) {
                    const float r0 = a0 - bits_to_f((uint16_t)h01, DT), r1 = a1 - bits_to_f((uint16_t)(h01 >> 16), DT);
                    const float r2 = a2 - bits_to_f((uint16_t)h23, DT), r3 = a3 - bits_to_f((uint16_t)(h23 >> 16), DT);
                    *(uint2 *)&vsl[VSL + (d + i) * VRS + 8 * kq] = uint2{pack2_hw<DT>(r0, r1), pack2_hw<DT>(r2, r3)};
                }
            }
        }
    };

    // scores in the base-2 domain (scale x log2 e), so each softmax term is one exp2
    const float sl2 = scale * 1.4426950408889634f;
    float m_run = -INFINITY, l_part = 0.f;
    f32x4 o[NO];
#pragma unroll
    for (int i = 0; i < NO; i++) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int nb = (qlast - kb0) / BK + 1;   // key blocks some row of the tile can see
    int bi = wave;                           // this wave's block index
    if (bi < nb) {
        if constexpr (KV16) gload16(kb0 + bi * BK);
        else gload(kb0 + bi * BK);
    }
    for (; bi < nb; bi += NW) {
        const int kb = kb0 + bi * BK;
        // the wave's own slice: its LDS ops stay in order
        if constexpr (KV16) lstore16();
        else lstore();
        if (bi + NW < nb) {
            if constexpr (KV16) gload16(kb + NW * BK);
            else gload(kb + NW * BK);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        // S^T tiles: keys 16j + 4*g4 + r (register r) for query ql
        f32x4 sc[BK / 16];
#pragma unroll
        for (int j = 0; j < BK / 16; j++) {
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NS; s++) {
                const int off = (16 * j + ql) * KRS + 64 * s + 16 * g4;
                const u32x4 kh = *(const u32x4 *)&ksl[off];
                acc = mfma16<DT>(kh, qh[s], acc);
                if constexpr (QP == 2) acc = mfma16<DT>(kh, qlo[s], acc);
                if constexpr (LO) acc = mfma16<DT>(*(const u32x4 *)&ksl[KSL + off], qh[s], acc);
            }
            sc[j] = acc;
        }
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < BK / 16; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int jg = kb + 16 * j + 4 * g4 + r;
                const float v = (jg >= jlo && jg <= t) ? sc[j][r] * sl2 : -INFINITY;
                sc[j][r] = v;
                mx = fmaxf(mx, v);
            }
        mx = max_rows(mx);
        const float m_new = fmaxf(m_run, mx);
        const float rescale = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        l_part *= rescale;
#pragma unroll
        for (int i = 0; i < NO; i++) o[i] *= rescale;
        // P (unnormalised) as B operands of O^T = V^T . P^T, 32-key steps
#pragma unroll
        for (int s2 = 0; s2 < BK / 32; s2++) {
            float p[8];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float a = sc[2 * s2][r], b = sc[2 * s2 + 1][r];
                p[r] = a == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(a - m_new);
                p[4 + r] = b == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(b - m_new);
            }
#pragma unroll
            for (int e = 0; e < 8; e++) l_part += p[e];
            u32x4 ph, pl;
            split8_hw<DT>(p, ph, pl);
#pragma unroll
            for (int i = 0; i < NO; i++) {
                const int off = (16 * i + ql) * VRS + 64 * s2 + 8 * g4;
                const uint2 a0 = *(const uint2 *)&vsl[off], a1 = *(const uint2 *)&vsl[off + 32];
                const u32x4 vh = u32x4{a0.x, a0.y, a1.x, a1.y};
                o[i] = mfma16<DT>(vh, ph, o[i]);
                if constexpr (QP == 2) o[i] = mfma16<DT>(vh, pl, o[i]);
                if constexpr (LO) {
                    const uint2 b0 = *(const uint2 *)&vsl[VSL + off], b1 = *(const uint2 *)&vsl[VSL + off + 32];
                    o[i] = mfma16<DT>(u32x4{b0.x, b0.y, b1.x, b1.y}, ph, o[i]);
                }
            }
        }
        // the next lstore rewrites this slice: its reads above must be issued first
        __builtin_amdgcn_wave_barrier();
    }
    // merge: wave w's (max, sum, O) for query q at mo[w][q], lo[w][q], oo[w][q][dim]
    const float l_w = sum_rows(l_part);
    __syncthreads();   // every wave is done with its K / V slices
    float *oo = (float *)lds;
    float *mo = oo + NW * BQ * OLD, *lsum = mo + NW * BQ;
    if (g4 == 0) {
        mo[wave * BQ + ql] = m_run;
        lsum[wave * BQ + ql] = l_w;
    }
#pragma unroll
    for (int i = 0; i < NO; i++)
        *(f32x4 *)&oo[(wave * BQ + ql) * OLD + 16 * i + 4 * g4] = o[i];
    __syncthreads();
    for (int e = tid; e < BQ * HD; e += kT) {
        const int q = e / HD, d = e % HD, tq = q0 + q;
        if (tq >= S) continue;
        float mm = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) mm = fmaxf(mm, mo[w * BQ + q]);
        float lt = 0.f, ot = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float mw = mo[w * BQ + q];
            const float f = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - mm);
            lt += lsum[w * BQ + q] * f;
            ot += oo[(w * BQ + q) * OLD + d] * f;
        }
        store_op16(att, (size_t)tq * qdim + h * HD + d, plane, ot * (1.0f / lt), DT);
    }
}

// The 64-query attention's tiles in the order the XCDs take them: chunks of QG consecutive
// query blocks (about one 1024-row sequence), within a chunk each kv head's QG blocks x its
// H/KVH q heads, the q heads of a kv head adjacent. The workgroups an XCD runs together then
// read the same sequence's K and V rows of one kv head (1 MB in fp32 at head dim 128), which
// its L2 keeps, instead of every XCD fetching every sequence's rows from memory.
__device__ __forceinline__ void attn64_tile(int t, int nqb, int H, int KVH, int &qb, int &h) {
    constexpr int QG = 16;
    const int R = H / KVH, r = t % R, u = t / R;
    const int span = QG * KVH, nc = nqb / QG;
    int kvh;
    if (u < nc * span) {
        const int c = u / span, rem = u % span;
        kvh = rem / QG;
        qb = c * QG + rem % QG;
    } else {
        const int v = u - nc * span, tail = nqb - nc * QG;
        kvh = v / tail;
        qb = nc * QG + v % tail;
    }
    h = kvh * R + r;
}

// The same attention with 64 queries x one head per workgroup (16 per wave) and the key
// blocks (64 keys) staged once per workgroup for all four waves, the next block loaded into
// registers while the current one is consumed. It stages a quarter of the K/V traffic of the
// 16-query form, which wins once the grid fills the chip on its own (long or many sequences);
// the 16-query form wins on short inputs, whose S/64 x H workgroups leave CUs idle. One-
// dimensional grid of ceil(S/64) x H workgroups, tiles in attn64_tile's order.
template <int DT, int HD, bool LO>
__global__ __launch_bounds__(kT) void k_attn_prefill_mfma64(const float *qf, const float *kf,
                                                          const float *vf, int S,
                                                          const int32_t *rowpos, int H, int KVH,
                                                          float scale, uint16_t *att, size_t plane) {
    constexpr int BQ = 64, BK = 64, NP = LO ? 2 : 1;
    constexpr int KRS = HD * 2 + 16;              // LDS bytes per K row (16-byte pad)
    constexpr int VRS = BK * 2 + 8;               // LDS bytes per V^T row (8-byte pad)
    constexpr int KT = BK * HD / 8;               // K staging tasks: (key, 8 dims)
    constexpr int VT = (BK / 4) * (HD / 4);       // V staging tasks: (4 keys, 4 dims)
    constexpr int KPT = (KT + kT - 1) / kT, VPT = (VT + kT - 1) / kT;
    constexpr int NS = HD / 32, NO = HD / 16;     // QK k-steps, O^T tiles
    __shared__ __attribute__((aligned(16))) uint8_t ks[NP][BK * KRS];
    __shared__ __attribute__((aligned(16))) uint8_t vts[NP][HD * VRS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g4 = lane >> 4, ql = lane & 15;
    const int nqb = (S + BQ - 1) / BQ;
    int qb, h;
    attn64_tile(xcd_tile(blockIdx.x, nqb * H), nqb, H, KVH, qb, h);
    const int q0 = qb * BQ;
    const int qdim = H * HD, kvdim = KVH * HD, kvh = h / (H / KVH);
    const int kstart = q0 - rowpos[q0];
    const int qlast = min(q0 + BQ, S) - 1;

    // this lane's query and its Q operand planes (B operand: dims 32s + 8*g4 .. +7)
    const int t = q0 + 16 * wave + ql;
    const bool tok = t < S;
    const int jlo = tok ? t - rowpos[t] : 0x7fffffff;
    u32x4 qh[NS], qlo[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        float f[8];
        if (tok) {
            const f32x4 a = *(const f32x4 *)(qf + (size_t)t * qdim + h * HD + 32 * s + 8 * g4);
            const f32x4 b = *(const f32x4 *)(qf + (size_t)t * qdim + h * HD + 32 * s + 8 * g4 + 4);
            f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) f[e] = 0.f;
        }
        split8<DT>(f, qh[s], qlo[s]);
    }
    const int wlast = min(q0 + 16 * wave + 15, S - 1);   // the wave's last row

    // staging registers for the next key block
    f32x4 kst[KPT][2], vst[VPT][4];
    auto gload = [&](int kb) {
#pragma unroll
        for (int u = 0; u < KPT; u++) {
            const int c = tid + u * kT;
            if (KT % kT != 0 && c >= KT) break;
            const int r = c / (HD / 8), d = (c % (HD / 8)) * 8, j = kb + r;
            const float *src = kf + (size_t)j * kvdim + kvh * HD + d;
            kst[u][0] = j < S ? *(const f32x4 *)src : f32x4{0.f, 0.f, 0.f, 0.f};
            kst[u][1] = j < S ? *(const f32x4 *)(src + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < VPT; u++) {
            const int c = tid + u * kT;
            if (VT % kT != 0 && c >= VT) break;
            const int kq = c / (HD / 4), d = (c % (HD / 4)) * 4;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int j = kb + 4 * kq + i;
                vst[u][i] = j < S ? *(const f32x4 *)(vf + (size_t)j * kvdim + kvh * HD + d)
                                  : f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
    };
    auto lstore = [&]() {
#pragma unroll
        for (int u = 0; u < KPT; u++) {
            const int c = tid + u * kT;
            if (KT % kT != 0 && c >= KT) break;
            const int r = c / (HD / 8), d = (c % (HD / 8)) * 8;
            const float f[8] = {kst[u][0].x, kst[u][0].y, kst[u][0].z, kst[u][0].w,
                                kst[u][1].x, kst[u][1].y, kst[u][1].z, kst[u][1].w};
            u32x4 hi, lo;
            if constexpr (LO) split8_hw<DT>(f, hi, lo);
            else hi = u32x4{pack2_exact<DT>(f[0], f[1]), pack2_exact<DT>(f[2], f[3]),
                            pack2_exact<DT>(f[4], f[5]), pack2_exact<DT>(f[6], f[7])};
            *(u32x4 *)&ks[0][r * KRS + d * 2] = hi;
            if constexpr (LO) *(u32x4 *)&ks[NP - 1][r * KRS + d * 2] = lo;
        }
#pragma unroll
        for (int u = 0; u < VPT; u++) {
            const int c = tid + u * kT;
            if (VT % kT != 0 && c >= VT) break;
            const int kq = c / (HD / 4), d = (c % (HD / 4)) * 4;
#pragma unroll
            for (int i = 0; i < 4; i++) {   // dim d + i: keys 4kq .. 4kq+3
                const float a0 = vst[u][0][i], a1 = vst[u][1][i], a2 = vst[u][2][i], a3 = vst[u][3][i];
                const uint32_t h01 = LO ? pack2_hw<DT>(a0, a1) : pack2_exact<DT>(a0, a1);
                const uint32_t h23 = LO ? pack2_hw<DT>(a2, a3) : pack2_exact<DT>(a2, a3);
                *(uint2 *)&vts[0][(d + i) * VRS + 8 * kq] = uint2{h01, h23};
                if constexpr (LO) {
                    const float r0 = a0 - bits_to_f((uint16_t)h01, DT), r1 = a1 - bits_to_f((uint16_t)(h01 >> 16), DT);
                    const float r2 = a2 - bits_to_f((uint16_t)h23, DT), r3 = a3 - bits_to_f((uint16_t)(h23 >> 16), DT);
                    *(uint2 *)&vts[NP - 1][(d + i) * VRS + 8 * kq] =
                        uint2{pack2_hw<DT>(r0, r1), pack2_hw<DT>(r2, r3)};
                }
            }
        }
    };

    // scores in the base-2 domain (scale x log2 e), so each softmax term is one exp2
    const float sl2 = scale * 1.4426950408889634f;
    float m_run = -INFINITY, l_part = 0.f;
    f32x4 o[NO];
#pragma unroll
    for (int i = 0; i < NO; i++) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int kb0 = kstart & ~(BK - 1);
    gload(kb0);
    for (int kb = kb0; kb <= qlast; kb += BK) {
        __syncthreads();   // every wave is done reading the previous block
        lstore();
        __syncthreads();
        if (kb + BK <= qlast) gload(kb + BK);
        if (q0 + 16 * wave >= S || wlast < kb) continue;   // no row of this wave sees the block
        // S^T tiles: keys 16j + 4*g4 + r (register r) for query ql
        f32x4 sc[BK / 16];
#pragma unroll
        for (int j = 0; j < BK / 16; j++) {
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NS; s++) {
                const int off = (16 * j + ql) * KRS + 64 * s + 16 * g4;
                const u32x4 kh = *(const u32x4 *)&ks[0][off];
                acc = mfma16<DT>(kh, qh[s], acc);
                acc = mfma16<DT>(kh, qlo[s], acc);
                if constexpr (LO) acc = mfma16<DT>(*(const u32x4 *)&ks[NP - 1][off], qh[s], acc);
            }
            sc[j] = acc;
        }
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < BK / 16; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int jg = kb + 16 * j + 4 * g4 + r;
                const float v = (jg >= jlo && jg <= t) ? sc[j][r] * sl2 : -INFINITY;
                sc[j][r] = v;
                mx = fmaxf(mx, v);
            }
        mx = max_rows(mx);
        const float m_new = fmaxf(m_run, mx);
        const float rescale = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        l_part *= rescale;
#pragma unroll
        for (int i = 0; i < NO; i++) o[i] *= rescale;
        // P (unnormalised) as B operands of O^T = V^T . P^T, two 32-key steps
#pragma unroll
        for (int s2 = 0; s2 < BK / 32; s2++) {
            float p[8];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float a = sc[2 * s2][r], b = sc[2 * s2 + 1][r];
                p[r] = a == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(a - m_new);
                p[4 + r] = b == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(b - m_new);
            }
#pragma unroll
            for (int e = 0; e < 8; e++) l_part += p[e];
            u32x4 ph, pl;
            split8_hw<DT>(p, ph, pl);
#pragma unroll
            for (int i = 0; i < NO; i++) {
                const int off = (16 * i + ql) * VRS + 64 * s2 + 8 * g4;
                const uint2 a0 = *(const uint2 *)&vts[0][off], a1 = *(const uint2 *)&vts[0][off + 32];
                const u32x4 vh = u32x4{a0.x, a0.y, a1.x, a1.y};
                o[i] = mfma16<DT>(vh, ph, o[i]);
                o[i] = mfma16<DT>(vh, pl, o[i]);
                if constexpr (LO) {
                    const uint2 b0 = *(const uint2 *)&vts[NP - 1][off], b1 = *(const uint2 *)&vts[NP - 1][off + 32];
                    o[i] = mfma16<DT>(u32x4{b0.x, b0.y, b1.x, b1.y}, ph, o[i]);
                }
            }
        }
    }
    const float l_tot = sum_rows(l_part);
    if (!tok) return;
    const float inv = 1.0f / l_tot;
#pragma unroll
    for (int i = 0; i < NO; i++)
#pragma unroll
        for (int r = 0; r < 4; r++)
            store_op16(att, (size_t)t * qdim + h * HD + 16 * i + 4 * g4 + r, plane, o[i][r] * inv, DT);
}

// Causal attention (forward_common.go:5-33): one wave per (query t, head h). Row t is
// position rowpos[t] of its sequence, whose rows are the rowpos[t] rows before it, so the keys
// are j in [t - rowpos[t], t]. Lanes walk the keys in blocks of 64; scores are kept in LDS,
// then the softmax and P.V with lanes over the head dims. decode_forms = 0 is the
// full-sequence form (accel_other.go:190-207: float64 exp terms summed unrounded); 1 is the
// decode form (infer.go:328-345: the float32-rounded terms summed). Both scale by
// float32(1/sum) and give masked keys exactly 0.
__global__ __launch_bounds__(kT) void k_attn_prefill(const float *qf, const float *kf,
                                                     const float *vf, int S, int seg_max,
                                                     const int32_t *rowpos, int H, int KVH,
                                                     int hd, float scale, int dt, int decode_forms,
                                                     uint16_t *att, size_t plane) {
    extern __shared__ float sh_scores[];   // [waves][seg_max]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x * (blockDim.x >> 6) + wave;
    const int h = blockIdx.y;
    if (t >= S) return;
    const int qdim = H * hd, kvdim = KVH * hd, kvh = h / (H / KVH);
    const int j0 = t - rowpos[t], n = rowpos[t] + 1;   // keys j0 .. t
    float *sc = sh_scores + (size_t)wave * seg_max;
    const float *q = qf + (size_t)t * qdim + h * hd;
    float mx = -INFINITY;
    for (int b = 0; b < n; b += 64) {
        const int jj = b + lane;
        float s = -INFINITY;
        if (jj < n) {
            const float *k = kf + (size_t)(j0 + jj) * kvdim + kvh * hd;
            float d = 0.f;
            for (int i = 0; i < hd; i += 4) {
                const f32x4 qa = *(const f32x4 *)(q + i), ka = *(const f32x4 *)(k + i);
#pragma unroll
                for (int w = 0; w < 4; w++) d = fmaf(qa[w], ka[w], d);
            }
            s = d * scale;
            sc[jj] = s;
        }
        mx = fmaxf(mx, s);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    double sum = 0;
    for (int jj = lane; jj < n; jj += 64) {
        const double e = exp((double)(sc[jj] - mx));
        sc[jj] = (float)e;
        sum += decode_forms ? (double)(float)e : e;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    const float inv = (float)(1.0 / sum);
    __builtin_amdgcn_wave_barrier();
    for (int i = lane; i < hd; i += 64) {
        float a = 0.f;
        for (int jj = 0; jj < n; jj++)
            a = fmaf(sc[jj] * inv, vf[(size_t)(j0 + jj) * kvdim + kvh * hd + i], a);
        store_op16(att, (size_t)t * qdim + h * hd + i, plane, a, dt);
    }
}

// Epilogue of the skinny GEMM for output columns n, n+1 of row m.
__device__ __forceinline__ void skinny_epilogue(const GemmArgs &g, int m, int n, float v0, float v1) {
    if (g.epi == G_GATE) {
        // columns 2q (W1) and 2q+1 (W3) of the interleaved weight rows
        store_op16(g.out16, (size_t)m * (g.N / 2) + (n >> 1), (size_t)g.M * (g.N / 2),
                   silu_gate<false>(v0, v1, g.decode_forms), g.dt);
        return;
    }
    const float v[2] = {v0, v1};
#pragma unroll
    for (int j = 0; j < 2; j++) {
        if (g.epi == G_STORE) g.out[(size_t)m * g.N + n + j] = v[j];
        else if (g.epi == G_RESID)
            g.out[(size_t)m * g.N + n + j] = g.resid[(size_t)m * g.N + n + j] + g.alpha * v[j];
        else g.out[(size_t)(n + j) * g.M + m] = v[j];
    }
}

// Skinny GEMM for batched decode: C[M, N] = A[M, K] . W[N, K]^T with M <= 32 token rows.
// Workgroup (x, y) owns 16 output columns and the K range [y*kc, (y+1)*kc); its four waves
// each take a quarter of that range for both 16-row MFMA blocks (hi and lo operand planes),
// issuing two k-steps of loads before their MFMAs, and the four partial tiles are added
// through LDS in a fixed order. With one K range the epilogue runs here; otherwise the tile
// goes to `partial` ([ranges][M][N]) for k_gemm_skinny_reduce. Needs kc % 128 == 0,
// N % 16 == 0.
template <int DT>
__global__ __launch_bounds__(kT) void k_gemm_skinny(GemmArgs g, float *partial, int kc) {
    __shared__ float part[4][32][17];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * 16;
    const int lr = lane & 15, lk = (lane >> 4) * 8;
    const int kq = kc / 4, kb = blockIdx.y * kc + wave * kq;
    const size_t lo = (size_t)g.M * g.K;
    const bool ok0 = lr < g.M, ok1 = 16 + lr < g.M;
    const uint16_t *a0 = g.A + (size_t)(ok0 ? lr : 0) * g.K + lk;
    const uint16_t *a1 = g.A + (size_t)(ok1 ? 16 + lr : 0) * g.K + lk;
    const uint16_t *bp = g.B + (size_t)(n0 + lr) * g.K + lk;
    const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
    f32x4 c0 = f32x4{0.f, 0.f, 0.f, 0.f}, c1 = c0;
    for (int k = kb; k < kb + kq; k += 64) {
        const bool two = k + 32 < kb + kq;
        u32x4 b[2], x0[2], x0l[2], x1[2], x1l[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int kk = k + 32 * u;
            const bool in = u == 0 || two;
            b[u] = in ? *(const u32x4 *)(bp + kk) : zero;
            x0[u] = in && ok0 ? *(const u32x4 *)(a0 + kk) : zero;
            x0l[u] = in && ok0 ? *(const u32x4 *)(a0 + lo + kk) : zero;
            x1[u] = in && ok1 ? *(const u32x4 *)(a1 + kk) : zero;
            x1l[u] = in && ok1 ? *(const u32x4 *)(a1 + lo + kk) : zero;
        }
#pragma unroll
        for (int u = 0; u < 2; u++) {
            c0 = mfma16<DT>(x0[u], b[u], c0);
            c0 = mfma16<DT>(x0l[u], b[u], c0);
            c1 = mfma16<DT>(x1[u], b[u], c1);
            c1 = mfma16<DT>(x1l[u], b[u], c1);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        part[wave][4 * (lane >> 4) + r][lr] = c0[r];
        part[wave][16 + 4 * (lane >> 4) + r][lr] = c1[r];
    }
    __syncthreads();
    const int m = threadIdx.x >> 3, nn = (threadIdx.x & 7) * 2;   // columns nn, nn+1 of row m
    if (m >= g.M) return;
    float v[2];
#pragma unroll
    for (int j = 0; j < 2; j++)
        v[j] = ((part[0][m][nn + j] + part[1][m][nn + j]) + part[2][m][nn + j]) + part[3][m][nn + j];
    if (gridDim.y == 1 && !g.partial_only) {
        skinny_epilogue(g, m, n0 + nn, v[0], v[1]);
    } else {
        float *dst = partial + ((size_t)blockIdx.y * g.M + m) * g.N + n0 + nn;
        dst[0] = v[0];
        dst[1] = v[1];
    }
}

// Skinny GEMM with the activation rows shared through LDS: workgroup (x, y) owns 64 output
// columns (16 per wave) and the K range [y*kc, (y+1)*kc), walked in 256-wide chunks. Each
// chunk's A rows (hi and lo planes, 32 rows, rows padded to 264 elements so the MFMA reads of
// 16 rows fall in distinct banks) are copied into LDS once for the four waves; each wave
// loads its 16 weight rows for the chunk (eight 16-byte loads per lane, in flight while A is
// staged) and issues four MFMAs per 32-wide k-step. The wave tiles go through LDS to the same
// epilogue / partial layout as k_gemm_skinny. Needs kc % 256 == 0 and N % 64 == 0.
constexpr int kSkA = 264;   // padded row of a staged A chunk (elements)
template <int DT>
__global__ __launch_bounds__(kT) void k_gemm_skinny64(GemmArgs g, float *partial, int kc) {
    __shared__ __attribute__((aligned(16))) uint16_t as[2][32][kSkA];
    __shared__ float part[4][32][17];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nw0 = blockIdx.x * 64 + wave * 16;
    const int lr = lane & 15, lk = (lane >> 4) * 8;
    const size_t lo = (size_t)g.M * g.K;
    const int kbeg = blockIdx.y * kc;
    const uint16_t *bp = g.B + (size_t)(nw0 + lr) * g.K + lk;
    const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
    f32x4 c0 = f32x4{0.f, 0.f, 0.f, 0.f}, c1 = c0;
    for (int k0 = kbeg; k0 < kbeg + kc; k0 += 256) {
        u32x4 b[8];
#pragma unroll
        for (int st = 0; st < 8; st++) b[st] = *(const u32x4 *)(bp + k0 + 32 * st);
        // the previous chunk's A reads are done (LDS only; the weight loads stay in flight)
        __asm__ __volatile__("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        for (int i = threadIdx.x; i < 2 * 32 * 32; i += kT) {
            const int pl = i >> 10, r = (i >> 5) & 31, u = i & 31;
            const u32x4 v = r < g.M ? *(const u32x4 *)(g.A + pl * lo + (size_t)r * g.K + k0 + u * 8) : zero;
            *(u32x4 *)&as[pl][r][u * 8] = v;
        }
        __asm__ __volatile__("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
        for (int st = 0; st < 8; st++) {
            const int kk = 32 * st + lk;
            const u32x4 x0 = *(const u32x4 *)&as[0][lr][kk], x0l = *(const u32x4 *)&as[1][lr][kk];
            const u32x4 x1 = *(const u32x4 *)&as[0][16 + lr][kk], x1l = *(const u32x4 *)&as[1][16 + lr][kk];
            c0 = mfma16<DT>(x0, b[st], c0);
            c0 = mfma16<DT>(x0l, b[st], c0);
            c1 = mfma16<DT>(x1, b[st], c1);
            c1 = mfma16<DT>(x1l, b[st], c1);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        part[wave][4 * (lane >> 4) + r][lr] = c0[r];
        part[wave][16 + 4 * (lane >> 4) + r][lr] = c1[r];
    }
    __syncthreads();
    const int m = threadIdx.x >> 3, nn = (threadIdx.x & 7) * 2;   // columns nn, nn+1 of row m
    if (m >= g.M) return;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int n = blockIdx.x * 64 + t * 16 + nn;
        const float v0 = part[t][m][nn], v1 = part[t][m][nn + 1];
        if (gridDim.y == 1 && !g.partial_only) {
            skinny_epilogue(g, m, n, v0, v1);
        } else {
            float *dst = partial + ((size_t)blockIdx.y * g.M + m) * g.N + n;
            dst[0] = v0;
            dst[1] = v1;
        }
    }
}

// Adds the K-range partials of the skinny GEMM in range order, then the epilogue.
__global__ __launch_bounds__(kT) void k_gemm_skinny_reduce(GemmArgs g, const float *partial, int ranges) {
    const int idx = blockIdx.x * kT + threadIdx.x;
    const int half = g.N / 2;
    if (idx >= g.M * half) return;
    const int m = idx / half, n = (idx % half) * 2;
    float v0 = 0.f, v1 = 0.f;
    for (int r = 0; r < ranges; r++) {
        const float *src = partial + ((size_t)r * g.M + m) * g.N + n;
        v0 += src[0];
        v1 += src[1];
    }
    skinny_epilogue(g, m, n, v0, v1);
}

constexpr int kMaxGroupB = 4;          // q heads per kv head in the batched attention
constexpr int kKvTile = 32 * 1024;     // LDS bytes for one chunk of K rows (and as many for V)

// Keys per split of the batched attention for a cache row of row_bytes: a chunk's K rows
// fill kKvTile, at most 256.
__host__ __device__ constexpr int attn_chunk(int row_bytes) {
    return kKvTile / row_bytes < 256 ? kKvTile / row_bytes : 256;
}

// Copies rows [0, n) of a cache slab (row r at byte r*stride) into LDS, rows of rb bytes
// packed back to back, with global_load_lds (each lane moves 16 bytes; a wave instruction
// fills 1 KB). Rows n..cap-1 of the tile re-read row n-1, so every lane reads valid memory.
__device__ __forceinline__ void rows_to_lds(const uint8_t *src, size_t stride, int n, int cap,
                                            int rb, uint8_t *lds) {
    const int lpr = rb / 16, rpi = 64 / lpr;   // lanes per row, rows per wave instruction
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int r_in = lane / lpr, c_in = (lane % lpr) * 16;
    for (int r0 = wave * rpi; r0 < cap; r0 += nw * rpi) {
        int r = r0 + r_in;
        if (r >= n) r = n - 1;
        __builtin_amdgcn_global_load_lds(
            (const __attribute__((address_space(1))) void *)(src + (size_t)r * stride + c_in),
            (__attribute__((address_space(3))) void *)(lds + (size_t)r0 * rb), 16, 0, 0);
    }
}

template <int KVT>
__device__ __forceinline__ float kv_elem(const uint8_t *row, int i) {
    if constexpr (KVT == SH_KV_F32) return ((const float *)row)[i];
    else return bits_to_f(((const uint16_t *)row)[i], KVT == SH_KV_BF16 ? SH_DTYPE_BF16 : SH_DTYPE_F16);
}

// Batched decode attention, split over the keys (one workgroup per (chunk, kv head,
// sequence); two fit on a CU): the chunk's K and V rows are copied into LDS in one burst,
// then the scores of the group's q heads (one thread per key, 16-byte slices visited in a
// rotated order so a wave's LDS reads spread over the banks), the chunk's max m and sum l
// of exp(s - m), and the unnormalised P.V (thread = one 16-byte slice of the V rows over a
// share of the keys; shares added through LDS, reusing the K tile), written as partials
// for k_attn_batch_combine. Sequence b attends to positions 0..pos[b] of its cache.
template <int KVT>
__global__ __launch_bounds__(kT) void k_attn_batch_partial(
    const float *q, const void *kc, const void *vc, size_t kv_seq_stride, const int32_t *pos,
    int H, int KVH, int hd, float scale, int nch, float *pm, float *pl, float *pacc) {
    __shared__ __attribute__((aligned(16))) uint8_t kt[kKvTile];
    __shared__ __attribute__((aligned(16))) uint8_t vt[kKvTile];
    __shared__ __attribute__((aligned(16))) float qs[kMaxGroupB * 256];
    __shared__ float sc[kMaxGroupB][256];
    __shared__ float redm[kMaxGroupB][kT / 64];
    constexpr int EB = KVT == SH_KV_F32 ? 4 : 2;
    const int rb = hd * EB, C = attn_chunk(rb);
    const int c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int P = pos[b] + 1;
    const int t0 = c * C;
    if (t0 >= P) return;
    const int n = min(C, P - t0);
    const int group = H / KVH, qdim = H * hd, kvdim = KVH * hd;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t base = ((size_t)b * kv_seq_stride + (size_t)t0 * kvdim + (size_t)g * hd) * EB;
    rows_to_lds((const uint8_t *)kc + base, (size_t)kvdim * EB, n, n, rb, kt);
    rows_to_lds((const uint8_t *)vc + base, (size_t)kvdim * EB, n, n, rb, vt);
    for (int i = threadIdx.x; i < group * hd; i += kT)
        qs[i] = q[(size_t)b * qdim + (size_t)g * group * hd + i];
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // scores: thread t <-> key t0 + t
    const int nsl = rb / 16;                   // 16-byte slices per row
    constexpr int EPS = 16 / EB;               // elements per slice
    for (int t = threadIdx.x; t < n; t += kT) {
        float d[kMaxGroupB] = {0.f, 0.f, 0.f, 0.f};
        const u32x4 *row = (const u32x4 *)(kt + (size_t)t * rb);
#pragma unroll 4
        for (int s0 = 0; s0 < nsl; s0++) {
            const int sl = (s0 + t) % nsl;
            const u32x4 raw = row[sl];
            float kf[8];
            if constexpr (KVT == SH_KV_F32) {
#pragma unroll
                for (int e = 0; e < 4; e++) kf[e] = __uint_as_float(raw[e]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int dtk = KVT == SH_KV_BF16 ? SH_DTYPE_BF16 : SH_DTYPE_F16;
                    kf[2 * e] = bits_to_f(raw[e] & 0xffffu, dtk);
                    kf[2 * e + 1] = bits_to_f(raw[e] >> 16, dtk);
                }
            }
#pragma unroll
            for (int h = 0; h < kMaxGroupB; h++) {
                if (h >= group) break;
#pragma unroll
                for (int e = 0; e < EPS; e++) d[h] = fmaf(qs[h * hd + sl * EPS + e], kf[e], d[h]);
            }
        }
#pragma unroll
        for (int h = 0; h < kMaxGroupB; h++)
            if (h < group) sc[h][t] = d[h] * scale;
    }
    __syncthreads();
    // per head: chunk max, exp terms, their sum
    for (int h = 0; h < group; h++) {
        float mx = -INFINITY;
        for (int t = threadIdx.x; t < n; t += kT) mx = fmaxf(mx, sc[h][t]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        if (lane == 0) redm[h][wave] = mx;
    }
    __syncthreads();
    float mh[kMaxGroupB];
    for (int h = 0; h < group; h++) {
        mh[h] = redm[h][0];
        for (int w = 1; w < kT / 64; w++) mh[h] = fmaxf(mh[h], redm[h][w]);
    }
    __syncthreads();
    for (int h = 0; h < group; h++) {
        float sum = 0.f;
        for (int t = threadIdx.x; t < n; t += kT) {
            const float e = expf(sc[h][t] - mh[h]);
            sc[h][t] = e;
            sum += e;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
        if (lane == 0) redm[h][wave] = sum;
    }
    __syncthreads();
    const size_t pbase = ((size_t)b * H + (size_t)g * group) * nch + c;
    if (threadIdx.x < group) {
        const int h = threadIdx.x;
        float l = 0.f;
        for (int w = 0; w < kT / 64; w++) l += redm[h][w];
        pm[pbase + (size_t)h * nch] = mh[h];
        pl[pbase + (size_t)h * nch] = l;
    }
    // P.V from LDS: thread (slice, key set) accumulates EPS dims of every head over the keys
    // t = ks, ks + nks, ...; the key-set partials go to LDS (the K tile is free now) and are
    // added in key-set order
    const int nks = kT / nsl;
    const int sl = threadIdx.x % nsl, ks = threadIdx.x / nsl;
    float acc[kMaxGroupB][8];
#pragma unroll
    for (int h = 0; h < kMaxGroupB; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[h][e] = 0.f;
#pragma unroll 4
    for (int t = ks; t < n; t += nks) {
        const u32x4 raw = ((const u32x4 *)(vt + (size_t)t * rb))[sl];
        float vf[8];
        if constexpr (KVT == SH_KV_F32) {
#pragma unroll
            for (int e = 0; e < 4; e++) vf[e] = __uint_as_float(raw[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int dtk = KVT == SH_KV_BF16 ? SH_DTYPE_BF16 : SH_DTYPE_F16;
                vf[2 * e] = bits_to_f(raw[e] & 0xffffu, dtk);
                vf[2 * e + 1] = bits_to_f(raw[e] >> 16, dtk);
            }
        }
#pragma unroll
        for (int h = 0; h < kMaxGroupB; h++) {
            if (h >= group) break;
            const float p = sc[h][t];
#pragma unroll
            for (int e = 0; e < EPS; e++) acc[h][e] = fmaf(p, vf[e], acc[h][e]);
        }
    }
    float *pv = (float *)kt;   // [nks][group * hd]
    const int gw = group * hd;
#pragma unroll
    for (int h = 0; h < kMaxGroupB; h++) {
        if (h >= group) break;
#pragma unroll
        for (int e = 0; e < EPS; e++) pv[(size_t)ks * gw + h * hd + sl * EPS + e] = acc[h][e];
    }
    __syncthreads();
    for (int k = threadIdx.x; k < gw; k += kT) {
        float a = 0.f;
        for (int r = 0; r < nks; r++) a += pv[(size_t)r * gw + k];
        pacc[(pbase + (size_t)(k / hd) * nch) * hd + k % hd] = a;
    }
}

// Tagged words for the streaming attention's split partials: (float bits, 32-bit tag) in one
// 64-bit device-scope store, so a reader knows a word is this layer's and step's without a
// fence (a device-scope release would write back the whole L2 on this part).
__device__ __forceinline__ void tag_put(uint64_t *p, float v, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
// The value of a tagged word once it carries `tag`. The wait is bounded (about a second): a
// word still missing then sets *err (the decode call reports the failure after the step) and is
// taken as it is, so no wave can hang.
__device__ __forceinline__ float tag_get(const uint64_t *p, uint32_t tag, int *err) {
    uint64_t w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int spins = 0;
    for (; (uint32_t)(w >> 32) != tag && spins < (1 << 22); spins++) {
        __builtin_amdgcn_s_sleep(1);
        w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if ((uint32_t)(w >> 32) != tag) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __uint_as_float((uint32_t)w);
}

constexpr int kAT = 512;                  // threads of the streaming batched attention
constexpr int kAWT = 1024;                // threads of its lane-group form (one workgroup per CU)

// The rows of the q|k|v projection that workgroup (kv head g, sequence b) of the batched
// attention needs, finished as k_row_qkv would finish the whole row and in the same float
// order: the skinny GEMM's K-range partials added in range order, then QK-norm and RoPE at
// position P - 1 for the group's q heads and for kv head g (qk_rope_row's per-head code,
// restricted to those heads). rowq gets the q heads, then k, then v; k and v as the cache
// holds them (rounded to its type), and written to the cache when `last`. The RoPE factors,
// the QK-norm gains and up to four ranges' partials are requested together at the start, so
// the prologue waits out one memory latency. NT threads; ends with a workgroup barrier.
template <int KVT, int HD, int GROUP, int NT = kAT>
__device__ __forceinline__ void batch_qkv_rows(const float *partial, int ranges, const QkRopeArgs &a,
                                               const void *kc, const void *vc, size_t kv_seq_stride, int kvdim,
                                               int b, int g, int P, bool last, float *rowq) {
    static_assert(HD <= 128 && (GROUP + 2) * HD <= 2 * NT && (GROUP + 1) * HD / 2 <= NT, "one pass per step");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tp = P - 1, half = HD / 2;
    // RoPE factors of pair tid, QK-norm gains of wave (head) w's elements lane, lane + 64
    float rc = 0.f, rsn = 0.f, gn0 = 0.f, gn1 = 0.f;
    if (tid < (GROUP + 1) * half) {
        const int pi = tid % half;
        rc = a.rope_cos[tp * half + pi];
        rsn = a.rope_sin[tp * half + pi];
    }
    const bool norm_wave = a.qk_norm && wave <= GROUP;
    if (norm_wave) {
        const float *gn = wave < GROUP ? a.q_norm : a.k_norm;
        if (lane < HD) gn0 = gn[lane];
        if (lane + 64 < HD) gn1 = gn[lane + 64];
    }
    const int nrow = a.qdim + 2 * a.kvdim;
    for (int i = tid; i < (GROUP + 2) * HD; i += NT) {
        const int col = i < GROUP * HD ? g * GROUP * HD + i
                                       : (i < (GROUP + 1) * HD ? a.qdim + g * HD + (i - GROUP * HD)
                                                               : a.qdim + a.kvdim + g * HD + (i - (GROUP + 1) * HD));
        float v = 0.f;
        for (int r0 = 0; r0 < ranges; r0 += 4) {
            float q[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (r0 + j < ranges) q[j] = partial[((size_t)(r0 + j) * gridDim.z + b) * nrow + col];
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (r0 + j < ranges) v += q[j];
        }
        rowq[i] = v;
    }
    __syncthreads();
    // QK-norm (wave w normalises head w: the q heads, then k), RoPE at pos[b]
    if (norm_wave) {
        float *v = rowq + wave * HD;
        double ss = 0;
        for (int i = lane; i < HD; i += 64) ss += (double)v[i] * (double)v[i];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
        const float rr = (float)(1.0 / sqrt(ss / (double)HD + a.qk_eps));
        if (lane < HD) v[lane] = v[lane] * rr * gn0;
        if (lane + 64 < HD) v[lane + 64] = v[lane + 64] * rr * gn1;
    }
    __syncthreads();
    if (tid < (GROUP + 1) * half) {
        const float e = rowq[2 * tid], o = rowq[2 * tid + 1];
        rowq[2 * tid] = e * rc - o * rsn;
        rowq[2 * tid + 1] = o * rc + e * rsn;
    }
    __syncthreads();
    // the k and v row into the cache (once per sequence and kv head), and as the cache holds
    // them into rowq
    for (int i = tid; i < 2 * HD; i += NT) {
        const float v = rowq[GROUP * HD + i];
        if (last) kv_store<KVT>(i < HD ? (void *)kc : (void *)vc,
                                (size_t)b * kv_seq_stride + (size_t)tp * kvdim + g * HD + (i % HD), v);
        rowq[GROUP * HD + i] = kv_round<KVT>(v);
    }
    __syncthreads();
}
constexpr int kChunkBytes = 16 * 1024;    // bytes of K rows per streamed chunk (as many of V)

// Batched decode attention that streams the cache (flash decoding): workgroup (split, kv
// head g, sequence b) walks its share of the chunks of C = 16 KB / row-bytes keys. It first
// finishes its rows of the q|k|v projection itself, as k_row_qkv would for the whole row and
// in the same float order: the skinny GEMM's K-range partials added in range order, then
// QK-norm and RoPE at pos[b] for the group's q heads and for kv head g (qk_rope_row's
// per-head code, restricted to those heads). The workgroup holding the sequence's last
// chunk writes k and v to the cache and patches that row of its LDS copy of the chunk (the
// chunk's global load may predate the write). Chunk
// i+1's K and V rows are loaded into registers (64 bytes per thread) while chunk i is
// computed from LDS, then written to the other pair of LDS buffers. (An LDS DMA would not
// overlap: the compiler makes every LDS read wait for all DMA in flight.)
// Per chunk: lane-sliced scores of the group's q heads (RB/16 lanes per row, the slice dot
// products added by DPP), the running maximum and the rescaled sum of exp terms (online
// softmax), and P.V by thread (dim, key group) with the chunk's weights from LDS. One split
// writes the output row directly (a GEMM operand, hi/lo planes); several splits leave
// (m, l, acc) partials, which the last split to finish merges. Sequence b attends to 0..pos[b].
template <int KVT, int HD, int GROUP>
__global__ __launch_bounds__(kAT) __attribute__((amdgpu_waves_per_eu(GROUP == 4 ? 2 : 4))) void k_attn_batch_stream(
    const float *partial, int ranges, QkRopeArgs a, const void *kc, const void *vc, size_t kv_seq_stride,
    const int32_t *pos, int H, int KVH, float scale, int nsplit, int nch_buf, int dt, size_t plane,
    uint16_t *att, uint64_t *tm, uint64_t *tl_, uint64_t *tacc, int *cnt, const uint32_t *gen, int layer,
    int n_layers, int max_seq, int *err) {
    constexpr int EB = KVT == SH_KV_F32 ? 4 : 2;
    constexpr int RB = HD * EB;                        // bytes per cache row
    constexpr int C = kChunkBytes / RB;                // keys per chunk
    constexpr int LPK = RB / 16, EPC = 16 / EB, PPW = 64 / LPK;
    constexpr int NW = kAT / 64;
    constexpr int NKG = kAT / HD;                      // key groups of the P.V threads
    constexpr int SB = C / (NW * PPW);                 // row blocks per wave per chunk
    static_assert(C % (NW * PPW) == 0 && C % (4 * NKG) == 0, "chunk tiling");
    __shared__ __attribute__((aligned(16))) uint8_t kbuf[2][kChunkBytes];
    __shared__ __attribute__((aligned(16))) uint8_t vbuf[2][kChunkBytes];
    __shared__ float sc[GROUP][C];
    __shared__ float redm[NW][GROUP], redl[NW][GROUP];
    __shared__ float part[NKG][GROUP][HD];
    __shared__ float rowq[(GROUP + 2) * HD];           // the group's q heads, then k, then v
    const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int P = pos[b] + 1;
    const int nchunks = (P + C - 1) / C;
    const int cps = (nchunks + nsplit - 1) / nsplit;
    const int c0 = split * cps, c1 = min(nchunks, c0 + cps);
    if (c0 >= c1) return;
    const int qdim = H * HD, kvdim = KVH * HD;
    // this call, step (position) and layer: never 0, the cleared words' tag
    const uint32_t tag = ((*gen * (uint32_t)(max_seq + 1) + (uint32_t)(P - 1)) * (uint32_t)n_layers +
                          (uint32_t)layer) + 1u;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t sbase = (size_t)b * kv_seq_stride + (size_t)g * HD;
    const int sl = lane % LPK, rin = lane / LPK;
    // Next-chunk prefetch through registers: thread tid holds 16-byte pieces tid + kAT*u of
    // the chunk's K rows and of its V rows (rows packed back to back); rows past the
    // sequence's last key re-read that key, and a chunk past the split's last re-reads that
    // chunk (never used), so every load is in bounds and none sits under a branch.
    constexpr int PPT = kChunkBytes / 16 / kAT;        // pieces per thread per operand
    static_assert(kChunkBytes % (16 * kAT) == 0, "chunk pieces split evenly");
    u32x4 pk[PPT], pv[PPT];
    auto fetch = [&](int ci) {
        ci = min(ci, c1 - 1);
        const int t0 = ci * C, n = min(C, P - t0);
        const size_t off = (sbase + (size_t)t0 * kvdim) * EB;
#pragma unroll
        for (int u = 0; u < PPT; u++) {
            const int pi = tid + kAT * u, r = min(pi / LPK, n - 1), c = pi % LPK;
            const size_t o = off + (size_t)r * kvdim * EB + (size_t)c * 16;
            pk[u] = *(const u32x4 *)((const uint8_t *)kc + o);
            pv[u] = *(const u32x4 *)((const uint8_t *)vc + o);
        }
    };
    // the last chunk's row of position pos[b] (-1: this workgroup holds no such row)
    const bool last = c1 == nchunks;
    const int prow = last ? P - 1 - (nchunks - 1) * C : -1;
    // LDS copy of a chunk; in the sequence's last chunk the threads that copied a piece of
    // row prow then overwrite it with this step's k / v as stored in the cache (from rowq)
    auto stash = [&](int buf, bool patch) {
#pragma unroll
        for (int u = 0; u < PPT; u++) {
            *(u32x4 *)(kbuf[buf] + (size_t)(tid + kAT * u) * 16) = pk[u];
            *(u32x4 *)(vbuf[buf] + (size_t)(tid + kAT * u) * 16) = pv[u];
        }
        if (!patch) return;
#pragma unroll
        for (int u = 0; u < PPT; u++) {
            const int pi = tid + kAT * u;
            if (pi / LPK != prow) continue;
            const int c = pi % LPK;
            uint32_t kk[4], vv[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if constexpr (KVT == SH_KV_F32) {
                    kk[e] = __float_as_uint(rowq[GROUP * HD + c * 4 + e]);
                    vv[e] = __float_as_uint(rowq[(GROUP + 1) * HD + c * 4 + e]);
                } else {
                    const int dtk = KVT == SH_KV_BF16 ? SH_DTYPE_BF16 : SH_DTYPE_F16;
                    const int i0 = c * 8 + 2 * e;
                    kk[e] = (uint32_t)f_to_bits(rowq[GROUP * HD + i0], dtk) |
                            ((uint32_t)f_to_bits(rowq[GROUP * HD + i0 + 1], dtk) << 16);
                    vv[e] = (uint32_t)f_to_bits(rowq[(GROUP + 1) * HD + i0], dtk) |
                            ((uint32_t)f_to_bits(rowq[(GROUP + 1) * HD + i0 + 1], dtk) << 16);
                }
            }
            *(u32x4 *)(kbuf[buf] + (size_t)pi * 16) = u32x4{kk[0], kk[1], kk[2], kk[3]};
            *(u32x4 *)(vbuf[buf] + (size_t)pi * 16) = u32x4{vv[0], vv[1], vv[2], vv[3]};
        }
    };
    float m_run[GROUP], L[GROUP], acc[GROUP];
#pragma unroll
    for (int h = 0; h < GROUP; h++) {
        m_run[h] = -INFINITY;
        L[h] = 0.f;
        acc[h] = 0.f;
    }
    const int d = tid % HD, kg = tid / HD;
    fetch(c0);   // the first chunks' loads go out before the q|k|v rows are finished
    batch_qkv_rows<KVT, HD, GROUP>(partial, ranges, a, kc, vc, kv_seq_stride, kvdim, b, g, P, last, rowq);
    float qr[GROUP][EPC];
#pragma unroll
    for (int h = 0; h < GROUP; h++)
#pragma unroll
        for (int e = 0; e < EPC; e++) qr[h][e] = rowq[h * HD + sl * EPC + e];
    stash(0, c0 == nchunks - 1);
    fetch(c0 + 1);   // in flight while chunk c0 is consumed
    __syncthreads();
    for (int ci = c0; ci < c1; ci++) {
        const int buf = (ci - c0) & 1;
        const int n = min(C, P - ci * C);
        // scores and each wave's maximum
        float mx[GROUP];
#pragma unroll
        for (int h = 0; h < GROUP; h++) mx[h] = -INFINITY;
#pragma unroll
        for (int j = 0; j < SB; j++) {
            const int t = (wave + j * NW) * PPW + rin;
            const u32x4 k4 = ((const u32x4 *)(kbuf[buf] + (size_t)t * RB))[sl];
            float kf[EPC];
            if constexpr (KVT == SH_KV_F32) {
#pragma unroll
                for (int e = 0; e < 4; e++) kf[e] = __uint_as_float(k4[e]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int dtk = KVT == SH_KV_BF16 ? SH_DTYPE_BF16 : SH_DTYPE_F16;
                    kf[2 * e] = bits_to_f(k4[e] & 0xffffu, dtk);
                    kf[2 * e + 1] = bits_to_f(k4[e] >> 16, dtk);
                }
            }
#pragma unroll
            for (int h = 0; h < GROUP; h++) {
                float dd = 0.f;
#pragma unroll
                for (int e = 0; e < EPC; e++) dd = fmaf(qr[h][e], kf[e], dd);
                dd = wsum<LPK>(dd) * scale;
                if (t < n) {
                    if (sl == 0) sc[h][t] = dd;
                    mx[h] = fmaxf(mx[h], dd);
                }
            }
        }
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            const float m = wmax<64>(mx[h]);
            if (lane == 0) redm[wave][h] = m;
        }
        __asm__ __volatile__("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        float mnew[GROUP], alpha[GROUP], ls[GROUP];
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            float m = m_run[h];
#pragma unroll
            for (int w = 0; w < NW; w++) m = fmaxf(m, redm[w][h]);
            alpha[h] = expf(m_run[h] - m);   // 0 before the first chunk
            mnew[h] = m;
            ls[h] = 0.f;
        }
        // exp terms (zero past the chunk's keys, so P.V reads whole chunks)
        for (int i = tid; i < GROUP * C; i += kAT) {
            const int h = i / C, t = i % C;
#pragma unroll
            for (int hh = 0; hh < GROUP; hh++) {
                if (hh != h) continue;
                const float p = t < n ? expf(sc[hh][t] - mnew[hh]) : 0.f;
                sc[hh][t] = p;
                ls[hh] += p;
            }
        }
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            const float s = wsum<64>(ls[h]);
            if (lane == 0) redl[wave][h] = s;
        }
        __asm__ __volatile__("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < NW; w++) s += redl[w][h];
            L[h] = L[h] * alpha[h] + s;
            m_run[h] = mnew[h];
            acc[h] *= alpha[h];
        }
        // P.V: keys kg, kg + NKG, ... of the chunk, four per batch
#pragma unroll
        for (int j = 0; j < C / NKG; j += 4) {
            float vv[4], pw[GROUP][4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int t = kg + (j + u) * NKG;
                vv[u] = kv_elem<KVT>(vbuf[buf] + (size_t)t * RB, d);
#pragma unroll
                for (int h = 0; h < GROUP; h++) pw[h][u] = sc[h][t];
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int h = 0; h < GROUP; h++) acc[h] = fmaf(pw[h][u], vv[u], acc[h]);
        }
        // chunk ci+1 into the other buffers (read last in chunk ci-1, before the previous
        // barrier), and chunk ci+2 into the registers; after the barrier every wave is done
        // with this chunk's buffers and sc. (Issued here, unconditionally, rather than at the
        // top of the loop under a branch: 2.89 -> 2.76 ms per 32-sequence Qwen3-shaped step.
        // Deeper register rings of 2-6 chunks at one workgroup per CU were slower.)
        if (ci + 1 < c1) stash(buf ^ 1, ci + 1 == nchunks - 1);
        fetch(ci + 2);
        __syncthreads();
    }
#pragma unroll
    for (int h = 0; h < GROUP; h++) part[kg][h][d] = acc[h];
    __asm__ __volatile__("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    for (int i = tid; i < GROUP * HD; i += kAT) {
        const int h = i / HD, dd = i % HD;
        float o = 0.f;
#pragma unroll
        for (int r = 0; r < NKG; r++) o += part[r][h][dd];
        float lh = 0.f, mh = 0.f;
#pragma unroll
        for (int hh = 0; hh < GROUP; hh++)
            if (hh == h) {
                lh = L[hh];
                mh = m_run[hh];
            }
        if (nsplit == 1) {
            store_op16(att, (size_t)b * qdim + (size_t)(g * GROUP + h) * HD + dd, plane, o / lh, dt);
        } else {
            const size_t pb = ((size_t)b * H + (size_t)g * GROUP + h) * nch_buf + split;
            tag_put(tacc + pb * HD + dd, o, tag);
            if (dd == 0) {
                tag_put(tm + pb, mh, tag);
                tag_put(tl_ + pb, lh, tag);
            }
        }
    }
    if (nsplit == 1) return;
    // The last of the sequence's key-holding splits to count in merges them, in the float
    // order sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s (splits in order),
    // reading the others' tagged partials, and clears the counter for the next layer.
    __shared__ int merge_s;
    __syncthreads();
    const int ns = (nchunks + cps - 1) / cps;
    int *ctr = cnt + (size_t)b * KVH + g;
    if (tid == 0) merge_s = atomicAdd(ctr, 1) == ns - 1;
    __syncthreads();
    if (!merge_s) return;
    if (tid == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int i = tid; i < GROUP * HD; i += kAT) {
        const int h = g * GROUP + i / HD, ii = i % HD;
        const size_t pb = ((size_t)b * H + h) * nch_buf;
        float M = -INFINITY;
        for (int c = 0; c < ns; c++) M = fmaxf(M, tag_get(tm + pb + c, tag, err));
        float Lsum = 0.f;
        for (int c = 0; c < ns; c++)
            Lsum += expf(tag_get(tm + pb + c, tag, err) - M) * tag_get(tl_ + pb + c, tag, err);
        const float invL = 1.0f / Lsum;
        float a = 0.f;
        for (int c = 0; c < ns; c++)
            a += expf(tag_get(tm + pb + c, tag, err) - M) * tag_get(tacc + (pb + c) * HD + ii, tag, err);
        store_op16(att, (size_t)b * qdim + (size_t)h * HD + ii, plane, a * invL, dt);
    }
}

// Batched decode attention with one online softmax per lane group and no barrier inside the
// key loop (head dims 64 and 128). Workgroup (split, kv head g, sequence b) takes the same
// split of the sequence's keys as k_attn_batch_stream, finishes its q|k|v rows the same way
// (batch_qkv_rows), and then each wave walks its own rows of the split: per iteration RWI
// = SBW * PPW rows, row r of a row block on LPK lanes (each lane one 16-byte slice of the K
// and V rows, loaded straight into registers one iteration ahead, no LDS staging). The lanes
// of a row finish its score (slice dot products added by DPP), fold it into their running
// (max, sum, P.V slice) for every q head of the group, in the base-2 domain (the score scaled
// by log2 e, so each term is one exp2), and the row's V slice is already in the same lanes.
// After the loop the row groups of a wave merge by lane swaps, the waves through LDS, and
// the splits as in k_attn_batch_stream (tagged partials, merged by the last split). Row pos[b]
// is taken from rowq (the cache row's load may predate the prologue's write).
template <int KVT, int HD, int GROUP, int SBW, int NSET>
__global__ __launch_bounds__(kAWT) void k_attn_batch_wave(
    const float *partial, int ranges, QkRopeArgs a, const void *kc, const void *vc, size_t kv_seq_stride,
    const int32_t *pos, int H, int KVH, float scale, int nsplit, int nch_buf, int dt, size_t plane,
    uint16_t *att, uint64_t *tm, uint64_t *tl_, uint64_t *tacc, int *cnt, const uint32_t *gen, int layer,
    int n_layers, int max_seq, int *err) {
    constexpr int EB = KVT == SH_KV_F32 ? 4 : 2;
    constexpr int RB = HD * EB;                        // bytes per cache row
    constexpr int C = kChunkBytes / RB;                // keys per split unit (as the stream kernel)
    constexpr int LPK = RB / 16, EPC = 16 / EB, PPW = 64 / LPK;
    constexpr int NW = kAWT / 64;
    constexpr int RWI = SBW * PPW, RI = NW * RWI;      // rows per wave / per workgroup per iteration
    static_assert(HD == 64 || HD == 128, "head dims of the lane-group form");
    __shared__ float rowq[(GROUP + 2) * HD];           // the group's q heads, then k, then v
    __shared__ float wm[NW][GROUP], wl[NW][GROUP];
    __shared__ __attribute__((aligned(16))) float wacc[NW][GROUP][HD];
    const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int P = pos[b] + 1;
    const int nchunks = (P + C - 1) / C;
    const int cps = (nchunks + nsplit - 1) / nsplit;
    const int c0 = split * cps, c1 = min(nchunks, c0 + cps);
    if (c0 >= c1) return;
    const int k0 = c0 * C, k1 = min(c1 * C, P);       // this split's keys
    const int qdim = H * HD, kvdim = KVH * HD;
    const uint32_t tag = ((*gen * (uint32_t)(max_seq + 1) + (uint32_t)(P - 1)) * (uint32_t)n_layers +
                          (uint32_t)layer) + 1u;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t sbase = (size_t)b * kv_seq_stride + (size_t)g * HD;
    const int sl = lane % LPK, rin = lane / LPK;
    const bool last = c1 == nchunks;
    const int nit = (k1 - k0 + RI - 1) / RI;
    // K and V slices of iteration it's rows (rows past the split's last key re-read it, so
    // every load is in bounds and none sits under a branch)
    auto fetch = [&](int it, u32x4 (&kr)[SBW], u32x4 (&vr)[SBW]) {
#pragma unroll
        for (int j = 0; j < SBW; j++) {
            const int t = min(k0 + it * RI + wave * RWI + j * PPW + rin, k1 - 1);
            const size_t o = (sbase + (size_t)t * kvdim) * EB + (size_t)sl * 16;
            kr[j] = *(const u32x4 *)((const uint8_t *)kc + o);
            vr[j] = *(const u32x4 *)((const uint8_t *)vc + o);
        }
    };
    // NSET register sets in a ring, each loaded NSET - 1 iterations ahead of its use
    u32x4 kr[NSET][SBW], vr[NSET][SBW];
#pragma unroll
    for (int u = 0; u + 1 < NSET; u++) fetch(u, kr[u], vr[u]);   // out before the q|k|v rows are finished
    batch_qkv_rows<KVT, HD, GROUP, kAWT>(partial, ranges, a, kc, vc, kv_seq_stride, kvdim, b, g, P, last, rowq);
    float qr[GROUP][EPC];
#pragma unroll
    for (int h = 0; h < GROUP; h++)
#pragma unroll
        for (int e = 0; e < EPC; e++) qr[h][e] = rowq[h * HD + sl * EPC + e];
    const float scale2 = scale * 1.4426950408889634f;
    // running state of this lane's row group: base-2 max (finite floor, so a group whose rows
    // are all masked so far rescales by 1), sum of terms, P.V over the lane's EPC dims
    float m[GROUP], l[GROUP], acc[GROUP][EPC];
#pragma unroll
    for (int h = 0; h < GROUP; h++) {
        m[h] = -1e30f;
        l[h] = 0.f;
#pragma unroll
        for (int e = 0; e < EPC; e++) acc[h][e] = 0.f;
    }
    auto unpack = [&](const u32x4 &r, float (&f)[EPC]) {
        if constexpr (KVT == SH_KV_F32) {
#pragma unroll
            for (int e = 0; e < 4; e++) f[e] = __uint_as_float(r[e]);
        } else {
            const int dtk = KVT == SH_KV_BF16 ? SH_DTYPE_BF16 : SH_DTYPE_F16;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                f[2 * e] = bits_to_f(r[e] & 0xffffu, dtk);
                f[2 * e + 1] = bits_to_f(r[e] >> 16, dtk);
            }
        }
    };
    auto compute = [&](int it, const u32x4 (&kr)[SBW], const u32x4 (&vr)[SBW]) {
        float sc[SBW][GROUP], vf[SBW][EPC];
        const bool tail = last && it == nit - 1;   // holds row P - 1
#pragma unroll
        for (int j = 0; j < SBW; j++) {
            const int t = k0 + it * RI + wave * RWI + j * PPW + rin;
            float kf[EPC];
            unpack(kr[j], kf);
            unpack(vr[j], vf[j]);
            if (__builtin_expect(tail, 0) && t == P - 1) {
#pragma unroll
                for (int e = 0; e < EPC; e++) {
                    kf[e] = rowq[GROUP * HD + sl * EPC + e];
                    vf[j][e] = rowq[(GROUP + 1) * HD + sl * EPC + e];
                }
            }
#pragma unroll
            for (int h = 0; h < GROUP; h++) {
                float d0 = 0.f, d1 = 0.f;
#pragma unroll
                for (int e = 0; e < EPC; e += 2) {
                    d0 = fmaf(qr[h][e], kf[e], d0);
                    d1 = fmaf(qr[h][e + 1], kf[e + 1], d1);
                }
                const float dd = wsum<LPK>(d0 + d1) * scale2;
                sc[j][h] = t < k1 ? dd : -INFINITY;
            }
        }
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            float mn = m[h];
#pragma unroll
            for (int j = 0; j < SBW; j++) mn = fmaxf(mn, sc[j][h]);
            const float f = __builtin_amdgcn_exp2f(m[h] - mn);
            m[h] = mn;
            float pw[SBW];
            float ls = l[h] * f;
#pragma unroll
            for (int j = 0; j < SBW; j++) {
                pw[j] = __builtin_amdgcn_exp2f(sc[j][h] - mn);
                ls += pw[j];
            }
            l[h] = ls;
#pragma unroll
            for (int e = 0; e < EPC; e++) {
                float o = acc[h][e] * f;
#pragma unroll
                for (int j = 0; j < SBW; j++) o = fmaf(pw[j], vf[j][e], o);
                acc[h][e] = o;
            }
        }
    };
    // unrolled by NSET, so no set is copied while its loads are in flight
    for (int it = 0; it < nit; it += NSET) {
#pragma unroll
        for (int u = 0; u < NSET; u++) {
            fetch(it + u + NSET - 1, kr[(u + NSET - 1) % NSET], vr[(u + NSET - 1) % NSET]);
            if (u == 0 || it + u < nit) compute(it + u, kr[u], vr[u]);
        }
    }
    // the PPW row groups of the wave (lanes sl + LPK * r) merged by lane swaps; every lane of
    // a slice ends with the same values
#pragma unroll
    for (int x = LPK; x < 64; x <<= 1) {
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            const float mo = __shfl_xor(m[h], x, 64), lo = __shfl_xor(l[h], x, 64);
            const float mn = fmaxf(m[h], mo);
            const float fa = __builtin_amdgcn_exp2f(m[h] - mn), fb = __builtin_amdgcn_exp2f(mo - mn);
            l[h] = l[h] * fa + lo * fb;
#pragma unroll
            for (int e = 0; e < EPC; e++) {
                const float ao = __shfl_xor(acc[h][e], x, 64);
                acc[h][e] = acc[h][e] * fa + ao * fb;
            }
            m[h] = mn;
        }
    }
    if (rin == 0) {
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
#pragma unroll
            for (int e = 0; e < EPC; e++) wacc[wave][h][sl * EPC + e] = acc[h][e];
            if (sl == 0) {
                wm[wave][h] = m[h];
                wl[wave][h] = l[h];
            }
        }
    }
    __syncthreads();
    for (int i = tid; i < GROUP * HD; i += kAWT) {
        const int h = i / HD, dd = i % HD;
        float M = -1e30f;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, wm[w][h]);
        float o = 0.f, lh = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float f = __builtin_amdgcn_exp2f(wm[w][h] - M);
            lh += wl[w][h] * f;
            o += wacc[w][h][dd] * f;
        }
        if (nsplit == 1) {
            store_op16(att, (size_t)b * qdim + (size_t)(g * GROUP + h) * HD + dd, plane, o / lh, dt);
        } else {
            const size_t pb = ((size_t)b * H + (size_t)g * GROUP + h) * nch_buf + split;
            tag_put(tacc + pb * HD + dd, o, tag);
            if (dd == 0) {
                tag_put(tm + pb, M, tag);
                tag_put(tl_ + pb, lh, tag);
            }
        }
    }
    if (nsplit == 1) return;
    // the last of the sequence's key-holding splits to count in merges them (base-2 maxima),
    // splits in order, and clears the counter for the next layer
    __shared__ int merge_s;
    __syncthreads();
    const int ns = (nchunks + cps - 1) / cps;
    int *ctr = cnt + (size_t)b * KVH + g;
    if (tid == 0) merge_s = atomicAdd(ctr, 1) == ns - 1;
    __syncthreads();
    if (!merge_s) return;
    if (tid == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // the splits' words requested four splits at a time (a word without the tag is polled
    // by tag_get), folded in split order
    for (int i = tid; i < GROUP * HD; i += kAWT) {
        const int h = g * GROUP + i / HD, ii = i % HD;
        const size_t pb = ((size_t)b * H + h) * nch_buf;
        float M = -INFINITY, Lsum = 0.f, acc_s = 0.f;
        for (int c0 = 0; c0 < ns; c0 += 4) {
            uint64_t w[4][3];
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (c0 + u < ns) {
                    w[u][0] = __hip_atomic_load(tm + pb + c0 + u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    w[u][1] = __hip_atomic_load(tl_ + pb + c0 + u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    w[u][2] = __hip_atomic_load(tacc + (pb + c0 + u) * HD + ii, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (c0 + u < ns) {
                    const size_t c = pb + c0 + u;
                    const float mc = (uint32_t)(w[u][0] >> 32) == tag ? __uint_as_float((uint32_t)w[u][0])
                                                                      : tag_get(tm + c, tag, err);
                    const float lc = (uint32_t)(w[u][1] >> 32) == tag ? __uint_as_float((uint32_t)w[u][1])
                                                                      : tag_get(tl_ + c, tag, err);
                    const float ac = (uint32_t)(w[u][2] >> 32) == tag ? __uint_as_float((uint32_t)w[u][2])
                                                                      : tag_get(tacc + c * HD + ii, tag, err);
                    const float mn = fmaxf(M, mc);
                    const float f = exp2f(M - mn), fc = exp2f(mc - mn);
                    Lsum = Lsum * f + lc * fc;
                    acc_s = acc_s * f + ac * fc;
                    M = mn;
                }
        }
        store_op16(att, (size_t)b * qdim + (size_t)h * HD + ii, plane, acc_s / Lsum, dt);
    }
}

// The streaming kernel for (kv type, head dim, group), or null when it has no instance.
typedef void (*AttnStreamKernel)(const float *, int, QkRopeArgs, const void *, const void *, size_t,
                                 const int32_t *, int, int, float, int, int, int, size_t, uint16_t *, uint64_t *,
                                 uint64_t *, uint64_t *, int *, const uint32_t *, int, int, int, int *);
template <int KVT>
AttnStreamKernel pick_attn_stream_kv(int hd, int group) {
    switch (hd * 8 + group) {
    case 32 * 8 + 1: return &k_attn_batch_stream<KVT, 32, 1>;
    case 32 * 8 + 2: return &k_attn_batch_stream<KVT, 32, 2>;
    case 32 * 8 + 4: return &k_attn_batch_stream<KVT, 32, 4>;
    case 64 * 8 + 1: return &k_attn_batch_wave<KVT, 64, 1, 2, 3>;
    case 64 * 8 + 2: return &k_attn_batch_wave<KVT, 64, 2, 2, 3>;
    case 64 * 8 + 4: return &k_attn_batch_stream<KVT, 64, 4>;
    case 128 * 8 + 1: return &k_attn_batch_wave<KVT, 128, 1, 2, 3>;
    case 128 * 8 + 2: return &k_attn_batch_wave<KVT, 128, 2, 2, 3>;
    default: return nullptr;
    }
}
// Threads of the streaming kernel pick_attn_stream returns (the lane-group form for 64- and
// 128-dim heads with one or two q heads per kv head; with four its registers would spill).
int attn_stream_threads(int hd, int group) { return (hd == 64 || hd == 128) && group <= 2 ? kAWT : kAT; }
AttnStreamKernel pick_attn_stream(int kv, int hd, int group) {
    if (kv == SH_KV_F32) return pick_attn_stream_kv<SH_KV_F32>(hd, group);
    if (kv == SH_KV_F16) return pick_attn_stream_kv<SH_KV_F16>(hd, group);
    return pick_attn_stream_kv<SH_KV_BF16>(hd, group);
}

// Merges the chunk partials of (q head h, sequence b): out = sum_c e^(m_c - M) acc_c /
// sum_c e^(m_c - M) l_c, written as a GEMM operand row.
__global__ __launch_bounds__(256) void k_attn_batch_combine(const float *pm, const float *pl,
                                                            const float *pacc, const int32_t *pos,
                                                            int H, int hd, int nch, int chunk,
                                                            int B, int dt, uint16_t *att) {
    const int h = blockIdx.x, b = blockIdx.y;
    const int nc = (pos[b] + chunk) / chunk;   // chunks holding keys 0..pos
    const size_t pb = ((size_t)b * H + h) * nch;
    float M = -INFINITY;
    for (int c = 0; c < nc; c++) M = fmaxf(M, pm[pb + c]);
    float L = 0.f;
    for (int c = 0; c < nc; c++) L += expf(pm[pb + c] - M) * pl[pb + c];
    const float invL = 1.0f / L;
    const size_t plane = (size_t)B * H * hd;
    for (int i = threadIdx.x; i < hd; i += blockDim.x) {
        float a = 0.f;
        for (int c = 0; c < nc; c++) a += expf(pm[pb + c] - M) * pacc[(pb + c) * hd + i];
        store_op16(att, (size_t)b * H * hd + (size_t)h * hd + i, plane, a * invL, dt);
    }
}

constexpr int kArgChunk = 4096;   // logits per workgroup of the first argmax pass

// First pass of the row argmax (infer.go:373-383, first maximum) of logits [B, V]: workgroup
// (blk, b) scans logits [blk*4096, (blk+1)*4096) of row b, 16 consecutive values per thread
// read as four float4, and writes its (max, first index). Needs V % 4 == 0.
__global__ __launch_bounds__(kT) void k_argmax_part(const float *logits, int V, int nblk,
                                                    float *pv, int32_t *pi) {
    __shared__ float bv[kT / 64];
    __shared__ int bi[kT / 64];
    const int blk = blockIdx.x, b = blockIdx.y;
    const float *row = logits + (size_t)b * V;
    const int i0 = blk * kArgChunk + threadIdx.x * 16;
    f32x4 x[4];
#pragma unroll
    for (int u = 0; u < 4; u++)
        x[u] = i0 + 4 * u < V ? *(const f32x4 *)(row + i0 + 4 * u)
                              : f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    float v = -INFINITY;
    int idx = 0x7fffffff;
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (x[u][e] > v) {   // ascending indices: strict > keeps the first maximum
                v = x[u][e];
                idx = i0 + 4 * u + e;
            }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        if (ov > v || (ov == v && oi < idx)) {
            v = ov;
            idx = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        bv[threadIdx.x >> 6] = v;
        bi[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        v = bv[0];
        idx = bi[0];
        for (int w = 1; w < kT / 64; w++)
            if (bv[w] > v || (bv[w] == v && bi[w] < idx)) {
                v = bv[w];
                idx = bi[w];
            }
        pv[(size_t)b * nblk + blk] = v;
        pi[(size_t)b * nblk + blk] = idx;
    }
}

// Second pass: one wave per row reduces the partials, then the sequence advances:
// hist[b][pos+1] = next, tok[b] = next, pos[b] += 1.
__global__ __launch_bounds__(64) void k_argmax_advance(const float *pv, const int32_t *pi,
                                                       int nblk, int32_t *tok, int32_t *pos,
                                                       int32_t *hist, int hist_stride) {
    const int b = blockIdx.x, lane = threadIdx.x;
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int k = lane; k < nblk; k += 64) {
        const float cv = pv[(size_t)b * nblk + k];
        const int ci = pi[(size_t)b * nblk + k];
        if (cv > v || (cv == v && ci < idx)) {
            v = cv;
            idx = ci;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        if (ov > v || (ov == v && oi < idx)) {
            v = ov;
            idx = oi;
        }
    }
    if (lane == 0) {
        const int next = idx == 0x7fffffff ? 0 : idx;
        const int p = pos[b];
        hist[(size_t)b * hist_stride + p + 1] = next;
        tok[b] = next;
        pos[b] = p + 1;
    }
}

// Window decode step tail (decode.go:55-70): reduce the argmax partials of the last
// column's logits, record the token (hist[*count]), shift the window left by one and append
// it (fillDecodeWindow of the grown token list, :83-94).
__global__ __launch_bounds__(kT) void k_window_advance(const float *pv, const int32_t *pi, int nblk,
                                                       int32_t *window, int seq, int32_t *hist,
                                                       int32_t *count) {
    __shared__ int next_s;
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        float v = -INFINITY;
        int idx = 0x7fffffff;
        for (int k = lane; k < nblk; k += 64)
            if (pv[k] > v || (pv[k] == v && pi[k] < idx)) {
                v = pv[k];
                idx = pi[k];
            }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(v, off, 64);
            const int oi = __shfl_xor(idx, off, 64);
            if (ov > v || (ov == v && oi < idx)) {
                v = ov;
                idx = oi;
            }
        }
        if (lane == 0) {
            next_s = idx == 0x7fffffff ? 0 : idx;
            const int c = *count;
            hist[c] = next_s;
            *count = c + 1;
        }
    }
    __syncthreads();
    // the shift reads window[i + 1] before any thread overwrites it: stage in registers
    // (seq <= 4096, so at most 16 values per thread)
    int vals[16];
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const int i = threadIdx.x + k * kT;
        if (i < seq - 1) vals[k] = window[i + 1];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const int i = threadIdx.x + k * kT;
        if (i < seq - 1) window[i] = vals[k];
    }
    if (threadIdx.x == 0) window[seq - 1] = next_s;
}

// Kernel, tile shape and K split of a 16-bit GEMM.
//  - Short inputs (M < 1024, not the classifier's very wide output): k_gemm_pipe, 64 x 64
//    tiles when they alone give every CU a workgroup (W1|W3 at S = 256: 256 tiles, 8.6 us
//    against 17.7 for the split 64 x 64 burst GEMM and its reduce), else 32 x 32 tiles with
//    K split in two or four until there are about 384 workgroups (qkv 7.6 us unsplit, Wo
//    3.9 and W2 6.2 in two ranges, against 14.9, 10.4 and 13.4 for the burst GEMM and its
//    row kernel's partial sums).
//  - Long inputs and very wide outputs (the classifier: half the re-reads of the activation
//    planes; 48 vs 57 us at S = 256, N = 32000): k_gemm_burst 128 x 128 tiles; shapes the
//    pipeline cannot take: 64 x 64 k_gemm_burst / k_gemm_tiled with K split (ranges of >= 256,
//    dividing K) until there are about 512 workgroups.
enum { GK_TILED64 = 0, GK_BIG = 1, GK_PIPE64 = 2, GK_PIPE32 = 3 };
struct GemmPlan {
    int kind, ranges, kc;
};
GemmPlan gemm_plan(int M, int N, int K) {
    GemmPlan p{};
    p.ranges = 1;
    p.kc = K;
    const bool big = (M >= 1024 || (M >= 256 && N >= 16384)) && N % 128 == 0;
    if (!big && K % 64 == 0) {
        const int t64 = ((M + 63) / 64) * (N / 64);
        if (N % 64 == 0 && t64 >= 256 && K / 64 >= 5) {
            p.kind = GK_PIPE64;
            return p;
        }
        if (N % 32 == 0 && K / 64 >= 3) {
            const int t32 = ((M + 31) / 32) * (N / 32);
            p.kind = GK_PIPE32;
            for (int r : {2, 4}) {
                if (t32 * p.ranges >= 384) break;
                if (K % (64 * r) == 0 && K / (64 * r) >= 3) p.ranges = r;
            }
            p.kc = K / p.ranges;
            return p;
        }
    }
    p.kind = big ? GK_BIG : GK_TILED64;
    const int tiles = big ? ((M + 127) / 128) * (N / 128) : ((M + 63) / 64) * (N / 64);
    // at most four K ranges: each more range adds a [M, N] fp32 partial for the row kernel
    // that sums them to read back
    for (int r : {2, 3, 4})
        if (K % (32 * r) == 0 && K / r >= 256 && tiles * r <= 768) p.ranges = r;
    if (tiles >= 512) p.ranges = 1;
    p.kc = K / p.ranges;
    return p;
}

// Lets the pipelined GEMMs use more than 64 KB of dynamic LDS (once per process, before any
// capture: called where models and convolutions are created).
hipError_t gemm_pipe_setup_once() {
    static hipError_t st = [] {
        const void *fns[] = {(const void *)k_gemm_pipe<SH_DTYPE_F16, 64, 64, 64, 6>,
                             (const void *)k_gemm_pipe<SH_DTYPE_BF16, 64, 64, 64, 6>,
                             (const void *)k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_F32>,
                             (const void *)k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_F16>,
                             (const void *)k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_BF16>,
                             (const void *)k_gemm_pipe_qkv64<SH_DTYPE_BF16, SH_KV_F32>,
                             (const void *)k_gemm_pipe_qkv64<SH_DTYPE_BF16, SH_KV_F16>,
                             (const void *)k_gemm_pipe_qkv64<SH_DTYPE_BF16, SH_KV_BF16>,
                             (const void *)k_gemm_pipe<SH_DTYPE_F16, 64, 64, 64, 6, 1>,
                             (const void *)k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_F32, 1>,
                             (const void *)k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_F16, 1>,
                             (const void *)k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_BF16, 1>};
        for (const void *f : fns) {
            const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kPipeBigLds);
            if (e != hipSuccess) return e;
        }
        for (const void *f : {(const void *)k_gemm_pipe<SH_DTYPE_F16, 32, 64, 64, 4>,
                              (const void *)k_gemm_pipe<SH_DTYPE_BF16, 32, 64, 64, 4>}) {
            const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kPipeWideLds);
            if (e != hipSuccess) return e;
        }
        const struct {
            const void *f;
            int bytes;
        } qkv32[] = {{(const void *)k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_F32, 1, 32>, qkv64_lds<32, 1>()},
                     {(const void *)k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_F16, 1, 32>, qkv64_lds<32, 1>()},
                     {(const void *)k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_BF16, 1, 32>, qkv64_lds<32, 1>()},
                     {(const void *)k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_F32, 2, 32>, qkv64_lds<32, 2>()},
                     {(const void *)k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_F16, 2, 32>, qkv64_lds<32, 2>()},
                     {(const void *)k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_BF16, 2, 32>, qkv64_lds<32, 2>()},
                     {(const void *)k_gemm_pipe_qkv64<SH_DTYPE_BF16, SH_KV_F32, 2, 32>, qkv64_lds<32, 2>()},
                     {(const void *)k_gemm_pipe_qkv64<SH_DTYPE_BF16, SH_KV_F16, 2, 32>, qkv64_lds<32, 2>()},
                     {(const void *)k_gemm_pipe_qkv64<SH_DTYPE_BF16, SH_KV_BF16, 2, 32>, qkv64_lds<32, 2>()}};
        for (const auto &q : qkv32) {
            const hipError_t e = hipFuncSetAttribute(q.f, hipFuncAttributeMaxDynamicSharedMemorySize, q.bytes);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }();
    return st;
}

// ranges_out given: K-range partials are left for the caller's row kernel (*ranges_out > 1)
// instead of being summed here; with one range the epilogue runs as usual.
// W8A8 projection: the fp32 A rows quantized one by one, then the int8 product and its epilogue.
hipError_t gemm_i8(const GemmArgs &g, hipStream_t s) {
    if (g.K % 128 || g.N % 64 || g.M < 1 || !g.a8 || !g.sa || !g.sw) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_quant_rows_i8, dim3(g.M), dim3(kT), 0, s, (const float *)g.A, g.K, g.a8, g.sa);
    const dim3 grid((g.M + 63) / 64, g.N / 64);
    if ((g.K / 64) % 4 == 0) hipLaunchKernelGGL((k_gemm_i8<64, 64, 4>), grid, dim3(kT), 0, s, g);
    else hipLaunchKernelGGL((k_gemm_i8<64, 64, 2>), grid, dim3(kT), 0, s, g);
    return hipGetLastError();
}

hipError_t gemm(const GemmArgs &g, int dt, float *partial, size_t part_cap, hipStream_t s,
                int *ranges_out = nullptr) {
    if (dt == SH_DTYPE_W8A8) {   // one K range: the epilogue runs in the product
        if (ranges_out) *ranges_out = 1;
        return gemm_i8(g, s);
    }
    if (g.K % 32 || g.N % 64) return hipErrorInvalidValue;
    const GemmPlan p = gemm_plan(g.M, g.N, g.K);
    if (p.ranges > 1 && (!partial || (size_t)p.ranges * g.M * g.N > part_cap))
        return hipErrorInvalidValue;   // the partial buffer must hold every K range
    const bool bf = dt == SH_DTYPE_BF16;
    if (p.kind == GK_PIPE64 || p.kind == GK_PIPE32) {
        hipError_t e0 = gemm_pipe_setup_once();
        if (e0 != hipSuccess) return e0;
        const bool one = g.one_plane && !bf;
        if (p.kind == GK_PIPE64) {
            const dim3 grid((g.M + 63) / 64, g.N / 64, p.ranges);
            if (bf) hipLaunchKernelGGL((k_gemm_pipe<SH_DTYPE_BF16, 64, 64, 64, 6>), grid, dim3(kT), kPipeBigLds, s, g, partial, p.kc);
            else if (one) hipLaunchKernelGGL((k_gemm_pipe<SH_DTYPE_F16, 64, 64, 64, 6, 1>), grid, dim3(kT), kPipeBigLds, s, g, partial, p.kc);
            else hipLaunchKernelGGL((k_gemm_pipe<SH_DTYPE_F16, 64, 64, 64, 6>), grid, dim3(kT), kPipeBigLds, s, g, partial, p.kc);
        } else {
            const dim3 grid((g.M + 31) / 32, g.N / 32, p.ranges);
            if (bf) hipLaunchKernelGGL((k_gemm_pipe<SH_DTYPE_BF16, 32, 32, 64, 4>), grid, dim3(kT), kPipeSmallLds, s, g, partial, p.kc);
            else if (one) hipLaunchKernelGGL((k_gemm_pipe<SH_DTYPE_F16, 32, 32, 64, 4, 1>), grid, dim3(kT), kPipeSmallLds, s, g, partial, p.kc);
            else hipLaunchKernelGGL((k_gemm_pipe<SH_DTYPE_F16, 32, 32, 64, 4>), grid, dim3(kT), kPipeSmallLds, s, g, partial, p.kc);
        }
    } else if (p.kind == GK_BIG) {
        // burst loads where the K range allows them (4 steps of 32 per burst for 128 x 128
        // tiles, 8 for 64 x 64, whose staging registers are half as many per step)
        const dim3 grid((g.M + 127) / 128, g.N / 128, p.ranges);
        if (p.kc % 128 == 0) {
            if (bf) hipLaunchKernelGGL((k_gemm_burst<SH_DTYPE_BF16, 128, 128, 4>), grid, dim3(kT), 0, s, g, partial, p.kc);
            else if (g.one_plane) hipLaunchKernelGGL((k_gemm_burst<SH_DTYPE_F16, 128, 128, 4, 1>), grid, dim3(kT), 0, s, g, partial, p.kc);
            else hipLaunchKernelGGL((k_gemm_burst<SH_DTYPE_F16, 128, 128, 4>), grid, dim3(kT), 0, s, g, partial, p.kc);
        } else {
            if (bf) hipLaunchKernelGGL((k_gemm_tiled<SH_DTYPE_BF16, 128, 128>), grid, dim3(kT), 0, s, g, partial, p.kc);
            else hipLaunchKernelGGL((k_gemm_tiled<SH_DTYPE_F16, 128, 128>), grid, dim3(kT), 0, s, g, partial, p.kc);
        }
    } else {
        const dim3 grid((g.M + 63) / 64, g.N / 64, p.ranges);
        if (p.kc % 256 == 0) {
            if (bf) hipLaunchKernelGGL((k_gemm_burst<SH_DTYPE_BF16, 64, 64, 8>), grid, dim3(kT), 0, s, g, partial, p.kc);
            else hipLaunchKernelGGL((k_gemm_burst<SH_DTYPE_F16, 64, 64, 8>), grid, dim3(kT), 0, s, g, partial, p.kc);
        } else {
            if (bf) hipLaunchKernelGGL((k_gemm_tiled<SH_DTYPE_BF16, 64, 64>), grid, dim3(kT), 0, s, g, partial, p.kc);
            else hipLaunchKernelGGL((k_gemm_tiled<SH_DTYPE_F16, 64, 64>), grid, dim3(kT), 0, s, g, partial, p.kc);
        }
    }
    hipError_t e = hipGetLastError();
    if (ranges_out) *ranges_out = p.ranges;
    if (e != hipSuccess || p.ranges == 1 || ranges_out) return e;
    const int pairs = g.M * (g.N / 2);
    hipLaunchKernelGGL(k_gemm_skinny_reduce, dim3((pairs + kT - 1) / kT), dim3(kT), 0, s, g,
                       (const float *)partial, p.ranges);
    return hipGetLastError();
}

}  // namespace

hipError_t gemm_setup() { return gemm_pipe_setup_once(); }

bool prefill_supported(const sh_model *m, std::string *why) {
    const sh_config &c = m->cfg;
    if (m->dtype == SH_DTYPE_W8A8 && (c.dim % 128 || m->qdim % 128 || c.hidden % 128)) {
        *why = "W8A8 full-sequence forward needs dim, n_heads*head_dim and hidden multiples of 128";
        return false;
    }
    if (c.dim % 64 || m->qdim % 64 || c.hidden % 64 || c.vocab % 64 || m->qkv_rows % 64 ||
        (2 * c.hidden) % 64) {
        *why = "full-sequence forward needs dims that are multiples of 64";
        return false;
    }
    if (m->qkv_rows > 4096 || c.dim > 4096) {
        *why = "q/k/v width or dim above 4096";
        return false;
    }
    return true;
}

// K-range partial elements the split GEMMs of an S-row forward need. A shorter input has
// fewer tiles and so may split K further: the need is not monotonic in S.
static size_t prefill_part_need(const sh_model *m, int S) {
    const sh_config &c = m->cfg;
    const size_t D = c.dim, F = c.hidden, Q = m->qdim, R = m->qkv_rows, V = c.vocab;
    size_t part = 1;
    for (auto nk : {std::make_pair(R, D), std::make_pair(D, Q), std::make_pair(2 * F, D),
                    std::make_pair(D, F), std::make_pair(V, D)}) {
        const GemmPlan gp = gemm_plan(S, (int)nk.first, (int)nk.second);
        if (gp.ranges > 1) part = std::max(part, (size_t)gp.ranges * S * nk.first);
    }
    return part;
}

hipError_t prefill_alloc(sh_model *m, int S, bool logits) {
    const size_t need = prefill_part_need(m, S);
    if (m->pf_cap >= S && (!logits || m->pf_logits) && m->pf_part_cap >= need) return hipSuccess;
    const bool want_logits = logits || m->pf_logits;
    S = std::max(S, m->pf_cap);
    const size_t part = std::max({need, m->pf_part_cap, prefill_part_need(m, S)});
    logits = want_logits;
    const sh_config &c = m->cfg;
    if (m->wd_ready) {   // the captured window step points into this scratch
        (void)hipGraphExecDestroy(m->wd_exec);
        m->wd_ready = false;
    }
    if (m->pf_ready) {   // so does the captured forward
        (void)hipGraphExecDestroy(m->pf_exec);
        m->pf_ready = false;
    }
    (void)hipFree(m->pf_arena);
    m->pf_arena = nullptr;
    m->pf_cap = 0;
    m->pf_part_cap = 0;
    m->pf_logits = nullptr;
    const size_t D = c.dim, F = c.hidden, Q = m->qdim, KV = m->kvdim, R = m->qkv_rows, V = c.vocab;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += (bytes + 255) / 256 * 256;
        return o;
    };
    const size_t o_tok = take(4 * S), o_pos = take(4 * S), o_seq = take(4 * S),
                 o_x = take(4 * S * D), o_x2 = take(4 * S * D), o_xn = take(4 * S * D),
                 o_qkv = take(4 * S * R), o_q = take(4 * S * Q), o_k = take(4 * S * KV),
                 o_v = take(4 * S * KV), o_att = take(4 * S * Q), o_gate = take(4 * S * F),
                 o_log = logits ? take(4 * V * S) : 0, o_cf = take(4 * S * D);
    const size_t o_part = take(4 * part);   // K-range partials of the split GEMMs
    const bool q8 = m->dtype == SH_DTYPE_W8A8;   // quantized A operand and its row scales
    const size_t o_a8 = q8 ? take((size_t)S * std::max({D, Q, F})) : 0, o_sa = q8 ? take(4 * S) : 0;
    hipError_t e = hipMalloc(&m->pf_arena, off);
    if (e != hipSuccess) return e;
    uint8_t *A = (uint8_t *)m->pf_arena;
    m->pf_tokens = (int32_t *)(A + o_tok);
    m->pf_rowpos = (int32_t *)(A + o_pos);
    m->pf_rowseq = (int32_t *)(A + o_seq);
    m->pf_x = (float *)(A + o_x);
    m->pf_x2 = (float *)(A + o_x2);
    m->pf_xn = (uint16_t *)(A + o_xn);
    m->pf_qkv = (float *)(A + o_qkv);
    m->pf_q = (float *)(A + o_q);
    m->pf_k = (float *)(A + o_k);
    m->pf_v = (float *)(A + o_v);
    m->pf_att = (uint16_t *)(A + o_att);
    m->pf_gate = (uint16_t *)(A + o_gate);
    m->pf_logits = logits ? (float *)(A + o_log) : nullptr;
    m->pf_cf = (float *)(A + o_cf);
    m->pf_part = (float *)(A + o_part);
    m->pf_part_cap = part;
    m->pf_a8 = q8 ? (int8_t *)(A + o_a8) : nullptr;
    m->pf_sa = q8 ? (float *)(A + o_sa) : nullptr;
    m->pf_cap = S;
    return hipSuccess;
}

namespace {

void *kv_layer_base(const sh_model *m, void *cache, int l) {
    const size_t kvb = m->cfg.kv_dtype == SH_KV_F32 ? 4 : 2;
    return (uint8_t *)cache + (size_t)l * m->cfg.max_seq * m->kvdim * kvb;
}
size_t kv_seq_stride(const sh_model *m) {
    return (size_t)m->cfg.n_layers * m->cfg.max_seq * m->kvdim;
}

QkRopeArgs qk_rope_args(const sh_model *m, const LayerDev &L, const int32_t *rowpos,
                        const int32_t *rowseq, float *q, float *k, float *v, int l, bool fill) {
    const sh_config &c = m->cfg;
    QkRopeArgs a{};
    a.qdim = m->qdim;
    a.kvdim = m->kvdim;
    a.hd = c.head_dim;
    a.qk_norm = c.qk_norm;
    a.q_norm = L.q_norm;
    a.k_norm = L.k_norm;
    a.qk_eps = c.qk_norm_eps;
    a.rope_cos = m->rope_cos;
    a.rope_sin = m->rope_sin;
    a.rowpos = rowpos;
    a.rowseq = rowseq;
    a.qo = q;
    a.ko = k;
    a.vo = v;
    a.kcache = fill ? kv_layer_base(m, m->kcache, l) : nullptr;
    a.vcache = fill ? kv_layer_base(m, m->vcache, l) : nullptr;
    a.kv_seq_stride = kv_seq_stride(m);
    a.write_cache = fill ? 1 : 0;
    a.round_kv = m->dtype == SH_DTYPE_W8A8 ? 1 : 0;   // W8A8 attends as the decode does
    return a;
}

hipError_t launch_qk_rope(const sh_model *m, const LayerDev &L, int rows, const float *qkv,
                          const int32_t *rowpos, const int32_t *rowseq, float *q, float *k,
                          float *v, int l, bool fill, hipStream_t s) {
    const QkRopeArgs a = qk_rope_args(m, L, rowpos, rowseq, q, k, v, l, fill);
    const int kv = m->cfg.kv_dtype;
    if (kv == SH_KV_F32) hipLaunchKernelGGL(k_qk_rope<SH_KV_F32>, dim3(rows), dim3(kT), 0, s, qkv, a);
    else if (kv == SH_KV_F16) hipLaunchKernelGGL(k_qk_rope<SH_KV_F16>, dim3(rows), dim3(kT), 0, s, qkv, a);
    else hipLaunchKernelGGL(k_qk_rope<SH_KV_BF16>, dim3(rows), dim3(kT), 0, s, qkv, a);
    return hipGetLastError();
}

// The fused q|k|v product and row epilogue (k_gemm_pipe_qkv64) applies to 16-bit models with
// 64-dim heads whose projection the pipelined 64 x 64 GEMM takes unsplit (short inputs).
bool qkv64_fused(const sh_model *m, int S) {
    const int D = m->cfg.dim;
    return m->dtype != SH_DTYPE_W8A8 && m->cfg.head_dim == 64 && S < 1024 && m->qkv_rows % 64 == 0 &&
           D % 64 == 0 && D / 64 >= 5;
}

// The one-plane fp16 forward (EvalLogits) with the fused q|k|v product: k and v are written
// as fp16 and its 16-query attention reads them so (the values it would round them to).
bool attn_kv16(const sh_model *m, int S) {
    return m->pf_one_plane && m->dtype == SH_DTYPE_F16 && qkv64_fused(m, S) &&
           (size_t)((S + 63) / 64) * m->cfg.n_heads < 256;
}

template <int BM>
void launch_qkv64_bm(const GemmArgs &g, const QkRopeArgs &a, int kv, hipStream_t s) {
    const dim3 grid((g.M + BM - 1) / BM, g.N / 64);
    const bool bf = g.dt == SH_DTYPE_BF16;
    const size_t lds1 = BM == 64 ? kPipeBigLds : qkv64_lds<BM, 1>(), lds2 = BM == 64 ? kPipeBigLds : qkv64_lds<BM, 2>();
    if (g.one_plane && !bf) {
        if (kv == SH_KV_F32) hipLaunchKernelGGL((k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_F32, 1, BM>), grid, dim3(kT), lds1, s, g, a);
        else if (kv == SH_KV_F16) hipLaunchKernelGGL((k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_F16, 1, BM>), grid, dim3(kT), lds1, s, g, a);
        else hipLaunchKernelGGL((k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_BF16, 1, BM>), grid, dim3(kT), lds1, s, g, a);
    } else if (kv == SH_KV_F32) {
        if (bf) hipLaunchKernelGGL((k_gemm_pipe_qkv64<SH_DTYPE_BF16, SH_KV_F32, 2, BM>), grid, dim3(kT), lds2, s, g, a);
        else hipLaunchKernelGGL((k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_F32, 2, BM>), grid, dim3(kT), lds2, s, g, a);
    } else if (kv == SH_KV_F16) {
        if (bf) hipLaunchKernelGGL((k_gemm_pipe_qkv64<SH_DTYPE_BF16, SH_KV_F16, 2, BM>), grid, dim3(kT), lds2, s, g, a);
        else hipLaunchKernelGGL((k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_F16, 2, BM>), grid, dim3(kT), lds2, s, g, a);
    } else {
        if (bf) hipLaunchKernelGGL((k_gemm_pipe_qkv64<SH_DTYPE_BF16, SH_KV_BF16, 2, BM>), grid, dim3(kT), lds2, s, g, a);
        else hipLaunchKernelGGL((k_gemm_pipe_qkv64<SH_DTYPE_F16, SH_KV_BF16, 2, BM>), grid, dim3(kT), lds2, s, g, a);
    }
}
// 32-row tiles for inputs of at most 32 rows (a 64-row tile would be mostly padding: the
// 16-position prompt forward 0.507 -> 0.470 ms); at 256 rows the 64-row tiles are faster
// (0.0025 ms per forward), although the 32-row grid has twice the workgroups
hipError_t launch_qkv64(const GemmArgs &g, const QkRopeArgs &a, int kv, hipStream_t s) {
    hipError_t e = gemm_pipe_setup_once();
    if (e != hipSuccess) return e;
    if (g.M <= 32) launch_qkv64_bm<32>(g, a, kv, s);
    else launch_qkv64_bm<64>(g, a, kv, s);
    return hipGetLastError();
}

// W8A8: the decode-order attention of `rows` query rows (k_attn_exact), keys from the
// token-major pf_k / pf_v of the forward or, with from_cache, from layer l of the KV cache.
hipError_t launch_attn_exact(const sh_model *m, int rows, const float *q, bool from_cache, int l,
                             const int32_t *rowpos, const int32_t *rowseq, float *att,
                             hipStream_t s) {
    const sh_config &c = m->cfg;
    const float inv = (float)(1.0 / sqrt((double)c.head_dim));
    const dim3 grid(rows, c.n_heads);
    const size_t stride = kv_seq_stride(m);
    if (c.head_dim > 256 || c.max_seq > kMaxSeqLds) return hipErrorInvalidValue;
    if (!from_cache)
        hipLaunchKernelGGL(k_attn_exact<SH_KV_F32>, grid, dim3(kT), 0, s, q, m->qdim,
                           (const void *)m->pf_k, (const void *)m->pf_v, stride, m->kvdim, 0,
                           rowpos, rowseq, c.n_heads, c.n_kv_heads, c.head_dim, inv, att);
    else {
        const void *kb = kv_layer_base(m, m->kcache, l), *vb = kv_layer_base(m, m->vcache, l);
#define SH_AE(KV) hipLaunchKernelGGL(k_attn_exact<KV>, grid, dim3(kT), 0, s, q, m->qdim, kb, vb, stride, \
                                     m->kvdim, 1, rowpos, rowseq, c.n_heads, c.n_kv_heads, c.head_dim, inv, att)
        if (c.kv_dtype == SH_KV_F32) SH_AE(SH_KV_F32);
        else if (c.kv_dtype == SH_KV_F16) SH_AE(SH_KV_F16);
        else SH_AE(SH_KV_BF16);
#undef SH_AE
    }
    return hipGetLastError();
}

// Causal attention of the S rows: the MFMA kernel for head dims 32 / 64 / 128, its K and V
// carried as hi/lo planes unless fill_kv has already rounded them to the model's 16-bit type.
hipError_t launch_attn_prefill(const sh_model *m, int S, int seg_max, bool fill_kv, float scale,
                               hipStream_t s) {
    const sh_config &c = m->cfg;
    const int dt = m->dtype;
    const size_t plane = (size_t)S * m->qdim;
    const bool exact = fill_kv && ((c.kv_dtype == SH_KV_BF16 && dt == SH_DTYPE_BF16) ||
                                   (c.kv_dtype == SH_KV_F16 && dt == SH_DTYPE_F16));
    // 64-query tiles when their grid alone covers the CUs, else 16-query tiles
    const bool wide = (size_t)((S + 63) / 64) * c.n_heads >= 256;
    const dim3 grid = wide ? dim3((S + 63) / 64 * c.n_heads) : dim3((S + 15) / 16, c.n_heads);
#define SH_ATT(DTV, HDV, LOV)                                                                   \
    do {                                                                                        \
        if (wide)                                                                               \
            hipLaunchKernelGGL((k_attn_prefill_mfma64<DTV, HDV, LOV>), grid, dim3(kT), 0, s,     \
                               m->pf_q, m->pf_k, m->pf_v, S, m->pf_rowpos, c.n_heads,             \
                               c.n_kv_heads, scale, m->pf_att, plane);                           \
        else                                                                                    \
            hipLaunchKernelGGL((k_attn_prefill_mfma<DTV, HDV, LOV>), grid, dim3(kT), 0, s,       \
                               m->pf_q, m->pf_k, m->pf_v, S, m->pf_rowpos, c.n_heads,             \
                               c.n_kv_heads, scale, m->pf_att, plane);                           \
    } while (0)
#define SH_ATT_HD(DTV, LOV)                                                                     \
    if (c.head_dim == 32) SH_ATT(DTV, 32, LOV);                                                  \
    else if (c.head_dim == 64) SH_ATT(DTV, 64, LOV);                                             \
    else SH_ATT(DTV, 128, LOV);
    if (m->pf_one_plane && dt == SH_DTYPE_F16 && !wide &&
        (c.head_dim == 32 || c.head_dim == 64 || c.head_dim == 128)) {
        // EvalLogits (fp16): Q, K, V and P as one fp16 plane each; its rows are positions
        // 0..S-1 of one sequence, so the kernel needs no position lookups
        if (c.head_dim == 32)
            hipLaunchKernelGGL((k_attn_prefill_mfma<SH_DTYPE_F16, 32, false, 1>), grid, dim3(kT), 0, s, m->pf_q,
                               m->pf_k, m->pf_v, S, nullptr, c.n_heads, c.n_kv_heads, scale, m->pf_att, plane);
        else if (c.head_dim == 64 && attn_kv16(m, S))   // k and v already fp16
            hipLaunchKernelGGL((k_attn_prefill_mfma<SH_DTYPE_F16, 64, false, 1, true>), grid, dim3(kT), 0, s,
                               m->pf_q, m->pf_k, m->pf_v, S, nullptr, c.n_heads, c.n_kv_heads, scale, m->pf_att,
                               plane);
        else if (c.head_dim == 64)
            hipLaunchKernelGGL((k_attn_prefill_mfma<SH_DTYPE_F16, 64, false, 1>), grid, dim3(kT), 0, s, m->pf_q,
                               m->pf_k, m->pf_v, S, nullptr, c.n_heads, c.n_kv_heads, scale, m->pf_att, plane);
        else
            hipLaunchKernelGGL((k_attn_prefill_mfma<SH_DTYPE_F16, 128, false, 1>), grid, dim3(kT), 0, s, m->pf_q,
                               m->pf_k, m->pf_v, S, nullptr, c.n_heads, c.n_kv_heads, scale, m->pf_att, plane);
    } else if (c.head_dim == 32 || c.head_dim == 64 || c.head_dim == 128) {
        if (dt == SH_DTYPE_BF16) {
            if (exact) { SH_ATT_HD(SH_DTYPE_BF16, false) } else { SH_ATT_HD(SH_DTYPE_BF16, true) }
        } else {
            if (exact) { SH_ATT_HD(SH_DTYPE_F16, false) } else { SH_ATT_HD(SH_DTYPE_F16, true) }
        }
    } else {
        const int wpb = kT / 64;
        hipLaunchKernelGGL(k_attn_prefill, dim3((S + wpb - 1) / wpb, c.n_heads), dim3(kT),
                           sizeof(float) * wpb * seg_max, s, m->pf_q, m->pf_k, m->pf_v, S,
                           seg_max, m->pf_rowpos, c.n_heads, c.n_kv_heads, c.head_dim, scale, dt,
                           fill_kv ? 1 : 0, m->pf_att, plane);
    }
#undef SH_ATT_HD
#undef SH_ATT
    return hipGetLastError();
}

}  // namespace

// Enqueues the forward of the S rows pf_tokens[0, S) (row t = position pf_rowpos[t] of
// sequence pf_rowseq[t]; a sequence's rows are consecutive, at most seg_max of them). With
// logits, the full-sequence classifier lands in pf_logits as [V, S]. With fill_kv, every
// row's k and v enter its sequence's KV cache and the layers use the decode forms of the
// softmax sum and SiLU, so the cache holds what a token-by-token decode of the same prompt
// would have written.
namespace {

// One layer of the forward over the S token-major rows in pf_x (rows as in enqueue_prefill);
// the layer's output replaces pf_x. in_normed: pf_xn already holds pf_x normalised with this
// layer's rms_att. next_gain (optional): the gain the caller normalises the output with next
// (next_final: stories.RMSNorm's form); where the last projection leaves K-range partials, the
// row kernel that sums them also writes those normalised rows to pf_xn and *out_normed says
// so. Split projections hand their partials to such row kernels rather than to a separate
// sum: q|k|v to the QK-norm/RoPE rows, Wo and W2 to the residual + RMSNorm rows.
hipError_t enqueue_layer(sh_model *m, int l, int S, int seg_max, bool fill_kv, bool in_normed,
                         const float *next_gain, int next_final, bool *out_normed) {
    const sh_config &c = m->cfg;
    const int dt = m->dtype;
    const int D = c.dim, F = c.hidden;
    hipStream_t s = m->stream;
    hipError_t e;
    const float scale = (float)(1.0 / sqrt((double)c.head_dim));
    const LayerDev &L = m->layers[l];
    if (out_normed) *out_normed = false;
    if (!in_normed)
        hipLaunchKernelGGL(k_rmsnorm_rows, dim3(S), dim3(kT), 0, s, m->pf_x, L.rms_att, D,
                           c.norm_eps, 0, dt, m->pf_xn, (size_t)S * D, nullptr);
    int ranges = 1;
    GemmArgs g{};
    g.A = m->pf_xn; g.B = (const uint16_t *)L.wqkv; g.M = S; g.N = m->qkv_rows; g.K = D;
    g.epi = G_STORE; g.out = m->pf_qkv; g.dt = dt; g.one_plane = m->pf_one_plane;
    g.sw = L.s_qkv; g.a8 = m->pf_a8; g.sa = m->pf_sa;
    if (qkv64_fused(m, S)) {
        QkRopeArgs a = qk_rope_args(m, L, m->pf_rowpos, m->pf_rowseq, m->pf_q, m->pf_k, m->pf_v, l, fill_kv);
        // one-plane fp16 (EvalLogits): k and v leave as the fp16 values its attention reads
        a.kv16 = attn_kv16(m, S);
        if ((e = launch_qkv64(g, a, c.kv_dtype, s)) != hipSuccess) return e;
    } else if ((e = gemm(g, dt, m->pf_part, m->pf_part_cap, s, &ranges)) != hipSuccess) {
        return e;
    } else if (ranges > 1) {
        const QkRopeArgs a = qk_rope_args(m, L, m->pf_rowpos, m->pf_rowseq, m->pf_q, m->pf_k, m->pf_v, l,
                                          fill_kv);
        const float *pp = m->pf_part;
        const int kv = c.kv_dtype;
        if (kv == SH_KV_F32) hipLaunchKernelGGL(k_row_qkv<SH_KV_F32>, dim3(S), dim3(1024), 0, s, pp, ranges, S, a);
        else if (kv == SH_KV_F16) hipLaunchKernelGGL(k_row_qkv<SH_KV_F16>, dim3(S), dim3(1024), 0, s, pp, ranges, S, a);
        else hipLaunchKernelGGL(k_row_qkv<SH_KV_BF16>, dim3(S), dim3(1024), 0, s, pp, ranges, S, a);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    } else if ((e = launch_qk_rope(m, L, S, m->pf_qkv, m->pf_rowpos, m->pf_rowseq, m->pf_q, m->pf_k,
                                   m->pf_v, l, fill_kv, s)) != hipSuccess) {
        return e;
    }
    if (dt == SH_DTYPE_W8A8)
        e = launch_attn_exact(m, S, m->pf_q, false, l, m->pf_rowpos, m->pf_rowseq, (float *)m->pf_att, s);
    else
        e = launch_attn_prefill(m, S, seg_max, fill_kv, scale, s);
    if (e != hipSuccess) return e;
    g = GemmArgs{};
    g.A = m->pf_att; g.B = (const uint16_t *)L.wo; g.M = S; g.N = D; g.K = m->qdim;
    g.epi = G_RESID; g.out = m->pf_x2; g.resid = m->pf_x; g.alpha = c.residual_scale; g.dt = dt;
    g.one_plane = m->pf_one_plane;
    g.sw = L.s_o; g.a8 = m->pf_a8; g.sa = m->pf_sa;
    if ((e = gemm(g, dt, m->pf_part, m->pf_part_cap, s, &ranges)) != hipSuccess) return e;
    if (ranges > 1) {
        if ((e = launch_row_resid_norm((const float *)m->pf_part, ranges, S, D, (const float *)m->pf_x,
                                       c.residual_scale, m->pf_x2, L.rms_ffn, c.norm_eps, 0, dt, m->pf_xn, s)) !=
            hipSuccess)
            return e;
    } else
        hipLaunchKernelGGL(k_rmsnorm_rows, dim3(S), dim3(kT), 0, s, m->pf_x2, L.rms_ffn, D,
                           c.norm_eps, 0, dt, m->pf_xn, (size_t)S * D, nullptr);
    g = GemmArgs{};
    g.A = m->pf_xn; g.B = (const uint16_t *)L.w13; g.M = S; g.N = 2 * F; g.K = D;
    g.epi = G_GATE; g.out16 = m->pf_gate; g.dt = dt; g.decode_forms = fill_kv || dt == SH_DTYPE_W8A8 ? 1 : 0;
    g.one_plane = m->pf_one_plane;
    g.sw = L.s_13; g.a8 = m->pf_a8; g.sa = m->pf_sa;
    if ((e = gemm(g, dt, m->pf_part, m->pf_part_cap, s)) != hipSuccess) return e;
    g = GemmArgs{};
    g.A = m->pf_gate; g.B = (const uint16_t *)L.w2; g.M = S; g.N = D; g.K = F;
    g.epi = G_RESID; g.out = m->pf_x; g.resid = m->pf_x2; g.alpha = c.residual_scale; g.dt = dt;
    g.one_plane = m->pf_one_plane;
    g.sw = L.s_2; g.a8 = m->pf_a8; g.sa = m->pf_sa;
    if (!next_gain) return gemm(g, dt, m->pf_part, m->pf_part_cap, s);
    if ((e = gemm(g, dt, m->pf_part, m->pf_part_cap, s, &ranges)) != hipSuccess) return e;
    if (ranges == 1) return hipSuccess;
    if ((e = launch_row_resid_norm((const float *)m->pf_part, ranges, S, D, (const float *)m->pf_x2,
                                   c.residual_scale, m->pf_x, next_gain, c.norm_eps, next_final, dt, m->pf_xn, s)) !=
        hipSuccess)
        return e;
    if (out_normed) *out_normed = true;
    return hipGetLastError();
}

// logits [V, S] = classifier . (the operand planes in pf_xn)
hipError_t enqueue_classifier(sh_model *m, int S) {
    GemmArgs g{};
    g.A = m->pf_xn; g.B = (const uint16_t *)m->cls; g.M = S; g.N = m->cfg.vocab; g.K = m->cfg.dim;
    g.epi = G_LOGITS_CF; g.out = m->pf_logits; g.dt = m->dtype; g.one_plane = m->pf_one_plane;
    g.sw = m->s_cls; g.a8 = m->pf_a8; g.sa = m->pf_sa;
    return gemm(g, m->dtype, m->pf_part, m->pf_part_cap, m->stream);
}

hipError_t launch_transpose(const float *src, int rows, int cols, float *dst, hipStream_t s) {
    hipLaunchKernelGGL(k_transpose, dim3((cols + 31) / 32, (rows + 31) / 32), dim3(kT), 0, s, src,
                       rows, cols, dst);
    return hipGetLastError();
}

}  // namespace

hipError_t enqueue_prefill(sh_model *m, int S, int seg_max, bool logits, bool fill_kv) {
    const sh_config &c = m->cfg;
    const int dt = m->dtype;
    const int D = c.dim;
    hipStream_t s = m->stream;
    hipError_t e;
    hipLaunchKernelGGL(k_embed_rows, dim3(S), dim3(kT), 0, s, (const uint16_t *)m->embed,
                       m->pf_tokens, c.vocab, D, dt, m->pf_x);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    // the final norm: stories.RMSNorm (cpu.go:97-111); W8A8 keeps the decode's rmsNormVec
    // (infer.go:242), whose result its classifier quantizer sees
    const int final_form = dt == SH_DTYPE_W8A8 ? 0 : 1;
    bool normed = false;
    for (int l = 0; l < c.n_layers; l++) {
        const bool last = l + 1 == c.n_layers;
        const float *next = !last ? m->layers[l + 1].rms_att : logits ? m->rms_final : nullptr;
        if ((e = enqueue_layer(m, l, S, seg_max, fill_kv, normed, next, last ? final_form : 0, &normed)) !=
            hipSuccess)
            return e;
    }
    if (!logits) return hipSuccess;
    if (!normed)
        hipLaunchKernelGGL(k_rmsnorm_rows, dim3(S), dim3(kT), 0, s, m->pf_x, m->rms_final, D,
                           c.norm_eps, final_form, dt, m->pf_xn, (size_t)S * D, nullptr);
    return enqueue_classifier(m, S);
}

hipError_t enqueue_layer_cf(sh_model *m, int l, int S) {
    const int D = m->cfg.dim;
    hipError_t e;
    if ((e = launch_transpose(m->pf_cf, D, S, m->pf_x, m->stream)) != hipSuccess) return e;
    if ((e = enqueue_layer(m, l, S, S, false, false, nullptr, 0, nullptr)) != hipSuccess) return e;
    return launch_transpose(m->pf_x, S, D, m->pf_cf, m->stream);
}

// After enqueue_layer_cf(m, l, S): the layer's intermediates, channel-first, in the output
// order of the reference's fused programs (ane/mil/stories_dynamic.go:162 and :222):
// sdpa [D + 2Q + 2KV, S] = (x2, q_rope, k_rope, v, att), ffn [D + 2F, S] = (x_next, h1, h3).
// The scratch the layer leaves holds them token-major (pf_x2; pf_q, pf_k, pf_v after
// QK-norm and RoPE; pf_att as the operand planes Wo consumed, hi + lo; pf_x2 = x, and pf_xn
// the W1|W3 operand planes); h1 and h3, which the layer only uses inside the SiLU-gate
// epilogue, come from the same W1|W3 product stored plainly into h13 [S, 2F] (interleaved
// rows: column 2r is h1[r], 2r+1 is h3[r]). ffn's x_next is the layer output in pf_cf.
hipError_t enqueue_layer_taps_cf(sh_model *m, int l, int S, float *sdpa, float *ffn, float *h13) {
    const sh_config &c = m->cfg;
    const int D = c.dim, F = c.hidden, Q = m->qdim, KV = m->kvdim;
    hipStream_t s = m->stream;
    hipError_t e;
    auto gather = [&](const float *src, int ncols, int col0, int cstep, int count, float *dst) {
        const size_t n = (size_t)count * S;
        hipLaunchKernelGGL(k_cf_gather, dim3((unsigned)((n + kT - 1) / kT)), dim3(kT), 0, s, src, S,
                           ncols, col0, cstep, count, dst);
        return hipGetLastError();
    };
    if (sdpa) {
        float *o = sdpa;
        if ((e = gather(m->pf_x2, D, 0, 1, D, o)) != hipSuccess) return e;
        o += (size_t)D * S;
        if ((e = gather(m->pf_q, Q, 0, 1, Q, o)) != hipSuccess) return e;
        o += (size_t)Q * S;
        if ((e = gather(m->pf_k, KV, 0, 1, KV, o)) != hipSuccess) return e;
        o += (size_t)KV * S;
        if ((e = gather(m->pf_v, KV, 0, 1, KV, o)) != hipSuccess) return e;
        o += (size_t)KV * S;
        const size_t n = (size_t)S * Q;   // pf_qkv ([S, qkv_rows] >= [S, Q]) is free now
        hipLaunchKernelGGL(k_planes_f32, dim3((unsigned)((n + kT - 1) / kT)), dim3(kT), 0, s,
                           m->pf_att, n, n, m->dtype, m->pf_qkv);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if ((e = gather(m->pf_qkv, Q, 0, 1, Q, o)) != hipSuccess) return e;
    }
    if (ffn) {
        GemmArgs g{};
        g.A = m->pf_xn; g.B = (const uint16_t *)m->layers[l].w13; g.M = S; g.N = 2 * F; g.K = D;
        g.epi = G_STORE; g.out = h13; g.dt = m->dtype;
        g.sw = m->layers[l].s_13; g.a8 = m->pf_a8; g.sa = m->pf_sa;
        if ((e = gemm(g, m->dtype, m->pf_part, m->pf_part_cap, s)) != hipSuccess) return e;
        if ((e = hipMemcpyAsync(ffn, m->pf_cf, sizeof(float) * D * S, hipMemcpyDeviceToDevice, s)) != hipSuccess)
            return e;
        if ((e = gather(h13, 2 * F, 0, 2, F, ffn + (size_t)D * S)) != hipSuccess) return e;
        if ((e = gather(h13, 2 * F, 1, 2, F, ffn + (size_t)(D + F) * S)) != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t enqueue_rms_final_cf(sh_model *m, int S) {
    const int D = m->cfg.dim;
    hipError_t e;
    if ((e = launch_transpose(m->pf_cf, D, S, m->pf_x, m->stream)) != hipSuccess) return e;
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(S), dim3(kT), 0, m->stream, m->pf_x, m->rms_final, D,
                       m->cfg.norm_eps, 1, m->dtype, nullptr, (size_t)0, m->pf_x2);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    return launch_transpose(m->pf_x2, S, D, m->pf_cf, m->stream);
}

hipError_t enqueue_classifier_cf(sh_model *m, int S) {
    const int D = m->cfg.dim;
    hipError_t e;
    if ((e = launch_transpose(m->pf_cf, D, S, m->pf_x, m->stream)) != hipSuccess) return e;
    const size_t n = (size_t)S * D;
    hipLaunchKernelGGL(k_to_planes, dim3((unsigned)((n + kT - 1) / kT)), dim3(kT), 0, m->stream,
                       m->pf_x, n, m->dtype, m->pf_xn, n);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    return enqueue_classifier(m, S);
}

size_t gemm_partial_elems(int M, int N, int K) {
    const GemmPlan p = gemm_plan(M, N, K);
    return p.ranges > 1 ? (size_t)p.ranges * M * N : 0;
}

hipError_t enqueue_linear_rows(const float *x, int M, int K, const uint16_t *w, int N, int dt,
                               uint16_t *planes, float *out, bool cf, float *partial,
                               size_t part_cap, hipStream_t s) {
    const size_t n = (size_t)M * K;
    hipLaunchKernelGGL(k_to_planes, dim3((unsigned)((n + kT - 1) / kT)), dim3(kT), 0, s, x, n, dt,
                       planes, n);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    GemmArgs g{};
    g.A = planes; g.B = w; g.M = M; g.N = N; g.K = K;
    g.epi = cf ? G_LOGITS_CF : G_STORE; g.out = out; g.dt = dt;
    return gemm(g, dt, partial, part_cap, s);
}

hipError_t enqueue_transpose(const float *src, int rows, int cols, float *dst, hipStream_t s) {
    return launch_transpose(src, rows, cols, dst, s);
}


namespace {
// K range per workgroup of the skinny GEMM: 256 (four waves x two k-steps, every load in
// flight at once) when that splits K evenly and the columns alone give too few workgroups.
// K range of the M <= 32-row products: 512 where K allows (the 32-sequence Qwen3-shaped step:
// 2.13 ms, against 2.17 with ranges of 256 and 2.23 with 1024), the whole K for very wide
// outputs (the classifier), whose grid alone covers the CUs.
int skinny_kc(int N, int K) {
    if (N / 16 >= 2048) return K;
    return K % 512 == 0 ? 512 : K % 256 == 0 ? 256 : K;
}

hipError_t skinny(const GemmArgs &g, int dt, float *partial, size_t part_cap, hipStream_t s) {
    if (g.K % 128 || g.N % 16 || g.M > 32) return hipErrorInvalidValue;
    if (dt == SH_DTYPE_W8A8) {   // one K range: "partials" are the finished [M, N] product
        GemmArgs h = g;
        if (g.partial_only) {
            if ((size_t)g.M * g.N > part_cap) return hipErrorInvalidValue;
            h.epi = G_STORE;
            h.out = partial;
        }
        return gemm_i8(h, s);
    }
    // the gate product runs unsplit on the pipelined GEMM, its SiLU gate in the epilogue (no
    // partials and no reduce kernel)
    const bool gate1 = g.epi == G_GATE && !g.partial_only && g.K % 64 == 0 && g.K / 64 >= 3 && g.N % 32 == 0;
    const int kc = gate1 ? g.K : skinny_kc(g.N, g.K), ranges = g.K / kc;
    if ((ranges > 1 || g.partial_only) && (size_t)ranges * g.M * g.N > part_cap)
        return hipErrorInvalidValue;   // the partial buffer must hold every K range
    const bool bf = dt == SH_DTYPE_BF16;
    // The pipelined GEMM with one 32-row tile over the rows, in the same K ranges (so the
    // row kernels and the attention sum the same partials): 32-column tiles, 64-column ones
    // for very wide outputs (the classifier). Against k_gemm_skinny64 / k_gemm_skinny on the
    // 32-sequence Qwen3-shaped step's products: qkv 5.2 -> 3.6 us, wo 4.5 -> 3.0, w13 6.6 ->
    // 4.2, w2 5.6 -> 3.4, the classifier 104 -> 68.
    if (kc % 64 == 0 && kc / 64 >= 3 && g.N % 32 == 0) {
        hipError_t e0 = gemm_pipe_setup_once();
        if (e0 != hipSuccess) return e0;
        GemmArgs h = g;
        if (g.partial_only && ranges == 1) {   // the "partial" is the plain product
            h.epi = G_STORE;
            h.out = partial;
        }
        if (g.N >= 16384 && g.N % 64 == 0) {
            const dim3 grid(1, g.N / 64, ranges);
            if (bf) hipLaunchKernelGGL((k_gemm_pipe<SH_DTYPE_BF16, 32, 64, 64, 4>), grid, dim3(kT), kPipeWideLds, s, h, partial, kc);
            else hipLaunchKernelGGL((k_gemm_pipe<SH_DTYPE_F16, 32, 64, 64, 4>), grid, dim3(kT), kPipeWideLds, s, h, partial, kc);
        } else {
            const dim3 grid(1, g.N / 32, ranges);
            if (bf) hipLaunchKernelGGL((k_gemm_pipe<SH_DTYPE_BF16, 32, 32, 64, 4>), grid, dim3(kT), kPipeSmallLds, s, h, partial, kc);
            else hipLaunchKernelGGL((k_gemm_pipe<SH_DTYPE_F16, 32, 32, 64, 4>), grid, dim3(kT), kPipeSmallLds, s, h, partial, kc);
        }
    } else if (g.N % 64 == 0 && kc % 256 == 0 && (g.N / 64) * ranges >= 256) {
        // 64-column workgroups share the A rows through LDS; narrow products whose 64-column
        // grid would leave CUs idle take 16-column workgroups instead
        const dim3 grid(g.N / 64, ranges);
        if (dt == SH_DTYPE_BF16) hipLaunchKernelGGL(k_gemm_skinny64<SH_DTYPE_BF16>, grid, dim3(kT), 0, s, g, partial, kc);
        else hipLaunchKernelGGL(k_gemm_skinny64<SH_DTYPE_F16>, grid, dim3(kT), 0, s, g, partial, kc);
    } else {
        const dim3 grid(g.N / 16, ranges);
        if (dt == SH_DTYPE_BF16) hipLaunchKernelGGL(k_gemm_skinny<SH_DTYPE_BF16>, grid, dim3(kT), 0, s, g, partial, kc);
        else hipLaunchKernelGGL(k_gemm_skinny<SH_DTYPE_F16>, grid, dim3(kT), 0, s, g, partial, kc);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || ranges == 1 || g.partial_only) return e;
    const int pairs = g.M * (g.N / 2);
    hipLaunchKernelGGL(k_gemm_skinny_reduce, dim3((pairs + kT - 1) / kT), dim3(kT), 0, s, g,
                       (const float *)partial, ranges);
    return hipGetLastError();
}
}  // namespace

hipError_t batch_alloc(sh_model *m, int B) {
    if (m->bt_cap >= B) return hipSuccess;
    const sh_config &c = m->cfg;
    if (m->bt_ready) {
        (void)hipGraphExecDestroy(m->bt_exec);
        m->bt_ready = false;
    }
    (void)hipFree(m->bt_arena);
    m->bt_arena = nullptr;
    m->bt_cap = 0;
    const size_t D = c.dim, F = c.hidden, Q = m->qdim, KV = m->kvdim, R = m->qkv_rows, V = c.vocab;
    const size_t W = std::max({D, Q, F});
    const int chunk = attn_chunk(c.head_dim * (c.kv_dtype == SH_KV_F32 ? 4 : 2));
    const size_t nch = ((size_t)c.max_seq + chunk - 1) / chunk;
    m->bt_nch = (int)nch;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += (bytes + 255) / 256 * 256;
        return o;
    };
    const size_t o_tok = take(4 * B), o_pos = take(4 * B), o_seq = take(4 * B),
                 o_hist = take(4 * (size_t)B * (c.max_seq + 1)), o_x = take(4 * B * D),
                 o_x2 = take(4 * B * D), o_xn = take(4 * B * W), o_qkv = take(4 * B * R),
                 o_q = take(4 * B * Q), o_k = take(4 * B * KV), o_v = take(4 * B * KV),
                 o_att = take(4 * B * Q), o_gate = take(4 * B * F), o_log = take(4 * B * V),
                 o_pm = take(4 * B * c.n_heads * nch), o_pl = take(4 * B * c.n_heads * nch),
                 o_pacc = take(4 * B * c.n_heads * nch * c.head_dim);
    // skinny-GEMM K-range partials: the largest (ranges x N) of the layer projections
    size_t part = 0;
    for (auto nk : {std::make_pair(R, D), std::make_pair(D, Q), std::make_pair(2 * F, D),
                    std::make_pair(D, F)}) {
        const size_t kc = skinny_kc((int)nk.first, (int)nk.second);
        part = std::max(part, nk.second / kc * nk.first);
    }
    if (skinny_kc((int)V, (int)D) != D)   // a split classifier GEMM keeps partials too
        part = std::max(part, D / skinny_kc((int)V, (int)D) * V);
    const size_t o_part = take(4 * B * std::max(part, (size_t)1));
    const size_t nblk = (V + kArgChunk - 1) / kArgChunk;
    const size_t o_apv = take(4 * B * nblk), o_api = take(4 * B * nblk);
    const bool q8 = m->dtype == SH_DTYPE_W8A8;   // quantized A operand and its row scales
    const size_t o_a8 = q8 ? take((size_t)B * W) : 0, o_sa = q8 ? take(4 * (size_t)B) : 0;
    // the streaming attention's tagged split partials, merge counters and call generation
    const size_t nt = (size_t)B * c.n_heads * nch;
    const size_t o_tm = take(8 * nt), o_tl = take(8 * nt), o_tacc = take(8 * nt * c.head_dim),
                 o_cnt = take(4 * (size_t)B * c.n_kv_heads), o_gen = take(4), o_err = take(4);
    const size_t o_tag0 = o_tm, tag_bytes = o_err + 4 - o_tm;
    hipError_t e = hipMalloc(&m->bt_arena, off);
    if (e != hipSuccess) return e;
    uint8_t *A = (uint8_t *)m->bt_arena;
    m->bt_tok = (int32_t *)(A + o_tok);
    m->bt_pos = (int32_t *)(A + o_pos);
    m->bt_seq = (int32_t *)(A + o_seq);
    m->bt_hist = (int32_t *)(A + o_hist);
    m->bt_x = (float *)(A + o_x);
    m->bt_x2 = (float *)(A + o_x2);
    m->bt_xn = (uint16_t *)(A + o_xn);
    m->bt_qkv = (float *)(A + o_qkv);
    m->bt_q = (float *)(A + o_q);
    m->bt_k = (float *)(A + o_k);
    m->bt_v = (float *)(A + o_v);
    m->bt_att = (uint16_t *)(A + o_att);
    m->bt_gate = (uint16_t *)(A + o_gate);
    m->bt_logits = (float *)(A + o_log);
    m->bt_pm = (float *)(A + o_pm);
    m->bt_pl = (float *)(A + o_pl);
    m->bt_pacc = (float *)(A + o_pacc);
    m->bt_part = (float *)(A + o_part);
    m->bt_part_cap = (size_t)B * std::max(part, (size_t)1);
    m->bt_apv = (float *)(A + o_apv);
    m->bt_api = (int32_t *)(A + o_api);
    m->bt_a8 = q8 ? (int8_t *)(A + o_a8) : nullptr;
    m->bt_sa = q8 ? (float *)(A + o_sa) : nullptr;
    m->bt_tm = (uint64_t *)(A + o_tm);
    m->bt_tl = (uint64_t *)(A + o_tl);
    m->bt_tacc = (uint64_t *)(A + o_tacc);
    m->bt_cnt = (int32_t *)(A + o_cnt);
    m->bt_gen = (uint32_t *)(A + o_gen);
    m->bt_err = (int32_t *)(A + o_err);
    m->bt_gen_host = 0;
    // tags 0 (never written), counters 0 (every merge leaves them at 0), generation 0
    if ((e = hipMemset(A + o_tag0, 0, tag_bytes)) != hipSuccess) return e;
    m->bt_cap = B;
    std::vector<int32_t> seq(B);
    for (int b = 0; b < B; b++) seq[b] = b;
    return hipMemcpy(m->bt_seq, seq.data(), 4 * (size_t)B, hipMemcpyHostToDevice);
}


// A new call generation for the streaming attention's tags (words of earlier calls never
// match); before the tags would wrap, the tagged words are cleared and the count restarts.
hipError_t batch_new_generation(sh_model *m) {
    const sh_config &c = m->cfg;
    const uint64_t span = (uint64_t)(c.max_seq + 1) * (uint64_t)c.n_layers;
    if ((uint64_t)(m->bt_gen_host + 2) * span >= 0xFFFFFFF0ull) {
        const size_t bytes = (size_t)((uint8_t *)m->bt_gen - (uint8_t *)m->bt_tm);
        hipError_t e = hipMemset(m->bt_tm, 0, bytes);
        if (e != hipSuccess) return e;
        m->bt_gen_host = 0;
    }
    m->bt_gen_host++;
    return hipMemcpy(m->bt_gen, &m->bt_gen_host, 4, hipMemcpyHostToDevice);
}

bool batch_supported(const sh_model *m, int B, std::string *why) {
    if (!prefill_supported(m, why)) return false;
    const sh_config &c = m->cfg;
    if (B < 1 || B > 32 || B > c.max_batch) {
        *why = "batch must be 1..min(32, max_batch)";
        return false;
    }
    if (c.dim % 128 || m->qdim % 128 || c.hidden % 128) {
        *why = "batched decode needs dim, n_heads*head_dim and hidden multiples of 128";
        return false;
    }
    if (c.n_heads / c.n_kv_heads > kMaxGroupB || (c.n_heads / c.n_kv_heads) * c.head_dim > kT) {
        *why = "batched decode needs (q heads per kv head) * head_dim <= 256";
        return false;
    }
    return true;
}

// One decode step for the B sequences: token bt_tok[b] at position bt_pos[b] of sequence b
// (its K/V appended to the cache), logits [B, V], then argmax and advance (bt_hist row b,
// column pos+1). Everything reads its positions from device memory, so the step can be
// captured once and replayed.
hipError_t enqueue_batch_step(sh_model *m, int B) {
    const sh_config &c = m->cfg;
    const int dt = m->dtype;
    const int D = c.dim, F = c.hidden;
    hipStream_t s = m->stream;
    hipError_t e;
    hipLaunchKernelGGL(k_embed_rows, dim3(B), dim3(kT), 0, s, (const uint16_t *)m->embed, m->bt_tok,
                       c.vocab, D, dt, m->bt_x);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(B), dim3(kT), 0, s, m->bt_x, m->layers[0].rms_att, D,
                       c.norm_eps, 0, dt, m->bt_xn, (size_t)B * D);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const float scale = (float)(1.0 / sqrt((double)c.head_dim));
    const int nch = m->bt_nch;
    const int kvb = c.kv_dtype == SH_KV_F32 ? 4 : 2;
    const int chunk = attn_chunk(c.head_dim * kvb);
    // streaming attention: enough splits of each sequence's keys to give about one
    // workgroup per CU, within the partial buffers (nch slots per head and sequence)
    const AttnStreamKernel astream = pick_attn_stream(c.kv_dtype, c.head_dim, c.n_heads / c.n_kv_heads);
    const int schunk = kChunkBytes / (c.head_dim * kvb);
    const int athreads = attn_stream_threads(c.head_dim, c.n_heads / c.n_kv_heads);
    const int awg = athreads == kAWT ? 256 : 512;   // workgroups that fill the chip
    int nsplit = std::max(1, (awg + B * c.n_kv_heads - 1) / (B * c.n_kv_heads));
    nsplit = std::min({nsplit, nch, (c.max_seq + schunk - 1) / schunk});
    // K ranges the row kernels sum (the W8A8 product leaves one)
    auto ranges = [dt](int N, int K) { return dt == SH_DTYPE_W8A8 ? 1 : K / skinny_kc(N, K); };
    for (int l = 0; l < c.n_layers; l++) {
        const LayerDev &L = m->layers[l];
        // q|k|v projection; row kernel: K-range sum, QK-norm, RoPE, KV append, q out
        GemmArgs g{};
        g.A = m->bt_xn; g.B = (const uint16_t *)L.wqkv; g.M = B; g.N = m->qkv_rows; g.K = D;
        g.dt = dt; g.partial_only = 1;
        g.sw = L.s_qkv; g.a8 = m->bt_a8; g.sa = m->bt_sa;
        if ((e = skinny(g, dt, m->bt_part, m->bt_part_cap, s)) != hipSuccess) return e;
        const QkRopeArgs qa = qk_rope_args(m, L, m->bt_pos, m->bt_seq, m->bt_q, nullptr, nullptr, l, true);
        const int rq = ranges(m->qkv_rows, D);
        // the streaming attention finishes its own q|k|v rows (and writes the cache row)
        const bool fused = astream && dt != SH_DTYPE_W8A8;
        if (fused) {
        } else if (c.kv_dtype == SH_KV_F32)
            hipLaunchKernelGGL(k_row_qkv<SH_KV_F32>, dim3(B), dim3(1024), 0, s, (const float *)m->bt_part, rq, B, qa);
        else if (c.kv_dtype == SH_KV_F16)
            hipLaunchKernelGGL(k_row_qkv<SH_KV_F16>, dim3(B), dim3(1024), 0, s, (const float *)m->bt_part, rq, B, qa);
        else
            hipLaunchKernelGGL(k_row_qkv<SH_KV_BF16>, dim3(B), dim3(1024), 0, s, (const float *)m->bt_part, rq, B, qa);
        if (!fused && (e = hipGetLastError()) != hipSuccess) return e;
        // attention over each sequence's cache, streamed by workgroup (split, kv head,
        // sequence); shapes without a streaming instance split over fixed chunks and merge;
        // W8A8 in the decode's order (its Wo quantizer must see the decode's values)
        const void *kc = kv_layer_base(m, m->kcache, l), *vc = kv_layer_base(m, m->vcache, l);
        if (dt == SH_DTYPE_W8A8) {
            if ((e = launch_attn_exact(m, B, m->bt_q, true, l, m->bt_pos, m->bt_seq, (float *)m->bt_att, s)) !=
                hipSuccess)
                return e;
        } else if (astream) {
            hipLaunchKernelGGL(astream, dim3(nsplit, c.n_kv_heads, B), dim3(athreads), 0, s,
                               (const float *)m->bt_part, rq, qa, kc, vc, kv_seq_stride(m), m->bt_pos, c.n_heads, c.n_kv_heads, scale, nsplit, nch,
                               dt, (size_t)B * c.n_heads * c.head_dim, m->bt_att, m->bt_tm, m->bt_tl,
                               m->bt_tacc, m->bt_cnt, m->bt_gen, l, c.n_layers, c.max_seq, m->bt_err);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        const dim3 grid(nch, c.n_kv_heads, B);
        const bool chunked = !astream && dt != SH_DTYPE_W8A8;
        if (!chunked) {
        } else if (c.kv_dtype == SH_KV_F32)
            hipLaunchKernelGGL(k_attn_batch_partial<SH_KV_F32>, grid, dim3(kT), 0, s, m->bt_q, kc, vc,
                               kv_seq_stride(m), m->bt_pos, c.n_heads, c.n_kv_heads, c.head_dim,
                               scale, nch, m->bt_pm, m->bt_pl, m->bt_pacc);
        else if (c.kv_dtype == SH_KV_F16)
            hipLaunchKernelGGL(k_attn_batch_partial<SH_KV_F16>, grid, dim3(kT), 0, s, m->bt_q, kc, vc,
                               kv_seq_stride(m), m->bt_pos, c.n_heads, c.n_kv_heads, c.head_dim,
                               scale, nch, m->bt_pm, m->bt_pl, m->bt_pacc);
        else
            hipLaunchKernelGGL(k_attn_batch_partial<SH_KV_BF16>, grid, dim3(kT), 0, s, m->bt_q, kc, vc,
                               kv_seq_stride(m), m->bt_pos, c.n_heads, c.n_kv_heads, c.head_dim,
                               scale, nch, m->bt_pm, m->bt_pl, m->bt_pacc);
        if (chunked) {
            if ((e = hipGetLastError()) != hipSuccess) return e;
            hipLaunchKernelGGL(k_attn_batch_combine, dim3(c.n_heads, B), dim3(256), 0, s, m->bt_pm,
                               m->bt_pl, m->bt_pacc, m->bt_pos, c.n_heads, c.head_dim, nch, chunk, B,
                               dt, m->bt_att);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        // Wo; row kernel: x2 = x + alpha * (att . Wo^T), then rmsnorm(x2) with rms_ffn
        g = GemmArgs{};
        g.A = m->bt_att; g.B = (const uint16_t *)L.wo; g.M = B; g.N = D; g.K = m->qdim;
        g.dt = dt; g.partial_only = 1;
        g.sw = L.s_o; g.a8 = m->bt_a8; g.sa = m->bt_sa;
        if ((e = skinny(g, dt, m->bt_part, m->bt_part_cap, s)) != hipSuccess) return e;
        if ((e = launch_row_resid_norm((const float *)m->bt_part, ranges(D, m->qdim), B, D,
                                       (const float *)m->bt_x, c.residual_scale, m->bt_x2, L.rms_ffn, c.norm_eps,
                                       0, dt, m->bt_xn, s)) != hipSuccess)
            return e;
        // W1/W3 with the SiLU gate
        g = GemmArgs{};
        g.A = m->bt_xn; g.B = (const uint16_t *)L.w13; g.M = B; g.N = 2 * F; g.K = D;
        g.epi = G_GATE; g.out16 = m->bt_gate; g.dt = dt; g.decode_forms = 1;
        g.sw = L.s_13; g.a8 = m->bt_a8; g.sa = m->bt_sa;
        if ((e = skinny(g, dt, m->bt_part, m->bt_part_cap, s)) != hipSuccess) return e;
        // W2; row kernel: x = x2 + alpha * (gate . W2^T), then rmsnorm(x) with the next
        // layer's rms_att, or rms_final (rmsNormVec, infer.go:242) after the last layer
        g = GemmArgs{};
        g.A = m->bt_gate; g.B = (const uint16_t *)L.w2; g.M = B; g.N = D; g.K = F;
        g.dt = dt; g.partial_only = 1;
        g.sw = L.s_2; g.a8 = m->bt_a8; g.sa = m->bt_sa;
        if ((e = skinny(g, dt, m->bt_part, m->bt_part_cap, s)) != hipSuccess) return e;
        const float *next_gain = l + 1 < c.n_layers ? m->layers[l + 1].rms_att : m->rms_final;
        if ((e = launch_row_resid_norm((const float *)m->bt_part, ranges(D, F), B, D, (const float *)m->bt_x2,
                                       c.residual_scale, m->bt_x, next_gain, c.norm_eps, 0, dt, m->bt_xn, s)) !=
            hipSuccess)
            return e;
    }
    GemmArgs g{};
    g.A = m->bt_xn; g.B = (const uint16_t *)m->cls; g.M = B; g.N = c.vocab; g.K = D;
    g.epi = G_STORE; g.out = m->bt_logits; g.dt = dt;
    g.sw = m->s_cls; g.a8 = m->bt_a8; g.sa = m->bt_sa;
    if ((e = skinny(g, dt, m->bt_part, m->bt_part_cap, s)) != hipSuccess) return e;
    const int nblk = (c.vocab + kArgChunk - 1) / kArgChunk;
    hipLaunchKernelGGL(k_argmax_part, dim3(nblk, B), dim3(kT), 0, s, m->bt_logits, c.vocab, nblk,
                       m->bt_apv, m->bt_api);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_argmax_advance, dim3(B), dim3(64), 0, s, m->bt_apv, m->bt_api, nblk,
                       m->bt_tok, m->bt_pos, m->bt_hist, c.max_seq + 1);
    return hipGetLastError();
}


hipError_t window_alloc(sh_model *m, int max_new) {
    const sh_config &c = m->cfg;
    if (m->wd_arena && m->wd_cap >= max_new) return hipSuccess;
    (void)hipFree(m->wd_arena);
    m->wd_arena = nullptr;
    m->wd_cap = 0;
    if (m->wd_ready) {
        (void)hipGraphExecDestroy(m->wd_exec);
        m->wd_ready = false;
    }
    const size_t D = c.dim, V = c.vocab;
    const size_t ranges = D / skinny_kc((int)V, (int)D);
    const size_t nblk = (V + kArgChunk - 1) / kArgChunk;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += (bytes + 255) / 256 * 256;
        return o;
    };
    const size_t o_xn = take(4 * D), o_log = take(4 * V), o_part = take(4 * ranges * V),
                 o_apv = take(4 * nblk), o_api = take(4 * nblk), o_hist = take(4 * (size_t)max_new),
                 o_cnt = take(4);
    hipError_t e = hipMalloc(&m->wd_arena, off);
    if (e != hipSuccess) return e;
    uint8_t *A = (uint8_t *)m->wd_arena;
    m->wd_xn = (uint16_t *)(A + o_xn);
    m->wd_logits = (float *)(A + o_log);
    m->wd_part = (float *)(A + o_part);
    m->wd_part_cap = ranges * V;
    m->wd_apv = (float *)(A + o_apv);
    m->wd_api = (int32_t *)(A + o_api);
    m->wd_hist = (int32_t *)(A + o_hist);
    m->wd_count = (int32_t *)(A + o_cnt);
    m->wd_cap = max_new;
    return hipSuccess;
}

// One window decode step over the `seq` ids in pf_tokens: the full causal forward
// (evalLogitsCPUInto numerics), stories.RMSNorm of the last row (cpu.go:97-111), its logits
// (MatMulVocabSeq's column seq-1), argmax, window shift.
hipError_t enqueue_window_step(sh_model *m, int seq) {
    const sh_config &c = m->cfg;
    const int dt = m->dtype, D = c.dim;
    hipStream_t s = m->stream;
    hipError_t e;
    if ((e = enqueue_prefill(m, seq, seq, false, false)) != hipSuccess) return e;
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(1), dim3(kT), 0, s, m->pf_x + (size_t)(seq - 1) * D,
                       m->rms_final, D, c.norm_eps, dt == SH_DTYPE_W8A8 ? 0 : 1, dt, m->wd_xn, (size_t)D);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    GemmArgs g{};
    g.A = m->wd_xn; g.B = (const uint16_t *)m->cls; g.M = 1; g.N = c.vocab; g.K = D;
    g.epi = G_STORE; g.out = m->wd_logits; g.dt = dt;
    g.sw = m->s_cls; g.a8 = m->pf_a8; g.sa = m->pf_sa;   // the forward is done with them
    if ((e = skinny(g, dt, m->wd_part, m->wd_part_cap, s)) != hipSuccess) return e;
    const int nblk = (c.vocab + kArgChunk - 1) / kArgChunk;
    hipLaunchKernelGGL(k_argmax_part, dim3(nblk, 1), dim3(kT), 0, s, m->wd_logits, c.vocab, nblk,
                       m->wd_apv, m->wd_api);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_window_advance, dim3(1), dim3(kT), 0, s, m->wd_apv, m->wd_api, nblk,
                       m->pf_tokens, seq, m->wd_hist, m->wd_count);
    return hipGetLastError();
}

}  // namespace sh
