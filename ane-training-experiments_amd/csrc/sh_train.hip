// sh_train.hip — the storiesane training step (ane/storiesane/engine.go:295-361 Step,
// train_full.go forwardTrainingCPU / runFinalHead / backwardAndApply) on gfx950, fp32.
//
// The reference trains in float32 on the CPU; so does this path: fp32 master weights, fp32
// activations, and every GEMM on v_mfma_f32_16x16x4_f32 (fp32 operands, exact products, fp32
// accumulation), so the step tracks the CPU's arithmetic rather than a 16-bit rounding of it.
// Activations are token-major ([S, C], row t = token t); the reference's channel-first
// [C, S] layout only changes addressing.
//
// Parameters, gradients and the two Adam moments live in four arenas of identical layout:
// the matrices first (per layer Wq|Wk|Wv rows, Wo, W1|W3 rows, W2; then the embedding, which
// is also the classifier), then the gains (per layer rms_att, rms_ffn; then rms_final). Adam
// is two launches, one per region (weight decay applies to the matrices and the embedding,
// not to the gains: train_full.go:909-919, :955-956).
//
// The reference's shortcuts are kept, since the step must match it:
//   - attention backward (train_full.go:247-301) gives gradients of the post-RoPE q and k,
//     which feed the projections' gradients without being rotated back;
//   - the RMSNorm backward (rmsnorm.go:32-47) multiplies its x.dot term by the gain;
//   - the classifier's embedding gradient covers only the rows of the window's target ids
//     (compactEmbedGrad, train_full.go:525-587).
#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "sh_internal.hpp"
#include "sh_wave.hpp"

namespace sh {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kTT = 256;   // threads of the row kernels

// ---- fp32 MFMA GEMM ----------------------------------------------------------------------
// C[M, N] = sum_k A(m, k) B(k, n) with A(m, k) = A[m*lda + k] (AK) or A[k*lda + m], and
// B(k, n) = B[n*ldb + k] (BK) or B[k*ldb + n]. Epilogue: EPI_STORE C = alpha*acc,
// EPI_RESID C = R + alpha*acc (R row-major with ldc). 64 x 64 tiles of 2 x 2 waves, K in
// blocks of 16 staged through LDS as [k][m] / [k][n] rows (padded by 16 floats, so the 16
// lanes of one MFMA operand read and the four k rows hit distinct banks), the next block
// loaded into registers while the current one is consumed. v_mfma_f32_16x16x4_f32 operands:
// lane l holds A[row l%16][k l/16] and B[k l/16][column l%16]; the result rows
// 4*(l/16) + r of column l%16. Leading dimensions and the base pointers are multiples of 4
// floats; tails in M, N and K are zero-filled.
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_PART = 2 };
constexpr int kGM = 64, kGN = 64, kGK = 16, kGP = 16;

template <bool AK>
__device__ __forceinline__ f32x4 gemm_load(const float *A, int lda, int rows, int K, int r0, int k0,
                                           int tid) {
    // AK: thread -> (row r0 + tid/4, k k0 + 4*(tid%4) .. +3); else (k k0 + tid/16, rows 4*(tid%16) ..)
    int r, k;
    if constexpr (AK) {
        r = r0 + tid / 4;
        k = k0 + (tid % 4) * 4;
        if (r < rows && k + 3 < K) return *(const f32x4 *)(A + (size_t)r * lda + k);
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (r < rows)
            for (int e = 0; e < 4; e++)
                if (k + e < K) v[e] = A[(size_t)r * lda + k + e];
        return v;
    } else {
        k = k0 + tid / 16;
        r = r0 + (tid % 16) * 4;
        if (k < K && r + 3 < rows) return *(const f32x4 *)(A + (size_t)k * lda + r);
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (k < K)
            for (int e = 0; e < 4; e++)
                if (r + e < rows) v[e] = A[(size_t)k * lda + r + e];
        return v;
    }
}

template <bool AK>
__device__ __forceinline__ void gemm_stage(float (*S)[kGM + kGP], f32x4 v, int tid) {
    if constexpr (AK) {
        const int r = tid / 4, k = (tid % 4) * 4;
        for (int e = 0; e < 4; e++) S[k + e][r] = v[e];
    } else {
        *(f32x4 *)&S[tid / 16][(tid % 16) * 4] = v;
    }
}

template <bool AK, bool BK, int EPI>
__global__ __launch_bounds__(256) void k_sgemm(const float *A, int lda, const float *B, int ldb,
                                               float *C, int ldc, int M, int N, int K, float alpha,
                                               const float *R, int kc) {
    __shared__ __attribute__((aligned(16))) float As[2][kGK][kGM + kGP];
    __shared__ __attribute__((aligned(16))) float Bs[2][kGK][kGN + kGP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    const int m0 = blockIdx.y * kGM, n0 = blockIdx.x * kGN;
    f32x4 acc[2][2];
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    // workgroup z covers k in [z*kc, min(K, (z+1)*kc)) (EPI_PART: one partial tile per z)
    const int kb = blockIdx.z * kc, ke = min(K, kb + kc);
    K = ke;
    f32x4 ra = gemm_load<AK>(A, lda, M, K, m0, kb, tid);
    f32x4 rb = gemm_load<BK>(B, ldb, N, K, n0, kb, tid);
    gemm_stage<AK>(As[0], ra, tid);
    gemm_stage<BK>(Bs[0], rb, tid);
    __syncthreads();
    int buf = 0;
    const int lr = lane & 15, lk = lane >> 4;
    for (int k0 = kb; k0 < K; k0 += kGK) {
        const bool more = k0 + kGK < K;
        if (more) {
            ra = gemm_load<AK>(A, lda, M, K, m0, k0 + kGK, tid);
            rb = gemm_load<BK>(B, ldb, N, K, n0, k0 + kGK, tid);
        }
#pragma unroll
        for (int kk = 0; kk < kGK; kk += 4) {
            const float a0 = As[buf][kk + lk][wm + lr], a1 = As[buf][kk + lk][wm + 16 + lr];
            const float b0 = Bs[buf][kk + lk][wn + lr], b1 = Bs[buf][kk + lk][wn + 16 + lr];
            acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, acc[1][1], 0, 0, 0);
        }
        if (more) {
            gemm_stage<AK>(As[buf ^ 1], ra, tid);
            gemm_stage<BK>(Bs[buf ^ 1], rb, tid);
        }
        __syncthreads();
        buf ^= 1;
    }
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++) {
            const int n = n0 + wn + j * 16 + lr;
            if (n >= N) continue;
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm + i * 16 + lk * 4 + r;
                if (m >= M) continue;
                const size_t o = (size_t)m * ldc + n;
                if constexpr (EPI == EPI_STORE) C[o] = alpha * acc[i][j][r];
                else if constexpr (EPI == EPI_RESID) C[o] = R[o] + alpha * acc[i][j][r];
                else C[(size_t)blockIdx.z * M * ldc + o] = acc[i][j][r];
            }
        }
}

// s_waitcnt immediate that waits until at most n vector memory operations of the wave are
// outstanding (gfx9 encoding: vmcnt bits 3:0 and 15:14; expcnt and lgkmcnt not waited for).
constexpr int sg_vm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// k_sgemm for tile-aligned shapes (M, N multiples of 64, every K range a multiple of 128),
// pipelined: the A and B tiles of each 32-k block (two 16-k sub-blocks) stream into a
// kSgNs-deep LDS ring by global_load_lds (each lane moves 16 bytes straight into LDS, a wave
// instruction fills 1 KB; waves 0-1 load A, waves 2-3 load B), so kSgNs - 1 blocks are always
// in flight. One barrier per block: wait for this wave's loads of block s (explicit vmcnt; the
// fence of __syncthreads would wait for every load in flight), s_barrier, issue block
// s + kSgNs - 1 into the slot block s - 1 used, MFMAs of block s. (Reading block s + 1's
// operands into a second register set during block s's MFMAs, with every iteration issuing
// one block, was slower: 4.43 against 4.26 ms per Stories110M S = 256 step; one 16-k
// block per slot in 6 slots took 4.26 ms, two per slot in 4 slots 4.24.)
// LDS layouts of each 16-k sub-tile, chosen so the MFMA reads spread over the banks:
//  k-contiguous operand (rows of the tile along m or n, 64 bytes of k each): 16-byte chunk c
//    of row r in slot c ^ ((r >> 1) & 3);
//  otherwise (rows along k, 256 bytes of m or n each): chunk c of k-row r in slot
//    c ^ (4 * ((r >> 2) & 3)).
// Within a sub-block, MFMA step j (of 4) has lane group l (lane / 16) on k = 4l + j, so a
// k-contiguous operand gives each lane its four steps' values in one 16-byte read. The
// products are fp32 and exact as in k_sgemm; only the order of the fp32 sums differs.
constexpr int kSgNs = 4, kSgKb = 16, kSgH = 2;   // ring slots; k per sub-block; sub-blocks per slot
template <bool XK>
__device__ __forceinline__ float sg_read(const uint8_t *T, int r, int j, int lk) {
    if constexpr (XK) {
        return ((const float *)(T + r * 64 + ((lk ^ ((r >> 1) & 3)) << 4)))[j];
    } else {
        const int k = 4 * lk + j;
        return ((const float *)(T + k * 256 + (((r >> 2) ^ (4 * ((k >> 2) & 3))) << 4)))[r & 3];
    }
}

template <bool AK, bool BK, int EPI>
__global__ __launch_bounds__(256) void k_sgemm_pipe(const float *A, int lda, const float *B, int ldb, float *C,
                                                    int ldc, int M, int N, int K, float alpha, const float *R,
                                                    int kc) {
    constexpr int TB = kGM * kSgKb * 4;   // bytes of one operand sub-tile (4 KB)
    constexpr int SB = 2 * kSgH * TB;     // a slot: the A sub-tiles, then the B sub-tiles
    __shared__ __attribute__((aligned(16))) uint8_t lds[kSgNs * SB];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    const int m0 = blockIdx.y * kGM, n0 = blockIdx.x * kGN;
    const int kb = blockIdx.z * kc, ke = min(K, kb + kc);
    const int nsteps = (ke - kb) / (kSgKb * kSgH);
    // this wave's two instructions per sub-block: operand X (A for waves 0-1, B for 2-3), tile
    // instructions q = 2 * (wave & 1) + i
    const bool isa = wave < 2;
    const bool xk = isa ? AK : BK;
    const float *X = isa ? A : B;
    const int ld = isa ? lda : ldb, r0 = isa ? m0 : n0;
    const float *src[2];
    int dst[2];
    size_t step[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int q = 2 * (wave & 1) + i;
        if (xk) {
            const int r = q * 16 + lane / 4, c = (lane % 4) ^ ((r >> 1) & 3);
            src[i] = X + (size_t)(r0 + r) * ld + kb + c * 4;
            step[i] = kSgKb;
        } else {
            const int kr = q * 4 + lane / 16, c = (lane % 16) ^ (4 * ((kr >> 2) & 3));
            src[i] = X + (size_t)(kb + kr) * ld + r0 + c * 4;
            step[i] = (size_t)kSgKb * ld;
        }
        dst[i] = (isa ? 0 : kSgH * TB) + q * 1024;
    }
    auto issue = [&](int st, int slot) {   // block st (kSgH sub-blocks) into ring slot `slot`
        uint8_t *base = lds + slot * SB;
#pragma unroll
        for (int h = 0; h < kSgH; h++)
#pragma unroll
            for (int i = 0; i < 2; i++)
                __builtin_amdgcn_global_load_lds(
                    (const __attribute__((address_space(1))) void *)(src[i] + (size_t)(st * kSgH + h) * step[i]),
                    (__attribute__((address_space(3))) void *)(base + h * TB + dst[i]), 16, 0, 0);
    };
    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int lr = lane & 15, lk = lane >> 4;
    auto compute = [&](int st) {
#pragma unroll
      for (int h = 0; h < kSgH; h++) {
        const uint8_t *TA = lds + (st % kSgNs) * SB + h * TB, *TBp = TA + kSgH * TB;
        float a[2][4], b[2][4];
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                a[i][j] = sg_read<AK>(TA, wm + i * 16 + lr, j, lk);
                b[i][j] = sg_read<BK>(TBp, wn + i * 16 + lr, j, lk);
            }
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int jj = 0; jj < 2; jj++)
                    acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][j], b[jj][j], acc[i][jj], 0, 0, 0);
      }
    };
#pragma unroll
    for (int st = 0; st < kSgNs - 1; st++) issue(st, st);
    int st = 0;
    for (; st < nsteps - (kSgNs - 1); st++) {
        __builtin_amdgcn_s_waitcnt(sg_vm_wait((kSgNs - 2) * 2 * kSgH));
        __builtin_amdgcn_s_barrier();
        issue(st + kSgNs - 1, (st + kSgNs - 1) % kSgNs);
        compute(st);
    }
    __builtin_amdgcn_s_waitcnt(sg_vm_wait(0));
    __builtin_amdgcn_s_barrier();
    for (; st < nsteps; st++) compute(st);
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++) {
            const int n = n0 + wn + j * 16 + lr;
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm + i * 16 + lk * 4 + r;
                const size_t o = (size_t)m * ldc + n;
                if constexpr (EPI == EPI_STORE) C[o] = alpha * acc[i][j][r];
                else if constexpr (EPI == EPI_RESID) C[o] = R[o] + alpha * acc[i][j][r];
                else C[(size_t)blockIdx.z * M * ldc + o] = acc[i][j][r];
            }
        }
}

// C = alpha * (sum over the K ranges in order of the partial tiles [ranges][M][ldc]), plus R
// when it is given (the residual epilogue).
__global__ void k_tr_reduce_ranges(const float *P, int ranges, int M, int N, int ldc, float alpha, const float *R,
                                   float *C) {
    const size_t n = (size_t)M * N;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (size_t)gridDim.x * blockDim.x) {
        const size_t m = e / N, c = e % N, o = m * ldc + c;
        float v = 0.f;
        for (int z = 0; z < ranges; z++) v += P[(size_t)z * M * ldc + o];
        C[o] = R ? R[o] + alpha * v : alpha * v;
    }
}

// ---- row kernels -------------------------------------------------------------------------

__device__ __forceinline__ double block_sum_d(double v, double *red) {
    v = wsum_d64(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double s = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) s += red[w];
    return s;
}

// cpu.go:41-72 EmbedLookup, token-major: out-of-range ids give a zero row.
__global__ void k_tr_embed(const float *embed, const uint16_t *tok, int vocab, int D, float *x) {
    const int t = blockIdx.x, id = tok[t];
    for (int i = threadIdx.x; i < D; i += blockDim.x)
        x[(size_t)t * D + i] = id < vocab ? embed[(size_t)id * D + i] : 0.f;
}

// accel_other.go:11-28 rmsNormCFWithRRMSImpl per row: float64 sum of squares, float32 scale,
// out = x*scale*w; the scale is kept for the backward.
__global__ __launch_bounds__(kTT) void k_tr_rmsnorm(const float *x, const float *w, int D, double eps,
                                                    float *out, float *rrms) {
    __shared__ double red[kTT / 64];
    const float *row = x + (size_t)blockIdx.x * D;
    double ss = 0;
    for (int i = threadIdx.x; i < D; i += blockDim.x) ss += (double)row[i] * (double)row[i];
    const double tot = block_sum_d(ss, red);
    const float scale = (float)(1.0 / sqrt(tot / (double)D + eps));
    if (threadIdx.x == 0) rrms[blockIdx.x] = scale;
    for (int i = threadIdx.x; i < D; i += blockDim.x)
        out[(size_t)blockIdx.x * D + i] = row[i] * scale * w[i];
}

// rope.go:26-46 on the q and k parts of row t of qkv [S, 3D] (e' = e*c - o*s, o' = o*c + e*s).
// A split product's K-range partials ([ranges][rows][ld]) handed to the forward row kernel
// that consumes the product instead of a separate sum: Y = R + alpha * (partials summed in
// range order), R optional — k_tr_reduce_ranges' arithmetic. p == nullptr: none.
struct PartIn {
    const float *p;
    int ranges;
    size_t stride;   // floats per range
    const float *R;
    float alpha;
};
__device__ __forceinline__ void sum_part_row(const PartIn &q, int t, int ld, int n, float *y) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const size_t o = (size_t)t * ld + i;
        float v = 0.f;
        for (int z = 0; z < q.ranges; z++) v += q.p[(size_t)z * q.stride + o];
        y[o] = q.R ? q.R[o] + q.alpha * v : q.alpha * v;
    }
}
constexpr int kPT = 1024;   // threads of the row kernels that sum partials
// k_tr_rmsnorm on row t of Y (written to x first)
__global__ __launch_bounds__(kPT) void k_tr_rmsnorm_part(float *x, const float *w, int D, double eps, float *out,
                                                         float *rrms, PartIn q) {
    __shared__ double red[kPT / 64];
    sum_part_row(q, blockIdx.x, D, D, x);   // each thread re-reads only its own columns below
    const float *row = x + (size_t)blockIdx.x * D;
    double ss = 0;
    for (int i = threadIdx.x; i < D; i += blockDim.x) ss += (double)row[i] * (double)row[i];
    const double tot = block_sum_d(ss, red);
    const float scale = (float)(1.0 / sqrt(tot / (double)D + eps));
    if (threadIdx.x == 0) rrms[blockIdx.x] = scale;
    for (int i = threadIdx.x; i < D; i += blockDim.x)
        out[(size_t)blockIdx.x * D + i] = row[i] * scale * w[i];
}
__global__ void k_tr_rope(float *qkv, int D, int hd, const float *cs, const float *sn);
// k_tr_rope on row t of the q|k|v product (summed into qkv first)
__global__ __launch_bounds__(kPT) void k_tr_rope_part(float *qkv, int D, int hd, const float *cs, const float *sn,
                                                      PartIn q) {
    const int t = blockIdx.x, half = hd / 2;
    sum_part_row(q, t, 3 * D, 3 * D, qkv);
    __syncthreads();
    for (int p = threadIdx.x; p < D; p += blockDim.x) {
        const int col = 2 * p, i = (col % hd) / 2;
        const float c = cs[t * half + i], s = sn[t * half + i];
        float *e = qkv + (size_t)t * 3 * D + col;
        const float ev = e[0], ov = e[1];
        e[0] = ev * c - ov * s;
        e[1] = ov * c + ev * s;
    }
}
__global__ void k_tr_rope(float *qkv, int D, int hd, const float *cs, const float *sn) {
    const int t = blockIdx.x, half = hd / 2;
    for (int p = threadIdx.x; p < D; p += blockDim.x) {   // D pairs: D/2 in q, D/2 in k
        const int col = 2 * p, i = (col % hd) / 2;
        const float c = cs[t * half + i], s = sn[t * half + i];
        float *e = qkv + (size_t)t * 3 * D + col;
        const float ev = e[0], ov = e[1];
        e[0] = ev * c - ov * s;
        e[1] = ov * c + ev * s;
    }
}

// forward_common.go:5-33 causalAttentionCF for (query t, head h), one wave: float32 scores
// summed over the head dims in order, softmax with float64 exp terms and sum (masked keys
// weigh exactly 0), then att[t] = sum over keys in order of p*v.
__global__ __launch_bounds__(64) void k_tr_attn_fwd(const float *qkv, int S, int D, int hd, float scale,
                                                    float *att) {
    extern __shared__ float sc[];
    const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const size_t ld = 3 * (size_t)D;
    const float *q = qkv + (size_t)t * ld + h * hd;
    float mx = -INFINITY;
    for (int s = lane; s <= t; s += 64) {
        const float *k = qkv + (size_t)s * ld + D + h * hd;
        float sum = 0.f;
        for (int i = 0; i < hd; i++) sum += q[i] * k[i];
        sum *= scale;
        sc[s] = sum;
        mx = fmaxf(mx, sum);
    }
    mx = wmax<64>(mx);
    double tot = 0;
    for (int s = lane; s <= t; s += 64) {
        const double e = exp((double)(sc[s] - mx));
        sc[s] = (float)e;
        tot += e;
    }
    tot = wsum_d64(tot);
    const float inv = (float)(1.0 / tot);
    __syncthreads();
    for (int s = lane; s <= t; s += 64) sc[s] *= inv;
    __syncthreads();
    if (lane < hd) {
        float a = 0.f;
        for (int s = 0; s <= t; s++) a += sc[s] * qkv[(size_t)s * ld + 2 * D + h * hd + lane];
        att[(size_t)t * D + h * hd + lane] = a;
    }
}

// train_full.go:247-301 for query t, head h: the row's probabilities recomputed as the
// reference does (float32 scores, max over s <= t, float64 exp and total, float32 inverse),
// dscore_s = dOut[t] . v[s], dsSum = sum_s p_s*dscore_s (in s order), ds_s =
// p_s*(dscore_s - dsSum)*scale, dq[t] = sum_s ds_s*k[s]. The row's max, inverse total and
// dsSum go to `stats` for the key-side kernel.
__global__ __launch_bounds__(64) void k_tr_attn_bwd_q(const float *qkv, const float *dout, int S, int D,
                                                      int hd, float scale, float *dqkv, float *stats) {
    extern __shared__ float sh[];
    float *pr = sh, *dsc = sh + S;
    const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x, H = D / hd;
    const size_t ld = 3 * (size_t)D;
    const float *q = qkv + (size_t)t * ld + h * hd;
    const float *go = dout + (size_t)t * D + h * hd;
    float mx = -INFINITY;
    for (int s = lane; s <= t; s += 64) {
        const float *k = qkv + (size_t)s * ld + D + h * hd;
        const float *v = qkv + (size_t)s * ld + 2 * D + h * hd;
        float sum = 0.f, dot = 0.f;
        for (int i = 0; i < hd; i++) sum += q[i] * k[i];
        for (int i = 0; i < hd; i++) dot += go[i] * v[i];
        sum *= scale;
        pr[s] = sum;
        dsc[s] = dot;
        mx = fmaxf(mx, sum);
    }
    mx = wmax<64>(mx);
    double tot = 0;
    for (int s = lane; s <= t; s += 64) {
        const double e = exp((double)(pr[s] - mx));
        pr[s] = (float)e;
        tot += e;
    }
    tot = wsum_d64(tot);
    const float inv = (float)(1.0 / tot);
    __syncthreads();
    for (int s = lane; s <= t; s += 64) pr[s] *= inv;
    __syncthreads();
    __shared__ float dss_sh;
    if (lane == 0) {
        float d = 0.f;
        for (int s = 0; s <= t; s++) d += pr[s] * dsc[s];
        dss_sh = d;
        float *st = stats + ((size_t)h * S + t) * 3;
        st[0] = mx;
        st[1] = inv;
        st[2] = d;
    }
    __syncthreads();
    const float dss = dss_sh;
    for (int s = lane; s <= t; s += 64) dsc[s] = pr[s] * (dsc[s] - dss) * scale;
    __syncthreads();
    if (lane < hd) {
        float a = 0.f;
        for (int s = 0; s <= t; s++) a += dsc[s] * qkv[(size_t)s * ld + D + h * hd + lane];
        dqkv[(size_t)t * ld + h * hd + lane] = a;
    }
    (void)H;
}

// Key side of train_full.go:247-301 for key s, head h: for every query t >= s the same p and
// ds as k_tr_attn_bwd_q (same operation order, from the row stats), then dk[s] = sum over t
// in order of ds*q[t] and dv[s] = sum over t in order of p*dOut[t].
__global__ __launch_bounds__(64) void k_tr_attn_bwd_kv(const float *qkv, const float *dout, int S, int D,
                                                       int hd, float scale, const float *stats,
                                                       float *dqkv) {
    extern __shared__ float sh[];
    float *pr = sh, *ds = sh + S;
    const int s = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const size_t ld = 3 * (size_t)D;
    const float *k = qkv + (size_t)s * ld + D + h * hd;
    const float *v = qkv + (size_t)s * ld + 2 * D + h * hd;
    for (int t = s + lane; t < S; t += 64) {
        const float *q = qkv + (size_t)t * ld + h * hd;
        const float *go = dout + (size_t)t * D + h * hd;
        float sum = 0.f, dot = 0.f;
        for (int i = 0; i < hd; i++) sum += q[i] * k[i];
        for (int i = 0; i < hd; i++) dot += go[i] * v[i];
        sum *= scale;
        const float *st = stats + ((size_t)h * S + t) * 3;
        const float p = (float)exp((double)(sum - st[0])) * st[1];
        pr[t] = p;
        ds[t] = p * (dot - st[2]) * scale;
    }
    __syncthreads();
    if (lane < hd) {
        float dk = 0.f, dv = 0.f;
        for (int t = s; t < S; t++) {
            dk += ds[t] * qkv[(size_t)t * ld + h * hd + lane];
            dv += pr[t] * dout[(size_t)t * D + h * hd + lane];
        }
        dqkv[(size_t)s * ld + D + h * hd + lane] = dk;
        dqkv[(size_t)s * ld + 2 * D + h * hd + lane] = dv;
    }
}

// ---- blocked attention (S <= kAttnMaxS): 16 rows of one head per workgroup, 64-row
// blocks staged in LDS; each dot product and each sum over keys or queries runs in the
// reference's order, so the results equal the one-wave-per-row kernels above.
constexpr int kAQ = 16;          // queries (or keys) per workgroup
constexpr int kAB = 64;          // rows per staged block
constexpr int kAttnMaxS = 256;   // score rows kept in LDS: 2 x 16 x (S + 16) floats (<= 64 KB dynamic)
constexpr int kAPad = 68;        // LDS row stride (floats) of a staged block: 16-byte rows, and
                                 // 16 rows 4 banks apart for the float4 reads
constexpr int kSPad = 16;        // extra floats per score row in LDS: the four rows a wave
                                 // touches start 16 banks apart instead of on one bank

// sum over i in order of a[i]*b[i] (float32, no fusing), four at a time from LDS (hd % 4 == 0)
__device__ __forceinline__ float dot_lds(const float *a, const float *b, int hd) {
    float sum = 0.f;
#pragma unroll 4
    for (int i = 0; i < hd; i += 4) {
        const f32x4 x = *(const f32x4 *)(a + i), y = *(const f32x4 *)(b + i);
        sum += x.x * y.x;
        sum += x.y * y.y;
        sum += x.z * y.z;
        sum += x.w * y.w;
    }
    return sum;
}

// float64 sum over the 16 lanes of a row group (each holding one value), uniform result.
__device__ __forceinline__ double sum16_d64(double v) {
    auto step = [](double x, auto ctrl_tag) {
        constexpr int Cc = decltype(ctrl_tag)::value;
        const uint64_t b = (uint64_t)__double_as_longlong(x);
        const uint32_t lo = dpp_u<Cc>((uint32_t)b), hi = dpp_u<Cc>((uint32_t)(b >> 32));
        return x + __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
    };
    v = step(v, std::integral_constant<int, kDppXor1>{});
    v = step(v, std::integral_constant<int, kDppXor2>{});
    v = step(v, std::integral_constant<int, kDppHalfMirror>{});
    v = step(v, std::integral_constant<int, kDppMirror>{});
    return v;
}

// Stages rows r0 .. r0+nr-1 (nr <= 64; rows at or past n skipped, or zero-filled when
// `zero`) of columns c0 .. c0+hd-1 of a row-major matrix (row stride ld, hd % 4 == 0) into
// LDS [nr][kAPad]: every thread issues its (at most four) 16-byte loads before any LDS store,
// so the loads are in flight together. blockDim.x == 256.
__device__ __forceinline__ void stage_rows(float *dst, const float *src, size_t ld, int c0, int r0, int n, int hd,
                                           int nr = kAB, bool zero = false) {
    const int per = hd / 4, total = nr * per;   // total <= 1024
    f32x4 v[4];
    int rr[4], cc[4];
    bool ok[4], in[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int e = threadIdx.x + 256 * k;
        rr[k] = e / per;
        cc[k] = (e % per) * 4;
        in[k] = e < total;
        ok[k] = in[k] && r0 + rr[k] < n;
        v[k] = ok[k] ? *(const f32x4 *)(src + (size_t)(r0 + rr[k]) * ld + c0 + cc[k]) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int k = 0; k < 4; k++)
        if (ok[k] || (zero && in[k])) *(f32x4 *)(dst + rr[k] * kAPad + cc[k]) = v[k];
}

// Forward for queries q0 .. q0+15 of head h (forward_common.go:5-33 order): scores per
// (query, key) summed over the head dims in order, row softmax (float64 exp and total,
// float32 inverse), att = sum over keys in order of p*v.
__global__ __launch_bounds__(256) void k_tr_attn_fwd_blk(const float *qkv, int S, int D, int hd, float scale,
                                                         float *att) {
    extern __shared__ __attribute__((aligned(16))) float sh[];
    float *qs = sh, *kv = qs + kAQ * kAPad, *sc = kv + kAB * kAPad;   // sc [16][S]
    const int q0 = blockIdx.x * kAQ, h = blockIdx.y, tid = threadIdx.x;
    const size_t ld = 3 * (size_t)D;
    const int qn = min(kAQ, S - q0), kend = min(S, q0 + kAQ);   // keys 0 .. kend-1
    const int SP = S + kSPad;
    stage_rows(qs, qkv, ld, h * hd, q0, S, hd, kAQ, true);
    const int q = tid / 16, j = tid % 16, t = q0 + q;
    for (int kb = 0; kb < kend; kb += kAB) {
        __syncthreads();
        stage_rows(kv, qkv, ld, D + h * hd, kb, kend, hd);
        __syncthreads();
        for (int u = 0; u < kAB / 16; u++) {
            const int s = kb + j + 16 * u;
            if (s < kend && q < qn && s <= t) sc[q * SP + s] = dot_lds(qs + q * kAPad, kv + (s - kb) * kAPad, hd) * scale;
        }
    }
    __syncthreads();
    // softmax of row q over keys 0..t: the 16 lanes of the row group share it
    float mx = -INFINITY;
    if (q < qn)
        for (int s = j; s <= t; s += 16) mx = fmaxf(mx, sc[q * SP + s]);
    mx = wmax<16>(mx);
    double tot = 0;
    if (q < qn)
        for (int s = j; s <= t; s += 16) {
            const double ev = exp((double)(sc[q * SP + s] - mx));
            sc[q * SP + s] = (float)ev;
            tot += ev;
        }
    tot = sum16_d64(tot);
    const float inv = (float)(1.0 / tot);
    if (q < qn)
        for (int s = j; s <= t; s += 16) sc[q * SP + s] *= inv;
    // P.V: thread (q, dims j, j+16, ...) sums over keys in order
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    for (int kb = 0; kb < kend; kb += kAB) {
        __syncthreads();
        stage_rows(kv, qkv, ld, 2 * D + h * hd, kb, kend, hd);
        __syncthreads();
        if (q < qn) {
            const int se = min(t + 1, min(kend, kb + kAB));
#pragma unroll 4
            for (int s = kb; s < se; s++) {
                const float p = sc[q * SP + s];
                for (int c = 0; c < 4; c++)
                    if (j + 16 * c < hd) a[c] += p * kv[(s - kb) * kAPad + j + 16 * c];
            }
        }
    }
    if (q < qn)
        for (int c = 0; c < 4; c++)
            if (j + 16 * c < hd) att[(size_t)t * D + h * hd + j + 16 * c] = a[c];
}

// Query side of train_full.go:247-301 for queries q0 .. q0+15 of head h, in the reference's
// order (see k_tr_attn_bwd_q); writes dq and the row stats.
__global__ __launch_bounds__(256) void k_tr_attn_bwd_q_blk(const float *qkv, const float *dout, int S, int D,
                                                           int hd, float scale, float *dqkv, float *stats) {
    extern __shared__ __attribute__((aligned(16))) float sh[];
    float *qs = sh, *gs = qs + kAQ * kAPad, *kv = gs + kAQ * kAPad, *pr = kv + kAB * kAPad, *dsc = pr + kAQ * (S + kSPad);
    __shared__ float dss_sh[kAQ];
    const int q0 = blockIdx.x * kAQ, h = blockIdx.y, tid = threadIdx.x;
    const size_t ld = 3 * (size_t)D;
    const int qn = min(kAQ, S - q0), kend = min(S, q0 + kAQ);
    const int SP = S + kSPad;
    stage_rows(qs, qkv, ld, h * hd, q0, S, hd, kAQ, true);
    stage_rows(gs, dout, D, h * hd, q0, S, hd, kAQ, true);
    const int q = tid / 16, j = tid % 16, t = q0 + q;
    for (int kb = 0; kb < kend; kb += kAB) {   // scores (K blocks), then dscores (V blocks)
        __syncthreads();
        stage_rows(kv, qkv, ld, D + h * hd, kb, kend, hd);
        __syncthreads();
        for (int u = 0; u < kAB / 16; u++) {
            const int s = kb + j + 16 * u;
            if (s < kend && q < qn && s <= t) pr[q * SP + s] = dot_lds(qs + q * kAPad, kv + (s - kb) * kAPad, hd) * scale;
        }
        __syncthreads();
        stage_rows(kv, qkv, ld, 2 * D + h * hd, kb, kend, hd);
        __syncthreads();
        for (int u = 0; u < kAB / 16; u++) {
            const int s = kb + j + 16 * u;
            if (s < kend && q < qn && s <= t) dsc[q * SP + s] = dot_lds(gs + q * kAPad, kv + (s - kb) * kAPad, hd);
        }
    }
    __syncthreads();
    float mx = -INFINITY;
    if (q < qn)
        for (int s = j; s <= t; s += 16) mx = fmaxf(mx, pr[q * SP + s]);
    mx = wmax<16>(mx);
    double tot = 0;
    if (q < qn)
        for (int s = j; s <= t; s += 16) {
            const double ev = exp((double)(pr[q * SP + s] - mx));
            pr[q * SP + s] = (float)ev;
            tot += ev;
        }
    tot = sum16_d64(tot);
    const float inv = (float)(1.0 / tot);
    if (q < qn)
        for (int s = j; s <= t; s += 16) pr[q * SP + s] *= inv;
    __syncthreads();
    if (j == 0 && q < qn) {   // dsSum in key order
        float d = 0.f;
#pragma unroll 8
        for (int s = 0; s <= t; s++) d += pr[q * SP + s] * dsc[q * SP + s];
        dss_sh[q] = d;
        float *st = stats + ((size_t)h * S + t) * 3;
        st[0] = mx;
        st[1] = inv;
        st[2] = d;
    }
    __syncthreads();
    if (q < qn) {
        const float dss = dss_sh[q];
        for (int s = j; s <= t; s += 16) dsc[q * SP + s] = pr[q * SP + s] * (dsc[q * SP + s] - dss) * scale;
    }
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    for (int kb = 0; kb < kend; kb += kAB) {   // dq = sum over keys in order of ds*k
        __syncthreads();
        stage_rows(kv, qkv, ld, D + h * hd, kb, kend, hd);
        __syncthreads();
        if (q < qn) {
            const int se = min(t + 1, min(kend, kb + kAB));
#pragma unroll 4
            for (int s = kb; s < se; s++) {
                const float d = dsc[q * SP + s];
                for (int c = 0; c < 4; c++)
                    if (j + 16 * c < hd) a[c] += d * kv[(s - kb) * kAPad + j + 16 * c];
            }
        }
    }
    if (q < qn)
        for (int c = 0; c < 4; c++)
            if (j + 16 * c < hd) dqkv[(size_t)t * ld + h * hd + j + 16 * c] = a[c];
}

// Key side for keys s0 .. s0+15 of head h (see k_tr_attn_bwd_kv): query blocks of 64 in
// ascending order, p and ds per (key, query) from the row stats, then dk and dv summed over
// queries in order.
__global__ __launch_bounds__(256) void k_tr_attn_bwd_kv_blk(const float *qkv, const float *dout, int S, int D,
                                                            int hd, float scale, const float *stats,
                                                            float *dqkv) {
    __shared__ __attribute__((aligned(16))) float ks[kAQ * kAPad], vs[kAQ * kAPad], qb[kAB * kAPad], gb[kAB * kAPad];
    __shared__ float pp[kAQ][kAB + kSPad], dd[kAQ][kAB + kSPad];
    const int s0 = blockIdx.x * kAQ, h = blockIdx.y, tid = threadIdx.x;
    const size_t ld = 3 * (size_t)D;
    const int sn = min(kAQ, S - s0);
    stage_rows(ks, qkv, ld, D + h * hd, s0, S, hd, kAQ, true);
    stage_rows(vs, qkv, ld, 2 * D + h * hd, s0, S, hd, kAQ, true);
    const int kk = tid / 16, j = tid % 16, s = s0 + kk;
    float dk[4] = {0.f, 0.f, 0.f, 0.f}, dv[4] = {0.f, 0.f, 0.f, 0.f};
    for (int tb = s0 - s0 % kAB; tb < S; tb += kAB) {
        __syncthreads();
        stage_rows(qb, qkv, ld, h * hd, tb, S, hd);
        stage_rows(gb, dout, D, h * hd, tb, S, hd);
        __syncthreads();
        for (int u = 0; u < kAB / 16; u++) {
            const int tl = j + 16 * u, t = tb + tl;
            float p = 0.f, d = 0.f;
            if (kk < sn && t < S && t >= s) {
                const float sum = dot_lds(qb + tl * kAPad, ks + kk * kAPad, hd) * scale;
                const float dot = dot_lds(gb + tl * kAPad, vs + kk * kAPad, hd);
                const float *st = stats + ((size_t)h * S + t) * 3;
                p = (float)exp((double)(sum - st[0])) * st[1];
                d = p * (dot - st[2]) * scale;
            }
            pp[kk][tl] = p;
            dd[kk][tl] = d;
        }
        __syncthreads();
        if (kk < sn) {
            const int tl0 = max(0, s - tb), tl1 = min(kAB, S - tb);
#pragma unroll 4
            for (int tl = tl0; tl < tl1; tl++) {
                const float p = pp[kk][tl], d = dd[kk][tl];
                for (int c = 0; c < 4; c++)
                    if (j + 16 * c < hd) {
                        dk[c] += d * qb[tl * kAPad + j + 16 * c];
                        dv[c] += p * gb[tl * kAPad + j + 16 * c];
                    }
            }
        }
    }
    if (kk < sn)
        for (int c = 0; c < 4; c++)
            if (j + 16 * c < hd) {
                dqkv[(size_t)s * ld + D + h * hd + j + 16 * c] = dk[c];
                dqkv[(size_t)s * ld + 2 * D + h * hd + j + 16 * c] = dv[c];
            }
}

// accel_other.go:70-75 siluGateForwardAccel on row t of h13 = [h1 | h3] ([S, 2F]).
__global__ void k_tr_silu_gate(const float *h13, int F, size_t n, float *gate) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const size_t t = i / F, j = i % F;
        const float h1 = h13[t * 2 * F + j], h3 = h13[t * 2 * F + F + j];
        const float sig = (float)(1.0 / (1.0 + exp(-(double)h1)));
        gate[i] = (h1 * sig) * h3;
    }
}

// accel_other.go:77-84 siluBackwardAccel: dh13 = [dh1 | dh3] per row.
__global__ void k_tr_silu_bwd(const float *dgate, const float *h13, int F, size_t n, float *dh13) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const size_t t = i / F, j = i % F;
        const float h1 = h13[t * 2 * F + j], h3 = h13[t * 2 * F + F + j];
        const float sig = (float)(1.0 / (1.0 + exp(-(double)h1)));
        const float sg = sig * (1 + h1 * (1 - sig));
        dh13[t * 2 * F + j] = dgate[i] * h3 * sg;
        dh13[t * 2 * F + F + j] = dgate[i] * (h1 * sig);
    }
}

// rmsnorm.go:32-47 per row: dot = sum_i dy*x*w (float64), dx = (dy - x*dot*r^2/D)*r*w in float64
// rounded once.
// addend given: dx = addend + the gradient (the backward's residual add, the gradient rounded
// to float32 first as when it is stored and then added).
__global__ __launch_bounds__(kTT) void k_tr_rms_bwd_dx(const float *dy, const float *x, const float *w,
                                                       const float *rrms, int D, float *dx,
                                                       const float *addend = nullptr) {
    __shared__ double red[kTT / 64];
    const size_t o = (size_t)blockIdx.x * D;
    double dot = 0;
    for (int i = threadIdx.x; i < D; i += blockDim.x) dot += (double)(dy[o + i] * x[o + i] * w[i]);
    dot = block_sum_d(dot, red);
    const double r = (double)rrms[blockIdx.x], r2 = (r * r) / (double)D;
    for (int i = threadIdx.x; i < D; i += blockDim.x) {
        const double v = (double)dy[o + i] - (double)x[o + i] * dot * r2;
        const float g = (float)(v * r * (double)w[i]);
        dx[o + i] = addend ? addend[o + i] + g : g;
    }
}

// k_tr_rms_bwd_dx on row t of a split product (dy written first: the gain gradient reads it)
__global__ __launch_bounds__(kPT) void k_tr_rms_bwd_dx_part(float *dy, const float *x, const float *w,
                                                            const float *rrms, int D, float *dx,
                                                            const float *addend, PartIn q) {
    __shared__ double red[kPT / 64];
    sum_part_row(q, blockIdx.x, D, D, dy);   // each thread re-reads only its own columns below
    const size_t o = (size_t)blockIdx.x * D;
    double dot = 0;
    for (int i = threadIdx.x; i < D; i += blockDim.x) dot += (double)(dy[o + i] * x[o + i] * w[i]);
    dot = block_sum_d(dot, red);
    const double r = (double)rrms[blockIdx.x], r2 = (r * r) / (double)D;
    for (int i = threadIdx.x; i < D; i += blockDim.x) {
        const double v = (double)dy[o + i] - (double)x[o + i] * dot * r2;
        const float g = (float)(v * r * (double)w[i]);
        dx[o + i] = addend ? addend[o + i] + g : g;
    }
}
// k_tr_silu_bwd with dgate the sum of a split product's partials (ld == F)
__global__ void k_tr_silu_bwd_part(const float *h13, int F, size_t n, float *dh13, PartIn q) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const size_t t = i / F, j = i % F;
        float v = 0.f;
        for (int z = 0; z < q.ranges; z++) v += q.p[(size_t)z * q.stride + i];
        const float dg = q.R ? q.R[i] + q.alpha * v : q.alpha * v;
        const float h1 = h13[t * 2 * F + j], h3 = h13[t * 2 * F + F + j];
        const float sig = (float)(1.0 / (1.0 + exp(-(double)h1)));
        const float sg = sig * (1 + h1 * (1 - sig));
        dh13[t * 2 * F + j] = dg * h3 * sg;
        dh13[t * 2 * F + F + j] = dg * (h1 * sig);
    }
}

// rmsnorm.go:32-47 gain gradient: the sum over t of float32(float64(dy*x)*r) (eight strided
// row groups, each in row order, then added in group order), stored
// (kDwStore), continued from dw[i] as rmsNormBackward does into an accumulator (kDwContinue, the
// layer gains under backwardAndAccumulate), or formed on its own and then added to dw[i]
// (kDwAdd: the final gain, addSlice at train_full.go:767).
enum { kDwStore = 0, kDwContinue = 1, kDwAdd = 2 };
constexpr int kDwCols = 32, kDwGroups = 8;   // columns per workgroup, row groups per column
__global__ __launch_bounds__(256) void k_tr_rms_bwd_dw(const float *dy, const float *x, const float *rrms, int S,
                                                       int D, int mode, float *dw) {
    // thread (row group g, column c): rows g, g + 8, ... summed in order; the eight group sums
    // then added in group order (each lane pair of a wave reads 2 rows x 128 bytes)
    __shared__ float part[kDwGroups][kDwCols];
    const int c = threadIdx.x % kDwCols, g = threadIdx.x / kDwCols;
    const int i = blockIdx.x * kDwCols + c;
    float acc = 0.f;
    if (i < D) {
        int t = g;
        for (; t + 3 * kDwGroups < S; t += 4 * kDwGroups) {   // four rows' loads in flight
            float a[4], b[4], r[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                a[u] = dy[(size_t)(t + u * kDwGroups) * D + i];
                b[u] = x[(size_t)(t + u * kDwGroups) * D + i];
                r[u] = rrms[t + u * kDwGroups];
            }
#pragma unroll
            for (int u = 0; u < 4; u++) acc += (float)((double)(a[u] * b[u]) * (double)r[u]);
        }
        for (; t < S; t += kDwGroups)
            acc += (float)((double)(dy[(size_t)t * D + i] * x[(size_t)t * D + i]) * (double)rrms[t]);
    }
    part[g][c] = acc;
    __syncthreads();
    if (g == 0 && i < D) {
        float sum = mode == kDwContinue ? dw[i] : 0.f;
#pragma unroll
        for (int k = 0; k < kDwGroups; k++) sum += part[k][c];
        dw[i] = mode == kDwAdd ? dw[i] + sum : sum;
    }
}

// cpu.go:173-253 CrossEntropyLoss for row t of logits [S, V] (in place -> dLogits): float32
// exp terms summed in float64, probabilities, then at the target p (floored at 1e-10) gives
// -log p and dLogits -= 1; a row with an out-of-range target is zeroed.
constexpr int kCeT = 1024;   // threads per vocabulary row: three passes over V floats each
__global__ __launch_bounds__(kCeT) void k_tr_ce_rows(float *lg, const uint16_t *tgt, int V, double *row_loss,
                                                     int *row_valid) {
    __shared__ double red[kCeT / 64];
    __shared__ float redf[kCeT / 64];
    float *row = lg + (size_t)blockIdx.x * V;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < V; i += blockDim.x) mx = fmaxf(mx, row[i]);
    mx = wmax<64>(mx);
    if ((threadIdx.x & 63) == 0) redf[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = redf[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) mx = fmaxf(mx, redf[w]);
    double sum = 0;
    for (int i = threadIdx.x; i < V; i += blockDim.x) {
        const float e = (float)exp((double)(row[i] - mx));
        row[i] = e;
        sum += (double)e;
    }
    sum = block_sum_d(sum, red);
    const float inv = (float)(1.0 / sum);
    for (int i = threadIdx.x; i < V; i += blockDim.x) row[i] *= inv;
    __syncthreads();
    const int t = tgt[blockIdx.x];
    if (t >= V) {
        for (int i = threadIdx.x; i < V; i += blockDim.x) row[i] = 0.f;
        if (threadIdx.x == 0) {
            row_loss[blockIdx.x] = 0;
            row_valid[blockIdx.x] = 0;
        }
        return;
    }
    if (threadIdx.x == 0) {
        float p = row[t];
        if (p < 1e-10f) p = 1e-10f;
        row_loss[blockIdx.x] = -log((double)p);
        row[t] -= 1.f;
        row_valid[blockIdx.x] = 1;
    }
}

// The mean loss (float64 sum over rows in order) and 1/valid for the row scaling.
__global__ void k_tr_ce_total(const double *row_loss, const int *row_valid, int S, float *out) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    double loss = 0;
    int valid = 0;
    for (int t = 0; t < S; t++) {
        loss += row_loss[t];
        valid += row_valid[t];
    }
    out[0] = valid ? (float)(loss / (double)valid) : 0.f;
    out[1] = valid ? (float)(1.0 / (double)valid) : 0.f;
}

__global__ void k_tr_scale_rows(float *lg, const int *row_valid, const float *inv_valid, int V) {
    if (!row_valid[blockIdx.x]) return;
    const float s = inv_valid[1];
    for (int i = threadIdx.x; i < V; i += blockDim.x) lg[(size_t)blockIdx.x * V + i] *= s;
}

// dlc[t][u] = dL[t][ids[u]] (the compact classifier gradient's operand, ld = ldc).
__global__ void k_tr_gather_cols(const float *dl, int V, const int32_t *ids, int U, int ldc, float *dlc) {
    const int t = blockIdx.x;
    for (int u = threadIdx.x; u < ldc; u += blockDim.x)
        dlc[(size_t)t * ldc + u] = u < U ? dl[(size_t)t * V + ids[u]] : 0.f;
}

// Compact classifier rows into the embedding gradient: stored, or added (add != 0) when the
// gradient region accumulates over windows.
__global__ void k_tr_scatter_rows(const float *gc, const int32_t *ids, int D, int add, float *gembed) {
    const int u = blockIdx.x;
    float *row = gembed + (size_t)ids[u] * D;
    for (int i = threadIdx.x; i < D; i += blockDim.x) row[i] = add ? row[i] + gc[(size_t)u * D + i] : gc[(size_t)u * D + i];
}

// cpu.go:74-95 EmbedBackward: row id of the embedding gradient += dx rows of its positions, in
// position order. Workgroup u owns distinct input id ids[u] (positions occ[off[u] .. off[u+1]),
// ascending), so rows are independent and each sum keeps the reference's order.
__global__ void k_tr_embed_bwd(const float *dx, const int32_t *ids, const int32_t *off, const int32_t *occ,
                               int D, float *gembed) {
    const int u = blockIdx.x;
    float *row = gembed + (size_t)ids[u] * D;
    for (int i = threadIdx.x; i < D; i += blockDim.x) {
        float acc = row[i];
        for (int k = off[u]; k < off[u + 1]; k++) acc += dx[(size_t)occ[k] * D + i];
        row[i] = acc;
    }
}

__global__ void k_tr_fill(float *p, size_t n, float v) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = v;
}


// Sum of squares of p[0, n) into per-block float64 partials (block order fixed).
__global__ __launch_bounds__(kTT) void k_tr_sumsq(const float *p, size_t n, float inv_ls, double *part) {
    __shared__ double red[kTT / 64];
    double s = 0;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float x = inv_ls != 1.f ? p[i] * inv_ls : p[i];
        s += (double)x * (double)x;
    }
    s = block_sum_d(s, red);
    if (threadIdx.x == 0) part[blockIdx.x] = s;
}

// train_full.go:932-969 adamUpdateCFWithInv, element-wise in float32.
// The gradient is first multiplied by the loss-scale inverse and then by the clipping factor
// (train_full.go:829-836, :149-181; each a float32 multiply, skipped when it is 1), and
// written back as Adam applies it.
__device__ __forceinline__ void adam_elem(float &w, float &g, float &m, float &v, bool wb, float lr, float b1,
                                          float b2, float eps, float wd, float ibc1, float ibc2, float inv_ls,
                                          float clip) {
    float gi = g;
    if (inv_ls != 1.f) gi *= inv_ls;
    if (clip != 1.f) gi *= clip;
    if (wb) g = gi;
    const float mi = b1 * m + (1 - b1) * gi;
    const float vi = b2 * v + (1 - b2) * gi * gi;
    m = mi;
    v = vi;
    const float mh = mi * ibc1, vh = vi * ibc2;
    float up = mh / ((float)sqrt((double)vh) + eps);
    if (wd != 0) up += wd * w;
    w -= lr * up;
}
// Four independent elements per thread per pass (i, i + stride, ...), all sixteen loads issued
// before any arithmetic, so each thread keeps four times the bytes in flight.
__global__ void k_tr_adam(float *w, float *g, float *m, float *v, size_t n, float lr, float b1, float b2,
                          float eps, float wd, float ibc1, float ibc2, float inv_ls, float clip) {
    const bool wb = inv_ls != 1.f || clip != 1.f;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + 3 * stride < n; i += 4 * stride) {
        float wa[4], ga[4], ma[4], va[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const size_t j = i + u * stride;
            wa[u] = w[j];
            ga[u] = g[j];
            ma[u] = m[j];
            va[u] = v[j];
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const size_t j = i + u * stride;
            adam_elem(wa[u], ga[u], ma[u], va[u], wb, lr, b1, b2, eps, wd, ibc1, ibc2, inv_ls, clip);
            w[j] = wa[u];
            m[j] = ma[u];
            v[j] = va[u];
            if (wb) g[j] = ga[u];
        }
    }
    for (; i < n; i += stride) adam_elem(w[i], g[i], m[i], v[i], wb, lr, b1, b2, eps, wd, ibc1, ibc2, inv_ls, clip);
}

// ---- fp32 MFMA attention (flash form) ----------------------------------------------------
// The forward (forward_common.go:5-33) and causalAttentionBackwardCF (train_full.go:247-301)
// on v_mfma_f32_16x16x4_f32: fp32 operands, exact products, fp32 accumulation, so they differ
// from the reference's sequential sums only in summation order. Tiles of 16 queries (or keys)
// per workgroup, head dims a multiple of 16, any S. Two product forms:
//  - tile_dot: C[16 rows][16 cols] = sum_d A[row][d] B[col][d], A and B row-major in LDS; the
//    result lane l holds column l%16, rows 4(l/16) + r in register r.
//  - tile_acc: C'[dims][16 cols] += M^T . T with T a tile in that result layout (lane l: column
//    l%16, k-rows 4(l/16) + r in register r) and M rows [k][dim] in LDS; MFMA r pairs lane
//    group l/16 with k-row 4(l/16) + r, so T feeds the B operand straight from registers.
// Row strides of HD + 4 floats keep both forms' LDS reads on distinct banks.
constexpr int kMQ = 16;   // query (or key) rows per workgroup
constexpr int kMB = 64;   // key (or query) rows per wave-block

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
template <int HD>
__device__ __forceinline__ f32x4 tile_dot(const float *a, const float *b, int lane) {
    constexpr int P = HD + 4;
    const int r = lane & 15, k = lane >> 4;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < HD; d += 4) acc = mfma4(a[r * P + d + k], b[r * P + d + k], acc);
    return acc;
}
// tile_dot with the B rows already in registers (breg[d/4] = B[l%16][d + l/16])
template <int HD>
__device__ __forceinline__ f32x4 tile_dot_rb(const float *a, const float *breg, int lane) {
    constexpr int P = HD + 4;
    const int r = lane & 15, k = lane >> 4;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < HD; d += 4) acc = mfma4(a[r * P + d + k], breg[d / 4], acc);
    return acc;
}
template <int HD>
__device__ __forceinline__ void tile_acc(f32x4 (&acc)[HD / 16], const float *m, const f32x4 &t, int lane) {
    constexpr int P = HD + 4;
    const int c = lane & 15, kg = lane >> 4;
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int i = 0; i < HD / 16; i++) acc[i] = mfma4(m[(4 * kg + r) * P + 16 * i + c], t[r], acc[i]);
}
// max / sum over the four lanes l, l^16, l^32, l^48 (one result column)
__device__ __forceinline__ float col_max(float v) {
    SwapPair s = swap16(__float_as_uint(v));
    v = fmaxf(__uint_as_float(s.a), __uint_as_float(s.b));
    s = swap32(__float_as_uint(v));
    return fmaxf(__uint_as_float(s.a), __uint_as_float(s.b));
}
__device__ __forceinline__ float col_sum(float v) {
    SwapPair s = swap16(__float_as_uint(v));
    v = __uint_as_float(s.a) + __uint_as_float(s.b);
    s = swap32(__float_as_uint(v));
    return __uint_as_float(s.a) + __uint_as_float(s.b);
}
// rows r0 .. r0+nr-1 (zero past n) of columns c0 .. c0+HD-1 of a row-major matrix into LDS
// [nr][HD + 4], by `nt` threads starting at thread index `t0`; loads first, then stores
template <int HD, int NR>
__device__ __forceinline__ void stage_tile(float *dst, const float *src, size_t ld, int c0, int r0, int n, int t0,
                                           int nt) {
    constexpr int PER = HD / 4, TOT = NR * PER;
    for (int e0 = 0; e0 < TOT; e0 += 4 * nt) {
        f32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int e = e0 + t0 + u * nt, r = e / PER, c = (e % PER) * 4;
            const bool ok = e < TOT && r0 + r < n;
            v[u] = ok ? *(const f32x4 *)(src + (size_t)(r0 + r) * ld + c0 + c) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int e = e0 + t0 + u * nt, r = e / PER, c = (e % PER) * 4;
            if (e < TOT) *(f32x4 *)(dst + r * (HD + 4) + c) = v[u];
        }
    }
}
template <int HD> constexpr size_t mf_lds_bytes() {
    return sizeof(float) * (size_t)(2 * kMQ * (HD + 4) + 4 * 2 * kMB * (HD + 4));
}

// Forward for queries q0 .. q0+15 of head h: the key blocks up to the tile's last query dealt
// round-robin to the four waves (own LDS slices); per block S^T = K.Q^T, the online softmax
// per query (float64 exp of score - running max, as the reference's exp), O^T += V^T.P^T;
// the waves' (max, sum, O) merged at the end. att = O / sum; stats[t] = (max, 1/sum).
template <int HD>
__global__ __launch_bounds__(256) void k_tr_attn_fwd_mf(const float *qkv, int S, int D, float scale, float *att,
                                                        float *stats) {
    constexpr int P = HD + 4, NO = HD / 16;
    __shared__ __attribute__((aligned(16))) float lds[mf_lds_bytes<HD>() / sizeof(float)];
    float *qs = lds, *slice = lds + 2 * kMQ * P;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int q0 = blockIdx.x * kMQ, h = blockIdx.y;
    const size_t ld = 3 * (size_t)D;
    float *kb_s = slice + wave * 2 * kMB * P, *vb_s = kb_s + kMB * P;
    stage_tile<HD, kMQ>(qs, qkv, ld, h * HD, q0, S, tid, 256);
    __syncthreads();
    const int qlast = min(q0 + kMQ, S) - 1;
    const int nb = qlast / kMB + 1;
    const int c = lane & 15, kg = lane >> 4, t = q0 + c;
    float m_run = -INFINITY, l_part = 0.f;
    f32x4 o[NO];
#pragma unroll
    for (int i = 0; i < NO; i++) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int bi = wave; bi < nb; bi += 4) {
        const int kb = bi * kMB;
        stage_tile<HD, kMB>(kb_s, qkv, ld, D + h * HD, kb, S, lane, 64);
        stage_tile<HD, kMB>(vb_s, qkv, ld, 2 * D + h * HD, kb, S, lane, 64);
        __builtin_amdgcn_wave_barrier();
        const int nj = min(kMB, qlast + 1 - kb + 15) / 16;   // 16-key tiles some query can see
        for (int j = 0; j < nj; j++) {
            f32x4 sc = tile_dot<HD>(kb_s + 16 * j * P, qs, lane);
            float mx = -INFINITY;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int key = kb + 16 * j + 4 * kg + r;
                sc[r] = key <= t ? sc[r] * scale : -INFINITY;
                mx = fmaxf(mx, sc[r]);
            }
            mx = col_max(mx);
            // a column with no visible key yet keeps max -inf and gets p = 0 (no branch: the
            // MFMAs below run on the whole wave)
            const float m_new = fmaxf(m_run, mx);
            const float m_use = m_new == -INFINITY ? 0.f : m_new;
            const float rs = m_run == -INFINITY ? 0.f : (float)exp((double)(m_run - m_use));
            m_run = m_new;
            l_part *= rs;
#pragma unroll
            for (int i = 0; i < NO; i++) o[i] *= rs;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                sc[r] = sc[r] == -INFINITY ? 0.f : (float)exp((double)(sc[r] - m_use));
                l_part += sc[r];
            }
            tile_acc<HD>(o, vb_s + 16 * j * P, sc, lane);
        }
        __builtin_amdgcn_wave_barrier();
    }
    // merge the waves: (max, sum) per query column, O^T per (dim, query)
    const float l_w = col_sum(l_part);
    __syncthreads();
    float *oo = slice, *mo = oo + 4 * HD * kMQ, *lo = mo + 4 * kMQ;
    if (kg == 0) {
        mo[wave * kMQ + c] = m_run;
        lo[wave * kMQ + c] = l_w;
    }
#pragma unroll
    for (int i = 0; i < NO; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) oo[(wave * HD + 16 * i + 4 * kg + r) * kMQ + c] = o[i][r];
    __syncthreads();
    for (int e = tid; e < kMQ * HD; e += 256) {
        const int q = e / HD, d = e % HD, tq = q0 + q;
        if (tq >= S) continue;
        float mm = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++) mm = fmaxf(mm, mo[w * kMQ + q]);
        float lt = 0.f, ot = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float mw = mo[w * kMQ + q];
            const float f = mw == -INFINITY ? 0.f : (float)exp((double)(mw - mm));
            lt += lo[w * kMQ + q] * f;
            ot += oo[(w * HD + d) * kMQ + q] * f;
        }
        const float inv = (float)(1.0 / (double)lt);
        att[(size_t)tq * D + h * HD + d] = ot * inv;
        if (d == 0) {
            float *st = stats + ((size_t)h * S + tq) * 3;
            st[0] = mm;
            st[1] = inv;
        }
    }
}

// Query side of the backward for queries q0 .. q0+15 of head h: dsSum_t = dO_t . O_t (equal
// to the reference's sum over keys of p*dp), then per key block (waves round-robin)
// P^T from the forward's (max, 1/sum), dP^T = V.dO^T, dS^T = P^T (dP^T - dsSum) scale,
// dQ^T += K^T.dS^T; the waves' dQ summed at the end. stats[t][2] = dsSum for the key side.
template <int HD>
__global__ __launch_bounds__(256) void k_tr_attn_bwd_q_mf(const float *qkv, const float *att, const float *dout,
                                                          int S, int D, float scale, float *dqkv, float *stats) {
    constexpr int P = HD + 4, NO = HD / 16;
    __shared__ __attribute__((aligned(16))) float lds[mf_lds_bytes<HD>() / sizeof(float)];
    __shared__ float dsum[kMQ];
    float *qs = lds, *gs = lds + kMQ * P, *slice = lds + 2 * kMQ * P;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int q0 = blockIdx.x * kMQ, h = blockIdx.y;
    const size_t ld = 3 * (size_t)D;
    float *kb_s = slice + wave * 2 * kMB * P, *vb_s = kb_s + kMB * P;
    stage_tile<HD, kMQ>(qs, qkv, ld, h * HD, q0, S, tid, 256);
    stage_tile<HD, kMQ>(gs, dout, D, h * HD, q0, S, tid, 256);
    if (tid < kMQ) {
        const int t = q0 + tid;
        float d = 0.f;
        if (t < S) {
            const float *a = att + (size_t)t * D + h * HD, *g = dout + (size_t)t * D + h * HD;
            for (int i = 0; i < HD; i++) d += g[i] * a[i];
            stats[((size_t)h * S + t) * 3 + 2] = d;
        }
        dsum[tid] = d;
    }
    __syncthreads();
    const int qlast = min(q0 + kMQ, S) - 1;
    const int nb = qlast / kMB + 1;
    const int c = lane & 15, kg = lane >> 4, t = q0 + c;
    float mq = 0.f, iq = 0.f;
    if (t < S) {
        mq = stats[((size_t)h * S + t) * 3];
        iq = stats[((size_t)h * S + t) * 3 + 1];
    }
    const float dq_sum = dsum[c];
    f32x4 dq[NO];
#pragma unroll
    for (int i = 0; i < NO; i++) dq[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int bi = wave; bi < nb; bi += 4) {
        const int kb = bi * kMB;
        stage_tile<HD, kMB>(kb_s, qkv, ld, D + h * HD, kb, S, lane, 64);
        stage_tile<HD, kMB>(vb_s, qkv, ld, 2 * D + h * HD, kb, S, lane, 64);
        __builtin_amdgcn_wave_barrier();
        const int nj = min(kMB, qlast + 1 - kb + 15) / 16;
        for (int j = 0; j < nj; j++) {
            const f32x4 sc = tile_dot<HD>(kb_s + 16 * j * P, qs, lane);
            const f32x4 dp = tile_dot<HD>(vb_s + 16 * j * P, gs, lane);
            f32x4 ds;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int key = kb + 16 * j + 4 * kg + r;
                const float p = key <= t ? (float)exp((double)(sc[r] * scale - mq)) * iq : 0.f;
                ds[r] = p * (dp[r] - dq_sum) * scale;
            }
            tile_acc<HD>(dq, kb_s + 16 * j * P, ds, lane);
        }
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    float *oo = slice;
#pragma unroll
    for (int i = 0; i < NO; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) oo[(wave * HD + 16 * i + 4 * kg + r) * kMQ + c] = dq[i][r];
    __syncthreads();
    for (int e = tid; e < kMQ * HD; e += 256) {
        const int q = e / HD, d = e % HD, tq = q0 + q;
        if (tq >= S) continue;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) v += oo[(w * HD + d) * kMQ + q];
        dqkv[(size_t)tq * ld + h * HD + d] = v;
    }
}

// Key side for keys s0 .. s0+15 of head h: the 16-query tiles from the key tile on dealt
// round-robin to the waves; per tile S = Q.K^T and dP = dO.V^T (K and V rows held in
// registers as B operands), P and dS from the row stats, dV^T += dO^T.P, dK^T += Q^T.dS;
// the waves' sums merged at the end.
template <int HD>
__global__ __launch_bounds__(256) void k_tr_attn_bwd_kv_mf(const float *qkv, const float *dout, int S, int D,
                                                           float scale, const float *stats, float *dqkv) {
    constexpr int P = HD + 4, NO = HD / 16;
    __shared__ __attribute__((aligned(16))) float lds[mf_lds_bytes<HD>() / sizeof(float)];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int s0 = blockIdx.x * kMQ, h = blockIdx.y;
    const size_t ld = 3 * (size_t)D;
    float *qt = lds + wave * 2 * kMB * P, *gt = qt + kMQ * P;   // the wave's query tile rows
    const int c = lane & 15, kg = lane >> 4, key = s0 + c;
    // K and V rows of key `key` as B operands: kreg[d/4] = K[key][d + kg]
    float kreg[HD / 4], vreg[HD / 4];
#pragma unroll
    for (int d = 0; d < HD; d += 4) {
        const bool ok = key < S;
        kreg[d / 4] = ok ? qkv[(size_t)key * ld + D + h * HD + d + kg] : 0.f;
        vreg[d / 4] = ok ? qkv[(size_t)key * ld + 2 * D + h * HD + d + kg] : 0.f;
    }
    f32x4 dk[NO], dv[NO];
#pragma unroll
    for (int i = 0; i < NO; i++) dk[i] = dv[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int ntiles = (S + kMQ - 1) / kMQ;
    for (int qt_i = blockIdx.x + wave; qt_i < ntiles; qt_i += 4) {
        const int tq0 = qt_i * kMQ;
        stage_tile<HD, kMQ>(qt, qkv, ld, h * HD, tq0, S, lane, 64);
        stage_tile<HD, kMQ>(gt, dout, D, h * HD, tq0, S, lane, 64);
        __builtin_amdgcn_wave_barrier();
        const f32x4 sc = tile_dot_rb<HD>(qt, kreg, lane);   // rows: queries tq0 + 4kg + r; column: key
        const f32x4 dp = tile_dot_rb<HD>(gt, vreg, lane);
        f32x4 p, ds;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int tq = tq0 + 4 * kg + r;
            float pv = 0.f, dv_ = 0.f;
            if (tq < S && key <= tq) {
                const float *st = stats + ((size_t)h * S + tq) * 3;
                pv = (float)exp((double)(sc[r] * scale - st[0])) * st[1];
                dv_ = pv * (dp[r] - st[2]) * scale;
            }
            p[r] = pv;
            ds[r] = dv_;
        }
        tile_acc<HD>(dv, gt, p, lane);
        tile_acc<HD>(dk, qt, ds, lane);
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    float *ok_ = lds, *ov = lds + 4 * HD * kMQ;
#pragma unroll
    for (int i = 0; i < NO; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            ok_[(wave * HD + 16 * i + 4 * kg + r) * kMQ + c] = dk[i][r];
            ov[(wave * HD + 16 * i + 4 * kg + r) * kMQ + c] = dv[i][r];
        }
    __syncthreads();
    for (int e = tid; e < kMQ * HD; e += 256) {
        const int k = e / HD, d = e % HD, s = s0 + k;
        if (s >= S) continue;
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            a += ok_[(w * HD + d) * kMQ + k];
            b += ov[(w * HD + d) * kMQ + k];
        }
        dqkv[(size_t)s * ld + D + h * HD + d] = a;
        dqkv[(size_t)s * ld + 2 * D + h * HD + d] = b;
    }
}

}  // namespace
}  // namespace sh

// ---- host side ---------------------------------------------------------------------------

struct sh_trainer {
    sh_config cfg;
    sh_train_options opt;
    int device;
    hipStream_t stream;
    int S, D, F, H, hd, V, L;
    // parameter arenas (weights, gradients, Adam m and v), identical layout
    size_t n_mat, n_all;
    float *p, *g, *m, *v;
    std::vector<size_t> o_qkv, o_wo, o_w13, o_w2, o_ra, o_rf;
    size_t o_embed, o_rfin;
    // activations (token-major) and scratch, one allocation
    void *act;
    struct Layer {
        float *x, *xn, *ra, *qkv, *att, *x2, *x2n, *rf, *h13, *gate;
    };
    std::vector<Layer> lc;
    float *xL, *xnf, *rfin, *logits, *dy, *dcur, *gx2, *gxn, *gatt, *ggate,
        *dh13, *dqkv, *stats, *dlc, *gc, *loss, *cos_t, *sin_t;
    double *row_loss, *sq_part;
    int *row_valid;
    int32_t *ids, *in_ids, *in_off, *in_occ;   // compact target ids; input ids' positions
    float *part;                               // split-K partial tiles
    size_t part_cap;
    uint16_t *tok_in, *tok_tgt;
    int ldc_u;   // padded compact width
    std::vector<uint16_t> tokens;
    uint64_t rng;
    sh_train_state state;
    hipEvent_t ev0, ev1;
    bool uploaded_globals;
    std::vector<bool> uploaded;
};

namespace sh {
namespace {

constexpr int kSqParts = 1024;

unsigned blocks_for(size_t n) { return (unsigned)std::min<size_t>((n + 255) / 256, 8192); }

// tile-aligned shapes (and 16-byte aligned rows) take the burst-load kernel
bool sgemm_aligned(int M, int N, int K, int kc) { return M % 64 == 0 && N % 64 == 0 && K % 128 == 0 && kc % 128 == 0; }

template <bool AK, bool BK, int EPI>
hipError_t sgemm(hipStream_t s, const float *A, int lda, const float *B, int ldb, float *C, int ldc, int M,
                 int N, int K, float alpha, const float *R = nullptr) {
    const dim3 grid((N + kGN - 1) / kGN, (M + kGM - 1) / kGM);
    if (sgemm_aligned(M, N, K, K))
        hipLaunchKernelGGL((k_sgemm_pipe<AK, BK, EPI>), grid, dim3(256), 0, s, A, lda, B, ldb, C, ldc, M, N, K, alpha, R, K);
    else
        hipLaunchKernelGGL((k_sgemm<AK, BK, EPI>), grid, dim3(256), 0, s, A, lda, B, ldb, C, ldc, M, N, K, alpha, R, K);
    return hipGetLastError();
}

// C = alpha * A.B with K split into ranges when the tiles alone leave most CUs idle: range
// partials in `part`, then their sum in range order (k_tr_reduce_ranges). Falls back to one
// range when `part` cannot hold them.
template <bool AK, bool BK>
// handoff given: with more than one range the partials are left for the consuming row kernel
// (handoff->p set, C not written); with one range C is written and handoff->p stays null.
hipError_t sgemm_split(hipStream_t s, const float *A, int lda, const float *B, int ldb, float *C, int ldc, int M,
                       int N, int K, float alpha, float *part, size_t part_cap, const float *R = nullptr,
                       PartIn *handoff = nullptr) {
    if (handoff) *handoff = PartIn{};
    const int tiles = ((N + kGN - 1) / kGN) * ((M + kGM - 1) / kGM);
    int ranges = 1;
    if (tiles < 192 && K >= 512) ranges = std::min(16, std::max(1, K / 256));
    if (ranges > 1 && (size_t)ranges * M * ldc > part_cap) ranges = 1;
    if (ranges == 1)
        return R ? sgemm<AK, BK, EPI_RESID>(s, A, lda, B, ldb, C, ldc, M, N, K, alpha, R)
                 : sgemm<AK, BK, EPI_STORE>(s, A, lda, B, ldb, C, ldc, M, N, K, alpha);
    int kc = (K / ranges + kGK - 1) / kGK * kGK;
    const bool al = sgemm_aligned(M, N, K, 128);
    if (al) kc = (K / ranges + 127) / 128 * 128;   // ranges of whole 128-k bursts
    ranges = (K + kc - 1) / kc;
    const dim3 grid((N + kGN - 1) / kGN, (M + kGM - 1) / kGM, ranges);
    if (al)
        hipLaunchKernelGGL((k_sgemm_pipe<AK, BK, EPI_PART>), grid, dim3(256), 0, s, A, lda, B, ldb, part, ldc, M, N,
                           K, 1.f, nullptr, kc);
    else
        hipLaunchKernelGGL((k_sgemm<AK, BK, EPI_PART>), grid, dim3(256), 0, s, A, lda, B, ldb, part, ldc, M, N, K,
                           1.f, nullptr, kc);
    if (handoff) {
        *handoff = PartIn{part, ranges, (size_t)M * ldc, R, alpha};
        return hipGetLastError();
    }
    const size_t n = (size_t)M * N;
    hipLaunchKernelGGL(k_tr_reduce_ranges, dim3(blocks_for(n)), dim3(256), 0, s, part, ranges, M, N, ldc, alpha, R,
                       C);
    return hipGetLastError();
}

// dW GEMM into the gradient arena: stored, or added onto what it holds (acc) when gradients
// accumulate over windows.
template <bool AK, bool BK>
hipError_t sgemm_grad(hipStream_t s, const float *A, int lda, const float *B, int ldb, float *C, int ldc, int M,
                      int N, int K, bool acc, float alpha = 1.f) {
    return acc ? sgemm<AK, BK, EPI_RESID>(s, A, lda, B, ldb, C, ldc, M, N, K, alpha, C)
               : sgemm<AK, BK, EPI_STORE>(s, A, lda, B, ldb, C, ldc, M, N, K, alpha);
}

// Forward (train_full.go:368-396) for the window in tok_in, then runFinalHead's CPU path
// (:435-523): logits, CrossEntropyLoss, dy = E^T dL * loss scale, the compact classifier
// embedding gradient, the final RMSNorm backward. acc: the gradient arena holds earlier
// windows' sums, which this window's embedding and final-gain gradients add onto.
hipError_t tr_forward_head(sh_trainer *T, int U, float loss_scale, bool acc) {
    hipStream_t s = T->stream;
    const int S = T->S, D = T->D, F = T->F, hd = T->hd, V = T->V;
    const float alpha = T->cfg.residual_scale, scale = (float)(1.0 / sqrt((double)hd));
    const double eps = T->cfg.norm_eps;
    hipError_t e;
    float *cur = T->lc[0].x;
    hipLaunchKernelGGL(k_tr_embed, dim3(S), dim3(256), 0, s, T->p + T->o_embed, T->tok_in, V, D, cur);
    // split products hand their partials to the row kernel that consumes them; hx: the
    // previous layer's W2 product, summed by this layer's RMSNorm
    PartIn hx{}, hq{}, hw{};
    auto rmsnorm = [&](float *x, const float *g, float *out, float *rr, const PartIn &q) {
        if (q.p) hipLaunchKernelGGL(k_tr_rmsnorm_part, dim3(S), dim3(kPT), 0, s, x, g, D, eps, out, rr, q);
        else hipLaunchKernelGGL(k_tr_rmsnorm, dim3(S), dim3(kTT), 0, s, x, g, D, eps, out, rr);
    };
    for (int l = 0; l < T->L; l++) {
        sh_trainer::Layer &C = T->lc[l];   // C.x == cur: the previous layer wrote it there
        rmsnorm(C.x, T->p + T->o_ra[l], C.xn, C.ra, hx);
        if ((e = sgemm_split<true, true>(s, C.xn, D, T->p + T->o_qkv[l], D, C.qkv, 3 * D, S, 3 * D, D, 1.f, T->part,
                                         T->part_cap, nullptr, &hq)))
            return e;
        if (hq.p) hipLaunchKernelGGL(k_tr_rope_part, dim3(S), dim3(kPT), 0, s, C.qkv, D, hd, T->cos_t, T->sin_t, hq);
        else hipLaunchKernelGGL(k_tr_rope, dim3(S), dim3(256), 0, s, C.qkv, D, hd, T->cos_t, T->sin_t);
        float *st = T->stats + (size_t)l * 3 * T->H * S;   // this layer's (max, 1/sum, dsSum) rows
        if (hd == 64)
            hipLaunchKernelGGL(k_tr_attn_fwd_mf<64>, dim3((S + kMQ - 1) / kMQ, T->H), dim3(256), 0, s, C.qkv, S, D,
                               scale, C.att, st);
        else if (hd == 32)
            hipLaunchKernelGGL(k_tr_attn_fwd_mf<32>, dim3((S + kMQ - 1) / kMQ, T->H), dim3(256), 0, s, C.qkv, S, D,
                               scale, C.att, st);
        else if (S <= kAttnMaxS)
            hipLaunchKernelGGL(k_tr_attn_fwd_blk, dim3((S + kAQ - 1) / kAQ, T->H), dim3(256),
                               sizeof(float) * (kAQ * kAPad + kAB * kAPad + kAQ * (S + kSPad)), s, C.qkv, S, D, hd, scale,
                               C.att);
        else
            hipLaunchKernelGGL(k_tr_attn_fwd, dim3(S, T->H), dim3(64), sizeof(float) * S, s, C.qkv, S, D, hd, scale,
                               C.att);
        if ((e = sgemm_split<true, true>(s, C.att, D, T->p + T->o_wo[l], D, C.x2, D, S, D, D, alpha, T->part,
                                         T->part_cap, C.x, &hw)))
            return e;
        rmsnorm(C.x2, T->p + T->o_rf[l], C.x2n, C.rf, hw);
        if ((e = sgemm_split<true, true>(s, C.x2n, D, T->p + T->o_w13[l], D, C.h13, 2 * F, S, 2 * F, D, 1.f, T->part,
                                         T->part_cap)))
            return e;
        const size_t nf = (size_t)S * F;
        hipLaunchKernelGGL(k_tr_silu_gate, dim3(blocks_for(nf)), dim3(256), 0, s, C.h13, F, nf, C.gate);
        float *next = l + 1 < T->L ? T->lc[l + 1].x : T->xL;
        if ((e = sgemm_split<true, true>(s, C.gate, F, T->p + T->o_w2[l], F, next, D, S, D, F, alpha, T->part,
                                         T->part_cap, C.x2, &hx)))
            return e;
        cur = next;
    }
    // final head
    rmsnorm(T->xL, T->p + T->o_rfin, T->xnf, T->rfin, hx);
    if ((e = sgemm<true, true, EPI_STORE>(s, T->xnf, D, T->p + T->o_embed, D, T->logits, V, S, V, D, 1.f)))
        return e;
    hipLaunchKernelGGL(k_tr_ce_rows, dim3(S), dim3(kCeT), 0, s, T->logits, T->tok_tgt, V, T->row_loss, T->row_valid);
    hipLaunchKernelGGL(k_tr_ce_total, dim3(1), dim3(64), 0, s, T->row_loss, T->row_valid, S, T->loss);
    hipLaunchKernelGGL(k_tr_scale_rows, dim3(S), dim3(1024), 0, s, T->logits, T->row_valid, T->loss, V);
    // dy[t][d] = (sum_v dL[t][v] E[v][d]) * loss scale (MatMulEmbedTScale)
    PartIn hy{};   // summed by the final RMSNorm backward below
    if ((e = sgemm_split<true, false>(s, T->logits, V, T->p + T->o_embed, D, T->dy, D, S, D, V, loss_scale,
                                      T->part, T->part_cap, nullptr, &hy)))
        return e;
    // classifier embedding gradient on the target rows: gc[u][d] = (sum_t dL[t][ids u] xnf[t][d]) * scale
    float *gemb = T->g + T->o_embed;
    if (!acc)
        hipLaunchKernelGGL(k_tr_fill, dim3(blocks_for((size_t)V * D)), dim3(256), 0, s, gemb, (size_t)V * D, 0.f);
    if (U > 0) {
        hipLaunchKernelGGL(k_tr_gather_cols, dim3(S), dim3(256), 0, s, T->logits, V, T->ids, U, T->ldc_u, T->dlc);
        if ((e = sgemm<false, false, EPI_STORE>(s, T->dlc, T->ldc_u, T->xnf, D, T->gc, D, U, D, S, loss_scale)))
            return e;
        hipLaunchKernelGGL(k_tr_scatter_rows, dim3(U), dim3(256), 0, s, T->gc, T->ids, D, (int)acc, gemb);
    }
    // final RMSNorm backward: dcur and the rms_final gradient
    if (hy.p)
        hipLaunchKernelGGL(k_tr_rms_bwd_dx_part, dim3(S), dim3(kPT), 0, s, T->dy, T->xL, T->p + T->o_rfin, T->rfin,
                           D, T->dcur, (const float *)nullptr, hy);
    else
        hipLaunchKernelGGL(k_tr_rms_bwd_dx, dim3(S), dim3(kTT), 0, s, T->dy, T->xL, T->p + T->o_rfin, T->rfin, D,
                           T->dcur);
    hipLaunchKernelGGL(k_tr_rms_bwd_dw, dim3((D + kDwCols - 1) / kDwCols), dim3(256), 0, s, T->dy, T->xL, T->rfin, S, D,
                       acc ? kDwAdd : kDwStore, T->g + T->o_rfin);
    return hipGetLastError();
}

// The layer loop of backwardAndApply (train_full.go:776-848) or backwardAndAccumulate
// (:709-774), CPU path, then EmbedBackward. acc: layer gradients add onto the arena's sums
// (no clearLayerGrad), as the accumulate loop writes into e.accum directly.
hipError_t tr_backward(sh_trainer *T, int n_in, bool acc) {
    hipStream_t s = T->stream;
    const int S = T->S, D = T->D, F = T->F, hd = T->hd;
    const float alpha = T->cfg.residual_scale, scale = (float)(1.0 / sqrt((double)hd));
    hipError_t e;
    for (int l = T->L - 1; l >= 0; l--) {
        sh_trainer::Layer &C = T->lc[l];
        // FFN: ggate = dout . W2 with dout = alpha dcur (the scale applied to the product),
        // (dh1, dh3), gxn = [dh1|dh3] . [W1;W3], RMS backward
        PartIn hg{}, hn{};   // split products' partials for the row kernels below
        if ((e = sgemm_split<true, false>(s, T->dcur, D, T->p + T->o_w2[l], F, T->ggate, F, S, F, D, alpha, T->part,
                                          T->part_cap, nullptr, &hg)))
            return e;
        const size_t nf = (size_t)S * F;
        if (hg.p)
            hipLaunchKernelGGL(k_tr_silu_bwd_part, dim3(blocks_for(nf)), dim3(256), 0, s, C.h13, F, nf, T->dh13, hg);
        else
            hipLaunchKernelGGL(k_tr_silu_bwd, dim3(blocks_for(nf)), dim3(256), 0, s, T->ggate, C.h13, F, nf, T->dh13);
        if ((e = sgemm_split<true, false>(s, T->dh13, 2 * F, T->p + T->o_w13[l], D, T->gxn, D, S, D, 2 * F, 1.f,
                                          T->part, T->part_cap, nullptr, &hn)))
            return e;
        // gx2 = dcur + the RMS backward's dx
        if (hn.p)
            hipLaunchKernelGGL(k_tr_rms_bwd_dx_part, dim3(S), dim3(kPT), 0, s, T->gxn, C.x2, T->p + T->o_rf[l], C.rf,
                               D, T->gx2, (const float *)T->dcur, hn);
        else
            hipLaunchKernelGGL(k_tr_rms_bwd_dx, dim3(S), dim3(kTT), 0, s, T->gxn, C.x2, T->p + T->o_rf[l], C.rf, D,
                               T->gx2, T->dcur);
        hipLaunchKernelGGL(k_tr_rms_bwd_dw, dim3((D + kDwCols - 1) / kDwCols), dim3(256), 0, s, T->gxn, C.x2, C.rf, S, D,
                           acc ? kDwContinue : kDwStore, T->g + T->o_rf[l]);
        // weight gradients: dW2 = dout^T gate (alpha dcur^T gate), d[W1;W3] = [dh1|dh3]^T x2n
        if ((e = sgemm_grad<false, false>(s, T->dcur, D, C.gate, F, T->g + T->o_w2[l], F, D, F, S, acc, alpha)))
            return e;
        if ((e = sgemm_grad<false, false>(s, T->dh13, 2 * F, C.x2n, D, T->g + T->o_w13[l], D, 2 * F, D, S, acc)))
            return e;
        // attention: gatt = dx2s . Wo with dx2s = alpha gx2, (dq, dk, dv),
        // gxn = [dq|dk|dv] . [Wq;Wk;Wv], RMS backward
        if ((e = sgemm_split<true, false>(s, T->gx2, D, T->p + T->o_wo[l], D, T->gatt, D, S, D, D, alpha, T->part,
                                          T->part_cap)))
            return e;
        float *st = T->stats + (size_t)l * 3 * T->H * S;   // the forward's (max, 1/sum) rows
        const dim3 tiles((S + kMQ - 1) / kMQ, T->H);
        if (hd == 64 || hd == 32) {
            if (hd == 64) {
                hipLaunchKernelGGL(k_tr_attn_bwd_q_mf<64>, tiles, dim3(256), 0, s, C.qkv, C.att, T->gatt, S, D, scale,
                                   T->dqkv, st);
                hipLaunchKernelGGL(k_tr_attn_bwd_kv_mf<64>, tiles, dim3(256), 0, s, C.qkv, T->gatt, S, D, scale, st,
                                   T->dqkv);
            } else {
                hipLaunchKernelGGL(k_tr_attn_bwd_q_mf<32>, tiles, dim3(256), 0, s, C.qkv, C.att, T->gatt, S, D, scale,
                                   T->dqkv, st);
                hipLaunchKernelGGL(k_tr_attn_bwd_kv_mf<32>, tiles, dim3(256), 0, s, C.qkv, T->gatt, S, D, scale, st,
                                   T->dqkv);
            }
        } else if (S <= kAttnMaxS) {
            hipLaunchKernelGGL(k_tr_attn_bwd_q_blk, dim3((S + kAQ - 1) / kAQ, T->H), dim3(256),
                               sizeof(float) * (2 * kAQ * kAPad + kAB * kAPad + 2 * kAQ * (S + kSPad)), s, C.qkv, T->gatt, S,
                               D, hd, scale, T->dqkv, st);
            hipLaunchKernelGGL(k_tr_attn_bwd_kv_blk, dim3((S + kAQ - 1) / kAQ, T->H), dim3(256), 0, s, C.qkv,
                               T->gatt, S, D, hd, scale, st, T->dqkv);
        } else {
            hipLaunchKernelGGL(k_tr_attn_bwd_q, dim3(S, T->H), dim3(64), 2 * sizeof(float) * S, s, C.qkv, T->gatt,
                               S, D, hd, scale, T->dqkv, st);
            hipLaunchKernelGGL(k_tr_attn_bwd_kv, dim3(S, T->H), dim3(64), 2 * sizeof(float) * S, s, C.qkv, T->gatt,
                               S, D, hd, scale, st, T->dqkv);
        }
        PartIn ha{};
        if ((e = sgemm_split<true, false>(s, T->dqkv, 3 * D, T->p + T->o_qkv[l], D, T->gxn, D, S, D, 3 * D, 1.f,
                                          T->part, T->part_cap, nullptr, &ha)))
            return e;
        // the next layer's dcur = gx2 + the RMS backward's dx
        if (ha.p)
            hipLaunchKernelGGL(k_tr_rms_bwd_dx_part, dim3(S), dim3(kPT), 0, s, T->gxn, C.x, T->p + T->o_ra[l], C.ra,
                               D, T->dcur, (const float *)T->gx2, ha);
        else
            hipLaunchKernelGGL(k_tr_rms_bwd_dx, dim3(S), dim3(kTT), 0, s, T->gxn, C.x, T->p + T->o_ra[l], C.ra, D,
                               T->dcur, T->gx2);
        hipLaunchKernelGGL(k_tr_rms_bwd_dw, dim3((D + kDwCols - 1) / kDwCols), dim3(256), 0, s, T->gxn, C.x, C.ra, S, D,
                           acc ? kDwContinue : kDwStore, T->g + T->o_ra[l]);
        // dWo = dx2s^T att (alpha gx2^T att), d[Wq;Wk;Wv] = [dq|dk|dv]^T xn
        if ((e = sgemm_grad<false, false>(s, T->gx2, D, C.att, D, T->g + T->o_wo[l], D, D, D, S, acc, alpha)))
            return e;
        if ((e = sgemm_grad<false, false>(s, T->dqkv, 3 * D, C.xn, D, T->g + T->o_qkv[l], D, 3 * D, D, S, acc)))
            return e;
    }
    if (n_in > 0)
        hipLaunchKernelGGL(k_tr_embed_bwd, dim3(n_in), dim3(256), 0, s, T->dcur, T->in_ids, T->in_off, T->in_occ, D,
                           T->g + T->o_embed);
    return hipGetLastError();
}

// The gradient arena times `inv` (the loss-scale undo of backwardAndApply, train_full.go:829-836,
// or flushPending's 1/pending/loss scale, engine.go:544-548), clipping (clipLayerGradients,
// :149-181) and Adam at 1-based step step_t (:838-842); k_tr_adam leaves the applied gradients
// in the arena.
hipError_t tr_apply(sh_trainer *T, float inv, int step_t) {
    hipStream_t s = T->stream;
    hipError_t e;
    float clip = 1.f;
    if (T->opt.grad_clip > 0) {
        hipLaunchKernelGGL(k_tr_sumsq, dim3(kSqParts), dim3(kTT), 0, s, T->g, T->n_all, inv, T->sq_part);
        std::vector<double> part(kSqParts);
        if ((e = hipMemcpyAsync(part.data(), T->sq_part, sizeof(double) * kSqParts, hipMemcpyDeviceToHost, s)) ||
            (e = hipStreamSynchronize(s)))
            return e;
        double norm2 = 0;
        for (double x : part) norm2 += x;
        if (norm2 > 0) {
            const float norm = (float)sqrt(norm2);
            if (norm > T->opt.grad_clip) clip = T->opt.grad_clip / norm;
        }
    }
    const float ibc1 = 1.f / (float)(1.0 - pow((double)T->opt.beta1, (double)step_t));
    const float ibc2 = 1.f / (float)(1.0 - pow((double)T->opt.beta2, (double)step_t));
    const sh_train_options &o = T->opt;
    hipLaunchKernelGGL(k_tr_adam, dim3(blocks_for(T->n_mat)), dim3(256), 0, s, T->p, T->g, T->m, T->v, T->n_mat,
                       o.lr, o.beta1, o.beta2, o.eps, o.weight_decay, ibc1, ibc2, inv, clip);
    const size_t ng = T->n_all - T->n_mat;
    hipLaunchKernelGGL(k_tr_adam, dim3(blocks_for(ng)), dim3(256), 0, s, T->p + T->n_mat, T->g + T->n_mat,
                       T->m + T->n_mat, T->v + T->n_mat, ng, o.lr, o.beta1, o.beta2, o.eps, 0.f, ibc1, ibc2, inv,
                       clip);
    return hipGetLastError();
}

// Distinct in-range target ids in order of first appearance (buildCompactVocab,
// train_full.go:560-587); an empty list when they exceed half of stories.Vocab (32000).
std::vector<int32_t> compact_ids(const uint16_t *tgt, int S, int V) {
    std::vector<int32_t> ids;
    std::vector<char> seen(V, 0);
    for (int t = 0; t < S; t++) {
        const int tok = tgt[t];
        if (tok >= V || seen[tok]) continue;
        seen[tok] = 1;
        ids.push_back(tok);
    }
    if ((int)ids.size() > 32000 / 2) ids.clear();
    return ids;
}

bool tr_ready(const sh_trainer *T) {
    if (!T) {
        set_error("nil trainer");
        return false;
    }
    for (bool u : T->uploaded)
        if (!u) {
            set_error("trainer weights are not fully uploaded");
            return false;
        }
    if (!T->uploaded_globals) {
        set_error("trainer weights are not fully uploaded");
        return false;
    }
    return true;
}

// flushPending (engine.go:540-565): the accumulated sums times float32(1/pending) / loss scale,
// clipped, then Adam; the arena keeps the applied gradients and the next window overwrites it.
bool tr_flush(sh_trainer *T) {
    if (T->state.pending_steps == 0) return true;
    float scale = (float)(1.0 / (double)T->state.pending_steps);
    if (T->opt.loss_scale > 0) scale /= T->opt.loss_scale;
    if (!hip_ok(tr_apply(T, scale, (int)T->state.adam_t + 1), "optimizer step")) return false;
    T->state.adam_t++;
    T->state.pending_steps = 0;
    T->state.cum_batches++;
    return true;
}

// One step on a given window: forward, loss, backward, then Adam (or, with accumulation, the
// gradients added to the pending sums and Adam once AccumSteps windows are in); the loss comes
// back.
bool tr_step_window(sh_trainer *T, const uint16_t *in, const uint16_t *tgt, float *loss_out) {
    (void)hipSetDevice(T->device);
    const int S = T->S;
    std::vector<int32_t> ids = compact_ids(tgt, S, T->V);
    const int U = (int)ids.size();
    // the input ids' positions, grouped by id (order of first appearance), positions ascending
    std::vector<int32_t> in_ids, in_off(1, 0), in_occ;
    {
        std::vector<int32_t> slot(T->V, -1);
        std::vector<std::vector<int32_t>> pos;
        for (int t = 0; t < S; t++) {
            const int tok = in[t];
            if (tok >= T->V) continue;
            if (slot[tok] < 0) {
                slot[tok] = (int32_t)in_ids.size();
                in_ids.push_back(tok);
                pos.emplace_back();
            }
            pos[slot[tok]].push_back(t);
        }
        for (auto &p : pos) {
            in_occ.insert(in_occ.end(), p.begin(), p.end());
            in_off.push_back((int32_t)in_occ.size());
        }
    }
    const int n_in = (int)in_ids.size();
    if (!hip_ok(hipMemcpyAsync(T->tok_in, in, 2 * (size_t)S, hipMemcpyHostToDevice, T->stream), "tokens") ||
        !hip_ok(hipMemcpyAsync(T->tok_tgt, tgt, 2 * (size_t)S, hipMemcpyHostToDevice, T->stream), "targets") ||
        (U && !hip_ok(hipMemcpyAsync(T->ids, ids.data(), 4 * (size_t)U, hipMemcpyHostToDevice, T->stream), "ids")) ||
        (n_in && !hip_ok(hipMemcpyAsync(T->in_ids, in_ids.data(), 4 * (size_t)n_in, hipMemcpyHostToDevice,
                                        T->stream), "ids")) ||
        (n_in && !hip_ok(hipMemcpyAsync(T->in_off, in_off.data(), 4 * (size_t)(n_in + 1), hipMemcpyHostToDevice,
                                        T->stream), "ids")) ||
        (n_in && !hip_ok(hipMemcpyAsync(T->in_occ, in_occ.data(), 4 * in_occ.size(), hipMemcpyHostToDevice,
                                        T->stream), "ids")) ||
        !hip_ok(hipEventRecord(T->ev0, T->stream), "event"))
        return false;
    // AccumSteps > 1: the first window after a flush stores its gradients, later ones add
    const bool accumulate = T->opt.accum_steps > 1;
    const bool acc = accumulate && T->state.pending_steps > 0;
    if (!hip_ok(tr_forward_head(T, U, T->opt.loss_scale, acc), "training forward") ||
        !hip_ok(tr_backward(T, n_in, acc), "training backward"))
        return false;
    if (!accumulate) {
        const float ls = T->opt.loss_scale;
        const float inv = (ls != 0 && ls != 1) ? (float)(1.0 / (double)ls) : 1.f;
        if (!hip_ok(tr_apply(T, inv, (int)T->state.adam_t + 1), "optimizer step")) return false;
        T->state.adam_t++;   // train_full.go:844-845
        T->state.cum_batches++;
    } else if (++T->state.pending_steps >= (uint32_t)T->opt.accum_steps) {   // train_full.go:769-772
        if (!tr_flush(T)) return false;
    }
    if (!hip_ok(hipEventRecord(T->ev1, T->stream), "event")) return false;
    float lv[2];
    if (!hip_ok(hipMemcpyAsync(lv, T->loss, sizeof lv, hipMemcpyDeviceToHost, T->stream), "loss") ||
        !hip_ok(hipStreamSynchronize(T->stream), "step sync"))
        return false;
    float ms = 0;
    (void)hipEventElapsedTime(&ms, T->ev0, T->ev1);
    T->state.last_loss = lv[0];
    T->state.cum_steps++;
    T->state.last_step_ms = ms;
    if (loss_out) *loss_out = lv[0];
    return true;
}

}  // namespace
}  // namespace sh

using namespace sh;

extern "C" {

sh_trainer *sh_trainer_create(const sh_config *cfg, const sh_train_options *opt_in) {
    if (!cfg) {
        set_error("sh_trainer_create: nil config");
        return nullptr;
    }
    const sh_config &c = *cfg;
    if (c.dim <= 0 || c.hidden <= 0 || c.n_layers <= 0 || c.n_heads <= 0 || c.head_dim <= 0 || c.vocab <= 0 ||
        c.n_heads * c.head_dim != c.dim || c.n_kv_heads != c.n_heads || c.qk_norm || c.head_dim > 64 ||
        c.head_dim % 4 || c.dim % 4 || c.hidden % 4 || c.vocab % 4 || c.vocab > 65535) {
        set_error("sh_trainer_create: the training step needs a Stories-shaped model: n_heads*head_dim == dim, "
                  "n_kv_heads == n_heads, no qk_norm, head_dim <= 64 and a multiple of 4, dim/hidden/vocab "
                  "multiples of 4, vocab <= 65535");
        return nullptr;
    }
    sh_train_options o{};
    if (opt_in) o = *opt_in;
    // Open's defaults (engine.go:153-186)
    if (o.seq <= 0) o.seq = 256;
    if (o.lr <= 0) o.lr = 3e-4f;
    if (o.accum_steps <= 0) o.accum_steps = 1;
    if (o.seed == 0) o.seed = 42;
    if (o.beta1 <= 0) o.beta1 = 0.9f;
    if (o.beta2 <= 0) o.beta2 = 0.999f;
    if (o.eps <= 0) o.eps = 1e-8f;
    if (o.grad_clip < 0) o.grad_clip = 0;
    if (o.loss_scale <= 0) o.loss_scale = 256;
    if (o.seq > 4096) {
        set_error("sh_trainer_create: seq must be <= 4096");
        return nullptr;
    }
    sh_trainer *T = new sh_trainer();
    T->cfg = c;
    T->opt = o;
    T->device = 0;
    (void)hipGetDevice(&T->device);
    T->S = o.seq;
    T->D = c.dim;
    T->F = c.hidden;
    T->H = c.n_heads;
    T->hd = c.head_dim;
    T->V = c.vocab;
    T->L = c.n_layers;
    T->uploaded.assign(T->L, false);
    T->uploaded_globals = false;
    const size_t D = T->D, F = T->F, V = T->V, S = T->S;
    size_t off = 0;
    for (int l = 0; l < T->L; l++) {
        T->o_qkv.push_back(off); off += 3 * D * D;
        T->o_wo.push_back(off); off += D * D;
        T->o_w13.push_back(off); off += 2 * F * D;
        T->o_w2.push_back(off); off += D * F;
    }
    T->o_embed = off; off += V * D;
    T->n_mat = off;
    for (int l = 0; l < T->L; l++) {
        T->o_ra.push_back(off); off += D;
        T->o_rf.push_back(off); off += D;
    }
    T->o_rfin = off; off += D;
    T->n_all = off;
    T->ldc_u = (int)((S + 3) / 4 * 4);
    // activations: per layer x, xn, qkv, att, x2, x2n, h13, gate, ra, rf; then the head and scratch
    size_t a = 0;
    auto take = [&](size_t bytes) { size_t o2 = a; a += (bytes + 255) / 256 * 256; return o2; };
    struct Off { size_t x, xn, ra, qkv, att, x2, x2n, rf, h13, gate; };
    std::vector<Off> lo(T->L);
    for (int l = 0; l < T->L; l++) {
        lo[l].x = take(4 * S * D); lo[l].xn = take(4 * S * D); lo[l].ra = take(4 * S);
        lo[l].qkv = take(4 * S * 3 * D); lo[l].att = take(4 * S * D); lo[l].x2 = take(4 * S * D);
        lo[l].x2n = take(4 * S * D); lo[l].rf = take(4 * S); lo[l].h13 = take(4 * S * 2 * F);
        lo[l].gate = take(4 * S * F);
    }
    const size_t o_xL = take(4 * S * D), o_xnf = take(4 * S * D), o_rfin = take(4 * S), o_lg = take(4 * S * V),
                 o_dy = take(4 * S * D), o_dcur = take(4 * S * D), o_gx2 = take(4 * S * D),
                 o_gxn = take(4 * S * D), o_gatt = take(4 * S * D), o_ggate = take(4 * S * F),
                 o_dh13 = take(4 * S * 2 * F), o_dqkv = take(4 * S * 3 * D), o_stats = take(4 * 3 * T->H * S * T->L),
                 o_dlc = take(4 * S * T->ldc_u), o_gc = take(4 * S * D), o_loss = take(16),
                 o_cos = take(4 * S * (T->hd / 2)), o_sin = take(4 * S * (T->hd / 2)), o_rl = take(8 * S),
                 o_sq = take(8 * kSqParts), o_rv = take(4 * S), o_ids = take(4 * S), o_ti = take(2 * S),
                 o_tt = take(2 * S), o_iid = take(4 * S), o_ioff = take(4 * (S + 1)), o_iocc = take(4 * S),
                 o_part = take(4 * 16 * S * std::max(3 * D, 2 * F));
    bool ok = hip_ok(hipStreamCreate(&T->stream), "stream") && hip_ok(hipEventCreate(&T->ev0), "event") &&
              hip_ok(hipEventCreate(&T->ev1), "event") &&
              hip_ok(hipMalloc(&T->p, 4 * T->n_all), "hipMalloc params") &&
              hip_ok(hipMalloc(&T->g, 4 * T->n_all), "hipMalloc grads") &&
              hip_ok(hipMalloc(&T->m, 4 * T->n_all), "hipMalloc adam m") &&
              hip_ok(hipMalloc(&T->v, 4 * T->n_all), "hipMalloc adam v") &&
              hip_ok(hipMalloc(&T->act, a), "hipMalloc activations") &&
              hip_ok(hipMemset(T->p, 0, 4 * T->n_all), "clear") && hip_ok(hipMemset(T->g, 0, 4 * T->n_all), "clear") &&
              hip_ok(hipMemset(T->m, 0, 4 * T->n_all), "clear") && hip_ok(hipMemset(T->v, 0, 4 * T->n_all), "clear");
    if (!ok) {
        sh_trainer_destroy(T);
        return nullptr;
    }
    uint8_t *A = (uint8_t *)T->act;
    T->lc.resize(T->L);
    for (int l = 0; l < T->L; l++) {
        auto &C = T->lc[l];
        C.x = (float *)(A + lo[l].x); C.xn = (float *)(A + lo[l].xn); C.ra = (float *)(A + lo[l].ra);
        C.qkv = (float *)(A + lo[l].qkv); C.att = (float *)(A + lo[l].att); C.x2 = (float *)(A + lo[l].x2);
        C.x2n = (float *)(A + lo[l].x2n); C.rf = (float *)(A + lo[l].rf); C.h13 = (float *)(A + lo[l].h13);
        C.gate = (float *)(A + lo[l].gate);
    }
    T->xL = (float *)(A + o_xL); T->xnf = (float *)(A + o_xnf); T->rfin = (float *)(A + o_rfin);
    T->logits = (float *)(A + o_lg); T->dy = (float *)(A + o_dy); T->dcur = (float *)(A + o_dcur);
    T->gx2 = (float *)(A + o_gx2);
    T->gxn = (float *)(A + o_gxn); T->gatt = (float *)(A + o_gatt);
    T->ggate = (float *)(A + o_ggate); T->dh13 = (float *)(A + o_dh13); T->dqkv = (float *)(A + o_dqkv);
    T->stats = (float *)(A + o_stats); T->dlc = (float *)(A + o_dlc); T->gc = (float *)(A + o_gc);
    T->loss = (float *)(A + o_loss); T->cos_t = (float *)(A + o_cos); T->sin_t = (float *)(A + o_sin);
    T->row_loss = (double *)(A + o_rl); T->sq_part = (double *)(A + o_sq); T->row_valid = (int *)(A + o_rv);
    T->ids = (int32_t *)(A + o_ids); T->tok_in = (uint16_t *)(A + o_ti); T->tok_tgt = (uint16_t *)(A + o_tt);
    T->in_ids = (int32_t *)(A + o_iid); T->in_off = (int32_t *)(A + o_ioff); T->in_occ = (int32_t *)(A + o_iocc);
    T->part = (float *)(A + o_part);
    T->part_cap = 16 * S * std::max(3 * D, 2 * F);
    // rope.go:5-24 buildRoPETables(seq, headDim): float64 angles, float32 cos / sin
    const int half = T->hd / 2;
    std::vector<float> cs((size_t)S * half), sn((size_t)S * half);
    for (size_t p = 0; p < S; p++)
        for (int i = 0; i < half; i++) {
            const double f = (double)p / pow(c.rope_theta, (double)(2 * i) / (double)T->hd);
            cs[p * half + i] = (float)cos(f);
            sn[p * half + i] = (float)sin(f);
        }
    if (!hip_ok(hipMemcpy(T->cos_t, cs.data(), 4 * cs.size(), hipMemcpyHostToDevice), "rope tables") ||
        !hip_ok(hipMemcpy(T->sin_t, sn.data(), 4 * sn.size(), hipMemcpyHostToDevice), "rope tables")) {
        sh_trainer_destroy(T);
        return nullptr;
    }
    T->rng = (((uint64_t)o.seed & 0xffffffffull) << 16) | 0x330E;   // engine.go:725-727
    T->state = sh_train_state{};
    return T;
}

int sh_trainer_upload_layer(sh_trainer *T, int32_t layer, const float *wq, const float *wk, const float *wv,
                            const float *wo, const float *w1, const float *w2, const float *w3,
                            const float *rms_att, const float *rms_ffn) {
    if (!T || layer < 0 || layer >= T->L || !wq || !wk || !wv || !wo || !w1 || !w2 || !w3 || !rms_att ||
        !rms_ffn) {
        set_error("sh_trainer_upload_layer: bad arguments");
        return -1;
    }
    (void)hipSetDevice(T->device);
    const size_t D = T->D, F = T->F;
    float *p = T->p;
    const bool ok =
        hip_ok(hipMemcpy(p + T->o_qkv[layer], wq, 4 * D * D, hipMemcpyHostToDevice), "upload") &&
        hip_ok(hipMemcpy(p + T->o_qkv[layer] + D * D, wk, 4 * D * D, hipMemcpyHostToDevice), "upload") &&
        hip_ok(hipMemcpy(p + T->o_qkv[layer] + 2 * D * D, wv, 4 * D * D, hipMemcpyHostToDevice), "upload") &&
        hip_ok(hipMemcpy(p + T->o_wo[layer], wo, 4 * D * D, hipMemcpyHostToDevice), "upload") &&
        hip_ok(hipMemcpy(p + T->o_w13[layer], w1, 4 * F * D, hipMemcpyHostToDevice), "upload") &&
        hip_ok(hipMemcpy(p + T->o_w13[layer] + F * D, w3, 4 * F * D, hipMemcpyHostToDevice), "upload") &&
        hip_ok(hipMemcpy(p + T->o_w2[layer], w2, 4 * D * F, hipMemcpyHostToDevice), "upload") &&
        hip_ok(hipMemcpy(p + T->o_ra[layer], rms_att, 4 * D, hipMemcpyHostToDevice), "upload") &&
        hip_ok(hipMemcpy(p + T->o_rf[layer], rms_ffn, 4 * D, hipMemcpyHostToDevice), "upload");
    if (ok) T->uploaded[layer] = true;
    return ok ? 0 : -1;
}

int sh_trainer_upload_globals(sh_trainer *T, const float *embed, const float *rms_final) {
    if (!T || !embed || !rms_final) {
        set_error("sh_trainer_upload_globals: bad arguments");
        return -1;
    }
    (void)hipSetDevice(T->device);
    const bool ok = hip_ok(hipMemcpy(T->p + T->o_embed, embed, 4 * (size_t)T->V * T->D, hipMemcpyHostToDevice),
                           "upload") &&
                    hip_ok(hipMemcpy(T->p + T->o_rfin, rms_final, 4 * (size_t)T->D, hipMemcpyHostToDevice), "upload");
    if (ok) T->uploaded_globals = true;
    return ok ? 0 : -1;
}

int sh_trainer_set_tokens(sh_trainer *T, const uint16_t *tokens, int64_t n) {
    if (!T || (!tokens && n)) {
        set_error("sh_trainer_set_tokens: bad arguments");
        return -1;
    }
    T->tokens.assign(tokens, tokens + n);
    return 0;
}

int sh_trainer_step(sh_trainer *T, float *loss) {
    if (!tr_ready(T)) return -1;
    const int S = T->S;
    if ((int64_t)T->tokens.size() < S + 1) {
        set_error("sh_trainer_step: not enough tokens");   // engine.go:299-301
        return -1;
    }
    // engine.go:307-316: the window start from drand48
    const uint64_t limit = (uint64_t)(T->tokens.size() - S - 1);
    uint64_t pos = 0;
    if (limit > 0) {
        T->rng = (0x5DEECE66Dull * T->rng + 0xBull) & ((1ull << 48) - 1);
        pos = (uint64_t)((double)T->rng / (double)(1ull << 48) * (double)limit);
        if (pos >= limit) pos = limit - 1;
    }
    T->state.token_pos = pos + S;
    return tr_step_window(T, T->tokens.data() + pos, T->tokens.data() + pos + 1, loss) ? 0 : -1;
}

int sh_trainer_step_window(sh_trainer *T, const uint16_t *input, const uint16_t *target, float *loss) {
    if (!tr_ready(T)) return -1;
    if (!input || !target) {
        set_error("sh_trainer_step_window: bad arguments");
        return -1;
    }
    return tr_step_window(T, input, target, loss) ? 0 : -1;
}

int sh_trainer_flush(sh_trainer *T) {
    if (!T) {
        set_error("storiesane flush: engine is closed");   // engine.go:399-401
        return -1;
    }
    (void)hipSetDevice(T->device);
    return tr_flush(T) && hip_ok(hipStreamSynchronize(T->stream), "flush sync") ? 0 : -1;
}

int sh_trainer_read(const sh_trainer *T, int32_t which, const char *name, float *dst, size_t n) {
    if (!T || !name || !dst || which < 0 || which > 3) {
        set_error("sh_trainer_read: bad arguments");
        return -1;
    }
    const float *base = which == SH_TRAIN_PARAMS ? T->p : which == SH_TRAIN_GRADS ? T->g
                        : which == SH_TRAIN_ADAM_M ? T->m : T->v;
    const size_t D = T->D, F = T->F;
    size_t off = 0, len = 0;
    const std::string s(name);
    int layer = -1;
    char key[32] = {0};
    if (s == "embed") {
        off = T->o_embed;
        len = (size_t)T->V * D;
    } else if (s == "rms_final") {
        off = T->o_rfin;
        len = D;
    } else if (sscanf(name, "layers.%d.%31s", &layer, key) == 2 && layer >= 0 && layer < T->L) {
        const std::string k(key);
        if (k == "wq") { off = T->o_qkv[layer]; len = D * D; }
        else if (k == "wk") { off = T->o_qkv[layer] + D * D; len = D * D; }
        else if (k == "wv") { off = T->o_qkv[layer] + 2 * D * D; len = D * D; }
        else if (k == "wo") { off = T->o_wo[layer]; len = D * D; }
        else if (k == "w1") { off = T->o_w13[layer]; len = F * D; }
        else if (k == "w3") { off = T->o_w13[layer] + F * D; len = F * D; }
        else if (k == "w2") { off = T->o_w2[layer]; len = D * F; }
        else if (k == "rms_att") { off = T->o_ra[layer]; len = D; }
        else if (k == "rms_ffn") { off = T->o_rf[layer]; len = D; }
    }
    if (!len) {
        set_error(std::string("sh_trainer_read: unknown tensor ") + name);
        return -1;
    }
    if (n != len) {
        set_error(std::string("sh_trainer_read: ") + name + " has " + std::to_string(len) + " values");
        return -1;
    }
    (void)hipSetDevice(T->device);
    return hip_ok(hipMemcpy(dst, base + off, 4 * len, hipMemcpyDeviceToHost), "read") ? 0 : -1;
}

int sh_trainer_state(const sh_trainer *T, sh_train_state *out) {
    if (!T || !out) {
        set_error("sh_trainer_state: nil argument");
        return -1;
    }
    *out = T->state;
    return 0;
}

void sh_trainer_destroy(sh_trainer *T) {
    if (!T) return;
    (void)hipSetDevice(T->device);
    (void)hipFree(T->p);
    (void)hipFree(T->g);
    (void)hipFree(T->m);
    (void)hipFree(T->v);
    (void)hipFree(T->act);
    if (T->stream) (void)hipStreamDestroy(T->stream);
    if (T->ev0) (void)hipEventDestroy(T->ev0);
    if (T->ev1) (void)hipEventDestroy(T->ev1);
    delete T;
}

}  // extern "C"
