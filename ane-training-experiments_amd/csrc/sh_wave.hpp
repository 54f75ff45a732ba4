// sh_wave.hpp — cross-lane reductions for wave64 on gfx950 built from DPP lane moves and the
// CDNA4 permlane swaps, instead of ds_bpermute (which goes through the LDS crossbar and costs
// a round trip of LDS latency per step).
//
// A group is N consecutive lanes (N a power of two, 2..64, groups aligned to N). After
// wsum<N>(v) every lane of a group holds the same value, the group's sum, combined as a
// butterfly: pairs, quads, 8-lane halves of a row, 16-lane rows, 32-lane halves, the wave.
//   xor 1, xor 2: DPP quad_perm [1,0,3,2] and [2,3,0,1]
//   8 lanes:      DPP row_half_mirror (lane i <- 7 - i within 8; the quads are uniform by then)
//   16 lanes:     DPP row_mirror (lane i <- 15 - i within a row)
//   32 lanes:     v_permlane16_swap (rows 0<->1 and 2<->3 exchanged between two registers)
//   64 lanes:     v_permlane32_swap (the two 32-lane halves exchanged)
// Each step adds two values that are equal on both partners, so the result is bitwise
// uniform across the group.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace sh {

constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // row_half_mirror
constexpr int kDppMirror = 0x140;     // row_mirror
constexpr int kDppRowShl8 = 0x108;    // row_shl:8 (lane i <- i + 8 within a row)

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

// Generic 32-bit lane moves and combination, so one butterfly serves float, int and the
// two halves of a double.
struct SwapPair {
    uint32_t a, b;   // a: the register's own rows/half kept or received, b: the other
};
__device__ __forceinline__ SwapPair swap16(uint32_t v) {
    const auto s = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return SwapPair{s[0], s[1]};
}
__device__ __forceinline__ SwapPair swap32(uint32_t v) {
    const auto s = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return SwapPair{s[0], s[1]};
}

template <int N>
__device__ __forceinline__ float wsum(float v) {
    static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "group of 1..64 lanes");
    if constexpr (N >= 2) v += __uint_as_float(dpp_u<kDppXor1>(__float_as_uint(v)));
    if constexpr (N >= 4) v += __uint_as_float(dpp_u<kDppXor2>(__float_as_uint(v)));
    if constexpr (N >= 8) v += __uint_as_float(dpp_u<kDppHalfMirror>(__float_as_uint(v)));
    if constexpr (N >= 16) v += __uint_as_float(dpp_u<kDppMirror>(__float_as_uint(v)));
    if constexpr (N >= 32) {
        const SwapPair s = swap16(__float_as_uint(v));
        v = __uint_as_float(s.a) + __uint_as_float(s.b);
    }
    if constexpr (N >= 64) {
        const SwapPair s = swap32(__float_as_uint(v));
        v = __uint_as_float(s.a) + __uint_as_float(s.b);
    }
    return v;
}

template <int N>
__device__ __forceinline__ int wsum_i(int v) {
    static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "group of 1..64 lanes");
    if constexpr (N >= 2) v += (int)dpp_u<kDppXor1>((uint32_t)v);
    if constexpr (N >= 4) v += (int)dpp_u<kDppXor2>((uint32_t)v);
    if constexpr (N >= 8) v += (int)dpp_u<kDppHalfMirror>((uint32_t)v);
    if constexpr (N >= 16) v += (int)dpp_u<kDppMirror>((uint32_t)v);
    if constexpr (N >= 32) {
        const SwapPair s = swap16((uint32_t)v);
        v = (int)s.a + (int)s.b;
    }
    if constexpr (N >= 64) {
        const SwapPair s = swap32((uint32_t)v);
        v = (int)s.a + (int)s.b;
    }
    return v;
}

template <int N>
__device__ __forceinline__ float wmax(float v) {
    static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "group of 1..64 lanes");
    if constexpr (N >= 2) v = fmaxf(v, __uint_as_float(dpp_u<kDppXor1>(__float_as_uint(v))));
    if constexpr (N >= 4) v = fmaxf(v, __uint_as_float(dpp_u<kDppXor2>(__float_as_uint(v))));
    if constexpr (N >= 8) v = fmaxf(v, __uint_as_float(dpp_u<kDppHalfMirror>(__float_as_uint(v))));
    if constexpr (N >= 16) v = fmaxf(v, __uint_as_float(dpp_u<kDppMirror>(__float_as_uint(v))));
    if constexpr (N >= 32) {
        const SwapPair s = swap16(__float_as_uint(v));
        v = fmaxf(__uint_as_float(s.a), __uint_as_float(s.b));
    }
    if constexpr (N >= 64) {
        const SwapPair s = swap32(__float_as_uint(v));
        v = fmaxf(__uint_as_float(s.a), __uint_as_float(s.b));
    }
    return v;
}

// float64 sum over the whole wave (both 32-bit halves moved by the same lane moves).
__device__ __forceinline__ double wsum_d64(double v) {
    auto step_dpp = [](double x, auto ctrl_tag) {
        constexpr int C = decltype(ctrl_tag)::value;
        const uint64_t b = (uint64_t)__double_as_longlong(x);
        const uint32_t lo = dpp_u<C>((uint32_t)b), hi = dpp_u<C>((uint32_t)(b >> 32));
        return x + __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
    };
    v = step_dpp(v, std::integral_constant<int, kDppXor1>{});
    v = step_dpp(v, std::integral_constant<int, kDppXor2>{});
    v = step_dpp(v, std::integral_constant<int, kDppHalfMirror>{});
    v = step_dpp(v, std::integral_constant<int, kDppMirror>{});
    {
        const uint64_t b = (uint64_t)__double_as_longlong(v);
        const SwapPair lo = swap16((uint32_t)b), hi = swap16((uint32_t)(b >> 32));
        v = __longlong_as_double((long long)(((uint64_t)hi.a << 32) | lo.a)) +
            __longlong_as_double((long long)(((uint64_t)hi.b << 32) | lo.b));
    }
    {
        const uint64_t b = (uint64_t)__double_as_longlong(v);
        const SwapPair lo = swap32((uint32_t)b), hi = swap32((uint32_t)(b >> 32));
        v = __longlong_as_double((long long)(((uint64_t)hi.a << 32) | lo.a)) +
            __longlong_as_double((long long)(((uint64_t)hi.b << 32) | lo.b));
    }
    return v;
}

// Value of lane + D for the lanes of the lower half of each group of 2D lanes (D = 8, 16,
// 32); other lanes receive an unspecified value.
template <int D>
__device__ __forceinline__ float from_lane_up(float v) {
    static_assert(D == 8 || D == 16 || D == 32, "D = 8, 16 or 32");
    if constexpr (D == 8) return __uint_as_float(dpp_u<kDppRowShl8>(__float_as_uint(v)));
    if constexpr (D == 16) return __uint_as_float(swap16(__float_as_uint(v)).b);
    return __uint_as_float(swap32(__float_as_uint(v)).b);
}

// First-maximum (value, index) over the whole wave: larger value, then smaller index.
__device__ __forceinline__ bool arg_better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}
template <int CTRL>
__device__ __forceinline__ void argmax_dpp_step(float &v, int &i) {
    const float ov = __uint_as_float(dpp_u<CTRL>(__float_as_uint(v)));
    const int oi = (int)dpp_u<CTRL>((uint32_t)i);
    if (arg_better(ov, oi, v, i)) {
        v = ov;
        i = oi;
    }
}
__device__ __forceinline__ void argmax_swap_step(SwapPair sv, SwapPair si, float &v, int &i) {
    float a = __uint_as_float(sv.a), b = __uint_as_float(sv.b);
    int ia = (int)si.a, ib = (int)si.b;
    if (arg_better(b, ib, a, ia)) {
        a = b;
        ia = ib;
    }
    v = a;
    i = ia;
}
__device__ __forceinline__ void wargmax(float &v, int &i) {
    argmax_dpp_step<kDppXor1>(v, i);
    argmax_dpp_step<kDppXor2>(v, i);
    argmax_dpp_step<kDppHalfMirror>(v, i);
    argmax_dpp_step<kDppMirror>(v, i);
    argmax_swap_step(swap16(__float_as_uint(v)), swap16((uint32_t)i), v, i);
    argmax_swap_step(swap32(__float_as_uint(v)), swap32((uint32_t)i), v, i);
}

}  // namespace sh
