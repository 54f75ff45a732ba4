// sh_tiles.hpp — workgroup-to-tile orders that keep the tiles sharing data on one XCD.
//
// MI355X has 8 XCDs, each with its own L2. The dispatcher deals the workgroups of a grid to
// the XCDs in turn (linear workgroup b to XCD b mod 8), and each XCD starts its share in
// order. A grid whose neighbouring workgroups read the same operand panels therefore spreads
// every panel over all 8 L2s, and each XCD fetches it from memory for itself. These orders
// give each XCD a consecutive range of logical tiles instead, so the tiles it runs together
// share its L2.
#pragma once

#include <hip/hip_runtime.h>

namespace sh {

// Workgroup b of a 1-D grid of nb runs logical tile xcd_tile(b, nb): XCD x takes logical
// tiles [x * nb/8, (x + 1) * nb/8) in order. (A tail of nb mod 8 workgroups keeps its own
// order.)
__device__ __forceinline__ int xcd_tile(int b, int nb) {
    const int nfull = nb & ~7;
    return b < nfull ? (b & 7) * (nfull >> 3) + (b >> 3) : b;
}

// The output tile (tx of gx, ty of gy) of this workgroup of a gx x gy grid (per blockIdx.z):
// groups of GM consecutive x tiles, each group's tiles y by y, in xcd_tile's order. With x the
// row tiles of a GEMM, the tiles an XCD runs together (two per CU) cover GM row panels of A x
// a few column panels of W, each read from memory once for the XCD instead of once per tile
// (on 32 x 1023 rows the row-tile-first grid fetched every A panel of the Qwen3-shaped q|k|v
// product once per column tile: 4.1 GB per layer against 1.26 GB with GM = 8). Measured: GM =
// 8 for the 128 x 128 tiles of long inputs (16: 102.5 -> 106 ms per 32 x 1023-row prefill),
// 4 for the short inputs' pipelined tiles (EvalLogits 0.551 -> 0.547 ms).
template <int GM = 8>
__device__ __forceinline__ void gemm_tile(int &tx, int &ty) {
    const int gx = gridDim.x, gy = gridDim.y;
    const int t = xcd_tile(blockIdx.x + blockIdx.y * gx, gx * gy);
    const int per = GM * gy, grp = t / per, first = grp * GM;
    const int gm = min(gx - first, GM), r = t - grp * per;
    tx = first + r % gm;
    ty = r / gm;
}

}  // namespace sh
