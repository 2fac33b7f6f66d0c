// XCD-aware placement of GEMM work items (output tiles x K ranges) onto the
// workgroups of a 1-D grid, shared by the GEMM kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace bsq {

// Work item of workgroup blockIdx.x in a 1-D grid of ny x nx output tiles
// times `splits` K ranges.  The hardware deals consecutive workgroups to the
// 8 XCDs round-robin (blockIdx.x % 8), and each XCD has its own L2: give XCD
// x a contiguous range of the logical order, which walks the K ranges
// outermost and, inside one, the tiles in groups of G tile rows with the
// column index outermost, so the workgroups resident on one XCD share a few
// A panels and a few B panels instead of touching every panel of both
// operands (which re-fetches them from HBM).  Outputs at most eight tiles
// wide (the range finder's n x q products) take G = 1, plain row order:
// every tile of a row panel then runs on the same XCD and the panel is
// fetched once.  The split index is part of the linear order, so the
// mapping stays XCD-aligned whatever the number of tiles.  A bijection onto
// the work items for any grid size.
constexpr int kXcds = 8, kGroupRows = 8;
__device__ __forceinline__ void xcd_tile(int ny, int nx, int splits, int &tm, int &tn, int &z) {
    const int bid = blockIdx.x;
    const int T = ny * nx, W = T * splits;
    const int xcd = bid % kXcds, loc = bid / kXcds;
    const int per = W / kXcds, rem = W % kXcds;
    const int L = xcd * per + min(xcd, rem) + loc;
    z = L / T;
    const int t = L - z * T;
    const int G = nx <= 8 ? 1 : kGroupRows;
    const int span = G * nx;
    const int first = (t / span) * G;
    const int rows = min(ny - first, G);
    const int in = t % span;
    tm = first + in % rows;
    tn = in / rows;
}

}  // namespace bsq
