// MFMA tiling of one linear of the persistent sequence, shared by the device kernel and the
// host plan compiler (which checks the limits with the same arithmetic the kernel uses).
//
// Workgroup g of G owns output features r0 .. r0 + nr - 1 (an even split of N).  Its
// "virtual rows" are those features' weight rows, followed (SiLU-gate) by the partner W2's
// rows: V = nr or 2 nr.  The share is computed with v_mfma_f32_16x16x32 tiles: A = 16
// virtual rows x 32 k of weights (one 16-byte chunk per lane), B = 32 k x 16 columns of
// activations, D = 16 x 16 fp32 partial sums.  Every activation is split into hi + lo
// halves of the weights' type, and the two halves are separate B columns.
//   - V > 16: RT = ceil(V / 16) row tiles, S = 1 segment; A row a of row tile rt is
//     virtual row 16 rt + a and B column c is x row c / 2, half c % 2.
//   - V <= 16: one row tile holds S in {1, 2, 4} K-segments of the share side by side
//     (the largest with V S <= 16, M S <= 8, S <= KB), interleaved: A row a is virtual row
//     a / S over segment a % S, B column c is x row (c / 2) / S over segment (c / 2) % S,
//     half c % 2, and only the entries of D whose row and column have the same segment
//     are kept.  For a given (virtual row, x row) they sit in 2 S neighbouring lanes, so a
//     lane-group sum adds the segments and both halves.
// Segment s covers 32-k blocks s KBs .. s KBs + KBs - 1 (KBs = ceil(KB / S)); a tile is
// (row tile rt, block step j), numbered t = rt KBs + j, T = RT KBs in all, and compute
// wave w of the workgroup's NW takes the contiguous tile range [w T / NW, (w + 1) T / NW).
#pragma once

#include <stdint.h>

namespace mt {

struct SeqTiles {
    uint32_t r0, nr;  // features of the share
    uint32_t V;       // virtual rows
    uint32_t S;       // K segments per row tile (1, 2 or 4)
    uint32_t ls;      // log2 S
    uint32_t RT;      // row tiles
    uint32_t KB;      // 32-k blocks of K
    uint32_t KBs;     // blocks per segment
    uint32_t T;       // tiles
};

__host__ __device__ inline SeqTiles seq_tiles(uint32_t N, uint32_t K, uint32_t M, bool gated, uint32_t g,
                                              uint32_t G) {
    SeqTiles t;
    t.r0 = static_cast<uint32_t>(static_cast<uint64_t>(g) * N / G);
    t.nr = static_cast<uint32_t>(static_cast<uint64_t>(g + 1) * N / G) - t.r0;
    t.V = t.nr * (gated ? 2u : 1u);
    t.KB = (K + 31) / 32;
    t.S = 1;
    t.ls = 0;
    if (t.V == 0) {
        t.RT = 0;
    } else if (t.V <= 16) {
        while (t.S < 4 && 2 * t.S * t.V <= 16 && 2 * t.S * M <= 8 && 2 * t.S <= t.KB) {
            t.S *= 2;
            t.ls++;
        }
        t.RT = 1;
    } else {
        t.RT = (t.V + 15) / 16;
    }
    t.KBs = (t.KB + t.S - 1) / t.S;
    t.T = t.RT * t.KBs;
    return t;
}

// Tile range of wave w of nw.
__host__ __device__ inline uint32_t seq_tile_begin(uint32_t T, uint32_t w, uint32_t nw) { return w * T / nw; }

}  // namespace mt
