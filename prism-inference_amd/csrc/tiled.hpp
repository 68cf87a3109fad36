// tiled.hpp -- the device layout of packed weight tensors ("64-row tiles").
//
// A tensor [rows][cols] in a native format (PTQ1 28 B/128, PQ2 34 B/128, Q2_K
// 84 B/256, Q8_0 34 B/32; src/kernels.rs:88-142) is stored on the device as
// tiles of 64 consecutive rows.  Inside a tile the row's "units" (128 weights;
// 256 for Q2_K) are stored unit-major, and each unit is split into pieces of
// 16, 8, 4 or 2 bytes.  Piece p of unit u of tile-row r sits at
//
//     tile_base + u * TRP * UB + poff[p] * TRP + r * psize[p]
//
// where UB is the unit's byte count and TRP the tile's row count rounded up to a
// multiple of 8 (64 for every tile but the last, whose padding rows are zero).
// A wavefront whose lane r owns tile-row r therefore reads every piece with one
// fully contiguous load instruction.  The bytes are the native bytes, permuted:
// the layout moves no more data than the native one (only the last tile carries
// up to 7 zero rows of padding), and the arithmetic is unchanged.
#pragma once

#include <stdint.h>

namespace prism {

constexpr uint32_t kTile = 64;

struct TiledFormat {
    uint32_t unit_weights;  // weights per unit
    uint32_t unit_bytes;    // native bytes per unit
    uint32_t npieces;
    uint32_t psize[9];      // piece sizes (bytes)
    uint32_t poff[9];       // piece offsets in units of TRP bytes (= prefix sums of psize)
    uint32_t nsrc[9];       // native byte offset of each piece within the unit
};

// PTQ1 (143): codes 0..15 | codes 16..23 | codes 24..25 + f16 scale.
// PQ2 (142): codes 2..17 | codes 18..33 | f16 scale 0..1.
// Q2_K (10): codes 16..79 in four pieces | sub-block scales 0..15 | d, dmin 80..83.
// Q8_0 (8), four 34-byte blocks per unit: codes of block j in pieces 2j, 2j+1
//   (native 34j+2 .. 34j+33) | the four f16 scales, block j's at bytes 2j..2j+1.
// TQ1_0 (34): codes 0..15 | 16..31 | 32..47 | 48..51 | f16 scale 52..53.
// TQ2_0 (35): codes 0..63 in four pieces | f16 scale 64..65.
__host__ __device__ inline bool tiled_format(uint32_t kind, TiledFormat *f) {
    switch (kind) {
    case 143:
        *f = {128, 28, 3, {16, 8, 4}, {0, 16, 24}, {0, 16, 24}};
        return true;
    case 142:
        *f = {128, 34, 3, {16, 16, 2}, {0, 16, 32}, {2, 18, 0}};
        return true;
    case 10:
        *f = {256, 84, 6, {16, 16, 16, 16, 16, 4}, {0, 16, 32, 48, 64, 80}, {16, 32, 48, 64, 0, 80}};
        return true;
    case 34:
        *f = {256, 54, 5, {16, 16, 16, 4, 2}, {0, 16, 32, 48, 52}, {0, 16, 32, 48, 52}};
        return true;
    case 35:
        *f = {256, 66, 5, {16, 16, 16, 16, 2}, {0, 16, 32, 48, 64}, {0, 16, 32, 48, 64}};
        return true;
    case 8:
        // The scale piece gathers four 2-byte fields; nsrc = 0 marks the gather.
        *f = {128, 136, 9, {16, 16, 16, 16, 16, 16, 16, 16, 8}, {0, 16, 32, 48, 64, 80, 96, 112, 128},
              {2, 18, 36, 52, 70, 86, 104, 120, 0}};
        return true;
    default:
        return false;
    }
}

__host__ __device__ inline uint32_t tile_rows_padded(uint64_t rows, uint64_t tile) {
    const uint64_t left = rows - tile * kTile;
    const uint32_t tr = left < kTile ? static_cast<uint32_t>(left) : kTile;
    return (tr + 7u) & ~7u;
}

// Device bytes of the tiled image (native bytes plus the last tile's padding rows).
__host__ __device__ inline uint64_t tiled_bytes(uint64_t rows, uint64_t row_bytes) {
    const uint64_t tiles = (rows + kTile - 1) / kTile;
    return ((tiles - 1) * kTile + tile_rows_padded(rows, tiles - 1)) * row_bytes;
}

}  // namespace prism
