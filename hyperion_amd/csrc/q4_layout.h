// Device-resident layout of a Q4/g64 projection ("tiled" layout).
//
// The reference keeps weights in MLX's layout (native/hyperion_mlx/src/weights.h:18-25:
// codes uint32 [n, k/8], scales and biases bf16 [n, k/64]). That layout is the I/O
// format here too (upload, export, quantize output); once resident, a projection is
// stored tile-major so that every load instruction of the kernels reads contiguous
// bytes:
//
//   tiles  = ceil(n / 16) row tiles of 16 rows; pairs = ceil(k / 128) pairs of groups.
//   codes  uint4 [tiles][pairs][64]: entry l = kb * 16 + j (kb in 0..3, j in 0..15)
//          holds, for row 16 * tile + j, packed words 2kb and 2kb+1 of group 2 * pair
//          (.x, .y) and of group 2 * pair + 1 (.z, .w). One pair of one tile is 1 KB.
//   sb     uint2 [tiles][pairs][16]: entry j holds (scale | bias << 16) of row
//          16 * tile + j for group 2 * pair (.x) and group 2 * pair + 1 (.y) as bf16
//          bit patterns. One pair of one tile is 128 B.
//   Rows past n and the group past k / 64 (odd group counts) are zero.
//
// With n % 16 == 0 and (k / 64) even the tiled layout has exactly the MLX layout's size.
#pragma once

#include <cstdint>

namespace hyperion::hip {

constexpr uint32_t kTileRows = 16;

struct TiledDims {
    uint32_t tiles;   // ceil(n / 16)
    uint32_t pairs;   // ceil(k / 128)

    static TiledDims of(uint32_t n, uint32_t k) {
        return TiledDims{(n + kTileRows - 1u) / kTileRows, (k / 64u + 1u) / 2u};
    }
    uint64_t code_bytes() const { return static_cast<uint64_t>(tiles) * pairs * 1024u; }
    uint64_t sb_bytes() const { return static_cast<uint64_t>(tiles) * pairs * 128u; }
};

}  // namespace hyperion::hip
