// Kind 5 tiles (variable-width column groups, channel-half x block-slice waves) and kind 6 (the
// same groups, waves split the blocks only): rows / 16, subtiles per work-group (at most), waves,
// prefetch depth.
#include "bsg_device.hpp"

namespace bsgk {

namespace {
const KernelEntry kEntries[] = {
    BSG_V(1, 1, 2, 4), BSG_V(1, 1, 4, 4), BSG_V(1, 1, 8, 4), BSG_V(1, 2, 2, 4), BSG_V(1, 2, 4, 4),
    BSG_V(1, 2, 8, 4), BSG_V(1, 3, 2, 4), BSG_V(1, 3, 4, 4), BSG_V(1, 3, 8, 4), BSG_V(1, 4, 2, 4),
    BSG_V(1, 4, 4, 4), BSG_V(1, 6, 2, 4), BSG_V(1, 6, 4, 4),
    BSG_V(2, 1, 2, 4), BSG_V(2, 1, 4, 4), BSG_V(2, 2, 2, 4), BSG_V(2, 2, 4, 4), BSG_V(2, 3, 2, 4),
    BSG_V(2, 3, 4, 4), BSG_V(2, 4, 2, 4), BSG_V(2, 4, 4, 4), BSG_V(2, 6, 2, 4), BSG_V(2, 6, 4, 4),
    BSG_V(4, 1, 2, 4), BSG_V(4, 1, 4, 4), BSG_V(4, 2, 2, 4), BSG_V(4, 2, 4, 4), BSG_V(4, 3, 2, 4),
    BSG_V(4, 3, 4, 4), BSG_V(4, 4, 2, 4), BSG_V(4, 4, 4, 4), BSG_V(4, 6, 2, 4), BSG_V(4, 6, 4, 2),
    // kind 6: every wave both channel halves, waves split the blocks
    BSG_V1(1, 3, 2, 4), BSG_V1(1, 3, 4, 4), BSG_V1(2, 3, 2, 4), BSG_V1(2, 3, 4, 2), BSG_V1(4, 3, 2, 2),
    BSG_V1(4, 3, 4, 2), BSG_V1(4, 2, 4, 2), BSG_V1(4, 3, 2, 4), BSG_V1(1, 1, 4, 4), BSG_V1(1, 2, 4, 4),
    // more loads in flight per compute unit for short slices (a slice costs one round of loads
    // per `depth` blocks): 8 block-slice waves, or depth 8
    BSG_V1(1, 1, 8, 4), BSG_V1(1, 1, 4, 8), BSG_V1(1, 2, 8, 4), BSG_V1(1, 2, 4, 8), BSG_V1(2, 1, 4, 4),
    BSG_V1(2, 2, 4, 4), BSG_V1(2, 1, 8, 4),
    // 6-subtile groups at 64 rows (N = 22016 over 256 compute units)
    BSG_V1(4, 6, 2, 2), BSG_V1(4, 6, 4, 2),
    // 32-row groups for 64-row batches (two row groups per column group; the second read of each
    // weight line is an L2 hit on the same XCD): more block-slice waves and prefetch depth
    BSG_V1(2, 2, 8, 4), BSG_V1(2, 2, 4, 8), BSG_V1(2, 3, 4, 4), BSG_V1(2, 4, 4, 4), BSG_V1(2, 4, 2, 4),
};
}  // namespace

const TileTable kTilesK5 = {kEntries, (int)(sizeof kEntries / sizeof kEntries[0])};

}  // namespace bsgk
