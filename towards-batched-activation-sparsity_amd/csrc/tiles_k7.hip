// Kind 7 tiles (kind 6 with the activations staged in LDS by 16-byte-per-lane loads): rows / 16,
// subtiles per work-group (at most), block-slice waves, prefetch depth.  Every tile keeps its
// wave reduction inside the waves' own activation slots (subtiles <= 2 x depth) and its LDS
// within a compute unit's 160 KiB.
#include "bsg_device.hpp"

namespace bsgk {

namespace {
const KernelEntry kEntries[] = {
    // 64 rows: 256 groups of 2-3 subtiles at N = 11008 / 12288, two, four or eight block-slice
    // waves (eight: two per SIMD)
    BSG_V1X(4, 3, 4, 2), BSG_V1X(4, 3, 4, 3), BSG_V1X(4, 3, 4, 4), BSG_V1X(4, 3, 2, 4), BSG_V1X(4, 2, 4, 2),
    BSG_V1X(4, 2, 4, 4), BSG_V1X(4, 3, 8, 2), BSG_V1X(4, 2, 8, 2),
    // 32 rows (one row group of a 32-row batch, or half of a 64-row one)
    BSG_V1X(2, 2, 4, 2), BSG_V1X(2, 3, 4, 2), BSG_V1X(2, 2, 4, 4), BSG_V1X(2, 3, 4, 4), BSG_V1X(2, 4, 4, 2),
    BSG_V1X(2, 2, 8, 2), BSG_V1X(2, 3, 8, 2),
    // 16 rows
    BSG_V1X(1, 1, 4, 4), BSG_V1X(1, 2, 4, 4), BSG_V1X(1, 3, 4, 4),
};
}  // namespace

const TileTable kTilesK7 = {kEntries, (int)(sizeof kEntries / sizeof kEntries[0])};

}  // namespace bsgk
