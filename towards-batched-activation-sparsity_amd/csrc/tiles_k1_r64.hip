// tiles_k1_r64.hip — instantiated tiles of libbsgemm: kind 1, 64 batch rows.

#include "bsg_device.hpp"

namespace bsgk {

namespace {
const KernelEntry kEntries[] = {
    BSG_K(4, 2, 1, 4), BSG_K(4, 2, 2, 2), BSG_K(4, 2, 2, 4), BSG_K(4, 2, 4, 2),
    BSG_K(4, 4, 1, 2), BSG_K(4, 4, 1, 4), BSG_K(4, 4, 2, 2), BSG_K(4, 4, 4, 1),
    BSG_K(4, 4, 4, 2),
    BSG_K(4, 8, 1, 2), BSG_K(4, 8, 2, 1), BSG_K(4, 8, 2, 2),
};
}  // namespace

const TileTable kTilesK1R64 = {kEntries, (int)(sizeof kEntries / sizeof kEntries[0])};

}  // namespace bsgk
