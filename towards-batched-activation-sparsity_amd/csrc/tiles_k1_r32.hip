// tiles_k1_r32.hip — instantiated tiles of libbsgemm: kind 1, 32 batch rows.

#include "bsg_device.hpp"

namespace bsgk {

namespace {
const KernelEntry kEntries[] = {
    BSG_K(2, 2, 1, 4), BSG_K(2, 2, 2, 4), BSG_K(2, 2, 4, 2), BSG_K(2, 2, 4, 4),
    BSG_K(2, 4, 1, 4), BSG_K(2, 4, 2, 2), BSG_K(2, 4, 2, 4), BSG_K(2, 4, 4, 2),
};
}  // namespace

const TileTable kTilesK1R32 = {kEntries, (int)(sizeof kEntries / sizeof kEntries[0])};

}  // namespace bsgk
