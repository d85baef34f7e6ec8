// tiles_k1_r16.hip — instantiated tiles of libbsgemm: kind 1, 16 batch rows.

#include "bsg_device.hpp"

namespace bsgk {

namespace {
const KernelEntry kEntries[] = {
    BSG_K(1, 1, 1, 4), BSG_K(1, 1, 1, 8), BSG_K(1, 1, 2, 4), BSG_K(1, 1, 2, 8),
    BSG_K(1, 1, 4, 2), BSG_K(1, 1, 4, 4), BSG_K(1, 1, 4, 8), BSG_K(1, 1, 8, 2),
    BSG_K(1, 1, 8, 4), BSG_K(1, 1, 8, 8),
    BSG_K(1, 2, 1, 4), BSG_K(1, 2, 1, 8), BSG_K(1, 2, 2, 4), BSG_K(1, 2, 2, 8),
    BSG_K(1, 2, 4, 2), BSG_K(1, 2, 4, 4), BSG_K(1, 2, 4, 8), BSG_K(1, 2, 8, 2),
    BSG_K(1, 2, 8, 4),
    BSG_K(1, 4, 1, 4), BSG_K(1, 4, 2, 4), BSG_K(1, 4, 4, 2), BSG_K(1, 4, 4, 4),
    BSG_K(1, 4, 8, 2),
    BSG_K(1, 8, 1, 2), BSG_K(1, 8, 2, 2), BSG_K(1, 8, 4, 2),
};
}  // namespace

const TileTable kTilesK1R16 = {kEntries, (int)(sizeof kEntries / sizeof kEntries[0])};

}  // namespace bsgk
