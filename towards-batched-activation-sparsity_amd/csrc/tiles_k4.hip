// tiles_k4.hip — instantiated tiles of libbsgemm: kind 4 (as kind 2, waves also split the two channel halves of every block).

#include "bsg_device.hpp"

namespace bsgk {

namespace {
const KernelEntry kEntries[] = {
    BSG_Y(4, 1, 8, 4), BSG_Y(4, 1, 8, 2), BSG_Y(4, 1, 8, 8), BSG_Y(4, 2, 8, 2), BSG_Y(4, 2, 8, 4),
    BSG_Y(4, 1, 4, 4), BSG_Y(4, 2, 4, 4), BSG_Y(4, 1, 4, 8),
    BSG_Y(2, 1, 8, 4), BSG_Y(2, 1, 4, 4), BSG_Y(2, 2, 4, 4),
    BSG_Y(1, 1, 8, 4), BSG_Y(1, 1, 4, 4),
};
}  // namespace

const TileTable kTilesK4 = {kEntries, (int)(sizeof kEntries / sizeof kEntries[0])};

}  // namespace bsgk
