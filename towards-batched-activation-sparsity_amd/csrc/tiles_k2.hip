// tiles_k2.hip — instantiated tiles of libbsgemm: kind 2 (X staged in LDS, waves split columns).

#include "bsg_device.hpp"

namespace bsgk {

namespace {
const KernelEntry kEntries[] = {
    BSG_X(1, 1, 2, 4), BSG_X(1, 1, 4, 4), BSG_X(1, 1, 4, 8), BSG_X(1, 1, 8, 4), BSG_X(1, 2, 2, 4),
    BSG_X(1, 2, 4, 4),
    BSG_X(2, 1, 2, 4), BSG_X(2, 1, 4, 4), BSG_X(2, 1, 4, 8), BSG_X(2, 2, 2, 4), BSG_X(2, 2, 4, 4),
    BSG_X(4, 1, 2, 4), BSG_X(4, 1, 4, 4), BSG_X(4, 1, 4, 8), BSG_X(4, 1, 8, 4), BSG_X(4, 2, 2, 2),
    BSG_X(4, 2, 2, 4), BSG_X(4, 2, 4, 2), BSG_X(4, 2, 4, 4), BSG_X(4, 4, 2, 2), BSG_X(4, 4, 4, 2),
};
}  // namespace

const TileTable kTilesK2 = {kEntries, (int)(sizeof kEntries / sizeof kEntries[0])};

}  // namespace bsgk
