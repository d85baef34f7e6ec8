// tiles_k3.hip — instantiated tiles of libbsgemm: kind 3 (fp32 dot products, 1-8 batch rows, X staged in LDS).

#include "bsg_device.hpp"

namespace bsgk {

namespace {
const KernelEntry kEntries[] = {
    BSG_F(1, 1, 2, 4), BSG_F(1, 1, 4, 4), BSG_F(1, 1, 4, 8), BSG_F(1, 1, 8, 4), BSG_F(1, 2, 4, 4),
    BSG_F(2, 1, 2, 4), BSG_F(2, 1, 4, 4), BSG_F(2, 1, 4, 8), BSG_F(2, 1, 8, 4), BSG_F(2, 2, 4, 4),
    BSG_F(4, 1, 2, 4), BSG_F(4, 1, 4, 4), BSG_F(4, 1, 4, 8), BSG_F(4, 1, 8, 4), BSG_F(4, 2, 4, 4),
    BSG_F(8, 1, 2, 4), BSG_F(8, 1, 4, 4), BSG_F(8, 1, 4, 8), BSG_F(8, 1, 8, 4), BSG_F(8, 2, 4, 4),
};
}  // namespace

const TileTable kTilesK3 = {kEntries, (int)(sizeof kEntries / sizeof kEntries[0])};

}  // namespace bsgk
