// Implicit-GEMM conv kernel instances for 4 tile shapes (one of the
// translation units conv_mfma_tiles_*.hip that split the instances so that
// they compile in parallel); the kernels are in conv_mfma_tile.hpp.
#include "conv_mfma_tile.hpp"

namespace pdefa {
namespace k {

bool launch_conv_tiles_b(int tile, const ConvArgs& a, bool vec, dim3 grid, hipStream_t s) {
    switch (tile) {
        case kTile128x128W8: launch_tile<128, 128, 64, 32, 1>(a, vec, grid, s); return true;
        case kTile128x32: launch_tile<128, 32, 32, 32, 1>(a, vec, grid, s); return true;
        case kTile32x16K4: launch_tile<32, 16, 32, 16, 4>(a, vec, grid, s); return true;
        case kTile16x32K8W8: launch_tile<16, 32, 16, 32, 8>(a, vec, grid, s); return true;
        default: return false;
    }
}

bool launch_group_tiles_b(int tile, const ConvGroupArgs& g, hipStream_t s) {
    switch (tile) {
        case kTile128x128W8: launch_group<128, 128, 64, 32, 1, kPrefetch>(g, s); return true;
        case kTile128x32: launch_group<128, 32, 32, 32, 1, kPrefetch>(g, s); return true;
        case kTile32x16K4: launch_group<32, 16, 32, 16, 4, kPrefetch>(g, s); return true;
        case kTile16x32K8W8: launch_group<16, 32, 16, 32, 8, kPrefetch>(g, s); return true;
        default: return false;
    }
}

}  // namespace k
}  // namespace pdefa
