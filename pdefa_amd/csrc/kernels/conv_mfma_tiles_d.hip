// Implicit-GEMM conv kernel instances for 3 tile shapes (one of the
// translation units conv_mfma_tiles_*.hip that split the instances so that
// they compile in parallel); the kernels are in conv_mfma_tile.hpp.
#include "conv_mfma_tile.hpp"

namespace pdefa {
namespace k {

bool launch_conv_tiles_d(int tile, const ConvArgs& a, bool vec, dim3 grid, hipStream_t s) {
    switch (tile) {
        case kTile64x128: launch_tile<64, 128, 32, 64, 1>(a, vec, grid, s); return true;
        case kTile32x64K2: launch_tile<32, 64, 32, 32, 2>(a, vec, grid, s); return true;
        case kTile32x64K4W8: launch_tile<32, 64, 32, 32, 4>(a, vec, grid, s); return true;
        default: return false;
    }
}

bool launch_group_tiles_d(int tile, const ConvGroupArgs& g, hipStream_t s) {
    switch (tile) {
        case kTile64x128: launch_group<64, 128, 32, 64, 1, kPrefetch>(g, s); return true;
        case kTile32x64K2: launch_group<32, 64, 32, 32, 2, kPrefetch>(g, s); return true;
        case kTile32x64K4W8: launch_group<32, 64, 32, 32, 4, kPrefetch>(g, s); return true;
        default: return false;
    }
}

}  // namespace k
}  // namespace pdefa
