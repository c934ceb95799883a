// Implicit-GEMM conv kernel instances for 4 tile shapes (one of the
// translation units conv_mfma_tiles_*.hip that split the instances so that
// they compile in parallel); the kernels are in conv_mfma_tile.hpp.
#include "conv_mfma_tile.hpp"

namespace pdefa {
namespace k {

bool launch_conv_tiles_a(int tile, const ConvArgs& a, bool vec, dim3 grid, hipStream_t s) {
    switch (tile) {
        case kTile128x128: launch_tile<128, 128, 64, 64, 1>(a, vec, grid, s); return true;
        case kTile64x64: launch_tile<64, 64, 32, 32, 1>(a, vec, grid, s); return true;
        case kTile16x16K4: launch_tile<16, 16, 16, 16, 4>(a, vec, grid, s); return true;
        case kTile16x32K4: launch_tile<16, 32, 16, 32, 4>(a, vec, grid, s); return true;
        default: return false;
    }
}

bool launch_group_tiles_a(int tile, const ConvGroupArgs& g, hipStream_t s) {
    switch (tile) {
        case kTile128x128: launch_group<128, 128, 64, 64, 1, kPrefetch>(g, s); return true;
        case kTile64x64: launch_group<64, 64, 32, 32, 1, kPrefetch>(g, s); return true;
        case kTile16x16K4: launch_group<16, 16, 16, 16, 4, kPrefetch>(g, s); return true;
        case kTile16x32K4: launch_group<16, 32, 16, 32, 4, kPrefetch>(g, s); return true;
        default: return false;
    }
}

}  // namespace k
}  // namespace pdefa
