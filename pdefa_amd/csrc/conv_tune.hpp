// Measured launch-shape choice for the implicit-GEMM convolution: the cost
// model ranks the candidate (tile, split-K) shapes, each candidate is timed on
// the device on scratch buffers of the layer's exact shape, and the fastest
// is kept for the life of the process (keyed by shape and device).
#pragma once

#include <hip/hip_runtime.h>

#include <vector>

#include "kernels.hpp"
#include "planner.hpp"

namespace pdefa {

// Called while planning, outside any stream capture; synchronises `s`.
k::ConvLaunchShape tune_conv(const ConvQuery& q, hipStream_t s);

// Times independent layers run one after another, each with its own launch
// shape `solo`, against one grouped launch for every implicit-GEMM tile
// (kept per process like tune_conv's choices).
ConvGroupTiming tune_conv_group(const std::vector<ConvQuery>& qs, const std::vector<k::ConvLaunchShape>& solo,
                                hipStream_t s);

// Number of shapes chosen by measurement so far (tests and diagnostics).
size_t conv_tune_cache_size();

}  // namespace pdefa
