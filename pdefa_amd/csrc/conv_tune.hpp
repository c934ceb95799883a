// Measured launch-shape choice for the implicit-GEMM convolution: the cost
// model ranks the candidate (tile, split-K) shapes, each candidate is timed on
// the device on scratch buffers of the layer's exact shape, and the fastest
// is kept for the life of the process (keyed by shape and device).  Choices
// found in the device kind's launch-shape table (tuning/<arch>.txt, measured
// once on such a device) are taken from it without timing, so that every
// process plans the same launch shapes and computes the same bits.
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

// Number of shapes chosen so far (tests and diagnostics).
size_t conv_tune_cache_size();

// Choices (single convs and groups) measured in this process, and taken from
// the launch-shape table.
void conv_tune_stats(size_t& measured, size_t& from_table);

}  // namespace pdefa
