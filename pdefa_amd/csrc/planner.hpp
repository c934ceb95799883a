// Lowers an `.engine` graph to a fixed device program for one input shape.
//
// Semantics are the ONNX operator semantics the reference session realises on
// the YOLOv8 path (PDEFA1.0/src/core/session.cpp:181-425 and
// session_parts/*.inc); layout is the planner's own: every rank-3/4
// intermediate is channels-last in one HBM arena, Slice/Reshape/Transpose are
// strided views, Concat inputs are written by their producers straight into
// the concat buffer, Conv -> Sigmoid -> Mul becomes the conv's SiLU epilogue
// (the fusion of session_fusion.inc:33-107) and a C2f residual Add becomes a
// conv epilogue add.
#pragma once

#include <climits>
#include <cstdint>
#include <functional>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "model.hpp"

namespace pdefa {

constexpr int32_t kBufWeight = -2;  // VRef::buf for a model weight (aux = weight index)

// A strided view of a planned buffer (or of a model weight).
struct VRef {
    int32_t buf = -1;
    int32_t aux = 0;
    int64_t off = 0;
    int32_t rank = 0;
    int64_t dims[k::kMaxRank] = {0, 0, 0, 0, 0, 0};
    int64_t str[k::kMaxRank] = {0, 0, 0, 0, 0, 0};
};

enum class StepKind : int32_t {
    ConvMfma, ConvDirect, Elt, MaxPool, Resize, Softmax, MaxPoolChain, DetectDecode, TopK, GatherElements
};

// Steps whose `b` view is a second input (read).
inline bool reads_second_input(StepKind k) { return k == StepKind::Elt || k == StepKind::GatherElements; }

struct Step {
    StepKind kind = StepKind::Elt;
    int32_t node = -1;  // graph node the step implements (first of a fused group)
    VRef out, a, b, res;
    VRef c;  // MaxPoolChain: third output; DetectDecode: divisor view
    bool has_res = false;
    // conv
    int32_t act = 0;
    float slope = 0.01f;
    int32_t KH = 1, KW = 1, sh = 1, sw = 1, ph = 0, pw = 0, dh = 1, dw = 1;
    int32_t tile = 0;
    bool vec = false;
    int32_t splits = 1, kt_per_split = 0;
    int32_t ws_buf = -1;
    int32_t groups = 1;  // conv groups (the weight holds Cin / groups input channels)
    // ConvMfma: nearest 2x upsample of out, written by the same epilogue
    // (up.buf == -1: none); it replaces the Resize step that read out
    VRef up;
    // >= 0: consecutive ConvMfma steps with the same id run as one grouped
    // launch of their common tile (k::launch_conv_mfma_group)
    int32_t group = -1;
    // eltwise
    int32_t elt = 0;
    float alpha = 0.0f;
    // softmax, topk, gather elements
    int32_t axis = 0;
    // TopK: the k largest along `axis` (ties: lower index first); this step
    // writes the values, or with topk_indices the indices (as float values)
    int64_t topk = 0;
    bool topk_indices = false;
    // DetectDecode: the DFL conv's weight (and bias) indices, number of bins,
    // and optionally (cls_in.buf != -1) the class scores whose sigmoid it
    // also writes to cls_out
    int32_t dfl_weight = -1;
    int32_t dfl_bias = -1;
    int32_t bins = 0;
    VRef cls_in, cls_out;
};

struct Buffer {
    int64_t elems = 0;
    int32_t first = INT32_MAX;
    int32_t last = -1;
    int64_t offset = 0;  // elements from the arena base
};

struct Plan {
    std::vector<std::vector<int64_t>> input_dims;
    std::vector<int32_t> input_bufs;          // contiguous NCHW staging, one per graph input
    std::vector<VRef> outputs;                // contiguous views, graph_outputs order
    std::vector<std::vector<int64_t>> output_dims;
    std::vector<bool> output_int32;           // the output holds indices (TopK), returned as I32
    std::vector<Step> steps;
    std::vector<Buffer> bufs;
    int64_t arena_elems = 0;
    int32_t n_copies = 0;                     // materialising copies the planner could not avoid
    // Leading steps that work image by image (convs and elementwise steps
    // whose views all have the batch as their outer dimension) on maps of at
    // least PlanOptions::early_hw pixels: they may run on chunks of the batch
    // as the input arrives.  Their buffers never share memory with each other.
    int32_t early_steps = 0;
};

// Shape of one implicit-GEMM conv (channels-last input and output).
struct ConvQuery {
    int32_t N, H, W, Cin, Ho, Wo, Cout, KH, KW, sh, sw, ph, pw, dh, dw, act;
    bool has_res, vec;
    bool wino;  // the Winograd kernel applies (3x3, stride 1, dilation 1, Cin % 4 == 0)
    int32_t groups = 1;  // Cin and Cout count all channels
};

// Measured comparison of independent convs launched one by one (each with
// its own launch shape) against one grouped launch of the fastest tile.
struct ConvGroupTiming {
    int tile = -1;             // fastest implicit-GEMM tile for the grouped launch
    double group_ms = 0.0;     // its time
    double separate_ms = 0.0;  // the layers launched one by one
};

struct PlanOptions {
    // When set, chooses the launch shape of every implicit-GEMM conv (the
    // runtime times candidates on the device); otherwise the cost model does.
    std::function<k::ConvLaunchShape(const ConvQuery&)> tune_conv;
    // When set (with tune_conv), independent convs that are ready at the same
    // point of the program are reordered next to each other and issued as one
    // grouped launch wherever the measurement says that is faster.
    std::function<ConvGroupTiming(const std::vector<ConvQuery>&, const std::vector<k::ConvLaunchShape>&)> tune_group;
    bool split_k = true;
    int force_tile = -1;   // >= 0: use this implicit-GEMM tile for every MFMA conv (tuning, tests)
    int force_splits = 0;  // > 0 with force_tile: split-K across workgroups into this many splits
    bool reuse_memory = true;  // share arena memory between tensors with disjoint lifetimes
    bool winograd_form_silu = true;  // match the reference's Winograd-layer SiLU
    // Split a fused Detect decode into one step per anchor range written by
    // different producers (the scales of a YOLO head) and, where the program
    // is reordered (tune_group), run each range's producers and its decode
    // before the next range's: the first ranges' outputs are then final while
    // the rest of the program still runs, so their download can overlap it.
    bool split_outputs = false;
    // > 0: Plan::early_steps covers the leading per-image steps whose outputs
    // have at least this many pixels (H * W)
    int64_t early_hw = 0;
};

// Throws std::runtime_error naming the node for an unsupported op or pattern.
Plan build_plan(const Model& m, const std::vector<std::vector<int64_t>>& input_dims, const PlanOptions& opt);

// Concurrent issue of a plan: steps ordered by the arena ranges they read and
// write (true and false data hazards); each step gets a capture stream, the
// steps it must wait for on other streams, and whether another stream waits
// for it.  Steps on one stream run in plan order.
struct Schedule {
    int n_streams = 1;
    std::vector<int> stream;              // per step
    std::vector<std::vector<int>> waits;  // per step: earlier steps on other streams
    std::vector<bool> recorded;           // per step: some later step waits for it
    std::vector<std::vector<int>> deps;   // per step: all direct hazards (before reduction)
};
Schedule schedule_plan(const Plan& p, int max_streams);

// Human-readable dump (one line per step) for tests and debugging.
std::string describe_plan(const Model& m, const Plan& p);

}  // namespace pdefa
