// `.engine` model: graph + host weights, parsed from the file format the
// reference loader reads (PDEFA1.0/src/loader/custom_loader.cpp:62-214).
#pragma once

#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "host_tensor.hpp"

namespace pdefa {

// OpType codes of the format (PDEFA1.0/include/engine/graph.hpp:20-73).
enum Op : int32_t {
    kOpUnknown = 0, kOpConv = 1, kOpMatMul = 2, kOpAdd = 3, kOpMul = 4, kOpSub = 5, kOpDiv = 6,
    kOpRelu = 10, kOpLeaky = 11, kOpSigmoid = 12, kOpTanh = 13, kOpSilu = 14, kOpGelu = 15,
    kOpMaxPool = 20, kOpAvgPool = 21, kOpBatchNorm = 22, kOpSoftmax = 30, kOpConcat = 31,
    kOpUpsample = 32, kOpResize = 33, kOpInput = 40, kOpOutput = 41, kOpReshape = 42,
    kOpTranspose = 43, kOpSlice = 44, kOpTopK = 50, kOpGatherElements = 51,
};
const char* op_name(int32_t op);

// The 128-byte OpParams record (PDEFA1.0/include/engine/graph.hpp:78-95),
// decoded field by field.
struct OpParams {
    int64_t stride_h = 1, stride_w = 1, pad_h = 0, pad_w = 0, dil_h = 1, dil_w = 1, groups = 1;
    int64_t kernel_h = 2, kernel_w = 2;
    int32_t axis = -1;
    int64_t scale_h = 2, scale_w = 2, target_h = 0, target_w = 0;
    uint8_t upsample_mode = 0;
    float eps = 1e-5f;
    uint8_t fused_activation = 0;
    float leaky_slope = 0.01f;
};

struct Node {
    int32_t op = kOpUnknown;
    std::string name;
    std::vector<int32_t> inputs;
    std::vector<int32_t> outputs;
    OpParams params;
};

// Input/output metadata of a v2 file.  dtype keeps the file's own DType code
// (12 = F32, PDEFA1.0/include/engine/dtype.hpp:36-62).
struct TensorInfo {
    std::string name;
    int32_t ndim = 0;
    int64_t shape[kMaxNdim] = {0, 0, 0, 0, 0, 0, 0, 0};
    int32_t dtype = 12;
};

struct DeviceModel;  // weights resident in HBM (runtime.hpp)

struct Model {
    std::string name;
    std::string source_path;  // the .engine file it was read from ("" when built otherwise)
    int32_t version = 0;
    std::vector<HostTensor> weights;
    std::vector<std::string> weight_names;
    std::vector<Node> nodes;
    std::vector<int32_t> graph_inputs;
    std::vector<int32_t> graph_outputs;
    std::vector<TensorInfo> input_infos;
    std::vector<TensorInfo> output_infos;

    std::mutex device_mu;
    std::shared_ptr<DeviceModel> device;  // created on first use on a GPU

    int32_t num_inputs() const { return static_cast<int32_t>(graph_inputs.size()); }
    int32_t num_outputs() const { return static_cast<int32_t>(graph_outputs.size()); }
};

// Parses `path`.  Returns false (and a reason) on a missing file, bad magic or
// version, truncation, or a weight dtype other than F32.
bool load_engine_file(const std::string& path, Model& out, std::string* why);

// Maps the file's DType code to the public EngineDType (F32 when unknown),
// as engine_api.cpp:70-82 does.
int32_t public_dtype(int32_t file_dtype);

}  // namespace pdefa
