#include "model.hpp"

#include <cstdio>
#include <cstring>

namespace pdefa {

const char* op_name(int32_t op) {
    switch (op) {
        case kOpConv: return "Conv2d";
        case kOpMatMul: return "MatMul";
        case kOpAdd: return "Add";
        case kOpMul: return "Mul";
        case kOpSub: return "Sub";
        case kOpDiv: return "Div";
        case kOpRelu: return "ReLU";
        case kOpLeaky: return "LeakyReLU";
        case kOpSigmoid: return "Sigmoid";
        case kOpTanh: return "Tanh";
        case kOpSilu: return "SiLU";
        case kOpGelu: return "GELU";
        case kOpMaxPool: return "MaxPool2d";
        case kOpAvgPool: return "AvgPool2d";
        case kOpBatchNorm: return "BatchNorm2d";
        case kOpSoftmax: return "Softmax";
        case kOpConcat: return "Concat";
        case kOpUpsample: return "Upsample";
        case kOpResize: return "Resize";
        case kOpInput: return "Input";
        case kOpOutput: return "Output";
        case kOpReshape: return "Reshape";
        case kOpTranspose: return "Transpose";
        case kOpSlice: return "Slice";
        case kOpTopK: return "TopK";
        case kOpGatherElements: return "GatherElements";
        default: return "Unknown";
    }
}

int32_t public_dtype(int32_t d) {
    switch (d) {
        case 12: return kF32;
        case 10: return kF16;
        case 11: return kBF16;
        case 2: return kI8;
        case 3: return kU8;
        case 6: return kI32;
        case 8: return kI64;
        case 1: return kBool;
        default: return kF32;
    }
}

namespace {

constexpr uint32_t kMagic = 0x4E474E45u;  // "ENGN"
constexpr size_t kParamsSize = 128;

class Reader {
   public:
    explicit Reader(std::FILE* f) : f_(f) {}
    template <typename T>
    bool pod(T& v) { return std::fread(&v, sizeof(T), 1, f_) == 1; }
    bool bytes(void* dst, size_t n) { return n == 0 || std::fread(dst, 1, n, f_) == n; }
    bool str(std::string& s, uint32_t limit = 4096) {
        uint32_t n = 0;
        if (!pod(n) || n > limit) return false;
        s.assign(n, '\0');
        return bytes(s.data(), n);
    }

   private:
    std::FILE* f_;
};

template <typename T>
T at(const unsigned char* p, size_t off) {
    T v;
    std::memcpy(&v, p + off, sizeof(T));
    return v;
}

OpParams decode_params(const unsigned char* p) {
    OpParams o;
    o.stride_h = at<int64_t>(p, 0);
    o.stride_w = at<int64_t>(p, 8);
    o.pad_h = at<int64_t>(p, 16);
    o.pad_w = at<int64_t>(p, 24);
    o.dil_h = at<int64_t>(p, 32);
    o.dil_w = at<int64_t>(p, 40);
    o.groups = at<int64_t>(p, 48);
    o.kernel_h = at<int64_t>(p, 56);
    o.kernel_w = at<int64_t>(p, 64);
    o.axis = at<int32_t>(p, 72);
    o.scale_h = at<int64_t>(p, 80);
    o.scale_w = at<int64_t>(p, 88);
    o.target_h = at<int64_t>(p, 96);
    o.target_w = at<int64_t>(p, 104);
    o.upsample_mode = at<uint8_t>(p, 112);
    o.eps = at<float>(p, 116);
    o.fused_activation = at<uint8_t>(p, 120);
    o.leaky_slope = at<float>(p, 124);
    return o;
}

bool read_info(Reader& r, TensorInfo& t) {
    if (!r.str(t.name)) return false;
    uint8_t nd = 0;
    if (!r.pod(nd) || nd > kMaxNdim) return false;
    t.ndim = nd;
    for (int d = 0; d < nd; ++d)
        if (!r.pod(t.shape[d])) return false;
    uint8_t dt = 0;
    if (!r.pod(dt)) return false;
    t.dtype = dt;
    return true;
}

struct WMeta {
    std::string name;
    uint8_t dtype = 0;
    int32_t rank = 0;
    int64_t dims[kMaxNdim] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint64_t offset = 0, size = 0;
};

}  // namespace

bool load_engine_file(const std::string& path, Model& m, std::string* why) {
    auto fail = [&](const char* msg) {
        if (why) *why = msg;
        return false;
    };
    std::FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return fail("cannot open model file");
    struct Closer {
        std::FILE* f;
        ~Closer() { std::fclose(f); }
    } closer{f};
    Reader r(f);

    uint32_t magic = 0, version = 0, nw = 0, nn = 0, ni = 0, no = 0;
    char brand[64];
    if (!r.pod(magic) || !r.pod(version)) return fail("truncated header");
    if (magic != kMagic) return fail("bad magic");
    if (version != 1 && version != 2) return fail("unsupported version");
    if (!r.pod(nw) || !r.pod(nn) || !r.pod(ni) || !r.pod(no) || !r.bytes(brand, sizeof(brand)))
        return fail("truncated header");

    std::vector<WMeta> wm(nw);
    for (auto& w : wm) {
        uint8_t rank = 0;
        if (!r.str(w.name) || !r.pod(w.dtype) || !r.pod(rank)) return fail("truncated weight table");
        if (rank > kMaxNdim) return fail("weight rank > 8");
        w.rank = rank;
        for (int d = 0; d < rank; ++d)
            if (!r.pod(w.dims[d])) return fail("truncated weight table");
        if (!r.pod(w.offset) || !r.pod(w.size)) return fail("truncated weight table");
    }

    std::vector<Node> nodes(nn);
    for (auto& n : nodes) {
        uint8_t op = 0;
        uint16_t nin = 0, nout = 0;
        if (!r.pod(op) || !r.str(n.name)) return fail("truncated node table");
        if (!r.pod(nin) || nin > 64 || !r.pod(nout) || nout > 64) return fail("bad node arity");
        n.op = op;
        n.inputs.resize(nin);
        n.outputs.resize(nout);
        for (auto& v : n.inputs)
            if (!r.pod(v)) return fail("truncated node table");
        for (auto& v : n.outputs)
            if (!r.pod(v)) return fail("truncated node table");
        unsigned char raw[kParamsSize];
        if (!r.bytes(raw, kParamsSize)) return fail("truncated node params");
        n.params = decode_params(raw);
    }

    std::vector<int32_t> gin(ni), gout(no);
    for (auto& v : gin)
        if (!r.pod(v)) return fail("truncated graph inputs");
    for (auto& v : gout)
        if (!r.pod(v)) return fail("truncated graph outputs");

    std::vector<TensorInfo> iinfo, oinfo;
    if (version >= 2) {
        iinfo.resize(ni);
        oinfo.resize(no);
        for (auto& t : iinfo)
            if (!read_info(r, t)) return fail("truncated input info");
        for (auto& t : oinfo)
            if (!read_info(r, t)) return fail("truncated output info");
    }

    const long data_start = std::ftell(f);
    if (data_start < 0) return fail("ftell failed");

    std::vector<HostTensor> weights;
    std::vector<std::string> names;
    weights.reserve(nw);
    for (auto& w : wm) {
        // F32 weights (all the reference converter writes, onnx_to_engine.py:428),
        // and I64 / I32 constants, which the reference loads typed
        // (custom_loader.cpp:87-101) and reads with get_tensor_int.
        if (w.dtype != 12 && w.dtype != 8 && w.dtype != 6)
            return fail(("weight '" + w.name + "': only F32, I64 and I32 weights are supported").c_str());
        HostTensor t = HostTensor::empty(w.dims, w.rank, public_dtype(w.dtype));
        if (t.nbytes != w.size && !(t.nbytes == 0 && w.size == 0)) {
            if (t.nbytes > w.size) return fail("weight blob smaller than its shape");
        }
        if (std::fseek(f, data_start + static_cast<long>(w.offset), SEEK_SET) != 0) return fail("bad weight offset");
        if (!r.bytes(t.data, t.nbytes)) return fail("truncated weight data");
        weights.push_back(std::move(t));
        names.push_back(std::move(w.name));
    }

    m.name = path;
    m.source_path = path;
    m.version = static_cast<int32_t>(version);
    m.weights = std::move(weights);
    m.weight_names = std::move(names);
    m.nodes = std::move(nodes);
    m.graph_inputs = std::move(gin);
    m.graph_outputs = std::move(gout);
    m.input_infos = std::move(iinfo);
    m.output_infos = std::move(oinfo);
    return true;
}

}  // namespace pdefa
