#include "planner.hpp"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstring>
#include <map>
#include <sstream>
#include <stdexcept>
#include <unordered_map>

namespace pdefa {

namespace {

using Dims = std::vector<int64_t>;

// A grouped launch must beat the separate launches it replaces by 3%.
constexpr double kGroupGain = 0.97;

[[noreturn]] void fail(const Model& m, int node, const std::string& msg) {
    std::string where = node >= 0 && node < static_cast<int>(m.nodes.size())
                            ? " (node " + std::to_string(node) + " '" + m.nodes[node].name + "' " +
                                  op_name(m.nodes[node].op) + ")"
                            : "";
    throw std::runtime_error("plan: " + msg + where);
}

int64_t prod(const Dims& d) {
    int64_t n = 1;
    for (auto v : d) n *= v;
    return n;
}

// ---------------------------------------------------------------- views ----
VRef make_view(int32_t buf, int64_t off, const Dims& dims, const int64_t* str) {
    VRef v;
    v.buf = buf;
    v.off = off;
    v.rank = static_cast<int32_t>(dims.size());
    for (int d = 0; d < v.rank; ++d) {
        v.dims[d] = dims[d];
        v.str[d] = str[d];
    }
    return v;
}

VRef contiguous_view(int32_t buf, const Dims& dims) {
    int64_t str[k::kMaxRank];
    int64_t s = 1;
    for (int d = static_cast<int>(dims.size()) - 1; d >= 0; --d) {
        str[d] = s;
        s *= dims[d];
    }
    return make_view(buf, 0, dims, str);
}

// Channels-last: logical dim 1 gets stride 1, the others keep their order.
VRef channels_last_view(int32_t buf, const Dims& dims) {
    const int r = static_cast<int>(dims.size());
    if (r < 3) return contiguous_view(buf, dims);
    int64_t str[k::kMaxRank];
    str[1] = 1;
    int64_t s = dims[1];
    for (int d = r - 1; d >= 2; --d) {
        str[d] = s;
        s *= dims[d];
    }
    str[0] = s;
    return make_view(buf, 0, dims, str);
}

Dims dims_of(const VRef& v) { return Dims(v.dims, v.dims + v.rank); }

bool views_equal(const VRef& a, const VRef& b) {
    if (a.buf != b.buf || a.aux != b.aux || a.off != b.off || a.rank != b.rank) return false;
    for (int d = 0; d < a.rank; ++d) {
        if (a.dims[d] != b.dims[d]) return false;
        if (a.dims[d] != 1 && a.str[d] != b.str[d]) return false;
    }
    return true;
}

VRef slice_view(VRef v, int axis, int64_t start, int64_t len, int64_t step = 1) {
    v.off += start * v.str[axis];
    v.dims[axis] = len;
    v.str[axis] *= step;
    return v;
}

VRef permute_view(const VRef& v, const std::vector<int32_t>& perm) {
    VRef o = v;
    for (int d = 0; d < v.rank; ++d) {
        o.dims[d] = v.dims[perm[d]];
        o.str[d] = v.str[perm[d]];
    }
    return o;
}

// Re-expresses view `v` with logical shape `nd` without moving data, when the
// strides allow it (the no-copy reshape rule: each group of old dims that is
// merged must be mutually contiguous).
bool reshape_view(const VRef& v, const Dims& nd, VRef* out) {
    if (nd.size() > static_cast<size_t>(k::kMaxRank)) return false;
    int64_t od[k::kMaxRank], os[k::kMaxRank];
    int orank = 0;
    for (int d = 0; d < v.rank; ++d)
        if (v.dims[d] != 1) {
            od[orank] = v.dims[d];
            os[orank++] = v.str[d];
        }
    int64_t ndd[k::kMaxRank], ns[k::kMaxRank];
    int map[k::kMaxRank];
    int nr = 0;
    for (size_t d = 0; d < nd.size(); ++d)
        if (nd[d] != 1) {
            map[nr] = static_cast<int>(d);
            ndd[nr++] = nd[d];
        }
    int64_t on = 1, nn = 1;
    for (int i = 0; i < orank; ++i) on *= od[i];
    for (int i = 0; i < nr; ++i) nn *= ndd[i];
    if (on != nn) return false;
    int oi = 0, oj = 1, ni = 0, nj = 1;
    while (ni < nr && oi < orank) {
        int64_t np = ndd[ni], op = od[oi];
        while (np != op) {
            if (np < op) {
                if (nj >= nr) return false;
                np *= ndd[nj++];
            } else {
                if (oj >= orank) return false;
                op *= od[oj++];
            }
        }
        for (int ok = oi; ok < oj - 1; ++ok)
            if (os[ok] != od[ok + 1] * os[ok + 1]) return false;
        ns[nj - 1] = os[oj - 1];
        for (int nk = nj - 1; nk > ni; --nk) ns[nk - 1] = ns[nk] * ndd[nk];
        ni = nj++;
        oi = oj++;
    }
    VRef o = v;
    o.rank = static_cast<int32_t>(nd.size());
    for (size_t d = 0; d < nd.size(); ++d) {
        o.dims[d] = nd[d];
        o.str[d] = 0;
    }
    for (int i = 0; i < nr; ++i) o.str[map[i]] = ns[i];
    *out = o;
    return true;
}

// Broadcasts view `a` to `dims` (numpy rules, trailing alignment).
VRef broadcast_view(const VRef& a, const Dims& dims) {
    VRef o;
    o.buf = a.buf;
    o.aux = a.aux;
    o.off = a.off;
    o.rank = static_cast<int32_t>(dims.size());
    const int pad = o.rank - a.rank;
    for (int d = 0; d < o.rank; ++d) {
        o.dims[d] = dims[d];
        const int s = d - pad;
        if (s < 0 || a.dims[s] == 1)
            o.str[d] = 0;
        else
            o.str[d] = a.str[s];
    }
    return o;
}

// ------------------------------------------------------------ graph ops ----
enum class EK { Conv, Elt, MaxPool, Resize, Softmax, Concat, Slice, Reshape, Transpose, TopK, GatherElements };

struct EOp {
    EK k = EK::Elt;
    int node = -1;
    std::vector<int32_t> in;
    int32_t out = 0;
    int act = 0;
    float slope = 0.01f;
    int32_t res = INT32_MIN;  // residual ref (conv)
    int elt = 0;
    float alpha = 0.0f;
    // resolved at shape inference
    int axis = 0;
    std::vector<int64_t> sl_start, sl_step;  // per dim (slice)
    std::vector<int32_t> perm;                // transpose
    Dims target;                              // reshape
    int32_t kref = 0;                         // topk: the k constant
    int64_t topk = 0;
    bool topk_indices = false;
    // concat slots (reverse pass) and which inputs need copies
    std::vector<VRef> slots;
    std::vector<bool> copy;
};

struct Val {
    bool known = false;
    Dims dims;
    bool has_view = false;
    VRef view;
    int producer = -1;
    bool is_output = false;
    bool is_input = false;
    int input_index = -1;
    bool is_weight = false;
    int weight_index = -1;
    std::vector<int> consumers;  // eop indices
    int nhwc_copy_buf = -1;      // graph input converted to channels-last for convs
    VRef nhwc_view;
};

// Bytes from a view's first element to the end of its last one.
int64_t view_span_bytes(const VRef& v) {
    int64_t last = 0;
    for (int d = 0; d < v.rank; ++d) last += (v.dims[d] - 1) * v.str[d];
    return 4 * (last + 1);
}

// The Winograd kernel addresses its input, transformed weights, output and
// residual with 32-bit byte offsets (spans under 1 GiB less 4 KiB).
bool wino_views_ok(const Step& s) {
    constexpr int64_t kMax = (int64_t{1} << 30) - 4096;
    const int64_t u_bytes = 4 * k::wino_packed_elems(static_cast<int>(s.out.dims[1]), static_cast<int>(s.a.dims[1]));
    return view_span_bytes(s.a) < kMax && u_bytes < kMax && view_span_bytes(s.out) < kMax &&
           (!s.has_res || view_span_bytes(s.res) < kMax);
}

// The kernel the reference's conv dispatcher (PDEFA1.0/src/ops/conv2d.cpp:484-651)
// sends a conv to, as far as it changes what a fused activation code computes:
// its direct kernel (groups 1, Cin <= 16, KH, KW <= 7, not a plain 1x1 with
// stride 1 and no padding; conv2d.cpp:599-611), its Winograd kernel (3x3,
// stride 1, dilation 1, groups 1, Cin <= 512; conv2d.cpp:616-629), or one of
// the others (DFL, depthwise, grouped GEMM, GEMM), which all apply the plain
// functions.
enum class RefConvPath { Direct, Winograd, Other };

RefConvPath reference_conv_path(const Step& s, int64_t cin_per_group) {
    if (s.groups != 1) return RefConvPath::Other;
    const bool pure_1x1 = s.KH == 1 && s.KW == 1 && s.ph == 0 && s.pw == 0 && s.sh == 1 && s.sw == 1 && s.dh == 1 &&
                          s.dw == 1;
    if (!pure_1x1 && cin_per_group <= 16 && s.KH <= 7 && s.KW <= 7) return RefConvPath::Direct;
    if (s.KH == 3 && s.KW == 3 && s.sh == 1 && s.sw == 1 && s.dh == 1 && s.dw == 1 && cin_per_group <= 512)
        return RefConvPath::Winograd;
    return RefConvPath::Other;
}

// The function a fused activation code stands for on the reference's path:
// code 5 on its Winograd kernel is the polynomial SiLU form
// (conv2d_winograd.cpp:81-101, unless `winograd_form_silu` is off), code 4 on
// its Winograd and direct kernels is tanh-form GELU (conv2d_winograd.cpp:108-111,
// conv2d_avx2.cpp:109-112), code 3 on its direct kernel is 1 / (1 + v)
// (conv2d_avx2.cpp:99-103).  Results equal the reference's only with the
// same functions.
int32_t reference_activation(int32_t code, RefConvPath path, bool winograd_form_silu) {
    if (path == RefConvPath::Direct) {
        if (code == k::kActSigmoid) return k::kActRecip1p;
        if (code == k::kActTanh) return k::kActGeluTanh;
    } else if (path == RefConvPath::Winograd) {
        if (code == k::kActTanh) return k::kActGeluTanh;
        if (code == k::kActSilu && winograd_form_silu) return k::kActSiluWinogradForm;
    }
    return code;
}

// Launch-shape query of an implicit-GEMM conv step.
ConvQuery conv_query(const Step& s) {
    ConvQuery q;
    q.N = static_cast<int32_t>(s.a.dims[0]);
    q.Cin = static_cast<int32_t>(s.a.dims[1]);  // all channels (groups of Cin / groups)
    q.H = static_cast<int32_t>(s.a.dims[2]);
    q.W = static_cast<int32_t>(s.a.dims[3]);
    q.Cout = static_cast<int32_t>(s.out.dims[1]);
    q.Ho = static_cast<int32_t>(s.out.dims[2]);
    q.Wo = static_cast<int32_t>(s.out.dims[3]);
    q.KH = s.KH;
    q.KW = s.KW;
    q.sh = s.sh;
    q.sw = s.sw;
    q.ph = s.ph;
    q.pw = s.pw;
    q.dh = s.dh;
    q.dw = s.dw;
    q.act = s.act;
    q.has_res = s.has_res;
    q.vec = s.vec;
    q.groups = s.groups;
    q.wino = s.vec && s.groups == 1 && k::wino_eligible(s.KH, s.KW, s.sh, s.sw, s.dh, s.dw, q.Cin) &&
             wino_views_ok(s);
    return q;
}

// The views a step reads and writes (model weights included; they are never
// written).  A split-K workspace counts as a write of its whole buffer.
void step_views(const Step& s, std::vector<VRef>& rd, std::vector<VRef>& wr) {
    rd.clear();
    wr.clear();
    wr.push_back(s.out);
    rd.push_back(s.a);
    if (s.has_res) rd.push_back(s.res);
    if (s.kind == StepKind::ConvMfma && s.up.buf != -1) wr.push_back(s.up);
    switch (s.kind) {
        case StepKind::Elt:
        case StepKind::GatherElements: rd.push_back(s.b); break;
        case StepKind::MaxPoolChain:
            wr.push_back(s.b);
            wr.push_back(s.c);
            break;
        case StepKind::DetectDecode:
            rd.push_back(s.b);
            rd.push_back(s.c);
            rd.push_back(s.res);
            if (s.cls_in.buf != -1) {
                rd.push_back(s.cls_in);
                wr.push_back(s.cls_out);
            }
            break;
        default: break;
    }
}

// Whether two views of planned buffers may share an element.  Distinct
// buffers never do before memory is assigned; two views of one buffer are
// disjoint when they are slices of one parent along one axis with disjoint
// index ranges there (the producers of one concat buffer).
bool views_may_overlap(const VRef& a, const VRef& b) {
    if (a.buf < 0 || b.buf < 0 || a.buf != b.buf) return false;
    // Disjoint element ranges (e.g. the slices of different scales in one
    // concat buffer, whose strides differ), over whole views or over one
    // item of a common outer dim: with equal outer strides S whose items'
    // ranges are disjoint and together span less than S, an element of one
    // view and one of the other differ by less than S within an item, so
    // they can only meet in the same item, where they do not.
    auto range = [](const VRef& v, int first, int64_t& lo, int64_t& hi) {
        lo = hi = v.off;
        for (int d = first; d < v.rank; ++d) {
            if (v.dims[d] <= 0) return false;
            const int64_t e = (v.dims[d] - 1) * v.str[d];
            (e < 0 ? lo : hi) += e;
        }
        return true;
    };
    int64_t alo, ahi, blo, bhi;
    if (!range(a, 0, alo, ahi) || !range(b, 0, blo, bhi)) return false;  // an empty view touches nothing
    if (ahi < blo || bhi < alo) return false;
    if (a.rank > 1 && b.rank > 1 && a.str[0] == b.str[0] && a.str[0] > 0 && range(a, 1, alo, ahi) &&
        range(b, 1, blo, bhi) && (ahi < blo || bhi < alo) && std::max(ahi, bhi) - std::min(alo, blo) < a.str[0])
        return false;
    if (a.rank != b.rank) return true;
    for (int d = 0; d < a.rank; ++d)
        if (a.str[d] != b.str[d]) return true;
    const int64_t diff = b.off - a.off;
    for (int d = 0; d < a.rank; ++d) {
        if (a.str[d] <= 0 || diff % a.str[d] != 0) continue;
        bool same_other = true;
        int64_t row = INT64_MAX;  // smallest stride of the other (non-trivial) axes
        for (int e = 0; e < a.rank; ++e) {
            if (e == d) continue;
            if (a.dims[e] != b.dims[e]) same_other = false;
            if (a.dims[e] > 1) row = std::min(row, a.str[e]);
        }
        if (!same_other) continue;
        const int64_t kk = diff / a.str[d];
        const bool disjoint = kk >= a.dims[d] || kk + b.dims[d] <= 0;
        const int64_t span = std::max(a.dims[d], kk + b.dims[d]) - std::min<int64_t>(0, kk);
        if (disjoint && (row == INT64_MAX || span * a.str[d] <= row)) return false;
    }
    return true;
}

class Planner {
   public:
    Planner(const Model& m, const std::vector<Dims>& in_dims, const PlanOptions& opt)
        : m_(m), in_dims_(in_dims), opt_(opt) {}

    Plan run() {
        if (in_dims_.size() != m_.graph_inputs.size())
            throw std::runtime_error("plan: expected " + std::to_string(m_.graph_inputs.size()) + " inputs");
        build_eops();
        infer_shapes();
        fuse_residuals();
        assign_storage();
        emit();
        fuse_steps();
        split_decode();
        group_convs();
        allocate();
        check_bounds();
        return std::move(plan_);
    }

   private:
    const Model& m_;
    std::vector<Dims> in_dims_;
    PlanOptions opt_;
    std::vector<EOp> eops_;
    std::map<int32_t, Val> vals_;
    Plan plan_;

    Val& val(int32_t ref) {
        auto it = vals_.find(ref);
        if (it != vals_.end()) return it->second;
        Val& v = vals_[ref];
        if (ref <= -1000) {
            const int w = -1000 - ref;
            if (w < 0 || w >= static_cast<int>(m_.weights.size())) throw std::runtime_error("plan: bad weight ref");
            v.is_weight = true;
            v.weight_index = w;
            v.known = true;
            const HostTensor& t = m_.weights[w];
            v.dims.assign(t.dims, t.dims + t.rank);
            v.has_view = true;
            v.view = contiguous_view(kBufWeight, v.dims);
            v.view.aux = w;
        } else if (ref < 0) {
            v.is_input = true;
            v.input_index = -1 - ref;
        }
        return v;
    }

    const HostTensor& weight_tensor(int32_t ref, int node) {
        if (ref > -1000) fail(m_, node, "expected a constant input");
        return m_.weights[-1000 - ref];
    }

    std::vector<int64_t> const_ints(int32_t ref, int node) {
        const HostTensor& t = weight_tensor(ref, node);
        std::vector<int64_t> v(static_cast<size_t>(t.numel()));
        // I64 / I32 as stored; F32 constants are truncated toward zero, as
        // get_tensor_int does (session_helpers.inc:156-170).
        for (size_t i = 0; i < v.size(); ++i) {
            if (t.dtype == kI64) v[i] = static_cast<const int64_t*>(t.data)[i];
            else if (t.dtype == kI32) v[i] = static_cast<const int32_t*>(t.data)[i];
            else v[i] = static_cast<int64_t>(t.f32()[i]);
        }
        return v;
    }

    int new_buf(int64_t elems) {
        Buffer b;
        b.elems = std::max<int64_t>(elems, 1);
        plan_.bufs.push_back(b);
        return static_cast<int>(plan_.bufs.size()) - 1;
    }

    // ---- 1. fused op list ------------------------------------------------
    void build_eops() {
        const auto& nodes = m_.nodes;
        std::unordered_map<int32_t, int> n_cons;  // node-level consumer counts
        for (const auto& n : nodes)
            for (int32_t r : n.inputs) n_cons[r]++;
        for (int32_t r : m_.graph_outputs) n_cons[r]++;
        std::vector<bool> absorbed(nodes.size(), false);

        for (size_t i = 0; i < nodes.size(); ++i) {
            if (absorbed[i]) continue;
            const Node& n = nodes[i];
            EOp e;
            e.node = static_cast<int>(i);
            e.in = n.inputs;
            if (n.outputs.empty()) {
                if (n.op == kOpInput || n.op == kOpOutput) continue;
                fail(m_, e.node, "node without outputs");
            }
            e.out = n.outputs[0];
            switch (n.op) {
                case kOpInput:
                case kOpOutput:
                    continue;
                case kOpConv: {
                    e.k = EK::Conv;
                    if (n.inputs.size() < 2) fail(m_, e.node, "conv needs input and weight");
                    e.act = n.params.fused_activation;
                    e.slope = n.params.leaky_slope;
                    const int32_t co = n.outputs[0];
                    const int cons = n_cons[co];
                    bool fused = false;
                    if (cons == 2 && e.act == 0) {
                        // Conv -> {Sigmoid, Mul(conv, sigmoid)}: SiLU (session_fusion.inc:33-81)
                        int sig = -1, mul = -1;
                        for (size_t j = i + 1; j < nodes.size(); ++j) {
                            const Node& s = nodes[j];
                            if (s.op == kOpSigmoid && s.inputs.size() == 1 && s.inputs[0] == co && !s.outputs.empty()) {
                                if (n_cons[s.outputs[0]] == 1) sig = static_cast<int>(j);
                                break;
                            }
                        }
                        if (sig >= 0) {
                            const int32_t so = nodes[sig].outputs[0];
                            for (size_t j = i + 1; j < nodes.size(); ++j) {
                                const Node& u = nodes[j];
                                if (u.op == kOpMul && u.inputs.size() == 2 && !u.outputs.empty() &&
                                    ((u.inputs[0] == co && u.inputs[1] == so) || (u.inputs[1] == co && u.inputs[0] == so))) {
                                    mul = static_cast<int>(j);
                                    break;
                                }
                            }
                        }
                        if (sig >= 0 && mul >= 0) {
                            e.act = k::kActSilu;
                            e.out = nodes[mul].outputs[0];
                            absorbed[sig] = absorbed[mul] = true;
                            fused = true;
                        }
                    }
                    if (!fused && cons == 1 && e.act == 0) {
                        // single-consumer ReLU / LeakyReLU / Sigmoid / Tanh (session_fusion.inc:85-107)
                        for (size_t j = i + 1; j < nodes.size(); ++j) {
                            const Node& s = nodes[j];
                            if (s.inputs.size() == 1 && s.inputs[0] == co && !s.outputs.empty()) {
                                int a = 0;
                                if (s.op == kOpRelu) a = k::kActRelu;
                                else if (s.op == kOpLeaky) a = k::kActLeaky;
                                else if (s.op == kOpSigmoid) a = k::kActSigmoid;
                                else if (s.op == kOpTanh) a = k::kActTanh;
                                if (a) {
                                    e.act = a;
                                    if (a == k::kActLeaky) e.slope = s.params.leaky_slope;
                                    e.out = s.outputs[0];
                                    absorbed[j] = true;
                                }
                                break;
                            }
                        }
                    }
                    break;
                }
                case kOpSigmoid: e.k = EK::Elt; e.elt = k::kEltSigmoid; break;
                case kOpRelu: e.k = EK::Elt; e.elt = k::kEltRelu; break;
                case kOpTanh: e.k = EK::Elt; e.elt = k::kEltTanh; break;
                case kOpSilu: e.k = EK::Elt; e.elt = k::kEltSilu; break;
                case kOpLeaky: e.k = EK::Elt; e.elt = k::kEltLeaky; e.alpha = n.params.leaky_slope; break;
                case kOpAdd: e.k = EK::Elt; e.elt = k::kEltAdd; break;
                case kOpSub: e.k = EK::Elt; e.elt = k::kEltSub; break;
                case kOpMul: e.k = EK::Elt; e.elt = k::kEltMul; break;
                case kOpDiv: e.k = EK::Elt; e.elt = k::kEltDiv; break;
                case kOpMaxPool:
                    if (n.params.kernel_h <= 0 || n.params.kernel_w <= 0) fail(m_, e.node, "global max pool unsupported");
                    e.k = EK::MaxPool;
                    break;
                case kOpResize:
                case kOpUpsample:
                    if (n.params.upsample_mode != 0) fail(m_, e.node, "only nearest resize is supported");
                    e.k = EK::Resize;
                    break;
                case kOpSoftmax: e.k = EK::Softmax; break;
                case kOpConcat: e.k = EK::Concat; break;
                case kOpSlice: e.k = EK::Slice; break;
                case kOpReshape: e.k = EK::Reshape; break;
                case kOpTranspose: e.k = EK::Transpose; break;
                case kOpTopK: {
                    // one step per used output (values, indices), each from the
                    // same sort (session_ops_math.inc:321-395)
                    if (n.inputs.size() < 2) fail(m_, e.node, "TopK needs the input and k");
                    e.k = EK::TopK;
                    e.kref = n.inputs[1];
                    e.in.resize(1);
                    if (n.outputs[0] >= 0) eops_.push_back(e);
                    if (n.outputs.size() >= 2 && n.outputs[1] >= 0) {
                        EOp ei = e;
                        ei.out = n.outputs[1];
                        ei.topk_indices = true;
                        eops_.push_back(std::move(ei));
                    }
                    continue;
                }
                case kOpGatherElements:
                    if (n.inputs.size() < 2) fail(m_, e.node, "GatherElements needs data and indices");
                    e.k = EK::GatherElements;
                    e.in.resize(2);
                    break;
                default:
                    fail(m_, e.node, "op not supported by the device executor");
            }
            if (e.k == EK::Elt) {
                const bool binary = e.elt == k::kEltAdd || e.elt == k::kEltSub || e.elt == k::kEltMul || e.elt == k::kEltDiv;
                if (binary && e.in.size() < 2) fail(m_, e.node, "binary op needs two inputs");
                if (!binary) e.in.resize(1);
            }
            eops_.push_back(std::move(e));
        }
        for (size_t i = 0; i < eops_.size(); ++i) {
            for (int32_t r : eops_[i].in) val(r).consumers.push_back(static_cast<int>(i));
            Val& o = val(eops_[i].out);
            if (o.producer >= 0) fail(m_, eops_[i].node, "tensor produced twice");
            o.producer = static_cast<int>(i);
        }
        for (int32_t r : m_.graph_outputs) val(r).is_output = true;
        for (size_t i = 0; i < m_.graph_inputs.size(); ++i) {
            Val& v = val(m_.graph_inputs[i]);
            v.is_input = true;
            v.input_index = static_cast<int>(i);
            v.known = true;
            v.dims = in_dims_[i];
        }
    }

    // ---- 2. shapes (ONNX semantics) --------------------------------------
    const Dims& dims(int32_t r, int node) {
        Val& v = val(r);
        if (!v.known) fail(m_, node, "input tensor " + std::to_string(r) + " is not available");
        return v.dims;
    }

    void infer_shapes() {
        const int64_t batch = in_dims_.empty() || in_dims_[0].empty() ? 1 : in_dims_[0][0];
        for (auto& e : eops_) {
            const Node& n = m_.nodes[e.node];
            const OpParams& p = n.params;
            Dims out;
            switch (e.k) {
                case EK::Conv: {
                    const Dims x = dims(e.in[0], e.node);
                    const Dims w = dims(e.in[1], e.node);
                    if (x.size() != 4 || w.size() != 4) fail(m_, e.node, "conv expects rank-4 input and weight");
                    const int64_t G = std::max<int64_t>(1, p.groups);
                    if (x[1] != w[1] * G || w[0] % G != 0) fail(m_, e.node, "conv channel mismatch");
                    if (!val(e.in[1]).is_weight) fail(m_, e.node, "conv weight must be a constant");
                    if (e.in.size() > 2 && !val(e.in[2]).is_weight) fail(m_, e.node, "conv bias must be a constant");
                    const int64_t ho = (x[2] + 2 * p.pad_h - ((w[2] - 1) * p.dil_h + 1)) / p.stride_h + 1;
                    const int64_t wo = (x[3] + 2 * p.pad_w - ((w[3] - 1) * p.dil_w + 1)) / p.stride_w + 1;
                    if (ho <= 0 || wo <= 0) fail(m_, e.node, "empty conv output");
                    out = {x[0], w[0], ho, wo};
                    break;
                }
                case EK::Elt: {
                    const Dims a = dims(e.in[0], e.node);
                    if (e.in.size() == 1) {
                        out = a;
                        break;
                    }
                    const Dims b = dims(e.in[1], e.node);
                    const size_t r = std::max(a.size(), b.size());
                    out.assign(r, 1);
                    for (size_t d = 0; d < r; ++d) {
                        const int64_t da = d < r - a.size() ? 1 : a[d - (r - a.size())];
                        const int64_t db = d < r - b.size() ? 1 : b[d - (r - b.size())];
                        if (da != db && da != 1 && db != 1) fail(m_, e.node, "broadcast mismatch");
                        out[d] = std::max(da, db);
                    }
                    break;
                }
                case EK::MaxPool: {
                    const Dims x = dims(e.in[0], e.node);
                    if (x.size() != 4) fail(m_, e.node, "max pool expects rank 4");
                    const int64_t ho = (x[2] + 2 * p.pad_h - p.kernel_h) / p.stride_h + 1;
                    const int64_t wo = (x[3] + 2 * p.pad_w - p.kernel_w) / p.stride_w + 1;
                    out = {x[0], x[1], ho, wo};
                    break;
                }
                case EK::Resize: {
                    // Target size: params, then a 4- or 2-element scales/sizes input, then 2x
                    // (session_ops_shape.inc:110-163).
                    const Dims x = dims(e.in[0], e.node);
                    if (x.size() != 4) fail(m_, e.node, "resize expects rank 4");
                    int64_t H = 0, W = 0;
                    if (n.op == kOpUpsample) {
                        H = x[2] * p.scale_h;
                        W = x[3] * p.scale_w;
                    } else {
                        H = p.target_h;
                        W = p.target_w;
                        if ((H <= 0 || W <= 0) && p.scale_h > 1 && p.scale_w > 1) {
                            H = x[2] * p.scale_h;
                            W = x[3] * p.scale_w;
                        }
                        if (H <= 0 || W <= 0) {
                            for (size_t j = 1; j < e.in.size() && j < 4; ++j) {
                                if (!val(e.in[j]).is_weight) continue;
                                const HostTensor& t = weight_tensor(e.in[j], e.node);
                                if (t.numel() == 4 || t.numel() == 2) {
                                    const int o = t.numel() == 4 ? 2 : 0;
                                    const float s0 = t.f32()[o], s1 = t.f32()[o + 1];
                                    if (s0 > 8.0f && s1 > 8.0f) {
                                        H = static_cast<int64_t>(s0 + 0.5f);
                                        W = static_cast<int64_t>(s1 + 0.5f);
                                    } else {
                                        H = static_cast<int64_t>(static_cast<float>(x[2]) * s0 + 0.5f);
                                        W = static_cast<int64_t>(static_cast<float>(x[3]) * s1 + 0.5f);
                                    }
                                    break;
                                }
                            }
                        }
                        if (H <= 0 || W <= 0) {
                            H = x[2] * 2;
                            W = x[3] * 2;
                        }
                    }
                    out = {x[0], x[1], H, W};
                    break;
                }
                case EK::Softmax: {
                    out = dims(e.in[0], e.node);
                    int ax = p.axis < 0 ? p.axis + static_cast<int>(out.size()) : p.axis;
                    if (ax < 0 || ax >= static_cast<int>(out.size())) fail(m_, e.node, "softmax axis out of range");
                    e.axis = ax;
                    break;
                }
                case EK::Concat: {
                    const Dims a = dims(e.in[0], e.node);
                    int ax = p.axis < 0 ? p.axis + static_cast<int>(a.size()) : p.axis;
                    if (ax < 0 || ax >= static_cast<int>(a.size())) fail(m_, e.node, "concat axis out of range");
                    e.axis = ax;
                    out = a;
                    out[ax] = 0;
                    for (int32_t r : e.in) {
                        const Dims b = dims(r, e.node);
                        if (b.size() != a.size()) fail(m_, e.node, "concat rank mismatch");
                        for (size_t d = 0; d < a.size(); ++d)
                            if (static_cast<int>(d) != ax && b[d] != a[d]) fail(m_, e.node, "concat shape mismatch");
                        out[ax] += b[ax];
                    }
                    break;
                }
                case EK::Slice: {
                    const Dims x = dims(e.in[0], e.node);
                    if (e.in.size() < 3) fail(m_, e.node, "slice needs starts and ends");
                    const auto starts = const_ints(e.in[1], e.node);
                    const auto ends = const_ints(e.in[2], e.node);
                    std::vector<int64_t> axes, steps;
                    if (e.in.size() > 3) axes = const_ints(e.in[3], e.node);
                    if (e.in.size() > 4) steps = const_ints(e.in[4], e.node);
                    out = x;
                    e.sl_start.assign(x.size(), 0);
                    e.sl_step.assign(x.size(), 1);
                    for (size_t j = 0; j < starts.size(); ++j) {
                        int64_t ax = axes.empty() ? static_cast<int64_t>(j) : axes[j];
                        if (ax < 0) ax += static_cast<int64_t>(x.size());
                        if (ax < 0 || ax >= static_cast<int64_t>(x.size())) fail(m_, e.node, "slice axis out of range");
                        const int64_t st = steps.empty() ? 1 : steps[j];
                        if (st <= 0) fail(m_, e.node, "only positive slice steps are supported");
                        const int64_t d = x[ax];
                        int64_t s = starts[j], en = ends[j];
                        if (s < 0) s += d;
                        if (en < 0) en += d;
                        s = std::min(std::max<int64_t>(s, 0), d);
                        en = std::min(std::max<int64_t>(en, 0), d);
                        if (en < s) en = s;
                        e.sl_start[ax] = s;
                        e.sl_step[ax] = st;
                        out[ax] = (en - s + st - 1) / st;
                    }
                    break;
                }
                case EK::Reshape: {
                    const Dims x = dims(e.in[0], e.node);
                    if (e.in.size() < 2) fail(m_, e.node, "reshape needs a shape input");
                    auto t = const_ints(e.in[1], e.node);
                    // The graph was exported for batch 1: a leading 1 follows the run's batch.
                    if (!t.empty() && t[0] == 1 && !x.empty() && x[0] == batch && batch > 1) t[0] = batch;
                    int neg = -1;
                    int64_t known = 1;
                    for (size_t d = 0; d < t.size(); ++d) {
                        if (t[d] == 0) t[d] = d < x.size() ? x[d] : 1;
                        if (t[d] == -1) neg = static_cast<int>(d);
                        else known *= t[d];
                    }
                    if (neg >= 0) t[neg] = known > 0 ? prod(x) / known : 0;
                    if (prod(t) != prod(x)) fail(m_, e.node, "reshape element count mismatch");
                    e.target = t;
                    out = t;
                    break;
                }
                case EK::TopK: {
                    const Dims x = dims(e.in[0], e.node);
                    const int r = static_cast<int>(x.size());
                    // The reference applies the axis to its storage, which is
                    // channels-last for rank 4 and logical otherwise.
                    if (r == 4 || r < 1) fail(m_, e.node, "TopK is supported on tensors of rank 1-3 and 5-6");
                    const int ax = p.axis < 0 ? p.axis + r : p.axis;
                    if (ax < 0 || ax >= r) fail(m_, e.node, "TopK axis out of range");
                    if (!val(e.kref).is_weight) fail(m_, e.node, "TopK k must be a constant");
                    const auto kv = const_ints(e.kref, e.node);
                    int64_t kk = kv.empty() ? 0 : kv[0];
                    if (kk <= 0 || kk > x[ax]) kk = x[ax];
                    if (x[ax] > k::kTopKMaxAxis) fail(m_, e.node, "TopK axis longer than 16384");
                    e.axis = ax;
                    e.topk = kk;
                    out = x;
                    out[ax] = kk;
                    break;
                }
                case EK::GatherElements: {
                    const Dims d = dims(e.in[0], e.node);
                    const Dims ix = dims(e.in[1], e.node);
                    const int r = static_cast<int>(d.size());
                    if (r == 4 || r < 1) fail(m_, e.node, "GatherElements is supported on tensors of rank 1-3 and 5-6");
                    if (static_cast<int>(ix.size()) != r) fail(m_, e.node, "GatherElements rank mismatch");
                    const int ax = p.axis < 0 ? p.axis + r : p.axis;
                    if (ax < 0 || ax >= r) fail(m_, e.node, "GatherElements axis out of range");
                    // the reference walks the indices with the data's outer and
                    // inner extents (session_ops_math.inc:414-427)
                    for (int q = 0; q < r; ++q)
                        if (q != ax && ix[q] != d[q]) fail(m_, e.node, "GatherElements: indices and data differ off the axis");
                    e.axis = ax;
                    out = ix;
                    break;
                }
                case EK::Transpose: {
                    const Dims x = dims(e.in[0], e.node);
                    if (e.in.size() < 2) fail(m_, e.node, "transpose needs a perm input");
                    const auto pv = const_ints(e.in[1], e.node);
                    if (pv.size() != x.size()) fail(m_, e.node, "perm rank mismatch");
                    e.perm.clear();
                    out.clear();
                    for (auto q : pv) {
                        const int64_t a = q < 0 ? q + static_cast<int64_t>(x.size()) : q;
                        if (a < 0 || a >= static_cast<int64_t>(x.size())) fail(m_, e.node, "bad perm");
                        e.perm.push_back(static_cast<int32_t>(a));
                        out.push_back(x[a]);
                    }
                    break;
                }
            }
            if (out.size() > static_cast<size_t>(k::kMaxRank)) fail(m_, e.node, "rank > 6 unsupported");
            Val& o = val(e.out);
            o.known = true;
            o.dims = out;
        }
        for (int32_t r : m_.graph_outputs)
            if (!val(r).known) throw std::runtime_error("plan: graph output " + std::to_string(r) + " is never produced");
    }

    // ---- 3. residual Add -> conv epilogue --------------------------------
    void fuse_residuals() {
        for (size_t i = 0; i < eops_.size(); ++i) {
            EOp& c = eops_[i];
            if (c.k != EK::Conv || c.res != INT32_MIN) continue;
            Val& o = val(c.out);
            if (o.is_output || o.consumers.size() != 1) continue;
            EOp& a = eops_[o.consumers[0]];
            if (a.k != EK::Elt || a.elt != k::kEltAdd || a.in.size() != 2) continue;
            const int32_t other = a.in[0] == c.out ? a.in[1] : a.in[0];
            if (other == c.out) continue;
            Val& r = val(other);
            if (r.is_weight || !r.known || r.dims != o.dims) continue;
            if (!r.is_input && !(r.producer >= 0 && r.producer < static_cast<int>(i))) continue;
            // conv now produces the Add's output; the Add disappears.
            c.res = other;
            r.consumers.erase(std::remove(r.consumers.begin(), r.consumers.end(), o.consumers[0]), r.consumers.end());
            r.consumers.push_back(static_cast<int>(i));
            const int32_t new_out = a.out;
            Val& no = val(new_out);
            no.producer = static_cast<int>(i);
            o.consumers.clear();
            o.producer = -1;
            c.out = new_out;
            a.k = EK::Elt;
            a.elt = -1;  // dead
        }
        eops_.erase(std::remove_if(eops_.begin(), eops_.end(), [](const EOp& e) { return e.k == EK::Elt && e.elt == -1; }),
                    eops_.end());
        // re-number producers/consumers after the erase
        for (auto& kv : vals_) {
            kv.second.producer = -1;
            kv.second.consumers.clear();
        }
        for (size_t i = 0; i < eops_.size(); ++i) {
            for (int32_t r : eops_[i].in) val(r).consumers.push_back(static_cast<int>(i));
            val(eops_[i].out).producer = static_cast<int>(i);
        }
    }

    // ---- 4. storage: reverse pass with concat placement ------------------
    bool view_kind(EK k) const { return k == EK::Slice || k == EK::Reshape || k == EK::Transpose; }

    void assign_fresh(Val& v, bool contiguous) {
        const int b = new_buf(prod(v.dims));
        v.view = contiguous ? contiguous_view(b, v.dims) : channels_last_view(b, v.dims);
        v.has_view = true;
    }

    // Can tensor `t` end up exactly at view `P` (a slot of concat `ce`) without a copy?
    bool try_place(int32_t t, const VRef& P, const EOp& ce, const VRef& S) {
        Val& v = val(t);
        if (v.is_weight) return false;
        if (v.has_view) return views_equal(v.view, P);
        if (v.is_input || v.is_output || v.producer < 0) return false;
        EOp& p = eops_[v.producer];
        switch (p.k) {
            case EK::Conv:
                if (P.rank == 4 && P.str[1] != 1) return false;
                break;
            case EK::Elt:
            case EK::MaxPool:
            case EK::Resize:
            case EK::Softmax:
            case EK::Concat:
                break;
            case EK::Reshape: {
                VRef q;
                if (!reshape_view(P, val(p.in[0]).dims, &q)) return false;
                if (!try_place(p.in[0], q, ce, S)) return false;
                break;
            }
            case EK::Transpose: {
                std::vector<int32_t> inv(p.perm.size());
                for (size_t d = 0; d < p.perm.size(); ++d) inv[p.perm[d]] = static_cast<int32_t>(d);
                if (!try_place(p.in[0], permute_view(P, inv), ce, S)) return false;
                break;
            }
            case EK::Slice: {
                // Only a single-axis, step-1 slice along the concat axis can be undone.
                const Dims& ud = val(p.in[0]).dims;
                int ax = -1;
                for (size_t d = 0; d < ud.size(); ++d) {
                    if (p.sl_step[d] != 1) return false;
                    if (p.sl_start[d] != 0 || ud[d] != v.dims[d]) {
                        if (ax >= 0) return false;
                        ax = static_cast<int>(d);
                    }
                }
                if (ax < 0 || ax != ce.axis) return false;
                // P must be a slot of S along the concat axis.
                if (P.rank != S.rank || P.buf != S.buf) return false;
                for (int d = 0; d < S.rank; ++d) {
                    if (P.str[d] != S.str[d]) return false;
                    if (d != ax && P.dims[d] != S.dims[d]) return false;
                }
                // The slot's position inside S along the axis:
                const int64_t pos = (P.off - S.off) / std::max<int64_t>(1, S.str[ax]);
                const int64_t base = pos - p.sl_start[ax];
                if (base < 0 || base + ud[ax] > S.dims[ax]) return false;
                // Every other input of `ce` overlapping [base, base + ud[ax]) must be a
                // slice of the same tensor sitting at its matching position.
                int64_t off = 0;
                for (size_t j = 0; j < ce.in.size(); ++j) {
                    const int64_t len = val(ce.in[j]).dims[ce.axis];
                    const bool overlap = off < base + ud[ax] && off + len > base;
                    if (overlap && ce.in[j] != t) {
                        Val& oj = val(ce.in[j]);
                        if (oj.producer < 0) return false;
                        const EOp& pj = eops_[oj.producer];
                        if (pj.k != EK::Slice || pj.in[0] != p.in[0] || off != base + pj.sl_start[ax]) return false;
                    }
                    off += len;
                }
                VRef q = P;
                q.off -= p.sl_start[ax] * P.str[ax];
                q.dims[ax] = ud[ax];
                if (!try_place(p.in[0], q, ce, S)) return false;
                break;
            }
        }
        v.view = P;
        v.has_view = true;
        return true;
    }

    void assign_storage() {
        for (int i = static_cast<int>(eops_.size()) - 1; i >= 0; --i) {
            EOp& e = eops_[i];
            Val& o = val(e.out);
            if (!o.has_view) {
                if (view_kind(e.k)) {
                    if (o.is_output) assign_fresh(o, true);  // materialised by a copy
                } else {
                    // A conv writes channels-last even for a graph output; the
                    // output is then copied to its contiguous buffer.
                    assign_fresh(o, o.is_output && e.k != EK::Conv);
                }
            }
            if (e.k == EK::Concat) {
                const VRef S = o.view;
                int64_t off = 0;
                e.slots.clear();
                e.copy.clear();
                for (int32_t t : e.in) {
                    const int64_t len = val(t).dims[e.axis];
                    const VRef P = slice_view(S, e.axis, off, len);
                    e.slots.push_back(P);
                    e.copy.push_back(!try_place(t, P, e, S));
                    off += len;
                }
            }
        }
    }

    // ---- 5. steps ---------------------------------------------------------
    VRef input_view(int32_t r) {
        Val& v = val(r);
        if (v.is_input && !v.has_view) {
            const int b = new_buf(prod(v.dims));
            plan_.input_bufs[v.input_index] = b;
            v.view = contiguous_view(b, v.dims);
            v.has_view = true;
        }
        if (!v.has_view) throw std::runtime_error("plan: tensor " + std::to_string(r) + " has no storage");
        return v.view;
    }

    void emit_copy(int node, const VRef& dst, const VRef& src) {
        Step s;
        s.kind = StepKind::Elt;
        s.node = node;
        s.elt = k::kEltCopy;
        s.out = dst;
        s.a = src;
        s.b = src;
        plan_.steps.push_back(s);
        plan_.n_copies++;
    }

    // Channels-last copy of a graph input, made once, for conv consumers.
    VRef conv_input_view(int32_t r, int node) {
        VRef x = input_view(r);
        Val& v = val(r);
        if (x.rank == 4 && x.str[1] != 1 && v.is_input) {
            if (v.nhwc_copy_buf < 0) {
                v.nhwc_copy_buf = new_buf(prod(v.dims));
                v.nhwc_view = channels_last_view(v.nhwc_copy_buf, v.dims);
                emit_copy(node, v.nhwc_view, x);
                plan_.n_copies--;  // the layout change of the input is expected
            }
            return v.nhwc_view;
        }
        return x;
    }

    void emit_conv(const EOp& e) {
        const Node& n = m_.nodes[e.node];
        const OpParams& p = n.params;
        const Dims& wd = val(e.in[1]).dims;
        const int64_t G = std::max<int64_t>(1, p.groups);
        // Tiny-Cin layers (the 3-channel stem) and tiny-Cout layers go to the
        // direct kernel, which reads any layout (no channels-last input copy);
        // so do grouped convs with few channels per group (depthwise), while
        // the others run their groups through the implicit GEMM.
        const bool small = G > 1 ? (wd[1] < 8 || wd[1] % 4 != 0 || wd[0] / G < 8)
                                 : (wd[0] < 8 || (wd[1] % 4 != 0 && wd[1] * wd[2] * wd[3] <= 64));
        const VRef x = small ? input_view(e.in[0]) : conv_input_view(e.in[0], e.node);
        const VRef y = val(e.out).view;
        Step s;
        s.node = e.node;
        s.out = y;
        s.a = x;
        s.KH = static_cast<int32_t>(wd[2]);
        s.KW = static_cast<int32_t>(wd[3]);
        s.sh = static_cast<int32_t>(p.stride_h);
        s.sw = static_cast<int32_t>(p.stride_w);
        s.ph = static_cast<int32_t>(p.pad_h);
        s.pw = static_cast<int32_t>(p.pad_w);
        s.dh = static_cast<int32_t>(p.dil_h);
        s.dw = static_cast<int32_t>(p.dil_w);
        s.groups = static_cast<int32_t>(G);
        const int64_t cin = wd[1], cout = wd[0];  // input channels per group, all output channels
        s.act = e.act;
        s.slope = e.slope;
        s.act = reference_activation(s.act, reference_conv_path(s, cin), opt_.winograd_form_silu);
        if (e.res != INT32_MIN) {
            s.has_res = true;
            s.res = input_view(e.res);
        }
        const bool cl = x.str[1] == 1 && y.str[1] == 1 && (!s.has_res || s.res.str[1] == 1);
        if (cl && !small) {
            s.kind = StepKind::ConvMfma;
            s.vec = cin % 4 == 0 && x.off % 4 == 0 && x.str[0] % 4 == 0 && x.str[2] % 4 == 0 && x.str[3] % 4 == 0;
            const int64_t M = y.dims[0] * y.dims[2] * y.dims[3];
            const int64_t K = cin * s.KH * s.KW;
            // The Winograd kernel needs the transformed weights packed at model
            // load for exactly these layers, and 16-byte aligned input pixels.
            const bool wino = s.vec && G == 1 &&
                              k::wino_eligible(s.KH, s.KW, s.sh, s.sw, s.dh, s.dw, static_cast<int>(cin)) &&
                              wino_views_ok(s);
            k::ConvLaunchShape ls;
            if (opt_.tune_conv && opt_.force_tile < 0 && opt_.split_k) {
                ls = opt_.tune_conv(conv_query(s));
            } else {
                ls = k::conv_select(M * G, static_cast<int>(cout / G), static_cast<int>(K), opt_.split_k, wino,
                                    static_cast<int>(cin));
            }
            if (k::is_wino_tile(opt_.force_tile)) {
                if (wino) ls = {opt_.force_tile, 1, static_cast<int>((K + k::kConvBK - 1) / k::kConvBK)};
            } else if (k::is_gemm_tile(opt_.force_tile)) {
                const int kg = k::conv_tile_shape(opt_.force_tile).kg;
                const int steps_total = static_cast<int>((K + k::kConvBK - 1) / k::kConvBK + kg - 1) / kg;
                const int want = std::max(1, std::min(opt_.force_splits, steps_total));
                const int steps = (steps_total + want - 1) / want;
                ls.tile = opt_.force_tile;
                ls.splits = (steps_total + steps - 1) / steps;
                ls.kt_per_split = steps * kg;
            }
            s.tile = ls.tile;
            s.splits = ls.splits;
            s.kt_per_split = ls.kt_per_split;
            if (s.splits > 1) s.ws_buf = new_buf(static_cast<int64_t>(s.splits) * M * cout);
        } else {
            s.kind = StepKind::ConvDirect;
        }
        plan_.steps.push_back(s);
    }

    void emit() {
        plan_.input_dims = in_dims_;
        plan_.input_bufs.assign(m_.graph_inputs.size(), -1);
        for (int32_t r : m_.graph_inputs) input_view(r);
        for (auto& e : eops_) {
            Val& o = val(e.out);
            switch (e.k) {
                case EK::Conv:
                    emit_conv(e);
                    break;
                case EK::Elt: {
                    Step s;
                    s.kind = StepKind::Elt;
                    s.node = e.node;
                    s.elt = e.elt;
                    s.alpha = e.alpha;
                    s.out = o.view;
                    s.a = broadcast_view(input_view(e.in[0]), o.dims);
                    s.b = e.in.size() > 1 ? broadcast_view(input_view(e.in[1]), o.dims) : s.a;
                    plan_.steps.push_back(s);
                    break;
                }
                case EK::MaxPool: {
                    const OpParams& p = m_.nodes[e.node].params;
                    Step s;
                    s.kind = StepKind::MaxPool;
                    s.node = e.node;
                    s.out = o.view;
                    s.a = input_view(e.in[0]);
                    s.KH = static_cast<int32_t>(p.kernel_h);
                    s.KW = static_cast<int32_t>(p.kernel_w);
                    s.sh = static_cast<int32_t>(p.stride_h);
                    s.sw = static_cast<int32_t>(p.stride_w);
                    s.ph = static_cast<int32_t>(p.pad_h);
                    s.pw = static_cast<int32_t>(p.pad_w);
                    plan_.steps.push_back(s);
                    break;
                }
                case EK::Resize: {
                    Step s;
                    s.kind = StepKind::Resize;
                    s.node = e.node;
                    s.out = o.view;
                    s.a = input_view(e.in[0]);
                    plan_.steps.push_back(s);
                    break;
                }
                case EK::Softmax: {
                    Step s;
                    s.kind = StepKind::Softmax;
                    s.node = e.node;
                    s.out = o.view;
                    s.a = input_view(e.in[0]);
                    s.axis = e.axis;
                    plan_.steps.push_back(s);
                    break;
                }
                case EK::Concat:
                    for (size_t j = 0; j < e.in.size(); ++j)
                        if (e.copy[j]) emit_copy(e.node, e.slots[j], input_view(e.in[j]));
                    break;
                case EK::TopK: {
                    Step s;
                    s.kind = StepKind::TopK;
                    s.node = e.node;
                    s.out = o.view;
                    s.a = input_view(e.in[0]);
                    s.axis = e.axis;
                    s.topk = e.topk;
                    s.topk_indices = e.topk_indices;
                    plan_.steps.push_back(s);
                    break;
                }
                case EK::GatherElements: {
                    Step s;
                    s.kind = StepKind::GatherElements;
                    s.node = e.node;
                    s.out = o.view;
                    s.a = input_view(e.in[0]);
                    s.b = input_view(e.in[1]);
                    s.axis = e.axis;
                    plan_.steps.push_back(s);
                    break;
                }
                case EK::Slice:
                case EK::Reshape:
                case EK::Transpose: {
                    VRef src = input_view(e.in[0]);
                    VRef f;
                    if (e.k == EK::Slice) {
                        f = src;
                        for (int d = 0; d < f.rank; ++d) f = slice_view(f, d, e.sl_start[d], o.dims[d], e.sl_step[d]);
                    } else if (e.k == EK::Transpose) {
                        f = permute_view(src, e.perm);
                    } else if (!reshape_view(src, e.target, &f)) {
                        // materialise in logical order, then the reshape is a view
                        const Dims sd = dims_of(src);
                        const int b = new_buf(prod(sd));
                        const VRef tmp = contiguous_view(b, sd);
                        emit_copy(e.node, tmp, src);
                        if (!reshape_view(tmp, e.target, &f)) fail(m_, e.node, "reshape failed");
                    }
                    if (o.has_view) {
                        if (!views_equal(f, o.view)) emit_copy(e.node, o.view, f);
                    } else {
                        o.view = f;
                        o.has_view = true;
                    }
                    break;
                }
            }
        }
        for (int32_t r : m_.graph_outputs) {
            Val& v = val(r);
            VRef ov = v.view;
            // graph outputs must be contiguous in logical order for the host copy
            const VRef want = contiguous_view(ov.buf, v.dims);
            if (ov.off != 0 || !views_equal(ov, want)) {
                const int b = new_buf(prod(v.dims));
                const VRef dst = contiguous_view(b, v.dims);
                emit_copy(-1, dst, ov);
                ov = dst;
            }
            plan_.outputs.push_back(ov);
            plan_.output_dims.push_back(v.dims);
            plan_.output_int32.push_back(holds_indices(r));
        }
    }

    // True when the value holds TopK indices: produced by an indices TopK,
    // directly or through Reshape / Slice / Transpose views (the reference
    // keeps the I32 tensor type through them).
    bool holds_indices(int32_t ref) {
        for (int hops = 0; hops < 1024; ++hops) {
            const Val& v = val(ref);
            if (v.producer < 0) return false;
            const EOp& e = eops_[v.producer];
            if (e.k == EK::TopK) return e.topk_indices;
            if ((e.k != EK::Reshape && e.k != EK::Slice && e.k != EK::Transpose) || e.in.empty()) return false;
            ref = e.in[0];
        }
        return false;
    }

    // ---- 5b. step fusion ---------------------------------------------------
    // Rewrites runs of emitted steps whose intermediates nothing else reads:
    //  - SPPF: three chained stride-1 same max pools -> one pass (MaxPoolChain);
    //  - the Detect head's DFL + dist2bbox (Softmax, 1x1 Conv to one channel,
    //    Sub, Add, Add, Div, Sub, Mul over the anchors/strides constants) ->
    //    one DetectDecode step, same arithmetic in the same order.
    bool reads_buf(const Step& s, int32_t buf) const {
        auto uses = [&](const VRef& v) { return v.buf == buf; };
        if (uses(s.a) || (s.has_res && uses(s.res))) return true;
        if ((reads_second_input(s.kind) || s.kind == StepKind::DetectDecode) && (uses(s.b) || uses(s.c))) return true;
        if (s.kind == StepKind::DetectDecode && s.cls_in.buf != -1 && uses(s.cls_in)) return true;
        return false;
    }
    // No step outside [lo, hi] reads `buf`, and it is not a graph output.
    bool private_buf(int32_t buf, size_t lo, size_t hi) const {
        if (buf < 0) return false;
        for (size_t i = 0; i < plan_.steps.size(); ++i)
            if ((i < lo || i > hi) && reads_buf(plan_.steps[i], buf)) return false;
        for (const VRef& o : plan_.outputs)
            if (o.buf == buf) return false;
        for (int32_t r : m_.graph_outputs)
            if (vals_.count(r) && vals_.at(r).view.buf == buf) return false;
        return true;
    }
    static bool is_elt(const Step& s, int op) { return s.kind == StepKind::Elt && s.elt == op; }
    static bool is_weight_view(const VRef& v) { return v.buf == kBufWeight; }

    bool match_sppf(size_t i) const {
        const auto& st = plan_.steps;
        if (i + 2 >= st.size()) return false;
        const Step& p0 = st[i];
        for (size_t j = 0; j < 3; ++j) {
            const Step& p = st[i + j];
            if (p.kind != StepKind::MaxPool || p.KH != p0.KH || p.KW != p0.KH || p.KH % 2 == 0 || p.KH > 7 || p.sh != 1 ||
                p.sw != 1 || p.ph != p0.KH / 2 || p.pw != p0.KH / 2)
                return false;
            if (p.out.rank != 4 || dims_of(p.out) != dims_of(p0.a)) return false;
        }
        return views_equal(st[i + 1].a, st[i].out) && views_equal(st[i + 2].a, st[i + 1].out);
    }

    bool match_decode(size_t i, Step* fused) const {
        const auto& st = plan_.steps;
        if (i + 7 >= st.size()) return false;
        const Step &sm = st[i], &cv = st[i + 1], &sub = st[i + 2], &add = st[i + 3], &sum = st[i + 4],
                   &dv = st[i + 5], &wh = st[i + 6], &mul = st[i + 7];
        if (sm.kind != StepKind::Softmax || sm.axis != 1 || sm.a.rank != 4 || sm.a.dims[2] != 4) return false;
        const int64_t N = sm.a.dims[0], R = sm.a.dims[1], A = sm.a.dims[3];
        // 1x1 conv of the softmax to one channel, no activation or residual
        if (cv.kind != StepKind::ConvDirect || !views_equal(cv.a, sm.out) || cv.KH != 1 || cv.KW != 1 || cv.sh != 1 ||
            cv.sw != 1 || cv.ph != 0 || cv.pw != 0 || cv.act != 0 || cv.has_res || cv.out.rank != 4 ||
            cv.out.dims[1] != 1 || cv.out.dims[2] != 4 || cv.out.dims[3] != A)
            return false;
        const Node& cn = m_.nodes[cv.node];
        if (cn.inputs.size() < 2 || cn.inputs[1] > -1000) return false;
        // distances d[side] live in cv.out; lt = sides 0..1, rb = sides 2..3
        const VRef& D = cv.out;
        auto side_view = [&](const VRef& v, int64_t first) {  // [N, 2, A] over sides first, first+1
            return v.buf == D.buf && v.rank == 3 && v.dims[1] == 2 && v.dims[2] == A &&
                   v.off == D.off + first * D.str[2] && v.str[1] == D.str[2] && v.str[2] == D.str[3];
        };
        auto anchors_ok = [&](const VRef& v) { return is_weight_view(v) && v.rank == 3 && v.dims[1] == 2; };
        if (!is_elt(sub, k::kEltSub) || !anchors_ok(sub.a) || !side_view(sub.b, 0)) return false;
        const VRef* anc_other = nullptr;
        if (is_elt(add, k::kEltAdd) && views_equal(add.a, sub.a) && side_view(add.b, 2)) anc_other = &add.a;
        if (is_elt(add, k::kEltAdd) && views_equal(add.b, sub.a) && side_view(add.a, 2)) anc_other = &add.b;
        if (!anc_other) return false;
        const bool sum_ok = is_elt(sum, k::kEltAdd) && ((views_equal(sum.a, sub.out) && views_equal(sum.b, add.out)) ||
                                                       (views_equal(sum.a, add.out) && views_equal(sum.b, sub.out)));
        if (!sum_ok) return false;
        if (!is_elt(dv, k::kEltDiv) || !views_equal(dv.a, sum.out) || !is_weight_view(dv.b)) return false;
        if (!is_elt(wh, k::kEltSub) || !views_equal(wh.a, add.out) || !views_equal(wh.b, sub.out)) return false;
        // mul reads the [N, 4, A] concat of (cxy, wh) times the strides constant
        if (!is_elt(mul, k::kEltMul) || !is_weight_view(mul.b) || mul.a.rank != 3 || mul.a.dims[1] != 4 ||
            mul.a.dims[2] != A || mul.out.rank != 3)
            return false;
        if (!views_equal(slice_view(mul.a, 1, 0, 2), dv.out) || !views_equal(slice_view(mul.a, 1, 2, 2), wh.out))
            return false;
        // every intermediate is read only inside the run
        for (int32_t b : {sm.out.buf, cv.out.buf, sub.out.buf, add.out.buf, sum.out.buf, mul.a.buf})
            if (!private_buf(b, i, i + 7)) return false;
        Step f;
        f.kind = StepKind::DetectDecode;
        f.node = sm.node;
        f.a = sm.a;
        f.b = sub.a;      // anchors
        f.c = dv.b;       // divisor
        f.res = mul.b;    // strides
        f.has_res = false;
        f.out = mul.out;
        f.dfl_weight = -1000 - cn.inputs[1];
        f.dfl_bias = (cn.inputs.size() > 2 && cn.inputs[2] <= -1000) ? -1000 - cn.inputs[2] : -1;
        f.bins = static_cast<int32_t>(R);
        (void)N;
        *fused = f;
        return true;
    }

    void fuse_steps() {
        std::vector<Step> out;
        auto& st = plan_.steps;
        for (size_t i = 0; i < st.size();) {
            if (match_sppf(i)) {  // all three outputs are still written
                Step f = st[i];
                f.kind = StepKind::MaxPoolChain;
                f.b = st[i + 1].out;
                f.c = st[i + 2].out;
                out.push_back(f);
                i += 3;
                continue;
            }
            // a conv whose output feeds a nearest 2x Resize right after it also
            // writes the upsampled copy (the FPN's upsample into its concat)
            // (not a compat-SiLU conv: its float64 second pass rewrites only y)
            if (st[i].kind == StepKind::ConvMfma && st[i].vec && !k::is_wino_tile(st[i].tile) && i + 1 < st.size() &&
                st[i].act != k::kActSiluWinogradForm && st[i + 1].kind == StepKind::Resize &&
                views_equal(st[i + 1].a, st[i].out)) {
                const VRef& y = st[i].out;
                const VRef& u = st[i + 1].out;
                if (u.rank == 4 && y.rank == 4 && u.dims[0] == y.dims[0] && u.dims[1] == y.dims[1] &&
                    u.dims[2] == 2 * y.dims[2] && u.dims[3] == 2 * y.dims[3] && u.str[1] == 1 && u.buf >= 0) {
                    Step f = st[i];
                    f.up = u;
                    out.push_back(f);
                    i += 2;
                    continue;
                }
            }
            Step f;
            if (match_decode(i, &f)) {
                i += 8;
                // the class-score sigmoid right after it (Detect's
                // cat(dbox, cls.sigmoid())) joins the same pass
                if (i < st.size() && is_elt(st[i], k::kEltSigmoid) && st[i].a.rank == 3 && st[i].out.rank == 3 &&
                    st[i].a.dims[0] == f.out.dims[0] && st[i].a.dims[2] == f.out.dims[2] &&
                    st[i].out.dims[0] == f.out.dims[0] && st[i].out.dims[1] == st[i].a.dims[1] &&
                    st[i].out.dims[2] == f.out.dims[2]) {
                    f.cls_in = st[i].a;
                    f.cls_out = st[i].out;
                    ++i;
                }
                out.push_back(f);
                continue;
            }
            out.push_back(st[i]);
            ++i;
        }
        st.swap(out);
    }

    // A fused Detect decode over anchors [0, A) whose input rows come from
    // different producers per anchor range (one conv per scale and branch,
    // writing its HxW pixels as consecutive anchors) becomes one decode step
    // per range, in anchor order.  Each part reads and writes only its
    // anchors, so it depends only on its own range's producers.
    void split_decode() {
        if (!opt_.split_outputs) return;
        auto& st = plan_.steps;
        std::vector<Step> out;
        for (size_t i = 0; i < st.size(); ++i) {
            const Step& d = st[i];
            out.push_back(d);
            if (d.kind != StepKind::DetectDecode || d.a.rank != 4 || d.a.buf < 0) continue;
            const int64_t A = d.a.dims[3], sa = d.a.str[3];
            if (sa <= 0 || A <= 1) continue;
            std::vector<int64_t> cuts = {0, A};
            bool ok = true;
            for (size_t j = 0; j < i && ok; ++j) {
                const VRef& v = st[j].out;
                if (v.buf != d.a.buf) continue;
                // [N, C, H, W] over anchors (rel / sa) + h * W + w, channels inside the row
                const int64_t rel = v.off - d.a.off;
                ok = st[j].kind == StepKind::ConvMfma && v.rank == 4 && v.str[3] == sa && v.str[2] == v.dims[3] * sa &&
                     v.str[1] == 1 && rel >= 0 && rel % sa + v.dims[1] <= sa;
                if (!ok) break;
                const int64_t a0 = rel / sa, a1 = a0 + v.dims[2] * v.dims[3];
                ok = a1 <= A;
                cuts.push_back(a0);
                cuts.push_back(a1);
            }
            std::sort(cuts.begin(), cuts.end());
            cuts.erase(std::unique(cuts.begin(), cuts.end()), cuts.end());
            if (!ok || cuts.size() < 3) continue;
            // every producer's range must fall inside one part
            for (size_t j = 0; j < i && ok; ++j) {
                const VRef& v = st[j].out;
                if (v.buf != d.a.buf) continue;
                const int64_t a0 = (v.off - d.a.off) / sa, a1 = a0 + v.dims[2] * v.dims[3];
                const auto lo = std::upper_bound(cuts.begin(), cuts.end(), a0);
                ok = lo != cuts.end() && *lo >= a1;
            }
            if (!ok) continue;
            // the anchor-indexed views: the last dim of every [.., A] view
            auto cut = [&](VRef v, int64_t a0, int64_t n) {
                if (v.buf == -1 || v.rank < 1 || v.dims[v.rank - 1] != A) return v;
                v.off += a0 * v.str[v.rank - 1];
                v.dims[v.rank - 1] = n;
                return v;
            };
            out.pop_back();
            for (size_t c = 0; c + 1 < cuts.size(); ++c) {
                const int64_t a0 = cuts[c], n = cuts[c + 1] - cuts[c];
                Step p = d;
                p.a = cut(d.a, a0, n);
                p.b = cut(d.b, a0, n);
                p.c = cut(d.c, a0, n);
                p.res = cut(d.res, a0, n);
                p.out = cut(d.out, a0, n);
                if (d.cls_in.buf != -1) {
                    p.cls_in = cut(d.cls_in, a0, n);
                    p.cls_out = cut(d.cls_out, a0, n);
                }
                out.push_back(p);
            }
        }
        st.swap(out);
    }

    // ---- 6. liveness + arena ----------------------------------------------
    bool groupable(const Step& s) const { return s.kind == StepKind::ConvMfma && s.vec && s.groups == 1; }

    // Reorders the program by list scheduling (the earliest ready step first)
    // and, where independent implicit-GEMM convs are ready together, asks the
    // measurement whether one grouped launch beats their own launches; a
    // group grows one ready conv at a time while each addition pays.
    void group_convs() {
        if (!opt_.tune_group || !opt_.tune_conv || opt_.force_tile >= 0 || !opt_.split_k) return;
        std::vector<Step>& st = plan_.steps;
        const int n = static_cast<int>(st.size());
        std::vector<std::vector<VRef>> rd(n), wr(n);
        for (int i = 0; i < n; ++i) step_views(st[i], rd[i], wr[i]);
        for (int i = 0; i < n; ++i)
            if (st[i].ws_buf >= 0) {
                VRef w;
                w.buf = st[i].ws_buf;
                w.rank = 1;
                w.dims[0] = plan_.bufs[st[i].ws_buf].elems;
                w.str[0] = 1;
                wr[i].push_back(w);
            }
        auto hit = [](const std::vector<VRef>& x, const std::vector<VRef>& y) {
            for (const VRef& u : x)
                for (const VRef& v : y)
                    if (views_may_overlap(u, v)) return true;
            return false;
        };
        std::vector<std::vector<int>> deps(n);
        for (int j = 0; j < n; ++j)
            for (int i = 0; i < j; ++i)
                if (hit(wr[i], rd[j]) || hit(wr[i], wr[j]) || hit(rd[i], wr[j])) deps[j].push_back(i);

        // Convs read only by the Detect decode (the head's last 1x1 convs of
        // every scale) wait until nothing else is ready: they then become
        // ready together, at the end, where they can share a launch.
        std::vector<char> sink(n, 0);
        for (int i = 0; i < n; ++i) {
            if (!groupable(st[i])) continue;
            bool any = false, only_decode = true;
            for (int j = i + 1; j < n; ++j)
                if (std::find(deps[j].begin(), deps[j].end(), i) != deps[j].end()) {
                    any = true;
                    only_decode = only_decode && st[j].kind == StepKind::DetectDecode;
                }
            sink[i] = any && only_decode;
        }

        // With a split Detect decode, each step takes the first decode part
        // it feeds as its priority and the list scheduling below runs the
        // ready steps of the lowest priority first: each anchor range's
        // producers and decode part before the next range's work.
        std::vector<int> pri(n, 0);
        if (opt_.split_outputs) {
            int parts = 0;
            for (int i = 0; i < n; ++i) parts += st[i].kind == StepKind::DetectDecode;
            if (parts > 1) {
                std::vector<std::vector<int>> users(n);
                for (int j = 0; j < n; ++j)
                    for (int i : deps[j]) users[i].push_back(j);
                int part = parts;
                std::vector<int> part_of(n, -1);
                for (int i = n - 1; i >= 0; --i)
                    if (st[i].kind == StepKind::DetectDecode) part_of[i] = --part;
                for (int i = n - 1; i >= 0; --i) {
                    pri[i] = part_of[i] >= 0 ? part_of[i] : parts;
                    for (int j : users[i]) pri[i] = std::min(pri[i], pri[j]);
                }
            }
        }

        std::vector<char> done(n, 0);
        std::vector<Step> out;
        int32_t next_group = 0;
        while (static_cast<int>(out.size()) < n) {
            std::vector<int> ready;
            for (int j = 0; j < n; ++j) {
                if (done[j]) continue;
                bool ok = true;
                for (int i : deps[j])
                    if (!done[i]) {
                        ok = false;
                        break;
                    }
                if (ok) ready.push_back(j);
            }
            int pmin = INT32_MAX;
            for (int j : ready) pmin = std::min(pmin, pri[j]);
            ready.erase(std::remove_if(ready.begin(), ready.end(), [&](int j) { return pri[j] != pmin; }), ready.end());
            // waiting sinks go behind every other ready step
            std::stable_partition(ready.begin(), ready.end(), [&](int j) { return !sink[j]; });
            if (!sink[ready.front()])
                ready.erase(std::remove_if(ready.begin(), ready.end(), [&](int j) { return sink[j] != 0; }),
                            ready.end());
            std::vector<int> S = {ready.front()};
            int tile = -1;
            if (groupable(st[S[0]])) {
                double cur_ms = 0.0, sep_ms = 0.0;
                // a conv writing an upsampled copy and a compat-SiLU conv take
                // different kernel builds, so they never share a launch
                auto kinds_mix = [&](const std::vector<int>& T) {
                    bool up = false, compat = false;
                    for (int t : T) {
                        up = up || st[t].up.buf != -1;
                        compat = compat || st[t].act == k::kActSiluWinogradForm;
                    }
                    return up && compat;
                };
                for (size_t r = 1; r < ready.size() && S.size() < static_cast<size_t>(k::kMaxConvGroup); ++r) {
                    const int c = ready[r];
                    if (!groupable(st[c])) continue;
                    std::vector<int> T = S;
                    T.push_back(c);
                    if (kinds_mix(T)) continue;
                    std::vector<ConvQuery> qs;
                    std::vector<k::ConvLaunchShape> solo;
                    for (int t : T) {
                        qs.push_back(conv_query(st[t]));
                        solo.push_back({st[t].tile, st[t].splits, st[t].kt_per_split});
                    }
                    const ConvGroupTiming g = opt_.tune_group(qs, solo);
                    if (g.tile < 0) continue;
                    // S alone costs cur_ms (grouped) or sep_ms (one conv); c alone
                    // costs what the separate launches of T add to those of S
                    const double base = (S.size() == 1 ? g.separate_ms : cur_ms + (g.separate_ms - sep_ms));
                    if (g.group_ms < kGroupGain * base) {
                        S = T;
                        tile = g.tile;
                        cur_ms = g.group_ms;
                        sep_ms = g.separate_ms;
                    }
                }
            }
            std::sort(S.begin(), S.end());
            for (int j : S) {
                Step s = st[j];
                if (S.size() > 1) {
                    const int kg = k::conv_tile_shape(tile).kg;
                    const int ktiles =
                        static_cast<int>((s.a.dims[1] / s.groups * s.KH * s.KW + k::kConvBK - 1) / k::kConvBK);
                    s.group = next_group;
                    s.tile = tile;
                    s.splits = 1;
                    s.kt_per_split = (ktiles + kg - 1) / kg * kg;
                    s.ws_buf = -1;
                }
                out.push_back(s);
                done[j] = 1;
            }
            if (S.size() > 1) ++next_group;
        }
        st = std::move(out);
    }

    void touch(const VRef& v, int step) {
        if (v.buf < 0) return;
        Buffer& b = plan_.bufs[v.buf];
        b.first = std::min(b.first, step);
        b.last = std::max(b.last, step);
    }

    // Every element a step's views (and the graph's input and output views)
    // can address lies inside the view's own buffer: a kernel indexes only
    // through these views, so a plan that passes cannot send one outside
    // its allocation.
    void check_bounds() const {
        auto check = [&](const VRef& v, int64_t step, const char* what) {
            if (v.buf < 0) return;
            if (v.buf >= static_cast<int32_t>(plan_.bufs.size()))
                throw std::logic_error("plan: step " + std::to_string(step) + " " + what + " names no buffer");
            int64_t lo = v.off, hi = v.off;
            for (int d = 0; d < v.rank; ++d) {
                if (v.dims[d] <= 0) return;
                const int64_t span = (v.dims[d] - 1) * v.str[d];
                if (span < 0) lo += span;
                else hi += span;
            }
            if (lo < 0 || hi >= plan_.bufs[v.buf].elems)
                throw std::logic_error("plan: step " + std::to_string(step) + " " + what + " view [" +
                                       std::to_string(lo) + ", " + std::to_string(hi) + "] outside its buffer of " +
                                       std::to_string(plan_.bufs[v.buf].elems) + " elements");
        };
        std::vector<VRef> rd, wr;
        for (size_t i = 0; i < plan_.steps.size(); ++i) {
            step_views(plan_.steps[i], rd, wr);
            for (const VRef& v : rd) check(v, static_cast<int64_t>(i), "read");
            for (const VRef& v : wr) check(v, static_cast<int64_t>(i), "write");
        }
        for (const VRef& v : plan_.outputs) check(v, -1, "graph output");
    }

    // Length of the leading run of steps that process each image on its own
    // (conv and elementwise steps whose every view has the batch N as its
    // outer dimension, or is broadcast over it) on outputs of at least
    // early_hw pixels, ending at a grouped launch's end.
    int early_prefix() const {
        if (opt_.early_hw <= 0 || plan_.input_dims.empty() || plan_.input_dims[0].empty()) return 0;
        const int64_t N = plan_.input_dims[0][0];
        if (N < 2) return 0;
        auto batch_view = [&](const VRef& v, bool broadcast_ok) {
            if (v.buf == -1 || v.buf == kBufWeight) return true;
            if (v.rank < 1) return false;
            if (v.dims[0] == N) return v.str[0] > 0 || N == 1;
            return broadcast_ok && v.dims[0] == 1;
        };
        const auto& st = plan_.steps;
        int e = 0;
        for (size_t i = 0; i < st.size(); ++i) {
            const Step& s = st[i];
            bool ok = false;
            if (s.kind == StepKind::ConvMfma || s.kind == StepKind::ConvDirect) {
                ok = s.out.rank == 4 && s.out.dims[2] * s.out.dims[3] >= opt_.early_hw && batch_view(s.out, false) &&
                     batch_view(s.a, false) && (!s.has_res || batch_view(s.res, false)) &&
                     (s.kind != StepKind::ConvMfma || s.up.buf == -1 || batch_view(s.up, false));
            } else if (s.kind == StepKind::Elt) {
                int64_t hw = 1;
                for (int d = 2; d < s.out.rank; ++d) hw *= s.out.dims[d];
                ok = s.out.rank >= 3 && hw >= opt_.early_hw && batch_view(s.out, false) && batch_view(s.a, true) &&
                     batch_view(s.b, true);
            }
            if (!ok) break;
            const bool group_continues = s.group >= 0 && i + 1 < st.size() && st[i + 1].group == s.group;
            if (!group_continues) e = static_cast<int>(i) + 1;
        }
        return e;
    }

    void allocate() {
        const int n = static_cast<int>(plan_.steps.size());
        if (!opt_.reuse_memory) {
            // every tensor keeps its own memory for the whole program
            for (Buffer& b : plan_.bufs) {
                b.first = -1;
                b.last = n;
            }
        }
        // The steps of one grouped launch run at the same time: each of them
        // uses its buffers over the whole span of the group.
        std::vector<int> lo(n), hi(n);
        for (int i = 0; i < n; ++i) {
            const int32_t g = plan_.steps[i].group;
            lo[i] = (g >= 0 && i > 0 && plan_.steps[i - 1].group == g) ? lo[i - 1] : i;
        }
        for (int i = n - 1; i >= 0; --i) {
            const int32_t g = plan_.steps[i].group;
            hi[i] = (g >= 0 && i + 1 < n && plan_.steps[i + 1].group == g) ? hi[i + 1] : i;
        }
        for (int i = 0; i < n; ++i) {
            const Step& s = plan_.steps[i];
            for (int t : {lo[i], hi[i]}) {
                touch(s.out, t);
                touch(s.a, t);
                if (reads_second_input(s.kind)) touch(s.b, t);
                if (s.kind == StepKind::MaxPoolChain) {
                    touch(s.b, t);
                    touch(s.c, t);
                }
                if (s.has_res) touch(s.res, t);
                if (s.kind == StepKind::DetectDecode && s.cls_in.buf != -1) {
                    touch(s.cls_in, t);
                    touch(s.cls_out, t);
                }
                if (s.kind == StepKind::ConvMfma && s.up.buf != -1) touch(s.up, t);
                if (s.ws_buf >= 0) {
                    plan_.bufs[s.ws_buf].first = std::min(plan_.bufs[s.ws_buf].first, t);
                    plan_.bufs[s.ws_buf].last = std::max(plan_.bufs[s.ws_buf].last, t);
                }
            }
        }
        for (int b : plan_.input_bufs) {
            plan_.bufs[b].first = -1;
            plan_.bufs[b].last = std::max(plan_.bufs[b].last, -1);
        }
        // the early steps run once per batch chunk, chunk after chunk: every
        // buffer they touch stays live over the whole early segment
        plan_.early_steps = early_prefix();
        if (plan_.early_steps > 0) {
            const int e = plan_.early_steps;
            for (Buffer& b : plan_.bufs)
                if (b.first <= b.last && b.first < e) {
                    b.first = std::min(b.first, 0);
                    b.last = std::max(b.last, e - 1);
                }
        }
        for (const VRef& o : plan_.outputs) {
            plan_.bufs[o.buf].first = std::min(plan_.bufs[o.buf].first, n);
            plan_.bufs[o.buf].last = n;
        }
        // Greedy by size: each buffer takes the lowest 256-byte aligned offset that
        // does not overlap a live-range-overlapping buffer already placed.
        std::vector<int> order(plan_.bufs.size());
        for (size_t i = 0; i < order.size(); ++i) order[i] = static_cast<int>(i);
        std::sort(order.begin(), order.end(), [&](int a, int b) {
            if (plan_.bufs[a].elems != plan_.bufs[b].elems) return plan_.bufs[a].elems > plan_.bufs[b].elems;
            return a < b;
        });
        constexpr int64_t kAlign = 64;  // floats
        std::vector<int> placed;
        int64_t top = 0;
        for (int id : order) {
            Buffer& b = plan_.bufs[id];
            if (b.last < b.first) {  // never used
                b.first = b.last = 0;
            }
            std::vector<std::pair<int64_t, int64_t>> busy;
            for (int q : placed) {
                const Buffer& o = plan_.bufs[q];
                if (o.first <= b.last && b.first <= o.last) busy.push_back({o.offset, o.offset + o.elems});
            }
            std::sort(busy.begin(), busy.end());
            int64_t off = 0;
            for (auto& iv : busy) {
                if (off + b.elems <= iv.first) break;
                off = std::max(off, (iv.second + kAlign - 1) / kAlign * kAlign);
            }
            b.offset = off;
            top = std::max(top, off + (b.elems + kAlign - 1) / kAlign * kAlign);
            placed.push_back(id);
        }
        plan_.arena_elems = top;
    }
};

const char* step_kind_name(StepKind k) {
    switch (k) {
        case StepKind::ConvMfma: return "conv_mfma";
        case StepKind::ConvDirect: return "conv_direct";
        case StepKind::Elt: return "eltwise";
        case StepKind::MaxPool: return "maxpool";
        case StepKind::Resize: return "resize";
        case StepKind::Softmax: return "softmax";
        case StepKind::MaxPoolChain: return "maxpool_chain";
        case StepKind::DetectDecode: return "detect_decode";
        case StepKind::TopK: return "topk";
        case StepKind::GatherElements: return "gather_elements";
    }
    return "?";
}

std::string fmt_view(const VRef& v) {
    std::ostringstream os;
    os << "b" << v.buf << "+" << v.off << "[";
    for (int d = 0; d < v.rank; ++d) os << (d ? "," : "") << v.dims[d];
    os << "]s[";
    for (int d = 0; d < v.rank; ++d) os << (d ? "," : "") << v.str[d];
    os << "]";
    return os.str();
}

}  // namespace

namespace {

// Arena element range [lo, hi) a view can touch (weights: none).
std::pair<int64_t, int64_t> view_range(const Plan& p, const VRef& v) {
    if (v.buf < 0) return {0, 0};
    int64_t lo = p.bufs[v.buf].offset + v.off, hi = lo;
    for (int d = 0; d < v.rank; ++d) {
        if (v.dims[d] <= 0) return {0, 0};
        const int64_t span = (v.dims[d] - 1) * v.str[d];
        if (span < 0) lo += span;
        else hi += span;
    }
    return {lo, hi + 1};
}

using Ranges = std::vector<std::pair<int64_t, int64_t>>;

bool overlap(const Ranges& a, const Ranges& b) {
    for (const auto& x : a)
        for (const auto& y : b)
            if (x.first < y.second && y.first < x.second && x.first < x.second && y.first < y.second) return true;
    return false;
}

}  // namespace

Schedule schedule_plan(const Plan& p, int max_streams) {
    const int n = static_cast<int>(p.steps.size());
    std::vector<Ranges> rd(n), wr(n);
    for (int i = 0; i < n; ++i) {
        const Step& s = p.steps[i];
        wr[i].push_back(view_range(p, s.out));
        rd[i].push_back(view_range(p, s.a));
        if (reads_second_input(s.kind)) rd[i].push_back(view_range(p, s.b));
        if (s.has_res) rd[i].push_back(view_range(p, s.res));
        if (s.kind == StepKind::MaxPoolChain) {
            wr[i].push_back(view_range(p, s.b));
            wr[i].push_back(view_range(p, s.c));
        }
        if (s.kind == StepKind::DetectDecode && s.cls_in.buf != -1) {
            rd[i].push_back(view_range(p, s.cls_in));
            wr[i].push_back(view_range(p, s.cls_out));
        }
        if (s.kind == StepKind::ConvMfma && s.up.buf != -1) wr[i].push_back(view_range(p, s.up));
        if (s.ws_buf >= 0) {
            const Buffer& b = p.bufs[s.ws_buf];
            wr[i].push_back({b.offset, b.offset + b.elems});
        }
    }
    Schedule sc;
    sc.stream.assign(n, 0);
    sc.waits.assign(n, {});
    sc.recorded.assign(n, false);
    sc.deps.assign(n, {});
    const size_t words = (static_cast<size_t>(n) + 63) / 64;
    std::vector<std::vector<uint64_t>> anc(n, std::vector<uint64_t>(words, 0));
    auto has = [&](int j, int i) { return (anc[j][i / 64] >> (i % 64)) & 1u; };
    std::vector<int> tail;  // last step of each stream
    for (int j = 0; j < n; ++j) {
        for (int i = 0; i < j; ++i)
            if (overlap(wr[i], rd[j]) || overlap(wr[i], wr[j]) || overlap(rd[i], wr[j])) sc.deps[j].push_back(i);
        for (int i : sc.deps[j]) {
            anc[j][i / 64] |= uint64_t{1} << (i % 64);
            for (size_t w = 0; w < words; ++w) anc[j][w] |= anc[i][w];
        }
        // direct hazards not implied by another direct hazard
        std::vector<int> red;
        for (int i : sc.deps[j]) {
            bool implied = false;
            for (int k2 : sc.deps[j])
                if (k2 != i && has(k2, i)) {
                    implied = true;
                    break;
                }
            if (!implied) red.push_back(i);
        }
        // stream: continue the chain of the latest reduced dependency if it is
        // a stream tail; else a stream whose tail is an ancestor (no false
        // ordering); else a new stream; else the stream with the oldest tail.
        int pick = -1;
        for (int t = 0; t < static_cast<int>(tail.size()); ++t)
            if (std::find(red.begin(), red.end(), tail[t]) != red.end() && (pick < 0 || tail[t] > tail[pick])) pick = t;
        if (pick < 0)
            for (int t = 0; t < static_cast<int>(tail.size()); ++t)
                if (has(j, tail[t]) && (pick < 0 || tail[t] > tail[pick])) pick = t;
        if (pick < 0 && static_cast<int>(tail.size()) < max_streams) {
            tail.push_back(-1);
            pick = static_cast<int>(tail.size()) - 1;
        }
        if (pick < 0) {
            pick = 0;
            for (int t = 1; t < static_cast<int>(tail.size()); ++t)
                if (tail[t] < tail[pick]) pick = t;
        }
        sc.stream[j] = pick;
        for (int i : red)
            if (sc.stream[i] != pick) {
                sc.waits[j].push_back(i);
                sc.recorded[i] = true;
            }
        tail[pick] = j;
    }
    sc.n_streams = std::max<int>(1, static_cast<int>(tail.size()));
    return sc;
}

Plan build_plan(const Model& m, const std::vector<std::vector<int64_t>>& input_dims, const PlanOptions& opt) {
    Planner p(m, input_dims, opt);
    return p.run();
}

std::string describe_plan(const Model& m, const Plan& p) {
    std::ostringstream os;
    int int32_outputs = 0;
    for (bool b : p.output_int32) int32_outputs += b;
    os << "steps=" << p.steps.size() << " bufs=" << p.bufs.size() << " arena_bytes=" << p.arena_elems * 4
       << " copies=" << p.n_copies << " int32_outputs=" << int32_outputs << " early_steps=" << p.early_steps << "\n";
    for (size_t i = 0; i < p.steps.size(); ++i) {
        const Step& s = p.steps[i];
        os << i << " " << step_kind_name(s.kind);
        if (s.kind == StepKind::Elt) os << "(" << s.elt << ")";
        if (s.kind == StepKind::ConvMfma)
            os << "(tile=" << k::conv_tile_name(s.tile) << ",vec=" << s.vec << ",splits=" << s.splits << ",act=" << s.act
               << ")";
        if (s.group >= 0) os << " group=" << s.group;
        if (s.kind == StepKind::ConvDirect) os << "(act=" << s.act << ")";
        if (s.kind == StepKind::ConvMfma || s.kind == StepKind::ConvDirect)
            os << " k=" << s.KH << "x" << s.KW << " s=" << s.sh << "x" << s.sw;
        if ((s.kind == StepKind::ConvMfma || s.kind == StepKind::ConvDirect) && s.groups > 1) os << " groups=" << s.groups;
        os << " node=" << s.node;
        if (s.node >= 0) os << " '" << m.nodes[s.node].name << "'";
        os << " out=" << fmt_view(s.out) << " a=" << fmt_view(s.a);
        if ((s.kind == StepKind::Elt && s.elt >= k::kEltAdd && s.elt <= k::kEltDiv) || s.kind == StepKind::GatherElements)
            os << " b=" << fmt_view(s.b);
        if (s.kind == StepKind::TopK)
            os << " axis=" << s.axis << " k=" << s.topk << (s.topk_indices ? " indices" : " values");
        if (s.kind == StepKind::GatherElements) os << " axis=" << s.axis;
        if (s.has_res) os << " res=" << fmt_view(s.res);
        if (s.kind == StepKind::ConvMfma && s.up.buf != -1) os << " up=" << fmt_view(s.up);
        if (s.kind == StepKind::DetectDecode && s.cls_in.buf != -1)
            os << " cls=" << fmt_view(s.cls_in) << " clsout=" << fmt_view(s.cls_out);
        os << "\n";
    }
    os << "arena";  // element offset of every buffer
    for (size_t b = 0; b < p.bufs.size(); ++b) os << " b" << b << "@" << p.bufs[b].offset;
    os << "\n";
    return os.str();
}

}  // namespace pdefa
