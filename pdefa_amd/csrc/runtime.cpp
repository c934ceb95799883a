#include "runtime.hpp"

#include "conv_tune.hpp"

#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <sstream>
#include <unordered_map>

namespace pdefa {

void hip_check(hipError_t e, const char* expr, const char* file, int line) {
    if (e == hipSuccess) return;
    std::ostringstream os;
    os << "HIP error " << hipGetErrorName(e) << " (" << hipGetErrorString(e) << ") at " << expr << " [" << file << ":"
       << line << "]";
    throw HipError(e, os.str());
}

bool device_available() {
    static int cached = -1;
    if (cached < 0) {
        int n = 0;
        cached = (hipGetDeviceCount(&n) == hipSuccess && n > 0) ? 1 : 0;
    }
    return cached == 1;
}

// Page-locking memory costs far more than a plain allocation, so freed
// blocks go back to a pool (sizes rounded up to 64 KiB) and a later request
// takes the smallest pooled block that holds it, at most twice its size.  The
// pool keeps up to 1 GiB; blocks beyond that are released.  Pooled blocks
// stay allocated until the process ends.  Page-locked bytes, live and
// pooled, stay under PDEFA_PINNED_LIMIT_MB (default 4096): a request beyond
// it first releases pooled blocks, then falls back to pageable memory.
// PDEFA_PINNED=0 turns page-locking off (every tensor pageable).
namespace {
constexpr size_t kPinnedGrain = 64 * 1024;
constexpr size_t kPinnedPoolCap = size_t{1} << 30;
std::mutex g_pinned_mu;
std::multimap<size_t, void*> g_pinned_pool;          // size -> free block
std::unordered_map<void*, size_t> g_pinned_size;      // every live or pooled block
size_t g_pinned_pooled = 0;
size_t g_pinned_total = 0;  // bytes of every live or pooled block

bool pinning_enabled() {
    static const bool on = [] {
        const char* e = std::getenv("PDEFA_PINNED");
        return !(e && e[0] == '0');
    }();
    return on;
}

size_t pinned_limit() {
    static const size_t lim = [] {
        const char* e = std::getenv("PDEFA_PINNED_LIMIT_MB");
        const long long mb = e ? std::atoll(e) : 4096;
        return static_cast<size_t>(mb > 0 ? mb : 0) << 20;
    }();
    return lim;
}
}  // namespace

void* pinned_alloc(size_t bytes) {
    if (!pinning_enabled() || !device_available()) return nullptr;
    const size_t sz = (bytes + kPinnedGrain - 1) / kPinnedGrain * kPinnedGrain;
    std::vector<void*> release;  // pooled blocks given back to make room
    {
        std::lock_guard<std::mutex> lk(g_pinned_mu);
        auto it = g_pinned_pool.lower_bound(sz);
        if (it != g_pinned_pool.end() && it->first <= 2 * sz) {
            void* p = it->second;
            g_pinned_pooled -= it->first;
            g_pinned_pool.erase(it);
            return p;
        }
        while (g_pinned_total + sz > pinned_limit() && !g_pinned_pool.empty()) {
            auto big = std::prev(g_pinned_pool.end());
            release.push_back(big->second);
            g_pinned_pooled -= big->first;
            g_pinned_total -= big->first;
            g_pinned_size.erase(big->second);
            g_pinned_pool.erase(big);
        }
        if (g_pinned_total + sz > pinned_limit()) {
            for (void* q : release) (void)hipHostFree(q);
            return nullptr;  // pageable fallback
        }
        g_pinned_total += sz;  // reserved before the allocation below
    }
    for (void* q : release) (void)hipHostFree(q);
    void* p = nullptr;
    if (hipHostMalloc(&p, sz, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        std::lock_guard<std::mutex> lk(g_pinned_mu);
        g_pinned_total -= sz;
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_pinned_mu);
    g_pinned_size[p] = sz;
    return p;
}

void pinned_free(void* p) {
    if (!p) return;
    std::unique_lock<std::mutex> lk(g_pinned_mu);
    auto it = g_pinned_size.find(p);
    const size_t sz = it == g_pinned_size.end() ? 0 : it->second;
    if (sz && g_pinned_pooled + sz <= kPinnedPoolCap) {
        g_pinned_pool.emplace(sz, p);
        g_pinned_pooled += sz;
        return;
    }
    if (it != g_pinned_size.end()) {
        g_pinned_total -= sz;
        g_pinned_size.erase(it);
    }
    lk.unlock();
    (void)hipHostFree(p);
}

namespace {

bool env_flag(const char* name, bool dflt) {
    const char* v = std::getenv(name);
    if (!v || !*v) return dflt;
    return !(v[0] == '0' || v[0] == 'n' || v[0] == 'N' || v[0] == 'f' || v[0] == 'F');
}

constexpr size_t kAlignFloats = 64;
constexpr int kMaxCaptureStreams = 8;
size_t align_up(size_t n) { return (n + kAlignFloats - 1) / kAlignFloats * kAlignFloats; }

// ---- pre-pack cache: the packed conv layouts of a model's device image,
// persisted next to its .engine file.  File: a header (magic, format
// version, device architecture, hashes of the raw weight image and of the
// blob layout, payload length and payload hash) and the payload, the packed
// part of the blob as floats.  The packed layouts are a deterministic
// function of the raw weights, the layout and the pack kernels, so a file
// whose header matches holds exactly what the device would pack; bump
// kPackFormat whenever a pack kernel or layout changes.
constexpr char kPackMagic[8] = {'P', 'D', 'F', 'A', 'P', 'A', 'C', 'K'};
constexpr uint32_t kPackFormat = 1;

struct PackHeader {
    char magic[8];
    uint32_t format;
    uint32_t reserved;
    char arch[32];
    uint64_t weights_hash, layout_hash, payload_floats, payload_hash;
};

std::atomic<int64_t> g_pack_read{0}, g_pack_written{0};

// FNV-1a over 32-bit words
uint64_t hash_words(const void* p, size_t words, uint64_t h = 1469598103934665603ull) {
    const uint32_t* w = static_cast<const uint32_t*>(p);
    for (size_t i = 0; i < words; ++i) h = (h ^ w[i]) * 1099511628211ull;
    return h;
}

std::string device_arch(int device) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return "";
    std::string a = prop.gcnArchName;
    return a.substr(0, a.find(':'));
}

// Reads the payload when the file's header matches; false otherwise (no
// file, another model, layout, architecture or format, truncation, or a
// payload that does not hash to its header's value).
bool read_pack_cache(const std::string& path, const PackHeader& want, std::vector<float>& payload) {
    std::FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    PackHeader h;
    bool ok = std::fread(&h, sizeof(h), 1, f) == 1 && std::memcmp(h.magic, want.magic, 8) == 0 &&
              h.format == want.format && std::memcmp(h.arch, want.arch, sizeof(h.arch)) == 0 &&
              h.weights_hash == want.weights_hash && h.layout_hash == want.layout_hash &&
              h.payload_floats == want.payload_floats;
    if (ok) {
        payload.resize(static_cast<size_t>(h.payload_floats));
        ok = std::fread(payload.data(), sizeof(float), payload.size(), f) == payload.size() &&
             hash_words(payload.data(), payload.size()) == h.payload_hash;
    }
    std::fclose(f);
    return ok;
}

// Writes the file through a temporary name and a rename, so that readers
// see a whole file or none; a failure leaves no file and is not an error
// (the cache only saves packing work).
bool write_pack_cache(const std::string& path, PackHeader h, const std::vector<float>& payload) {
    h.payload_hash = hash_words(payload.data(), payload.size());
    const std::string tmp = path + ".tmp" + std::to_string(static_cast<long long>(getpid()));
    std::FILE* f = std::fopen(tmp.c_str(), "wb");
    if (!f) return false;
    bool ok = std::fwrite(&h, sizeof(h), 1, f) == 1 &&
              std::fwrite(payload.data(), sizeof(float), payload.size(), f) == payload.size();
    ok = std::fclose(f) == 0 && ok;
    if (ok) ok = std::rename(tmp.c_str(), path.c_str()) == 0;
    if (!ok) std::remove(tmp.c_str());
    return ok;
}

}  // namespace

void pack_cache_stats(int64_t& read, int64_t& written) {
    read = g_pack_read.load();
    written = g_pack_written.load();
}

DeviceModel::~DeviceModel() {
    if (blob) (void)hipFree(blob);
}

std::shared_ptr<DeviceModel> upload_model(const Model& m) {
    auto dm = std::make_shared<DeviceModel>();
    PDEFA_HIP(hipGetDevice(&dm->device));
    // Blob layout: [raw weights | conv biases], copied from the host, then
    // every packed conv weight layout, written on the device from the raw
    // weights (the host never touches those regions).
    std::vector<size_t> woff(m.weights.size());
    size_t total = 0;
    for (size_t i = 0; i < m.weights.size(); ++i) {
        woff[i] = total;
        total += align_up(static_cast<size_t>(std::max<int64_t>(1, m.weights[i].numel())));
    }
    struct PackPlan {
        size_t node, wpk_off, bias_off, dpk_off, wino_off;
        int cout, cin, kh, kw, w, b, groups;  // cin: per group
        bool wino;
    };
    std::vector<PackPlan> pp;
    for (size_t i = 0; i < m.nodes.size(); ++i) {
        const Node& n = m.nodes[i];
        if (n.op != kOpConv || n.inputs.size() < 2 || n.inputs[1] > -1000) continue;
        const int w = -1000 - n.inputs[1];
        if (w >= static_cast<int>(m.weights.size()) || m.weights[w].rank != 4) continue;
        const HostTensor& wt = m.weights[w];
        PackPlan p{};
        p.node = i;
        p.cout = static_cast<int>(wt.dims[0]);
        p.cin = static_cast<int>(wt.dims[1]);
        p.kh = static_cast<int>(wt.dims[2]);
        p.kw = static_cast<int>(wt.dims[3]);
        p.w = w;
        p.b = (n.inputs.size() > 2 && n.inputs[2] <= -1000) ? -1000 - n.inputs[2] : -1;
        if (p.b >= 0 && m.weights[p.b].numel() < p.cout) p.b = -1;
        const OpParams& op = n.params;
        p.groups = static_cast<int>(std::max<int64_t>(1, op.groups));
        if (p.cout % p.groups != 0) continue;  // the planner reports the mismatch
        p.wino = p.groups == 1 && k::wino_eligible(p.kh, p.kw, static_cast<int>(op.stride_h),
                                                   static_cast<int>(op.stride_w), static_cast<int>(op.dil_h),
                                                   static_cast<int>(op.dil_w), p.cin);
        p.bias_off = total;
        total += align_up(static_cast<size_t>(p.cout));
        pp.push_back(p);
    }
    const size_t host_floats = std::max<size_t>(total, kAlignFloats);
    total = host_floats;
    for (auto& p : pp) {
        const int64_t w_group = k::packed_weight_elems(p.cout / p.groups, p.kh * p.kw * p.cin);
        p.wpk_off = total;
        total += align_up(static_cast<size_t>(w_group * p.groups));
        p.dpk_off = total;
        total += align_up(static_cast<size_t>(p.groups > 1 ? k::grouped_direct_packed_elems(p.cout, p.cin, p.kh, p.kw)
                                                           : k::direct_packed_elems(p.cout, p.kh * p.kw * p.cin)));
        if (p.wino) {
            p.wino_off = total;
            total += align_up(static_cast<size_t>(k::wino_packed_elems(p.cout, p.cin)));
        }
    }
    // host image of the uploaded part (alignment gaps and absent biases zero)
    std::vector<float> host(host_floats, 0.0f);
    for (size_t i = 0; i < m.weights.size(); ++i) {
        const HostTensor& t = m.weights[i];
        if (!t.nbytes) continue;
        if (t.dtype == kF32) {
            std::memcpy(host.data() + woff[i], t.data, t.nbytes);
        } else {
            // integer constants reach the device as float values (exact
            // below 2^24, which covers every index a kernel reads)
            float* d = host.data() + woff[i];
            for (int64_t j = 0; j < t.numel(); ++j)
                d[j] = t.dtype == kI64 ? static_cast<float>(static_cast<const int64_t*>(t.data)[j])
                                       : static_cast<float>(static_cast<const int32_t*>(t.data)[j]);
        }
    }
    for (const auto& p : pp)
        if (p.b >= 0) std::memcpy(host.data() + p.bias_off, m.weights[p.b].data, sizeof(float) * p.cout);
    dm->blob_bytes = total * sizeof(float);
    PDEFA_HIP(hipMalloc(&dm->blob, dm->blob_bytes));
    PDEFA_HIP(hipMemcpy(dm->blob, host.data(), host_floats * sizeof(float), hipMemcpyHostToDevice));
    dm->wptr.resize(m.weights.size());
    for (size_t i = 0; i < m.weights.size(); ++i) dm->wptr[i] = dm->blob + woff[i];
    dm->packs.resize(m.nodes.size());
    for (const auto& p : pp) {
        DeviceModel::Pack& pk = dm->packs[p.node];
        pk.wpk = dm->blob + p.wpk_off;
        pk.bias = dm->blob + p.bias_off;
        pk.dpk = dm->blob + p.dpk_off;
        pk.groups = p.groups;
        if (p.wino) pk.wino = dm->blob + p.wino_off;
    }
    // the pre-pack cache (PDEFA_PACK_CACHE=1, models read from a file)
    const size_t packed_floats = total - host_floats;
    const bool cache = packed_floats > 0 && !m.source_path.empty() && env_flag("PDEFA_PACK_CACHE", false);
    PackHeader hdr{};
    std::string cache_path;
    if (cache) {
        const std::string arch = device_arch(dm->device);
        std::memcpy(hdr.magic, kPackMagic, sizeof(hdr.magic));
        hdr.format = kPackFormat;
        std::snprintf(hdr.arch, sizeof(hdr.arch), "%s", arch.c_str());
        hdr.weights_hash = hash_words(host.data(), host.size());
        std::vector<uint64_t> lay = {total, host_floats};
        for (const auto& p : pp)
            for (uint64_t v : {static_cast<uint64_t>(p.node), static_cast<uint64_t>(p.wpk_off),
                               static_cast<uint64_t>(p.dpk_off), static_cast<uint64_t>(p.wino ? p.wino_off : 0),
                               static_cast<uint64_t>(p.cout), static_cast<uint64_t>(p.cin), static_cast<uint64_t>(p.kh),
                               static_cast<uint64_t>(p.kw), static_cast<uint64_t>(p.groups)})
                lay.push_back(v);
        hdr.layout_hash = hash_words(lay.data(), lay.size() * 2);
        hdr.payload_floats = packed_floats;
        cache_path = m.source_path + "." + arch + ".pack";
        std::vector<float> payload;
        if (!arch.empty() && read_pack_cache(cache_path, hdr, payload)) {
            PDEFA_HIP(hipMemcpy(dm->blob + host_floats, payload.data(), packed_floats * sizeof(float),
                                hipMemcpyHostToDevice));
            dm->packs_from_cache = true;
            g_pack_read.fetch_add(1);
            return dm;
        }
    }
    hipStream_t s;
    PDEFA_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    try {
        for (const auto& p : pp) {
            DeviceModel::Pack& pk = dm->packs[p.node];
            // group g: weight rows [g*Cout/G, (g+1)*Cout/G) packed at g * w_group
            const int cout_g = p.cout / p.groups;
            const int64_t w_group = k::packed_weight_elems(cout_g, p.kh * p.kw * p.cin);
            for (int g = 0; g < p.groups; ++g) {
                k::launch_pack_conv_weights(pk.wpk + g * w_group,
                                            dm->wptr[p.w] + static_cast<int64_t>(g) * cout_g * p.cin * p.kh * p.kw,
                                            cout_g, p.cin, p.kh, p.kw, s);
                PDEFA_HIP(hipGetLastError());
            }
            k::launch_pack_direct_weights(pk.dpk, dm->wptr[p.w], p.cout, p.cin, p.kh, p.kw, p.groups, s);
            PDEFA_HIP(hipGetLastError());
            if (p.wino) {
                k::launch_pack_wino_weights(pk.wino, dm->wptr[p.w], p.cout, p.cin, s);
                PDEFA_HIP(hipGetLastError());
            }
        }
        PDEFA_HIP(hipStreamSynchronize(s));
    } catch (...) {
        (void)hipStreamDestroy(s);
        throw;
    }
    PDEFA_HIP(hipStreamDestroy(s));
    if (cache && hdr.arch[0]) {
        std::vector<float> payload(packed_floats);
        PDEFA_HIP(hipMemcpy(payload.data(), dm->blob + host_floats, packed_floats * sizeof(float),
                            hipMemcpyDeviceToHost));
        if (write_pack_cache(cache_path, hdr, payload)) g_pack_written.fetch_add(1);
    }
    return dm;
}

std::shared_ptr<DeviceModel> device_model(Model& m) {
    std::lock_guard<std::mutex> g(m.device_mu);
    if (!m.device) m.device = upload_model(m);
    return m.device;
}

// ------------------------------------------------------------------ Session

Session::Session(Model& m) : model_(&m) {
    inputs_.assign(static_cast<size_t>(m.num_inputs()), nullptr);
    use_graph_ = env_flag("PDEFA_HIP_GRAPH", true);
    // PDEFA_CONCURRENT=1: independent branches of the program become parallel
    // graph branches; tensors then keep their own memory so that reuse adds no
    // false ordering.  Off by default: on YOLOv8 the critical path holds ~80%
    // of the steps and the measured gain was within noise.
    concurrent_ = use_graph_ && env_flag("PDEFA_CONCURRENT", false);
    keep_tensors_ = env_flag("PDEFA_KEEP_TENSORS", false);
    opts_.reuse_memory = !concurrent_ && !keep_tensors_;
    // PDEFA_SPLIT_OUTPUTS=0: the Detect decode stays one step and every
    // output is downloaded after the whole program
    opts_.split_outputs = use_graph_ && !concurrent_ && env_flag("PDEFA_SPLIT_OUTPUTS", true);
    // PDEFA_INPUT_CHUNKS=c (default 2; 0 or 1: off): batches of two or more
    // images upload in c slices, and the early steps run on each slice as
    // it lands; PDEFA_EARLY_HW: the smallest output map (H * W) of an early step
    if (const char* c = std::getenv("PDEFA_INPUT_CHUNKS")) input_chunks_ = std::atoi(c);
    if (const char* h = std::getenv("PDEFA_EARLY_HW")) early_hw_ = std::atoll(h);
    opts_.split_k = env_flag("PDEFA_SPLITK", true);
    if (const char* t = std::getenv("PDEFA_CONV_TILE")) {
        for (int i = 0; i < k::kNumConvShapes; ++i)
            if (std::strcmp(t, k::conv_tile_name(i)) == 0) opts_.force_tile = i;
        if (opts_.force_tile < 0) throw std::runtime_error(std::string("PDEFA_CONV_TILE: unknown tile ") + t);
    }
    if (const char* sp = std::getenv("PDEFA_CONV_SPLITS")) opts_.force_splits = std::atoi(sp);
    const char* silu = std::getenv("PDEFA_SILU");
    opts_.winograd_form_silu = !(silu && std::strcmp(silu, "exact") == 0);
    // PDEFA_AUTOTUNE=0: conv launch shapes from the cost model alone
    autotune_ = env_flag("PDEFA_AUTOTUNE", true);
    // PDEFA_GROUP=0: every conv keeps its own launch (no grouped launches)
    group_convs_ = env_flag("PDEFA_GROUP", true);
    // PDEFA_GROUP_TILE=<tile>: take every group the planner offers, with this
    // implicit-GEMM tile (tests of the grouped kernel)
    if (const char* t = std::getenv("PDEFA_GROUP_TILE")) {
        for (int i = 0; i < k::kNumConvShapes; ++i)
            if (k::is_gemm_tile(i) && std::strcmp(t, k::conv_tile_name(i)) == 0) group_tile_ = i;
        if (group_tile_ < 0) throw std::runtime_error(std::string("PDEFA_GROUP_TILE: unknown tile ") + t);
    }
}

Session::~Session() {
    try {
        release_prepared();
    } catch (...) {
    }
    for (hipStream_t s : side_streams_) (void)hipStreamDestroy(s);
    if (copy_out_) (void)hipStreamDestroy(copy_out_);
    if (copy_in_) (void)hipStreamDestroy(copy_in_);
    if (stream_) (void)hipStreamDestroy(stream_);
    for (StagedInput& st : staged_) {
        if (st.dev_px) (void)hipFree(st.dev_px);
        if (st.host_px) (void)hipHostFree(st.host_px);
    }
    if (dec_ws_) (void)hipFree(dec_ws_);
    if (dec_host_) (void)hipHostFree(dec_host_);
}

std::vector<std::vector<k::YoloDetection>> Session::decode(int32_t idx, const std::vector<double>& metas, double conf,
                                                           double iou, int32_t max_det) {
    if (!prep_ || runs == 0) throw std::runtime_error("decode needs a completed run");
    const Plan& plan = prep_->plan;
    if (idx < 0 || idx >= static_cast<int32_t>(plan.outputs.size())) throw std::runtime_error("output index out of range");
    const VRef& o = plan.outputs[idx];
    const auto& od = plan.output_dims[idx];
    std::vector<int64_t> dims(od.begin(), od.end());
    while (dims.size() > 3 && dims.front() == 1) dims.erase(dims.begin());
    if (o.rank != static_cast<int32_t>(od.size()) || dims.size() != 3)
        throw std::runtime_error("decode: output must be [N, 4 + classes, A]");
    if (max_det < 0) throw std::runtime_error("decode: max_det must be >= 0");
    const int32_t N = static_cast<int32_t>(dims[0]), C = static_cast<int32_t>(dims[1]), A = static_cast<int32_t>(dims[2]);
    if (!metas.empty() && metas.size() != static_cast<size_t>(5) * N)
        throw std::runtime_error("decode: one letterbox meta per image expected");
    const int r = o.rank;
    k::YoloDecodeArgs a;
    a.out = prep_->arena + plan.bufs.at(o.buf).offset + o.off;
    a.sn = o.str[r - 3];
    a.sc = o.str[r - 2];
    a.sa = o.str[r - 1];
    a.N = N;
    a.C = C;
    a.A = A;
    a.conf = conf;
    a.iou = iou;
    a.max_det = max_det;
    a.max_cand = std::min(A, k::kYoloMaxCandidates);
    a.max_cand_pow2 = 1;
    while (a.max_cand_pow2 < a.max_cand) a.max_cand_pow2 <<= 1;
    // workspace: boxes, keys (8-byte), class, run info, counts, ndet, metas, detections
    auto up8 = [](size_t b) { return (b + 255) / 256 * 256; };
    const size_t na = static_cast<size_t>(N) * A;
    const size_t b_boxes = up8(na * 4 * sizeof(double)), b_keys = up8(na * 8), b_cls = up8(na * 4), b_seg = up8(na * 4);
    const size_t b_cnt = up8(static_cast<size_t>(N) * 4), b_ndet = up8(static_cast<size_t>(N) * 4);
    const size_t b_meta = up8(static_cast<size_t>(N) * 5 * sizeof(double));
    const size_t b_dets = up8(static_cast<size_t>(N) * std::max(max_det, 1) * sizeof(k::YoloDetection));
    const size_t need = b_boxes + b_keys + b_cls + b_seg + b_cnt + b_ndet + b_meta + b_dets;
    PDEFA_HIP(hipStreamSynchronize(stream_));
    if (need > dec_ws_bytes_) {
        if (dec_ws_) (void)hipFree(dec_ws_);
        dec_ws_ = nullptr;
        dec_ws_bytes_ = 0;
        PDEFA_HIP(hipMalloc(&dec_ws_, need));
        dec_ws_bytes_ = need;
    }
    const size_t host_need = b_ndet + b_dets + b_meta;
    if (host_need > dec_host_bytes_) {
        if (dec_host_) (void)hipHostFree(dec_host_);
        dec_host_ = nullptr;
        dec_host_bytes_ = 0;
        PDEFA_HIP(hipHostMalloc(&dec_host_, host_need, hipHostMallocDefault));
        dec_host_bytes_ = host_need;
    }
    char* w = static_cast<char*>(dec_ws_);
    a.boxes = reinterpret_cast<double*>(w);
    w += b_boxes;
    a.keys = reinterpret_cast<unsigned long long*>(w);
    w += b_keys;
    a.cls = reinterpret_cast<int32_t*>(w);
    w += b_cls;
    a.seg = reinterpret_cast<int32_t*>(w);
    w += b_seg;
    a.counts = reinterpret_cast<int32_t*>(w);
    w += b_cnt;
    a.ndet = reinterpret_cast<int32_t*>(w);
    w += b_ndet;
    double* dmeta = reinterpret_cast<double*>(w);
    w += b_meta;
    a.dets = reinterpret_cast<k::YoloDetection*>(w);
    char* h = static_cast<char*>(dec_host_);
    int32_t* h_ndet = reinterpret_cast<int32_t*>(h);
    k::YoloDetection* h_dets = reinterpret_cast<k::YoloDetection*>(h + b_ndet);
    double* h_meta = reinterpret_cast<double*>(h + b_ndet + b_dets);
    if (!metas.empty()) {
        std::memcpy(h_meta, metas.data(), metas.size() * sizeof(double));
        PDEFA_HIP(hipMemcpyAsync(dmeta, h_meta, metas.size() * sizeof(double), hipMemcpyHostToDevice, stream_));
        a.meta = dmeta;
    }
    k::launch_yolo_decode(a, stream_);
    PDEFA_HIP(hipGetLastError());
    PDEFA_HIP(hipMemcpyAsync(h_ndet, a.ndet, static_cast<size_t>(N) * 4, hipMemcpyDeviceToHost, stream_));
    if (max_det > 0)
        PDEFA_HIP(hipMemcpyAsync(h_dets, a.dets, static_cast<size_t>(N) * max_det * sizeof(k::YoloDetection),
                                 hipMemcpyDeviceToHost, stream_));
    PDEFA_HIP(hipStreamSynchronize(stream_));
    std::vector<std::vector<k::YoloDetection>> out(N);
    for (int32_t i = 0; i < N; ++i) {
        if (h_ndet[i] < 0)
            throw std::runtime_error("decode: more than " + std::to_string(a.max_cand) +
                                     " anchors pass conf_thres in one image");
        out[i].assign(h_dets + static_cast<size_t>(i) * max_det, h_dets + static_cast<size_t>(i) * max_det + h_ndet[i]);
    }
    return out;
}

void Session::set_input(int32_t idx, const HostTensor* t) {
    if (idx < 0 || idx >= static_cast<int32_t>(inputs_.size())) return;  // ignored, as the reference does
    inputs_[idx] = t;
    if (idx < static_cast<int32_t>(staged_.size())) staged_[idx].images.clear();
}

std::vector<LetterboxGeometry> Session::set_images(int32_t idx, const std::vector<ImageRef>& images, int32_t tw,
                                                   int32_t th, float scale, float pad) {
    if (idx < 0 || idx >= static_cast<int32_t>(inputs_.size())) throw std::runtime_error("input index out of range");
    if (images.empty()) throw std::runtime_error("set_images: no images");
    if (tw <= 0 || th <= 0) throw std::runtime_error("set_images: target size must be positive");
    if (!device_available()) throw std::runtime_error("no HIP device available for the session");
    size_t total = 0;
    for (const ImageRef& im : images) {
        if (!im.pixels || im.width <= 0 || im.height <= 0 || (im.channels != 1 && im.channels != 3 && im.channels != 4))
            throw std::runtime_error("set_images: empty image or unsupported channel count");
        total += static_cast<size_t>(im.width) * im.height * im.channels;
        total = (total + 255) / 256 * 256;
    }
    // the previous run's upload has finished reading the pinned staging
    if (stream_) PDEFA_HIP(hipStreamSynchronize(stream_));
    if (staged_.size() < inputs_.size()) staged_.resize(inputs_.size());
    StagedInput& st = staged_[idx];
    st.images.clear();
    if (total > st.host_cap) {
        if (st.host_px) (void)hipHostFree(st.host_px);
        st.host_px = nullptr;
        st.host_cap = 0;
        PDEFA_HIP(hipHostMalloc(reinterpret_cast<void**>(&st.host_px), total, hipHostMallocDefault));
        st.host_cap = total;
    }
    st.tw = tw;
    st.th = th;
    st.scale = scale;
    st.pad = pad;
    std::vector<LetterboxGeometry> geo;
    size_t off = 0;
    for (const ImageRef& im : images) {
        const size_t n = static_cast<size_t>(im.width) * im.height * im.channels;
        std::memcpy(st.host_px + off, im.pixels, n);
        StagedImage si;
        si.offset = off;
        si.img = im;
        si.img.pixels = nullptr;
        si.g = letterbox_geometry(im.width, im.height, tw, th);
        st.images.push_back(si);
        geo.push_back(si.g);
        off = (off + n + 255) / 256 * 256;
    }
    inputs_[idx] = nullptr;
    return geo;
}

const HostTensor* Session::output(int32_t idx) const {
    if (!prep_ || idx < 0 || idx >= static_cast<int32_t>(prep_->outputs.size())) return nullptr;
    if (runs == 0) return nullptr;
    return &prep_->outputs[idx];
}

Session::Prepared::~Prepared() {
    for (InChunk& c : in_chunks) {
        if (c.exec) (void)hipGraphExecDestroy(c.exec);
        if (c.graph) (void)hipGraphDestroy(c.graph);
        if (c.ready) (void)hipEventDestroy(c.ready);
    }
    for (Segment& g : segments) {
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
        if (g.graph) (void)hipGraphDestroy(g.graph);
        if (g.done) (void)hipEventDestroy(g.done);
    }
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    for (hipEvent_t e : events)
        if (e) (void)hipEventDestroy(e);
    if (arena) (void)hipFree(arena);
    for (float* h : host_out)
        if (h) (void)hipHostFree(h);
}

void Session::release_prepared() {
    if (!prep_) return;
    if (stream_) (void)hipStreamSynchronize(stream_);
    if (copy_out_) (void)hipStreamSynchronize(copy_out_);
    if (copy_in_) (void)hipStreamSynchronize(copy_in_);
    prep_.reset();
}

namespace {

int64_t view_extent_check(const VRef& r, int64_t limit, const char* what, int step) {
    int64_t lo = r.off, hi = r.off;
    for (int d = 0; d < r.rank; ++d) {
        if (r.dims[d] <= 0) return 0;
        const int64_t span = (r.dims[d] - 1) * r.str[d];
        if (span >= 0) hi += span;
        else lo += span;
    }
    if (lo < 0 || hi >= limit) {
        std::ostringstream os;
        os << "plan view out of bounds (" << what << ", step " << step << "): [" << lo << ", " << hi << "] vs " << limit;
        throw std::runtime_error(os.str());
    }
    return hi;
}

std::string step_label(const Model& m, const Step& s, int idx) {
    std::ostringstream os;
    if (s.node >= 0) {
        const Node& n = m.nodes[s.node];
        os << "node_" << s.node << "_op" << n.op << " '" << n.name << "' [";
    } else {
        os << "step_" << idx << "_copy 'output' [";
    }
    for (int d = 0; d < s.out.rank; ++d) os << (d ? "," : "") << s.out.dims[d];
    os << "]";
    return os.str();
}

}  // namespace

void Session::prepare(const std::vector<std::vector<int64_t>>& dims) {
    release_prepared();
    auto p = std::make_unique<Prepared>();
    PlanOptions opts = opts_;
    // A single image gains nothing from either: its decode parts would only
    // split the head's grouped launches, and there is no second slice to
    // upload behind the first.
    const int64_t batch = dims.empty() || dims[0].empty() ? 0 : dims[0][0];
    bool same_batch = true;
    for (const auto& d : dims) same_batch = same_batch && !d.empty() && d[0] == batch;
    opts.split_outputs = opts.split_outputs && batch >= 2;
    const int chunks = input_chunks_;
    opts.early_hw = (use_graph_ && !concurrent_ && !keep_tensors_ && same_batch && chunks > 1 && batch >= chunks &&
                     batch % chunks == 0)
                        ? early_hw_
                        : 0;
    if (autotune_) {
        opts.tune_conv = [this](const ConvQuery& q) { return tune_conv(q, stream_); };
        // grouped launches change the program order; the concurrent capture
        // keeps one launch per step
        if (group_convs_ && !concurrent_)
            opts.tune_group = [this](const std::vector<ConvQuery>& qs, const std::vector<k::ConvLaunchShape>& solo) {
                return tune_conv_group(qs, solo, stream_);
            };
        if (group_convs_ && !concurrent_ && group_tile_ >= 0)
            opts.tune_group = [t = group_tile_](const std::vector<ConvQuery>& qs,
                                                const std::vector<k::ConvLaunchShape>&) {
                ConvGroupTiming g;  // every offered group, with this tile
                g.tile = t;
                g.group_ms = 1.0;
                g.separate_ms = static_cast<double>(qs.size());
                return g;
            };
    }
    p->plan = build_plan(*model_, dims, opts);
    const Plan& plan = p->plan;
    if (concurrent_) p->sched = schedule_plan(plan, kMaxCaptureStreams);
    PDEFA_HIP(hipMalloc(&p->arena, static_cast<size_t>(std::max<int64_t>(plan.arena_elems, 64)) * sizeof(float)));
    prep_ = std::move(p);  // owned from here so a throw below releases it

    auto V = [&](const VRef& r, const char* what, int step) -> k::View {
        k::View v;
        int64_t limit;
        float* base;
        if (r.buf == kBufWeight) {
            base = dev_->wptr.at(r.aux);
            limit = std::max<int64_t>(1, model_->weights.at(r.aux).numel());
        } else {
            const Buffer& b = plan.bufs.at(r.buf);
            base = prep_->arena + b.offset;
            limit = b.elems;
        }
        view_extent_check(r, limit, what, step);
        v.ptr = base + r.off;
        v.rank = r.rank;
        for (int d = 0; d < r.rank; ++d) {
            v.dims[d] = r.dims[d];
            v.str[d] = r.str[d];
        }
        return v;
    };

    for (size_t i = 0; i < plan.steps.size(); ++i) {
        const Step& s = plan.steps[i];
        const int si = static_cast<int>(i);
        Launch l;
        l.kind = s.kind;
        l.step = si;
        l.label = step_label(*model_, s, si);
        switch (s.kind) {
            case StepKind::ConvMfma: {
                const Node& n = model_->nodes.at(s.node);
                const DeviceModel::Pack& pk = dev_->packs.at(s.node);
                if (!pk.wpk) throw std::runtime_error("conv weights were not packed: " + n.name);
                const k::View x = V(s.a, "conv x", si), y = V(s.out, "conv y", si);
                if (x.str[1] != 1 || y.str[1] != 1) throw std::runtime_error("conv_mfma needs channels-last views");
                k::ConvArgs& c = l.conv;
                c.x = x.ptr;
                c.N = static_cast<int32_t>(x.dims[0]);
                c.groups = s.groups;
                c.Cin = static_cast<int32_t>(x.dims[1] / s.groups);  // per group
                c.H = static_cast<int32_t>(x.dims[2]);
                c.W = static_cast<int32_t>(x.dims[3]);
                c.x_sn = x.str[0];
                c.x_sh = x.str[2];
                c.x_sw = x.str[3];
                c.y = y.ptr;
                c.Cout = static_cast<int32_t>(y.dims[1] / s.groups);
                c.Ho = static_cast<int32_t>(y.dims[2]);
                c.Wo = static_cast<int32_t>(y.dims[3]);
                c.y_sn = y.str[0];
                c.y_sh = y.str[2];
                c.y_sw = y.str[3];
                if (s.has_res) {
                    const k::View r = V(s.res, "conv res", si);
                    if (r.str[1] != 1) throw std::runtime_error("conv residual must be channels-last");
                    c.res = r.ptr;
                    c.r_sn = r.str[0];
                    c.r_sh = r.str[2];
                    c.r_sw = r.str[3];
                }
                const HostTensor& wt = model_->weights.at(-1000 - n.inputs[1]);
                if (wt.dims[0] != static_cast<int64_t>(c.Cout) * s.groups || wt.dims[1] != c.Cin ||
                    x.dims[1] != static_cast<int64_t>(c.Cin) * s.groups || pk.groups != s.groups)
                    throw std::runtime_error("conv weight shape mismatch");
                if (k::is_wino_tile(s.tile)) {
                    if (!pk.wino) throw std::runtime_error("Winograd weights were not packed: " + n.name);
                    c.wpk = pk.wino;
                } else {
                    c.wpk = pk.wpk;
                }
                c.bias = pk.bias;
                // K-major weights for the compat SiLU's float64 recomputation;
                // PDEFA_JUMP_WINDOW widens its band (tests: 0.5 recomputes
                // every output of such a conv), PDEFA_JUMP_FIX=0 turns it off
                if (s.act == k::kActSiluWinogradForm && s.groups == 1 && env_flag("PDEFA_JUMP_FIX", true)) {
                    c.w_kmaj = pk.wpk;
                    if (const char* jw = std::getenv("PDEFA_JUMP_WINDOW")) {
                        const float w = std::strtof(jw, nullptr);
                        if (!(w > 0.0f && w <= 0.5f)) throw std::runtime_error("PDEFA_JUMP_WINDOW must be in (0, 0.5]");
                        c.jump_window = w;
                    }
                }
                c.KH = s.KH;
                c.KW = s.KW;
                c.sh = s.sh;
                c.sw = s.sw;
                c.ph = s.ph;
                c.pw = s.pw;
                c.dh = s.dh;
                c.dw = s.dw;
                c.K = c.KH * c.KW * c.Cin;
                c.ktiles = (c.K + k::kConvBK - 1) / k::kConvBK;
                c.w_group = k::packed_weight_elems(c.Cout, c.K);
                c.act = s.act;
                c.slope = s.slope;
                c.splits = s.splits;
                c.kt_per_split = s.kt_per_split;
                if (s.up.buf != -1) {
                    const k::View u = V(s.up, "conv upsampled out", si);
                    if (u.str[1] != 1 || u.dims[0] != c.N || u.dims[1] != c.Cout || u.dims[2] != 2 * c.Ho ||
                        u.dims[3] != 2 * c.Wo)
                        throw std::runtime_error("conv upsampled output must be channels-last [N, Cout, 2Ho, 2Wo]");
                    c.up = u.ptr;
                    c.u_sn = u.str[0];
                    c.u_sh = u.str[2];
                    c.u_sw = u.str[3];
                }
                if (s.splits > 1) {
                    const Buffer& wb = plan.bufs.at(s.ws_buf);
                    const int64_t need = static_cast<int64_t>(s.splits) * c.N * c.Ho * c.Wo * c.Cout;
                    if (wb.elems < need) throw std::runtime_error("split-K workspace too small");
                    c.ws = prep_->arena + wb.offset;
                }
                // output extent must match the conv arithmetic
                if ((c.H + 2 * c.ph - ((c.KH - 1) * c.dh + 1)) / c.sh + 1 != c.Ho ||
                    (c.W + 2 * c.pw - ((c.KW - 1) * c.dw + 1)) / c.sw + 1 != c.Wo)
                    throw std::runtime_error("conv output size mismatch");
                l.tile = s.tile;
                l.vec = s.vec;
                break;
            }
            case StepKind::ConvDirect: {
                const Node& n = model_->nodes.at(s.node);
                k::ConvDirectArgs& d = l.direct;
                d.x = V(s.a, "conv x", si);
                d.y = V(s.out, "conv y", si);
                if (s.has_res) d.res = V(s.res, "conv res", si);
                const int w = -1000 - n.inputs[1];
                const HostTensor& wt = model_->weights.at(w);
                if (wt.dims[0] != d.y.dims[1] || wt.dims[1] * s.groups != d.x.dims[1])
                    throw std::runtime_error("conv weight shape mismatch");
                const DeviceModel::Pack& pk = dev_->packs.at(s.node);
                if (pk.groups != s.groups) throw std::runtime_error("conv weights packed for other groups");
                d.groups = s.groups;
                if (!pk.dpk || !pk.bias) throw std::runtime_error("conv weights not packed");
                d.wpk = pk.dpk;
                d.bias = pk.bias;
                d.KH = s.KH;
                d.KW = s.KW;
                d.sh = s.sh;
                d.sw = s.sw;
                d.ph = s.ph;
                d.pw = s.pw;
                d.dh = s.dh;
                d.dw = s.dw;
                d.act = s.act;
                d.slope = s.slope;
                break;
            }
            case StepKind::Elt:
                l.out = V(s.out, "elt out", si);
                l.a = V(s.a, "elt a", si);
                l.b = V(s.b, "elt b", si);
                l.elt = s.elt;
                l.alpha = s.alpha;
                break;
            case StepKind::MaxPoolChain:
                l.out = V(s.out, "pool out0", si);
                l.b = V(s.b, "pool out1", si);
                l.c = V(s.c, "pool out2", si);
                l.a = V(s.a, "pool in", si);
                l.kh = s.KH;
                break;
            case StepKind::DetectDecode: {
                k::DetectDecodeArgs& d = l.decode;
                d.x = V(s.a, "decode x", si);
                d.anchors = V(s.b, "decode anchors", si);
                d.two = V(s.c, "decode divisor", si);
                d.strides = V(s.res, "decode strides", si);
                d.out = V(s.out, "decode out", si);
                const HostTensor& w = model_->weights.at(static_cast<size_t>(s.dfl_weight));
                if (w.numel() != s.bins || w.dtype != kF32) throw std::runtime_error("DFL weight shape mismatch");
                d.dfl_w = dev_->wptr.at(static_cast<size_t>(s.dfl_weight));
                d.dfl_bias = 0.0f;
                if (s.dfl_bias >= 0) {
                    const HostTensor& bt = model_->weights.at(static_cast<size_t>(s.dfl_bias));
                    if (bt.numel() != 1 || bt.dtype != kF32) throw std::runtime_error("DFL bias shape mismatch");
                    d.dfl_bias = static_cast<const float*>(bt.data)[0];
                }
                d.bins = s.bins;
                if (s.cls_in.buf != -1) {
                    d.cls = V(s.cls_in, "decode class scores", si);
                    d.cls_out = V(s.cls_out, "decode class out", si);
                }
                break;
            }
            case StepKind::TopK:
                l.out = V(s.out, "topk out", si);
                l.a = V(s.a, "topk in", si);
                l.axis = s.axis;
                l.topk = s.topk;
                l.topk_indices = s.topk_indices;
                break;
            case StepKind::GatherElements:
                l.out = V(s.out, "gather out", si);
                l.a = V(s.a, "gather data", si);
                l.b = V(s.b, "gather indices", si);
                l.axis = s.axis;
                break;
            case StepKind::MaxPool:
            case StepKind::Resize:
            case StepKind::Softmax:
                l.out = V(s.out, "out", si);
                l.a = V(s.a, "in", si);
                l.kh = s.KH;
                l.kw = s.KW;
                l.sh = s.sh;
                l.sw = s.sw;
                l.ph = s.ph;
                l.pw = s.pw;
                l.axis = s.axis;
                break;
        }
        // a member of a grouped launch joins the launch of the previous step
        if (s.group >= 0 && i > 0 && plan.steps[i - 1].group == s.group) {
            Launch& g = prep_->launches.back();
            if (g.group.empty()) g.group.push_back(g.conv);
            g.group.push_back(l.conv);
            g.label += " + " + l.label;
            if (g.group.size() > static_cast<size_t>(k::kMaxConvGroup) || !l.vec || l.tile != g.tile)
                throw std::runtime_error("bad conv group at step " + std::to_string(i));
            continue;
        }
        prep_->launches.push_back(std::move(l));
    }
    for (int32_t b : plan.input_bufs)
        if (b < 0) throw std::runtime_error("graph input has no staging buffer");
    for (size_t i = 0; i < plan.outputs.size(); ++i) {
        const VRef& o = plan.outputs[i];
        int64_t n = 1;
        for (auto d : plan.output_dims[i]) n *= d;
        view_extent_check(o, plan.bufs.at(o.buf).elems, "output", -1);
        float* h = nullptr;
        PDEFA_HIP(hipHostMalloc(reinterpret_cast<void**>(&h), static_cast<size_t>(std::max<int64_t>(n, 1)) * sizeof(float),
                                hipHostMallocDefault));
        prep_->host_out.push_back(h);
        HostTensor t;
        // TopK indices leave as I32, as the reference's indices tensor is
        // (session_ops_math.inc:346); the device holds them as float values
        t.dtype = (i < plan.output_int32.size() && plan.output_int32[i]) ? kI32 : kF32;
        t.rank = static_cast<int32_t>(plan.output_dims[i].size());
        for (int d = 0; d < t.rank; ++d) t.dims[d] = plan.output_dims[i][d];
        t.data = h;
        t.nbytes = static_cast<size_t>(n) * sizeof(float);
        t.owns = false;
        prep_->outputs.push_back(std::move(t));
    }
    plan_input_chunks();
    plan_segments();
}

void Session::launch_one(const Launch& l, hipStream_t s) {
    switch (l.kind) {
        case StepKind::ConvMfma:
            if (!l.group.empty())
                k::launch_conv_mfma_group(l.group.data(), static_cast<int>(l.group.size()), l.tile, s);
            else if (k::is_wino_tile(l.tile))
                k::launch_conv_wino(l.conv, l.tile == k::kTileWino64 ? 64 : 32, s);
            else
                k::launch_conv_mfma(l.conv, l.tile, l.vec, s);
            break;
        case StepKind::ConvDirect: k::launch_conv_direct(l.direct, s); break;
        case StepKind::Elt: k::launch_eltwise(l.elt, l.out, l.a, l.b, l.alpha, s); break;
        case StepKind::MaxPool: k::launch_maxpool(l.out, l.a, l.kh, l.kw, l.sh, l.sw, l.ph, l.pw, s); break;
        case StepKind::Resize: k::launch_resize_nearest(l.out, l.a, s); break;
        case StepKind::Softmax: k::launch_softmax(l.out, l.a, l.axis, s); break;
        case StepKind::MaxPoolChain: k::launch_maxpool_chain(l.out, l.b, l.c, l.a, l.kh, s); break;
        case StepKind::DetectDecode: k::launch_detect_decode(l.decode, s); break;
        case StepKind::TopK: k::launch_topk(l.out, l.a, l.axis, l.topk, l.topk_indices, s); break;
        case StepKind::GatherElements: k::launch_gather_elements(l.out, l.a, l.b, l.axis, s); break;
    }
}

// Issues the program on stream_ (capture origin) plus side streams following
// prep_->sched: a fork event brings the side streams into the capture, a step
// waits for its cross-stream hazards through events, and every side stream
// joins back into stream_ at the end, so the captured graph holds exactly the
// hazard edges and independent branches become parallel graph branches.
void Session::capture_concurrent() {
    const Schedule& sc = prep_->sched;
    const int ns = sc.n_streams;
    while (static_cast<int>(side_streams_.size()) < ns - 1) {
        hipStream_t s;
        PDEFA_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
        side_streams_.push_back(s);
    }
    const size_t n = prep_->launches.size();
    if (prep_->events.empty()) {
        prep_->events.assign(n + ns, nullptr);
        for (size_t i = 0; i < n; ++i)
            if (sc.recorded[i]) PDEFA_HIP(hipEventCreateWithFlags(&prep_->events[i], hipEventDisableTiming));
        for (int t = 0; t < ns; ++t) PDEFA_HIP(hipEventCreateWithFlags(&prep_->events[n + t], hipEventDisableTiming));
    }
    auto st = [&](int t) { return t == 0 ? stream_ : side_streams_[static_cast<size_t>(t - 1)]; };
    PDEFA_HIP(hipEventRecord(prep_->events[n], stream_));  // fork
    for (int t = 1; t < ns; ++t) PDEFA_HIP(hipStreamWaitEvent(st(t), prep_->events[n], 0));
    for (size_t j = 0; j < n; ++j) {
        hipStream_t s = st(sc.stream[j]);
        for (int i : sc.waits[j]) PDEFA_HIP(hipStreamWaitEvent(s, prep_->events[static_cast<size_t>(i)], 0));
        launch_one(prep_->launches[j], s);
        if (sc.recorded[j]) PDEFA_HIP(hipEventRecord(prep_->events[j], s));
    }
    for (int t = 1; t < ns; ++t) {  // join
        PDEFA_HIP(hipEventRecord(prep_->events[n + t], st(t)));
        PDEFA_HIP(hipStreamWaitEvent(stream_, prep_->events[n + t], 0));
    }
}

void Session::launch_all(hipStream_t s) {
    for (const Launch& l : prep_->launches) launch_one(l, s);
}

void Session::capture_launches(size_t first, size_t last, hipGraph_t* graph, hipGraphExec_t* exec) {
    PDEFA_HIP(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
    try {
        for (size_t i = first; i <= last && i < prep_->launches.size(); ++i) launch_one(prep_->launches[i], stream_);
    } catch (...) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(stream_, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
    }
    PDEFA_HIP(hipStreamEndCapture(stream_, graph));
    PDEFA_HIP(hipGraphInstantiate(exec, *graph, nullptr, nullptr, 0));
}

void Session::capture_list(const std::vector<Launch>& ls, hipGraph_t* graph, hipGraphExec_t* exec) {
    PDEFA_HIP(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
    try {
        for (const Launch& l : ls) launch_one(l, stream_);
    } catch (...) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(stream_, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
    }
    PDEFA_HIP(hipStreamEndCapture(stream_, graph));
    PDEFA_HIP(hipGraphInstantiate(exec, *graph, nullptr, nullptr, 0));
}

namespace {

// The view restricted to images [first, first + n) of its outer (batch)
// dimension; a view broadcast over the batch (outer dimension 1) stays.
k::View batch_slice(k::View v, int64_t N, int64_t first, int64_t n) {
    if (v.ptr == nullptr || v.rank < 1 || v.dims[0] != N) return v;
    v.ptr += first * v.str[0];
    v.dims[0] = n;
    return v;
}

void conv_slice(k::ConvArgs& c, int64_t first, int64_t n) {
    c.x += first * c.x_sn;
    c.y += first * c.y_sn;
    if (c.res) c.res += first * c.r_sn;
    if (c.up) c.up += first * c.u_sn;
    c.N = static_cast<int32_t>(n);
}

}  // namespace

// Input chunks: when the plan has early steps (a batch of two or more images
// that splits evenly into input_chunks_ slices), each slice gets its own copy
// of the early launches, restricted to its images: convs and elementwise
// steps index images through the batch stride only, so each image's results
// are those of the whole-batch launch bit for bit (same launch shapes, same
// summation order); a split-K workspace is reused slice after slice in stream
// order.
void Session::plan_input_chunks() {
    Prepared& P = *prep_;
    P.in_chunks.clear();
    P.early_launches = 0;
    const Plan& plan = P.plan;
    if (plan.early_steps <= 0 || input_chunks_ <= 1) return;
    const int64_t N = plan.input_dims.at(0).at(0);
    const int64_t c = input_chunks_;
    if (N % c != 0) return;
    size_t e = 0;
    while (e < P.launches.size() && P.launches[e].step >= 0 && P.launches[e].step < plan.early_steps) ++e;
    if (e == 0 || e == P.launches.size()) return;
    for (int32_t b : plan.input_bufs) {  // contiguous, batch outermost
        const Buffer& buf = plan.bufs.at(b);
        if (buf.elems % N != 0) return;
    }
    const int64_t n = N / c;
    for (int64_t ci = 0; ci < c; ++ci) {
        Prepared::InChunk ch;
        ch.first = ci * n;
        ch.n = n;
        for (size_t li = 0; li < e; ++li) {
            Launch l = P.launches[li];
            switch (l.kind) {
                case StepKind::ConvMfma:
                    if (l.group.empty()) {
                        conv_slice(l.conv, ch.first, n);
                    } else {
                        for (k::ConvArgs& g : l.group) conv_slice(g, ch.first, n);
                        l.conv = l.group.front();
                    }
                    break;
                case StepKind::ConvDirect:
                    l.direct.x = batch_slice(l.direct.x, N, ch.first, n);
                    l.direct.y = batch_slice(l.direct.y, N, ch.first, n);
                    if (l.direct.res.ptr) l.direct.res = batch_slice(l.direct.res, N, ch.first, n);
                    break;
                case StepKind::Elt:
                    l.out = batch_slice(l.out, N, ch.first, n);
                    l.a = batch_slice(l.a, N, ch.first, n);
                    l.b = batch_slice(l.b, N, ch.first, n);
                    break;
                default:
                    return;  // the planner's early steps are convs and elementwise steps only
            }
            ch.launches.push_back(std::move(l));
        }
        P.in_chunks.push_back(std::move(ch));
    }
    P.early_launches = e;
}

// Cuts the program after each decode part but the last (the parts of a
// Detect decode the planner split by anchor range) when the parts' outputs
// tile whole graph outputs: a run then downloads each part's rows while the
// later segments compute.  Each part writes [N, C, A_part] views (the box
// rows and, right after them, the class rows) of a dense output; a region
// is one pitched copy of N * C rows where the images' rows follow each other
// evenly, else one per image.
void Session::plan_segments() {
    Prepared& P = *prep_;
    P.segments.clear();
    P.out_split.assign(P.outputs.size(), 0);
    if (!use_graph_ || concurrent_) return;
    const size_t first0 = P.early_launches;
    // the program after the input chunks' early launches as one segment
    auto late_only = [&] {
        P.segments.clear();
        std::fill(P.out_split.begin(), P.out_split.end(), 0);
        if (first0 == 0) return;
        Segment g;
        g.first = first0;
        g.last = P.launches.size() - 1;
        P.segments.push_back(std::move(g));
    };
    if (!opts_.split_outputs) return late_only();
    const Plan& plan = P.plan;
    struct Part {
        size_t launch;
        std::vector<Region> regions;
    };
    std::vector<Part> parts;
    std::vector<int64_t> covered(P.outputs.size(), 0);
    for (size_t li = 0; li < P.launches.size(); ++li) {
        const Launch& l = P.launches[li];
        if (l.kind != StepKind::DetectDecode || l.step < 0) continue;
        const Step& s = plan.steps.at(static_cast<size_t>(l.step));
        size_t o = P.outputs.size();
        for (size_t i = 0; i < plan.outputs.size(); ++i)
            if (plan.outputs[i].buf == s.out.buf) o = i;
        if (o == P.outputs.size()) continue;
        const VRef& O = plan.outputs[o];
        // the output view must be dense row-major for host offsets to follow
        // buffer offsets
        int64_t numel = 1;
        bool dense = O.buf >= 0;
        for (int d = O.rank - 1; d >= 0 && dense; --d) {
            dense = O.str[d] == numel;
            numel *= O.dims[d];
        }
        if (!dense) return late_only();
        VRef v = s.out;
        if (s.cls_in.buf != -1) {
            const VRef& c = s.cls_out;
            if (c.buf != v.buf || c.rank != 3 || v.rank != 3 || c.off != v.off + v.dims[1] * v.str[1] ||
                c.str[0] != v.str[0] || c.str[1] != v.str[1] || c.str[2] != v.str[2] || c.dims[0] != v.dims[0] ||
                c.dims[2] != v.dims[2])
                return late_only();
            v.dims[1] += c.dims[1];
        }
        if (v.rank != 3 || v.str[2] != 1 || v.dims[0] <= 0 || v.dims[1] <= 0 || v.dims[2] <= 0) return late_only();
        const int64_t rel = v.off - O.off;
        const int64_t span = (v.dims[0] - 1) * v.str[0] + (v.dims[1] - 1) * v.str[1] + v.dims[2];
        if (rel < 0 || rel + span > numel) return late_only();
        Part part{li, {}};
        const bool even = v.dims[0] == 1 || v.str[0] == v.dims[1] * v.str[1];
        for (int64_t n = 0; n < (even ? 1 : v.dims[0]); ++n) {
            Region r;
            r.out = o;
            r.dev = plan.bufs.at(v.buf).offset + v.off + n * v.str[0];
            r.host = rel + n * v.str[0];
            r.width = v.dims[2];
            r.rows = even ? v.dims[0] * v.dims[1] : v.dims[1];
            r.pitch = v.str[1];
            part.regions.push_back(r);
        }
        covered[o] += v.dims[0] * v.dims[1] * v.dims[2];
        parts.push_back(std::move(part));
    }
    if (parts.size() < 2) return late_only();
    for (const Part& p : parts) {
        const size_t o = p.regions.front().out;
        int64_t numel = 1;
        for (auto d : plan.output_dims[o]) numel *= d;
        if (covered[o] != numel) return late_only();  // the parts leave rows of the output to a full download
        P.out_split[o] = 1;
    }
    const size_t cuts = parts.size() - 1;
    size_t first = first0;
    for (size_t k = 0; k <= cuts; ++k) {
        Segment g;
        g.first = first;
        g.last = k < cuts ? parts[k].launch : P.launches.size() - 1;
        g.regions = parts[k].regions;
        first = g.last + 1;
        P.segments.push_back(std::move(g));
    }
}

// One run: the inputs (slice by slice on copy_in_ when the early launches
// run per input chunk: chunk c's early graph waits for its slice only), then
// the segments on the session stream; after each segment but the last its
// regions go down on copy_out_ (waiting for that segment only); the last
// segment's regions and the other outputs follow it on the session stream.
// Ends with everything finished.
void Session::run_segments() {
    Prepared& P = *prep_;
    const Plan& plan = P.plan;
    if (!copy_out_) PDEFA_HIP(hipStreamCreateWithFlags(&copy_out_, hipStreamNonBlocking));
    if (P.in_chunks.empty() || has_staged()) {
        upload_inputs();
        for (Prepared::InChunk& c : P.in_chunks) {
            if (!c.exec) capture_list(c.launches, &c.graph, &c.exec);
            PDEFA_HIP(hipGraphLaunch(c.exec, stream_));
        }
    } else {
        if (!copy_in_) PDEFA_HIP(hipStreamCreateWithFlags(&copy_in_, hipStreamNonBlocking));
        const int64_t N = plan.input_dims.at(0).at(0);
        // the session stream's earlier work (the previous run) is finished:
        // runs end synchronised
        for (Prepared::InChunk& c : P.in_chunks) {
            if (!c.exec) capture_list(c.launches, &c.graph, &c.exec);
            if (!c.ready) PDEFA_HIP(hipEventCreateWithFlags(&c.ready, hipEventDisableTiming));
            for (size_t i = 0; i < inputs_.size(); ++i) {
                const HostTensor* t = inputs_[i];
                const size_t per_image = t->nbytes / static_cast<size_t>(N);
                float* dst = P.arena + plan.bufs.at(plan.input_bufs[i]).offset;
                PDEFA_HIP(hipMemcpyAsync(reinterpret_cast<char*>(dst) + c.first * per_image,
                                         static_cast<const char*>(t->data) + c.first * per_image,
                                         static_cast<size_t>(c.n) * per_image, hipMemcpyHostToDevice, copy_in_));
            }
            PDEFA_HIP(hipEventRecord(c.ready, copy_in_));
        }
        for (Prepared::InChunk& c : P.in_chunks) {
            PDEFA_HIP(hipStreamWaitEvent(stream_, c.ready, 0));
            PDEFA_HIP(hipGraphLaunch(c.exec, stream_));
        }
    }
    auto copy = [&](const Region& r, hipStream_t s) {
        PDEFA_HIP(hipMemcpy2DAsync(P.host_out[r.out] + r.host, static_cast<size_t>(r.pitch) * sizeof(float),
                                   P.arena + r.dev, static_cast<size_t>(r.pitch) * sizeof(float),
                                   static_cast<size_t>(r.width) * sizeof(float), static_cast<size_t>(r.rows),
                                   hipMemcpyDeviceToHost, s));
    };
    for (size_t k = 0; k < P.segments.size(); ++k) {
        Segment& g = P.segments[k];
        if (!g.exec) capture_launches(g.first, g.last, &g.graph, &g.exec);
        PDEFA_HIP(hipGraphLaunch(g.exec, stream_));
        if (k + 1 < P.segments.size()) {
            if (!g.done) PDEFA_HIP(hipEventCreateWithFlags(&g.done, hipEventDisableTiming));
            PDEFA_HIP(hipEventRecord(g.done, stream_));
            PDEFA_HIP(hipStreamWaitEvent(copy_out_, g.done, 0));
            for (const Region& r : g.regions) copy(r, copy_out_);
        } else {
            for (const Region& r : g.regions) copy(r, stream_);
        }
    }
    for (size_t i = 0; i < plan.outputs.size(); ++i) {
        if (P.out_split[i]) continue;
        const float* src = P.arena + plan.bufs.at(plan.outputs[i].buf).offset + plan.outputs[i].off;
        PDEFA_HIP(hipMemcpyAsync(P.host_out[i], src, P.outputs[i].nbytes, hipMemcpyDeviceToHost, stream_));
    }
    PDEFA_HIP(hipStreamSynchronize(stream_));
    PDEFA_HIP(hipStreamSynchronize(copy_out_));
    if (copy_in_) PDEFA_HIP(hipStreamSynchronize(copy_in_));
}

void Session::upload_inputs() {
    const Plan& plan = prep_->plan;
    for (size_t i = 0; i < inputs_.size(); ++i) {
        float* dst = prep_->arena + plan.bufs.at(plan.input_bufs[i]).offset;
        if (i < staged_.size() && !staged_[i].images.empty()) {
            StagedInput& st = staged_[i];
            const StagedImage& last = st.images.back();
            const size_t bytes = last.offset + static_cast<size_t>(last.img.width) * last.img.height * last.img.channels;
            if (bytes > st.dev_cap) {
                PDEFA_HIP(hipStreamSynchronize(stream_));
                if (st.dev_px) (void)hipFree(st.dev_px);
                st.dev_px = nullptr;
                st.dev_cap = 0;
                PDEFA_HIP(hipMalloc(reinterpret_cast<void**>(&st.dev_px), bytes));
                st.dev_cap = bytes;
            }
            PDEFA_HIP(hipMemcpyAsync(st.dev_px, st.host_px, bytes, hipMemcpyHostToDevice, stream_));
            const size_t plane = static_cast<size_t>(st.tw) * st.th;
            for (size_t b = 0; b < st.images.size(); ++b) {
                const StagedImage& si = st.images[b];
                k::LetterboxArgs la;
                la.src = st.dev_px + si.offset;
                la.w = si.img.width;
                la.h = si.img.height;
                la.ch = si.img.channels;
                la.dst = dst + b * 3 * plane;
                la.tw = st.tw;
                la.th = st.th;
                la.sw = si.g.scaled_w;
                la.sh = si.g.scaled_h;
                la.px = si.g.pad_x;
                la.py = si.g.pad_y;
                la.inv = 1.0f / si.g.ratio;
                la.scale = st.scale;
                la.pad = st.pad;
                k::launch_letterbox(la, stream_);
            }
            PDEFA_HIP(hipGetLastError());
            continue;
        }
        const HostTensor* t = inputs_[i];
        PDEFA_HIP(hipMemcpyAsync(dst, t->data, t->nbytes, hipMemcpyHostToDevice, stream_));
    }
}

void Session::download_outputs() {
    const Plan& plan = prep_->plan;
    for (size_t i = 0; i < plan.outputs.size(); ++i) {
        const float* src = prep_->arena + plan.bufs.at(plan.outputs[i].buf).offset + plan.outputs[i].off;
        PDEFA_HIP(hipMemcpyAsync(prep_->host_out[i], src, prep_->outputs[i].nbytes, hipMemcpyDeviceToHost, stream_));
    }
}

void Session::run() {
    const auto t0 = std::chrono::high_resolution_clock::now();
    if (!device_available()) throw std::runtime_error("no HIP device available for the session");
    std::vector<std::vector<int64_t>> dims;
    for (size_t i = 0; i < inputs_.size(); ++i) {
        if (i < staged_.size() && !staged_[i].images.empty()) {
            const StagedInput& st = staged_[i];
            dims.push_back({static_cast<int64_t>(st.images.size()), 3, st.th, st.tw});
            continue;
        }
        const HostTensor* t = inputs_[i];
        if (!t) throw std::runtime_error("input " + std::to_string(i) + " is not set");
        if (t->dtype != kF32) throw std::runtime_error("input " + std::to_string(i) + " must be F32");
        dims.emplace_back(t->dims, t->dims + t->rank);
    }
    if (!dev_) dev_ = device_model(*model_);
    if (!stream_) PDEFA_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
    if (!prep_ || prep_->plan.input_dims != dims) prepare(dims);
    const bool per_step = prof_fn_ != nullptr || std::getenv("ENGINE_PROFILE_CSV") != nullptr;
    const bool segmented = use_graph_ && !per_step && !prep_->segments.empty();
    if (!segmented) upload_inputs();  // run_segments uploads (by slices) itself
    if (per_step) {
        std::vector<double> ms;
        std::vector<std::string> labels;
        time_steps(ms, labels);
        if (prof_fn_)
            for (size_t i = 0; i < ms.size(); ++i) prof_fn_(labels[i].c_str(), ms[i], prof_user_);
        if (const char* path = std::getenv("ENGINE_PROFILE_CSV")) {
            if (std::FILE* f = std::fopen(path, "a")) {
                for (size_t i = 0; i < ms.size(); ++i) std::fprintf(f, "%zu,\"%s\",%.6f\n", i, labels[i].c_str(), ms[i]);
                std::fclose(f);
            }
        }
    } else if (segmented) {
        run_segments();
    } else if (use_graph_) {
        if (!prep_->exec) {
            if (concurrent_) {
                PDEFA_HIP(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
                try {
                    capture_concurrent();
                } catch (...) {
                    hipGraph_t g = nullptr;
                    (void)hipStreamEndCapture(stream_, &g);
                    if (g) (void)hipGraphDestroy(g);
                    throw;
                }
                PDEFA_HIP(hipStreamEndCapture(stream_, &prep_->graph));
                PDEFA_HIP(hipGraphInstantiate(&prep_->exec, prep_->graph, nullptr, nullptr, 0));
            } else {
                capture_launches(0, prep_->launches.size() - 1, &prep_->graph, &prep_->exec);
            }
        }
        PDEFA_HIP(hipGraphLaunch(prep_->exec, stream_));
    } else {
        launch_all(stream_);
        PDEFA_HIP(hipGetLastError());
    }
    if (per_step || !use_graph_ || prep_->segments.empty()) {
        download_outputs();
        PDEFA_HIP(hipStreamSynchronize(stream_));
    }
    for (size_t i = 0; i < prep_->outputs.size(); ++i) {
        HostTensor& t = prep_->outputs[i];
        if (t.dtype != kI32) continue;
        // float-valued indices (exact integers) -> int32, in place
        float* f = prep_->host_out[i];
        int32_t* d = reinterpret_cast<int32_t*>(f);
        for (int64_t j = 0; j < t.numel(); ++j) d[j] = static_cast<int32_t>(f[j]);
    }
    const auto t1 = std::chrono::high_resolution_clock::now();
    last_run_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    ++runs;
}

double Session::replay(int32_t iters) {
    if (!prep_ || runs == 0) throw std::runtime_error("replay needs a completed run");
    hipEvent_t a, b;
    PDEFA_HIP(hipEventCreate(&a));
    PDEFA_HIP(hipEventCreate(&b));
    PDEFA_HIP(hipEventRecord(a, stream_));
    if (use_graph_ && !concurrent_ && !prep_->exec)
        capture_launches(0, prep_->launches.size() - 1, &prep_->graph, &prep_->exec);
    for (int32_t i = 0; i < iters; ++i) {
        if (prep_->exec)
            PDEFA_HIP(hipGraphLaunch(prep_->exec, stream_));
        else
            launch_all(stream_);
    }
    PDEFA_HIP(hipEventRecord(b, stream_));
    PDEFA_HIP(hipEventSynchronize(b));
    float ms = 0.0f;
    PDEFA_HIP(hipEventElapsedTime(&ms, a, b));
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return ms;
}

void Session::time_steps(std::vector<double>& ms, std::vector<std::string>& labels) {
    const size_t n = prep_->launches.size();
    std::vector<hipEvent_t> ev(n + 1);
    for (auto& e : ev) PDEFA_HIP(hipEventCreate(&e));
    PDEFA_HIP(hipEventRecord(ev[0], stream_));
    for (size_t i = 0; i < n; ++i) {
        launch_one(prep_->launches[i], stream_);
        PDEFA_HIP(hipEventRecord(ev[i + 1], stream_));
    }
    PDEFA_HIP(hipEventSynchronize(ev[n]));
    ms.assign(n, 0.0);
    labels.clear();
    for (size_t i = 0; i < n; ++i) {
        float t = 0.0f;
        PDEFA_HIP(hipEventElapsedTime(&t, ev[i], ev[i + 1]));
        ms[i] = t;
        labels.push_back(prep_->launches[i].label);
    }
    for (auto& e : ev) (void)hipEventDestroy(e);
}

double Session::repeat_step(int32_t idx, int32_t iters) {
    if (!prep_ || runs == 0) throw std::runtime_error("repeat_step needs a completed run");
    if (idx < 0 || idx >= static_cast<int32_t>(prep_->launches.size()) || iters <= 0)
        throw std::runtime_error("repeat_step: bad step index or count");
    const Launch& l = prep_->launches[static_cast<size_t>(idx)];
    launch_one(l, stream_);  // warm
    hipEvent_t a, b;
    PDEFA_HIP(hipEventCreate(&a));
    PDEFA_HIP(hipEventCreate(&b));
    PDEFA_HIP(hipEventRecord(a, stream_));
    for (int32_t i = 0; i < iters; ++i) launch_one(l, stream_);
    PDEFA_HIP(hipEventRecord(b, stream_));
    PDEFA_HIP(hipEventSynchronize(b));
    float ms = 0.0f;
    PDEFA_HIP(hipEventElapsedTime(&ms, a, b));
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return ms / iters;
}

void Session::step_stats(int32_t iters, std::vector<double>& ms, std::vector<int32_t>& kind,
                         std::vector<int64_t>& flops) {
    if (!prep_ || runs == 0) throw std::runtime_error("step_stats needs a completed run");
    const size_t n = prep_->launches.size();
    ms.assign(n, 0.0);
    std::vector<double> one;
    std::vector<std::string> labels;
    for (int32_t it = 0; it < iters; ++it) {
        time_steps(one, labels);
        for (size_t i = 0; i < n; ++i) ms[i] += one[i] / iters;
    }
    kind.resize(n);
    flops.assign(n, 0);
    for (size_t i = 0; i < n; ++i) {
        const Launch& l = prep_->launches[i];
        kind[i] = static_cast<int32_t>(l.kind);
        if (l.kind == StepKind::ConvMfma) {
            auto conv_flops = [](const k::ConvArgs& c) {
                return 2LL * c.N * c.Cout * c.groups * c.Cin * c.KH * c.KW * static_cast<int64_t>(c.Ho) * c.Wo;
            };
            if (l.group.empty()) flops[i] = conv_flops(l.conv);
            for (const k::ConvArgs& c : l.group) flops[i] += conv_flops(c);
        } else if (l.kind == StepKind::ConvDirect) {
            const k::ConvDirectArgs& d = l.direct;
            flops[i] = 2LL * d.y.dims[0] * d.y.dims[1] * (d.x.dims[1] / d.groups) * d.KH * d.KW * d.y.dims[2] *
                       d.y.dims[3];
        }
    }
}

std::string Session::plan_text() const { return prep_ ? describe_plan(*model_, prep_->plan) : std::string(); }

void Session::read_conv_input(const std::string& node, std::vector<float>& dst, int64_t dims[4]) {
    if (!keep_tensors_) throw std::runtime_error("tensors are not kept: create the session with PDEFA_KEEP_TENSORS=1");
    if (!prep_ || runs == 0) throw std::runtime_error("read_conv_input needs a completed run");
    const Plan& plan = prep_->plan;
    const Step* st = nullptr;
    for (const Step& s : plan.steps)
        if ((s.kind == StepKind::ConvMfma || s.kind == StepKind::ConvDirect) && s.node >= 0 &&
            model_->nodes.at(s.node).name == node)
            st = &s;
    if (!st) throw std::runtime_error("no conv step implements node " + node);
    const VRef& r = st->a;
    if (r.rank != 4 || r.buf < 0) throw std::runtime_error("conv input is not a rank-4 arena view");
    k::View in;
    in.ptr = prep_->arena + plan.bufs.at(r.buf).offset + r.off;
    in.rank = 4;
    k::View out;
    out.rank = 4;
    int64_t n = 1;
    for (int d = 3; d >= 0; --d) {
        in.dims[d] = out.dims[d] = dims[d] = r.dims[d];
        in.str[d] = r.str[d];
        out.str[d] = n;
        n *= r.dims[d];
    }
    float* tmp = nullptr;
    PDEFA_HIP(hipMalloc(&tmp, static_cast<size_t>(std::max<int64_t>(n, 1)) * sizeof(float)));
    out.ptr = tmp;
    try {
        k::launch_eltwise(k::kEltCopy, out, in, in, 0.0f, stream_);
        dst.resize(static_cast<size_t>(n));
        PDEFA_HIP(hipMemcpyAsync(dst.data(), tmp, static_cast<size_t>(n) * sizeof(float), hipMemcpyDeviceToHost,
                                 stream_));
        PDEFA_HIP(hipStreamSynchronize(stream_));
    } catch (...) {
        (void)hipFree(tmp);
        throw;
    }
    PDEFA_HIP(hipFree(tmp));
}

// ------------------------------------------------------------- ops_matmul

namespace {

struct MatmulScratch {
    std::mutex mu;
    hipStream_t stream = nullptr;
    float* buf = nullptr;
    size_t cap = 0;  // floats
    ~MatmulScratch() {
        if (buf) (void)hipFree(buf);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

MatmulScratch& matmul_scratch() {
    static MatmulScratch s;
    return s;
}

// Device buffers of one C = A @ B (floats, each 64-aligned): A, B, B packed
// K-major for the MFMA conv core, a zero bias, C, and the split-K partials.
struct MatmulLayout {
    size_t nA = 0, nB = 0, nP = 0, nBias = 0, nC = 0, nW = 0;
    k::ConvLaunchShape ls;
    size_t total() const { return nA + nB + nP + nBias + nC + nW; }
};

MatmulLayout matmul_layout(int64_t M, int64_t K, int64_t N) {
    if (M >= (int64_t{1} << 31) || K >= (int64_t{1} << 30) || N >= (int64_t{1} << 30))
        throw std::runtime_error("ops_matmul: shape too large");
    MatmulLayout L;
    L.nA = align_up(static_cast<size_t>(M * K));
    L.nB = align_up(static_cast<size_t>(K * N));
    L.nP = align_up(static_cast<size_t>(k::packed_weight_elems(static_cast<int>(N), static_cast<int>(K))));
    L.nBias = align_up(static_cast<size_t>(N));
    L.nC = align_up(static_cast<size_t>(M * N));
    L.ls = k::conv_select(M, static_cast<int>(N), static_cast<int>(K), true);
    L.nW = L.ls.splits > 1 ? align_up(static_cast<size_t>(L.ls.splits) * M * N) : 0;
    return L;
}

// Host A, B in; host C out; the device buffers at `base` (L.total() floats).
void matmul_on(const MatmulLayout& L, float* base, const float* A, const float* B, float* C, int64_t M, int64_t K,
               int64_t N, hipStream_t s) {
    float* dA = base;
    float* dB = dA + L.nA;
    float* dP = dB + L.nB;
    float* dBias = dP + L.nP;
    float* dC = dBias + L.nBias;
    float* dW = dC + L.nC;
    PDEFA_HIP(hipMemcpyAsync(dA, A, sizeof(float) * M * K, hipMemcpyHostToDevice, s));
    PDEFA_HIP(hipMemcpyAsync(dB, B, sizeof(float) * K * N, hipMemcpyHostToDevice, s));
    PDEFA_HIP(hipMemsetAsync(dBias, 0, L.nBias * sizeof(float), s));
    k::launch_pack_gemm_b(dP, dB, static_cast<int>(K), static_cast<int>(N), s);
    k::ConvArgs c;
    c.x = dA;
    c.N = 1;
    c.H = static_cast<int32_t>(M);
    c.W = 1;
    c.Cin = static_cast<int32_t>(K);
    c.x_sn = M * K;
    c.x_sh = K;
    c.x_sw = K;
    c.y = dC;
    c.Ho = static_cast<int32_t>(M);
    c.Wo = 1;
    c.Cout = static_cast<int32_t>(N);
    c.y_sn = M * N;
    c.y_sh = N;
    c.y_sw = N;
    c.wpk = dP;
    c.bias = dBias;
    c.K = static_cast<int32_t>(K);
    c.ktiles = static_cast<int>((K + k::kConvBK - 1) / k::kConvBK);
    c.splits = L.ls.splits;
    c.kt_per_split = L.ls.kt_per_split;
    c.ws = L.ls.splits > 1 ? dW : nullptr;
    k::launch_conv_mfma(c, L.ls.tile, K % 4 == 0, s);
    PDEFA_HIP(hipGetLastError());
    PDEFA_HIP(hipMemcpyAsync(C, dC, sizeof(float) * M * N, hipMemcpyDeviceToHost, s));
    PDEFA_HIP(hipStreamSynchronize(s));
}

}  // namespace

void device_matmul(const float* A, const float* B, float* C, int64_t M, int64_t K, int64_t N) {
    if (!device_available()) throw std::runtime_error("no HIP device available for ops_matmul");
    if (M <= 0 || K <= 0 || N <= 0) return;
    const MatmulLayout L = matmul_layout(M, K, N);
    MatmulScratch& sc = matmul_scratch();
    std::lock_guard<std::mutex> g(sc.mu);
    if (!sc.stream) PDEFA_HIP(hipStreamCreateWithFlags(&sc.stream, hipStreamNonBlocking));
    if (L.total() > sc.cap) {
        if (sc.buf) PDEFA_HIP(hipFree(sc.buf));
        sc.buf = nullptr;
        sc.cap = 0;
        PDEFA_HIP(hipMalloc(&sc.buf, L.total() * sizeof(float)));
        sc.cap = L.total();
    }
    matmul_on(L, sc.buf, A, B, C, M, K, N, sc.stream);
}

void device_matmul_noalloc(const float* A, const float* B, float* C, int64_t M, int64_t K, int64_t N) {
    if (!device_available()) throw std::runtime_error("no HIP device available for ops_matmul");
    if (M <= 0 || K <= 0 || N <= 0) return;
    const MatmulLayout L = matmul_layout(M, K, N);
    static std::mutex mu;  // calls share this device's scratch array: one at a time
    std::lock_guard<std::mutex> g(mu);
    size_t cap = 0;
    float* base = noalloc_scratch(cap);
    if (L.total() > cap) {
        std::ostringstream os;
        os << "ops_matmul_noalloc: a " << M << "x" << K << " @ " << K << "x" << N << " product needs "
           << L.total() * sizeof(float) << " bytes of device scratch, more than the " << cap * sizeof(float)
           << " bytes of the static scratch array";
        throw std::invalid_argument(os.str());
    }
    // the null stream: nothing is created
    matmul_on(L, base, A, B, C, M, K, N, nullptr);
}

}  // namespace pdefa
