#include "conv_tune.hpp"

#include <dlfcn.h>

#include <algorithm>
#include <array>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <stdexcept>
#include <string>

#include "runtime.hpp"

namespace pdefa {

namespace {

constexpr size_t kMaxCandidates = 12;          // the cost model's best ones are timed
constexpr int64_t kMaxWorkspaceBytes = 256LL << 20;  // split-K partials of one candidate
constexpr double kKeepModelChoice = 0.97;      // another shape must beat the model's by 3%
constexpr int kTimingPasses = 2;                // timing passes over the candidates

constexpr size_t kKeyInts = 21;  // device, then the 20 shape fields of a ConvQuery
using Key = std::array<int32_t, kKeyInts>;

using GroupKey = std::vector<int32_t>;

std::mutex g_mu;
std::map<Key, k::ConvLaunchShape> g_cache;
std::map<GroupKey, ConvGroupTiming> g_group_cache;
size_t g_measured = 0, g_from_table = 0;

Key make_key(const ConvQuery& q, int device) {
    return {device, q.N,  q.H,  q.W,  q.Cin, q.Ho, q.Wo, q.Cout, q.KH, q.KW, q.sh,
            q.sw,   q.ph, q.pw, q.dh, q.dw,  q.act, q.has_res ? 1 : 0, q.vec ? 1 : 0, q.wino ? 1 : 0, q.groups};
}

// ---- persisted choices
//
// A launch-shape table holds measured choices for one kind of device (its
// architecture name and compute-unit count), so that a process plans the
// same launch shapes as the one that measured them, without timing:
//
//   device gfx950 256
//   conv <20 shape ints> <tile> <splits> <k steps per split>
//   group <members> {<20 shape ints> <tile> <splits> <k steps per split>}... <tile> <group ms> <separate ms>
//
// The table is read from PDEFA_TUNE_TABLE, or by default from
// tuning/<arch>.txt beside the library's directory, when a plan first needs
// it and again whenever PDEFA_TUNE_TABLE names another file;
// PDEFA_TUNE_TABLE=0 disables it.  With PDEFA_TUNE_RECORD=<file> every choice measured in this
// process is appended to that file in the same format.

struct Table {
    bool loaded = false;
    std::string path;  // the file it was read from
    std::string arch;
    int cus = 0;
    std::map<std::vector<int32_t>, k::ConvLaunchShape> conv;  // shape ints (no device)
    std::map<std::vector<int32_t>, ConvGroupTiming> group;     // members' ints (no device)
};
std::map<int, Table> g_tables;  // per device

void device_kind(int device, std::string& arch, int& cus) {
    hipDeviceProp_t p;
    PDEFA_HIP(hipGetDeviceProperties(&p, device));
    arch = p.gcnArchName;
    arch = arch.substr(0, arch.find(':'));
    cus = p.multiProcessorCount;
}

std::string default_table_path(const std::string& arch) {
    Dl_info info;
    if (!dladdr(reinterpret_cast<void*>(&tune_conv), &info) || !info.dli_fname) return {};
    std::string lib = info.dli_fname;
    const size_t slash = lib.rfind('/');
    const std::string dir = slash == std::string::npos ? std::string(".") : lib.substr(0, slash);
    return dir + "/../tuning/" + arch + ".txt";
}

std::vector<int32_t> shape_ints(const Key& k) { return std::vector<int32_t>(k.begin() + 1, k.end()); }

Table& table_for(int device) {
    Table& t = g_tables[device];
    const char* env = std::getenv("PDEFA_TUNE_TABLE");
    if (t.loaded && env && t.path != env) {
        // PDEFA_TUNE_TABLE names another file now: drop the old table and the
        // choices this process took from it (or measured beside it)
        t.conv.clear();
        t.group.clear();
        t.loaded = false;
        g_cache.clear();
        g_group_cache.clear();
    }
    if (t.loaded) return t;
    t.loaded = true;
    device_kind(device, t.arch, t.cus);
    std::string path = env ? std::string(env) : default_table_path(t.arch);
    t.path = path;
    if (path.empty() || path == "0") return t;
    std::ifstream f(path);
    if (!f) return t;
    std::string line, tag;
    bool match = false;
    while (std::getline(f, line)) {
        std::istringstream is(line);
        if (!(is >> tag) || tag[0] == '#') continue;
        if (tag == "device") {
            std::string arch;
            int cus = 0;
            is >> arch >> cus;
            match = arch == t.arch && cus == t.cus;
            continue;
        }
        if (!match) continue;
        if (tag == "conv") {
            std::vector<int32_t> key(kKeyInts - 1);
            k::ConvLaunchShape ls{};
            for (auto& v : key) is >> v;
            is >> ls.tile >> ls.splits >> ls.kt_per_split;
            if (is && ls.tile >= 0 && ls.tile < k::kNumConvShapes && ls.splits >= 1) t.conv[key] = ls;
        } else if (tag == "group") {
            int n = 0;
            is >> n;
            if (n < 2 || n > k::kMaxConvGroup) continue;
            std::vector<int32_t> key(static_cast<size_t>(n) * (kKeyInts - 1 + 3));
            for (auto& v : key) is >> v;
            ConvGroupTiming g;
            is >> g.tile >> g.group_ms >> g.separate_ms;
            if (is && k::is_gemm_tile(g.tile)) t.group[key] = g;
        }
    }
    return t;
}

void record_line(const Table& t, const std::string& body) {
    const char* path = std::getenv("PDEFA_TUNE_RECORD");
    if (!path || !*path) return;
    if (std::FILE* f = std::fopen(path, "a")) {
        std::fprintf(f, "device %s %d\n%s\n", t.arch.c_str(), t.cus, body.c_str());
        std::fclose(f);
    }
}

std::string ints_text(const std::vector<int32_t>& v) {
    std::ostringstream os;
    for (size_t i = 0; i < v.size(); ++i) os << (i ? " " : "") << v[i];
    return os.str();
}

struct DeviceBuffer {
    float* p = nullptr;
    explicit DeviceBuffer(int64_t elems) { PDEFA_HIP(hipMalloc(&p, static_cast<size_t>(std::max<int64_t>(elems, 1)) * 4)); }
    ~DeviceBuffer() {
        if (p) (void)hipFree(p);
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
};

struct Events {
    hipEvent_t a = nullptr, b = nullptr;
    Events() {
        PDEFA_HIP(hipEventCreate(&a));
        PDEFA_HIP(hipEventCreate(&b));
    }
    ~Events() {
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
    }
};

void launch(const k::ConvArgs& a, int tile, bool vec, hipStream_t s) {
    if (k::is_wino_tile(tile))
        k::launch_conv_wino(a, tile == k::kTileWino64 ? 64 : 32, s);
    else
        k::launch_conv_mfma(a, tile, vec, s);
}

// Dense channels-last scratch tensors of one layer's shape; values do not
// affect timing (zeros).  The residual, when the layer has one, reads the
// output tensor itself: each element is read and then written by the same
// lane.
struct LayerScratch {
    int64_t x_elems, out_elems, w_group, w_elems;
    DeviceBuffer x, y, w, bias, ws;
    k::ConvArgs a;
    LayerScratch(const ConvQuery& q, int max_splits, hipStream_t s)
        : x_elems(static_cast<int64_t>(q.N) * q.H * q.W * q.Cin),
          out_elems(static_cast<int64_t>(q.N) * q.Ho * q.Wo * q.Cout),
          w_group(k::packed_weight_elems(q.Cout / q.groups, q.KH * q.KW * (q.Cin / q.groups))),
          w_elems(std::max(w_group * q.groups, q.wino ? k::wino_packed_elems(q.Cout, q.Cin) : int64_t{0})),
          x(x_elems),
          y(out_elems),
          w(w_elems),
          bias(q.Cout),
          ws(max_splits > 1 ? static_cast<int64_t>(max_splits) * out_elems : 1) {
        PDEFA_HIP(hipMemsetAsync(x.p, 0, static_cast<size_t>(x_elems) * 4, s));
        PDEFA_HIP(hipMemsetAsync(w.p, 0, static_cast<size_t>(w_elems) * 4, s));
        PDEFA_HIP(hipMemsetAsync(bias.p, 0, static_cast<size_t>(q.Cout) * 4, s));
        PDEFA_HIP(hipMemsetAsync(y.p, 0, static_cast<size_t>(out_elems) * 4, s));
        const int K = q.KH * q.KW * (q.Cin / q.groups);
        a.x = x.p;
        a.N = q.N;
        a.H = q.H;
        a.W = q.W;
        a.Cin = q.Cin / q.groups;
        a.groups = q.groups;
        a.w_group = w_group;
        a.x_sw = q.Cin;
        a.x_sh = static_cast<int64_t>(q.W) * q.Cin;
        a.x_sn = static_cast<int64_t>(q.H) * q.W * q.Cin;
        a.y = y.p;
        a.Ho = q.Ho;
        a.Wo = q.Wo;
        a.Cout = q.Cout / q.groups;
        a.y_sw = q.Cout;
        a.y_sh = static_cast<int64_t>(q.Wo) * q.Cout;
        a.y_sn = static_cast<int64_t>(q.Ho) * q.Wo * q.Cout;
        if (q.has_res) {
            a.res = y.p;
            a.r_sw = a.y_sw;
            a.r_sh = a.y_sh;
            a.r_sn = a.y_sn;
        }
        a.wpk = w.p;
        a.bias = bias.p;
        a.KH = q.KH;
        a.KW = q.KW;
        a.sh = q.sh;
        a.sw = q.sw;
        a.ph = q.ph;
        a.pw = q.pw;
        a.dh = q.dh;
        a.dw = q.dw;
        a.K = K;
        a.ktiles = (K + k::kConvBK - 1) / k::kConvBK;
        a.act = q.act;
        a.ws = ws.p;
    }
    void shape(const k::ConvLaunchShape& ls) {
        a.splits = ls.splits;
        a.kt_per_split = ls.kt_per_split;
    }
};

// Average ms per repetition of `body` (after one untimed call).
template <typename F>
double time_reps(F&& body, hipStream_t s, Events& ev, int reps) {
    body();
    PDEFA_HIP(hipEventRecord(ev.a, s));
    for (int i = 0; i < reps; ++i) body();
    PDEFA_HIP(hipEventRecord(ev.b, s));
    PDEFA_HIP(hipEventSynchronize(ev.b));
    float ms = 0.0f;
    PDEFA_HIP(hipEventElapsedTime(&ms, ev.a, ev.b));
    return static_cast<double>(ms) / reps;
}

// Repetitions for about 100 us of timed work, at least 3.
int reps_for(double first_ms) { return std::max(3, std::min(20, static_cast<int>(0.1 / std::max(first_ms, 1e-3)))); }

}  // namespace

k::ConvLaunchShape tune_conv(const ConvQuery& q, hipStream_t s) {
    int device = 0;
    PDEFA_HIP(hipGetDevice(&device));
    const Key key = make_key(q, device);
    std::lock_guard<std::mutex> lock(g_mu);
    Table& table = table_for(device);
    if (auto it = g_cache.find(key); it != g_cache.end()) return it->second;
    if (auto it = table.conv.find(shape_ints(key)); it != table.conv.end()) {
        ++g_from_table;
        g_cache.emplace(key, it->second);
        return it->second;
    }

    const int64_t M = static_cast<int64_t>(q.N) * q.Ho * q.Wo;
    const int K = q.KH * q.KW * (q.Cin / q.groups);  // per group
    std::vector<k::ConvLaunchShape> all =
        k::conv_candidates(M * q.groups, q.Cout / q.groups, K, true, q.wino, q.Cin);
    // the cost model's best implicit-GEMM shapes, plus every Winograd shape
    std::vector<k::ConvLaunchShape> cands;
    for (const auto& c : all)
        if (k::is_wino_tile(c.tile) || cands.size() < kMaxCandidates) cands.push_back(c);
    const int64_t out_elems = M * q.Cout;
    int max_splits = 1;
    std::vector<k::ConvLaunchShape> usable;
    for (const auto& c : cands) {
        if (c.splits > 1 && static_cast<int64_t>(c.splits) * out_elems * 4 > kMaxWorkspaceBytes) continue;
        usable.push_back(c);
        max_splits = std::max(max_splits, c.splits);
    }
    k::ConvLaunchShape best = cands.front();
    if (usable.size() > 1) {
        LayerScratch L(q, max_splits, s);
        Events ev;
        L.shape(usable.front());
        const double first = time_reps([&] { launch(L.a, usable.front().tile, q.vec, s); }, s, ev, 1);
        const int reps = reps_for(first);
        // two interleaved passes over the candidates, each scored by its
        // faster pass: a candidate is not lost to one slow measurement
        std::vector<double> ms(usable.size(), 0.0);
        for (int pass = 0; pass < kTimingPasses; ++pass)
            for (size_t i = 0; i < usable.size(); ++i) {
                L.shape(usable[i]);
                const double t = time_reps([&] { launch(L.a, usable[i].tile, q.vec, s); }, s, ev, reps);
                ms[i] = pass == 0 ? t : std::min(ms[i], t);
            }
        double best_ms = 0.0;
        for (size_t i = 0; i < usable.size(); ++i)
            if (i == 0 || ms[i] < best_ms * kKeepModelChoice) {
                best_ms = ms[i];
                best = usable[i];
            }
        PDEFA_HIP(hipStreamSynchronize(s));
    }
    ++g_measured;
    g_cache.emplace(key, best);
    record_line(table, "conv " + ints_text(shape_ints(key)) + " " + std::to_string(best.tile) + " " +
                           std::to_string(best.splits) + " " + std::to_string(best.kt_per_split));
    return best;
}

ConvGroupTiming tune_conv_group(const std::vector<ConvQuery>& qs, const std::vector<k::ConvLaunchShape>& solo,
                                hipStream_t s) {
    if (qs.size() != solo.size() || qs.size() < 2 || qs.size() > static_cast<size_t>(k::kMaxConvGroup))
        throw std::runtime_error("tune_conv_group: bad group");
    int device = 0;
    PDEFA_HIP(hipGetDevice(&device));
    GroupKey key;  // device, then per member its shape ints and solo launch shape
    key.push_back(device);
    for (size_t i = 0; i < qs.size(); ++i) {
        const Key k1 = make_key(qs[i], device);
        key.insert(key.end(), k1.begin() + 1, k1.end());
        key.push_back(solo[i].tile);
        key.push_back(solo[i].splits);
        key.push_back(solo[i].kt_per_split);
    }
    std::lock_guard<std::mutex> lock(g_mu);
    Table& table = table_for(device);
    if (auto it = g_group_cache.find(key); it != g_group_cache.end()) return it->second;
    const std::vector<int32_t> tkey(key.begin() + 1, key.end());
    if (auto it = table.group.find(tkey); it != table.group.end()) {
        ++g_from_table;
        g_group_cache.emplace(key, it->second);
        return it->second;
    }

    std::vector<std::unique_ptr<LayerScratch>> L;
    for (size_t i = 0; i < qs.size(); ++i) {
        if (!qs[i].vec) throw std::runtime_error("tune_conv_group: grouped layers need vector loads");
        L.push_back(std::make_unique<LayerScratch>(qs[i], solo[i].splits, s));
        L.back()->shape(solo[i]);
    }
    Events ev;
    auto separate = [&] {
        for (size_t i = 0; i < qs.size(); ++i) launch(L[i]->a, solo[i].tile, qs[i].vec, s);
    };
    ConvGroupTiming r;
    const int reps = reps_for(time_reps(separate, s, ev, 1));
    std::vector<k::ConvArgs> probs(qs.size());
    auto group_args = [&](int t) {
        const int kg = k::conv_tile_shape(t).kg;
        for (size_t i = 0; i < qs.size(); ++i) {
            probs[i] = L[i]->a;
            probs[i].splits = 1;
            probs[i].kt_per_split = (probs[i].ktiles + kg - 1) / kg * kg;
        }
    };
    // interleaved passes as in tune_conv, each time scored by its faster pass
    std::vector<double> ms(k::kNumConvShapes, 0.0);
    for (int pass = 0; pass < kTimingPasses; ++pass) {
        const double sep = time_reps(separate, s, ev, reps);
        r.separate_ms = pass == 0 ? sep : std::min(r.separate_ms, sep);
        for (int t = 0; t < k::kNumConvShapes; ++t) {
            if (!k::is_gemm_tile(t)) continue;
            group_args(t);
            const double g = time_reps(
                [&] { k::launch_conv_mfma_group(probs.data(), static_cast<int>(probs.size()), t, s); }, s, ev, reps);
            ms[t] = pass == 0 ? g : std::min(ms[t], g);
        }
    }
    for (int t = 0; t < k::kNumConvShapes; ++t)
        if (k::is_gemm_tile(t) && (r.tile < 0 || ms[t] < r.group_ms)) {
            r.tile = t;
            r.group_ms = ms[t];
        }
    PDEFA_HIP(hipStreamSynchronize(s));
    ++g_measured;
    g_group_cache.emplace(std::move(key), r);
    char times[64];
    std::snprintf(times, sizeof(times), " %d %.17g %.17g", r.tile, r.group_ms, r.separate_ms);
    record_line(table, "group " + std::to_string(qs.size()) + " " + ints_text(tkey) + times);
    return r;
}

size_t conv_tune_cache_size() {
    std::lock_guard<std::mutex> lock(g_mu);
    return g_cache.size();
}

void conv_tune_stats(size_t& measured, size_t& from_table) {
    std::lock_guard<std::mutex> lock(g_mu);
    measured = g_measured;
    from_table = g_from_table;
}

}  // namespace pdefa
