// Device runtime: model weights resident in HBM (uploaded once, conv weights
// pre-packed for the MFMA kernel) and the per-session executor that runs a
// planned program on its own HIP stream, captured once as a hipGraph and
// replayed on every run.
#pragma once

#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "host_tensor.hpp"
#include "kernels.hpp"
#include "letterbox.hpp"
#include "model.hpp"
#include "planner.hpp"

namespace pdefa {

struct HipError : std::runtime_error {
    hipError_t code;
    HipError(hipError_t c, const std::string& what) : std::runtime_error(what), code(c) {}
};

void hip_check(hipError_t e, const char* expr, const char* file, int line);
#define PDEFA_HIP(expr) ::pdefa::hip_check((expr), #expr, __FILE__, __LINE__)

// True when a HIP device is present (counts devices without creating a context).
bool device_available();

struct DeviceModel {
    int device = 0;
    float* blob = nullptr;  // one allocation: raw weights, packed conv weights, padded biases
    size_t blob_bytes = 0;
    std::vector<float*> wptr;  // raw weight i
    struct Pack {
        float* wpk = nullptr;
        float* bias = nullptr;  // Cout floats, zeros when the conv has no bias
        float* dpk = nullptr;   // direct-conv layout (k::direct_packed_elems)
        float* wino = nullptr;  // Winograd-transformed weights (3x3 stride-1 convs only)
        int groups = 1;         // wpk holds one packed block per group; dpk the grouped layout
    };
    std::vector<Pack> packs;  // by node index (empty for non-conv nodes)
    bool packs_from_cache = false;  // the packed layouts came from the pre-pack cache file
    ~DeviceModel();
};

// Uploads and packs on the current device (throws on HIP errors).  With
// PDEFA_PACK_CACHE=1 in the environment and a model read from a file, the
// packed layouts are read from the pre-pack cache file next to it
// ("<engine>.<gfx arch>.pack") when that file matches the weights, the
// layout and the device architecture, and written there after packing on
// the device otherwise.
std::shared_ptr<DeviceModel> upload_model(const Model& m);

// Pre-pack cache files read and written by this process.
void pack_cache_stats(int64_t& read, int64_t& written);
std::shared_ptr<DeviceModel> device_model(Model& m);  // lazily, once per model

class Session {
   public:
    using ProfileFn = void (*)(const char*, double, void*);

    explicit Session(Model& m);
    ~Session();
    Session(const Session&) = delete;
    Session& operator=(const Session&) = delete;

    int32_t num_inputs() const { return model_->num_inputs(); }
    int32_t num_outputs() const { return model_->num_outputs(); }
    void set_input(int32_t idx, const HostTensor* t);
    // Input `idx` becomes the letterbox of `images` (batch = images.size(),
    // planar fp32 [n, 3, th, tw]) computed on the device at the next run: the
    // 8-bit pixels are copied now into pinned staging memory (the caller may
    // release them), uploaded and letterboxed on the session stream before
    // the program.  Returns each image's geometry.  set_input(idx, ...)
    // replaces it.
    std::vector<LetterboxGeometry> set_images(int32_t idx, const std::vector<ImageRef>& images, int32_t tw,
                                              int32_t th, float scale, float pad);
    void run();  // throws
    const HostTensor* output(int32_t idx) const;
    // YOLO decode + per-class NMS of output `idx` (a [N, 4 + classes, A] head
    // resident from the last run) on the device; metas: 5 doubles per image
    // (ratio, pad_x, pad_y, orig_w, orig_h) or empty for no letterbox
    // mapping.  Returns each image's detections in the reference's order.
    std::vector<std::vector<k::YoloDetection>> decode(int32_t idx, const std::vector<double>& metas, double conf,
                                                      double iou, int32_t max_det);

    // Re-runs the prepared program `iters` times on the input already in HBM
    // (no host copies); returns the elapsed device time in ms (HIP events).
    double replay(int32_t iters);
    // Launches are the plan's steps, except that a grouped launch issues
    // several conv steps at once.
    // Runs each launch once with HIP events around it; fills per-launch ms.
    void time_steps(std::vector<double>& ms, std::vector<std::string>& labels);
    // Issues launch `idx` `iters` times back to back between two HIP events
    // on the session stream; returns the average ms per launch.
    double repeat_step(int32_t idx, int32_t iters);
    // Average per-launch device time over `iters` launch-by-launch replays,
    // with the kind and the algorithmic flops (2*N*Cout*Cin*KH*KW*Ho*Wo summed
    // over the launch's convs).
    void step_stats(int32_t iters, std::vector<double>& ms, std::vector<int32_t>& kind,
                    std::vector<int64_t>& flops);

    void set_profile(ProfileFn fn, void* user) {
        prof_fn_ = fn;
        prof_user_ = user;
    }
    double last_run_ms = 0.0;
    uint64_t runs = 0;
    std::string plan_text() const;
    const Plan* plan() const { return prep_ ? &prep_->plan : nullptr; }
    // With PDEFA_KEEP_TENSORS=1 at creation every tensor keeps its own arena
    // memory (the program and its launch shapes are unchanged): after a run,
    // the logical [N, C, H, W] input of the conv step implementing graph node
    // `node` is copied into `dst` (contiguous, N*C*H*W floats); dims receives
    // N, C, H, W.  Throws when tensors are not kept or no conv step
    // implements the node.
    void read_conv_input(const std::string& node, std::vector<float>& dst, int64_t dims[4]);

   private:
    struct Launch {
        StepKind kind;
        k::ConvArgs conv;
        std::vector<k::ConvArgs> group;  // grouped launch: every member (conv is the first)
        int tile = 0;
        bool vec = false;
        k::ConvDirectArgs direct;
        k::View out, a, b, c;
        k::DetectDecodeArgs decode;
        int elt = 0;
        float alpha = 0.0f;
        int kh = 0, kw = 0, sh = 1, sw = 1, ph = 0, pw = 0, axis = 0;
        int64_t topk = 0;
        bool topk_indices = false;
        std::string label;
        int step = -1;  // the plan step it issues (the first of a grouped launch)
    };
    // A rectangle of an output copied to the host: `rows` rows of `width`
    // floats, `pitch` floats apart, at element offset dev (arena) / host
    // (the output's pinned buffer).
    struct Region {
        size_t out = 0;
        int64_t dev = 0, host = 0, width = 0, rows = 0, pitch = 0;
    };
    // A piece of the program cut after a decode part: its launches run as
    // one graph, then the outputs that part finished go down on copy_out_
    // while the next pieces run.
    struct Segment {
        size_t first = 0, last = 0;  // launches [first, last]
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        hipEvent_t done = nullptr;
        std::vector<Region> regions;
    };
    struct Prepared {
        Plan plan;
        float* arena = nullptr;
        std::vector<Launch> launches;
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        Schedule sched;                  // concurrent issue order of the captured graph
        std::vector<hipEvent_t> events;  // per step (recorded ones only) + per extra stream join
        std::vector<float*> host_out;  // pinned
        std::vector<HostTensor> outputs;
        // Runs cut after the decode parts of a split Detect head (empty: the
        // whole program is one graph): out_split[i] marks outputs whose
        // download is the segments' regions.
        std::vector<Segment> segments;
        std::vector<char> out_split;
        // Batch chunks of the early steps (Plan::early_steps): chunk c runs
        // launches [0, early_launches) on images [first, first + n) once its
        // slice of the input has landed, while later slices still upload.
        struct InChunk {
            int64_t first = 0, n = 0;
            std::vector<Launch> launches;
            hipGraph_t graph = nullptr;
            hipGraphExec_t exec = nullptr;
            hipEvent_t ready = nullptr;  // its input slice uploaded
        };
        std::vector<InChunk> in_chunks;
        size_t early_launches = 0;
        ~Prepared();
    };

    void prepare(const std::vector<std::vector<int64_t>>& dims);
    void release_prepared();
    void launch_all(hipStream_t s);
    // records launches [first, last] as a graph on the session stream
    void capture_launches(size_t first, size_t last, hipGraph_t* graph, hipGraphExec_t* exec);
    void capture_list(const std::vector<Launch>& ls, hipGraph_t* graph, hipGraphExec_t* exec);
    void plan_input_chunks();  // fills prep_->in_chunks (or leaves them empty)
    void plan_segments();  // fills prep_->segments (or leaves them empty)
    void run_segments();   // one run through the segments, downloads included
    void capture_concurrent();  // records the program as a multi-stream hipGraph
    void launch_one(const Launch& l, hipStream_t s);
    void upload_inputs();
    void download_outputs();

    // Device letterbox input (set_images): pinned copy of the pixels, the
    // device buffer they are uploaded to, and per image its geometry.
    struct StagedImage {
        size_t offset = 0;
        ImageRef img;  // pixels unused (they live in the input's host_px at offset)
        LetterboxGeometry g;
    };
    // Each input has its own staging buffers (grow-only), so that images
    // staged for one input never overwrite another's.
    struct StagedInput {
        std::vector<StagedImage> images;
        int32_t tw = 0, th = 0;
        float scale = 1.0f, pad = 0.0f;
        uint8_t* host_px = nullptr;  // pinned
        size_t host_cap = 0;
        uint8_t* dev_px = nullptr;
        size_t dev_cap = 0;
    };
    std::vector<StagedInput> staged_;  // per input; empty images = host tensor input
    bool has_staged() const {
        for (const StagedInput& st : staged_)
            if (!st.images.empty()) return true;
        return false;
    }
    // decode workspace (device, grow-only) and its pinned result staging
    void* dec_ws_ = nullptr;
    size_t dec_ws_bytes_ = 0;
    void* dec_host_ = nullptr;
    size_t dec_host_bytes_ = 0;

    Model* model_;
    std::shared_ptr<DeviceModel> dev_;
    hipStream_t stream_ = nullptr;
    std::vector<hipStream_t> side_streams_;  // capture-only streams for concurrent branches
    hipStream_t copy_out_ = nullptr;         // downloads that overlap the program's later segments
    hipStream_t copy_in_ = nullptr;          // input slices uploaded while earlier chunks compute
    int input_chunks_ = 2;                   // PDEFA_INPUT_CHUNKS (<= 1: the input goes up whole)
    int64_t early_hw_ = 80 * 80;             // PDEFA_EARLY_HW: smallest map the early steps produce
    bool concurrent_ = true;
    std::vector<const HostTensor*> inputs_;
    std::unique_ptr<Prepared> prep_;
    ProfileFn prof_fn_ = nullptr;
    void* prof_user_ = nullptr;
    bool use_graph_ = true;
    bool keep_tensors_ = false;  // PDEFA_KEEP_TENSORS=1: no arena reuse (read_conv_input)
    PlanOptions opts_;
    bool autotune_ = true;  // time candidate conv launch shapes while planning
    bool group_convs_ = true;  // grouped launches of independent convs (measured)
    int group_tile_ = -1;      // >= 0: every offered group is taken with this tile
};

// C = A[M,K] @ B[K,N] on the device (the ops_matmul path); host pointers.
void device_matmul(const float* A, const float* B, float* C, int64_t M, int64_t K, int64_t N);

// The same product with its device buffers (A, B, packed B, bias, C, split-K
// partials) in the static scratch array instead of allocated memory; throws
// std::invalid_argument when they do not fit it.  Calls in one process are
// serialized (they share the array).
void device_matmul_noalloc(const float* A, const float* B, float* C, int64_t M, int64_t K, int64_t N);

// Address of the current device's static scratch array (kernels/noalloc.hip)
// and its size in floats; looked up once per device.
float* noalloc_scratch(size_t& floats);

}  // namespace pdefa
