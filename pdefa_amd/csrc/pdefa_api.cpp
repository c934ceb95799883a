// pdefa_* C ABI (image / letterbox / box mapping) plus the pdefa_amd_*
// extensions used by the benchmark and the tests.  Image decoding is not part
// of the GPU hot path: binary PPM/PGM are read here; PNG/JPEG are reported as
// unsupported.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "letterbox.hpp"
#include "../../include/pdefa_amd_ext.h"
#include "conv_tune.hpp"
#include "../../include/pdefa_c_api.h"
#include "api_internal.hpp"

using pdefa::HostTensor;
using pdefa::api::clear_error;
using pdefa::api::guarded;
using pdefa::api::set_error;

struct PdefaImage {
    int32_t width = 0, height = 0, channels = 0;
    std::vector<uint8_t> pixels;  // row-major, interleaved
};

namespace {

bool read_token(std::istream& in, std::string& tok) {
    tok.clear();
    char c;
    while (in.get(c)) {
        if (c == '#') {
            std::string skip;
            std::getline(in, skip);
            continue;
        }
        if (std::isspace(static_cast<unsigned char>(c))) {
            if (!tok.empty()) return true;
            continue;
        }
        tok.push_back(c);
    }
    return !tok.empty();
}

// Binary PPM (P6, RGB8) and PGM (P5, GRAY8), maxval <= 255.
std::unique_ptr<PdefaImage> load_pnm(const std::string& path, std::string* why) {
    std::ifstream in(path, std::ios::binary);
    if (!in) {
        *why = "cannot open image file";
        return nullptr;
    }
    std::string magic, w, h, mx;
    if (!read_token(in, magic) || (magic != "P6" && magic != "P5")) {
        *why = "unsupported image format (binary PPM/PGM only; PNG/JPEG decoding is not built in)";
        return nullptr;
    }
    if (!read_token(in, w) || !read_token(in, h) || !read_token(in, mx)) {
        *why = "truncated PNM header";
        return nullptr;
    }
    auto img = std::make_unique<PdefaImage>();
    img->width = std::atoi(w.c_str());
    img->height = std::atoi(h.c_str());
    img->channels = magic == "P6" ? 3 : 1;
    if (img->width <= 0 || img->height <= 0 || std::atoi(mx.c_str()) > 255) {
        *why = "unsupported PNM dimensions or depth";
        return nullptr;
    }
    img->pixels.resize(static_cast<size_t>(img->width) * img->height * img->channels);
    in.read(reinterpret_cast<char*>(img->pixels.data()), static_cast<std::streamsize>(img->pixels.size()));
    if (static_cast<size_t>(in.gcount()) != img->pixels.size()) {
        *why = "truncated PNM pixel data";
        return nullptr;
    }
    return img;
}

// Letterbox restated from imageloader/src/preprocess.cpp:15-144: ratio =
// min(tw/w, th/h); scaled = clamp(round(src*ratio), 1, target); centred
// integer pads; source x = dx/ratio truncated, x0 clamped to w-2; bilinear
// with the scale folded into the row weights (letterbox_blend); pad value
// written raw; NCHW.
void letterbox(const PdefaImage& img, int tw, int th, float scale, float pad, float* out, PdefaPreprocessMeta* m) {
    const int sw_src = img.width, sh_src = img.height, ch = img.channels;
    const pdefa::LetterboxGeometry g = pdefa::letterbox_geometry(sw_src, sh_src, tw, th);
    const float ratio = g.ratio;
    const int sw = g.scaled_w, sh = g.scaled_h, px = g.pad_x, py = g.pad_y;
    const size_t plane = static_cast<size_t>(tw) * th;
    std::fill(out, out + 3 * plane, pad);
    const float inv = 1.0f / ratio;
    std::vector<int> x0v(sw), x1v(sw);
    std::vector<float> fxv(sw);
    for (int dx = 0; dx < sw; ++dx) {
        const float sx = dx * inv;
        int x0 = static_cast<int>(sx);
        if (x0 > sw_src - 2 && sw_src > 1) x0 = sw_src - 2;
        x0v[dx] = x0;
        x1v[dx] = x0 + 1 < sw_src ? x0 + 1 : x0;
        fxv[dx] = sx - x0;
    }
    const uint8_t* src = img.pixels.data();
    for (int dy = 0; dy < sh; ++dy) {
        const float sy = dy * inv;
        int y0 = static_cast<int>(sy);
        if (y0 > sh_src - 2 && sh_src > 1) y0 = sh_src - 2;
        const int y1 = y0 + 1 < sh_src ? y0 + 1 : y0;
        const float fy = sy - y0;
        const float wy0 = (1.0f - fy) * scale, wy1 = fy * scale;
        const uint8_t* r0 = src + static_cast<size_t>(y0) * sw_src * ch;
        const uint8_t* r1 = src + static_cast<size_t>(y1) * sw_src * ch;
        const size_t row = static_cast<size_t>(dy + py) * tw + px;
        for (int dx = 0; dx < sw; ++dx) {
            const int a = x0v[dx], b = x1v[dx];
            const float w1 = fxv[dx], w0 = 1.0f - w1;
            for (int c = 0; c < 3; ++c) {
                const int sc = ch == 1 ? 0 : c;
                out[c * plane + row + dx] =
                    pdefa::letterbox_blend(r0[a * ch + sc], r0[b * ch + sc], r1[a * ch + sc], r1[b * ch + sc], w0, w1,
                                           wy0, wy1);
            }
        }
    }
    if (m) {
        m->target_w = tw;
        m->target_h = th;
        m->orig_w = sw_src;
        m->orig_h = sh_src;
        m->pad_x = px;
        m->pad_y = py;
        m->scaled_w = sw;
        m->scaled_h = sh;
        m->ratio = ratio;
    }
}

EngineStatus letterbox_tensor(const PdefaImage& img, int tw, int th, float scale, float pad, EngineTensor** out,
                              PdefaPreprocessMeta* meta) {
    if (tw <= 0 || th <= 0) {
        set_error("target size must be positive");
        return ENGINE_ERR_INVALID_ARG;
    }
    const int64_t shape[4] = {1, 3, th, tw};
    HostTensor t = HostTensor::empty(shape, 4, pdefa::kF32);
    letterbox(img, tw, th, scale, pad, t.f32(), meta);
    *out = pdefa::api::wrap(std::move(t));
    return ENGINE_OK;
}

}  // namespace

extern "C" {

PDEFA_EXPORT const char* pdefa_version(void) { return engine_version(); }
PDEFA_EXPORT const char* pdefa_last_error(void) { return pdefa::api::last_error(); }

PDEFA_EXPORT PdefaImage* pdefa_image_load(const char* path) {
    if (!path) {
        set_error("path null");
        return nullptr;
    }
    clear_error();
    try {
        std::string why;
        auto img = load_pnm(path, &why);
        if (!img) set_error(why);
        return img.release();
    } catch (const std::exception& e) {
        set_error(e.what());
        return nullptr;
    }
}

PDEFA_EXPORT void pdefa_image_free(PdefaImage* img) { delete img; }
PDEFA_EXPORT int32_t pdefa_image_width(const PdefaImage* img) { return img ? img->width : 0; }
PDEFA_EXPORT int32_t pdefa_image_height(const PdefaImage* img) { return img ? img->height : 0; }
PDEFA_EXPORT int32_t pdefa_image_channels(const PdefaImage* img) { return img ? img->channels : 0; }
PDEFA_EXPORT int32_t pdefa_image_format(const PdefaImage* img) {
    if (!img) return -1;
    return img->channels == 1 ? PDEFA_PIXFMT_GRAY8 : (img->channels == 4 ? PDEFA_PIXFMT_RGBA8 : PDEFA_PIXFMT_RGB8);
}
PDEFA_EXPORT const uint8_t* pdefa_image_pixels(const PdefaImage* img, size_t* out_bytes) {
    if (!img) return nullptr;
    if (out_bytes) *out_bytes = img->pixels.size();
    return img->pixels.data();
}

PDEFA_EXPORT EngineStatus pdefa_preprocess_letterbox(const PdefaImage* img, const PdefaPreprocessConfig* cfg,
                                                     EngineTensor** out_tensor, PdefaPreprocessMeta* out_meta) {
    if (!img || !cfg || !out_tensor) {
        set_error("null arg");
        return ENGINE_ERR_NULL_PTR;
    }
    *out_tensor = nullptr;
    return guarded([&] {
        clear_error();
        return letterbox_tensor(*img, cfg->target_w, cfg->target_h, cfg->scale, cfg->pad_value, out_tensor, out_meta);
    });
}

PDEFA_EXPORT EngineStatus pdefa_prepare_for_engine(const char* path, int32_t target_w, int32_t target_h, float scale,
                                                   float pad_value, EngineTensor** out_tensor,
                                                   PdefaPreprocessMeta* out_meta) {
    if (!path || !out_tensor) {
        set_error("null arg");
        return ENGINE_ERR_NULL_PTR;
    }
    *out_tensor = nullptr;
    return guarded([&] {
        clear_error();
        std::string why;
        auto img = load_pnm(path, &why);
        if (!img) {
            set_error("prepare_for_engine failed: " + why);
            return ENGINE_ERR_RUNTIME;
        }
        return letterbox_tensor(*img, target_w, target_h, scale, pad_value, out_tensor, out_meta);
    });
}

PDEFA_EXPORT EngineStatus pdefa_load_image_as_tensor(const char* image_path, int32_t target_w, int32_t target_h,
                                                     EngineTensor** out_tensor) {
    return pdefa_prepare_for_engine(image_path, target_w, target_h, 1.0f / 255.0f, 0.0f, out_tensor, nullptr);
}

// imageloader/src/engine_api.cpp:59-90
PDEFA_EXPORT EngineStatus pdefa_map_box_to_original(const float* in_box, const PdefaPreprocessMeta* meta, float* out_box) {
    if (!in_box || !meta || !out_box) {
        set_error("null arg");
        return ENGINE_ERR_NULL_PTR;
    }
    auto mx = [&](float x) {
        float v = (x - static_cast<float>(meta->pad_x)) / meta->ratio;
        return v < 0.f ? 0.f : (v > static_cast<float>(meta->orig_w) ? static_cast<float>(meta->orig_w) : v);
    };
    auto my = [&](float y) {
        float v = (y - static_cast<float>(meta->pad_y)) / meta->ratio;
        return v < 0.f ? 0.f : (v > static_cast<float>(meta->orig_h) ? static_cast<float>(meta->orig_h) : v);
    };
    const float b[4] = {mx(in_box[0]), my(in_box[1]), mx(in_box[2]), my(in_box[3])};
    std::memcpy(out_box, b, sizeof(b));
    return ENGINE_OK;
}

PDEFA_EXPORT EngineStatus pdefa_map_point_to_original(float* x, float* y, const PdefaPreprocessMeta* meta) {
    if (!x || !y || !meta) {
        set_error("null arg");
        return ENGINE_ERR_NULL_PTR;
    }
    *x = (*x - static_cast<float>(meta->pad_x)) / meta->ratio;
    *y = (*y - static_cast<float>(meta->pad_y)) / meta->ratio;
    if (*x < 0.f) *x = 0.f;
    if (*y < 0.f) *y = 0.f;
    if (*x > static_cast<float>(meta->orig_w)) *x = static_cast<float>(meta->orig_w);
    if (*y > static_cast<float>(meta->orig_h)) *y = static_cast<float>(meta->orig_h);
    return ENGINE_OK;
}

// ------------------------------------------------------------ extensions

PDEFA_EXPORT EngineStatus pdefa_amd_session_replay(EngineSession* sess, int32_t iters, double* out_ms) {
    if (!sess || sess->magic != kMagicSession) return ENGINE_ERR_INVALID_HANDLE;
    if (!out_ms) return ENGINE_ERR_NULL_PTR;
    if (iters <= 0) return ENGINE_ERR_INVALID_ARG;
    return guarded([&] {
        clear_error();
        *out_ms = sess->inner->replay(iters);
        return ENGINE_OK;
    });
}

PDEFA_EXPORT EngineStatus pdefa_amd_session_step_times(EngineSession* sess, int32_t iters, double* ms, int32_t* kind,
                                                       int64_t* flops, int32_t cap, int32_t* n) {
    if (!sess || sess->magic != kMagicSession) return ENGINE_ERR_INVALID_HANDLE;
    if (!n || iters <= 0) return ENGINE_ERR_INVALID_ARG;
    return guarded([&] {
        clear_error();
        std::vector<double> m;
        std::vector<int32_t> k;
        std::vector<int64_t> f;
        sess->inner->step_stats(iters, m, k, f);
        *n = static_cast<int32_t>(m.size());
        for (int32_t i = 0; i < *n && i < cap; ++i) {
            if (ms) ms[i] = m[i];
            if (kind) kind[i] = k[i];
            if (flops) flops[i] = f[i];
        }
        return ENGINE_OK;
    });
}

PDEFA_EXPORT EngineStatus pdefa_amd_session_step_repeat(EngineSession* sess, int32_t step, int32_t iters,
                                                        double* out_ms) {
    if (!sess || sess->magic != kMagicSession) return ENGINE_ERR_INVALID_HANDLE;
    if (!out_ms) return ENGINE_ERR_NULL_PTR;
    if (iters <= 0 || step < 0) return ENGINE_ERR_INVALID_ARG;
    return guarded([&] {
        clear_error();
        *out_ms = sess->inner->repeat_step(step, iters);
        return ENGINE_OK;
    });
}

PDEFA_EXPORT PdefaImage* pdefa_amd_image_from_pixels(const uint8_t* pixels, int32_t width, int32_t height,
                                                     int32_t channels) {
    clear_error();
    if (!pixels || width <= 0 || height <= 0 || (channels != 1 && channels != 3 && channels != 4)) {
        set_error("image_from_pixels: null pixels, empty size or unsupported channel count");
        return nullptr;
    }
    try {
        auto img = std::make_unique<PdefaImage>();
        img->width = width;
        img->height = height;
        img->channels = channels;
        img->pixels.assign(pixels, pixels + static_cast<size_t>(width) * height * channels);
        return img.release();
    } catch (const std::exception& e) {
        set_error(e.what());
        return nullptr;
    }
}

PDEFA_EXPORT EngineStatus pdefa_amd_session_set_images(EngineSession* sess, int32_t input_index, int32_t count,
                                                       const PdefaImage* const* images,
                                                       const PdefaPreprocessConfig* cfg,
                                                       PdefaPreprocessMeta* metas_out) {
    if (!sess || sess->magic != kMagicSession) return ENGINE_ERR_INVALID_HANDLE;
    if (!images || !cfg) return ENGINE_ERR_NULL_PTR;
    if (count <= 0 || cfg->target_w <= 0 || cfg->target_h <= 0) return ENGINE_ERR_INVALID_ARG;
    return guarded([&] {
        clear_error();
        std::vector<pdefa::ImageRef> refs;
        for (int32_t i = 0; i < count; ++i) {
            const PdefaImage* im = images[i];
            if (!im) {
                set_error("image is NULL");
                return ENGINE_ERR_NULL_PTR;
            }
            if (im->pixels.empty() || im->width <= 0 || im->height <= 0 ||
                (im->channels != 1 && im->channels != 3 && im->channels != 4)) {
                set_error("image is empty or has an unsupported channel count");
                return ENGINE_ERR_INVALID_ARG;
            }
            refs.push_back({im->pixels.data(), im->width, im->height, im->channels});
        }
        const std::vector<pdefa::LetterboxGeometry> geo =
            sess->inner->set_images(input_index, refs, cfg->target_w, cfg->target_h, cfg->scale, cfg->pad_value);
        if (metas_out)
            for (int32_t i = 0; i < count; ++i) {
                PdefaPreprocessMeta& m = metas_out[i];
                m.target_w = cfg->target_w;
                m.target_h = cfg->target_h;
                m.orig_w = refs[i].width;
                m.orig_h = refs[i].height;
                m.pad_x = geo[i].pad_x;
                m.pad_y = geo[i].pad_y;
                m.scaled_w = geo[i].scaled_w;
                m.scaled_h = geo[i].scaled_h;
                m.ratio = geo[i].ratio;
            }
        return ENGINE_OK;
    });
}

PDEFA_EXPORT EngineStatus pdefa_amd_session_decode(EngineSession* sess, int32_t output_index,
                                                   const PdefaPreprocessMeta* metas, int32_t n_metas,
                                                   double conf_thres, double iou_thres, int32_t max_det,
                                                   PdefaAmdDetection* dets, int32_t* counts) {
    if (!sess || sess->magic != kMagicSession) return ENGINE_ERR_INVALID_HANDLE;
    if (!counts || (max_det > 0 && !dets)) return ENGINE_ERR_NULL_PTR;
    if (max_det < 0 || n_metas < 0 || (n_metas > 0 && !metas)) return ENGINE_ERR_INVALID_ARG;
    return guarded([&] {
        clear_error();
        std::vector<double> m;
        for (int32_t i = 0; i < n_metas; ++i)
            m.insert(m.end(), {static_cast<double>(metas[i].ratio), static_cast<double>(metas[i].pad_x),
                               static_cast<double>(metas[i].pad_y), static_cast<double>(metas[i].orig_w),
                               static_cast<double>(metas[i].orig_h)});
        const auto res = sess->inner->decode(output_index, m, conf_thres, iou_thres, max_det);
        static_assert(sizeof(PdefaAmdDetection) == sizeof(pdefa::k::YoloDetection), "detection layout");
        for (size_t i = 0; i < res.size(); ++i) {
            counts[i] = static_cast<int32_t>(res[i].size());
            for (size_t j = 0; j < res[i].size(); ++j) {
                const pdefa::k::YoloDetection& d = res[i][j];
                PdefaAmdDetection& o = dets[i * static_cast<size_t>(max_det) + j];
                o.x1 = d.x1;
                o.y1 = d.y1;
                o.x2 = d.x2;
                o.y2 = d.y2;
                o.conf = d.conf;
                o.cls = d.cls;
                o.anchor = d.anchor;
            }
        }
        return ENGINE_OK;
    });
}

PDEFA_EXPORT EngineStatus pdefa_amd_session_plan(const EngineSession* sess, char* buf, size_t cap, size_t* out_len) {
    if (!sess || sess->magic != kMagicSession) return ENGINE_ERR_INVALID_HANDLE;
    return guarded([&] {
        const std::string s = sess->inner->plan_text();
        if (out_len) *out_len = s.size();
        if (buf && cap) {
            const size_t n = std::min(cap - 1, s.size());
            std::memcpy(buf, s.data(), n);
            buf[n] = '\0';
        }
        return ENGINE_OK;
    });
}

PDEFA_EXPORT EngineStatus pdefa_amd_session_read_conv_input(EngineSession* sess, const char* node, float* dst,
                                                           size_t cap, int64_t* dims) {
    if (!sess || sess->magic != kMagicSession) return ENGINE_ERR_INVALID_HANDLE;
    if (!node || !dims) return ENGINE_ERR_NULL_PTR;
    return guarded([&] {
        clear_error();
        std::vector<float> v;
        sess->inner->read_conv_input(node, v, dims);
        if (v.size() > cap || (!dst && !v.empty())) {
            set_error("read_conv_input: the destination holds fewer floats than the tensor");
            return ENGINE_ERR_INVALID_ARG;
        }
        if (!v.empty()) std::memcpy(dst, v.data(), v.size() * sizeof(float));
        return ENGINE_OK;
    });
}

PDEFA_EXPORT EngineStatus pdefa_amd_plan_model(const EngineModel* m, const int64_t* shape, int32_t ndim, char* buf,
                                               size_t cap, size_t* out_len) {
    if (!m || m->magic != kMagicModel) return ENGINE_ERR_INVALID_HANDLE;
    if (!shape || ndim <= 0 || ndim > 6) return ENGINE_ERR_INVALID_ARG;
    return guarded([&] {
        clear_error();
        std::vector<std::vector<int64_t>> dims(static_cast<size_t>(m->inner->num_inputs()),
                                               std::vector<int64_t>(shape, shape + ndim));
        pdefa::PlanOptions opt;
        if (const char* r = std::getenv("PDEFA_REUSE_MEMORY")) opt.reuse_memory = r[0] != '0';
        // as a session plans it: the Detect decode split per anchor range
        const char* so = std::getenv("PDEFA_SPLIT_OUTPUTS");
        opt.split_outputs = !(so && so[0] == '0');
        if (const char* g = std::getenv("PDEFA_PLAN_GROUP_ALL"); g && g[0] == '1') {
            // Host-only stand-ins for the device measurements: launch shapes
            // from the cost model, and every group the grouping pass offers
            // is taken (tests of the reordering it implies).
            opt.tune_conv = [](const pdefa::ConvQuery& q) {
                const int64_t M = static_cast<int64_t>(q.N) * q.Ho * q.Wo;
                return pdefa::k::conv_select(M, q.Cout, q.KH * q.KW * q.Cin, true, q.wino, q.Cin);
            };
            opt.tune_group = [](const std::vector<pdefa::ConvQuery>& qs, const std::vector<pdefa::k::ConvLaunchShape>&) {
                pdefa::ConvGroupTiming t;
                t.tile = pdefa::k::kTile32x32K4;
                t.separate_ms = static_cast<double>(qs.size());
                t.group_ms = 1.0;
                return t;
            };
        }
        const pdefa::Plan p = pdefa::build_plan(*m->inner, dims, opt);
        std::string s = pdefa::describe_plan(*m->inner, p);
        const pdefa::Schedule sc = pdefa::schedule_plan(p, 8);
        std::ostringstream os;
        os << "schedule streams=" << sc.n_streams << "\n";
        for (size_t i = 0; i < sc.stream.size(); ++i) {
            os << i << " stream=" << sc.stream[i] << " deps=";
            for (int d : sc.deps[i]) os << d << ",";
            os << " waits=";
            for (int w : sc.waits[i]) os << w << ",";
            os << "\n";
        }
        s += os.str();
        if (out_len) *out_len = s.size();
        if (buf && cap) {
            const size_t n = std::min(cap - 1, s.size());
            std::memcpy(buf, s.data(), n);
            buf[n] = '\0';
        }
        return ENGINE_OK;
    });
}

PDEFA_EXPORT const char* pdefa_amd_device_name(void) {
    static std::string name = [] {
        if (!pdefa::device_available()) return std::string("none");
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, 0) != hipSuccess) return std::string("unknown");
        // the marketing name can be empty (it is on some drivers): then the
        // architecture, compute units and memory identify the device
        std::string n = p.name;
        if (n.find_first_not_of(' ') == std::string::npos) n = "AMD GPU";
        std::ostringstream os;
        os << n << " (" << p.gcnArchName << ", " << p.multiProcessorCount << " CUs, "
           << (p.totalGlobalMem >> 30) << " GiB)";
        return os.str();
    }();
    return name.c_str();
}

PDEFA_EXPORT EngineStatus pdefa_amd_tune_stats(int64_t* measured, int64_t* from_table) {
    if (!measured || !from_table) return ENGINE_ERR_NULL_PTR;
    size_t m = 0, t = 0;
    pdefa::conv_tune_stats(m, t);
    *measured = static_cast<int64_t>(m);
    *from_table = static_cast<int64_t>(t);
    return ENGINE_OK;
}

PDEFA_EXPORT EngineStatus pdefa_amd_pack_cache_stats(int64_t* read, int64_t* written) {
    if (!read || !written) return ENGINE_ERR_NULL_PTR;
    pdefa::pack_cache_stats(*read, *written);
    return ENGINE_OK;
}

}  // extern "C"
