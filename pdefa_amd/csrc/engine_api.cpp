// engine_* C ABI: handles, model/session lifecycle and ops_matmul.
// Behaviour follows PDEFA1.0/src/api/engine_api.cpp (cited per function);
// compute runs through the device runtime (runtime.cpp).
#include <cpuid.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <fstream>
#include <set>
#include <string>
#include <thread>
#include <utility>

#include "api_internal.hpp"

using pdefa::HostTensor;
using pdefa::api::clear_error;
using pdefa::api::guarded;
using pdefa::api::set_error;
using pdefa::api::valid;

namespace pdefa {
namespace api {

namespace {
thread_local std::string g_error;
}

void set_error(const std::string& msg) noexcept {
    try {
        g_error = msg;
    } catch (...) {
    }
}
void clear_error() noexcept { g_error.clear(); }
const char* last_error() noexcept { return g_error.c_str(); }

EngineTensor* wrap(HostTensor&& t) {
    auto* h = new EngineTensor();
    h->owned = std::make_unique<HostTensor>(std::move(t));
    return h;
}

}  // namespace api
}  // namespace pdefa

namespace {

int32_t logical_cores() {
    const unsigned n = std::thread::hardware_concurrency();
    return n > 0 ? static_cast<int32_t>(n) : 1;
}

int32_t physical_cores() {
    std::ifstream f("/proc/cpuinfo");
    std::string line;
    std::set<std::pair<int, int>> cores;
    int phys = 0;
    while (std::getline(f, line)) {
        if (line.rfind("physical id", 0) == 0) phys = std::atoi(line.substr(line.find(':') + 1).c_str());
        if (line.rfind("core id", 0) == 0) cores.insert({phys, std::atoi(line.substr(line.find(':') + 1).c_str())});
    }
    return cores.empty() ? logical_cores() : static_cast<int32_t>(cores.size());
}

bool cpu_has(const char* feat) {
    __builtin_cpu_init();
    if (std::strcmp(feat, "avx2") == 0) return __builtin_cpu_supports("avx2");
    if (std::strcmp(feat, "avx512f") == 0) return __builtin_cpu_supports("avx512f");
    return false;
}

bool valid_dtype(EngineDType dt) { return dt >= ENGINE_F32 && dt <= ENGINE_BOOL; }

}  // namespace

extern "C" {

// ---------------------------------------------------------------- meta
// engine_api.cpp:355-392
PDEFA_EXPORT const char* engine_version(void) { return "1.0.3"; }

PDEFA_EXPORT const char* engine_last_error(void) { return pdefa::api::last_error(); }

PDEFA_EXPORT const char* engine_status_string(EngineStatus s) {
    switch (s) {
        case ENGINE_OK: return "OK";
        case ENGINE_ERR_NULL_PTR: return "null pointer";
        case ENGINE_ERR_INVALID_HANDLE: return "invalid handle";
        case ENGINE_ERR_OUT_OF_MEMORY: return "out of memory";
        case ENGINE_ERR_FILE_NOT_FOUND: return "file not found";
        case ENGINE_ERR_INVALID_FORMAT: return "invalid format";
        case ENGINE_ERR_INVALID_SHAPE: return "invalid shape";
        case ENGINE_ERR_INVALID_ARG: return "invalid argument";
        case ENGINE_ERR_RUNTIME: return "runtime error";
        case ENGINE_ERR_NOT_IMPL: return "not implemented";
        default: return "unknown";
    }
}

PDEFA_EXPORT size_t engine_dtype_size(EngineDType dt) { return pdefa::dt_size(dt); }

PDEFA_EXPORT const char* engine_simd_level(void) {
    if (cpu_has("avx512f")) return "AVX-512";
    if (cpu_has("avx2")) return "AVX2";
    return "scalar";
}

PDEFA_EXPORT const char* engine_cpu_brand(void) {
    static std::string brand = [] {
        unsigned int r[12] = {0};
        unsigned int a, b, c, d;
        if (__get_cpuid(0x80000000u, &a, &b, &c, &d) && a >= 0x80000004u) {
            for (unsigned int i = 0; i < 3; ++i) __get_cpuid(0x80000002u + i, &r[4 * i], &r[4 * i + 1], &r[4 * i + 2], &r[4 * i + 3]);
            std::string s(reinterpret_cast<const char*>(r), 48);
            s = s.c_str();
            const size_t p = s.find_first_not_of(' ');
            return p == std::string::npos ? std::string("unknown CPU") : s.substr(p);
        }
        return std::string("unknown CPU");
    }();
    return brand.c_str();
}

// ---------------------------------------------------------------- context
// engine_api.cpp:398-443
PDEFA_EXPORT EngineStatus engine_context_create(EngineContext** out_ctx) {
    if (!out_ctx) {
        set_error("out_ctx is null");
        return ENGINE_ERR_NULL_PTR;
    }
    *out_ctx = nullptr;
    return guarded([&] {
        clear_error();
        auto* c = new EngineContext();
        c->num_threads = logical_cores();
        *out_ctx = c;
        return ENGINE_OK;
    });
}

PDEFA_EXPORT void engine_context_destroy(EngineContext* ctx) {
    if (!ctx || ctx->magic != kMagicContext) return;
    ctx->magic = 0;
    delete ctx;
}

PDEFA_EXPORT EngineStatus engine_context_set_num_threads(EngineContext* ctx, int32_t n) {
    if (!ctx || ctx->magic != kMagicContext) return ENGINE_ERR_INVALID_HANDLE;
    if (n <= 0) {
        set_error("num_threads must be > 0");
        return ENGINE_ERR_INVALID_ARG;
    }
    ctx->num_threads = n;
    return ENGINE_OK;
}

PDEFA_EXPORT int32_t engine_context_get_num_threads(const EngineContext* ctx) {
    if (!ctx || ctx->magic != kMagicContext) return 0;
    return ctx->num_threads;
}

PDEFA_EXPORT int32_t engine_context_num_physical_cores(void) { return physical_cores(); }
PDEFA_EXPORT int32_t engine_context_has_avx2(void) { return cpu_has("avx2") ? 1 : 0; }
PDEFA_EXPORT int32_t engine_context_has_avx512(void) { return cpu_has("avx512f") ? 1 : 0; }

// ---------------------------------------------------------------- tensor
// engine_api.cpp:449-567
PDEFA_EXPORT EngineStatus engine_tensor_create(EngineTensor** out_t, const int64_t* shape, int32_t ndim,
                                               EngineDType dtype) {
    if (!out_t || !shape) {
        set_error("null argument");
        return ENGINE_ERR_NULL_PTR;
    }
    *out_t = nullptr;
    if (!valid_dtype(dtype) || ndim < 0 || ndim > pdefa::kMaxNdim) {
        set_error("invalid dtype or rank");
        return ENGINE_ERR_INVALID_ARG;
    }
    return guarded([&] {
        clear_error();
        *out_t = pdefa::api::wrap(HostTensor::empty_pinned(shape, ndim, dtype));
        return ENGINE_OK;
    });
}

PDEFA_EXPORT EngineStatus engine_tensor_create_from_data(EngineTensor** out_t, const int64_t* shape, int32_t ndim,
                                                         EngineDType dtype, const void* data, size_t bytes) {
    if (!out_t || !shape || !data) {
        set_error("null argument");
        return ENGINE_ERR_NULL_PTR;
    }
    *out_t = nullptr;
    if (!valid_dtype(dtype) || ndim < 0 || ndim > pdefa::kMaxNdim) {
        set_error("invalid dtype or rank");
        return ENGINE_ERR_INVALID_ARG;
    }
    return guarded([&] {
        clear_error();
        HostTensor t = HostTensor::empty_pinned(shape, ndim, dtype);
        if (bytes > t.nbytes) {
            set_error("data too large");
            return ENGINE_ERR_INVALID_ARG;
        }
        if (bytes) std::memcpy(t.data, data, bytes);
        *out_t = pdefa::api::wrap(std::move(t));
        return ENGINE_OK;
    });
}

PDEFA_EXPORT EngineStatus engine_tensor_data(EngineTensor* t, void** out_data, size_t* out_bytes) {
    if (!valid(t)) return ENGINE_ERR_INVALID_HANDLE;
    if (!out_data) return ENGINE_ERR_NULL_PTR;
    *out_data = t->ptr()->data;
    if (out_bytes) *out_bytes = t->ptr()->nbytes;
    return ENGINE_OK;
}

PDEFA_EXPORT EngineStatus engine_tensor_shape(const EngineTensor* t, int64_t* out_shape, int32_t* out_ndim) {
    if (!valid(t)) return ENGINE_ERR_INVALID_HANDLE;
    const HostTensor* h = t->ptr();
    if (out_shape)
        for (int i = 0; i < h->rank; ++i) out_shape[i] = h->dims[i];
    if (out_ndim) *out_ndim = h->rank;
    return ENGINE_OK;
}

PDEFA_EXPORT EngineStatus engine_tensor_copy_from(EngineTensor* t, const void* src, size_t bytes) {
    if (!valid(t)) return ENGINE_ERR_INVALID_HANDLE;
    if (!src) return ENGINE_ERR_NULL_PTR;
    if (t->is_borrowed()) {
        set_error("cannot write to borrowed tensor");
        return ENGINE_ERR_INVALID_ARG;
    }
    if (bytes > t->ptr()->nbytes) return ENGINE_ERR_INVALID_ARG;
    if (bytes) std::memcpy(t->ptr()->data, src, bytes);
    return ENGINE_OK;
}

PDEFA_EXPORT EngineStatus engine_tensor_copy_to(const EngineTensor* t, void* dst, size_t bytes) {
    if (!valid(t)) return ENGINE_ERR_INVALID_HANDLE;
    if (!dst) return ENGINE_ERR_NULL_PTR;
    if (bytes > t->ptr()->nbytes) return ENGINE_ERR_INVALID_ARG;
    if (bytes) std::memcpy(dst, t->ptr()->data, bytes);
    return ENGINE_OK;
}

PDEFA_EXPORT int64_t engine_tensor_numel(const EngineTensor* t) { return valid(t) ? t->ptr()->numel() : 0; }

PDEFA_EXPORT EngineDType engine_tensor_dtype(const EngineTensor* t) {
    return valid(t) ? static_cast<EngineDType>(t->ptr()->dtype) : ENGINE_F32;
}

PDEFA_EXPORT int32_t engine_tensor_rank(const EngineTensor* t) { return valid(t) ? t->ptr()->rank : 0; }

PDEFA_EXPORT void engine_tensor_destroy(EngineTensor* t) {
    if (!t || t->magic != kMagicTensor) return;
    if (t->is_borrowed()) return;  // session-owned wrapper
    t->magic = 0;
    delete t;
}

// ---------------------------------------------------------------- model
// engine_api.cpp:573-614
PDEFA_EXPORT EngineStatus engine_model_load(EngineContext* ctx, const char* path, EngineModel** out_model) {
    (void)ctx;
    if (!out_model || !path) {
        set_error("null argument");
        return ENGINE_ERR_NULL_PTR;
    }
    *out_model = nullptr;
    return guarded([&] {
        clear_error();
        auto m = std::make_unique<EngineModel>();
        m->inner = std::make_unique<pdefa::Model>();
        std::string why;
        if (!pdefa::load_engine_file(path, *m->inner, &why)) {
            set_error("failed to load model file: " + why);
            return ENGINE_ERR_INVALID_FORMAT;
        }
        // Weights go to HBM once, at load, when a device is present.
        if (pdefa::device_available()) pdefa::device_model(*m->inner);
        *out_model = m.release();
        return ENGINE_OK;
    });
}

PDEFA_EXPORT EngineStatus engine_model_input_count(const EngineModel* m, int32_t* out_n) {
    if (!m || m->magic != kMagicModel) return ENGINE_ERR_INVALID_HANDLE;
    if (out_n) *out_n = m->inner->num_inputs();
    return ENGINE_OK;
}

PDEFA_EXPORT EngineStatus engine_model_output_count(const EngineModel* m, int32_t* out_n) {
    if (!m || m->magic != kMagicModel) return ENGINE_ERR_INVALID_HANDLE;
    if (out_n) *out_n = m->inner->num_outputs();
    return ENGINE_OK;
}

PDEFA_EXPORT EngineStatus engine_model_name(const EngineModel* m, const char** out_name) {
    if (!m || m->magic != kMagicModel) return ENGINE_ERR_INVALID_HANDLE;
    if (!out_name) return ENGINE_ERR_NULL_PTR;
    *out_name = m->inner->name.c_str();
    return ENGINE_OK;
}

PDEFA_EXPORT void engine_model_destroy(EngineModel* m) {
    if (!m || m->magic != kMagicModel) return;
    m->magic = 0;
    delete m;
}

namespace {

// engine_api.cpp:756-832: v2 metadata when present, else [1,3,640,640] /
// [1,84,8400] F32 defaults.
EngineStatus model_info(const EngineModel* m, int32_t idx, bool input, const char** out_name, int64_t* out_shape,
                        int32_t* out_ndim, EngineDType* out_dtype) {
    if (!m || m->magic != kMagicModel) return ENGINE_ERR_INVALID_HANDLE;
    const pdefa::Model& md = *m->inner;
    const int32_t count = input ? md.num_inputs() : md.num_outputs();
    if (idx < 0 || idx >= count) {
        set_error(input ? "input index out of range" : "output index out of range");
        return ENGINE_ERR_INVALID_ARG;
    }
    static thread_local std::string name_buf;
    const auto& infos = input ? md.input_infos : md.output_infos;
    if (idx < static_cast<int32_t>(infos.size())) {
        const pdefa::TensorInfo& ti = infos[idx];
        if (out_name) {
            name_buf = ti.name.empty() ? std::string(input ? "input_" : "output_") + std::to_string(idx) : ti.name;
            *out_name = name_buf.c_str();
        }
        if (out_shape)
            for (int i = 0; i < ti.ndim; ++i) out_shape[i] = ti.shape[i];
        if (out_ndim) *out_ndim = ti.ndim;
        if (out_dtype) *out_dtype = static_cast<EngineDType>(pdefa::public_dtype(ti.dtype));
        return ENGINE_OK;
    }
    if (out_name) {
        name_buf = std::string(input ? "input_" : "output_") + std::to_string(idx);
        *out_name = name_buf.c_str();
    }
    if (input) {
        if (out_shape) {
            out_shape[0] = 1;
            out_shape[1] = 3;
            out_shape[2] = 640;
            out_shape[3] = 640;
        }
        if (out_ndim) *out_ndim = 4;
    } else {
        if (out_shape) {
            out_shape[0] = 1;
            out_shape[1] = 84;
            out_shape[2] = 8400;
        }
        if (out_ndim) *out_ndim = 3;
    }
    if (out_dtype) *out_dtype = ENGINE_F32;
    return ENGINE_OK;
}

}  // namespace

PDEFA_EXPORT EngineStatus engine_model_input_info(const EngineModel* m, int32_t idx, const char** out_name,
                                                  int64_t* out_shape, int32_t* out_ndim, EngineDType* out_dtype) {
    return model_info(m, idx, true, out_name, out_shape, out_ndim, out_dtype);
}

PDEFA_EXPORT EngineStatus engine_model_output_info(const EngineModel* m, int32_t idx, const char** out_name,
                                                   int64_t* out_shape, int32_t* out_ndim, EngineDType* out_dtype) {
    return model_info(m, idx, false, out_name, out_shape, out_ndim, out_dtype);
}

// ---------------------------------------------------------------- session
// engine_api.cpp:620-693
PDEFA_EXPORT EngineStatus engine_session_create(EngineContext* ctx, EngineModel* model, EngineSession** out_sess) {
    (void)ctx;
    if (!out_sess) return ENGINE_ERR_NULL_PTR;
    *out_sess = nullptr;
    if (!model || model->magic != kMagicModel) return ENGINE_ERR_INVALID_HANDLE;
    return guarded([&] {
        clear_error();
        auto* s = new EngineSession();
        s->inner = std::make_unique<pdefa::Session>(*model->inner);
        *out_sess = s;
        return ENGINE_OK;
    });
}

PDEFA_EXPORT EngineStatus engine_session_set_input(EngineSession* sess, int32_t index, const EngineTensor* input) {
    if (!sess || sess->magic != kMagicSession) return ENGINE_ERR_INVALID_HANDLE;
    if (!valid(input)) return ENGINE_ERR_INVALID_HANDLE;
    sess->inner->set_input(index, input->ptr());
    return ENGINE_OK;
}

PDEFA_EXPORT EngineStatus engine_session_run(EngineSession* sess) {
    if (!sess || sess->magic != kMagicSession) return ENGINE_ERR_INVALID_HANDLE;
    return guarded([&] {
        clear_error();
        sess->inner->run();
        return ENGINE_OK;
    });
}

PDEFA_EXPORT EngineStatus engine_session_get_output(const EngineSession* sess, int32_t index,
                                                    const EngineTensor** out_t) {
    if (!out_t) return ENGINE_ERR_NULL_PTR;
    *out_t = nullptr;
    if (!sess || sess->magic != kMagicSession) return ENGINE_ERR_INVALID_HANDLE;
    const HostTensor* t = sess->inner->output(index);
    if (!t) {
        set_error("output not available");
        return ENGINE_ERR_INVALID_ARG;
    }
    // Borrowed per-thread wrapper, as the reference returns (engine_api.cpp:670-675):
    // valid until the next call on this thread or the session's next run.
    static thread_local EngineTensor wrapper;
    wrapper.magic = kMagicTensor;
    wrapper.owned.reset();
    wrapper.borrowed = const_cast<HostTensor*>(t);
    *out_t = &wrapper;
    return ENGINE_OK;
}

PDEFA_EXPORT void engine_session_destroy(EngineSession* sess) {
    if (!sess || sess->magic != kMagicSession) return;
    sess->magic = 0;
    delete sess;
}

// Intermediates live in a reused HBM arena and are not kept after a run; the
// reference likewise frees them once consumed (session.cpp:329-338).
PDEFA_EXPORT EngineStatus engine_session_debug_intermediate(const EngineSession* sess, int32_t idx,
                                                            const EngineTensor** out_t) {
    (void)idx;
    if (!out_t) return ENGINE_ERR_NULL_PTR;
    *out_t = nullptr;
    if (!sess || sess->magic != kMagicSession) return ENGINE_ERR_INVALID_HANDLE;
    set_error("intermediate not available");
    return ENGINE_ERR_INVALID_ARG;
}

PDEFA_EXPORT EngineStatus engine_session_get_stats(const EngineSession* sess, EngineSessionStats* out_stats) {
    if (!sess || sess->magic != kMagicSession) return ENGINE_ERR_INVALID_HANDLE;
    if (!out_stats) return ENGINE_ERR_NULL_PTR;
    out_stats->last_run_ms = sess->inner->last_run_ms;
    out_stats->runs = sess->inner->runs;
    return ENGINE_OK;
}

PDEFA_EXPORT EngineStatus engine_session_set_profile_callback(EngineSession* sess, EngineProfileFn fn, void* user) {
    if (!sess || sess->magic != kMagicSession) return ENGINE_ERR_INVALID_HANDLE;
    sess->inner->set_profile(fn, user);
    return ENGINE_OK;
}

PDEFA_EXPORT EngineStatus engine_session_clear_profile_callback(EngineSession* sess) {
    if (!sess || sess->magic != kMagicSession) return ENGINE_ERR_INVALID_HANDLE;
    sess->inner->set_profile(nullptr, nullptr);
    return ENGINE_OK;
}

// engine_api.cpp:699-750
PDEFA_EXPORT EngineStatus engine_run_simple(const char* model_path, const EngineTensor* const* inputs,
                                            int32_t num_inputs, EngineTensor** outputs, int32_t num_outputs) {
    if (!model_path || !inputs || !outputs) return ENGINE_ERR_NULL_PTR;
    return guarded([&] {
        clear_error();
        pdefa::Model model;
        std::string why;
        if (!pdefa::load_engine_file(model_path, model, &why)) {
            set_error("failed to load model: " + why);
            return ENGINE_ERR_INVALID_FORMAT;
        }
        pdefa::Session sess(model);
        for (int32_t i = 0; i < num_inputs; ++i) {
            if (!inputs[i]) return ENGINE_ERR_NULL_PTR;
            sess.set_input(i, inputs[i]->ptr());
        }
        sess.run();
        for (int32_t i = 0; i < num_outputs; ++i) {
            const HostTensor* t = sess.output(i);
            outputs[i] = t ? pdefa::api::wrap(t->clone()) : nullptr;
        }
        return ENGINE_OK;
    });
}

// ---------------------------------------------------------------- matmul

namespace {

using GemmFn = void (*)(const float*, const float*, float*, int64_t, int64_t, int64_t);

// The shape rules of ops::matmul (matmul.cpp:59-135): F32 only; rank > 2
// on either side is batched [..., M, K] x [..., K, N] (or a 2-D B shared by
// every batch), one GEMM per batch; mismatched shapes leave `out` untouched
// and still return ENGINE_OK.  (The reference does not check that `out` or
// a batched B hold the whole batch; here such calls are no-ops too.)
EngineStatus matmul_front(const EngineTensor* a, const EngineTensor* b, EngineTensor* out, GemmFn gemm) {
    if (!valid(a) || !valid(b) || !valid(out)) return ENGINE_ERR_INVALID_HANDLE;
    if (out->is_borrowed()) {
        set_error("cannot write to borrowed tensor");
        return ENGINE_ERR_INVALID_ARG;
    }
    return guarded([&] {
        clear_error();
        const HostTensor& A = *a->ptr();
        const HostTensor& B = *b->ptr();
        HostTensor& Cc = *out->ptr();
        if (A.dtype != pdefa::kF32 || B.dtype != pdefa::kF32 || Cc.dtype != pdefa::kF32) return ENGINE_OK;
        if (A.rank > 2 || B.rank > 2) {
            if (A.rank < 2 || B.rank < 2 || Cc.rank < 2) return ENGINE_OK;
            if (A.dim(A.rank - 1) != B.dim(B.rank - 2)) return ENGINE_OK;
            const int64_t M = A.dim(A.rank - 2), K = A.dim(A.rank - 1), N = B.dim(B.rank - 1);
            int64_t batch = 1;
            for (int i = 0; i < A.rank - 2; ++i) batch *= A.dims[i];
            if (batch <= 0 || Cc.numel() < batch * M * N) return ENGINE_OK;
            const int64_t bstride = B.rank == 2 ? 0 : K * N;
            if (bstride && B.numel() < batch * K * N) return ENGINE_OK;
            for (int64_t i = 0; i < batch; ++i)
                gemm(A.f32() + i * M * K, B.f32() + i * bstride, Cc.f32() + i * M * N, M, K, N);
            return ENGINE_OK;
        }
        if (A.rank != 2 || B.rank != 2 || Cc.rank != 2) return ENGINE_OK;
        const int64_t M = A.dims[0], K = A.dims[1], N = B.dims[1];
        if (B.dims[0] != K || Cc.dims[0] != M || Cc.dims[1] != N) return ENGINE_OK;
        gemm(A.f32(), B.f32(), Cc.f32(), M, K, N);
        return ENGINE_OK;
    });
}

}  // namespace

// engine_api.cpp:898-914 -> ops::matmul (matmul.cpp:59-135), on the GPU.
PDEFA_EXPORT EngineStatus engine_ops_matmul(const EngineTensor* a, const EngineTensor* b, EngineTensor* out) {
    return matmul_front(a, b, out, &pdefa::device_matmul);
}

// engine_ops_matmul with its device buffers in the static scratch array.
PDEFA_EXPORT EngineStatus pdefa_amd_ops_matmul_noalloc(const EngineTensor* a, const EngineTensor* b,
                                                       EngineTensor* out) {
    return matmul_front(a, b, out, &pdefa::device_matmul_noalloc);
}

}  // extern "C"
