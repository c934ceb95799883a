/* oracle/ref_driver.cpp — test infrastructure, NOT product code.
 *
 * A thin C-ABI driver around the reference engine's own C++ classes, compiled
 * together with the reference sources (see oracle/Makefile) into
 * oracle/_ref/libpdefa_ref.so.  It is the checker for the MI355X build: tests,
 * smoke() and bench.py's CPU-baseline leg load it through ctypes; nothing in
 * the product links or calls it.
 *
 * Only the engine core is compiled (tensor/model/session/ops/kernels/loader/
 * memory/runtime).  PDEFA1.0/src/api/engine_api.cpp is left out because it
 * includes a CMake-generated header (engine/version.hpp); this driver reaches
 * the same objects the C API wraps:
 *   - engine_model_load     -> loader::load_engine_file  (engine_api.cpp:573-592)
 *   - engine_session_create -> Session(model)            (engine_api.cpp:620-634)
 *   - engine_session_run    -> Session::run              (engine_api.cpp:649-652)
 *   - engine_session_get_output -> Session::output       (engine_api.cpp:654-677)
 *   - engine_ops_matmul     -> ops::matmul               (engine_api.cpp:898-914)
 *   - pdefa_preprocess_letterbox -> imageloader::preprocess_letterbox
 *                                                        (pdefa_c_api.cpp:84-126)
 */
#include "engine/loader/custom_loader.hpp"
#include "engine/model.hpp"
#include "engine/session.hpp"
#include "engine/tensor.hpp"
#include "engine/ops/matmul.hpp"
#include "engine/runtime/thread_pool.hpp"
#include "imageloader/preprocess.hpp"

#include <cstdint>
#include <cstring>
#include <memory>
#include <vector>

namespace {

struct RefSession {
    std::unique_ptr<engine::Session> sess;
    engine::Tensor input;   // owned copy of the caller's NCHW input
};

}  // namespace

extern "C" {

__attribute__((visibility("default"))) void* ref_model_load(const char* path) {
    auto m = std::make_unique<engine::Model>();
    if (!engine::loader::load_engine_file(path, *m)) return nullptr;
    return m.release();
}

__attribute__((visibility("default"))) void ref_model_free(void* m) {
    delete static_cast<engine::Model*>(m);
}

__attribute__((visibility("default"))) void* ref_session_new(void* m) {
    if (!m) return nullptr;
    auto* s = new RefSession();
    s->sess = std::make_unique<engine::Session>(*static_cast<engine::Model*>(m));
    return s;
}

__attribute__((visibility("default"))) void ref_session_free(void* s) {
    delete static_cast<RefSession*>(s);
}

/* Copies `input` (F32, shape[ndim]) into a session-owned tensor, binds it as
 * graph input 0 and runs the graph once.  Returns 0 on success. */
__attribute__((visibility("default"))) int ref_session_run(void* sp, const float* input,
                                                           const int64_t* shape, int ndim) {
    auto* s = static_cast<RefSession*>(sp);
    if (!s || !input || !shape || ndim <= 0 || ndim > 8) return -1;
    engine::Shape sh(shape, ndim);
    if (s->input.is_empty() || s->input.shape() != sh) {
        s->input = engine::Tensor::empty(sh, engine::DType::F32);
        if (s->input.is_empty()) return -2;
    }
    std::memcpy(s->input.data(), input, s->input.nbytes());
    s->sess->set_input(0, &s->input);
    return s->sess->run() ? 0 : -3;
}

/* Re-runs with the already bound input (timing loops). */
__attribute__((visibility("default"))) int ref_session_rerun(void* sp) {
    auto* s = static_cast<RefSession*>(sp);
    if (!s) return -1;
    return s->sess->run() ? 0 : -3;
}

__attribute__((visibility("default"))) double ref_session_last_ms(void* sp) {
    auto* s = static_cast<RefSession*>(sp);
    return s ? s->sess->stats().last_run_ms : -1.0;
}

__attribute__((visibility("default"))) int ref_output_count(void* sp) {
    auto* s = static_cast<RefSession*>(sp);
    return s ? s->sess->num_outputs() : 0;
}

/* Writes the output's dims into shape[8]; returns its rank, or -1. */
__attribute__((visibility("default"))) int ref_output_shape(void* sp, int idx, int64_t* shape) {
    auto* s = static_cast<RefSession*>(sp);
    if (!s) return -1;
    const engine::Tensor* t = s->sess->output(idx);
    if (!t) return -1;
    for (int d = 0; d < t->rank(); ++d) shape[d] = t->dim(d);
    return t->rank();
}

/* Output idx as float values (I32 / I64 outputs, such as TopK indices, are
 * converted value by value). */
__attribute__((visibility("default"))) int ref_output_copy(void* sp, int idx, float* dst, int64_t n) {
    auto* s = static_cast<RefSession*>(sp);
    if (!s || !dst) return -1;
    const engine::Tensor* t = s->sess->output(idx);
    if (!t || t->numel() != n) return -1;
    if (t->dtype() == engine::DType::I32) {
        for (int64_t i = 0; i < n; ++i) dst[i] = static_cast<float>(t->data<int32_t>()[i]);
    } else if (t->dtype() == engine::DType::I64) {
        for (int64_t i = 0; i < n; ++i) dst[i] = static_cast<float>(t->data<int64_t>()[i]);
    } else {
        std::memcpy(dst, t->data(), t->nbytes());
    }
    return 0;
}

/* Element type of output idx (the engine's DType code), or -1. */
__attribute__((visibility("default"))) int ref_output_dtype(void* sp, int idx) {
    auto* s = static_cast<RefSession*>(sp);
    if (!s) return -1;
    const engine::Tensor* t = s->sess->output(idx);
    return t ? static_cast<int>(t->dtype()) : -1;
}

__attribute__((visibility("default"))) void ref_set_threads(int n) {
    engine::runtime::GlobalPool::set_num_threads(n);
}

/* C[M,N] = A[M,K] @ B[K,N] through ops::matmul (the engine_ops_matmul path). */
__attribute__((visibility("default"))) int ref_matmul(const float* A, const float* B, float* C,
                                                      int64_t M, int64_t K, int64_t N) {
    int64_t da[2] = {M, K}, db[2] = {K, N}, dc[2] = {M, N};
    engine::Tensor a = engine::Tensor::empty(engine::Shape(da, 2), engine::DType::F32);
    engine::Tensor b = engine::Tensor::empty(engine::Shape(db, 2), engine::DType::F32);
    engine::Tensor c = engine::Tensor::empty(engine::Shape(dc, 2), engine::DType::F32);
    if (a.is_empty() || b.is_empty() || c.is_empty()) return -1;
    std::memcpy(a.data(), A, a.nbytes());
    std::memcpy(b.data(), B, b.nbytes());
    engine::ops::matmul(a, b, c);
    std::memcpy(C, c.data(), c.nbytes());
    return 0;
}

/* Letterbox of an 8-bit interleaved image into out[3*th*tw] (NCHW planes).
 * meta[0..7] = target_w, target_h, pad_x, pad_y, scaled_w, scaled_h, and
 * ratio is returned through *ratio. */
__attribute__((visibility("default"))) int ref_letterbox(const uint8_t* pix, int w, int h, int ch,
                                                         int tw, int th, float scale, float pad,
                                                         float* out, int32_t* meta, float* ratio) {
    imageloader::Image img;
    img.width = (uint32_t)w;
    img.height = (uint32_t)h;
    img.format = ch == 1 ? imageloader::PixelFormat::GRAY8
               : ch == 4 ? imageloader::PixelFormat::RGBA8
                         : imageloader::PixelFormat::RGB8;
    img.pixels.assign(pix, pix + (size_t)w * h * ch);
    imageloader::PreprocessConfig cfg;
    cfg.target_w = tw;
    cfg.target_h = th;
    cfg.scale = scale;
    cfg.pad_value = pad;
    imageloader::PreprocessResult r = imageloader::preprocess_letterbox(img, cfg);
    if (r.data.size() != (size_t)3 * tw * th) return -1;
    std::memcpy(out, r.data.data(), r.data.size() * sizeof(float));
    meta[0] = r.target_w; meta[1] = r.target_h;
    meta[2] = r.pad_x;    meta[3] = r.pad_y;
    meta[4] = r.scaled_w; meta[5] = r.scaled_h;
    *ratio = r.ratio;
    return 0;
}

}  // extern "C"
