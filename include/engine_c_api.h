/* engine_c_api.h — the engine_* half of the drop-in C ABI of libpdefa_native.so.
 *
 * Every declaration here replaces the function of the same name declared in
 * the reference's PDEFA1.0/include/engine/engine_c_api.h and exported through
 * pdefa/pdefa.def:19-96; names, argument meaning, ownership and status codes
 * are kept so the reference's ctypes layer binds unchanged.  Each group cites
 * the reference implementation it replaces (PDEFA1.0/src/api/engine_api.cpp).
 *
 * Compute placement: Session::run and engine_ops_matmul execute on the first
 * visible HIP device (MI355X / gfx950); every other ops_* function is a host
 * helper, as in the reference.
 */
#ifndef PDEFA_AMD_ENGINE_C_API_H
#define PDEFA_AMD_ENGINE_C_API_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define PDEFA_EXPORT __attribute__((visibility("default")))
#else
#define PDEFA_EXPORT
#endif

#ifdef __cplusplus
extern "C" {
#endif

typedef struct EngineContext EngineContext;
typedef struct EngineModel EngineModel;
typedef struct EngineSession EngineSession;
typedef struct EngineTensor EngineTensor;

/* Status codes: engine_c_api.h:39-51 of the reference. */
typedef enum EngineStatus {
    ENGINE_OK = 0,
    ENGINE_ERR_NULL_PTR = 1,
    ENGINE_ERR_INVALID_HANDLE = 2,
    ENGINE_ERR_OUT_OF_MEMORY = 3,
    ENGINE_ERR_FILE_NOT_FOUND = 4,
    ENGINE_ERR_INVALID_FORMAT = 5,
    ENGINE_ERR_INVALID_SHAPE = 6,
    ENGINE_ERR_INVALID_ARG = 7,
    ENGINE_ERR_RUNTIME = 8,
    ENGINE_ERR_NOT_IMPL = 9,
    ENGINE_ERR_UNKNOWN = 99
} EngineStatus;

/* Tensor element types: engine_c_api.h:53-62 of the reference. */
typedef enum EngineDType {
    ENGINE_F32 = 0,
    ENGINE_F16 = 1,
    ENGINE_BF16 = 2,
    ENGINE_I8 = 3,
    ENGINE_U8 = 4,
    ENGINE_I32 = 5,
    ENGINE_I64 = 6,
    ENGINE_BOOL = 7
} EngineDType;

/* ---- meta (engine_api.cpp:355-392) ---- */
PDEFA_EXPORT const char* engine_version(void);
PDEFA_EXPORT const char* engine_last_error(void);
PDEFA_EXPORT const char* engine_status_string(EngineStatus s);
PDEFA_EXPORT size_t engine_dtype_size(EngineDType dt);
/* Host SIMD level of the host-side helpers ("AVX-512", "AVX2", "scalar"). */
PDEFA_EXPORT const char* engine_simd_level(void);
PDEFA_EXPORT const char* engine_cpu_brand(void);

/* ---- context (engine_api.cpp:398-443) ---- */
PDEFA_EXPORT EngineStatus engine_context_create(EngineContext** out_ctx);
PDEFA_EXPORT void engine_context_destroy(EngineContext* ctx);
/* n <= 0 -> ENGINE_ERR_INVALID_ARG; sets the host worker count. */
PDEFA_EXPORT EngineStatus engine_context_set_num_threads(EngineContext* ctx, int32_t n);
PDEFA_EXPORT int32_t engine_context_get_num_threads(const EngineContext* ctx);
PDEFA_EXPORT int32_t engine_context_num_physical_cores(void);
PDEFA_EXPORT int32_t engine_context_has_avx2(void);
PDEFA_EXPORT int32_t engine_context_has_avx512(void);

/* ---- tensor: caller-owned host tensors (engine_api.cpp:449-567) ---- */
PDEFA_EXPORT EngineStatus engine_tensor_create(EngineTensor** out_t, const int64_t* shape, int32_t ndim,
                                               EngineDType dtype);
PDEFA_EXPORT EngineStatus engine_tensor_create_from_data(EngineTensor** out_t, const int64_t* shape, int32_t ndim,
                                                         EngineDType dtype, const void* data, size_t bytes);
PDEFA_EXPORT EngineStatus engine_tensor_data(EngineTensor* t, void** out_data, size_t* out_bytes);
PDEFA_EXPORT EngineStatus engine_tensor_shape(const EngineTensor* t, int64_t* out_shape, int32_t* out_ndim);
PDEFA_EXPORT EngineStatus engine_tensor_copy_from(EngineTensor* t, const void* src, size_t bytes);
PDEFA_EXPORT EngineStatus engine_tensor_copy_to(const EngineTensor* t, void* dst, size_t bytes);
PDEFA_EXPORT int64_t engine_tensor_numel(const EngineTensor* t);
PDEFA_EXPORT EngineDType engine_tensor_dtype(const EngineTensor* t);
PDEFA_EXPORT int32_t engine_tensor_rank(const EngineTensor* t);
/* No-op on borrowed tensors (session outputs). */
PDEFA_EXPORT void engine_tensor_destroy(EngineTensor* t);

/* ---- model (engine_api.cpp:573-614, 756-832) ----
 * engine_model_load parses the .engine file; on a GPU host it also uploads the
 * weights to HBM once and packs every conv weight for the MFMA kernel. */
PDEFA_EXPORT EngineStatus engine_model_load(EngineContext* ctx, const char* path, EngineModel** out_model);
PDEFA_EXPORT EngineStatus engine_model_input_count(const EngineModel* m, int32_t* out_n);
PDEFA_EXPORT EngineStatus engine_model_output_count(const EngineModel* m, int32_t* out_n);
PDEFA_EXPORT EngineStatus engine_model_name(const EngineModel* m, const char** out_name);
PDEFA_EXPORT void engine_model_destroy(EngineModel* m);
PDEFA_EXPORT EngineStatus engine_model_input_info(const EngineModel* m, int32_t idx, const char** out_name,
                                                  int64_t* out_shape, int32_t* out_ndim, EngineDType* out_dtype);
PDEFA_EXPORT EngineStatus engine_model_output_info(const EngineModel* m, int32_t idx, const char** out_name,
                                                   int64_t* out_shape, int32_t* out_ndim, EngineDType* out_dtype);

/* ---- session (engine_api.cpp:620-693, 838-892) ----
 * set_input keeps the caller's pointer; run copies the input to HBM, runs the
 * planned device program (one hipGraph launch) and copies the outputs back;
 * get_output returns a borrowed host tensor valid until the next run. */
PDEFA_EXPORT EngineStatus engine_session_create(EngineContext* ctx, EngineModel* model, EngineSession** out_sess);
PDEFA_EXPORT EngineStatus engine_session_set_input(EngineSession* sess, int32_t index, const EngineTensor* input);
PDEFA_EXPORT EngineStatus engine_session_run(EngineSession* sess);
PDEFA_EXPORT EngineStatus engine_session_get_output(const EngineSession* sess, int32_t index,
                                                    const EngineTensor** out_t);
PDEFA_EXPORT void engine_session_destroy(EngineSession* sess);
PDEFA_EXPORT EngineStatus engine_session_debug_intermediate(const EngineSession* sess, int32_t idx,
                                                            const EngineTensor** out_t);

typedef struct {
    double last_run_ms;
    uint64_t runs;
} EngineSessionStats;
PDEFA_EXPORT EngineStatus engine_session_get_stats(const EngineSession* sess, EngineSessionStats* out_stats);

typedef void (*EngineProfileFn)(const char* node_name, double ms, void* user);
/* With a callback set, run() times every device step with HIP events and
 * reports "node_<i>_op<k> '<name>' [dims]" per step. */
PDEFA_EXPORT EngineStatus engine_session_set_profile_callback(EngineSession* sess, EngineProfileFn fn, void* user);
PDEFA_EXPORT EngineStatus engine_session_clear_profile_callback(EngineSession* sess);

PDEFA_EXPORT EngineStatus engine_run_simple(const char* model_path, const EngineTensor* const* inputs,
                                            int32_t num_inputs, EngineTensor** outputs, int32_t num_outputs);

/* ---- ops (engine_api.cpp:898-1660) ---- */
PDEFA_EXPORT EngineStatus engine_ops_add(const EngineTensor* a, const EngineTensor* b, EngineTensor** out);
PDEFA_EXPORT EngineStatus engine_ops_sub(const EngineTensor* a, const EngineTensor* b, EngineTensor** out);
PDEFA_EXPORT EngineStatus engine_ops_mul(const EngineTensor* a, const EngineTensor* b, EngineTensor** out);
PDEFA_EXPORT EngineStatus engine_ops_div(const EngineTensor* a, const EngineTensor* b, EngineTensor** out);
/* C = A @ B on the GPU (fp32 MFMA); out pre-allocated [M,N]; a shape mismatch
 * leaves out untouched and returns ENGINE_OK, as ops::matmul does
 * (PDEFA1.0/src/ops/matmul.cpp:107-135). */
PDEFA_EXPORT EngineStatus engine_ops_matmul(const EngineTensor* a, const EngineTensor* b, EngineTensor* out);
PDEFA_EXPORT EngineStatus engine_ops_relu(EngineTensor* t);
PDEFA_EXPORT EngineStatus engine_ops_silu(EngineTensor* t);
PDEFA_EXPORT EngineStatus engine_ops_sigmoid(EngineTensor* t);
PDEFA_EXPORT EngineStatus engine_ops_tanh(EngineTensor* t);
PDEFA_EXPORT EngineStatus engine_ops_gelu(EngineTensor* t);
PDEFA_EXPORT EngineStatus engine_ops_clip(EngineTensor* t, float lo, float hi);
PDEFA_EXPORT EngineStatus engine_ops_softmax(EngineTensor* t, int32_t axis);
PDEFA_EXPORT EngineStatus engine_ops_reduce_max(const EngineTensor* a, int32_t axis, int32_t keepdims, EngineTensor** out);
PDEFA_EXPORT EngineStatus engine_ops_reduce_sum(const EngineTensor* a, int32_t axis, int32_t keepdims, EngineTensor** out);
PDEFA_EXPORT EngineStatus engine_ops_reduce_mean(const EngineTensor* a, int32_t axis, int32_t keepdims, EngineTensor** out);
PDEFA_EXPORT EngineStatus engine_ops_argmax(const EngineTensor* a, int32_t axis, int32_t keepdims, EngineTensor** out);
PDEFA_EXPORT EngineStatus engine_ops_gather(const EngineTensor* a, const EngineTensor* indices, int32_t axis,
                                            EngineTensor** out);
PDEFA_EXPORT EngineStatus engine_ops_reshape(const EngineTensor* a, const int64_t* shape, int32_t rank, EngineTensor** out);
PDEFA_EXPORT EngineStatus engine_ops_transpose(const EngineTensor* a, const int32_t* perm, int32_t rank,
                                               EngineTensor** out);
PDEFA_EXPORT EngineStatus engine_ops_concat(const EngineTensor* const* inputs, int32_t n, int32_t axis, EngineTensor** out);
PDEFA_EXPORT EngineStatus engine_ops_stack(const EngineTensor* const* inputs, int32_t n, int32_t axis, EngineTensor** out);

/* ---- random (engine_api.cpp:1093-1140): std::mt19937_64(seed) with
 * std::normal_distribution<float>(0,1) / std::uniform_real_distribution<float>(0,1). */
PDEFA_EXPORT EngineStatus engine_random_randn(const int64_t* shape, int32_t rank, uint64_t seed, EngineTensor** out);
PDEFA_EXPORT EngineStatus engine_random_rand(const int64_t* shape, int32_t rank, uint64_t seed, EngineTensor** out);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* PDEFA_AMD_ENGINE_C_API_H */
