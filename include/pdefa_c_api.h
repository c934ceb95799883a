/* pdefa_c_api.h — the pdefa_* half of the drop-in C ABI of libpdefa_native.so.
 *
 * Each declaration replaces the function of the same name in the reference's
 * pdefa/include/pdefa_c_api.h:25-94 (implementation pdefa/src/pdefa_c_api.cpp),
 * exported through pdefa/pdefa.def:3-17.
 *
 * Image decoding is outside the GPU hot path: pdefa_image_load reads binary
 * PPM/PGM (P6/P5, 8-bit) and reports ENGINE_ERR_NOT_IMPL-style failures
 * (NULL + message) for PNG/JPEG; letterboxing restates
 * imageloader/src/preprocess.cpp:15-144 on the host.
 */
#ifndef PDEFA_AMD_PDEFA_C_API_H
#define PDEFA_AMD_PDEFA_C_API_H

#include <stddef.h>
#include <stdint.h>

#include "engine_c_api.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- meta (pdefa_c_api.cpp:36-41) ---- */
PDEFA_EXPORT const char* pdefa_version(void);
/* The last error of any engine_* or pdefa_* call on this thread. */
PDEFA_EXPORT const char* pdefa_last_error(void);

/* ---- image (pdefa_c_api.cpp:44-82) ---- */
typedef struct PdefaImage PdefaImage;
typedef enum {
    PDEFA_PIXFMT_GRAY8 = 0,
    PDEFA_PIXFMT_RGB8 = 1,
    PDEFA_PIXFMT_RGBA8 = 2,
    PDEFA_PIXFMT_GRAY16 = 3,
} PdefaPixelFormat;

PDEFA_EXPORT PdefaImage* pdefa_image_load(const char* path);
PDEFA_EXPORT void pdefa_image_free(PdefaImage* img);
PDEFA_EXPORT int32_t pdefa_image_width(const PdefaImage* img);
PDEFA_EXPORT int32_t pdefa_image_height(const PdefaImage* img);
PDEFA_EXPORT int32_t pdefa_image_channels(const PdefaImage* img);
PDEFA_EXPORT int32_t pdefa_image_format(const PdefaImage* img);
PDEFA_EXPORT const uint8_t* pdefa_image_pixels(const PdefaImage* img, size_t* out_bytes);

/* ---- preprocess (pdefa_c_api.cpp:84-172) ---- */
typedef struct {
    int32_t target_w;
    int32_t target_h;
    float scale;
    float pad_value;
} PdefaPreprocessConfig;

typedef struct {
    int32_t target_w, target_h;
    int32_t orig_w, orig_h;
    int32_t pad_x, pad_y;
    int32_t scaled_w, scaled_h;
    float ratio;
} PdefaPreprocessMeta;

PDEFA_EXPORT EngineStatus pdefa_preprocess_letterbox(const PdefaImage* img, const PdefaPreprocessConfig* cfg,
                                                     EngineTensor** out_tensor, PdefaPreprocessMeta* out_meta);
PDEFA_EXPORT EngineStatus pdefa_prepare_for_engine(const char* path, int32_t target_w, int32_t target_h, float scale,
                                                   float pad_value, EngineTensor** out_tensor,
                                                   PdefaPreprocessMeta* out_meta);
PDEFA_EXPORT EngineStatus pdefa_load_image_as_tensor(const char* image_path, int32_t target_w, int32_t target_h,
                                                     EngineTensor** out_tensor);

/* ---- post-process (pdefa_c_api.cpp:175-213; imageloader map_box_to_original) ---- */
PDEFA_EXPORT EngineStatus pdefa_map_box_to_original(const float* in_box, const PdefaPreprocessMeta* meta, float* out_box);
PDEFA_EXPORT EngineStatus pdefa_map_point_to_original(float* x, float* y, const PdefaPreprocessMeta* meta);

#ifdef __cplusplus
}
#endif
#endif /* PDEFA_AMD_PDEFA_C_API_H */
