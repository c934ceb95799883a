/* pdefa_amd_ext.h — entry points of libpdefa_native.so with no counterpart in
 * the reference.  They serve benchmarking and testing of the device program,
 * and the on-device letterbox input; the drop-in ABI (engine_c_api.h,
 * pdefa_c_api.h) does not depend on them.
 */
#ifndef PDEFA_AMD_EXT_H
#define PDEFA_AMD_EXT_H

#include <stddef.h>
#include <stdint.h>

#include "engine_c_api.h"
#include "pdefa_c_api.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Re-runs the session's prepared device program `iters` times on the input
 * already resident in HBM (uploaded by the last engine_session_run), with no
 * host copies; *out_ms = elapsed device time from HIP events on the session's
 * stream.  Requires one completed engine_session_run. */
PDEFA_EXPORT EngineStatus pdefa_amd_session_replay(EngineSession* sess, int32_t iters, double* out_ms);

/* Average device time of each launch of the prepared program over `iters`
 * launch-by-launch replays (HIP events between launches on the session
 * stream).  A launch is one step of the plan, or several convs issued as one
 * grouped launch.  Per launch: ms[i], kind[i] (0 conv_mfma, 1 conv_direct,
 * 2 eltwise, 3 maxpool, 4 resize, 5 softmax, 6 maxpool chain, 7 detect decode)
 * and flops[i] (sum of 2*N*Cout*Cin*KH*KW*Ho*Wo over its convs, else 0).
 * *n = number of launches; at most `cap` entries are written. */
PDEFA_EXPORT EngineStatus pdefa_amd_session_step_times(EngineSession* sess, int32_t iters, double* ms, int32_t* kind,
                                                       int64_t* flops, int32_t cap, int32_t* n);

/* Issues launch `step` of the prepared program (numbered as in
 * pdefa_amd_session_step_times) `iters` times back to back (after one warm-up
 * launch) between two HIP events on the session's stream; *out_ms = average
 * device time per launch.  Every launch is idempotent (it
 * reads its inputs and overwrites its outputs).  Requires one completed
 * engine_session_run. */
PDEFA_EXPORT EngineStatus pdefa_amd_session_step_repeat(EngineSession* sess, int32_t step, int32_t iters,
                                                        double* out_ms);

/* On-device letterbox input (no counterpart in the reference, whose
 * pdefa_preprocess_letterbox, imageloader/src/preprocess.cpp:15-144, runs on
 * the host): input `input_index` of the session becomes the letterbox of the
 * `count` images (batch = count, planar F32 [count, 3, target_h, target_w],
 * with cfg's target size, scale and pad value), computed on the GPU at the
 * next engine_session_run from the images' 8-bit pixels, which are copied
 * into pinned memory by this call (the images may be freed afterwards).
 * metas_out (count entries, may be NULL) receives each image's
 * PdefaPreprocessMeta, as pdefa_preprocess_letterbox would.  The values
 * equal pdefa_preprocess_letterbox's bit for bit.  engine_session_set_input
 * on the same index replaces it. */
PDEFA_EXPORT EngineStatus pdefa_amd_session_set_images(EngineSession* sess, int32_t input_index, int32_t count,
                                                       const PdefaImage* const* images,
                                                       const PdefaPreprocessConfig* cfg,
                                                       PdefaPreprocessMeta* metas_out);

/* A PdefaImage holding a copy of `width` x `height` interleaved 8-bit pixels
 * with `channels` = 1, 3 or 4 (no counterpart in the reference, which builds
 * images only by decoding files, pdefa_c_api.cpp:28-82); free it with
 * pdefa_image_free.  NULL on invalid arguments (pdefa_last_error says why). */
PDEFA_EXPORT PdefaImage* pdefa_amd_image_from_pixels(const uint8_t* pixels, int32_t width, int32_t height,
                                                     int32_t channels);

/* One detection of pdefa_amd_session_decode: the box in original-image
 * pixels (letterbox-mapped when a meta is given), score and class as the
 * reference's decode_yolo returns them (its Python floats are doubles), and
 * the head anchor the detection came from. */
typedef struct {
    double x1, y1, x2, y2, conf;
    int32_t cls;
    int32_t anchor;
} PdefaAmdDetection;

/* YOLO decode + per-class greedy NMS of output `output_index` of the last
 * engine_session_run, on the GPU (no counterpart in the reference, whose
 * decode_yolo runs in Python, pdefa/python/src/pdefa/_bindings.py:1095-1212,
 * with the same results: same detections, order and double values).  The
 * output must be a [N, 4 + classes, A] head resident from that run.  metas:
 * NULL (boxes stay in input pixels) or one PdefaPreprocessMeta per image
 * (n_metas == N).  dets receives N * max_det entries (image i's first
 * counts[i] entries at dets + i * max_det, best first); counts receives N.
 * At most 16384 anchors per image may pass conf_thres (ENGINE_ERR_RUNTIME
 * otherwise). */
PDEFA_EXPORT EngineStatus pdefa_amd_session_decode(EngineSession* sess, int32_t output_index,
                                                   const PdefaPreprocessMeta* metas, int32_t n_metas,
                                                   double conf_thres, double iou_thres, int32_t max_det,
                                                   PdefaAmdDetection* dets, int32_t* counts);

/* Text dump of the session's current device program (one line per kernel). */
PDEFA_EXPORT EngineStatus pdefa_amd_session_plan(const EngineSession* sess, char* buf, size_t cap, size_t* out_len);

/* The logical [N, C, H, W] input of the conv step that implements graph node
 * `node`, as the last run computed it, copied into dst (contiguous NCHW,
 * N*C*H*W floats, at most `cap`); dims receives N, C, H, W.  Needs a session
 * created with PDEFA_KEEP_TENSORS=1 in the environment, in which every
 * tensor keeps its own device memory (the program and its launch shapes
 * are the same as without it); ENGINE_ERR_INVALID_ARG otherwise or when no
 * conv step implements the node.  No counterpart in the reference (its
 * engine_session_debug_intermediate reads the NHWC tensors its own
 * interpreter keeps); tests use it to inspect a conv's inputs. */
PDEFA_EXPORT EngineStatus pdefa_amd_session_read_conv_input(EngineSession* sess, const char* node, float* dst,
                                                           size_t cap, int64_t* dims);

/* Plans `m` for inputs of the given shape without touching a GPU and returns
 * the program text (planner tests on hosts without a device).  With
 * PDEFA_PLAN_GROUP_ALL=1 in the environment, launch shapes come from the cost
 * model and every conv group the grouping pass offers is taken (a test of the
 * reordering that grouped launches imply). */
PDEFA_EXPORT EngineStatus pdefa_amd_plan_model(const EngineModel* m, const int64_t* shape, int32_t ndim, char* buf,
                                               size_t cap, size_t* out_len);

/* "<name> (<gcnArch>, <compute units> CUs, <memory> GiB)" of HIP device 0
 * ("AMD GPU" when the driver reports no marketing name), or "none". */
PDEFA_EXPORT const char* pdefa_amd_device_name(void);

/* engine_ops_matmul (same arguments, shape rules, results and error
 * behaviour) for callers that cannot allocate device memory (tight serving
 * loops, harnesses that forbid hipMalloc); it has no counterpart in the
 * reference.  Its device buffers
 * (A, B, B packed for the MFMA core, a zero bias, C and split-K partials)
 * live in a static 32 MiB scratch array that each GPU holds from the
 * library's load until the process ends: no hipMalloc, hipFree or other
 * allocating routine is called, and work is issued on the null stream.
 * A product whose buffers exceed the array (roughly 4 (MK + KN + MN)
 * bytes plus padding and partials > 32 MiB) returns ENGINE_ERR_INVALID_ARG
 * with a message saying so.  Every call on a GPU shares that GPU's array,
 * which keeps the last call's contents; calls in one process are
 * serialized by a lock, since overlapping calls on one GPU would race on
 * the array. */
PDEFA_EXPORT EngineStatus pdefa_amd_ops_matmul_noalloc(const EngineTensor* a, const EngineTensor* b,
                                                       EngineTensor* out);

/* Conv launch-shape choices made so far in this process: *measured = timed
 * on the device while planning, *from_table = read from the device kind's
 * launch-shape table (tuning/<arch>.txt beside the library directory, or
 * PDEFA_TUNE_TABLE).  A process whose choices all come from the table plans
 * the same launch shapes, hence the same results, as every other such
 * process. */
PDEFA_EXPORT EngineStatus pdefa_amd_tune_stats(int64_t* measured, int64_t* from_table);

/* Pre-pack cache files read (*read) and written (*written) by this process.
 * With PDEFA_PACK_CACHE=1 in the environment, a model loaded from an .engine
 * file keeps its packed conv weight layouts (implicit GEMM, direct and
 * Winograd) in "<engine path>.<gfx arch>.pack" beside it: the first load on a
 * device kind packs on the device and writes the file, later loads read it
 * when its header matches the weights, the layout and the architecture, and
 * pack again (rewriting it) when it does not.  The persisted counterpart of
 * the reference's in-memory, pointer-keyed pack caches, which it clears at
 * every model load (PDEFA1.0/src/loader/custom_loader.cpp:207-211). */
PDEFA_EXPORT EngineStatus pdefa_amd_pack_cache_stats(int64_t* read, int64_t* written);

#ifdef __cplusplus
}
#endif
#endif /* PDEFA_AMD_EXT_H */
