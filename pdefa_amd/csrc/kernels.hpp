// Launch interface between the host runtime and the HIP kernels (gfx950).
// Everything here is plain structs of device pointers, sizes and strides; the
// launchers check the shapes they are given before launching.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

namespace pdefa {
namespace k {

constexpr int kMaxRank = 6;

// A strided view of fp32 device memory.  dims/str are in elements; the view's
// element (i0..i{r-1}) lives at ptr[sum i_d * str_d].  Strides may be 0
// (broadcast) on inputs.
struct View {
    float* ptr = nullptr;
    int32_t rank = 0;
    int64_t dims[kMaxRank] = {0, 0, 0, 0, 0, 0};
    int64_t str[kMaxRank] = {0, 0, 0, 0, 0, 0};
};

// Fused epilogue activation codes.  1-5 follow the reference's
// Conv2dConfig::FusedActivation numbering (PDEFA1.0/include/engine/ops/conv2d.hpp:16-24).
// 6-8 are what some of the reference's conv kernels evaluate for codes 5, 4
// and 3 (the planner picks them by the reference's dispatch rule):
//   6  the SiLU form of its Winograd epilogue
//      (PDEFA1.0/src/kernels/simd/avx2/conv2d_winograd.cpp:81-101);
//   7  tanh-form GELU, 0.5 v (1 + tanh(0.7978845608 (v + 0.044715 v^3))),
//      which its Winograd and direct kernels apply for code 4
//      (conv2d_winograd.cpp:108-111, conv2d_avx2.cpp:109-112);
//   8  1 / (1 + v), which its direct kernel applies for code 3
//      (PDEFA1.0/src/kernels/simd/avx2/conv2d_avx2.cpp:99-103).
enum Act : int32_t {
    kActNone = 0,
    kActRelu = 1,
    kActLeaky = 2,
    kActSigmoid = 3,
    kActTanh = 4,
    kActSilu = 5,
    kActSiluWinogradForm = 6,
    kActGeluTanh = 7,
    kActRecip1p = 8,
};

// Implicit-GEMM convolution tile configurations.  A workgroup is 4 or 8 waves
// and computes a BM x BN output tile; each wave owns a WM x WN sub-tile of 32x32
// MFMA blocks (16x16 blocks where WM or WN is 16) and one of KG interleaved K
// slices.  KG > 1 splits K across the
// waves of one workgroup (partial tiles summed through LDS in slice order),
// which multiplies the workgroup count of small layers without any
// cross-workgroup traffic.
struct ConvTileShape {
    int bm, bn, wm, wn, kg;
};
enum ConvTile : int32_t {
    kTile128x128 = 0,   // 2x2 waves of 64x64
    kTile128x64 = 1,    // 2x2 waves of 64x32
    kTile64x128 = 2,    // 2x2 waves of 32x64
    kTile64x64 = 3,     // 2x2 waves of 32x32
    kTile128x32 = 4,    // 4x1 waves of 32x32
    kTile64x32K2 = 5,   // 2x1 waves of 32x32, K split in 2
    kTile32x64K2 = 6,   // 1x2 waves of 32x32, K split in 2
    kTile32x32K4 = 7,   // 1 wave tile of 32x32, K split in 4
    // 8-wave workgroups (512 lanes, two waves per SIMD): one wave's LDS round
    // trip and barrier wait overlap the other's MFMAs
    kTile128x64W8 = 8,     // 4x2 waves of 32x32
    kTile64x64K2W8 = 9,    // 2x2 waves of 32x32, K split in 2
    kTile128x128W8 = 10,   // 2x4 waves of 64x32
    kTile64x128W8 = 11,    // 2x4 waves of 32x32
    kTile32x64K4W8 = 12,   // 1x2 waves of 32x32, K split in 4
    kTile32x32K8W8 = 13,   // 1 wave tile of 32x32, K split in 8 (small-M, long-K layers)
    // Winograd F(2x2,3x3) kernel (3x3 stride-1 convs), 32 tiles x BN channels
    kTileWino64 = 14,
    kTileWino32 = 15,
    // Small tiles on the 16x16x4 MFMA (v_mfma_f32_16x16x4_f32) for layers
    // whose 32x32 tile grid leaves most of the 256 CUs idle (batch 1 at
    // 20x20 to 40x40): four times the workgroups of 32x32k4 at the same K
    // split, a quarter of the MFMA chain per pipeline step.
    kTile16x16K4 = 16,     // 1 wave tile of 16x16, K split in 4
    kTile16x32K4 = 17,     // 1 wave tile of 16x32, K split in 4
    kTile32x16K4 = 18,     // 1 wave tile of 32x16, K split in 4
    kTile16x32K8W8 = 19,   // 1 wave tile of 16x32, K split in 8
    kTile32x16K8W8 = 20,   // 1 wave tile of 32x16, K split in 8
    kNumConvShapes = 21,   // tile ids (implicit-GEMM and Winograd)
};
inline bool is_wino_tile(int tile) { return tile == kTileWino64 || tile == kTileWino32; }
// An implicit-GEMM tile id (conv_mfma_kernel).
inline bool is_gemm_tile(int tile) { return tile >= 0 && tile < kNumConvShapes && !is_wino_tile(tile); }
ConvTileShape conv_tile_shape(int tile);
const char* conv_tile_name(int tile);

// Packed conv weights: [ceil(Cout/32)][ceil(K/32)][32 co][32 k] with
// k = (kh*KW + kw)*Cin + ci, zero padded.  32-wide blocks serve every tile.
constexpr int kConvBK = 32;
constexpr int kConvBN = 32;

// NHWC implicit GEMM: M = N*Ho*Wo, Ncol = Cout, K = KH*KW*Cin with k ordered
// (kh, kw, ci).  Input/output/residual are channels-last views (channel stride
// 1) described by their n/h/w strides.
// Division of 0 <= n < 2^31 by a launch-invariant divisor 1 <= d < 2^31 as
// one 32x32 -> 64-bit multiply and a shift: q = (n * m) >> s with
// s = 31 + ceil(log2 d) and m = ceil(2^s / d), which is below 2^32.  Exact:
// with m d = 2^s + e, 0 <= e < d, n m / 2^s = n / d + n e / (d 2^s) and
// n e / (d 2^s) < 2^(31 - s) <= 1 / d, too little to reach the next integer.
struct FastDiv {
    uint32_t m = 0x80000000u;  // d = 1
    uint32_t s = 31;
};
inline FastDiv make_fastdiv(int64_t d) {
    FastDiv f;
    if (d < 1 || d >= (int64_t{1} << 31)) return f;  // callers check their divisors' range
    uint32_t l = 0;
    while ((int64_t{1} << l) < d) ++l;
    f.s = 31 + l;
    f.m = static_cast<uint32_t>(((uint64_t{1} << f.s) + static_cast<uint64_t>(d) - 1) / static_cast<uint64_t>(d));
    return f;
}

struct ConvArgs {
    const float* x = nullptr;
    int64_t x_sn = 0, x_sh = 0, x_sw = 0;
    int32_t N = 0, H = 0, W = 0, Cin = 0;
    float* y = nullptr;
    int64_t y_sn = 0, y_sh = 0, y_sw = 0;
    int32_t Ho = 0, Wo = 0, Cout = 0;
    const float* res = nullptr;  // optional residual added after the activation
    int64_t r_sn = 0, r_sh = 0, r_sw = 0;
    const float* wpk = nullptr;
    const float* bias = nullptr;  // >= Cout floats
    // the K-major packed weights (the layout above; the same as wpk on the
    // implicit-GEMM path, the Winograd path's wpk holds U): with act ==
    // kActSiluWinogradForm the epilogue recomputes outputs next to a jump of
    // that SiLU from them in float64 (kernels/jump_fix.hpp); nullptr skips it.
    // jump_window: the flagged band's half-width relative to
    // max(1, |x log2 e|) (kJumpWindow; 0.5 flags every output)
    const float* w_kmaj = nullptr;
    float jump_window = 1.52587890625e-05f;
    int32_t KH = 1, KW = 1, sh = 1, sw = 1, ph = 0, pw = 0, dh = 1, dw = 1;
    int32_t K = 0;        // KH*KW*Cin
    int32_t ktiles = 0;   // ceil(K / 32): 32-wide K blocks of the packed weights
    int32_t act = 0;
    float slope = 0.01f;
    // split-K across workgroups: splits > 1 writes raw partial sums to
    // ws[split][M][Cout] (split z covers K blocks [z*kt_per_split, ...)) and a
    // reduce kernel sums them in split order, then applies the epilogue.
    float* ws = nullptr;
    int32_t splits = 1;
    int32_t kt_per_split = 0;  // multiple of the tile's KG
    // groups > 1: a grouped convolution.  Cin, Cout, K and ktiles are then per
    // group: group g reads input channels [g*Cin, (g+1)*Cin), writes output
    // channels [g*Cout, (g+1)*Cout) (and the same channels of res and up),
    // takes packed weights wpk + g*w_group and biases bias + g*Cout; the grid
    // runs splits*groups in z and a split-K workspace holds
    // [groups][splits][M][Cout].
    int32_t groups = 1;
    int64_t w_group = 0;
    // optional nearest 2x upsample of the result, written alongside y:
    // up[n, 2ho + i, 2wo + j, co] = y[n, ho, wo, co] for i, j in {0, 1}
    // (channels-last, n/h/w strides), e.g. straight into a concat buffer
    float* up = nullptr;
    int64_t u_sn = 0, u_sh = 0, u_sw = 0;
    // divisors of the implicit-GEMM kernel's index arithmetic, set by its
    // launchers: Ho*Wo, Wo, Cin, KW, and the grid's m tiles, m*n tiles and
    // splits
    FastDiv fd_howo, fd_wo, fd_cin, fd_kw, fd_gx, fd_gxy, fd_splits;
};

// Tile and split-K choice for an implicit GEMM of this shape on the 256 CUs.
struct ConvLaunchShape {
    int tile = kTile64x64;
    int splits = 1;
    int kt_per_split = 0;
};
ConvLaunchShape conv_select(int64_t M, int Cout, int K, bool allow_split, bool wino_ok = false, int Cin = 0);
// Every tile with one split and with its best split count (and, with
// wino_ok, the Winograd kernel for a 3x3 stride-1 layer of Cin channels),
// cheapest predicted first (conv_select is the first); the candidates a
// measured choice times.
std::vector<ConvLaunchShape> conv_candidates(int64_t M, int Cout, int K, bool allow_split, bool wino_ok = false,
                                             int Cin = 0);

// Host-side checks + launch.  vec selects 16-byte input loads (requires
// Cin % 4 == 0 and 16-byte aligned pixel rows).
void launch_conv_mfma(const ConvArgs& a, int tile, bool vec, hipStream_t s);

// Independent convolutions (no split-K, vector loads) issued as one launch of
// one tile shape: workgroups of every problem run side by side, so several
// small layers fill the chip together instead of one after another.
constexpr int kMaxConvGroup = 8;
struct ConvGroupArgs {
    int32_t count = 0;
    int32_t tile_begin[kMaxConvGroup + 1] = {};  // prefix sums of the problems' tile counts
    int32_t m_tiles[kMaxConvGroup] = {};         // m blocks of each problem
    ConvArgs p[kMaxConvGroup];
};
static_assert(sizeof(ConvGroupArgs) <= 4096, "grouped launch arguments must fit the 4 KiB kernel-argument segment");
void launch_conv_mfma_group(const ConvArgs* probs, int count, int tile, hipStream_t s);

// Winograd F(2x2,3x3) on MFMA for 3x3 / stride 1 / dilation 1 convs with
// Cin % 4 == 0 and Cin >= 8 (any padding).  a.wpk holds the transformed
// weights U = G g G^T as [16][ceil(Cin/8)*2][ceil(Cout/64)*64][4]
// (launch_pack_wino_weights from the OIHW weights); splits must be 1.
// bn = 32 or 64 output channels per workgroup.  Input, transformed weights,
// output and residual are addressed by 32-bit byte offsets: each must span
// less than 1 GiB - 4 KiB (wino_views_fit), with non-negative strides.
bool wino_eligible(int KH, int KW, int sh, int sw, int dh, int dw, int Cin);
bool wino_views_fit(const ConvArgs& a);
int64_t wino_packed_elems(int Cout, int Cin);
void launch_conv_wino(const ConvArgs& a, int bn, hipStream_t s);
void launch_pack_wino_weights(float* dst, const float* w_oihw, int Cout, int Cin, hipStream_t s);

// Direct convolution over arbitrary strided NCHW-logical views (any layout),
// for layers the implicit GEMM does not take: tiny Cin (the 3-channel stem,
// read straight from the NCHW input) or tiny Cout.  One lane computes one
// output pixel for a block of direct_cb(Cout) output channels; the workgroup
// writes its tile through LDS so that stores are coalesced along channels.
inline int direct_cb(int Cout) { return Cout <= 16 ? 16 : (Cout <= 32 ? 32 : (Cout <= 48 ? 48 : 64)); }
struct ConvDirectArgs {
    View x;    // logical [N, Cin, H, W]
    View y;    // logical [N, Cout, Ho, Wo]
    View res;  // optional, same logical shape as y (ptr == nullptr if absent)
    const float* wpk = nullptr;  // [ceil(Cout/CB)][Cin*KH*KW][CB], CB = direct_cb(Cout), k = (ci, kh, kw)
    const float* bias = nullptr;
    int32_t KH = 1, KW = 1, sh = 1, sw = 1, ph = 0, pw = 0, dh = 1, dw = 1;
    int32_t act = 0;
    float slope = 0.01f;
    // groups > 1: grouped convolution with Cin/groups input channels per
    // group (depthwise when that is 1); wpk is then [KH*KW][Cin/groups][Cout]
    // (output channel fastest, k::grouped_direct_packed_elems)
    int32_t groups = 1;
};
void launch_conv_direct(const ConvDirectArgs& a, hipStream_t s);
inline int64_t grouped_direct_packed_elems(int Cout, int Cin_g, int KH, int KW) {
    return static_cast<int64_t>(KH) * KW * Cin_g * Cout;
}
// Packs OIHW weights [Cout][Cin_g][KH][KW] (device, contiguous) into the
// direct-kernel layout of ConvDirectArgs::wpk (grouped when groups > 1).
void launch_pack_direct_weights(float* dst, const float* w, int Cout, int Cin_g, int KH, int KW, int groups,
                                hipStream_t s);

// Letterbox of one interleaved 8-bit image (ch = 1, 3 or 4) into the planar
// fp32 tensor dst[3][th][tw]: the scaled window (sw x sh at px, py) is
// bilinear-sampled with inv = 1/ratio, the rest is `pad`.
struct LetterboxArgs {
    const uint8_t* src = nullptr;
    int32_t w = 0, h = 0, ch = 0;
    float* dst = nullptr;
    int32_t tw = 0, th = 0, sw = 0, sh = 0, px = 0, py = 0;
    float inv = 1.0f, scale = 1.0f, pad = 0.0f;
};
void launch_letterbox(const LetterboxArgs& a, hipStream_t s);

// YOLO head decode + per-class greedy NMS (the reference's decode_yolo in
// float64), per image of a [N, 4 + classes, A] head; see yolo_decode.hip.
struct YoloDetection {
    double x1, y1, x2, y2, conf;
    int32_t cls, anchor;
};
constexpr int kYoloMaxCandidates = 16384;  // anchors passing conf_thres per image
struct YoloDecodeArgs {
    const float* out = nullptr;  // head element (n, c, a) at out[n*sn + c*sc + a*sa]
    int64_t sn = 0, sc = 0, sa = 0;
    int32_t N = 0, C = 0, A = 0;
    double conf = 0.25, iou = 0.45;
    int32_t max_det = 300;
    int32_t max_cand = 0, max_cand_pow2 = 0;  // candidate capacity (<= A) and its power-of-two ceiling
    const double* meta = nullptr;  // per image: ratio, pad_x, pad_y, orig_w, orig_h; nullptr = no mapping
    // workspace, per image: boxes [A][4], class [A], keys [A], run info [A]; counts [N]
    double* boxes = nullptr;
    int32_t* cls = nullptr;
    unsigned long long* keys = nullptr;
    int32_t* seg = nullptr;
    int32_t* counts = nullptr;
    // results: dets [N][max_det], ndet [N] (-1: more than max_cand candidates)
    YoloDetection* dets = nullptr;
    int32_t* ndet = nullptr;
};
void launch_yolo_decode(const YoloDecodeArgs& a, hipStream_t s);

// Elementwise over out's logical shape; a/b are broadcast views of the same rank.
enum EltOp : int32_t {
    kEltCopy = 0,
    kEltAdd = 1,
    kEltSub = 2,
    kEltMul = 3,
    kEltDiv = 4,
    kEltSigmoid = 5,
    kEltRelu = 6,
    kEltTanh = 7,
    kEltLeaky = 8,
    kEltSilu = 9,
};
void launch_eltwise(int op, const View& out, const View& a, const View& b, float alpha,
                    hipStream_t s);

// Max pooling over logical [N, C, H, W] views (padding never wins).
void launch_maxpool(const View& out, const View& in, int kh, int kw, int sh, int sw, int ph,
                    int pw, hipStream_t s);

// Nearest resize over logical [N, C, H, W] views: src = min(floor(dst * in/out), in-1)
// with the ratio computed in fp32 as the reference does.
void launch_resize_nearest(const View& out, const View& in, hipStream_t s);

// Softmax along `axis` of the logical shape.
void launch_softmax(const View& out, const View& in, int axis, hipStream_t s);

// TopK along `axis` (PDEFA1.0/src/core/session_parts/session_ops_math.inc:321-395):
// the k largest values of each row in descending order, ties broken by the
// lower index; `out` receives the values, or with `indices` the indices as
// float values (exact: the axis is at most kTopKMaxAxis long).  One
// workgroup sorts one row in LDS.
constexpr int64_t kTopKMaxAxis = 16384;
void launch_topk(const View& out, const View& in, int axis, int64_t k, bool indices, hipStream_t s);

// GatherElements along `axis` (session_ops_math.inc:397-432): out[...] =
// data[... with the axis coordinate replaced by idx[...]]; indices are read
// as float values truncated toward zero, negative ones count from the end,
// and ones still out of range read element 0 of the axis.  idx and out have
// the data's extents off the axis.
void launch_gather_elements(const View& out, const View& data, const View& idx, int axis, hipStream_t s);

// Three chained stride-1 "same" max pools of kernel k (the SPPF block) in one
// pass: out0 = pool_k(in), out1 = pool_k(out0) = pool_{2k-1}(in),
// out2 = pool_k(out1) = pool_{3k-2}(in) (max composes exactly; padding never
// wins).  Logical [N, C, H, W] views.
void launch_maxpool_chain(const View& out0, const View& out1, const View& out2, const View& in, int k,
                          hipStream_t s);

// YOLOv8 box decode, the Detect head's DFL + dist2bbox subgraph in one pass:
// per anchor a and side s, softmax over the R bins of x[n, :, s, a], expected
// bin d_s = sum_b p_b * w_b (+ bias) (the 1x1 DFL conv), then with
// (ax, ay) = anchors[n, :, a]: x1 = ax - d0, y1 = ay - d1, x2 = ax + d2,
// y2 = ay + d3, out[n, :, a] = ((x1 + x2) / two, (y1 + y2) / two, x2 - x1,
// y2 - y1) * strides[n, :, a] -- the same fp32 operations, in the same order,
// as the unfused Softmax, Conv, Sub, Add, Add, Div, Sub, Concat, Mul nodes.
struct DetectDecodeArgs {
    View x;        // [N, R, 4, A]
    View anchors;  // [N, 2, A] (broadcast)
    View two;      // [N, 2, A] (broadcast)
    View strides;  // [N, 4, A] (broadcast)
    View out;      // [N, 4, A]
    const float* dfl_w = nullptr;  // R floats
    float dfl_bias = 0.0f;
    int32_t bins = 16;
    // optional (cls.ptr != nullptr): cls_out = sigmoid(cls), both [N, C, A];
    // one pass over the head rows when each anchor's row holds its 4*16 box
    // bins followed by its C class scores
    View cls;
    View cls_out;
};
void launch_detect_decode(const DetectDecodeArgs& a, hipStream_t s);

// Packs conv weights [Cout, Cin, KH, KW] (device, contiguous) into the packed
// layout above.
void launch_pack_conv_weights(float* dst, const float* w, int Cout, int Cin, int KH, int KW, hipStream_t s);
// Packs a row-major B[K, N] matrix the same way (a 1x1 conv with Cin = K).
void launch_pack_gemm_b(float* dst, const float* b, int K, int N, hipStream_t s);

// Elements of packed weights.
int64_t packed_weight_elems(int Cout, int K);
// Elements of direct-conv packed weights.
inline int64_t direct_packed_elems(int Cout, int K) {
    const int cb = direct_cb(Cout);
    return static_cast<int64_t>((Cout + cb - 1) / cb) * K * cb;
}

}  // namespace k
}  // namespace pdefa
