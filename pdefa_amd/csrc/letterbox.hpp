// Letterbox geometry of imageloader/src/preprocess.cpp:15-35 (the reference's
// preprocess_letterbox_direct), shared by the host letterbox and the device
// path: ratio = min(tw/w, th/h) in fp32, scaled size = clamp(round(src *
// ratio), 1, target) with std::round (halves away from zero), centred
// integer pads.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstdint>

namespace pdefa {

struct LetterboxGeometry {
    float ratio = 1.0f;
    int32_t scaled_w = 0, scaled_h = 0, pad_x = 0, pad_y = 0;
};

inline LetterboxGeometry letterbox_geometry(int32_t src_w, int32_t src_h, int32_t tw, int32_t th) {
    LetterboxGeometry g;
    g.ratio = std::min(static_cast<float>(tw) / static_cast<float>(src_w),
                       static_cast<float>(th) / static_cast<float>(src_h));
    g.scaled_w = std::clamp(static_cast<int>(std::round(static_cast<float>(src_w) * g.ratio)), 1, tw);
    g.scaled_h = std::clamp(static_cast<int>(std::round(static_cast<float>(src_h) * g.ratio)), 1, th);
    g.pad_x = (tw - g.scaled_w) / 2;
    g.pad_y = (th - g.scaled_h) / 2;
    return g;
}

// One output value of the bilinear blend
// (p00 w0 + p10 w1) wy0 + (p01 w0 + p11 w1) wy1 of preprocess.cpp:106-120,
// rounded as the reference's own build evaluates it: GCC contracts each
// a * b + c * d there into fma(a, b, c * d) (imageloader/CMakeLists.txt:41
// compiles with -mfma, and GCC's default contraction fuses the first product
// of each sum).  Host and device use this one function, so the device tensor
// equals pdefa_preprocess_letterbox's, and the reference's, bit for bit.
#if defined(__HIPCC__) || defined(__HIP__)
__host__ __device__
#endif
inline float letterbox_blend(float p00, float p10, float p01, float p11, float w0, float w1, float wy0, float wy1) {
#pragma clang fp contract(off)
    const float top = std::fma(p00, w0, p10 * w1);
    const float bot = std::fma(p01, w0, p11 * w1);
    return std::fma(top, wy0, bot * wy1);
}

// One interleaved 8-bit image (1, 3 or 4 channels; channels 0..2 are used).
struct ImageRef {
    const uint8_t* pixels = nullptr;
    int32_t width = 0, height = 0, channels = 0;
};

}  // namespace pdefa
