// Shared pieces of the two Winograd F(2x2,3x3) kernels (conv_wino.hip: a
// 2-D tile block per workgroup with its patch region staged in LDS;
// conv_wino_strip.hip: a strip of 32 tiles whose lanes load their own patch
// rows): types, limits, byte-extent helpers.  Included only by those files.
#pragma once

#include "../kernels.hpp"

#include <cstdint>
#include <stdexcept>
#include <string>

namespace pdefa {
namespace k {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int uintx4 __attribute__((ext_vector_type(4)));

namespace wino {

constexpr int kWT = 32;  // tiles per workgroup (GEMM rows)
constexpr int kCK = 8;   // input channels per K step (4 per lane half)
constexpr int kXcds = 8;
constexpr int kMaxCin = 4096;
// Input, weights, output and residual are addressed by 32-bit byte offsets
// from their base.  Their spans stay under kWinoMaxViewBytes, so an offset
// derived from kWinoNoPixel (less up to 16 bytes, or plus a valid offset, or
// plus itself) always lands past the buffer range.
constexpr int32_t kWinoNoPixel = 1 << 30;
constexpr int32_t kWinoMaxViewBytes = kWinoNoPixel - 4096;
// buffer resource word 3 for raw 32-bit buffer access
constexpr int kWinoBufferFlags = 0x00020000;

inline int wino_cin_pad(int Cin) { return (Cin + kCK - 1) / kCK * kCK; }
inline int wino_cout_pad(int Cout) { return (Cout + 63) / 64 * 64; }

[[noreturn]] inline void fail(const std::string& m) { throw std::runtime_error("conv_wino: " + m); }
// Bytes from a view's base to the end of its last element.
inline int64_t view_bytes(int N, int H, int W, int C, int64_t sn, int64_t sh, int64_t sw) {
    return 4 * ((N - 1) * sn + (H - 1) * sh + (W - 1) * sw + C);
}

// n / d for 0 <= n < 2^31 (kernels.hpp FastDiv)
__device__ __forceinline__ int wdiv(int n, FastDiv f) {
    return static_cast<int>((static_cast<uint64_t>(static_cast<uint32_t>(n)) * f.m) >> f.s);
}

// Byte extents of the input, transformed weights, output and residual.
struct WinoBytes {
    int x, u, y, r;
    int vec;  // outputs (and residuals) as 16-byte runs
};

}  // namespace wino

// The strip kernel's launch (conv_wino_strip.hip): bn = 64 output channels
// a workgroup (the only width it is built for), tiles_h x tiles_w tiles per
// image, the shape checks already made by launch_conv_wino.
void launch_conv_wino_strip(const ConvArgs& a, int bn, int tiles_h, int tiles_w, wino::WinoBytes b, hipStream_t s);

}  // namespace k
}  // namespace pdefa
