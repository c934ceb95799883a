// Bandwidth-bound kernels over strided views: elementwise/broadcast, max pool,
// nearest resize, softmax along an axis, and a direct convolution for layers
// the implicit-GEMM kernel does not take (arbitrary strides, tiny Cout).
//
// All kernels walk the logical output index with the innermost logical
// dimension fastest, except the NCHW-logical spatial kernels which walk
// (n, h, w, c) so that channels-last outputs are written contiguously.
#include "../kernels.hpp"
#include "act.hpp"

#include <algorithm>
#include <stdexcept>
#include <string>

namespace pdefa {
namespace k {

namespace {

unsigned grid_for(int64_t total, int block = 256) {
    const int64_t b = (total + block - 1) / block;
    return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(b, 1 << 20)));
}

void check_view(const View& v, const char* what) {
    if (!v.ptr) throw std::runtime_error(std::string("null view: ") + what);
    if (v.rank < 1 || v.rank > kMaxRank) throw std::runtime_error(std::string("bad view rank: ") + what);
}

int64_t numel(const View& v) {
    int64_t n = 1;
    for (int d = 0; d < v.rank; ++d) n *= v.dims[d];
    return n;
}

}  // namespace

__global__ __launch_bounds__(256) void eltwise_kernel(int op, View out, View a, View b, float alpha, int64_t total) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int64_t rem = i, oo = 0, ao = 0, bo = 0;
        for (int d = out.rank - 1; d >= 0; --d) {
            const int64_t n = out.dims[d];
            const int64_t idx = rem % n;
            rem /= n;
            oo += idx * out.str[d];
            ao += idx * a.str[d];
            bo += idx * b.str[d];
        }
        const float x = a.ptr[ao];
        float r;
        switch (op) {
            case kEltAdd: r = x + b.ptr[bo]; break;
            case kEltSub: r = x - b.ptr[bo]; break;
            case kEltMul: r = x * b.ptr[bo]; break;
            case kEltDiv: r = x / b.ptr[bo]; break;
            case kEltSigmoid: r = 1.0f / (1.0f + expf(-x)); break;
            case kEltRelu: r = x > 0.0f ? x : 0.0f; break;
            case kEltTanh: r = tanhf(x); break;
            case kEltLeaky: r = x > 0.0f ? x : x * alpha; break;
            case kEltSilu: r = x / (1.0f + expf(-x)); break;
            default: r = x; break;
        }
        out.ptr[oo] = r;
    }
}

void launch_eltwise(int op, const View& out, const View& a, const View& b, float alpha, hipStream_t s) {
    check_view(out, "eltwise out");
    check_view(a, "eltwise a");
    const bool binary = op == kEltAdd || op == kEltSub || op == kEltMul || op == kEltDiv;
    if (binary) check_view(b, "eltwise b");
    if (a.rank != out.rank || (binary && b.rank != out.rank)) throw std::runtime_error("eltwise: rank mismatch");
    const int64_t total = numel(out);
    if (total == 0) return;
    hipLaunchKernelGGL(eltwise_kernel, dim3(grid_for(total)), dim3(256), 0, s, op, out, a, binary ? b : a, alpha,
                       total);
}

__global__ __launch_bounds__(256) void maxpool_kernel(View out, View in, int kh, int kw, int sh, int sw, int ph,
                                                      int pw, int64_t total) {
    const int64_t N = out.dims[0], C = out.dims[1], Ho = out.dims[2], Wo = out.dims[3];
    const int64_t H = in.dims[2], W = in.dims[3];
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int64_t t = i;
        const int64_t c = t % C; t /= C;
        const int64_t wo = t % Wo; t /= Wo;
        const int64_t ho = t % Ho;
        const int64_t n = t / Ho;
        (void)N;
        const float* base = in.ptr + n * in.str[0] + c * in.str[1];
        float m = -3.402823466e+38f;
        for (int a = 0; a < kh; ++a) {
            const int64_t hi = ho * sh - ph + a;
            if (hi < 0 || hi >= H) continue;
            for (int b = 0; b < kw; ++b) {
                const int64_t wi = wo * sw - pw + b;
                if (wi < 0 || wi >= W) continue;
                const float v = base[hi * in.str[2] + wi * in.str[3]];
                m = v > m ? v : m;
            }
        }
        out.ptr[n * out.str[0] + c * out.str[1] + ho * out.str[2] + wo * out.str[3]] = m;
    }
}

void launch_maxpool(const View& out, const View& in, int kh, int kw, int sh, int sw, int ph, int pw, hipStream_t s) {
    check_view(out, "maxpool out");
    check_view(in, "maxpool in");
    if (out.rank != 4 || in.rank != 4) throw std::runtime_error("maxpool: rank 4 views expected");
    if (out.dims[0] != in.dims[0] || out.dims[1] != in.dims[1]) throw std::runtime_error("maxpool: N/C mismatch");
    const int64_t total = numel(out);
    if (total == 0) return;
    hipLaunchKernelGGL(maxpool_kernel, dim3(grid_for(total)), dim3(256), 0, s, out, in, kh, kw, sh, sw, ph, pw, total);
}

__global__ __launch_bounds__(256) void resize_nearest_kernel(View out, View in, float ry, float rx, int64_t total) {
    const int64_t C = out.dims[1], Ho = out.dims[2], Wo = out.dims[3];
    const int64_t H = in.dims[2], W = in.dims[3];
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int64_t t = i;
        const int64_t c = t % C; t /= C;
        const int64_t wo = t % Wo; t /= Wo;
        const int64_t ho = t % Ho;
        const int64_t n = t / Ho;
        int64_t hi = static_cast<int64_t>(static_cast<float>(ho) * ry);
        int64_t wi = static_cast<int64_t>(static_cast<float>(wo) * rx);
        hi = hi < H - 1 ? hi : H - 1;
        wi = wi < W - 1 ? wi : W - 1;
        out.ptr[n * out.str[0] + c * out.str[1] + ho * out.str[2] + wo * out.str[3]] =
            in.ptr[n * in.str[0] + c * in.str[1] + hi * in.str[2] + wi * in.str[3]];
    }
}

void launch_resize_nearest(const View& out, const View& in, hipStream_t s) {
    check_view(out, "resize out");
    check_view(in, "resize in");
    if (out.rank != 4 || in.rank != 4) throw std::runtime_error("resize: rank 4 views expected");
    if (out.dims[0] != in.dims[0] || out.dims[1] != in.dims[1]) throw std::runtime_error("resize: N/C mismatch");
    const float ry = static_cast<float>(in.dims[2]) / static_cast<float>(out.dims[2]);
    const float rx = static_cast<float>(in.dims[3]) / static_cast<float>(out.dims[3]);
    const int64_t total = numel(out);
    if (total == 0) return;
    hipLaunchKernelGGL(resize_nearest_kernel, dim3(grid_for(total)), dim3(256), 0, s, out, in, ry, rx, total);
}

__global__ __launch_bounds__(256) void softmax_kernel(View out, View in, int axis, int64_t rows) {
    const int64_t L = in.dims[axis];
    for (int64_t r = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; r < rows;
         r += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int64_t rem = r, io = 0, oo = 0;
        for (int d = in.rank - 1; d >= 0; --d) {
            if (d == axis) continue;
            const int64_t idx = rem % in.dims[d];
            rem /= in.dims[d];
            io += idx * in.str[d];
            oo += idx * out.str[d];
        }
        const int64_t is = in.str[axis], os = out.str[axis];
        float mx = -1e30f;
        for (int64_t j = 0; j < L; ++j) {
            const float v = in.ptr[io + j * is];
            mx = v > mx ? v : mx;
        }
        float sum = 0.0f;
        for (int64_t j = 0; j < L; ++j) {
            const float e = expf(in.ptr[io + j * is] - mx);
            out.ptr[oo + j * os] = e;
            sum += e;
        }
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (int64_t j = 0; j < L; ++j) out.ptr[oo + j * os] *= inv;
    }
}

void launch_softmax(const View& out, const View& in, int axis, hipStream_t s) {
    check_view(out, "softmax out");
    check_view(in, "softmax in");
    if (out.rank != in.rank || axis < 0 || axis >= in.rank) throw std::runtime_error("softmax: bad axis/rank");
    const int64_t rows = numel(in) / std::max<int64_t>(1, in.dims[axis]);
    if (rows == 0) return;
    hipLaunchKernelGGL(softmax_kernel, dim3(grid_for(rows)), dim3(256), 0, s, out, in, axis, rows);
}

__global__ __launch_bounds__(256) void conv_direct_kernel(ConvDirectArgs a, int64_t total) {
    const int64_t Co = a.y.dims[1], Ho = a.y.dims[2], Wo = a.y.dims[3];
    const int64_t Ci = a.x.dims[1], H = a.x.dims[2], W = a.x.dims[3];
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int64_t t = i;
        const int64_t co = t % Co; t /= Co;
        const int64_t wo = t % Wo; t /= Wo;
        const int64_t ho = t % Ho;
        const int64_t n = t / Ho;
        float acc = 0.0f;
        const float* xb = a.x.ptr + n * a.x.str[0];
        const float* wb = a.w + co * Ci * a.KH * a.KW;
        for (int64_t c = 0; c < Ci; ++c) {
            for (int kh = 0; kh < a.KH; ++kh) {
                const int64_t hi = ho * a.sh - a.ph + kh * a.dh;
                if (hi < 0 || hi >= H) continue;
                for (int kw = 0; kw < a.KW; ++kw) {
                    const int64_t wi = wo * a.sw - a.pw + kw * a.dw;
                    if (wi < 0 || wi >= W) continue;
                    acc += xb[c * a.x.str[1] + hi * a.x.str[2] + wi * a.x.str[3]] *
                           wb[(c * a.KH + kh) * a.KW + kw];
                }
            }
        }
        if (a.bias) acc += a.bias[co];
        float v = apply_act(acc, a.act, a.slope);
        if (a.res.ptr) v += a.res.ptr[n * a.res.str[0] + co * a.res.str[1] + ho * a.res.str[2] + wo * a.res.str[3]];
        a.y.ptr[n * a.y.str[0] + co * a.y.str[1] + ho * a.y.str[2] + wo * a.y.str[3]] = v;
    }
}

void launch_conv_direct(const ConvDirectArgs& a, hipStream_t s) {
    check_view(a.x, "conv_direct x");
    check_view(a.y, "conv_direct y");
    if (!a.w) throw std::runtime_error("conv_direct: null weights");
    if (a.x.rank != 4 || a.y.rank != 4) throw std::runtime_error("conv_direct: rank 4 views expected");
    const int64_t total = numel(a.y);
    if (total == 0) return;
    hipLaunchKernelGGL(conv_direct_kernel, dim3(grid_for(total)), dim3(256), 0, s, a, total);
}

}  // namespace k
}  // namespace pdefa
