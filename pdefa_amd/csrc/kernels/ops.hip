// Bandwidth-bound kernels over strided views: elementwise/broadcast, max pool,
// nearest resize, softmax along an axis, and a direct convolution for layers
// the implicit-GEMM kernel does not take (arbitrary strides, tiny Cout).
//
// All kernels walk the logical output index with the innermost logical
// dimension fastest, except the NCHW-logical spatial kernels which walk
// (n, h, w, c) so that channels-last outputs are written contiguously.
#include "../letterbox.hpp"
#include "../kernels.hpp"
#include "act.hpp"

#include <algorithm>
#include <cstdlib>
#include <mutex>
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

// Views with every offset inside int32 take the int32 instantiations (the
// index decomposition is most of the work of these kernels).
template <typename I>
struct IView {
    float* ptr;
    int32_t rank;
    I dims[kMaxRank];
    I str[kMaxRank];
};

template <typename I>
IView<I> iview(const View& v) {
    IView<I> r{};
    r.ptr = v.ptr;
    r.rank = v.rank;
    for (int d = 0; d < kMaxRank; ++d) {
        r.dims[d] = static_cast<I>(v.dims[d]);
        r.str[d] = static_cast<I>(v.str[d]);
    }
    return r;
}

// True when every element offset of the view (and its element count) fits in int32.
bool fits_i32(const View& v) {
    int64_t ext = 0, n = 1;
    for (int d = 0; d < v.rank; ++d) {
        if (v.dims[d] <= 0) return true;
        ext += (v.dims[d] - 1) * (v.str[d] < 0 ? -v.str[d] : v.str[d]);
        n *= v.dims[d];
    }
    return ext < (int64_t{1} << 31) && n < (int64_t{1} << 31);
}

// Logistic sigmoid, as the Sigmoid operator evaluates it.
__device__ __forceinline__ float sigmoid_elt(float x) { return 1.0f / (1.0f + expf(-x)); }

// One element of an elementwise op (y: the second operand, unused by unary ops).
__device__ __forceinline__ float elt_apply(int op, float x, float y, float alpha) {
    switch (op) {
        case kEltAdd: return x + y;
        case kEltSub: return x - y;
        case kEltMul: return x * y;
        case kEltDiv: return x / y;
        case kEltSigmoid: return sigmoid_elt(x);
        case kEltRelu: return x > 0.0f ? x : 0.0f;
        case kEltTanh: return tanhf(x);
        case kEltLeaky: return x > 0.0f ? x : x * alpha;
        case kEltSilu: return x / (1.0f + expf(-x));
        default: return x;
    }
}

template <typename I>
__global__ __launch_bounds__(256) void eltwise_kernel(int op, IView<I> out, IView<I> a, IView<I> b, float alpha,
                                                      I total) {
    for (I i = blockIdx.x * static_cast<I>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<I>(gridDim.x) * blockDim.x) {
        I rem = i, oo = 0, ao = 0, bo = 0;
        for (int d = out.rank - 1; d >= 0; --d) {
            const I n = out.dims[d];
            const I idx = rem % n;
            rem /= n;
            oo += idx * out.str[d];
            ao += idx * a.str[d];
            bo += idx * b.str[d];
        }
        out.ptr[oo] = elt_apply(op, a.ptr[ao], b.ptr[bo], alpha);
    }
}

// The three views of an elementwise op with adjacent dims merged wherever
// every view is contiguous across them (and size-1 dims dropped), innermost
// last: most graph tensors collapse to one or two dims.
struct EltDims {
    int32_t rank = 0;
    int32_t dims[kMaxRank] = {};
    int32_t so[kMaxRank] = {}, sa[kMaxRank] = {}, sb[kMaxRank] = {};
};

// Float4 form: the innermost collapsed dim is contiguous in out and a (and in
// b, or b is constant along it: b_splat) and a multiple of 4 long, every
// base and outer stride 16-byte aligned; one lane per 4 consecutive elements,
// each computed exactly as eltwise_kernel computes it.
__global__ __launch_bounds__(256) void eltwise_vec_kernel(int op, float* out, const float* a, const float* b,
                                                          bool b_splat, EltDims d, float alpha, int32_t total4) {
    const int32_t inner = d.dims[d.rank - 1];
    for (int32_t i = blockIdx.x * 256 + threadIdx.x; i < total4; i += gridDim.x * 256) {
        int32_t e = i * 4;
        const int32_t ix = e % inner;
        e /= inner;
        int32_t oo = ix, ao = ix, bo = b_splat ? 0 : ix;
        for (int k = d.rank - 2; k >= 0; --k) {
            const int32_t idx = e % d.dims[k];
            e /= d.dims[k];
            oo += idx * d.so[k];
            ao += idx * d.sa[k];
            bo += idx * d.sb[k];
        }
        const float4 x = *reinterpret_cast<const float4*>(a + ao);
        float4 y;
        if (b_splat) {
            const float v = b[bo];
            y = make_float4(v, v, v, v);
        } else {
            y = *reinterpret_cast<const float4*>(b + bo);
        }
        float4 r;
        r.x = elt_apply(op, x.x, y.x, alpha);
        r.y = elt_apply(op, x.y, y.y, alpha);
        r.z = elt_apply(op, x.z, y.z, alpha);
        r.w = elt_apply(op, x.w, y.w, alpha);
        *reinterpret_cast<float4*>(out + oo) = r;
    }
}

// A unary op whose output is contiguous along one collapsed dim (Q) and
// whose input along another (P), e.g. NCHW <-> NHWC at a graph's edges: per
// index of the other (outer) dims, a P x Q transpose in 32 x 32 tiles through
// LDS, so that both the reads (along P) and the writes (along Q) are
// coalesced.  Each element is computed exactly as eltwise_kernel computes it.
struct TransDims {
    int32_t P = 0, Q = 0;
    int32_t so_p = 0, sa_q = 0;  // output stride along P, input stride along Q
    int32_t rank = 0;            // outer dims
    int32_t dims[kMaxRank] = {}, so[kMaxRank] = {}, sa[kMaxRank] = {};
};

__global__ __launch_bounds__(256) void transpose_elt_kernel(int op, float* out, const float* a, TransDims d,
                                                            float alpha) {
    __shared__ float tile[32][33];
    const int tiles_p = (d.P + 31) / 32;
    const int p0 = (blockIdx.x % tiles_p) * 32;
    const int q0 = (blockIdx.x / tiles_p) * 32;
    int32_t o = blockIdx.y, ob = 0, ab = 0;
    for (int k = d.rank - 1; k >= 0; --k) {
        const int32_t idx = o % d.dims[k];
        o /= d.dims[k];
        ob += idx * d.so[k];
        ab += idx * d.sa[k];
    }
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int q = q0 + ty + 8 * r, p = p0 + tx;
        if (q < d.Q && p < d.P) tile[ty + 8 * r][tx] = a[ab + q * d.sa_q + p];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int p = p0 + ty + 8 * r, q = q0 + tx;
        if (p < d.P && q < d.Q) out[ob + p * d.so_p + q] = elt_apply(op, tile[tx][ty + 8 * r], 0.0f, alpha);
    }
}

namespace {

// Collapsed dims of (out, a, b); false if some extent or stride exceeds int32.
// An elementwise op may visit its elements in any order, so the dims are
// first ordered by the output's stride (largest first): a channels-last
// tensor then has its contiguous channel dim innermost.
bool collapse_elt(const View& o, const View& a, const View& b, EltDims& c) {
    int order[kMaxRank];
    for (int k = 0; k < o.rank; ++k) order[k] = k;
    std::stable_sort(order, order + o.rank,
                     [&](int x, int y) { return std::abs(o.str[x]) > std::abs(o.str[y]); });
    int64_t dims[kMaxRank], so[kMaxRank], sa[kMaxRank], sb[kMaxRank];
    int r = 0;
    for (int kk = 0; kk < o.rank; ++kk) {
        const int k = order[kk];
        if (o.dims[k] == 1) continue;
        if (r > 0 && so[r - 1] == o.str[k] * o.dims[k] && sa[r - 1] == a.str[k] * o.dims[k] &&
            sb[r - 1] == b.str[k] * o.dims[k]) {
            dims[r - 1] *= o.dims[k];
            so[r - 1] = o.str[k];
            sa[r - 1] = a.str[k];
            sb[r - 1] = b.str[k];
            continue;
        }
        dims[r] = o.dims[k];
        so[r] = o.str[k];
        sa[r] = a.str[k];
        sb[r] = b.str[k];
        ++r;
    }
    if (r == 0) {
        dims[0] = 1;
        so[0] = sa[0] = sb[0] = 1;
        r = 1;
    }
    c.rank = r;
    for (int k = 0; k < r; ++k) {
        const int64_t m = std::max({dims[k], std::abs(so[k]), std::abs(sa[k]), std::abs(sb[k])});
        if (m >= (int64_t{1} << 31)) return false;
        c.dims[k] = static_cast<int32_t>(dims[k]);
        c.so[k] = static_cast<int32_t>(so[k]);
        c.sa[k] = static_cast<int32_t>(sa[k]);
        c.sb[k] = static_cast<int32_t>(sb[k]);
    }
    return true;
}

bool aligned16(const float* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

void launch_eltwise(int op, const View& out, const View& a, const View& b, float alpha, hipStream_t s) {
    check_view(out, "eltwise out");
    check_view(a, "eltwise a");
    const bool binary = op == kEltAdd || op == kEltSub || op == kEltMul || op == kEltDiv;
    if (binary) check_view(b, "eltwise b");
    if (a.rank != out.rank || (binary && b.rank != out.rank)) throw std::runtime_error("eltwise: rank mismatch");
    const int64_t total = numel(out);
    if (total == 0) return;
    const View& bb = binary ? b : a;
    // float4 path (see eltwise_vec_kernel)
    EltDims c;
    if (total < (int64_t{1} << 31) && fits_i32(out) && fits_i32(a) && fits_i32(bb) && collapse_elt(out, a, bb, c)) {
        const int in = c.rank - 1;
        const bool b_splat = binary && c.sb[in] == 0;
        bool vec = c.dims[in] % 4 == 0 && c.so[in] == 1 && c.sa[in] == 1 && (b_splat || c.sb[in] == 1) &&
                   aligned16(out.ptr) && aligned16(a.ptr) && (b_splat || aligned16(bb.ptr));
        // (a b constant along the inner dim is read one float at a time)
        for (int k = 0; k < in; ++k) vec = vec && c.so[k] % 4 == 0 && c.sa[k] % 4 == 0 && (b_splat || c.sb[k] % 4 == 0);
        if (vec) {
            const int32_t total4 = static_cast<int32_t>(total / 4);
            hipLaunchKernelGGL(eltwise_vec_kernel, dim3(grid_for(total4)), dim3(256), 0, s, op, out.ptr, a.ptr,
                               bb.ptr, b_splat, c, alpha, total4);
            return;
        }
        // tiled transpose (see transpose_elt_kernel): a unary op, the output
        // contiguous along the inner collapsed dim Q, the input along dim P
        int pj = -1;
        for (int k = 0; k < in; ++k)
            if (c.sa[k] == 1) pj = k;
        if (!binary && c.so[in] == 1 && c.sa[in] != 1 && pj >= 0 && c.dims[in] >= 8 && c.dims[pj] >= 8) {
            TransDims t;
            t.P = c.dims[pj];
            t.Q = c.dims[in];
            t.so_p = c.so[pj];
            t.sa_q = c.sa[in];
            int64_t outer = 1;
            for (int k = 0; k < in; ++k) {
                if (k == pj) continue;
                t.dims[t.rank] = c.dims[k];
                t.so[t.rank] = c.so[k];
                t.sa[t.rank] = c.sa[k];
                ++t.rank;
                outer *= c.dims[k];
            }
            const int64_t tiles = static_cast<int64_t>((t.P + 31) / 32) * ((t.Q + 31) / 32);
            if (outer <= 65535 && tiles < (int64_t{1} << 31)) {
                hipLaunchKernelGGL(transpose_elt_kernel, dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(outer)),
                                   dim3(256), 0, s, op, out.ptr, a.ptr, t, alpha);
                return;
            }
        }
    }
    if (fits_i32(out) && fits_i32(a) && fits_i32(bb))
        hipLaunchKernelGGL(eltwise_kernel<int32_t>, dim3(grid_for(total)), dim3(256), 0, s, op, iview<int32_t>(out),
                           iview<int32_t>(a), iview<int32_t>(bb), alpha, static_cast<int32_t>(total));
    else
        hipLaunchKernelGGL(eltwise_kernel<int64_t>, dim3(grid_for(total)), dim3(256), 0, s, op, iview<int64_t>(out),
                           iview<int64_t>(a), iview<int64_t>(bb), alpha, total);
}

template <typename I>
__global__ __launch_bounds__(256) void maxpool_kernel(IView<I> out, IView<I> in, int kh, int kw, int sh, int sw, int ph,
                                                      int pw, I total) {
    const I C = out.dims[1], Ho = out.dims[2], Wo = out.dims[3];
    const I H = in.dims[2], W = in.dims[3];
    for (I i = blockIdx.x * static_cast<I>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<I>(gridDim.x) * blockDim.x) {
        I t = i;
        const I c = t % C; t /= C;
        const I wo = t % Wo; t /= Wo;
        const I ho = t % Ho;
        const I n = t / Ho;
        const float* base = in.ptr + n * in.str[0] + c * in.str[1];
        float m = -3.402823466e+38f;
        for (int a = 0; a < kh; ++a) {
            const I hi = ho * sh - ph + a;
            if (hi < 0 || hi >= H) continue;
            for (int b = 0; b < kw; ++b) {
                const I wi = wo * sw - pw + b;
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
    if (fits_i32(out) && fits_i32(in))
        hipLaunchKernelGGL(maxpool_kernel<int32_t>, dim3(grid_for(total)), dim3(256), 0, s, iview<int32_t>(out),
                           iview<int32_t>(in), kh, kw, sh, sw, ph, pw, static_cast<int32_t>(total));
    else
        hipLaunchKernelGGL(maxpool_kernel<int64_t>, dim3(grid_for(total)), dim3(256), 0, s, iview<int64_t>(out),
                           iview<int64_t>(in), kh, kw, sh, sw, ph, pw, total);
}

template <typename I>
__global__ __launch_bounds__(256) void resize_nearest_kernel(IView<I> out, IView<I> in, float ry, float rx, I total) {
    const I C = out.dims[1], Ho = out.dims[2], Wo = out.dims[3];
    const I H = in.dims[2], W = in.dims[3];
    for (I i = blockIdx.x * static_cast<I>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<I>(gridDim.x) * blockDim.x) {
        I t = i;
        const I c = t % C; t /= C;
        const I wo = t % Wo; t /= Wo;
        const I ho = t % Ho;
        const I n = t / Ho;
        I hi = static_cast<I>(static_cast<float>(ho) * ry);
        I wi = static_cast<I>(static_cast<float>(wo) * rx);
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
    if (fits_i32(out) && fits_i32(in))
        hipLaunchKernelGGL(resize_nearest_kernel<int32_t>, dim3(grid_for(total)), dim3(256), 0, s, iview<int32_t>(out),
                           iview<int32_t>(in), ry, rx, static_cast<int32_t>(total));
    else
        hipLaunchKernelGGL(resize_nearest_kernel<int64_t>, dim3(grid_for(total)), dim3(256), 0, s, iview<int64_t>(out),
                           iview<int64_t>(in), ry, rx, total);
}

template <typename I>
__global__ __launch_bounds__(256) void softmax_kernel(IView<I> out, IView<I> in, int axis, I rows) {
    const I L = in.dims[axis];
    for (I r = blockIdx.x * static_cast<I>(blockDim.x) + threadIdx.x; r < rows;
         r += static_cast<I>(gridDim.x) * blockDim.x) {
        I rem = r, io = 0, oo = 0;
        for (int d = in.rank - 1; d >= 0; --d) {
            if (d == axis) continue;
            const I idx = rem % in.dims[d];
            rem /= in.dims[d];
            io += idx * in.str[d];
            oo += idx * out.str[d];
        }
        const I is = in.str[axis], os = out.str[axis];
        float mx = -1e30f;
        for (I j = 0; j < L; ++j) {
            const float v = in.ptr[io + j * is];
            mx = v > mx ? v : mx;
        }
        float sum = 0.0f;
        for (I j = 0; j < L; ++j) {
            const float e = expf(in.ptr[io + j * is] - mx);
            out.ptr[oo + j * os] = e;
            sum += e;
        }
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (I j = 0; j < L; ++j) out.ptr[oo + j * os] *= inv;
    }
}

// Softmax over a contiguous axis of L = 4*Q elements (Q <= 16), one row per
// lane held in registers: 16-byte loads and stores, int32 row decomposition.
// Same arithmetic as the generic kernel (max, exp(x - max), sum, * 1/sum).
template <int Q>
__global__ __launch_bounds__(256) void softmax_vec_kernel(IView<int32_t> out, IView<int32_t> in, int axis,
                                                          int32_t rows) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    for (int32_t r = blockIdx.x * 256 + threadIdx.x; r < rows; r += gridDim.x * 256) {
        int32_t rem = r, io = 0, oo = 0;
        for (int d = in.rank - 1; d >= 0; --d) {
            if (d == axis) continue;
            const int32_t idx = rem % in.dims[d];
            rem /= in.dims[d];
            io += idx * in.str[d];
            oo += idx * out.str[d];
        }
        f4 v[Q];
#pragma unroll
        for (int q = 0; q < Q; ++q) v[q] = *reinterpret_cast<const f4*>(in.ptr + io + 4 * q);
        float mx = -1e30f;
#pragma unroll
        for (int q = 0; q < Q; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) mx = v[q][e] > mx ? v[q][e] : mx;
        float sum = 0.0f;
#pragma unroll
        for (int q = 0; q < Q; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[q][e] = expf(v[q][e] - mx);
                sum += v[q][e];
            }
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
#pragma unroll
        for (int q = 0; q < Q; ++q) *reinterpret_cast<f4*>(out.ptr + oo + 4 * q) = v[q] * inv;
    }
}

void launch_softmax(const View& out, const View& in, int axis, hipStream_t s) {
    check_view(out, "softmax out");
    check_view(in, "softmax in");
    if (out.rank != in.rank || axis < 0 || axis >= in.rank) throw std::runtime_error("softmax: bad axis/rank");
    const int64_t L = in.dims[axis];
    const int64_t rows = numel(in) / std::max<int64_t>(1, L);
    if (rows == 0) return;
    const bool i32 = fits_i32(out) && fits_i32(in);
    bool vec = i32 && in.str[axis] == 1 && out.str[axis] == 1 && L % 4 == 0 && L >= 4 && L <= 64 &&
               (reinterpret_cast<uintptr_t>(in.ptr) & 15) == 0 && (reinterpret_cast<uintptr_t>(out.ptr) & 15) == 0;
    for (int d = 0; d < in.rank && vec; ++d)
        if (d != axis && (in.str[d] % 4 != 0 || out.str[d] % 4 != 0)) vec = false;
    const unsigned g = grid_for(rows);
    if (vec) {
        const IView<int32_t> o = iview<int32_t>(out), x = iview<int32_t>(in);
        const int32_t r = static_cast<int32_t>(rows);
        switch (L / 4) {
            case 1: hipLaunchKernelGGL(softmax_vec_kernel<1>, dim3(g), dim3(256), 0, s, o, x, axis, r); return;
            case 2: hipLaunchKernelGGL(softmax_vec_kernel<2>, dim3(g), dim3(256), 0, s, o, x, axis, r); return;
            case 4: hipLaunchKernelGGL(softmax_vec_kernel<4>, dim3(g), dim3(256), 0, s, o, x, axis, r); return;
            case 8: hipLaunchKernelGGL(softmax_vec_kernel<8>, dim3(g), dim3(256), 0, s, o, x, axis, r); return;
            case 16: hipLaunchKernelGGL(softmax_vec_kernel<16>, dim3(g), dim3(256), 0, s, o, x, axis, r); return;
            default: break;
        }
    }
    if (i32)
        hipLaunchKernelGGL(softmax_kernel<int32_t>, dim3(g), dim3(256), 0, s, iview<int32_t>(out), iview<int32_t>(in),
                           axis, static_cast<int32_t>(rows));
    else
        hipLaunchKernelGGL(softmax_kernel<int64_t>, dim3(g), dim3(256), 0, s, iview<int64_t>(out), iview<int64_t>(in),
                           axis, rows);
}

// Dispatch slot `lin` (of `total`) runs on XCD lin % 8: the block index that
// gives each XCD a contiguous range of blocks.
__device__ __forceinline__ int32_t xcd_block(int32_t lin, int32_t total) {
    const int32_t q = total / 8, rmd = total % 8, xcd = lin % 8;
    return xcd * q + min(xcd, rmd) + lin / 8;
}

// SPPF: three chained k x k stride-1 same-padded max pools in one pass.  A
// workgroup takes a T x T pixel tile of CB channels: it stages the tile plus
// a 3r halo in LDS (outside the image: -FLT_MAX, so padding never wins), takes
// the row maxima over radii r, 2r and 3r, then the column maxima of those:
// the separable form of the square windows of sides 2r+1, 4r+1 and 6r+1.
// Channel fastest, so channels-last views are read and written contiguously.
constexpr int kPoolTile = 8;
constexpr int kPoolCb = 16;
constexpr int kPoolMaxR = 3;

template <int r>
__global__ __launch_bounds__(256) void maxpool_chain_kernel(IView<int32_t> o0, IView<int32_t> o1, IView<int32_t> o2,
                                                            IView<int32_t> in, int tiles_w) {
    constexpr int T = kPoolTile, CB = kPoolCb;
    constexpr int R3 = 3 * r;
    constexpr int RH = T + 2 * R3;  // staged rows and columns
    constexpr int NL = (RH * RH * CB + 255) / 256;  // staged elements per lane
    __shared__ float reg[RH * RH * CB];    // [RH][RH][CB]
    __shared__ float hz[3 * RH * T * CB];  // [3][RH][T][CB]
    const int C = o0.dims[1], H = in.dims[2], W = in.dims[3];
    const int th = blockIdx.x / tiles_w, tw = blockIdx.x - th * tiles_w;
    const int h0 = th * T, w0 = tw * T, c0 = blockIdx.y * CB, n = blockIdx.z;
    const float* base = in.ptr + n * in.str[0];
    // every lane's loads are issued before the first is waited for
    float v[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int i = threadIdx.x + 256 * j;
        const int c = i % CB, p = i / CB;
        const int rx = p % RH, ry = p / RH;
        const int h = h0 - R3 + ry, w = w0 - R3 + rx;
        const bool ok = (i < RH * RH * CB) & (h >= 0) & (h < H) & (w >= 0) & (w < W) & (c0 + c < C);
        const float x = base[ok ? (c0 + c) * in.str[1] + h * in.str[2] + w * in.str[3] : 0];
        v[j] = ok ? x : -3.402823466e+38f;
    }
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int i = threadIdx.x + 256 * j;
        if (i < RH * RH * CB) reg[i] = v[j];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < RH * T * CB; i += 256) {
        const int c = i % CB, p = i / CB;
        const int tx = p % T, ry = p / T;
        const float* row = reg + ry * RH * CB + c;
        const int x = R3 + tx;
        float m = row[x * CB];
        float out[3];
        int d = 1;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            for (; d <= (k + 1) * r; ++d) {
                const float a = row[(x - d) * CB], b = row[(x + d) * CB];
                m = a > m ? a : m;
                m = b > m ? b : m;
            }
            out[k] = m;
        }
#pragma unroll
        for (int k = 0; k < 3; ++k) hz[((k * RH + ry) * T + tx) * CB + c] = out[k];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < T * T * CB; i += 256) {
        const int c = i % CB, p = i / CB;
        const int tx = p % T, ty = p / T;
        const int h = h0 + ty, w = w0 + tx;
        if (h >= H || w >= W || c0 + c >= C) continue;
        const int y = R3 + ty;
        float res[3];
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const float* col = hz + (k * RH * T + tx) * CB + c;  // row stride T*CB
            const int rad = (k + 1) * r;
            float m = col[y * T * CB];
            for (int d = 1; d <= rad; ++d) {
                const float a = col[(y - d) * T * CB], b = col[(y + d) * T * CB];
                m = a > m ? a : m;
                m = b > m ? b : m;
            }
            res[k] = m;
        }
        const int cc = c0 + c;
        o0.ptr[n * o0.str[0] + cc * o0.str[1] + h * o0.str[2] + w * o0.str[3]] = res[0];
        o1.ptr[n * o1.str[0] + cc * o1.str[1] + h * o1.str[2] + w * o1.str[3]] = res[1];
        o2.ptr[n * o2.str[0] + cc * o2.str[1] + h * o2.str[2] + w * o2.str[3]] = res[2];
    }
}

// The same three pools over channels-last views (channel stride 1, C and
// every pixel stride a multiple of 4, 16-byte aligned bases): each lane
// moves float4 runs of 4 channels, so a workgroup's T x T x CB tile (plus the
// 3r halo) is staged, swept and stored with a quarter of the instructions.
template <int r>
__global__ __launch_bounds__(256) void maxpool_chain_vec_kernel(IView<int32_t> o0, IView<int32_t> o1, IView<int32_t> o2,
                                                                IView<int32_t> in, int tiles_w) {
    constexpr int T = kPoolTile, CB = kPoolCb, G = CB / 4;  // G float4 groups per pixel
    constexpr int R3 = 3 * r;
    constexpr int RH = T + 2 * R3;
    constexpr int NL = (RH * RH * G + 255) / 256;
    __shared__ float4 reg[RH * RH * G];    // [RH][RH][G]
    __shared__ float4 hz[3 * RH * T * G];  // [3][RH][T][G]
    const int C = o0.dims[1], H = in.dims[2], W = in.dims[3];
    const int th = blockIdx.x / tiles_w, tw = blockIdx.x - th * tiles_w;
    const int h0 = th * T, w0 = tw * T, c0 = blockIdx.y * CB, n = blockIdx.z;
    const float* base = in.ptr + n * in.str[0];
    const float4 lowest = make_float4(-3.402823466e+38f, -3.402823466e+38f, -3.402823466e+38f, -3.402823466e+38f);
    auto vmax = [](float4 a, float4 b) {
        return make_float4(b.x > a.x ? b.x : a.x, b.y > a.y ? b.y : a.y, b.z > a.z ? b.z : a.z, b.w > a.w ? b.w : a.w);
    };
    float4 v[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int i = threadIdx.x + 256 * j;
        const int g = i % G, p = i / G;
        const int rx = p % RH, ry = p / RH;
        const int h = h0 - R3 + ry, w = w0 - R3 + rx;
        const bool ok = (i < RH * RH * G) & (h >= 0) & (h < H) & (w >= 0) & (w < W) & (c0 + 4 * g < C);
        const float4 x = *reinterpret_cast<const float4*>(base + (ok ? c0 + 4 * g + h * in.str[2] + w * in.str[3] : 0));
        // (a float4 select, written per component)
        v[j].x = ok ? x.x : lowest.x;
        v[j].y = ok ? x.y : lowest.y;
        v[j].z = ok ? x.z : lowest.z;
        v[j].w = ok ? x.w : lowest.w;
    }
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int i = threadIdx.x + 256 * j;
        if (i < RH * RH * G) reg[i] = v[j];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < RH * T * G; i += 256) {
        const int g = i % G, p = i / G;
        const int tx = p % T, ry = p / T;
        const float4* row = reg + ry * RH * G + g;
        const int x = R3 + tx;
        // running maximum over radii 1..3r; the three widths are its values at r, 2r, 3r
        float4 m = row[x * G], m1 = m, m2 = m;
#pragma unroll
        for (int d = 1; d <= R3; ++d) {
            m = vmax(vmax(m, row[(x - d) * G]), row[(x + d) * G]);
            if (d == r) m1 = m;
            if (d == 2 * r) m2 = m;
        }
        hz[((0 * RH + ry) * T + tx) * G + g] = m1;
        hz[((1 * RH + ry) * T + tx) * G + g] = m2;
        hz[((2 * RH + ry) * T + tx) * G + g] = m;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < T * T * G; i += 256) {
        const int g = i % G, p = i / G;
        const int tx = p % T, ty = p / T;
        const int h = h0 + ty, w = w0 + tx;
        if (h >= H || w >= W || c0 + 4 * g >= C) continue;
        const int y = R3 + ty;
        // column maximum of row-maxima plane k over radius rad (row stride T*G)
        auto colmax = [&](int k, auto rad_c) {
            constexpr int rad = decltype(rad_c)::value;
            const float4* col = hz + (k * RH * T + tx) * G + g;
            float4 m = col[y * T * G];
#pragma unroll
            for (int d = 1; d <= rad; ++d) m = vmax(vmax(m, col[(y - d) * T * G]), col[(y + d) * T * G]);
            return m;
        };
        const float4 r0 = colmax(0, std::integral_constant<int, r>{});
        const float4 r1 = colmax(1, std::integral_constant<int, 2 * r>{});
        const float4 r2 = colmax(2, std::integral_constant<int, 3 * r>{});
        const int cc = c0 + 4 * g;
        *reinterpret_cast<float4*>(o0.ptr + n * o0.str[0] + cc + h * o0.str[2] + w * o0.str[3]) = r0;
        *reinterpret_cast<float4*>(o1.ptr + n * o1.str[0] + cc + h * o1.str[2] + w * o1.str[3]) = r1;
        *reinterpret_cast<float4*>(o2.ptr + n * o2.str[0] + cc + h * o2.str[2] + w * o2.str[3]) = r2;
    }
}

// The same three pools over a whole channels-last plane per workgroup, for
// maps of up to 1024 pixels (SPPF at 20x20 for a 640 input): the workgroup
// stages all H x W pixels of its 4*G channels once -- no halo re-reads -- and
// writes each output element once, so the kernel moves the algorithmic bytes
// (one read of the input, one write of each output).  Windows are clipped at
// the image edge; the running maximum starts at -FLT_MAX, the floor of the
// reference's pools (pooling.cpp:53-91).
constexpr int kPoolPlaneMax = 1024;  // pixels
template <int r, int G>
__global__ __launch_bounds__(256) void maxpool_plane_vec_kernel(IView<int32_t> o0, IView<int32_t> o1,
                                                                IView<int32_t> o2, IView<int32_t> in) {
    extern __shared__ float4 plane[];  // [H*W][G] input, then [3][H*W][G] row maxima
    const int H = in.dims[2], W = in.dims[3], HW = H * W;
    // each XCD takes a contiguous range of (image, channel group) planes:
    // neighbouring channel groups share cache lines, which one L2 then
    // fetches and writes once
    const int bid = xcd_block(blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);
    const int n = bid / gridDim.x;
    const int c0 = (bid - n * gridDim.x) * 4 * G;
    float4* const reg = plane;
    float4* const hz = plane + HW * G;
    const float* base = in.ptr + n * in.str[0] + c0;
    const float4 lowest = make_float4(-3.402823466e+38f, -3.402823466e+38f, -3.402823466e+38f, -3.402823466e+38f);
    auto vmax = [](float4 a, float4 b) {
        return make_float4(b.x > a.x ? b.x : a.x, b.y > a.y ? b.y : a.y, b.z > a.z ? b.z : a.z, b.w > a.w ? b.w : a.w);
    };
    for (int i = threadIdx.x; i < HW * G; i += 256) {
        const int g = i % G, p = i / G;
        const int h = p / W, w = p - h * W;
        reg[i] = *reinterpret_cast<const float4*>(base + 4 * g + h * in.str[2] + w * in.str[3]);
    }
    __syncthreads();
    // row maxima over radii r, 2r, 3r (one running maximum).  A window
    // position past the image edge reads the edge pixel instead -- it lies
    // inside the window too, so the maximum is unchanged -- which keeps the
    // reads unconditional, all issued before the maxima are taken.
    for (int i = threadIdx.x; i < HW * G; i += 256) {
        const int g = i % G, p = i / G;
        const int h = p / W, w = p - h * W;
        const float4* row = reg + h * W * G + g;
        float4 lf[3 * r + 1], rt[3 * r + 1];
#pragma unroll
        for (int d = 1; d <= 3 * r; ++d) {
            lf[d] = row[max(w - d, 0) * G];
            rt[d] = row[min(w + d, W - 1) * G];
        }
        float4 m = vmax(lowest, reg[i]), m1 = m, m2 = m;
#pragma unroll
        for (int d = 1; d <= 3 * r; ++d) {
            m = vmax(vmax(m, lf[d]), rt[d]);
            if (d == r) m1 = m;
            if (d == 2 * r) m2 = m;
        }
        hz[i] = m1;
        hz[HW * G + i] = m2;
        hz[2 * HW * G + i] = m;
    }
    __syncthreads();
    // column maxima of row-maxima plane k over radius (k + 1) r, stored
    for (int i = threadIdx.x; i < HW * G; i += 256) {
        const int g = i % G, p = i / G;
        const int h = p / W, w = p - h * W;
        auto colmax = [&](int k, auto rad_c) {
            constexpr int rad = decltype(rad_c)::value;
            const float4* col = hz + k * HW * G + w * G + g;
            float4 up[rad + 1], dn[rad + 1];
#pragma unroll
            for (int d = 1; d <= rad; ++d) {
                up[d] = col[max(h - d, 0) * W * G];
                dn[d] = col[min(h + d, H - 1) * W * G];
            }
            float4 m = col[h * W * G];
#pragma unroll
            for (int d = 1; d <= rad; ++d) m = vmax(vmax(m, up[d]), dn[d]);
            return m;
        };
        const float4 r0 = colmax(0, std::integral_constant<int, r>{});
        const float4 r1 = colmax(1, std::integral_constant<int, 2 * r>{});
        const float4 r2 = colmax(2, std::integral_constant<int, 3 * r>{});
        const int cc = c0 + 4 * g;
        *reinterpret_cast<float4*>(o0.ptr + n * o0.str[0] + cc + h * o0.str[2] + w * o0.str[3]) = r0;
        *reinterpret_cast<float4*>(o1.ptr + n * o1.str[0] + cc + h * o1.str[2] + w * o1.str[3]) = r1;
        *reinterpret_cast<float4*>(o2.ptr + n * o2.str[0] + cc + h * o2.str[2] + w * o2.str[3]) = r2;
    }
}

namespace {

// Channels-last float4 form applies: channel stride 1, C and the pixel
// strides multiples of 4 floats, 16-byte aligned bases.
bool pool_vec_ok(const View& v) {
    return v.str[1] == 1 && v.dims[1] % 4 == 0 && v.str[0] % 4 == 0 && v.str[2] % 4 == 0 && v.str[3] % 4 == 0 &&
           (reinterpret_cast<uintptr_t>(v.ptr) & 15) == 0;
}

}  // namespace

void launch_maxpool_chain(const View& out0, const View& out1, const View& out2, const View& in, int k,
                          hipStream_t s) {
    check_view(out0, "maxpool_chain out0");
    check_view(out1, "maxpool_chain out1");
    check_view(out2, "maxpool_chain out2");
    check_view(in, "maxpool_chain in");
    if (out0.rank != 4 || out1.rank != 4 || out2.rank != 4 || in.rank != 4)
        throw std::runtime_error("maxpool_chain: rank 4 views expected");
    if (k < 1 || k % 2 == 0 || k / 2 > kPoolMaxR) throw std::runtime_error("maxpool_chain: odd kernel <= 7 expected");
    for (int d = 0; d < 4; ++d)
        if (out0.dims[d] != in.dims[d] || out1.dims[d] != in.dims[d] || out2.dims[d] != in.dims[d])
            throw std::runtime_error("maxpool_chain: same-size outputs expected");
    if (numel(out0) == 0) return;
    if (!(fits_i32(out0) && fits_i32(out1) && fits_i32(out2) && fits_i32(in)))
        throw std::runtime_error("maxpool_chain: views exceed int32 indexing");
    const int64_t N = in.dims[0], C = in.dims[1], H = in.dims[2], W = in.dims[3];
    const int64_t tiles_h = (H + kPoolTile - 1) / kPoolTile, tiles_w = (W + kPoolTile - 1) / kPoolTile;
    const int64_t cblocks = (C + kPoolCb - 1) / kPoolCb;
    if (tiles_h * tiles_w > 0x7fffffff || cblocks > 65535 || N > 65535)
        throw std::runtime_error("maxpool_chain: grid too large");
    const dim3 grid(static_cast<unsigned>(tiles_h * tiles_w), static_cast<unsigned>(cblocks), static_cast<unsigned>(N));
    const auto o0 = iview<int32_t>(out0), o1 = iview<int32_t>(out1), o2 = iview<int32_t>(out2);
    const auto x = iview<int32_t>(in);
    const int tw = static_cast<int>(tiles_w);
    if (pool_vec_ok(out0) && pool_vec_ok(out1) && pool_vec_ok(out2) && pool_vec_ok(in) && H * W <= kPoolPlaneMax &&
        N * (C / 4) >= 128) {
        // whole planes of 4 channels a workgroup (input + three row-maxima
        // planes: 64 bytes a pixel of LDS); 8 channels where the workgroups
        // would exceed the CUs
        const bool g2 = H * W * 2 <= kPoolPlaneMax && C % 8 == 0 && N * (C / 4) > 256;
        const int64_t per = g2 ? 8 : 4;
        // (taken where the planes give at least 128 workgroups: with fewer,
        // the tiled kernel's more workgroups finish sooner)
        const dim3 pgrid(static_cast<unsigned>(C / per), static_cast<unsigned>(N));
        const size_t lds = sizeof(float) * 4 * static_cast<size_t>(H * W) * per;
        auto go = [&](auto r_c) {
            constexpr int R = decltype(r_c)::value;
            if (g2)
                hipLaunchKernelGGL((maxpool_plane_vec_kernel<R, 2>), pgrid, dim3(256), lds, s, o0, o1, o2, x);
            else
                hipLaunchKernelGGL((maxpool_plane_vec_kernel<R, 1>), pgrid, dim3(256), lds, s, o0, o1, o2, x);
        };
        switch (k / 2) {
            case 0: go(std::integral_constant<int, 0>{}); break;
            case 1: go(std::integral_constant<int, 1>{}); break;
            case 2: go(std::integral_constant<int, 2>{}); break;
            default: go(std::integral_constant<int, 3>{}); break;
        }
        return;
    }
    if (pool_vec_ok(out0) && pool_vec_ok(out1) && pool_vec_ok(out2) && pool_vec_ok(in)) {
        switch (k / 2) {
            case 0: hipLaunchKernelGGL(maxpool_chain_vec_kernel<0>, grid, dim3(256), 0, s, o0, o1, o2, x, tw); break;
            case 1: hipLaunchKernelGGL(maxpool_chain_vec_kernel<1>, grid, dim3(256), 0, s, o0, o1, o2, x, tw); break;
            case 2: hipLaunchKernelGGL(maxpool_chain_vec_kernel<2>, grid, dim3(256), 0, s, o0, o1, o2, x, tw); break;
            default: hipLaunchKernelGGL(maxpool_chain_vec_kernel<3>, grid, dim3(256), 0, s, o0, o1, o2, x, tw); break;
        }
        return;
    }
    switch (k / 2) {
        case 0: hipLaunchKernelGGL(maxpool_chain_kernel<0>, grid, dim3(256), 0, s, o0, o1, o2, x, tw); break;
        case 1: hipLaunchKernelGGL(maxpool_chain_kernel<1>, grid, dim3(256), 0, s, o0, o1, o2, x, tw); break;
        case 2: hipLaunchKernelGGL(maxpool_chain_kernel<2>, grid, dim3(256), 0, s, o0, o1, o2, x, tw); break;
        default: hipLaunchKernelGGL(maxpool_chain_kernel<3>, grid, dim3(256), 0, s, o0, o1, o2, x, tw); break;
    }
}

// DFL expectation of one side: softmax over the R bins (max, exp(x - max),
// sum in bin order, * 1/sum, as softmax_kernel) and the weighted sum in bin
// order (the direct conv's accumulation order) plus the bias.
template <int R, typename W>
__device__ __forceinline__ float dfl_side(float (&v)[R], const W& w, float bias) {
    float mx = -1e30f;
#pragma unroll
    for (int b = 0; b < R; ++b) mx = v[b] > mx ? v[b] : mx;
    float sum = 0.0f;
#pragma unroll
    for (int b = 0; b < R; ++b) {
        v[b] = expf(v[b] - mx);
        sum += v[b];
    }
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < R; ++b) acc = fmaf(v[b] * inv, w[b], acc);
    return acc + bias;
}

// The per-anchor inputs of the box decode: anchor point, divisor, strides.
struct BoxIn {
    float ax, ay, tx, ty, st[4];
};

__device__ __forceinline__ BoxIn load_box_in(const DetectDecodeArgs& a, int32_t n, int32_t an) {
    auto at = [&](const View& v, int c) {
        return v.ptr[n * v.str[0] + c * v.str[1] + static_cast<int64_t>(an) * v.str[2]];
    };
    return BoxIn{at(a.anchors, 0), at(a.anchors, 1), at(a.two, 0), at(a.two, 1),
                 {at(a.strides, 0), at(a.strides, 1), at(a.strides, 2), at(a.strides, 3)}};
}

// dist2bbox of one anchor from its four side distances d, then * stride.
__device__ __forceinline__ void decode_box(const DetectDecodeArgs& a, int32_t n, int32_t an, const float (&d)[4],
                                           const BoxIn& b) {
    const float x1 = b.ax - d[0], y1 = b.ay - d[1];
    const float x2 = b.ax + d[2], y2 = b.ay + d[3];
    const float r[4] = {(x1 + x2) / b.tx, (y1 + y2) / b.ty, x2 - x1, y2 - y1};
#pragma unroll
    for (int c = 0; c < 4; ++c)
        a.out.ptr[n * a.out.str[0] + c * a.out.str[1] + static_cast<int64_t>(an) * a.out.str[2]] = r[c] * b.st[c];
}

// One lane per (n, anchor); see kernels.hpp for the arithmetic.  R > 0: the
// bin count is R and each side's R bins are contiguous and 16-byte aligned
// (the Detect head's [anchor][144] rows), loaded as float4 into registers;
// R == 0: any bin count and strides.
template <int R>
__global__ __launch_bounds__(256) void detect_decode_kernel(DetectDecodeArgs a, int32_t N, int32_t A) {
    const int32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= N * A) return;
    const int32_t n = i / A;
    const int32_t an = i - n * A;
    const View& x = a.x;  // offsets within int32 (checked by the launcher)
    const int32_t xs1 = static_cast<int32_t>(x.str[1]);
    float d[4];
#pragma unroll
    for (int side = 0; side < 4; ++side) {
        const float* xs = x.ptr + static_cast<int32_t>(n * x.str[0] + side * x.str[2] + an * x.str[3]);
        if constexpr (R > 0) {
            float v[R];
#pragma unroll
            for (int q = 0; q < R / 4; ++q) {
                const float4 t = reinterpret_cast<const float4*>(xs)[q];
                v[4 * q] = t.x;
                v[4 * q + 1] = t.y;
                v[4 * q + 2] = t.z;
                v[4 * q + 3] = t.w;
            }
            d[side] = dfl_side<R>(v, a.dfl_w, a.dfl_bias);
        } else {
            float mx = -1e30f;
            for (int b = 0; b < a.bins; ++b) {
                const float v = xs[b * xs1];
                mx = v > mx ? v : mx;
            }
            float sum = 0.0f;
            for (int b = 0; b < a.bins; ++b) sum += expf(xs[b * xs1] - mx);
            const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
            float acc = 0.0f;
            for (int b = 0; b < a.bins; ++b) acc = fmaf(expf(xs[b * xs1] - mx) * inv, a.dfl_w[b], acc);
            d[side] = acc + a.dfl_bias;
        }
    }
    decode_box(a, n, an, d, load_box_in(a, n, an));
}

// The whole head output of kHeadAnchors consecutive anchors of one image per
// workgroup, when each anchor's row holds its 4*R box bins followed by its C
// class scores (row stride S floats, the Detect head's [anchor][144] concat):
// the rows are read once, coalesced, into LDS (row pitch S + 1 floats, so the
// per-anchor reads below hit distinct banks); lane (side, anchor) takes one
// side's DFL expectation, kHeadAnchors lanes decode the boxes, and the class sigmoids
// are written class-major with consecutive lanes on consecutive anchors.
constexpr int kHeadAnchors = 16;
constexpr int kHeadMaxRow = 252;  // floats per anchor row (S % 4 == 0, S + 1 <= 255)
constexpr int kHeadThreads = 256;  // lanes a workgroup
constexpr int kHeadLoads = (kHeadAnchors * kHeadMaxRow / 4 + kHeadThreads - 1) / kHeadThreads;  // float4 loads per lane
static_assert(4 * kHeadAnchors <= kHeadThreads, "one lane per (side, anchor) in the DFL phase");
template <int R>
__global__ __launch_bounds__(kHeadThreads) void detect_head_kernel(DetectDecodeArgs a, int32_t A, int32_t C, int32_t S) {
    extern __shared__ __attribute__((aligned(16))) float rows[];
    __shared__ float dist[4][kHeadAnchors];
    const int tid = threadIdx.x;
    const int32_t tiles = (A + kHeadAnchors - 1) / kHeadAnchors;
    // workgroups go round-robin over the 8 XCDs: each XCD takes a contiguous
    // range of anchor tiles, so the 64-byte runs that neighbouring tiles
    // write into one class row meet in the same L2
    const int32_t bid = xcd_block(blockIdx.x, gridDim.x);
    const int32_t n = bid / tiles;
    const int32_t a0 = (bid - n * tiles) * kHeadAnchors;
    const int cnt = min(kHeadAnchors, A - a0);
    const int P = S + 1;
    const float4* src = reinterpret_cast<const float4*>(a.x.ptr + n * a.x.str[0] + static_cast<int64_t>(a0) * S);
    // the tile's rows as float4s q = (row r, chunk j): every load of this
    // lane issued before the first LDS store, so their latencies overlap;
    // r = q / (S/4) as (q + 0.5) * (4/S) in fp32, exact for q < 2^12
    const int S4 = S / 4;
    const int q4 = cnt * S4;
    const float inv_s4 = 1.0f / static_cast<float>(S4);
    float4 v[kHeadLoads];
#pragma unroll
    for (int k = 0; k < kHeadLoads; ++k) {
        const int q = tid + kHeadThreads * k;
        v[k] = src[q < q4 ? q : 0];
    }
    // the DFL weights (lanes of the DFL phase) and the decode inputs of
    // anchor a0 + tid (lanes of the decode phase), loaded with the rows so
    // that their latency overlaps the rows'
    float dw[R];
    if (tid < 4 * kHeadAnchors) {
#pragma unroll
        for (int i = 0; i < R; ++i) dw[i] = a.dfl_w[i];
    }
    BoxIn box{};
    if (tid < kHeadAnchors) box = load_box_in(a, n, a0 + min(tid, cnt - 1));
#pragma unroll
    for (int k = 0; k < kHeadLoads; ++k) {
        const int q = tid + kHeadThreads * k;
        if (q < q4) {
            const int r = static_cast<int>((static_cast<float>(q) + 0.5f) * inv_s4);
            float* dst = rows + r * P + 4 * (q - r * S4);
            dst[0] = v[k].x;
            dst[1] = v[k].y;
            dst[2] = v[k].z;
            dst[3] = v[k].w;
        }
    }
    __syncthreads();
    if (tid < 4 * kHeadAnchors) {
        const int an = tid % kHeadAnchors, side = tid / kHeadAnchors;
        float d = 0.0f;
        if (an < cnt) {
            float v[R];
            const float* b = rows + an * P + side * R;
#pragma unroll
            for (int i = 0; i < R; ++i) v[i] = b[i];
            d = dfl_side<R>(v, dw, a.dfl_bias);
        }
        dist[side][an] = d;
    }
    __syncthreads();
    if (tid < cnt) {
        const float d[4] = {dist[0][tid], dist[1][tid], dist[2][tid], dist[3][tid]};
        decode_box(a, n, a0 + tid, d, box);
    }
    const View& o = a.cls_out;
    float* ob = o.ptr + n * o.str[0] + static_cast<int64_t>(a0) * o.str[2];
    for (int q = tid; q < C * kHeadAnchors; q += kHeadThreads) {
        const int c = q / kHeadAnchors, an = q - c * kHeadAnchors;
        if (an < cnt) ob[c * o.str[1] + an * o.str[2]] = sigmoid_elt(rows[an * P + 4 * R + c]);
    }
}

void launch_detect_decode(const DetectDecodeArgs& a, hipStream_t s) {
    check_view(a.x, "decode x");
    check_view(a.anchors, "decode anchors");
    check_view(a.two, "decode divisor");
    check_view(a.strides, "decode strides");
    check_view(a.out, "decode out");
    if (!a.dfl_w || a.bins < 1) throw std::runtime_error("decode: missing DFL weights");
    if (a.x.rank != 4 || a.x.dims[1] != a.bins || a.x.dims[2] != 4) throw std::runtime_error("decode: x must be [N, R, 4, A]");
    const int64_t N = a.x.dims[0], A = a.x.dims[3];
    for (const View* v : {&a.anchors, &a.two, &a.strides, &a.out})
        if (v->rank != 3 || v->dims[0] != N || v->dims[2] != A) throw std::runtime_error("decode: [N, C, A] views expected");
    if (a.anchors.dims[1] != 2 || a.two.dims[1] != 2 || a.strides.dims[1] != 4 || a.out.dims[1] != 4)
        throw std::runtime_error("decode: channel counts");
    if (N * A >= (int64_t{1} << 31) || !fits_i32(a.x)) throw std::runtime_error("decode: views exceed int32 indexing");
    int64_t C = 0;
    if (a.cls.ptr) {
        check_view(a.cls, "decode class scores");
        check_view(a.cls_out, "decode class out");
        if (a.cls.rank != 3 || a.cls_out.rank != 3 || a.cls.dims[0] != N || a.cls.dims[2] != A ||
            a.cls_out.dims[0] != N || a.cls_out.dims[2] != A || a.cls_out.dims[1] != a.cls.dims[1])
            throw std::runtime_error("decode: class views must be [N, C, A]");
        C = a.cls.dims[1];
    }
    if (N * A == 0) return;
    // the fused path: rows of [4*16 box bins | C class scores], stride S
    const int64_t S = a.x.str[3];
    const bool head = C > 0 && a.bins == 16 && a.x.str[1] == 1 && a.x.str[2] == 16 && S % 4 == 0 && S >= 64 + C &&
                      S + 1 <= 255 && a.cls.ptr == a.x.ptr + 64 && a.cls.str[1] == 1 && a.cls.str[2] == S &&
                      (N == 1 || (a.cls.str[0] == a.x.str[0] && a.x.str[0] % 4 == 0)) &&
                      reinterpret_cast<uintptr_t>(a.x.ptr) % 16 == 0;
    if (head) {
        const int64_t tiles = (A + kHeadAnchors - 1) / kHeadAnchors;
        const size_t lds = sizeof(float) * kHeadAnchors * static_cast<size_t>(S + 1);
        hipLaunchKernelGGL(detect_head_kernel<16>, dim3(static_cast<unsigned>(N * tiles)), dim3(kHeadThreads), lds, s, a,
                           static_cast<int32_t>(A), static_cast<int32_t>(C), static_cast<int32_t>(S));
        return;
    }
    const dim3 grid(static_cast<unsigned>((N * A + 255) / 256));
    const bool vec16 = a.bins == 16 && a.x.str[1] == 1 && reinterpret_cast<uintptr_t>(a.x.ptr) % 16 == 0 &&
                       (N == 1 || a.x.str[0] % 4 == 0) && a.x.str[2] % 4 == 0 && (A == 1 || a.x.str[3] % 4 == 0);
    if (vec16)
        hipLaunchKernelGGL(detect_decode_kernel<16>, grid, dim3(256), 0, s, a, static_cast<int32_t>(N), static_cast<int32_t>(A));
    else
        hipLaunchKernelGGL(detect_decode_kernel<0>, grid, dim3(256), 0, s, a, static_cast<int32_t>(N), static_cast<int32_t>(A));
    if (C > 0) launch_eltwise(kEltSigmoid, a.cls_out, a.cls, a.cls, 0.0f, s);
}

// ---- TopK -------------------------------------------------------------------

namespace {

// Offset of row `r` of a view with the axis dimension left out.
__device__ __forceinline__ int64_t row_offset(const View& v, int axis, int64_t r) {
    int64_t off = 0;
    for (int d = v.rank - 1; d >= 0; --d) {
        if (d == axis) continue;
        const int64_t c = r % v.dims[d];
        r /= v.dims[d];
        off += c * v.str[d];
    }
    return off;
}

// Sort key: ascending keys = descending values, then ascending index; -0.0
// keys as +0.0 (the two compare equal, so they tie and go by index).
__device__ __forceinline__ unsigned long long topk_key(float v, int32_t i) {
    uint32_t u = __float_as_uint(v);
    if (u == 0x80000000u) u = 0u;
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);  // order-preserving
    return (static_cast<unsigned long long>(~u) << 32) | static_cast<uint32_t>(i);
}

// One workgroup per row: the row's keys in LDS (padded to a power of two
// P with keys that sort last), a bitonic sort, the first k written.
__global__ __launch_bounds__(1024) void topk_kernel(View out, View in, int axis, int64_t k, int P, bool indices) {
    extern __shared__ unsigned long long keys[];
    const int64_t r = blockIdx.x;
    const int64_t L = in.dims[axis];
    const float* src = in.ptr + row_offset(in, axis, r);
    const int64_t sa = in.str[axis];
    for (int i = threadIdx.x; i < P; i += blockDim.x)
        keys[i] = i < L ? topk_key(src[i * sa], i) : ~0ull;
    __syncthreads();
    for (int size = 2; size <= P; size <<= 1) {
        for (int j = size >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < P; i += blockDim.x) {
                const int ij = i ^ j;
                if (ij > i) {
                    const unsigned long long a = keys[i], b = keys[ij];
                    const bool up = (i & size) == 0;
                    if ((a > b) == up) {
                        keys[i] = b;
                        keys[ij] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    float* dst = out.ptr + row_offset(out, axis, r);
    const int64_t so = out.str[axis];
    for (int64_t j = threadIdx.x; j < k; j += blockDim.x) {
        const int32_t idx = static_cast<int32_t>(keys[j] & 0xffffffffull);
        dst[j * so] = indices ? static_cast<float>(idx) : src[idx * sa];
    }
}

// One lane per output element.
__global__ __launch_bounds__(256) void gather_elements_kernel(View out, View data, View idx, int axis, int64_t total) {
    for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < total; e += static_cast<int64_t>(gridDim.x) * 256) {
        int64_t rem = e, o_off = 0, i_off = 0, d_off = 0, ca = 0;
        for (int d = out.rank - 1; d >= 0; --d) {
            const int64_t c = rem % out.dims[d];
            rem /= out.dims[d];
            o_off += c * out.str[d];
            i_off += c * idx.str[d];
            if (d == axis) ca = c;
            else d_off += c * data.str[d];
        }
        (void)ca;
        const int64_t n = data.dims[axis];
        int64_t g = static_cast<int64_t>(idx.ptr[i_off]);  // toward zero
        if (g < 0) g += n;
        if (g < 0 || g >= n) g = 0;
        out.ptr[o_off] = data.ptr[d_off + g * data.str[axis]];
    }
}

}  // namespace

void launch_topk(const View& out, const View& in, int axis, int64_t k, bool indices, hipStream_t s) {
    check_view(out, "topk out");
    check_view(in, "topk in");
    if (out.rank != in.rank || axis < 0 || axis >= in.rank) throw std::runtime_error("topk: bad axis/rank");
    const int64_t L = in.dims[axis];
    if (L < 1 || L > kTopKMaxAxis) throw std::runtime_error("topk: axis length out of range");
    if (k < 1 || k > L || out.dims[axis] != k) throw std::runtime_error("topk: bad k");
    for (int d = 0; d < in.rank; ++d)
        if (d != axis && out.dims[d] != in.dims[d]) throw std::runtime_error("topk: shape mismatch");
    const int64_t rows = numel(in) / L;
    if (rows == 0) return;
    if (rows >= (int64_t{1} << 31)) throw std::runtime_error("topk: too many rows");
    int P = 2;
    while (P < L) P <<= 1;
    const size_t lds = sizeof(unsigned long long) * static_cast<size_t>(P);
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&topk_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  static_cast<int>(sizeof(unsigned long long) * kTopKMaxAxis));
    });
    hipLaunchKernelGGL(topk_kernel, dim3(static_cast<unsigned>(rows)), dim3(1024), lds, s, out, in, axis, k, P,
                       indices);
}

void launch_gather_elements(const View& out, const View& data, const View& idx, int axis, hipStream_t s) {
    check_view(out, "gather out");
    check_view(data, "gather data");
    check_view(idx, "gather indices");
    if (out.rank != data.rank || idx.rank != data.rank || axis < 0 || axis >= data.rank)
        throw std::runtime_error("gather_elements: bad axis/rank");
    for (int d = 0; d < data.rank; ++d) {
        if (out.dims[d] != idx.dims[d]) throw std::runtime_error("gather_elements: out and indices differ");
        if (d != axis && idx.dims[d] != data.dims[d]) throw std::runtime_error("gather_elements: shape mismatch");
    }
    if (data.dims[axis] < 1) throw std::runtime_error("gather_elements: empty axis");
    const int64_t total = numel(out);
    if (total == 0) return;
    hipLaunchKernelGGL(gather_elements_kernel, dim3(grid_for(total)), dim3(256), 0, s, out, data, idx, axis, total);
}

// Letterbox of one interleaved 8-bit image into a planar fp32 [3, th, tw]
// tensor (imageloader/src/preprocess.cpp:15-144): lane = one output pixel,
// three channels.  Pixels outside the scaled window take the pad value as
// is; inside, source x = dx * (1/ratio) truncated, x0 clamped to w-2, and
// (p00*w0 + p10*w1)*wy0 + (p01*w0 + p11*w1)*wy1 with the scale folded into
// the row weights, with the fused multiply-adds of letterbox_blend and
// every other product and sum rounded separately (contraction is off here:
// it would also take fx = sx - x0 from the unrounded product), as the host
// path computes it.
__global__ __launch_bounds__(256) void letterbox_kernel(LetterboxArgs a) {
#pragma clang fp contract(off)
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= a.tw * a.th) return;
    const int oy = idx / a.tw, ox = idx - oy * a.tw;
    const int dx = ox - a.px, dy = oy - a.py;
    const size_t plane = static_cast<size_t>(a.tw) * a.th;
    float v[3] = {a.pad, a.pad, a.pad};
    if (dx >= 0 && dx < a.sw && dy >= 0 && dy < a.sh) {
        const float sx = static_cast<float>(dx) * a.inv;
        int x0 = static_cast<int>(sx);
        if (x0 > a.w - 2 && a.w > 1) x0 = a.w - 2;
        const int x1 = x0 + 1 < a.w ? x0 + 1 : x0;
        const float fx = sx - static_cast<float>(x0);
        const float sy = static_cast<float>(dy) * a.inv;
        int y0 = static_cast<int>(sy);
        if (y0 > a.h - 2 && a.h > 1) y0 = a.h - 2;
        const int y1 = y0 + 1 < a.h ? y0 + 1 : y0;
        const float fy = sy - static_cast<float>(y0);
        const float wy0 = (1.0f - fy) * a.scale, wy1 = fy * a.scale;
        const float w0 = 1.0f - fx, w1 = fx;
        const uint8_t* r0 = a.src + static_cast<size_t>(y0) * a.w * a.ch;
        const uint8_t* r1 = a.src + static_cast<size_t>(y1) * a.w * a.ch;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const int sc = a.ch == 1 ? 0 : c;
            v[c] = letterbox_blend(r0[x0 * a.ch + sc], r0[x1 * a.ch + sc], r1[x0 * a.ch + sc], r1[x1 * a.ch + sc],
                                   w0, w1, wy0, wy1);
        }
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) a.dst[c * plane + idx] = v[c];
}

void launch_letterbox(const LetterboxArgs& a, hipStream_t s) {
    if (!a.src || !a.dst) throw std::runtime_error("letterbox: null pointer");
    if (a.w <= 0 || a.h <= 0 || (a.ch != 1 && a.ch != 3 && a.ch != 4)) throw std::runtime_error("letterbox: image");
    if (a.tw <= 0 || a.th <= 0 || static_cast<int64_t>(a.tw) * a.th >= (int64_t{1} << 31))
        throw std::runtime_error("letterbox: target size");
    if (a.sw < 1 || a.sh < 1 || a.px < 0 || a.py < 0 || a.px + a.sw > a.tw || a.py + a.sh > a.th)
        throw std::runtime_error("letterbox: geometry");
    const int64_t total = static_cast<int64_t>(a.tw) * a.th;
    hipLaunchKernelGGL(letterbox_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, s, a);
}

// Direct convolution: lane = one output pixel, CB output channels of the
// workgroup's channel block.  Weights are pre-packed [ceil(Cout/CB)][K][CB]
// (K = Cin*KH*KW, k = (ci, kh, kw)) so the CB weights of one k are one
// contiguous, wave-uniform read (scalar loads); each input value loaded feeds
// CB FMAs.  Index math is int32 within one image.
//
// KS = 3: 3x3 taps, the nine loads of each input channel in flight before its
// FMAs.  CL: the output block is channels-last and whole
// (and so is the residual), so each lane applies bias + activation (ACT, or
// the runtime code for kActGeneric) in registers and stores its pixel's CB
// channels as float4 runs; otherwise the 256 x CB result tile goes through
// LDS and is stored with consecutive lanes on consecutive channels.
template <int CB, int KS, bool CL, int ACT>
__global__ __launch_bounds__(256) void conv_direct_kernel(ConvDirectArgs a, int P) {
    __shared__ float tile[CL ? 1 : 256 * (CB + 1)];
    const int p0 = blockIdx.x * 256;
    const int p = p0 + threadIdx.x;
    const int cob = blockIdx.y;
    const int Co = static_cast<int>(a.y.dims[1]), Ho = static_cast<int>(a.y.dims[2]), Wo = static_cast<int>(a.y.dims[3]);
    const int Ci = static_cast<int>(a.x.dims[1]), H = static_cast<int>(a.x.dims[2]), W = static_cast<int>(a.x.dims[3]);
    const int K = Ci * a.KH * a.KW;
    const int HoWo = Ho * Wo;
    float acc[CB];
#pragma unroll
    for (int j = 0; j < CB; ++j) acc[j] = 0.0f;
    const int pc = p < P ? p : P - 1;  // lanes past the end compute a valid pixel, store nothing
    const int n = pc / HoWo;
    const int rem = pc - n * HoWo;
    const int ho = rem / Wo;
    const int wo = rem - ho * Wo;
    {
        const float* xb = a.x.ptr + static_cast<int64_t>(n) * a.x.str[0];
        const int xsc = static_cast<int>(a.x.str[1]), xsh = static_cast<int>(a.x.str[2]);
        const int xsw = static_cast<int>(a.x.str[3]);
        const int hi0 = ho * a.sh - a.ph, wi0 = wo * a.sw - a.pw;
        const float* wk = a.wpk + static_cast<int64_t>(cob) * K * CB;
        if constexpr (KS > 0) {
            int off[KS * KS];
            bool tok[KS * KS];
#pragma unroll
            for (int kh = 0; kh < KS; ++kh)
#pragma unroll
                for (int kw = 0; kw < KS; ++kw) {
                    const int hi = hi0 + kh * a.dh, wi = wi0 + kw * a.dw;
                    tok[kh * KS + kw] = (static_cast<unsigned>(hi) < static_cast<unsigned>(H)) &
                                        (static_cast<unsigned>(wi) < static_cast<unsigned>(W));
                    off[kh * KS + kw] = tok[kh * KS + kw] ? hi * xsh + wi * xsw : 0;
                }
            for (int c = 0; c < Ci; ++c, wk += KS * KS * CB) {
                const float* xc = xb + c * xsc;
                float xv[KS * KS];
#pragma unroll
                for (int t = 0; t < KS * KS; ++t) {
                    const float v = xc[off[t]];
                    xv[t] = tok[t] ? v : 0.0f;
                }
#pragma unroll
                for (int t = 0; t < KS * KS; ++t)
#pragma unroll
                    for (int j = 0; j < CB; ++j) acc[j] += xv[t] * wk[t * CB + j];
            }
        } else {
            for (int c = 0; c < Ci; ++c) {
                for (int kh = 0; kh < a.KH; ++kh) {
                    const int hi = hi0 + kh * a.dh;
                    const bool hok = static_cast<unsigned>(hi) < static_cast<unsigned>(H);
                    for (int kw = 0; kw < a.KW; ++kw, wk += CB) {
                        const int wi = wi0 + kw * a.dw;
                        const bool ok = hok && static_cast<unsigned>(wi) < static_cast<unsigned>(W);
                        const float xv = ok ? xb[c * xsc + hi * xsh + wi * xsw] : 0.0f;
#pragma unroll
                        for (int j = 0; j < CB; ++j) acc[j] += xv * wk[j];
                    }
                }
            }
        }
    }
    if constexpr (CL) {
        if (p >= P) return;
        const int c0 = cob * CB;
        float* yp = a.y.ptr + static_cast<int64_t>(n) * a.y.str[0] + static_cast<int64_t>(ho) * a.y.str[2] +
                    static_cast<int64_t>(wo) * a.y.str[3] + c0;
        const float* rp = a.res.ptr ? a.res.ptr + static_cast<int64_t>(n) * a.res.str[0] +
                                          static_cast<int64_t>(ho) * a.res.str[2] +
                                          static_cast<int64_t>(wo) * a.res.str[3] + c0
                                    : nullptr;
#pragma unroll
        for (int q = 0; q < CB / 4; ++q) {
            float4 v;
            float* vv = reinterpret_cast<float*>(&v);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                vv[e] = act_fixed<ACT>(acc[4 * q + e] + (a.bias ? a.bias[c0 + 4 * q + e] : 0.0f), a.act, a.slope);
            if (rp) {
                const float4 r = reinterpret_cast<const float4*>(rp)[q];
                v.x += r.x;
                v.y += r.y;
                v.z += r.z;
                v.w += r.w;
            }
            reinterpret_cast<float4*>(yp)[q] = v;
        }
        return;
    } else {
#pragma unroll
        for (int j = 0; j < CB; ++j) tile[threadIdx.x * (CB + 1) + j] = acc[j];
        __syncthreads();
        const int nc = min(CB, Co - cob * CB);
        for (int idx = threadIdx.x; idx < 256 * CB; idx += 256) {
            const int pl = idx / CB, j = idx - (idx / CB) * CB;
            const int pp = p0 + pl;
            if (pp >= P || j >= nc) continue;
            const int co = cob * CB + j;
            const int nn = pp / HoWo;
            const int rr = pp - nn * HoWo;
            const int oh = rr / Wo;
            const int ow = rr - oh * Wo;
            float v = apply_act(tile[pl * (CB + 1) + j] + (a.bias ? a.bias[co] : 0.0f), a.act, a.slope);
            if (a.res.ptr)
                v += a.res.ptr[static_cast<int64_t>(nn) * a.res.str[0] + static_cast<int64_t>(co) * a.res.str[1] +
                               static_cast<int64_t>(oh) * a.res.str[2] + static_cast<int64_t>(ow) * a.res.str[3]];
            a.y.ptr[static_cast<int64_t>(nn) * a.y.str[0] + static_cast<int64_t>(co) * a.y.str[1] +
                    static_cast<int64_t>(oh) * a.y.str[2] + static_cast<int64_t>(ow) * a.y.str[3]] = v;
        }
    }
}

namespace {

template <int CB, int KS, bool CL>
void launch_direct_act(const ConvDirectArgs& a, dim3 grid, int P, hipStream_t s) {
    if (CL && a.act == kActSilu)
        hipLaunchKernelGGL((conv_direct_kernel<CB, KS, CL, kActSilu>), grid, dim3(256), 0, s, a, P);
    else
        hipLaunchKernelGGL((conv_direct_kernel<CB, KS, CL, kActGeneric>), grid, dim3(256), 0, s, a, P);
}

template <int CB>
void launch_direct_cb(const ConvDirectArgs& a, dim3 grid, int P, bool k3, bool cl, hipStream_t s) {
    if (k3 && cl) launch_direct_act<CB, 3, true>(a, grid, P, s);
    else if (k3) launch_direct_act<CB, 3, false>(a, grid, P, s);
    else if (cl) launch_direct_act<CB, 0, true>(a, grid, P, s);
    else launch_direct_act<CB, 0, false>(a, grid, P, s);
}

}  // namespace

// Grouped convolution (groups > 1, few channels per group: depthwise and
// the like): lane = (output pixel, output channel), channel fastest, so that
// channels-last inputs, the [tap][ci][Cout] weights and channels-last outputs
// are read and written at consecutive addresses across a wave.  The sum
// starts from the bias and runs over the taps (kh, kw) in order, then the
// group's input channels.  Input offsets within one image fit int32
// (checked by the launcher).
__global__ __launch_bounds__(256) void conv_grouped_kernel(ConvDirectArgs a, int32_t total) {
    const int32_t idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    const int32_t C = static_cast<int32_t>(a.y.dims[1]), Ho = static_cast<int32_t>(a.y.dims[2]),
                  Wo = static_cast<int32_t>(a.y.dims[3]);
    const int32_t co = idx % C;
    int32_t t = idx / C;
    const int32_t wo = t % Wo;
    t /= Wo;
    const int32_t ho = t % Ho;
    const int32_t n = t / Ho;
    const int32_t cout_g = C / a.groups, cin_g = static_cast<int32_t>(a.x.dims[1]) / a.groups;
    const int32_t H = static_cast<int32_t>(a.x.dims[2]), W = static_cast<int32_t>(a.x.dims[3]);
    const int32_t xs1 = static_cast<int32_t>(a.x.str[1]), xs2 = static_cast<int32_t>(a.x.str[2]),
                  xs3 = static_cast<int32_t>(a.x.str[3]);
    const float* xb = a.x.ptr + n * a.x.str[0] + static_cast<int64_t>(co / cout_g) * cin_g * a.x.str[1];
    float acc = a.bias ? a.bias[co] : 0.0f;
    for (int kh = 0; kh < a.KH; ++kh) {
        const int32_t ih = ho * a.sh - a.ph + kh * a.dh;
        if (static_cast<uint32_t>(ih) >= static_cast<uint32_t>(H)) continue;
        for (int kw = 0; kw < a.KW; ++kw) {
            const int32_t iw = wo * a.sw - a.pw + kw * a.dw;
            if (static_cast<uint32_t>(iw) >= static_cast<uint32_t>(W)) continue;
            const float* xp = xb + ih * xs2 + iw * xs3;
            const float* wp = a.wpk + static_cast<int64_t>((kh * a.KW + kw) * cin_g) * C + co;
            for (int ci = 0; ci < cin_g; ++ci) acc = fmaf(xp[ci * xs1], wp[static_cast<int64_t>(ci) * C], acc);
        }
    }
    float v = apply_act(acc, a.act, a.slope);
    if (a.res.ptr) v += a.res.ptr[n * a.res.str[0] + co * a.res.str[1] + ho * a.res.str[2] + wo * a.res.str[3]];
    a.y.ptr[n * a.y.str[0] + co * a.y.str[1] + ho * a.y.str[2] + wo * a.y.str[3]] = v;
}

// Direct-kernel weight layouts from the OIHW weights [Cout][Cin/G][KH][KW]:
// groups == 1: [ceil(Cout/CB)][Cin*KH*KW][CB] (CB = direct_cb(Cout), zero
// padded past Cout); groups > 1: [KH*KW][Cin/G][Cout].  One lane per
// destination element.
__global__ void pack_direct_weights_kernel(float* dst, const float* w, int Cout, int Cin_g, int KH, int KW, int groups,
                                           int cb, int64_t total) {
    const int K = Cin_g * KH * KW;
    const int taps = KH * KW;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        float v = 0.0f;
        if (groups > 1) {
            const int co = static_cast<int>(i % Cout);
            const int64_t t = i / Cout;
            const int ci = static_cast<int>(t % Cin_g);
            const int tap = static_cast<int>(t / Cin_g);
            v = w[(static_cast<int64_t>(co) * Cin_g + ci) * taps + tap];
        } else {
            const int c = static_cast<int>(i % cb);
            const int64_t t = i / cb;
            const int kk = static_cast<int>(t % K);
            const int co = static_cast<int>(t / K) * cb + c;
            if (co < Cout) v = w[static_cast<int64_t>(co) * K + kk];
        }
        dst[i] = v;
    }
}

void launch_pack_direct_weights(float* dst, const float* w, int Cout, int Cin_g, int KH, int KW, int groups,
                                hipStream_t s) {
    if (!dst || !w || Cout <= 0 || Cin_g <= 0 || KH <= 0 || KW <= 0 || groups <= 0)
        throw std::runtime_error("pack_direct_weights: bad arguments");
    const int K = Cin_g * KH * KW;
    const int64_t total =
        groups > 1 ? grouped_direct_packed_elems(Cout, Cin_g, KH, KW) : direct_packed_elems(Cout, K);
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 65535));
    hipLaunchKernelGGL(pack_direct_weights_kernel, dim3(blocks), dim3(256), 0, s, dst, w, Cout, Cin_g, KH, KW, groups,
                       direct_cb(Cout), total);
}

void launch_conv_direct(const ConvDirectArgs& a, hipStream_t s) {
    check_view(a.x, "conv_direct x");
    check_view(a.y, "conv_direct y");
    if (!a.wpk) throw std::runtime_error("conv_direct: null weights");
    if (a.x.rank != 4 || a.y.rank != 4) throw std::runtime_error("conv_direct: rank 4 views expected");
    if (a.res.ptr && a.res.rank != 4) throw std::runtime_error("conv_direct: rank 4 residual expected");
    const int64_t P = a.y.dims[0] * a.y.dims[2] * a.y.dims[3];
    if (P == 0 || a.y.dims[1] == 0) return;
    auto extent = [](const View& v) {
        int64_t e = 1;
        for (int d = 1; d < 4; ++d) e += (v.dims[d] - 1) * std::abs(v.str[d]);
        return e;
    };
    if (a.groups > 1) {
        if (a.x.dims[1] % a.groups != 0 || a.y.dims[1] % a.groups != 0)
            throw std::runtime_error("conv_direct: channels not divisible by groups");
        if (a.res.ptr && (a.res.dims[1] != a.y.dims[1] || a.res.dims[2] != a.y.dims[2]))
            throw std::runtime_error("conv_direct: residual shape");
        const int64_t total = P * a.y.dims[1];
        if (total >= (int64_t{1} << 31) || extent(a.x) >= (int64_t{1} << 31))
            throw std::runtime_error("conv_direct: shape exceeds int32 indexing");
        hipLaunchKernelGGL(conv_grouped_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, s, a,
                           static_cast<int32_t>(total));
        return;
    }
    const int cb = direct_cb(static_cast<int>(a.y.dims[1]));
    if (P >= (int64_t{1} << 31) || extent(a.x) >= (int64_t{1} << 31) ||
        a.x.dims[1] * a.KH * a.KW * 64 >= (int64_t{1} << 31))
        throw std::runtime_error("conv_direct: shape exceeds int32 indexing");
    const dim3 grid(static_cast<unsigned>((P + 255) / 256), static_cast<unsigned>((a.y.dims[1] + cb - 1) / cb));
    const int Pi = static_cast<int>(P);
    const bool k3 = a.KH == 3 && a.KW == 3;
    // channels-last output (and residual) with whole 16-byte aligned channel blocks
    auto cl_view = [&](const View& v) {
        return v.str[1] == 1 && v.str[0] % 4 == 0 && v.str[2] % 4 == 0 && v.str[3] % 4 == 0 &&
               reinterpret_cast<uintptr_t>(v.ptr) % 16 == 0;
    };
    const bool cl = a.y.dims[1] % cb == 0 && cl_view(a.y) && (!a.res.ptr || cl_view(a.res));
    switch (cb) {
        case 16: launch_direct_cb<16>(a, grid, Pi, k3, cl, s); break;
        case 32: launch_direct_cb<32>(a, grid, Pi, k3, cl, s); break;
        case 48: launch_direct_cb<48>(a, grid, Pi, k3, cl, s); break;
        default: launch_direct_cb<64>(a, grid, Pi, k3, cl, s); break;
    }
}

}  // namespace k
}  // namespace pdefa
