// Implicit-GEMM convolution on CDNA4 fp32 matrix cores (v_mfma_f32_32x32x2_f32).
//
// GEMM view of an NHWC convolution: C[m, co] = sum_k A[m, k] * B[k, co] with
// m = (n, ho, wo), k = (kh, kw, ci) and A gathered on the fly from the input
// (no im2col buffer).  One workgroup = 4 waves (256 lanes) computes a BM x BN
// output tile; each wave owns a (BM/WAVES_M) x (BN/WAVES_N) sub-tile made of
// 32x32 MFMA blocks.  K advances BK = 16 at a time through double-buffered LDS
// tiles stored k-contiguous ([row][BK + 4]) so each lane feeds four MFMA steps
// from one 16-byte LDS read: lane half h supplies k = 8q + 4h + j for step
// (q, j), the same k for A and B, which covers the 16 k of a tile exactly once.
//
// Epilogue: + bias, activation, + optional residual (the C2f bottleneck add),
// stored through the output view's strides so the result can land directly in
// a channel slice of a concat buffer.
#include "../kernels.hpp"
#include "act.hpp"

#include <stdexcept>
#include <string>

namespace pdefa {
namespace k {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace {

constexpr int BK = kConvBK;
constexpr int LDS_STRIDE = BK + 4;  // floats; keeps rows 16-byte aligned

}  // namespace

template <int BM, int BN, int WAVES_M, bool VEC>
__global__ __launch_bounds__(256) void conv_mfma_kernel(ConvArgs a) {
    constexpr int WAVES_N = 4 / WAVES_M;
    constexpr int WM = BM / WAVES_M;
    constexpr int WN = BN / WAVES_N;
    constexpr int TM = WM / 32;
    constexpr int TN = WN / 32;
    constexpr int A_ROWS = BM / 64;             // rows per thread (4 lanes per row)
    constexpr int B_LOADS = (BN * 4 + 255) / 256;
    static_assert(TM >= 1 && TN >= 1 && WM % 32 == 0 && WN % 32 == 0, "tile");

    __shared__ __attribute__((aligned(16))) float As[2][BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) float Bs[2][BN * LDS_STRIDE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wave_m = wave % WAVES_M;
    const int wave_n = wave / WAVES_M;
    const int HoWo = a.Ho * a.Wo;
    const int M = a.N * HoWo;
    const int m0 = blockIdx.x * BM;
    const int ntile = blockIdx.y;
    const int n0 = ntile * BN;
    const int kt_begin = blockIdx.z * a.kt_per_split;
    const int kt_end = min(a.ktiles, kt_begin + a.kt_per_split);
    const int taps = a.KH * a.KW;

    // ---- A-loader state: this thread loads float4 chunk `chunk` of rows r0 + 64 i.
    const int chunk = tid & 3;
    int row_hi0[A_ROWS];
    int row_wi0[A_ROWS];
    const float* row_base[A_ROWS];
    bool row_ok[A_ROWS];
#pragma unroll
    for (int r = 0; r < A_ROWS; ++r) {
        const int m = m0 + (tid >> 2) + 64 * r;
        row_ok[r] = m < M;
        const int mm = row_ok[r] ? m : 0;
        const int n = mm / HoWo;
        const int rem = mm - n * HoWo;
        const int ho = rem / a.Wo;
        const int wo = rem - ho * a.Wo;
        row_hi0[r] = ho * a.sh - a.ph;
        row_wi0[r] = wo * a.sw - a.pw;
        row_base[r] = a.x + static_cast<int64_t>(n) * a.x_sn;
    }
    int tap = 0, ci = 0, kh = 0, kw = 0;
    if (VEC) {
        const int k0 = kt_begin * BK + chunk * 4;
        tap = k0 / a.Cin;
        ci = k0 - tap * a.Cin;
        kh = tap / a.KW;
        kw = tap - kh * a.KW;
    }

    const float* wtile = a.wpk + static_cast<int64_t>(ntile) * a.ktiles * (BN * BK);

    floatx4 areg[A_ROWS];
    floatx4 breg[B_LOADS];

    auto load_tiles = [&](int kt) {
        if (VEC) {
            const int dy = kh * a.dh, dx = kw * a.dw;
            const bool tap_ok = tap < taps;
#pragma unroll
            for (int r = 0; r < A_ROWS; ++r) {
                const int hi = row_hi0[r] + dy;
                const int wi = row_wi0[r] + dx;
                const bool ok = row_ok[r] && tap_ok && static_cast<unsigned>(hi) < static_cast<unsigned>(a.H) &&
                                static_cast<unsigned>(wi) < static_cast<unsigned>(a.W);
                if (ok) {
                    areg[r] = *reinterpret_cast<const floatx4*>(
                        row_base[r] + static_cast<int64_t>(hi) * a.x_sh + static_cast<int64_t>(wi) * a.x_sw + ci);
                } else {
                    areg[r] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
                }
            }
        } else {
#pragma unroll
            for (int r = 0; r < A_ROWS; ++r) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int kk = kt * BK + chunk * 4 + e;
                    float v = 0.0f;
                    if (row_ok[r] && kk < a.K) {
                        const int t = kk / a.Cin;
                        const int c = kk - t * a.Cin;
                        const int yh = t / a.KW;
                        const int xw = t - yh * a.KW;
                        const int hi = row_hi0[r] + yh * a.dh;
                        const int wi = row_wi0[r] + xw * a.dw;
                        if (static_cast<unsigned>(hi) < static_cast<unsigned>(a.H) &&
                            static_cast<unsigned>(wi) < static_cast<unsigned>(a.W)) {
                            v = row_base[r][static_cast<int64_t>(hi) * a.x_sh + static_cast<int64_t>(wi) * a.x_sw + c];
                        }
                    }
                    areg[r][e] = v;
                }
            }
        }
        const float* bt = wtile + static_cast<int64_t>(kt) * (BN * BK);
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) {
            const int idx = tid + 256 * i;
            if (idx < BN * 4) breg[i] = *reinterpret_cast<const floatx4*>(bt + idx * 4);
        }
    };
    auto advance_k = [&]() {
        if (VEC) {
            ci += BK;
            while (ci >= a.Cin) {
                ci -= a.Cin;
                ++tap;
                if (++kw == a.KW) {
                    kw = 0;
                    ++kh;
                }
            }
        }
    };
    auto store_tiles = [&](int buf) {
#pragma unroll
        for (int r = 0; r < A_ROWS; ++r) {
            const int row = (tid >> 2) + 64 * r;
            *reinterpret_cast<floatx4*>(&As[buf][row * LDS_STRIDE + chunk * 4]) = areg[r];
        }
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) {
            const int idx = tid + 256 * i;
            if (idx < BN * 4) {
                *reinterpret_cast<floatx4*>(&Bs[buf][(idx >> 2) * LDS_STRIDE + (idx & 3) * 4]) = breg[i];
            }
        }
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    int cur = 0;
    if (kt_begin < kt_end) {
        load_tiles(kt_begin);
        advance_k();
        store_tiles(0);
        __syncthreads();
    }
    const int half = lane >> 5;
    const int l32 = lane & 31;
    for (int kt = kt_begin; kt < kt_end; ++kt) {
        const bool more = kt + 1 < kt_end;
        if (more) {
            load_tiles(kt + 1);
            advance_k();
        }
        const float* Ab = As[cur];
        const float* Bb = Bs[cur];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            floatx4 av[TM], bv[TN];
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
                const int row = wave_m * WM + tm * 32 + l32;
                av[tm] = *reinterpret_cast<const floatx4*>(&Ab[row * LDS_STRIDE + q * 8 + half * 4]);
            }
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                const int col = wave_n * WN + tn * 32 + l32;
                bv[tn] = *reinterpret_cast<const floatx4*>(&Bb[col * LDS_STRIDE + q * 8 + half * 4]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                    for (int tn = 0; tn < TN; ++tn)
                        acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[tm][j], bv[tn][j], acc[tm][tn], 0, 0, 0);
        }
        if (more) store_tiles(cur ^ 1);
        __syncthreads();
        cur ^= 1;
    }

    // ---- epilogue.  32x32 block register e of lane l holds
    // row 8*(e/4) + 4*(l/32) + e%4, column l%32.
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int row = wave_m * WM + tm * 32 + (e >> 2) * 8 + half * 4 + (e & 3);
            const int m = m0 + row;
            if (m >= M) continue;
            if (a.splits > 1) {
                float* wrow = a.ws + (static_cast<int64_t>(blockIdx.z) * M + m) * a.Cout;
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) {
                    const int col = n0 + wave_n * WN + tn * 32 + l32;
                    if (col < a.Cout) wrow[col] = acc[tm][tn][e];
                }
                continue;
            }
            const int n = m / HoWo;
            const int rem = m - n * HoWo;
            const int ho = rem / a.Wo;
            const int wo = rem - ho * a.Wo;
            float* yrow = a.y + static_cast<int64_t>(n) * a.y_sn + static_cast<int64_t>(ho) * a.y_sh +
                          static_cast<int64_t>(wo) * a.y_sw;
            const float* rrow = a.res ? a.res + static_cast<int64_t>(n) * a.r_sn + static_cast<int64_t>(ho) * a.r_sh +
                                            static_cast<int64_t>(wo) * a.r_sw
                                      : nullptr;
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                const int col = n0 + wave_n * WN + tn * 32 + l32;
                if (col < a.Cout) {
                    float v = apply_act(acc[tm][tn][e] + a.bias[col], a.act, a.slope);
                    if (rrow) v += rrow[col];
                    yrow[col] = v;
                }
            }
        }
    }
}

// Sums split-K partials in split order, then bias + activation + residual.
__global__ __launch_bounds__(256) void conv_splitk_reduce(ConvArgs a) {
    const int HoWo = a.Ho * a.Wo;
    const int64_t M = static_cast<int64_t>(a.N) * HoWo;
    const int64_t total = M * a.Cout;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t m = i / a.Cout;
        const int col = static_cast<int>(i - m * a.Cout);
        float s = 0.0f;
        for (int z = 0; z < a.splits; ++z) s += a.ws[(z * M + m) * a.Cout + col];
        const int n = static_cast<int>(m / HoWo);
        const int rem = static_cast<int>(m - static_cast<int64_t>(n) * HoWo);
        const int ho = rem / a.Wo;
        const int wo = rem - ho * a.Wo;
        float v = apply_act(s + a.bias[col], a.act, a.slope);
        if (a.res) v += a.res[n * a.r_sn + ho * a.r_sh + wo * a.r_sw + col];
        a.y[n * a.y_sn + ho * a.y_sh + wo * a.y_sw + col] = v;
    }
}

int conv_tile_bm(int tile) {
    switch (tile) {
        case kTile128x32: case kTile128x64: case kTile128x128: return 128;
        case kTile64x64: case kTile64x128: return 64;
    }
    return 0;
}
int conv_tile_bn(int tile) {
    switch (tile) {
        case kTile128x32: return 32;
        case kTile128x64: case kTile64x64: return 64;
        case kTile128x128: case kTile64x128: return 128;
    }
    return 0;
}

int64_t packed_weight_elems(int Cout, int K, int bn) {
    const int64_t cout_pad = (Cout + bn - 1) / bn * bn;
    const int64_t k_pad = (K + BK - 1) / BK * BK;
    return cout_pad * k_pad;
}

namespace {

template <int BM, int BN, int WAVES_M>
void launch_tile(const ConvArgs& a, bool vec, dim3 grid, hipStream_t s) {
    if (vec)
        hipLaunchKernelGGL((conv_mfma_kernel<BM, BN, WAVES_M, true>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((conv_mfma_kernel<BM, BN, WAVES_M, false>), grid, dim3(256), 0, s, a);
}

void fail(const std::string& m) { throw std::runtime_error("conv_mfma: " + m); }

}  // namespace

void launch_conv_mfma(const ConvArgs& a, int tile, bool vec, hipStream_t s) {
    const int bm = conv_tile_bm(tile), bn = conv_tile_bn(tile);
    if (bm == 0) fail("unknown tile");
    if (!a.x || !a.y || !a.wpk || !a.bias) fail("null pointer");
    if (a.N <= 0 || a.H <= 0 || a.W <= 0 || a.Cin <= 0 || a.Ho <= 0 || a.Wo <= 0 || a.Cout <= 0) fail("empty shape");
    if (a.K != a.KH * a.KW * a.Cin) fail("K mismatch");
    if (a.ktiles != (a.K + BK - 1) / BK) fail("ktiles mismatch");
    const int64_t M = static_cast<int64_t>(a.N) * a.Ho * a.Wo;
    if (M >= (int64_t{1} << 31)) fail("M too large");
    if (a.splits < 1 || a.kt_per_split < 1 || static_cast<int64_t>(a.splits) * a.kt_per_split < a.ktiles) fail("bad split");
    if (a.splits > 1 && !a.ws) fail("split-K without workspace");
    if (vec) {
        if (a.Cin % 4 != 0) fail("vector loads need Cin % 4 == 0");
        if ((reinterpret_cast<uintptr_t>(a.x) & 15) || (a.x_sn & 3) || (a.x_sh & 3) || (a.x_sw & 3))
            fail("vector loads need 16-byte aligned rows");
    }
    const dim3 grid(static_cast<unsigned>((M + bm - 1) / bm), static_cast<unsigned>((a.Cout + bn - 1) / bn),
                    static_cast<unsigned>(a.splits));
    switch (tile) {
        case kTile128x32: launch_tile<128, 32, 4>(a, vec, grid, s); break;
        case kTile128x64: launch_tile<128, 64, 2>(a, vec, grid, s); break;
        case kTile128x128: launch_tile<128, 128, 2>(a, vec, grid, s); break;
        case kTile64x64: launch_tile<64, 64, 2>(a, vec, grid, s); break;
        case kTile64x128: launch_tile<64, 128, 2>(a, vec, grid, s); break;
    }
    if (a.splits > 1) {
        const int64_t total = M * a.Cout;
        const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 65535));
        hipLaunchKernelGGL(conv_splitk_reduce, dim3(blocks), dim3(256), 0, s, a);
    }
}

__global__ void pack_conv_weights_kernel(float* dst, const float* w, int Cout, int Cin, int KH, int KW,
                                         int bn, int ktiles, int64_t total) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int kk = static_cast<int>(i % BK);
        int64_t t = i / BK;
        const int nn = static_cast<int>(t % bn);
        t /= bn;
        const int kt = static_cast<int>(t % ktiles);
        const int nt = static_cast<int>(t / ktiles);
        const int co = nt * bn + nn;
        const int kidx = kt * BK + kk;
        const int K = KH * KW * Cin;
        float v = 0.0f;
        if (co < Cout && kidx < K) {
            const int tap = kidx / Cin;
            const int c = kidx - tap * Cin;
            const int kh = tap / KW;
            const int kw = tap - kh * KW;
            v = w[((static_cast<int64_t>(co) * Cin + c) * KH + kh) * KW + kw];
        }
        dst[i] = v;
    }
}

__global__ void pack_gemm_b_kernel(float* dst, const float* b, int K, int N, int bn, int ktiles, int64_t total) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int kk = static_cast<int>(i % BK);
        int64_t t = i / BK;
        const int nn = static_cast<int>(t % bn);
        t /= bn;
        const int kt = static_cast<int>(t % ktiles);
        const int nt = static_cast<int>(t / ktiles);
        const int col = nt * bn + nn;
        const int kidx = kt * BK + kk;
        dst[i] = (col < N && kidx < K) ? b[static_cast<int64_t>(kidx) * N + col] : 0.0f;
    }
}

void launch_pack_conv_weights(float* dst, const float* w, int Cout, int Cin, int KH, int KW, int bn,
                              hipStream_t s) {
    const int K = KH * KW * Cin;
    const int ktiles = (K + BK - 1) / BK;
    const int64_t total = packed_weight_elems(Cout, K, bn);
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 65535));
    hipLaunchKernelGGL(pack_conv_weights_kernel, dim3(blocks), dim3(256), 0, s, dst, w, Cout, Cin, KH, KW, bn,
                       ktiles, total);
}

void launch_pack_gemm_b(float* dst, const float* b, int K, int N, int bn, hipStream_t s) {
    const int ktiles = (K + BK - 1) / BK;
    const int64_t total = packed_weight_elems(N, K, bn);
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 65535));
    hipLaunchKernelGGL(pack_gemm_b_kernel, dim3(blocks), dim3(256), 0, s, dst, b, K, N, bn, ktiles, total);
}

}  // namespace k
}  // namespace pdefa
