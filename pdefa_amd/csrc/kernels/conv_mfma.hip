// Implicit-GEMM convolution on CDNA4 fp32 matrix cores (v_mfma_f32_32x32x2_f32).
//
// GEMM view of an NHWC convolution: C[m, co] = sum_k A[m, k] * B[k, co] with
// m = (n, ho, wo), k = (kh, kw, ci) and A gathered on the fly from the input
// (no im2col buffer).  One workgroup = 4 waves (256 lanes) computes a BM x BN
// output tile; each wave owns a (BM/WAVES_M) x (BN/WAVES_N) sub-tile made of
// 32x32 MFMA blocks.
//
// K advances BK = 32 at a time.  Global loads run two K-tiles ahead of the
// MFMAs (two register stages) into two LDS stages whose rows are padded to 36
// floats; each lane feeds four MFMA steps from one 16-byte LDS read: lane half
// h supplies k = 8q + 4h + j for step (q, j), the same k for A and B, which
// covers the 32 k of a tile exactly once.
//
// Split-K (small-M deep layers): each split writes its partial tile to a
// workspace and a reduce kernel sums the partials in split order (so the result
// does not depend on scheduling) and applies the epilogue.  An in-kernel
// "last split reduces" fixup was measured slower: on this multi-XCD part the
// device-scope release/acquire it needs writes back and invalidates the L2.
//
// Epilogue: + bias, activation, + optional residual (the C2f bottleneck add),
// stored through the output view's strides so the result can land directly in
// a channel slice of a concat buffer.
#include "../kernels.hpp"
#include "act.hpp"

#include <mutex>
#include <stdexcept>
#include <string>
#include <type_traits>

namespace pdefa {
namespace k {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace {

constexpr int BK = kConvBK;         // 32
constexpr int CHUNKS = BK / 4;      // float4 chunks per tile row
constexpr int LDS_STRIDE = BK + 4;  // floats; 16-byte aligned rows, conflict-free float4 reads

template <int BM, int BN>
constexpr size_t lds_bytes() {
    return sizeof(float) * 2 * (BM + BN) * LDS_STRIDE;
}

}  // namespace

template <int BM, int BN, int WAVES_M, bool VEC>
__global__ __launch_bounds__(256) void conv_mfma_kernel(ConvArgs a) {
    constexpr int WAVES_N = 4 / WAVES_M;
    constexpr int WM = BM / WAVES_M;
    constexpr int WN = BN / WAVES_N;
    constexpr int TM = WM / 32;
    constexpr int TN = WN / 32;
    constexpr int ROW_STEP = 256 / CHUNKS;   // rows covered by one pass of 256 lanes
    constexpr int A_ROWS = BM / ROW_STEP;    // A float4 loads per lane per tile
    constexpr int B_LOADS = (BN * CHUNKS + 255) / 256;
    static_assert(TM >= 1 && TN >= 1 && WM % 32 == 0 && WN % 32 == 0, "tile");
    static_assert(BM % ROW_STEP == 0, "BM");

    extern __shared__ __attribute__((aligned(16))) float smem[];
    float* As[2] = {smem, smem + BM * LDS_STRIDE};
    float* Bs[2] = {smem + 2 * BM * LDS_STRIDE, smem + 2 * BM * LDS_STRIDE + BN * LDS_STRIDE};

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

    // ---- A loader: this lane loads float4 chunk `chunk` of rows r0 + ROW_STEP*i.
    // Offsets within one image fit in int32 (checked by the launcher).
    const int chunk = tid % CHUNKS;
    const int r0 = tid / CHUNKS;
    int row_hi0[A_ROWS];
    int row_wi0[A_ROWS];
    int row_off0[A_ROWS];
    const float* row_base[A_ROWS];
    bool row_ok[A_ROWS];
    const int xsh = static_cast<int>(a.x_sh), xsw = static_cast<int>(a.x_sw);
#pragma unroll
    for (int r = 0; r < A_ROWS; ++r) {
        const int m = m0 + r0 + ROW_STEP * r;
        row_ok[r] = m < M;
        const int mm = row_ok[r] ? m : 0;
        const int n = mm / HoWo;
        const int rem = mm - n * HoWo;
        const int ho = rem / a.Wo;
        const int wo = rem - ho * a.Wo;
        row_hi0[r] = ho * a.sh - a.ph;
        row_wi0[r] = wo * a.sw - a.pw;
        row_off0[r] = row_hi0[r] * xsh + row_wi0[r] * xsw;
        row_base[r] = a.x + static_cast<int64_t>(n) * a.x_sn;
    }
    // (tap, ci, kh, kw) of this lane's chunk in the next tile to load
    int tap = 0, ci = 0, kh = 0, kw = 0;
    if (VEC) {
        const int k0 = kt_begin * BK + chunk * 4;
        tap = k0 / a.Cin;
        ci = k0 - tap * a.Cin;
        kh = tap / a.KW;
        kw = tap - kh * a.KW;
    }
    const bool cin_ge_bk = a.Cin >= BK;  // then a tile advance wraps Cin at most once

    const float* wtile = a.wpk + static_cast<int64_t>(ntile) * a.ktiles * (BN * BK);

    // Register stages.  Loads are issued unconditionally (out-of-range A rows
    // read the tensor base, tiles past the end re-read the last tile) and the
    // in-range mask is applied when the stage is written to LDS, so the loads
    // of the newest tile stay in flight while the previous stage is stored.
    floatx4 areg[2][A_ROWS];
    floatx4 breg[2][B_LOADS];
    unsigned amask[2] = {0u, 0u};

    auto load_tile = [&](int kt, floatx4* ar, floatx4* br, unsigned& mask) {
        unsigned mk = 0;
        if (VEC) {
            const int dy = kh * a.dh, dx = kw * a.dw;
            const int doff = dy * xsh + dx * xsw + ci;
            const bool tap_ok = tap < taps;
#pragma unroll
            for (int r = 0; r < A_ROWS; ++r) {
                const int hi = row_hi0[r] + dy;
                const int wi = row_wi0[r] + dx;
                const bool ok = row_ok[r] && tap_ok && static_cast<unsigned>(hi) < static_cast<unsigned>(a.H) &&
                                static_cast<unsigned>(wi) < static_cast<unsigned>(a.W);
                const float* p = row_base[r] + (ok ? row_off0[r] + doff : 0);
                ar[r] = *reinterpret_cast<const floatx4*>(p);
                mk |= static_cast<unsigned>(ok) << r;
            }
            // advance this lane's chunk to the next tile's k
            ci += BK;
            if (cin_ge_bk) {
                const bool wrap = ci >= a.Cin;
                ci = wrap ? ci - a.Cin : ci;
                tap += wrap;
                kw += wrap;
                const bool row = kw == a.KW;
                kw = row ? 0 : kw;
                kh += row;
            } else {
#pragma unroll
                for (int w = 0; w < BK / 4; ++w) {
                    const bool wrap = ci >= a.Cin;
                    ci = wrap ? ci - a.Cin : ci;
                    tap += wrap;
                    kw += wrap;
                    const bool row = kw == a.KW;
                    kw = row ? 0 : kw;
                    kh += row;
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
                            v = row_base[r][hi * xsh + wi * xsw + c];
                        }
                    }
                    ar[r][e] = v;
                }
            }
            mk = ~0u;
        }
        mask = mk;
        const float* bt = wtile + static_cast<int64_t>(min(kt, kt_end - 1)) * (BN * BK);
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) {
            const int idx = tid + 256 * i;
            if ((BN * CHUNKS) % 256 == 0 || idx < BN * CHUNKS) br[i] = *reinterpret_cast<const floatx4*>(bt + idx * 4);
        }
    };
    auto store_tile = [&](int buf, const floatx4* ar, const floatx4* br, unsigned mask) {
        float* A = As[buf];
        float* B = Bs[buf];
        const floatx4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < A_ROWS; ++r)
            *reinterpret_cast<floatx4*>(&A[(r0 + ROW_STEP * r) * LDS_STRIDE + chunk * 4]) =
                ((mask >> r) & 1u) ? ar[r] : zero;
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) {
            const int idx = tid + 256 * i;
            if ((BN * CHUNKS) % 256 == 0 || idx < BN * CHUNKS)
                *reinterpret_cast<floatx4*>(&B[(idx / CHUNKS) * LDS_STRIDE + (idx % CHUNKS) * 4]) = br[i];
        }
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int half = lane >> 5;
    const int l32 = lane & 31;
    auto compute_tile = [&](int buf) {
        const float* Ab = As[buf];
        const float* Bb = Bs[buf];
#pragma unroll
        for (int q = 0; q < BK / 8; ++q) {
            floatx4 av[TM], bv[TN];
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
                av[tm] = *reinterpret_cast<const floatx4*>(
                    &Ab[(wave_m * WM + tm * 32 + l32) * LDS_STRIDE + q * 8 + half * 4]);
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
                bv[tn] = *reinterpret_cast<const floatx4*>(
                    &Bb[(wave_n * WN + tn * 32 + l32) * LDS_STRIDE + q * 8 + half * 4]);
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                    for (int tn = 0; tn < TN; ++tn)
                        acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[tm][j], bv[tn][j], acc[tm][tn], 0, 0, 0);
        }
    };

    // ---- software pipeline: tile t is loaded at iteration t-2, stored to LDS
    // at iteration t-1 and multiplied at iteration t.
    const int nk = kt_end - kt_begin;
    if (nk > 0) {
        load_tile(kt_begin, areg[0], breg[0], amask[0]);
        load_tile(kt_begin + 1, areg[1], breg[1], amask[1]);
        store_tile(0, areg[0], breg[0], amask[0]);
        __syncthreads();
    }
    auto iteration = [&](int it, auto stage) {
        constexpr int S = decltype(stage)::value;  // it % 2
        load_tile(kt_begin + it + 2, areg[S], breg[S], amask[S]);
        compute_tile(S);
        if (it + 1 < nk) store_tile(S ^ 1, areg[S ^ 1], breg[S ^ 1], amask[S ^ 1]);
        __syncthreads();
    };
    int it = 0;
    for (; it + 1 < nk; it += 2) {
        iteration(it, std::integral_constant<int, 0>{});
        iteration(it + 1, std::integral_constant<int, 1>{});
    }
    if (it < nk) iteration(it, std::integral_constant<int, 0>{});

    // ---- split-K: publish the partial, the last arriving split reduces
    if (a.splits > 1) {
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wave_m * WM + tm * 32 + (e >> 2) * 8 + half * 4 + (e & 3);
                if (m >= M) continue;
                float* wrow = a.ws + (static_cast<int64_t>(blockIdx.z) * M + m) * a.Cout;
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) {
                    const int col = n0 + wave_n * WN + tn * 32 + l32;
                    if (col < a.Cout) wrow[col] = acc[tm][tn][e];
                }
            }
        return;  // the reduce kernel finishes
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
    const int M = a.N * HoWo;
    const int total = M * a.Cout;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const int m = i / a.Cout;
        const int col = i - m * a.Cout;
        float s = 0.0f;
        for (int z = 0; z < a.splits; ++z) s += a.ws[(static_cast<int64_t>(z) * M + m) * a.Cout + col];
        const int n = m / HoWo;
        const int rem = m - n * HoWo;
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

template <int BM, int BN, int WAVES_M, bool VEC>
void launch_one(const ConvArgs& a, dim3 grid, hipStream_t s) {
    constexpr size_t bytes = lds_bytes<BM, BN>();
    static std::once_flag once;
    std::call_once(once, [] {
        if (bytes > 65536)
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&conv_mfma_kernel<BM, BN, WAVES_M, VEC>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    });
    hipLaunchKernelGGL((conv_mfma_kernel<BM, BN, WAVES_M, VEC>), grid, dim3(256), bytes, s, a);
}

template <int BM, int BN, int WAVES_M>
void launch_tile(const ConvArgs& a, bool vec, dim3 grid, hipStream_t s) {
    if (vec)
        launch_one<BM, BN, WAVES_M, true>(a, grid, s);
    else
        launch_one<BM, BN, WAVES_M, false>(a, grid, s);
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
    if (M * std::max(a.Cout, 1) >= (int64_t{1} << 31)) fail("M * Cout too large");
    if (a.splits < 1 || a.kt_per_split < 1 || static_cast<int64_t>(a.splits) * a.kt_per_split < a.ktiles ||
        static_cast<int64_t>(a.splits - 1) * a.kt_per_split >= a.ktiles)
        fail("bad split");
    if (a.splits > 1 && !a.ws) fail("split-K without workspace");
    if (a.x_sh < 0 || a.x_sw < 0 ||
        static_cast<int64_t>(a.H - 1) * a.x_sh + static_cast<int64_t>(a.W - 1) * a.x_sw + a.Cin >= (int64_t{1} << 31))
        fail("input image extent exceeds int32 offsets");
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
