// Implicit-GEMM convolution on CDNA4 fp32 matrix cores: host-side launch
// shapes, cost model and checks, the split-K reduce kernel and the weight
// packing kernels.  The tile kernels are in conv_mfma_tile.hpp, instantiated
// in conv_mfma_tiles_*.hip.
#include "conv_mfma_tile.hpp"

namespace pdefa {
namespace k {

// Tile launchers of conv_mfma_tiles_{a..e}.hip: false when `tile` is not one
// of that file's shapes.
bool launch_conv_tiles_a(int tile, const ConvArgs& a, bool vec, dim3 grid, hipStream_t s);
bool launch_group_tiles_a(int tile, const ConvGroupArgs& g, hipStream_t s);
bool launch_conv_tiles_b(int tile, const ConvArgs& a, bool vec, dim3 grid, hipStream_t s);
bool launch_group_tiles_b(int tile, const ConvGroupArgs& g, hipStream_t s);
bool launch_conv_tiles_c(int tile, const ConvArgs& a, bool vec, dim3 grid, hipStream_t s);
bool launch_group_tiles_c(int tile, const ConvGroupArgs& g, hipStream_t s);
bool launch_conv_tiles_d(int tile, const ConvArgs& a, bool vec, dim3 grid, hipStream_t s);
bool launch_group_tiles_d(int tile, const ConvGroupArgs& g, hipStream_t s);
bool launch_conv_tiles_e(int tile, const ConvArgs& a, bool vec, dim3 grid, hipStream_t s);
bool launch_group_tiles_e(int tile, const ConvGroupArgs& g, hipStream_t s);

// Sums split-K partials in split order, then bias + activation + residual.
// Every lane of a workgroup runs the same number of iterations (a lane past
// the end computes element 0 and stores nothing), so the compat SiLU's
// float64 recomputation (jump_fix.hpp) runs with whole waves.
__global__ __launch_bounds__(256) void conv_splitk_reduce(ConvArgs a) {
    const int HoWo = a.Ho * a.Wo;
    const int M = a.N * HoWo;
    const int per_group = M * a.Cout;
    const int total = per_group * a.groups;
    const bool fix = a.act == kActSiluWinogradForm && a.w_kmaj != nullptr;  // groups == 1 (launcher)
    for (int base = blockIdx.x * blockDim.x; base < total; base += gridDim.x * blockDim.x) {
        const bool live = base + static_cast<int>(threadIdx.x) < total;
        const int i = live ? base + static_cast<int>(threadIdx.x) : 0;
        const int grp = i / per_group;
        const int ig = i - grp * per_group;
        const int m = ig / a.Cout;
        const int col = ig - m * a.Cout;
        const int64_t slab = static_cast<int64_t>(grp) * a.splits;
        float s = 0.0f;
        for (int z = 0; z < a.splits; ++z) s += a.ws[((slab + z) * M + m) * a.Cout + col];
        const int n = m / HoWo;
        const int rem = m - n * HoWo;
        const int ho = rem / a.Wo;
        const int wo = rem - ho * a.Wo;
        const int64_t c = static_cast<int64_t>(grp) * a.Cout + col;  // channel of the whole conv
        float pre = s + a.bias[c];
        if (fix) {
            const uint32_t bits = live & silu_winograd_near_jump(pre, a.jump_window);
            if (__builtin_amdgcn_ballot_w64(bits != 0) != 0) {
                const int lane = threadIdx.x & 63;
                uint32_t left = bits;
                while (true) {  // flagged lanes one at a time, the whole wave summing
                    const uint64_t lanes = __builtin_amdgcn_ballot_w64(left != 0);
                    if (lanes == 0) break;
                    const int src = __builtin_ctzll(lanes);
                    const double d = conv_point_f64(a, __shfl(n, src, 64), __shfl(ho, src, 64),
                                                    __shfl(wo, src, 64), __shfl(col, src, 64), 0);
                    if (lane == src) {
                        pre = static_cast<float>(d);
                        left = 0;
                    }
                }
            }
        }
        if (!live) continue;
        float v = apply_act(pre, a.act, a.slope);
        if (a.res) v += a.res[n * a.r_sn + ho * a.r_sh + wo * a.r_sw + c];
        a.y[n * a.y_sn + ho * a.y_sh + wo * a.y_sw + c] = v;
        if (a.up) {
            float* u = a.up + n * a.u_sn + 2 * ho * a.u_sh + 2 * wo * a.u_sw + c;
            u[0] = v;
            u[a.u_sw] = v;
            u[a.u_sh] = v;
            u[a.u_sh + a.u_sw] = v;
        }
    }
}

namespace {

// indexed by tile id; the Winograd ids (14, 15) have no implicit-GEMM shape
constexpr ConvTileShape kShapes[kNumConvShapes] = {
    {128, 128, 64, 64, 1}, {128, 64, 64, 32, 1}, {64, 128, 32, 64, 1}, {64, 64, 32, 32, 1},
    {128, 32, 32, 32, 1},  {64, 32, 32, 32, 2},  {32, 64, 32, 32, 2},  {32, 32, 32, 32, 4},
    {128, 64, 32, 32, 1},  {64, 64, 32, 32, 2},  {128, 128, 64, 32, 1}, {64, 128, 32, 32, 1},
    {32, 64, 32, 32, 4},   {32, 32, 32, 32, 8},  {0, 0, 0, 0, 0},       {0, 0, 0, 0, 0},
    {16, 16, 16, 16, 4},   {16, 32, 16, 32, 4},  {32, 16, 32, 16, 4},   {16, 32, 16, 32, 8},
    {32, 16, 32, 16, 8},
};
constexpr const char* kNames[kNumConvShapes] = {
    "128x128",  "128x64",    "64x128",    "64x64",     "128x32",    "64x32k2",   "32x64k2",
    "32x32k4",  "128x64w8",  "64x64k2w8", "128x128w8", "64x128w8",  "32x64k4w8", "32x32k8w8",
    "wino64",   "wino32",    "16x16k4",   "16x32k4",   "32x16k4",   "16x32k8w8", "32x16k8w8"};

}  // namespace


ConvTileShape conv_tile_shape(int tile) {
    if (!is_gemm_tile(tile)) return {0, 0, 0, 0, 0};
    return kShapes[tile];
}
const char* conv_tile_name(int tile) { return tile >= 0 && tile < kNumConvShapes ? kNames[tile] : "?"; }

int64_t packed_weight_elems(int Cout, int K) {
    const int64_t cout_pad = (Cout + kConvBN - 1) / kConvBN * kConvBN;
    const int64_t k_pad = (K + BK - 1) / BK * BK;
    return cout_pad * k_pad;
}

// Cost model in CU cycles.  A pipeline step of a workgroup takes the longer
// of its MFMA time (shared with the other workgroups resident on the same CU,
// c = ceil(workgroups / 256)) and a latency floor (a step's loads, LDS round
// trip and barrier); add workgroup start-up, a fixed per-kernel cost and, for
// split-K, the reduce kernel and the partial traffic.  Tile efficiencies and
// the floor are calibrated on YOLOv8 layer shapes.
namespace {

// Predicted cycles of one (tile, splits) launch shape.
double conv_cost(int64_t M, int Cout, int ktiles, int t, int splits, int steps) {
    constexpr double kCus = 256.0;
    constexpr double kKernelCycles = 10000.0;  // launch + completion of one kernel
    constexpr double kWgCycles = 1500.0;       // workgroup start-up (first loads)
    constexpr double kStepFloor = 2200.0;      // latency floor of one pipeline step
    constexpr double kEff[kNumConvShapes] = {1.0, 0.8, 0.8, 0.85, 0.8, 0.75, 0.75, 0.7, 0.85, 0.85, 0.9,
                                             0.85, 0.75, 0.65, 1.0, 1.0, 0.55, 0.6, 0.6, 0.55, 0.55};
    // 8-wave tiles hide part of a step's latency behind the other wave of the
    // SIMD; a 16x16 block's step runs a quarter of the MFMA chain
    constexpr double kFloorScale[kNumConvShapes] = {1,    1,    1,    1,   1,   1,   1,   1,   0.75, 0.75, 0.75,
                                                    0.75, 0.75, 0.8,  1,   1,   0.6, 0.7, 0.7, 0.55, 0.55};
    const ConvTileShape& sh = kShapes[t];
    const int64_t wgs0 = ((M + sh.bm - 1) / sh.bm) * ((Cout + sh.bn - 1) / sh.bn);
    const double c = std::ceil(static_cast<double>(wgs0 * splits) / kCus);
    const double mfma_step = 2.0 * sh.bm * sh.bn * sh.kg * BK / 256.0 / kEff[t];
    double cost = kKernelCycles + kWgCycles + steps * std::max(c * mfma_step, kStepFloor * kFloorScale[t]);
    if (splits > 1) cost += kKernelCycles + static_cast<double>(splits) * M * Cout * 4.0 / 2048.0;
    (void)ktiles;
    return cost;
}

}  // namespace

std::vector<ConvLaunchShape> conv_candidates(int64_t M, int Cout, int K, bool allow_split, bool wino_ok, int Cin) {
    const int ktiles = (K + BK - 1) / BK;
    struct Scored {
        double cost;
        ConvLaunchShape ls;
    };
    std::vector<Scored> out;
    for (int t = 0; t < kNumConvShapes; ++t) {
        if (!is_gemm_tile(t)) continue;
        const ConvTileShape& sh = kShapes[t];
        const int steps_total = (ktiles + sh.kg - 1) / sh.kg;
        const int max_splits = allow_split ? std::min(16, std::max(1, steps_total / 2)) : 1;
        Scored one{0.0, {}}, best{1e300, {}};
        for (int sp = 1; sp <= max_splits; ++sp) {
            const int steps = (steps_total + sp - 1) / sp;
            const int splits = (steps_total + steps - 1) / steps;
            if (splits != sp) continue;
            const double cost = conv_cost(M, Cout, ktiles, t, splits, steps);
            const Scored sc{cost, {t, splits, steps * sh.kg}};
            if (splits == 1) one = sc;
            if (cost < best.cost * 0.999) best = sc;
        }
        out.push_back(one);
        if (best.ls.splits > 1) out.push_back(best);
    }
    if (wino_ok) {
        // 32 output 2x2 tiles x BN channels per workgroup, 8 input channels per
        // step, 16*BN/32 MFMAs of 64 cycles per wave and step, no barrier in the loop
        const int64_t tiles = (M + 3) / 4;  // about M/4 2x2 tiles
        const int steps = (Cin + 7) / 8;
        for (int bn : {64, 32}) {
            const int64_t wgs = (tiles + 31) / 32 * ((Cout + bn - 1) / bn);
            const double c = std::ceil(static_cast<double>(wgs) / 256.0);
            const double step = std::max(c * 16.0 * (bn / 32) * 64.0 / 0.8, 1400.0);
            const double cost = 10000.0 + 3000.0 + steps * step;
            out.push_back({cost, {bn == 64 ? kTileWino64 : kTileWino32, 1, ktiles}});
        }
    }
    std::stable_sort(out.begin(), out.end(), [](const Scored& a, const Scored& b) { return a.cost < b.cost; });
    std::vector<ConvLaunchShape> r;
    for (const Scored& sc : out) r.push_back(sc.ls);
    return r;
}

ConvLaunchShape conv_select(int64_t M, int Cout, int K, bool allow_split, bool wino_ok, int Cin) {
    return conv_candidates(M, Cout, K, allow_split, wino_ok, Cin).front();
}

namespace {

void check_conv(const ConvArgs& a, const ConvTileShape& sh, bool vec) {
    if (!a.x || !a.y || !a.wpk || !a.bias) fail("null pointer");
    if (a.N <= 0 || a.H <= 0 || a.W <= 0 || a.Cin <= 0 || a.Ho <= 0 || a.Wo <= 0 || a.Cout <= 0) fail("empty shape");
    if (a.K != a.KH * a.KW * a.Cin) fail("K mismatch");
    if (a.ktiles != (a.K + BK - 1) / BK) fail("ktiles mismatch");
    const int64_t M = static_cast<int64_t>(a.N) * a.Ho * a.Wo;
    if (a.groups < 1) fail("groups < 1");
    if (M * std::max(a.Cout, 1) * a.groups >= (int64_t{1} << 31)) fail("M * Cout too large");
    if (a.groups > 1 && a.w_group < packed_weight_elems(a.Cout, a.K)) fail("packed weights per group too small");
    if (a.splits < 1 || a.kt_per_split < 1 || a.kt_per_split % sh.kg != 0 ||
        static_cast<int64_t>(a.splits) * a.kt_per_split < a.ktiles ||
        static_cast<int64_t>(a.splits - 1) * a.kt_per_split >= a.ktiles)
        fail("bad split");
    if (a.splits > 1 && !a.ws) fail("split-K without workspace");
    if (a.w_kmaj && a.act == kActSiluWinogradForm && a.groups != 1)
        fail("the compat SiLU's float64 recomputation takes ungrouped convs");
    if (a.up && (a.u_sn < 0 || a.u_sh < 0 || a.u_sw < 0)) fail("negative upsample strides");
    if (a.x_sh < 0 || a.x_sw < 0 ||
        static_cast<int64_t>(a.H - 1) * a.x_sh + static_cast<int64_t>(a.W - 1) * a.x_sw + a.Cin >= (int64_t{1} << 31))
        fail("input image extent exceeds int32 offsets");
    if (vec) {
        if (a.Cin % 4 != 0) fail("vector loads need Cin % 4 == 0");
        if ((reinterpret_cast<uintptr_t>(a.x) & 15) || (a.x_sn & 3) || (a.x_sh & 3) || (a.x_sw & 3))
            fail("vector loads need 16-byte aligned rows");
    }
}

// The problem's divisors for the kernel's index arithmetic (every one below
// 2^31: check_conv bounds the extents).
ConvArgs with_divisors(const ConvArgs& a) {
    ConvArgs b = a;
    b.fd_howo = make_fastdiv(static_cast<int64_t>(a.Ho) * a.Wo);
    b.fd_wo = make_fastdiv(a.Wo);
    b.fd_cin = make_fastdiv(a.Cin);
    b.fd_kw = make_fastdiv(a.KW);
    return b;
}

}  // namespace

void launch_conv_mfma(const ConvArgs& a, int tile, bool vec, hipStream_t s) {
    const ConvTileShape sh = conv_tile_shape(tile);
    if (sh.bm == 0) fail("unknown tile");
    check_conv(a, sh, vec);
    const int64_t M = static_cast<int64_t>(a.N) * a.Ho * a.Wo;
    const int64_t gx = (M + sh.bm - 1) / sh.bm, gy = (a.Cout + sh.bn - 1) / sh.bn;
    const int64_t gz = static_cast<int64_t>(a.splits) * a.groups;
    if (gx * gy * gz >= (int64_t{1} << 31) || gy > 65535 || gz > 65535) fail("grid too large");
    const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy), static_cast<unsigned>(gz));
    ConvArgs b = with_divisors(a);
    b.fd_gx = make_fastdiv(gx);
    b.fd_gxy = make_fastdiv(gx * gy);
    b.fd_splits = make_fastdiv(a.splits);
    if (!(launch_conv_tiles_a(tile, b, vec, grid, s) || launch_conv_tiles_b(tile, b, vec, grid, s) ||
          launch_conv_tiles_c(tile, b, vec, grid, s) || launch_conv_tiles_d(tile, b, vec, grid, s) ||
          launch_conv_tiles_e(tile, b, vec, grid, s)))
        fail("unknown tile");
    if (a.splits > 1) {
        const int64_t total = M * a.Cout * a.groups;
        const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 65535));
        hipLaunchKernelGGL(conv_splitk_reduce, dim3(blocks), dim3(256), 0, s, a);
    }
}

void launch_conv_mfma_group(const ConvArgs* probs, int count, int tile, hipStream_t s) {
    const ConvTileShape sh = conv_tile_shape(tile);
    if (sh.bm == 0) fail("unknown tile");
    if (count < 1 || count > kMaxConvGroup) fail("group size out of range");
    ConvGroupArgs g;
    g.count = count;
    int64_t total = 0;
    for (int i = 0; i < count; ++i) {
        const ConvArgs& a = probs[i];
        check_conv(a, sh, true);
        if (a.splits != 1) fail("grouped problems take no split-K");
        if (a.groups != 1) fail("grouped launches take no grouped convs");
        const int64_t M = static_cast<int64_t>(a.N) * a.Ho * a.Wo;
        const int64_t gx = (M + sh.bm - 1) / sh.bm, gy = (a.Cout + sh.bn - 1) / sh.bn;
        g.tile_begin[i] = static_cast<int32_t>(total);
        g.m_tiles[i] = static_cast<int32_t>(gx);
        g.p[i] = with_divisors(a);
        g.p[i].fd_gx = make_fastdiv(gx);
        total += gx * gy;
        if (total >= (int64_t{1} << 31)) fail("grid too large");
    }
    g.tile_begin[count] = static_cast<int32_t>(total);
    if (!(launch_group_tiles_a(tile, g, s) || launch_group_tiles_b(tile, g, s) ||
          launch_group_tiles_c(tile, g, s) || launch_group_tiles_d(tile, g, s) ||
          launch_group_tiles_e(tile, g, s)))
        fail("unknown tile");
}

__global__ void pack_conv_weights_kernel(float* dst, const float* w, int Cout, int Cin, int KH, int KW, int ktiles,
                                         int64_t total) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int kk = static_cast<int>(i % BK);
        int64_t t = i / BK;
        const int nn = static_cast<int>(t % kConvBN);
        t /= kConvBN;
        const int kt = static_cast<int>(t % ktiles);
        const int nt = static_cast<int>(t / ktiles);
        const int co = nt * kConvBN + nn;
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

__global__ void pack_gemm_b_kernel(float* dst, const float* b, int K, int N, int ktiles, int64_t total) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int kk = static_cast<int>(i % BK);
        int64_t t = i / BK;
        const int nn = static_cast<int>(t % kConvBN);
        t /= kConvBN;
        const int kt = static_cast<int>(t % ktiles);
        const int nt = static_cast<int>(t / ktiles);
        const int col = nt * kConvBN + nn;
        const int kidx = kt * BK + kk;
        dst[i] = (col < N && kidx < K) ? b[static_cast<int64_t>(kidx) * N + col] : 0.0f;
    }
}

void launch_pack_conv_weights(float* dst, const float* w, int Cout, int Cin, int KH, int KW, hipStream_t s) {
    const int K = KH * KW * Cin;
    const int ktiles = (K + BK - 1) / BK;
    const int64_t total = packed_weight_elems(Cout, K);
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 65535));
    hipLaunchKernelGGL(pack_conv_weights_kernel, dim3(blocks), dim3(256), 0, s, dst, w, Cout, Cin, KH, KW, ktiles,
                       total);
}

void launch_pack_gemm_b(float* dst, const float* b, int K, int N, hipStream_t s) {
    const int ktiles = (K + BK - 1) / BK;
    const int64_t total = packed_weight_elems(N, K);
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 65535));
    hipLaunchKernelGGL(pack_gemm_b_kernel, dim3(blocks), dim3(256), 0, s, dst, b, K, N, ktiles, total);
}

}  // namespace k
}  // namespace pdefa
