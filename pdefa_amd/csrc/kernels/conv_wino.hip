// Winograd F(2x2, 3x3) convolution on CDNA4 fp32 matrix cores.
//
// For 3x3, stride 1, dilation 1 convolutions over NHWC tensors (the layers
// the reference runs through its own Winograd F(2x2,3x3) kernel,
// PDEFA1.0/src/kernels/simd/avx2/conv2d_winograd.cpp:179-341).  Output 2x2
// tiles t = (n, th, tw) read the 4x4 input patch d at rows 2th-ph.., columns
// 2tw-pw..; with V = B^T d B, U = G g G^T (weights, transformed once at model
// load) and Y = A^T M A, the 16 transformed positions e = (i, j) are 16
// independent GEMMs M_e[t, co] = sum_ci V_e[t, ci] U_e[ci, co]: 16*Cin*Cout
// MACs per 4 outputs instead of 36.
//
//   B^T = [1 0 -1 0; 0 1 1 0; 0 -1 1 0; 0 1 0 -1]
//   G   = [1 0 0; 1/2 1/2 1/2; 1/2 -1/2 1/2; 0 0 1]
//   A^T = [1 1 1 0; 0 1 -1 -1]
//
// A workgroup (4 waves) computes 32 tiles x BN output channels.  Wave i owns
// the transformed row i (positions (i, 0..3)) for all 32 tiles and BN
// channels: 4 x BN/32 accumulator blocks of 32x32.  The GEMM operands come
// straight from global memory (L1/L2), no LDS and no barrier in the K loop:
// lane (tile l%32, half h) loads the two patch rows that row i of B^T combines
// (16-byte runs of 4 channels, half h taking channels 4h..4h+3 of each 8-wide
// K step), forms V_(i,0..3) in registers, and pairs them with U_(i,j) float4s
// of the same 4 channels; MFMA m of a step uses channel 4h+m on half h, the
// same k for A and B.  Loads run one K step ahead.  At the end each wave
// applies the column transform (A^T over j) in registers, the 4 waves exchange
// those rows through LDS, and the row transform (A^T over i), bias,
// activation and residual produce each tile's 2x2 outputs, stored through the
// output view's strides.
#include "../kernels.hpp"
#include "act.hpp"

#include <algorithm>
#include <mutex>
#include <stdexcept>
#include <string>
#include <type_traits>

namespace pdefa {
namespace k {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace {

constexpr int kWT = 32;  // tiles per workgroup (GEMM rows)
constexpr int kCK = 8;   // input channels per K step (4 per lane half)
constexpr int kXcds = 8;
constexpr int kMaxCin = 4096;
constexpr int kXchRow = kWT + 4;  // exchange rows: 32 tiles + 4 floats of padding

int wino_cin_pad(int Cin) { return (Cin + kCK - 1) / kCK * kCK; }
int wino_cout_pad(int Cout) { return (Cout + 63) / 64 * 64; }

void fail(const std::string& m) { throw std::runtime_error("conv_wino: " + m); }

}  // namespace

// Patch positions outside the image read this instead of the input (their
// lanes then need no per-element mask): zeros, one channel run of any Cin.
__device__ __attribute__((aligned(16))) float g_wino_zero[kMaxCin];

bool wino_eligible(int KH, int KW, int sh, int sw, int dh, int dw, int Cin) {
    return KH == 3 && KW == 3 && sh == 1 && sw == 1 && dh == 1 && dw == 1 && Cin % 4 == 0 && Cin >= 8 &&
           Cin <= kMaxCin;
}

int64_t wino_packed_elems(int Cout, int Cin) {
    return 16LL * wino_cin_pad(Cin) * wino_cout_pad(Cout);
}

// U = G g G^T per (co, ci), stored [e][ci/4][Cout_pad][ci%4] with ci padded
// to a multiple of 8 and Cout to a multiple of 64 (zeros).
__global__ void pack_wino_weights_kernel(float* dst, const float* w, int Cout, int Cin, int cip, int cop) {
    const int64_t total = static_cast<int64_t>(cop) * cip;
    for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
         idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int co = static_cast<int>(idx / cip);
        const int ci = static_cast<int>(idx - static_cast<int64_t>(co) * cip);
        float u[16];
        if (co < Cout && ci < Cin) {
            const float* g = w + (static_cast<int64_t>(co) * Cin + ci) * 9;
            float gg[4][3];  // G g
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                const float g0 = g[0 * 3 + c], g1 = g[1 * 3 + c], g2 = g[2 * 3 + c];
                gg[0][c] = g0;
                gg[1][c] = 0.5f * (g0 + g1 + g2);
                gg[2][c] = 0.5f * (g0 - g1 + g2);
                gg[3][c] = g2;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float a0 = gg[r][0], a1 = gg[r][1], a2 = gg[r][2];
                u[r * 4 + 0] = a0;
                u[r * 4 + 1] = 0.5f * (a0 + a1 + a2);
                u[r * 4 + 2] = 0.5f * (a0 - a1 + a2);
                u[r * 4 + 3] = a2;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) u[e] = 0.0f;
        }
        const int cq = cip / 4;
#pragma unroll
        for (int e = 0; e < 16; ++e)
            dst[((static_cast<int64_t>(e) * cq + ci / 4) * cop + co) * 4 + (ci % 4)] = u[e];
    }
}

template <int BN, int ACT, bool RES>
__global__ __launch_bounds__(256) void conv_wino_kernel(ConvArgs a, int tiles_h, int tiles_w) {
    constexpr int CB = BN / 32;  // 32-wide channel blocks per wave
    __shared__ __attribute__((aligned(16))) float xch[4 * 2 * BN * kXchRow];  // [row i][column c][channel][tile]
    // per tile of the workgroup: output / residual offset of its (0, 0) pixel
    // and which of its four pixels exist (bit 0: the tile, 1: column 1, 2: row 1)
    __shared__ int64_t s_yoff[kWT], s_roff[kWT];
    __shared__ int s_vm[kWT];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wi_row = tid >> 6;  // transformed row i of this wave
    const int half = lane >> 5;
    const int l32 = lane & 31;
    const int tiles_img = tiles_h * tiles_w;
    const int T = a.N * tiles_img;

    // XCD-aware order: dispatch slot `lin` runs on XCD lin % 8; each XCD takes
    // a contiguous range of (tile block fastest) workgroup indices.
    const int gx = gridDim.x;
    const int total = gx * gridDim.y;
    const int lin = blockIdx.x + gx * blockIdx.y;
    const int q = total / kXcds, rmd = total % kXcds, xcd = lin % kXcds;
    const int wid = xcd * q + min(xcd, rmd) + lin / kXcds;
    const int by = wid / gx;
    const int bx = wid - by * gx;
    const int t0 = bx * kWT;
    const int n0 = by * BN;
    const int cop = (a.Cout + 63) / 64 * 64;
    const int cq = (a.Cin + kCK - 1) / kCK * (kCK / 4);

    // bias of this lane's epilogue channel (read now, used after the K loop)
    const int e_col = tid % BN;
    const float bias_v = n0 + e_col < a.Cout ? a.bias[n0 + e_col] : 0.0f;
    if (tid < kWT) {  // read after the barrier that precedes the epilogue
        const int tg = t0 + tid;
        int vm = 0;
        int64_t yo = 0, ro = 0;
        if (tg < T) {
            const int nn = tg / tiles_img;
            const int rr = tg - nn * tiles_img;
            const int oh0 = 2 * (rr / tiles_w);
            const int ow0 = 2 * (rr - (rr / tiles_w) * tiles_w);
            vm = 1 | (ow0 + 1 < a.Wo ? 2 : 0) | (oh0 + 1 < a.Ho ? 4 : 0);
            yo = static_cast<int64_t>(nn) * a.y_sn + static_cast<int64_t>(oh0) * a.y_sh +
                 static_cast<int64_t>(ow0) * a.y_sw;
            ro = static_cast<int64_t>(nn) * a.r_sn + static_cast<int64_t>(oh0) * a.r_sh +
                 static_cast<int64_t>(ow0) * a.r_sw;
        }
        s_yoff[tid] = yo;
        s_roff[tid] = ro;
        s_vm[tid] = vm;
    }

    // this lane's tile and the two patch rows that row i of B^T combines:
    // s_b = d[ra][b] + sg * d[rb][b]
    const int t = t0 + l32;
    const bool t_ok = t < T;
    const int tt = t_ok ? t : 0;
    const int n = tt / tiles_img;
    const int trem = tt - n * tiles_img;
    const int th = trem / tiles_w;
    const int tw = trem - th * tiles_w;
    const int ra = wi_row == 2 ? 2 : (wi_row == 0 ? 0 : 1);
    const int rb = wi_row == 0 ? 2 : (wi_row == 2 ? 1 : (wi_row == 1 ? 2 : 3));
    const float sg = wi_row == 1 ? 1.0f : -1.0f;
    const float* xb = a.x + static_cast<int64_t>(n) * a.x_sn;  // offsets within one image fit int32
    // channel-0 address of each patch position, the zero run outside the image
    const float* pp[2][4];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int hi = 2 * th - a.ph + (r == 0 ? ra : rb);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int wi = 2 * tw - a.pw + b;
            const bool ok = t_ok & (static_cast<unsigned>(hi) < static_cast<unsigned>(a.H)) &
                            (static_cast<unsigned>(wi) < static_cast<unsigned>(a.W));
            pp[r][b] = ok ? xb + (hi * static_cast<int>(a.x_sh) + wi * static_cast<int>(a.x_sw)) : g_wino_zero;
        }
    }
    // U float4 of (position (i, j), channel group, this lane's output channel of block cb)
    const floatx4* up = reinterpret_cast<const floatx4*>(a.wpk) + n0 + l32;

    floatx4 dreg[2][2][4];
    floatx4 ureg[2][4][CB];
    // Channels past Cin (the last step's upper half when Cin % 8 == 4) read the
    // last 4 channels again; their U rows are zero, so they add nothing.
    auto load = [&](int s, floatx4 (&d)[2][4], floatx4 (&u)[4][CB]) {
        const int c = min(s * kCK + half * 4, a.Cin - 4);
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int b = 0; b < 4; ++b) d[r][b] = *reinterpret_cast<const floatx4*>(pp[r][b] + c);
        const int cg = s * (kCK / 4) + half;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
                u[j][cb] = up[(static_cast<int64_t>(wi_row * 4 + j) * cq + cg) * cop + cb * 32];
    };

    floatx16 acc[4][CB];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[j][cb][e] = 0.0f;

    // V = (B^T d B) row i for the 4 channels of this lane half (zero outside
    // the image and past Cin), then the step's MFMAs
    auto compute = [&](int s, const floatx4 (&d)[2][4], const floatx4 (&u)[4][CB]) {
        (void)s;
        floatx4 sv[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) sv[b] = d[0][b] + sg * d[1][b];
        floatx4 v[4];
        v[0] = sv[0] - sv[2];
        v[1] = sv[1] + sv[2];
        v[2] = sv[2] - sv[1];
        v[3] = sv[1] - sv[3];
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int cb = 0; cb < CB; ++cb)
                    acc[j][cb] = __builtin_amdgcn_mfma_f32_32x32x2f32(v[j][m], u[j][cb][m], acc[j][cb], 0, 0, 0);
    };

    // Loads run one K step (8 channels) ahead.  With BN = 64 scheduling
    // barriers keep each step's loads ahead of the previous step's MFMAs
    // (left alone, the scheduler sinks them below to save registers, and every
    // step then waits a full L2 round trip); BN = 32 keeps two waves per SIMD
    // without them, which hides that wait instead.
    const int ns = (a.Cin + kCK - 1) / kCK;  // K steps
    load(0, dreg[0], ureg[0]);
    int s = 0;
    for (; s + 2 < ns; s += 2) {
        load(s + 1, dreg[1], ureg[1]);
        if constexpr (BN == 64) __builtin_amdgcn_sched_barrier(0);
        compute(s, dreg[0], ureg[0]);
        if constexpr (BN == 64) __builtin_amdgcn_sched_barrier(0);
        load(s + 2, dreg[0], ureg[0]);
        if constexpr (BN == 64) __builtin_amdgcn_sched_barrier(0);
        compute(s + 1, dreg[1], ureg[1]);
        if constexpr (BN == 64) __builtin_amdgcn_sched_barrier(0);
    }
    if (s + 1 < ns) {
        load(s + 1, dreg[1], ureg[1]);
        if constexpr (BN == 64) __builtin_amdgcn_sched_barrier(0);
        compute(s, dreg[0], ureg[0]);
        compute(s + 1, dreg[1], ureg[1]);
    } else {
        compute(s, dreg[0], ureg[0]);
    }

    // column transform in registers: P[i][0] = M0 + M1 + M2, P[i][1] = M1 - M2 - M3.
    // 32x32 block register e of lane l holds tile row 8*(e/4) + 4*(l/32) + e%4,
    // column l%32: registers 4q..4q+3 are four consecutive tiles, stored as one
    // 16-byte run of the [channel][tile] exchange (rows padded to 36 floats).
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            const int col = cb * 32 + l32;
            const int trow = 8 * qd + 4 * half;
            floatx4 p0, p1;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int e = 4 * qd + k;
                const float m0 = acc[0][cb][e], m1 = acc[1][cb][e], m2 = acc[2][cb][e], m3 = acc[3][cb][e];
                p0[k] = m0 + m1 + m2;
                p1[k] = m1 - m2 - m3;
            }
            *reinterpret_cast<floatx4*>(&xch[((wi_row * 2 + 0) * BN + col) * kXchRow + trow]) = p0;
            *reinterpret_cast<floatx4*>(&xch[((wi_row * 2 + 1) * BN + col) * kXchRow + trow]) = p1;
        }
    __syncthreads();

    // row transform, bias, activation, residual: lane = (channel, blocks of 4
    // tile rows), channel fastest; every LDS read, then every residual load,
    // then every store of the lane in flight together (straight-line, predicated)
    constexpr int RPT = kWT * BN / 256;  // tile rows per lane
    constexpr int NB = RPT / 4;          // blocks of 4 tile rows per lane
    constexpr int GSTEP = 256 / BN;      // lanes per channel
    const int co = n0 + e_col;
    const bool co_ok = co < a.Cout;
    float yv[RPT][4];
    int64_t yo[RPT], ro[RPT];
    int vm[RPT];
#pragma unroll
    for (int bk = 0; bk < NB; ++bk) {
        const int trow0 = 4 * (tid / BN + bk * GSTEP);
        floatx4 p[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int c = 0; c < 2; ++c)
                p[i][c] = *reinterpret_cast<const floatx4*>(&xch[((i * 2 + c) * BN + e_col) * kXchRow + trow0]);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int rk = bk * 4 + k;
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                yv[rk][c] = p[0][c][k] + p[1][c][k] + p[2][c][k];      // output row 0, column c
                yv[rk][2 + c] = p[1][c][k] - p[2][c][k] - p[3][c][k];  // output row 1, column c
            }
            yo[rk] = s_yoff[trow0 + k];
            ro[rk] = s_roff[trow0 + k];
            vm[rk] = co_ok ? s_vm[trow0 + k] : 0;
        }
    }
    // pixel q = (r, c) = (q / 2, q % 2) exists when bit 0, and bit 1 for c = 1, bit 2 for r = 1
    auto pix_ok = [](int m, int q) { return (m & 1) && (!(q & 1) || (m & 2)) && (!(q & 2) || (m & 4)); };
    float rv[RPT][4];
    if constexpr (RES) {
#pragma unroll
        for (int k = 0; k < RPT; ++k)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const bool ok = pix_ok(vm[k], q);
                const int64_t o = ro[k] + (q >> 1) * a.r_sh + (q & 1) * a.r_sw + co;
                const float r = a.res[ok ? o : 0];
                rv[k][q] = ok ? r : 0.0f;
            }
    }
#pragma unroll
    for (int k = 0; k < RPT; ++k)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float v = act_fixed<ACT>(yv[k][q] + bias_v, a.act, a.slope);
            if (RES) v += rv[k][q];
            if (pix_ok(vm[k], q)) a.y[yo[k] + (q >> 1) * a.y_sh + (q & 1) * a.y_sw + co] = v;
        }
}

namespace {

template <int BN, int ACT>
void launch_act(const ConvArgs& a, dim3 grid, int th, int tw, hipStream_t s) {
    if (a.res)
        hipLaunchKernelGGL((conv_wino_kernel<BN, ACT, true>), grid, dim3(256), 0, s, a, th, tw);
    else
        hipLaunchKernelGGL((conv_wino_kernel<BN, ACT, false>), grid, dim3(256), 0, s, a, th, tw);
}

template <int BN>
void launch_bn(const ConvArgs& a, dim3 grid, int th, int tw, hipStream_t s) {
    switch (a.act) {
        case kActSilu: launch_act<BN, kActSilu>(a, grid, th, tw, s); break;
        case kActSiluWinogradForm: launch_act<BN, kActSiluWinogradForm>(a, grid, th, tw, s); break;
        case kActNone: launch_act<BN, kActNone>(a, grid, th, tw, s); break;
        default: launch_act<BN, kActGeneric>(a, grid, th, tw, s); break;
    }
}

}  // namespace

void launch_conv_wino(const ConvArgs& a, int bn, hipStream_t s) {
    if (bn != 32 && bn != 64) fail("bn must be 32 or 64");
    if (!a.x || !a.y || !a.wpk || !a.bias) fail("null pointer");
    if (a.up) fail("no upsampled output on the Winograd path");
    if (a.groups != 1) fail("grouped convs take the implicit GEMM");
    if (!wino_eligible(a.KH, a.KW, a.sh, a.sw, a.dh, a.dw, a.Cin)) fail("not a 3x3 stride-1 conv with Cin % 4 == 0");
    if (a.N <= 0 || a.H <= 0 || a.W <= 0 || a.Cout <= 0) fail("empty shape");
    if (a.Ho != a.H + 2 * a.ph - 2 || a.Wo != a.W + 2 * a.pw - 2 || a.Ho <= 0 || a.Wo <= 0) fail("output size");
    if (a.x_sw % 4 != 0 || a.x_sh % 4 != 0 || a.x_sn % 4 != 0 || reinterpret_cast<uintptr_t>(a.x) % 16 != 0)
        fail("input rows must be 16-byte aligned");
    // per-image input offsets (and the largest patch read) in int32
    const int64_t img_extent = static_cast<int64_t>(a.H) * a.x_sh + static_cast<int64_t>(a.W) * a.x_sw + a.Cin;
    if (img_extent >= (int64_t{1} << 31)) fail("image too large for int32 offsets");
    const int64_t tiles_h = (a.Ho + 1) / 2, tiles_w = (a.Wo + 1) / 2;
    const int64_t T = a.N * tiles_h * tiles_w;
    if (T >= (int64_t{1} << 31)) fail("too many tiles");
    const dim3 grid(static_cast<unsigned>((T + kWT - 1) / kWT), static_cast<unsigned>((a.Cout + bn - 1) / bn));
    if (grid.y > 65535) fail("grid");
    if (bn == 64)
        launch_bn<64>(a, grid, static_cast<int>(tiles_h), static_cast<int>(tiles_w), s);
    else
        launch_bn<32>(a, grid, static_cast<int>(tiles_h), static_cast<int>(tiles_w), s);
}

void launch_pack_wino_weights(float* dst, const float* w, int Cout, int Cin, hipStream_t s) {
    const int cip = wino_cin_pad(Cin), cop = wino_cout_pad(Cout);
    const int64_t total = static_cast<int64_t>(cop) * cip;
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 65535));
    hipLaunchKernelGGL(pack_wino_weights_kernel, dim3(blocks), dim3(256), 0, s, dst, w, Cout, Cin, cip, cop);
}

}  // namespace k
}  // namespace pdefa
