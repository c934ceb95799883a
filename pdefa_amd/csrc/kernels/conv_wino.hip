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
// A workgroup (4 waves) computes a block of 32 tiles of one image (a 2-D
// block, (32 >> b) x (1 << b) tiles, its shape chosen on the host to cover
// the tile map with the fewest blocks) x BN output channels.  Wave i owns the
// transformed row i (positions (i, 0..3)) for all 32 tiles and BN channels:
// 4 x BN/32 accumulator blocks of 32x32.  Each K step (8 input channels) the
// workgroup copies the block's input patch region -- every pixel once, 16-byte
// runs of 4 channels, range-checked buffer loads that return zeros outside
// the image -- into one of three LDS stages; lane (tile l%32, half h) reads
// the two patch rows that row i of B^T combines from there (half h taking
// channels 4h..4h+3 of the step), forms V_(i,0..3) in registers, and pairs
// them with U_(i,j) float4s of the same 4 channels loaded one step ahead;
// MFMA m of a step uses channel 4h+m on half h, the same k for A and B.  The
// K loop is software-pipelined over the three stages with one barrier per
// step: while step s's MFMAs run, step s+1's patch values are read and
// transformed, step s+2's patch goes from registers to its stage and step
// s+3's is loaded.  At the end each wave applies the column transform (A^T
// over j) in registers, the 4 waves exchange those rows through LDS (the
// stages' memory), and the row transform (A^T over i), bias, activation and
// residual produce each tile's 2x2 outputs, written with range-checked buffer
// stores at per-pixel offsets of the output view.
//
// launch_conv_wino runs this staged form for BN = 32 and the strip form
// (conv_wino_strip.hip, no LDS staging) for BN = 64; both give the same bits.
#include "../kernels.hpp"
#include "act.hpp"
#include "conv_wino_common.hpp"
#include "jump_fix.hpp"

#include <algorithm>
#include <mutex>
#include <stdexcept>
#include <string>
#include <type_traits>

namespace pdefa {
namespace k {

using namespace wino;

namespace {

// Input pixels of the largest tile-block patch region ((2*32+2) x 4 for a
// 32x1 or 1x32 block): the LDS patch stage holds this many pixels per half.
constexpr int kWinoMaxPatchPixels = 66 * 4;

}  // namespace

// A workgroup's 32 output tiles form a block of (32 >> tbw_log2) x
// (1 << tbw_log2) tiles of one image; block_rows x block_cols blocks cover an
// image's tiles_h x tiles_w tile map.
struct WinoGeom {
    int32_t tiles_h, tiles_w, tbw_log2, block_rows, block_cols;
    // divisors of the index arithmetic (kernels.hpp FastDiv): the grid's y
    // extent (channel blocks), blocks per image, block columns, patch row
    // width 2 * tbw + 2
    FastDiv fd_gy, fd_blocks_img, fd_block_cols, fd_pw;
};

bool wino_eligible(int KH, int KW, int sh, int sw, int dh, int dw, int Cin) {
    return KH == 3 && KW == 3 && sh == 1 && sw == 1 && dh == 1 && dw == 1 && Cin % 4 == 0 && Cin >= 8 &&
           Cin <= kMaxCin;
}

bool wino_views_fit(const ConvArgs& a) {
    const int64_t xb = view_bytes(a.N, a.H, a.W, a.Cin, a.x_sn, a.x_sh, a.x_sw);
    const int64_t ub = wino_packed_elems(a.Cout, a.Cin) * 4;
    const int64_t yb = view_bytes(a.N, a.Ho, a.Wo, a.Cout, a.y_sn, a.y_sh, a.y_sw);
    const int64_t rb = a.res ? view_bytes(a.N, a.Ho, a.Wo, a.Cout, a.r_sn, a.r_sh, a.r_sw) : 0;
    return xb < kWinoMaxViewBytes && ub < kWinoMaxViewBytes && yb < kWinoMaxViewBytes && rb < kWinoMaxViewBytes;
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
__global__ __launch_bounds__(256) void conv_wino_kernel(ConvArgs a, WinoGeom geo, int x_bytes, int u_bytes,
                                                        int y_bytes, int r_bytes, int vec_out) {
    constexpr int CB = BN / 32;  // 32-wide channel blocks per wave
    // Exchange rows [row i][column c][tile] hold BN channels and 8 floats of
    // padding: the two lane halves of a column-transform write (tiles 4
    // apart) then fall on disjoint LDS banks.  The exchange reuses the
    // memory of the patch stages (it is written after the K loop).
    constexpr int kXchRow = BN + 8;
    constexpr int kXchFloats = 4 * 2 * kWT * kXchRow;
    constexpr int kStageFloats = 3 * 2 * kWinoMaxPatchPixels * 4;  // [stage][half][pixel][4 channels]
    __shared__ __attribute__((aligned(16))) float smem[kXchFloats > kStageFloats ? kXchFloats : kStageFloats];
    float* const xch = smem;
    // per tile of the workgroup: byte offsets of its four output (and
    // residual) pixels (r, c) at [2r + c], kWinoNoPixel for pixels outside
    // the output (or outside the tile map)
    __shared__ __attribute__((aligned(16))) int32_t s_yo4[kWT][4];
    __shared__ __attribute__((aligned(16))) int32_t s_ro4[RES ? kWT : 1][4];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wi_row = tid >> 6;  // transformed row i of this wave
    const int half = lane >> 5;
    const int l32 = lane & 31;
    const int tiles_h = geo.tiles_h, tiles_w = geo.tiles_w;
    const int tbw = 1 << geo.tbw_log2, tbh = kWT >> geo.tbw_log2;  // tile block: tbh x tbw tiles
    const int PW = 2 * tbw + 2;  // its input patch region: (2 tbh + 2) x PW pixels
    const int PP = (2 * tbh + 2) * PW;

    // XCD-aware order: dispatch slot `lin` runs on XCD lin % 8; each XCD takes
    // a contiguous range of (channel block fastest) workgroup indices, so the
    // workgroups that read one tile block's input patch for its channel
    // blocks run one after another on one XCD and all but the first read it
    // from that XCD's L2.
    const int gx = gridDim.x, gy = gridDim.y;
    const int total = gx * gy;
    const int lin = blockIdx.x + gx * blockIdx.y;
    const int q = total / kXcds, rmd = total % kXcds, xcd = lin % kXcds;
    const int wid = xcd * q + min(xcd, rmd) + lin / kXcds;
    const int bx = wdiv(wid, geo.fd_gy);
    const int by = wid - bx * gy;
    // tile block bx: image bn, block row bbr, block column bbc
    const int blocks_img = geo.block_rows * geo.block_cols;
    const int bn = wdiv(bx, geo.fd_blocks_img);
    const int brem = bx - bn * blocks_img;
    const int bbr = wdiv(brem, geo.fd_block_cols);
    const int bbc = brem - bbr * geo.block_cols;
    const int th0 = bbr * tbh, tw0 = bbc * tbw;  // first tile of the block
    const int n0 = by * BN;
    const int cop = (a.Cout + 63) / 64 * 64;
    const int cq = (a.Cin + kCK - 1) / kCK * (kCK / 4);

    // The epilogue's lane = (tile, 4 consecutive channels), channels fastest:
    // the lane's channels are the same for each of its CB tiles.  Their biases
    // are read now, used after the K loop.
    constexpr int G4 = BN / 4;  // channel groups per tile
    const int c4 = (tid % G4) * 4;
    int32_t cob[4];  // byte offset of each channel, kWinoNoPixel past Cout
    floatx4 bias4;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int co = n0 + c4 + k;
        cob[k] = co < a.Cout ? co * 4 : kWinoNoPixel;
        bias4[k] = co < a.Cout ? a.bias[co] : 0.0f;
    }

    if (tid < kWT) {  // read after the barrier that precedes the epilogue
        const int th = th0 + (tid >> geo.tbw_log2);
        const int tw = tw0 + (tid & (tbw - 1));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int oh = 2 * th + (q >> 1), ow = 2 * tw + (q & 1);
            const bool ok = th < tiles_h && tw < tiles_w && oh < a.Ho && ow < a.Wo;
            const int64_t yo = static_cast<int64_t>(bn) * a.y_sn + static_cast<int64_t>(oh) * a.y_sh +
                               static_cast<int64_t>(ow) * a.y_sw;
            s_yo4[tid][q] = ok ? static_cast<int32_t>(yo * 4) : kWinoNoPixel;
            if constexpr (RES) {
                const int64_t ro = static_cast<int64_t>(bn) * a.r_sn + static_cast<int64_t>(oh) * a.r_sh +
                                   static_cast<int64_t>(ow) * a.r_sw;
                s_ro4[tid][q] = ok ? static_cast<int32_t>(ro * 4) : kWinoNoPixel;
            }
        }
    }

    // Patch stages: each K step (8 input channels) the workgroup copies the
    // block's patch region -- every input pixel once, 4 channels per 16-byte
    // load, zeros outside the image and past Cin -- into one of three LDS
    // stages ([half][pixel][4 channels]); the waves read their tiles' patch
    // rows from there.  Thread t owns slots t, t + 256, t + 512 (slot =
    // 2 * pixel + channel half).
    const __amdgpu_buffer_rsrc_t xbuf =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.x), 0, x_bytes, kWinoBufferFlags);
    const __amdgpu_buffer_rsrc_t ubuf =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.wpk), 0, u_bytes, kWinoBufferFlags);
    constexpr int kSlots = 3;
    constexpr int kStage = 2 * kWinoMaxPatchPixels * 4;  // floats per stage
    int32_t soff[kSlots];  // byte offset of the slot's 4 channels at step 0 (kWinoNoPixel: zeros)
    int32_t sdst[kSlots];  // LDS float index of the slot within a stage (-1: no slot)
    bool shi[kSlots];      // upper channel half
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const int slot = tid + 256 * j;
        const int p = slot >> 1, h = slot & 1;
        const int pr = wdiv(p, geo.fd_pw), pc = p - pr * PW;
        const int hi = 2 * th0 - a.ph + pr, wi = 2 * tw0 - a.pw + pc;
        const bool inside = p < PP && (static_cast<unsigned>(hi) < static_cast<unsigned>(a.H)) &&
                            (static_cast<unsigned>(wi) < static_cast<unsigned>(a.W));
        const int64_t o = static_cast<int64_t>(bn) * a.x_sn + static_cast<int64_t>(hi) * a.x_sh +
                          static_cast<int64_t>(wi) * a.x_sw;
        soff[j] = inside ? static_cast<int32_t>(o * 4) + h * 16 : kWinoNoPixel;
        sdst[j] = p < PP ? (h * kWinoMaxPatchPixels + p) * 4 : -1;
        shi[j] = h != 0;
    }
    const int32_t d_step = kCK * 4;  // bytes per K step of patch channels
    const int ns = (a.Cin + kCK - 1) / kCK;  // K steps
    // the upper half of the last step lies past Cin when Cin % 8 == 4: zeros
    const bool last_half_past = (a.Cin & 4) != 0;
    floatx4 sreg[kSlots];
    auto load_patch = [&](int st) {
        const bool past = last_half_past && st == ns - 1;
#pragma unroll
        for (int j = 0; j < kSlots; ++j)
            sreg[j] = __builtin_bit_cast(
                floatx4, __builtin_amdgcn_raw_buffer_load_b128(xbuf, past && shi[j] ? kWinoNoPixel : soff[j],
                                                               st * d_step, 0));
    };
    auto store_patch = [&](int stage) {
        float* dst = smem + stage * kStage;
#pragma unroll
        for (int j = 0; j < kSlots; ++j)
            if (sdst[j] >= 0) *reinterpret_cast<floatx4*>(dst + sdst[j]) = sreg[j];
    };

    // this lane's tile within the block and the two patch rows that row i of
    // B^T combines: s_b = d[ra][b] + sg * d[rb][b]
    const int tr = l32 >> geo.tbw_log2, tc = l32 & (tbw - 1);
    const int ra = wi_row == 2 ? 2 : (wi_row == 0 ? 0 : 1);
    const int rb = wi_row == 0 ? 2 : (wi_row == 2 ? 1 : (wi_row == 1 ? 2 : 3));
    const float sg = wi_row == 1 ? 1.0f : -1.0f;
    // LDS float index of patch position (ra / rb, b = 0) of this lane's half
    const int pa = (half * kWinoMaxPatchPixels + (2 * tr + ra) * PW + 2 * tc) * 4;
    const int pb = (half * kWinoMaxPatchPixels + (2 * tr + rb) * PW + 2 * tc) * 4;
    // byte offset of the U float4 of (position (i, j), channel group `half`,
    // this lane's output channel of block 0); block cb adds cb * 512 bytes,
    // K step s adds s * 2 * cop float4s
    int32_t uoff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) uoff[j] = ((((wi_row * 4 + j) * cq + half) * cop) + n0 + l32) * 16;
    const int32_t u_step = 2 * cop * 16;  // bytes per K step of U

    floatx4 ureg[2][4][CB];
    auto load_u = [&](int st, floatx4 (&u)[4][CB]) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
                u[j][cb] = __builtin_bit_cast(
                    floatx4, __builtin_amdgcn_raw_buffer_load_b128(ubuf, uoff[j] + cb * 512, st * u_step, 0));
    };

    floatx16 acc[4][CB];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[j][cb][e] = 0.0f;

    // the lane's patch values of one step from an LDS stage, and V = (B^T d B)
    // row i of them for the 4 channels of this lane half
    floatx4 dreg[2][4];
    floatx4 v[4];
    auto read_d = [&](int stage) {
        const float* src = smem + stage * kStage;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            dreg[0][b] = *reinterpret_cast<const floatx4*>(src + pa + 4 * b);
            dreg[1][b] = *reinterpret_cast<const floatx4*>(src + pb + 4 * b);
        }
    };
    auto transform = [&] {
        floatx4 sv[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) sv[b] = dreg[0][b] + sg * dreg[1][b];
        v[0] = sv[0] - sv[2];
        v[1] = sv[1] + sv[2];
        v[2] = sv[2] - sv[1];
        v[3] = sv[1] - sv[3];
    };
    auto mfmas = [&](const floatx4 (&u)[4][CB]) {
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int cb = 0; cb < CB; ++cb)
                    acc[j][cb] = __builtin_amdgcn_mfma_f32_32x32x2f32(v[j][m], u[j][cb][m], acc[j][cb], 0, 0, 0);
    };

    // Software pipeline over three LDS stages: while step s's MFMAs run, the
    // patch values of step s + 1 are read from LDS and transformed, step
    // s + 2's patch (in registers) goes to its stage and step s + 3's is
    // loaded; U runs one step ahead in registers.  One barrier per step:
    // the stage written in step s was last read in step s - 2.
    load_patch(0);
    load_u(0, ureg[0]);
    store_patch(0);
    if (ns > 1) {
        load_patch(1);
        store_patch(1);
    }
    if (ns > 2) load_patch(2);
    __syncthreads();
    read_d(0);
    transform();
    auto step = [&](int st, auto cur_c, auto ub_c) {
        constexpr int CUR = decltype(cur_c)::value;  // stage of step st
        constexpr int UB = decltype(ub_c)::value;    // U registers of step st
        const bool next = st + 1 < ns;
        if (next) {
            read_d((CUR + 1) % 3);
            load_u(st + 1, ureg[UB ^ 1]);
        }
        mfmas(ureg[UB]);
        if (st + 2 < ns) {
            store_patch((CUR + 2) % 3);
            if (st + 3 < ns) load_patch(st + 3);
        }
        if (next) transform();
        __syncthreads();
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    for (int st = 0; st < ns; st += 6) {
        step(st, I0{}, I0{});
        if (st + 1 < ns) step(st + 1, I1{}, I1{});
        if (st + 2 < ns) step(st + 2, I2{}, I0{});
        if (st + 3 < ns) step(st + 3, I0{}, I1{});
        if (st + 4 < ns) step(st + 4, I1{}, I0{});
        if (st + 5 < ns) step(st + 5, I2{}, I1{});
    }

    // column transform in registers: P[i][0] = M0 + M1 + M2, P[i][1] = M1 - M2 - M3.
    // 32x32 block register e of lane l holds tile row 8*(e/4) + 4*(l/32) + e%4,
    // column (channel) l%32, written to the channel-fastest exchange.
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int col = cb * 32 + l32;
            const int trow = 8 * (e / 4) + 4 * half + e % 4;
            const float m0 = acc[0][cb][e], m1 = acc[1][cb][e], m2 = acc[2][cb][e], m3 = acc[3][cb][e];
            xch[((wi_row * 2 + 0) * kWT + trow) * kXchRow + col] = m0 + m1 + m2;
            xch[((wi_row * 2 + 1) * kWT + trow) * kXchRow + col] = m1 - m2 - m3;
        }
    __syncthreads();

    // row transform, bias, activation, residual: lane = (tile, 4 consecutive
    // channels), CB tiles per lane.  Outputs and residuals move as 16-byte
    // runs when vec_out is set (output and residual rows 16-byte aligned,
    // Cout % 4 == 0), else as single floats, channels past Cout skipped.
    // Stores are non-temporal (cache policy 2).  Buffer-range checks drop
    // stores (and zero loads) at kWinoNoPixel offsets, so pixels outside the
    // output need no branch.
    const __amdgpu_buffer_rsrc_t ybuf = __builtin_amdgcn_make_buffer_rsrc(a.y, 0, y_bytes, kWinoBufferFlags);
    const __amdgpu_buffer_rsrc_t rbuf =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(RES ? a.res : a.y), 0, RES ? r_bytes : 0,
                                          kWinoBufferFlags);
    floatx4 yv[CB][4];
    int32_t yo[CB][4], ro[CB][4];
#pragma unroll
    for (int r = 0; r < CB; ++r) {
        const int tl = tid / G4 + r * (256 / G4);
        floatx4 p[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int c = 0; c < 2; ++c)
                p[i][c] = *reinterpret_cast<const floatx4*>(&xch[((i * 2 + c) * kWT + tl) * kXchRow + c4]);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            yv[r][c] = p[0][c] + p[1][c] + p[2][c];      // output row 0, column c
            yv[r][2 + c] = p[1][c] - p[2][c] - p[3][c];  // output row 1, column c
        }
        const int4 y4 = *reinterpret_cast<const int4*>(&s_yo4[tl][0]);
        yo[r][0] = y4.x;
        yo[r][1] = y4.y;
        yo[r][2] = y4.z;
        yo[r][3] = y4.w;
        if constexpr (RES) {
            const int4 r4 = *reinterpret_cast<const int4*>(&s_ro4[tl][0]);
            ro[r][0] = r4.x;
            ro[r][1] = r4.y;
            ro[r][2] = r4.z;
            ro[r][3] = r4.w;
        }
    }
    // compat SiLU with the float64 second pass (a.w_kmaj set): bit
    // 16 r + 4 q + k flags element (r, q, k), whose pre-activation lies next
    // to a jump; the stores below leave flagged elements out
    constexpr bool FIX = ACT == kActSiluWinogradForm;
    const bool fix = FIX && a.w_kmaj != nullptr;
    uint32_t bits = 0;
    // channels of this lane that exist (bit k: channel n0 + c4 + k < Cout)
    const uint32_t kmask = static_cast<uint32_t>(cob[0] != kWinoNoPixel) | (uint32_t{cob[1] != kWinoNoPixel} << 1) |
                           (uint32_t{cob[2] != kWinoNoPixel} << 2) | (uint32_t{cob[3] != kWinoNoPixel} << 3);
    // the activation of the 4 channels of pixel q of tile pass r (the
    // compat SiLU four at a time, flagging its near-jump elements)
    auto act4 = [&](int r, int q, floatx4 pre) {
        floatx4 v;
        if constexpr (FIX) {
            floatx4 d;
            v = silu_winograd_form4(pre, a.jump_window, &d);
            const float dmin = fminf(fminf(d[0], d[1]), fminf(d[2], d[3]));
            if (fix && yo[r][q] != kWinoNoPixel && dmin <= 0.0f) {  // rare
                const uint32_t nb = uint32_t{d[0] <= 0.0f} | (uint32_t{d[1] <= 0.0f} << 1) |
                                    (uint32_t{d[2] <= 0.0f} << 2) | (uint32_t{d[3] <= 0.0f} << 3);
                bits |= (nb & kmask) << (16 * r + 4 * q);
            }
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = act_fixed<ACT>(pre[k], a.act, a.slope);
        }
        return v;
    };
    if (vec_out) {
        floatx4 rv[CB][4];
        if constexpr (RES) {
#pragma unroll
            for (int r = 0; r < CB; ++r)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    rv[r][q] = __builtin_bit_cast(
                        floatx4, __builtin_amdgcn_raw_buffer_load_b128(rbuf, ro[r][q] + cob[0], 0, 0));
        }
        floatx4 v[CB][4];
#pragma unroll
        for (int r = 0; r < CB; ++r)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                v[r][q] = act4(r, q, yv[r][q] + bias4);
                if constexpr (RES) v[r][q] += rv[r][q];
            }
        if (!FIX || __builtin_amdgcn_ballot_w64(bits != 0) == 0) {
#pragma unroll
            for (int r = 0; r < CB; ++r)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uintx4, v[r][q]), ybuf,
                                                           yo[r][q] + cob[0], 0, 2);
        } else {  // a flagged element in the wave: single floats, flagged ones left out
#pragma unroll
            for (int r = 0; r < CB; ++r)
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        __builtin_amdgcn_raw_buffer_store_b32(
                            __float_as_uint(v[r][q][k]), ybuf,
                            (bits >> (16 * r + 4 * q + k)) & 1u ? kWinoNoPixel : yo[r][q] + cob[k], 0, 2);
        }
    } else {
        float rv[CB][4][4];
        if constexpr (RES) {
#pragma unroll
            for (int r = 0; r < CB; ++r)
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        rv[r][q][k] =
                            __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rbuf, ro[r][q] + cob[k], 0, 0));
        }
#pragma unroll
        for (int r = 0; r < CB; ++r)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const floatx4 v = act4(r, q, yv[r][q] + bias4);
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    __builtin_amdgcn_raw_buffer_store_b32(
                        __float_as_uint(RES ? v[k] + rv[r][q][k] : v[k]), ybuf,
                        (bits >> (16 * r + 4 * q + k)) & 1u ? kWinoNoPixel : yo[r][q] + cob[k], 0, 2);
            }
    }
    if constexpr (FIX) {
        if (a.w_kmaj) {
            // element (r, q, k): tile tl = tid / G4 + r * (256 / G4), pixel
            // (row q >> 1, column q & 1), channel n0 + c4 + k; its offsets
            // are still in s_yo4 / s_ro4
            fix_near_jumps(
                a, bits, 0,
                [&](int e, int& n, int& oh, int& ow, int& co) {
                    const int tl = tid / G4 + (e >> 4) * (256 / G4);
                    n = bn;
                    oh = 2 * (th0 + (tl >> geo.tbw_log2)) + ((e >> 3) & 1);
                    ow = 2 * (tw0 + (tl & (tbw - 1))) + ((e >> 2) & 1);
                    co = n0 + c4 + (e & 3);
                },
                [&](int e, float pre) {
                    const int tl = tid / G4 + (e >> 4) * (256 / G4);
                    const int q = (e >> 2) & 3;
                    const int32_t cb = (n0 + c4 + (e & 3)) * 4;
                    float v = act_fixed<ACT>(pre, a.act, a.slope);
                    if constexpr (RES)
                        v += __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rbuf, s_ro4[tl][q] + cb, 0, 0));
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), ybuf, s_yo4[tl][q] + cb, 0, 2);
                });
        }
    }
}

namespace {

template <int BN, int ACT>
void launch_act(const ConvArgs& a, dim3 grid, WinoGeom g, WinoBytes b, hipStream_t s) {
    if (a.res)
        hipLaunchKernelGGL((conv_wino_kernel<BN, ACT, true>), grid, dim3(256), 0, s, a, g, b.x, b.u, b.y, b.r, b.vec);
    else
        hipLaunchKernelGGL((conv_wino_kernel<BN, ACT, false>), grid, dim3(256), 0, s, a, g, b.x, b.u, b.y, b.r, b.vec);
}

template <int BN>
void launch_bn(const ConvArgs& a, dim3 grid, WinoGeom g, WinoBytes b, hipStream_t s) {
    switch (a.act) {
        case kActSilu: launch_act<BN, kActSilu>(a, grid, g, b, s); break;
        case kActSiluWinogradForm: launch_act<BN, kActSiluWinogradForm>(a, grid, g, b, s); break;
        case kActNone: launch_act<BN, kActNone>(a, grid, g, b, s); break;
        default: launch_act<BN, kActGeneric>(a, grid, g, b, s); break;
    }
}

// The tile block with the fewest blocks over the tile map (ties: the squarer
// block, whose patch region has the least halo).
WinoGeom wino_geometry(int64_t tiles_h, int64_t tiles_w) {
    WinoGeom best{};
    int64_t best_blocks = -1, best_halo = 0;
    for (int lg = 0; lg <= 5; ++lg) {
        const int64_t tbw = int64_t{1} << lg, tbh = kWT / tbw;
        const int64_t rows = (tiles_h + tbh - 1) / tbh, cols = (tiles_w + tbw - 1) / tbw;
        const int64_t blocks = rows * cols;
        const int64_t halo = (2 * tbh + 2) * (2 * tbw + 2);
        if (best_blocks < 0 || blocks < best_blocks || (blocks == best_blocks && halo < best_halo)) {
            best_blocks = blocks;
            best_halo = halo;
            best = {static_cast<int32_t>(tiles_h), static_cast<int32_t>(tiles_w), lg, static_cast<int32_t>(rows),
                    static_cast<int32_t>(cols)};
        }
    }
    return best;
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
    const int64_t tiles_h = (a.Ho + 1) / 2, tiles_w = (a.Wo + 1) / 2;
    if (tiles_h >= (int64_t{1} << 24) || tiles_w >= (int64_t{1} << 24)) fail("too many tiles");
    if (a.x_sn < 0 || a.x_sh < 0 || a.x_sw < 0 || a.y_sn < 0 || a.y_sh < 0 || a.y_sw < 0 ||
        (a.res && (a.r_sn < 0 || a.r_sh < 0 || a.r_sw < 0)))
        fail("negative strides");
    if (!wino_views_fit(a)) fail("input, weights, output or residual span 1 GiB - 4 KiB or more");
    WinoBytes b;
    b.x = static_cast<int>(view_bytes(a.N, a.H, a.W, a.Cin, a.x_sn, a.x_sh, a.x_sw));
    b.u = static_cast<int>(wino_packed_elems(a.Cout, a.Cin) * 4);
    b.y = static_cast<int>(view_bytes(a.N, a.Ho, a.Wo, a.Cout, a.y_sn, a.y_sh, a.y_sw));
    b.r = a.res ? static_cast<int>(view_bytes(a.N, a.Ho, a.Wo, a.Cout, a.r_sn, a.r_sh, a.r_sw)) : 0;
    auto rows16 = [](const float* p, int64_t sn, int64_t sh, int64_t sw) {
        return reinterpret_cast<uintptr_t>(p) % 16 == 0 && sn % 4 == 0 && sh % 4 == 0 && sw % 4 == 0;
    };
    b.vec = a.Cout % 4 == 0 && rows16(a.y, a.y_sn, a.y_sh, a.y_sw) &&
            (!a.res || rows16(a.res, a.r_sn, a.r_sh, a.r_sw));
    // 64 channels a workgroup: the strip form (conv_wino_strip.hip), the
    // same outputs bit for bit
    if (bn == 64) {
        launch_conv_wino_strip(a, 64, static_cast<int>(tiles_h), static_cast<int>(tiles_w), b, s);
        return;
    }
    WinoGeom geo = wino_geometry(tiles_h, tiles_w);
    const int64_t blocks = static_cast<int64_t>(a.N) * geo.block_rows * geo.block_cols;
    if (blocks >= (int64_t{1} << 31)) fail("too many tiles");
    geo.fd_gy = make_fastdiv((a.Cout + 31) / 32);
    geo.fd_blocks_img = make_fastdiv(static_cast<int64_t>(geo.block_rows) * geo.block_cols);
    geo.fd_block_cols = make_fastdiv(geo.block_cols);
    geo.fd_pw = make_fastdiv(2 * (int64_t{1} << geo.tbw_log2) + 2);
    const dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>((a.Cout + 31) / 32));
    if (grid.y > 65535) fail("grid");
    launch_bn<32>(a, grid, geo, b, s);
}

void launch_pack_wino_weights(float* dst, const float* w, int Cout, int Cin, hipStream_t s) {
    const int cip = wino_cin_pad(Cin), cop = wino_cout_pad(Cout);
    const int64_t total = static_cast<int64_t>(cop) * cip;
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 65535));
    hipLaunchKernelGGL(pack_wino_weights_kernel, dim3(blocks), dim3(256), 0, s, dst, w, Cout, Cin, cip, cop);
}

}  // namespace k
}  // namespace pdefa
