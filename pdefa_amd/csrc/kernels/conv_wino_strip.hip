// Winograd F(2x2, 3x3) convolution on CDNA4 fp32 matrix cores, the strip
// form: a workgroup (4 waves) computes 32 consecutive output tiles (of the
// flattened (n, th, tw) tile list) x BN output channels, and each lane loads
// the two input patch rows its row of B^T combines straight from global
// memory (L1/L2), with no LDS staging and no barrier in the K loop.  The
// transforms, the MFMA order, the epilogue and therefore every output bit
// are those of the tile-block kernel (conv_wino.hip, which describes the
// algorithm); launch_conv_wino takes this form for 64 output channels a
// workgroup, where it measured faster: there each wave holds two 32-wide
// channel blocks of accumulators, the workgroup's MFMA work per patch load
// doubles, and the LDS staging's barrier per K step costs more than the
// patch re-reads it saves.
//
// Lane (tile l%32, half h) takes channels 4h..4h+3 of each 8-wide K step; the
// patch and U loads are buffer loads run one K step ahead, issued one after
// each of the step's first MFMAs (scheduling-group barriers).
#include "../kernels.hpp"
#include "act.hpp"
#include "conv_wino_common.hpp"
#include "jump_fix.hpp"

namespace pdefa {
namespace k {

using namespace wino;

template <int BN, int ACT, bool RES>
__global__ __launch_bounds__(256) void conv_wino_strip_kernel(ConvArgs a, int tiles_h, int tiles_w, FastDiv fd_img,
                                                              FastDiv fd_tw, FastDiv fd_gy, int x_bytes, int u_bytes,
                                                              int y_bytes, int r_bytes, int vec_out) {
    constexpr int CB = BN / 32;  // 32-wide channel blocks per wave
    // Exchange rows [row i][column c][tile] hold BN channels and 8 floats of
    // padding: the two lane halves of a column-transform write (tiles 4
    // apart) then fall on disjoint LDS banks.
    constexpr int kXchRow = BN + 8;
    __shared__ __attribute__((aligned(16))) float xch[4 * 2 * kWT * kXchRow];
    // per tile of the workgroup: byte offsets of its four output (and
    // residual) pixels (r, c) at [2r + c], kWinoNoPixel for pixels outside
    // the output (or past the last tile)
    __shared__ __attribute__((aligned(16))) int32_t s_yo4[kWT][4];
    __shared__ __attribute__((aligned(16))) int32_t s_ro4[RES ? kWT : 1][4];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wi_row = tid >> 6;  // transformed row i of this wave
    const int half = lane >> 5;
    const int l32 = lane & 31;
    const int tiles_img = tiles_h * tiles_w;
    const int T = a.N * tiles_img;

    // XCD-aware order: dispatch slot `lin` runs on XCD lin % 8; each XCD takes
    // a contiguous range of (channel block fastest) workgroup indices, so the
    // channel blocks of one strip of tiles read its input patches one after
    // another from one XCD's L2.
    const int gx = gridDim.x, gy = gridDim.y;
    const int total = gx * gy;
    const int lin = blockIdx.x + gx * blockIdx.y;
    const int q = total / kXcds, rmd = total % kXcds, xcd = lin % kXcds;
    const int wid = xcd * q + min(xcd, rmd) + lin / kXcds;
    const int bx = wdiv(wid, fd_gy);
    const int by = wid - bx * gy;
    const int t0 = bx * kWT;
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
        const int tg = t0 + tid;
        const int nn = wdiv(tg, fd_img);
        const int rr = tg - nn * tiles_img;
        const int trow = wdiv(rr, fd_tw);
        const int oh0 = 2 * trow;
        const int ow0 = 2 * (rr - trow * tiles_w);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int oh = oh0 + (q >> 1), ow = ow0 + (q & 1);
            const bool ok = tg < T && oh < a.Ho && ow < a.Wo;
            const int64_t yo = static_cast<int64_t>(nn) * a.y_sn + static_cast<int64_t>(oh) * a.y_sh +
                               static_cast<int64_t>(ow) * a.y_sw;
            s_yo4[tid][q] = ok ? static_cast<int32_t>(yo * 4) : kWinoNoPixel;
            if constexpr (RES) {
                const int64_t ro = static_cast<int64_t>(nn) * a.r_sn + static_cast<int64_t>(oh) * a.r_sh +
                                   static_cast<int64_t>(ow) * a.r_sw;
                s_ro4[tid][q] = ok ? static_cast<int32_t>(ro * 4) : kWinoNoPixel;
            }
        }
    }

    // this lane's tile and the two patch rows that row i of B^T combines:
    // s_b = d[ra][b] + sg * d[rb][b]
    const int t = t0 + l32;
    const bool t_ok = t < T;
    const int tt = t_ok ? t : 0;
    const int n = wdiv(tt, fd_img);
    const int trem = tt - n * tiles_img;
    const int th = wdiv(trem, fd_tw);
    const int tw = trem - th * tiles_w;
    const int ra = wi_row == 2 ? 2 : (wi_row == 0 ? 0 : 1);
    const int rb = wi_row == 0 ? 2 : (wi_row == 2 ? 1 : (wi_row == 1 ? 2 : 3));
    const float sg = wi_row == 1 ? 1.0f : -1.0f;
    // Patch and weight loads are buffer loads: a per-lane 32-bit byte offset,
    // the K step's advance in a scalar offset, the channel block in the
    // immediate.  Patch positions outside the image get kWinoNoPixel, past
    // the input's buffer range, and load zeros.
    const __amdgpu_buffer_rsrc_t xbuf =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.x), 0, x_bytes, kWinoBufferFlags);
    const __amdgpu_buffer_rsrc_t ubuf =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.wpk), 0, u_bytes, kWinoBufferFlags);
    // byte offset of channel 4*half of each patch position
    int32_t doff[2][4];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int hi = 2 * th - a.ph + (r == 0 ? ra : rb);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int wi = 2 * tw - a.pw + b;
            const bool ok = t_ok & (static_cast<unsigned>(hi) < static_cast<unsigned>(a.H)) &
                            (static_cast<unsigned>(wi) < static_cast<unsigned>(a.W));
            const int64_t o = static_cast<int64_t>(n) * a.x_sn + static_cast<int64_t>(hi) * a.x_sh +
                              static_cast<int64_t>(wi) * a.x_sw;
            doff[r][b] = ok ? static_cast<int32_t>(o * 4) + half * 16 : kWinoNoPixel;
        }
    }
    // byte offset of the U float4 of (position (i, j), channel group `half`,
    // this lane's output channel of block 0); block cb adds cb * 512 bytes,
    // K step s adds s * 2 * cop float4s
    int32_t uoff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) uoff[j] = ((((wi_row * 4 + j) * cq + half) * cop) + n0 + l32) * 16;
    const int32_t d_step = kCK * 4;      // bytes per K step of patch channels
    const int32_t u_step = 2 * cop * 16;  // bytes per K step of U

    floatx4 dreg[2][2][4];
    floatx4 ureg[2][4][CB];
    // Channels past Cin (the upper half of the last step when Cin % 8 == 4)
    // read the last 4 channels again (`back` = 16 bytes on that half of the
    // last step); their U rows are zero, so they add nothing.
    const int32_t last_back = (a.Cin & 4) && half ? 16 : 0;
    auto load = [&](int s, floatx4 (&d)[2][4], floatx4 (&u)[4][CB], int32_t back) {
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                d[r][b] = __builtin_bit_cast(
                    floatx4, __builtin_amdgcn_raw_buffer_load_b128(xbuf, doff[r][b] - back, s * d_step, 0));
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
                u[j][cb] = __builtin_bit_cast(
                    floatx4, __builtin_amdgcn_raw_buffer_load_b128(ubuf, uoff[j] + cb * 512, s * u_step, 0));
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

    // Loads run one K step (8 channels) ahead.  Scheduling barriers keep each
    // step's loads among the previous step's MFMAs (left alone, the scheduler
    // sinks them below to save registers, and every step then waits a full L2
    // round trip).
    const int ns = (a.Cin + kCK - 1) / kCK;  // K steps
    auto back_of = [&](int t) { return t == ns - 1 ? last_back : 0; };
    // A load instruction's issue must not leave the matrix core idle (one
    // wave per SIMD with BN = 64, two with BN = 32): the next step's loads go
    // one after each of the step's first MFMAs (after the transform that
    // feeds them).
    auto interleave = [&] {
        {
            constexpr int kLoads = 8 + 4 * CB, kMfma = 16 * CB;
            __builtin_amdgcn_sched_group_barrier(0x002, 64, 0);  // vector ALU (the transform)
#pragma unroll
            for (int i = 0; i < kLoads; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
            }
            __builtin_amdgcn_sched_group_barrier(0x008, kMfma - kLoads, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    load(0, dreg[0], ureg[0], back_of(0));
    int s = 0;
    for (; s + 2 < ns; s += 2) {
        load(s + 1, dreg[1], ureg[1], back_of(s + 1));
        compute(s, dreg[0], ureg[0]);
        interleave();
        load(s + 2, dreg[0], ureg[0], back_of(s + 2));
        compute(s + 1, dreg[1], ureg[1]);
        interleave();
    }
    if (s + 1 < ns) {
        load(s + 1, dreg[1], ureg[1], back_of(s + 1));
        compute(s, dreg[0], ureg[0]);
        interleave();
        compute(s + 1, dreg[1], ureg[1]);
    } else {
        compute(s, dreg[0], ureg[0]);
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
                    const int tg = t0 + tid / G4 + (e >> 4) * (256 / G4);
                    n = wdiv(tg, fd_img);
                    const int rr = tg - n * tiles_img;
                    const int trow = wdiv(rr, fd_tw);
                    oh = 2 * trow + ((e >> 3) & 1);
                    ow = 2 * (rr - trow * tiles_w) + ((e >> 2) & 1);
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
void launch_strip_act(const ConvArgs& a, dim3 grid, int th, int tw, FastDiv fi, FastDiv ft, FastDiv fg, WinoBytes b,
                      hipStream_t s) {
    if (a.res)
        hipLaunchKernelGGL((conv_wino_strip_kernel<BN, ACT, true>), grid, dim3(256), 0, s, a, th, tw, fi, ft, fg, b.x,
                           b.u, b.y, b.r, b.vec);
    else
        hipLaunchKernelGGL((conv_wino_strip_kernel<BN, ACT, false>), grid, dim3(256), 0, s, a, th, tw, fi, ft, fg, b.x,
                           b.u, b.y, b.r, b.vec);
}

template <int BN>
void launch_strip_bn(const ConvArgs& a, dim3 grid, int th, int tw, FastDiv fi, FastDiv ft, FastDiv fg, WinoBytes b,
                     hipStream_t s) {
    switch (a.act) {
        case kActSilu: launch_strip_act<BN, kActSilu>(a, grid, th, tw, fi, ft, fg, b, s); break;
        case kActSiluWinogradForm: launch_strip_act<BN, kActSiluWinogradForm>(a, grid, th, tw, fi, ft, fg, b, s); break;
        case kActNone: launch_strip_act<BN, kActNone>(a, grid, th, tw, fi, ft, fg, b, s); break;
        default: launch_strip_act<BN, kActGeneric>(a, grid, th, tw, fi, ft, fg, b, s); break;
    }
}

}  // namespace

void launch_conv_wino_strip(const ConvArgs& a, int bn, int tiles_h, int tiles_w, WinoBytes b, hipStream_t s) {
    const int64_t T = static_cast<int64_t>(a.N) * tiles_h * tiles_w;
    if (T >= (int64_t{1} << 31)) fail("too many tiles");
    const dim3 grid(static_cast<unsigned>((T + kWT - 1) / kWT), static_cast<unsigned>((a.Cout + bn - 1) / bn));
    if (grid.y > 65535) fail("grid");
    const FastDiv fi = make_fastdiv(static_cast<int64_t>(tiles_h) * tiles_w), ft = make_fastdiv(tiles_w),
                  fg = make_fastdiv(grid.y);
    if (bn != 64) fail("the strip form takes 64 channels a workgroup");
    launch_strip_bn<64>(a, grid, tiles_h, tiles_w, fi, ft, fg, b, s);
}

}  // namespace k
}  // namespace pdefa
