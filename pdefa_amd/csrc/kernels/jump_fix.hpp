// Float64 recomputation of conv outputs whose fp32 pre-activation lies next
// to a jump of the reference's Winograd-epilogue SiLU.
//
// That SiLU (silu_winograd_form) is discontinuous where -x log2 e crosses a
// half-integer: its output jumps by ~2% of |x| there.  Two fp32 summation
// orders of one conv output differ by a few units in the last place of the
// sum of the magnitudes of its terms, so an output whose -x log2 e lies that
// close to a half-integer can land on either side of the jump depending on
// the order -- the reference's AVX2 order, the device's MFMA order and the
// exactly rounded sum need not agree.  The device takes the side of the
// exactly rounded sum: every epilogue of a compat-SiLU conv flags the outputs
// within kJumpWindow of a jump, leaves them out of its stores, and then the
// wave recomputes each flagged output in float64 from the conv input and the
// K-major packed weights and writes it with the activation applied to that
// sum rounded to fp32.  Outside the window the fp32 sum is
// on the exact sum's side: the window exceeds the fp32 summation error of
// the YOLOv8 layers by a margin (the sum of the terms' magnitudes times
// 2^-24 stays below 5e-7 of max(1, |x log2 e|) on them, the window is 2^-16
// of it).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../kernels.hpp"

namespace pdefa {
namespace k {

// Default half-width of the flagged band around each jump, relative to
// max(1, |x log2 e|) (ConvArgs::jump_window).
constexpr float kJumpWindow = 1.52587890625e-05f;  // 2^-16

// True when -x log2 e (rounded to fp32 as silu_winograd_form rounds it) lies
// within window * max(1, |x log2 e|) of a half-integer, inside the range
// where the form's polynomial branch applies.
__device__ __forceinline__ bool silu_winograd_near_jump(float x, float window) {
    bool near;
    (void)silu_winograd_form(x, window, &near);
    return near;
}

// One lane's double moved across the wave by a DPP control (both halves).
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(b), CTRL, 0xf, 0xf, false));
    const uint32_t hi =
        static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(b >> 32), CTRL, 0xf, 0xf, false));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

// The sum of v over the 64 lanes of the wave, in every lane: within each row
// of 16 lanes by DPP (quad swaps, then rotations by 4 and 8 lanes), then the
// four row sums read from lanes 0, 16, 32 and 48 -- register moves instead
// of LDS round trips.
__device__ __forceinline__ double wave_sum_f64(double v) {
    v += dpp_f64<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f64<0x4E>(v);   // quad_perm [2,3,0,1]: every lane holds its quad's sum
    v += dpp_f64<0x124>(v);  // row_ror:4
    v += dpp_f64<0x128>(v);  // row_ror:8: every lane holds its row's sum
    auto row = [&](int l) {
        const uint64_t b = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(b), l));
        const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(b >> 32), l));
        return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
    };
    return (row(0) + row(16)) + (row(32) + row(48));
}

// bias[g*Cout + co] + sum over (kh, kw, ci) of
// x[n, oh*sh - ph + kh*dh, ow*sw - pw + kw*dw, g*Cin + ci] * w[co][k] in
// float64, w the K-major packed weights (k = (kh*KW + kw)*Cin + ci, 32 x 32
// blocks [co/32][k/32][co%32][k%32], one block set per group).  The 64 lanes
// of the wave split the channels (lane l takes ci = l, l + 64, ...; its
// loads are contiguous across lanes) and every lane returns the total.
// Every load is unconditional -- taps outside the image and lanes past Cin
// read a clamped in-range address and zero the product with a select -- so
// a 3x3 conv's loads of two channel chunks (36 per lane) are in flight
// together instead of one branch and one wait each.
// All 64 lanes must be active; (n, oh, ow, co, g) must name an output
// element of the conv.
__device__ __forceinline__ double conv_point_f64(const ConvArgs& a, int n, int oh, int ow, int co, int g) {
    const int lane = threadIdx.x & 63;
    const int ih0 = oh * a.sh - a.ph, iw0 = ow * a.sw - a.pw;
    const float* xb = a.x + static_cast<int64_t>(n) * a.x_sn + static_cast<int64_t>(g) * a.Cin;
    const float* wb = a.w_kmaj + static_cast<int64_t>(g) * a.w_group +
                      static_cast<int64_t>(co >> 5) * a.ktiles * (kConvBN * kConvBK) + (co & 31) * kConvBK;
    auto w_at = [&](int k) { return wb[static_cast<int64_t>(k >> 5) * (kConvBN * kConvBK) + (k & 31)]; };
    const float bias = a.bias[static_cast<int64_t>(g) * a.Cout + co];
    double s = 0.0;
    if (a.KH == 3 && a.KW == 3) {
        // two 64-channel chunks per round: a conv of up to 128 input channels
        // waits for one round of loads
        for (int c0 = 0; c0 < a.Cin; c0 += 128) {
            float xv[2][9], wv[2][9];
            bool ok[2][9];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const bool cok = c0 + 64 * h + lane < a.Cin;
                const int ci = cok ? c0 + 64 * h + lane : a.Cin - 1;
#pragma unroll
                for (int t = 0; t < 9; ++t) {
                    const int ih = ih0 + (t / 3) * a.dh, iw = iw0 + (t % 3) * a.dw;
                    ok[h][t] = cok & (static_cast<unsigned>(ih) < static_cast<unsigned>(a.H)) &
                               (static_cast<unsigned>(iw) < static_cast<unsigned>(a.W));
                    const int ihc = min(max(ih, 0), a.H - 1), iwc = min(max(iw, 0), a.W - 1);
                    xv[h][t] = xb[static_cast<int64_t>(ihc) * a.x_sh + static_cast<int64_t>(iwc) * a.x_sw + ci];
                    wv[h][t] = w_at(t * a.Cin + ci);
                }
            }
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int t = 0; t < 9; ++t)
                    s = __builtin_fma(static_cast<double>(ok[h][t] ? xv[h][t] : 0.0f), static_cast<double>(wv[h][t]),
                                      s);
        }
    } else {
        for (int c0 = 0; c0 < a.Cin; c0 += 64) {
            const bool cok = c0 + lane < a.Cin;
            const int ci = cok ? c0 + lane : a.Cin - 1;
            for (int kh = 0; kh < a.KH; ++kh) {
                const int ih = ih0 + kh * a.dh;
                const int ihc = min(max(ih, 0), a.H - 1);
                for (int kw = 0; kw < a.KW; ++kw) {
                    const int iw = iw0 + kw * a.dw;
                    const bool ok = cok & (static_cast<unsigned>(ih) < static_cast<unsigned>(a.H)) &
                                    (static_cast<unsigned>(iw) < static_cast<unsigned>(a.W));
                    const int iwc = min(max(iw, 0), a.W - 1);
                    const float xv = xb[static_cast<int64_t>(ihc) * a.x_sh + static_cast<int64_t>(iwc) * a.x_sw + ci];
                    const float wv = w_at((kh * a.KW + kw) * a.Cin + ci);
                    s = __builtin_fma(static_cast<double>(ok ? xv : 0.0f), static_cast<double>(wv), s);
                }
            }
        }
    }
    return wave_sum_f64(s) + static_cast<double>(bias);
}

// Second pass of a compat-SiLU epilogue, after its stores, which leave the
// flagged elements out: for each lane's flagged elements (bit e of `bits`),
// coord(e, n, oh, ow, co) gives the element's output coordinates and
// store(e, pre) writes the element from its float64 pre-activation rounded
// to fp32 (activation, residual as the first pass).  The flagged elements of
// the wave are taken one at a time, lowest lane first.  The branch is
// uniform: with nothing flagged this costs one ballot.  The residual a
// store reads must not share elements with the output.
template <typename Bits, typename Coord, typename Store>
__device__ __forceinline__ void fix_near_jumps(const ConvArgs& a, Bits bits, int g, Coord&& coord, Store&& store) {
    if (__builtin_amdgcn_ballot_w64(bits != 0) == 0) return;
    const int lane = threadIdx.x & 63;
    while (true) {
        const uint64_t lanes = __builtin_amdgcn_ballot_w64(bits != 0);
        if (lanes == 0) break;
        const int src = __builtin_ctzll(lanes);  // wave-uniform: lanes come from a ballot
        const uint64_t b64 = static_cast<uint64_t>(bits);
        const uint64_t lb = static_cast<uint64_t>(static_cast<uint32_t>(
                                __builtin_amdgcn_readlane(static_cast<int>(b64), src))) |
                            (static_cast<uint64_t>(static_cast<uint32_t>(
                                 __builtin_amdgcn_readlane(static_cast<int>(b64 >> 32), src)))
                             << 32);
        const int e = __builtin_ctzll(lb);
        int n, oh, ow, co;
        coord(e, n, oh, ow, co);
        n = __builtin_amdgcn_readlane(n, src);
        oh = __builtin_amdgcn_readlane(oh, src);
        ow = __builtin_amdgcn_readlane(ow, src);
        co = __builtin_amdgcn_readlane(co, src);
        const double s = conv_point_f64(a, n, oh, ow, co, g);
        if (lane == src) {
            store(e, static_cast<float>(s));
            bits &= ~(static_cast<Bits>(1) << e);
        }
    }
}

}  // namespace k
}  // namespace pdefa
