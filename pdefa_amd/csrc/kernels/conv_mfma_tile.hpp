// Implicit-GEMM convolution kernels: the tile template shared by the
// translation units that instantiate it (conv_mfma_tiles_*.hip, a few tile
// shapes each, so that the builds of the many kernel instances run in
// parallel) and the host-side launch templates.  Included only by those
// files and conv_mfma.hip.
//
// Implicit-GEMM convolution on CDNA4 fp32 matrix cores (v_mfma_f32_32x32x2_f32,
// and v_mfma_f32_16x16x4_f32 for the small tiles).
//
// GEMM view of an NHWC convolution: C[m, co] = sum_k A[m, k] * B[k, co] with
// m = (n, ho, wo), k = (kh, kw, ci) and A gathered on the fly from the input
// (no im2col buffer).  One workgroup = 4 or 8 waves computes a BM x BN
// output tile.  Each wave owns a WM x WN sub-tile of MB x MB MFMA blocks (MB =
// 32, or 16 when WM or WN is 16) and one of KG K slices: a pipeline step advances K by BKT = 32*KG, slice g of the
// step (32 k wide) feeding the waves of group g.  With KG > 1 the slices'
// partial tiles are summed through LDS in slice order at the end.
//
// Global loads run two steps ahead of the MFMAs (two register stages) into two
// LDS stages whose rows are padded to 36 floats; each lane feeds four MFMA
// steps from one 16-byte LDS read: with 32x32 blocks lane half h supplies
// k = 8q + 4h + j for step (q, j), with 16x16 blocks lane quarter h supplies
// k = 16q + 4h + j, the same k for A and B, which covers the 32 k of a slice
// once.
// Loads are issued unconditionally: A chunks outside the input (rows past M,
// padding pixels, taps past the kernel) read a zero chunk, out-of-range K
// blocks and N rows re-read the last valid block (such columns are never
// stored), so a loaded stage goes to LDS as it is and the loads of the newest
// step stay in flight while the previous stage is stored.
//
// Workgroups are dispatched round-robin over the 8 XCDs, each with its own L2;
// the tile index is remapped so that every XCD works through a contiguous
// range of tiles (neighbouring output rows share input rows and all tiles of
// one N block share weights).
//
// Split-K across workgroups (layers whose tile grid cannot fill the chip even
// with KG = 4): each split writes its partial tile to a workspace and a reduce
// kernel sums the partials in split order and applies the epilogue.
//
// Epilogue: + bias, activation, + optional residual (the C2f bottleneck add),
// stored through the output view's strides so the result can land directly in
// a channel slice of a concat buffer.
#pragma once

#include "../kernels.hpp"
#include "act.hpp"
#include "jump_fix.hpp"

#include <algorithm>
#include <cmath>
#include <mutex>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

namespace pdefa {
namespace k {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace {

constexpr int BK = kConvBK;         // 32: K per slice and per packed block
constexpr int LDS_STRIDE = BK + 4;  // floats; 16-byte aligned rows, conflict-free float4 reads
constexpr int kXcds = 8;

// Stage buffers (two stages of KG A and B slices), then the per-row output
// offset table of the epilogue (three int64 per tile row: output, residual,
// upsampled output).
template <int BM, int BN, int KG>
constexpr size_t lds_stage_bytes() {
    return sizeof(float) * 2 * KG * (BM + BN) * LDS_STRIDE;
}
template <int BM, int BN, int KG>
constexpr size_t lds_bytes() {
    return lds_stage_bytes<BM, BN, KG>() + 3 * sizeof(int64_t) * BM;
}

}  // namespace

template <int... J, typename F>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, J...>, F&& f) {
    (f(std::integral_constant<int, J>{}), ...);
}
// f(integral_constant<int, j>) for j = 0 .. N-1, unrolled at compile time.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(std::make_integer_sequence<int, N>{}, f);
}

template <int BM, int BN, int WM, int WN, int KG>
constexpr int tile_threads() {
    return 64 * (BM / WM) * (BN / WN) * KG;
}

// MFMA block edge of a wave tile: 32x32 blocks, or 16x16 where the wave tile
// is 16 wide in either dimension.
template <int WM, int WN>
constexpr int mfma_block() {
    return (WM % 32 == 0 && WN % 32 == 0) ? 32 : 16;
}

// Where the epilogues send the stores of tile elements outside the output
// (rows past M, channels past Cout, outputs left to the float64 pass): one
// slot per lane of a workgroup, written and never read.  A store through a
// selected pointer instead of a branch keeps each element's activation out
// of a conditional block, so the activations of a lane's elements
// interleave instead of each waiting out its own chain of latencies.
__device__ float g_epilogue_discard[512];

// What the loads of A chunks outside the input (rows past M, taps past the
// kernel, pixels in the padding) read instead: four zeros, never written.
// Loading zeros, rather than zeroing a loaded chunk by a select, leaves the
// loaded registers untouched until their LDS store, so the wait for a load
// sits at that store, a pipeline step after the load; with the select the
// compiler placed it, and the wait, right behind the load.
__device__ __attribute__((aligned(16))) float g_zero_chunk[4];

// n / d for 0 <= n < 2^31 (kernels.hpp FastDiv)
__device__ __forceinline__ int fdiv(int n, FastDiv f) {
    return static_cast<int>((static_cast<uint64_t>(static_cast<uint32_t>(n)) * f.m) >> f.s);
}

// XCD-aware tile order: dispatch slot `lin` (of `total`) runs on XCD lin % 8;
// give each XCD a contiguous range of tile indices.
__device__ __forceinline__ int xcd_tile(int lin, int total) {
    const int q = total / kXcds, rmd = total % kXcds, xcd = lin % kXcds;
    return xcd * q + min(xcd, rmd) + lin / kXcds;
}

// Epilogue builds of the implicit-GEMM kernels, kept apart so that a larger
// epilogue does not raise every other build's register count: kEpiPlain
// (bias, activation, residual), kEpiFix (also the compat SiLU's float64
// second pass, jump_fix.hpp; grouped launches), kEpiFixOnly (the compat
// SiLU with its second pass alone: one conv's launch), kEpiUp (also an
// upsampled copy of the output).  One launch never needs both the second
// pass and an upsampled copy (the launchers check).
constexpr int kEpiPlain = 0, kEpiFix = 1, kEpiUp = 2, kEpiFixOnly = 3;

// One BM x BN output tile (m block bx, n block by) of K split bz of problem a.
template <int BM, int BN, int WM, int WN, int KG, int PF, bool VEC, int EPI>
__device__ __forceinline__ void conv_tile(const ConvArgs& a, const int bx, const int by, const int bz,
                                          const int grp) {
    constexpr int WAVES_M = BM / WM;
    constexpr int WAVES_N = BN / WN;
    constexpr int NT = tile_threads<BM, BN, WM, WN, KG>();  // 256 or 512 lanes
    static_assert(NT == 256 || NT == 512, "4 or 8 waves per workgroup");
    constexpr int MB = mfma_block<WM, WN>();
    constexpr int TM = WM / MB;
    constexpr int TN = WN / MB;
    // accumulator registers per lane and block: lane l, register e holds row
    // acc_row(e) and column l % MB of its MFMA block
    constexpr int NE = MB * MB / 64;
    using AccT = std::conditional_t<MB == 32, floatx16, floatx4>;
    constexpr int BKT = BK * KG;            // K per pipeline step
    constexpr int CH = BKT / 4;             // float4 chunks per tile row per step
    constexpr int ROW_STEP = NT / CH;       // rows covered by one pass of all lanes
    constexpr int A_ROWS = BM / ROW_STEP;   // A float4 loads per lane per step
    constexpr int B_ROWS = BN / ROW_STEP;   // B float4 loads per lane per step
    static_assert(WM % MB == 0 && WN % MB == 0 && BM % ROW_STEP == 0 && BN % ROW_STEP == 0, "tile");
    static_assert(BM * BN >= NT, "one reduced element per lane at least");
    // One wave per K slice (a single wave tile, KG > 1): each wave loads,
    // stages and multiplies its own slice only, so the pipeline needs no
    // workgroup barrier; LDS operations of one wave complete in issue order,
    // so its stage writes are seen by its own later reads.  The slices meet
    // once, in the epilogue's reduction.
    constexpr bool WP = WAVES_M * WAVES_N == 1 && KG > 1;
    static_assert(!WP || ROW_STEP == 8, "a wave covers 8 rows of its slice per pass");

    extern __shared__ __attribute__((aligned(16))) float smem[];
    // stage st, slice g: A tile at smem + (st*KG + g)*BM*LDS_STRIDE, B tiles after all A tiles
    auto As = [&](int st, int g) { return smem + (st * KG + g) * BM * LDS_STRIDE; };
    auto Bs = [&](int st, int g) { return smem + 2 * KG * BM * LDS_STRIDE + (st * KG + g) * BN * LDS_STRIDE; };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wg = wave % KG;
    const int wave_m = (wave / KG) % WAVES_M;
    const int wave_n = (wave / KG) / WAVES_M;
    const int HoWo = a.Ho * a.Wo;
    const int M = a.N * HoWo;
    // group grp of a grouped conv: its channel offsets (0 when groups == 1)
    const int64_t g_in = static_cast<int64_t>(grp) * a.Cin;
    const int64_t g_out = static_cast<int64_t>(grp) * a.Cout;

    const int m0 = bx * BM;
    const int n0 = by * BN;
    const int kb_begin = bz * a.kt_per_split;  // first K block of this split
    const int kb_end = min(a.ktiles, kb_begin + a.kt_per_split);
    const int nk = (kb_end - kb_begin + KG - 1) / KG;  // pipeline steps
    const int taps = a.KH * a.KW;

    // Bias of this lane's output columns, loaded now so its latency hides
    // behind the K loop (the epilogue only reads registers).
    const int half = lane >> 5;
    const int lcol = lane & (MB - 1);  // column of this lane in its MFMA blocks
    // tile row of accumulator register e of this lane (within its MFMA block)
    auto acc_row = [&](int e) { return MB == 32 ? (e >> 2) * 8 + half * 4 + (e & 3) : (lane >> 4) * 4 + e; };
    float bias_lane[KG == 1 ? TN : 1];
    if constexpr (KG == 1) {
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
            const int co = n0 + wave_n * WN + tn * MB + lcol;
            bias_lane[tn] = co < a.Cout ? a.bias[g_out + co] : 0.0f;
        }
    } else {
        const int co = n0 + tid % BN;
        bias_lane[0] = co < a.Cout ? a.bias[g_out + co] : 0.0f;
    }

    // ---- loaders: this lane loads float4 chunk `chunk` (slice chunk / 8) of
    // rows r0 + ROW_STEP*i of the A tile and of the B tile (with one wave per
    // slice: the chunks of the wave's own slice).
    // Offsets within one image fit in int32 (checked by the launcher).
    const int chunk = WP ? wave * 8 + (lane & 7) : tid % CH;
    const int r0 = WP ? lane >> 3 : tid / CH;
    const int cg = chunk / 8;  // slice of this chunk
    const int cc = chunk % 8;  // chunk within the slice
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
        const int n = fdiv(mm, a.fd_howo);
        const int rem = mm - n * HoWo;
        const int ho = fdiv(rem, a.fd_wo);
        const int wo = rem - ho * a.Wo;
        row_hi0[r] = ho * a.sh - a.ph;
        row_wi0[r] = wo * a.sw - a.pw;
        row_off0[r] = row_hi0[r] * xsh + row_wi0[r] * xsw;
        row_base[r] = a.x + static_cast<int64_t>(n) * a.x_sn + g_in;
    }
    // (tap, ci, kh, kw) of this lane's chunk in the next step to load
    int tap = 0, ci = 0, kh = 0, kw = 0;
    if (VEC) {
        const int k0 = kb_begin * BK + chunk * 4;
        tap = fdiv(k0, a.fd_cin);
        ci = k0 - tap * a.Cin;
        kh = fdiv(tap, a.fd_kw);
        kw = tap - kh * a.KW;
    }
    // Quotients of small non-negative ints by Cin and KW as (q + 0.5) * (1/d)
    // in fp32: the relative error stays below 2^-23 while the true quotient is
    // at least 0.5/d from an integer for q < 2^22, so truncation is exact.
    // Branch-free, so a pipeline iteration stays one basic block.
    const float inv_cin = 1.0f / static_cast<float>(a.Cin);
    const float inv_kw = 1.0f / static_cast<float>(a.KW);

    // B rows of this lane: packed block row of output channel n0 + r0 + ROW_STEP*i
    // (clamped to the last packed block; such columns are never stored).
    const int nblocks = (a.Cout + kConvBN - 1) / kConvBN;
    const float* brow[B_ROWS];
#pragma unroll
    for (int i = 0; i < B_ROWS; ++i) {
        const int co = n0 + r0 + ROW_STEP * i;
        const int nb = min(co / kConvBN, nblocks - 1);
        brow[i] = a.wpk + grp * a.w_group + static_cast<int64_t>(nb) * a.ktiles * (kConvBN * BK) +
                  (co % kConvBN) * BK + cc * 4;
    }

    floatx4 areg[PF][A_ROWS];
    floatx4 breg[PF][B_ROWS];

    auto load_step = [&](int kb0, floatx4* ar, floatx4* br) {
        if (VEC) {
            const int dy = kh * a.dh, dx = kw * a.dw;
            const int doff = dy * xsh + dx * xsw + ci;
            const bool tap_ok = tap < taps;
#pragma unroll
            for (int r = 0; r < A_ROWS; ++r) {
                const int hi = row_hi0[r] + dy;
                const int wi = row_wi0[r] + dx;
                const bool ok = row_ok[r] & tap_ok & (static_cast<unsigned>(hi) < static_cast<unsigned>(a.H)) &
                                (static_cast<unsigned>(wi) < static_cast<unsigned>(a.W));
                const float* p = ok ? row_base[r] + row_off0[r] + doff : g_zero_chunk;
                ar[r] = *reinterpret_cast<const floatx4*>(p);
            }
            // advance this lane's chunk to the next step's k
            ci += BKT;
            const int w = static_cast<int>((static_cast<float>(ci) + 0.5f) * inv_cin);
            ci -= w * a.Cin;
            tap += w;
            kw += w;
            const int rw = static_cast<int>((static_cast<float>(kw) + 0.5f) * inv_kw);
            kw -= rw * a.KW;
            kh += rw;
        } else {
#pragma unroll
            for (int r = 0; r < A_ROWS; ++r) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int kk = kb0 * BK + chunk * 4 + e;
                    float v = 0.0f;
                    if (row_ok[r] && kk < a.K) {
                        const int t = fdiv(kk, a.fd_cin);
                        const int c = kk - t * a.Cin;
                        const int yh = fdiv(t, a.fd_kw);
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
        }
        const int kb = min(kb0 + cg, a.ktiles - 1);
#pragma unroll
        for (int i = 0; i < B_ROWS; ++i)
            br[i] = *reinterpret_cast<const floatx4*>(brow[i] + static_cast<int64_t>(kb) * (kConvBN * BK));
    };
    auto store_step = [&](int st, const floatx4* ar, const floatx4* br) {
        float* A = As(st, cg);
        float* B = Bs(st, cg);
#pragma unroll
        for (int r = 0; r < A_ROWS; ++r)
            *reinterpret_cast<floatx4*>(&A[(r0 + ROW_STEP * r) * LDS_STRIDE + cc * 4]) = ar[r];
#pragma unroll
        for (int i = 0; i < B_ROWS; ++i)
            *reinterpret_cast<floatx4*>(&B[(r0 + ROW_STEP * i) * LDS_STRIDE + cc * 4]) = br[i];
    };

    AccT acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < NE; ++e) acc[i][j][e] = 0.0f;

    // 32x32 blocks: lane (half h, row l % 32) reads k = 8q + 4h .. +3 and feeds
    // them to MFMA steps (q, 0..3) of 2 k each; 16x16 blocks: lane (quarter h,
    // row l % 16) reads k = 16q + 4h .. +3 for steps (q, 0..3) of 4 k each.
    constexpr int KQ = MB == 32 ? 8 : 16;  // k per quad of MFMA steps
    const int krd = MB == 32 ? half * 4 : (lane >> 4) * 4;
    auto compute_step = [&](int st) {
        const float* Ab = As(st, wg);
        const float* Bb = Bs(st, wg);
#pragma unroll
        for (int qq = 0; qq < BK / KQ; ++qq) {
            floatx4 av[TM], bv[TN];
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
                av[tm] = *reinterpret_cast<const floatx4*>(
                    &Ab[(wave_m * WM + tm * MB + lcol) * LDS_STRIDE + qq * KQ + krd]);
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
                bv[tn] = *reinterpret_cast<const floatx4*>(
                    &Bb[(wave_n * WN + tn * MB + lcol) * LDS_STRIDE + qq * KQ + krd]);
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                    for (int tn = 0; tn < TN; ++tn) {
                        if constexpr (MB == 32)
                            acc[tm][tn] =
                                __builtin_amdgcn_mfma_f32_32x32x2f32(av[tm][j], bv[tn][j], acc[tm][tn], 0, 0, 0);
                        else
                            acc[tm][tn] =
                                __builtin_amdgcn_mfma_f32_16x16x4f32(av[tm][j], bv[tn][j], acc[tm][tn], 0, 0, 0);
                    }
        }
    };

    // ---- software pipeline: step t is loaded at iteration t-PF into register
    // stage t % PF, stored to LDS stage t % 2 at iteration t-1 and multiplied
    // at iteration t.  The main loop (unrolled to a multiple of both stage
    // counts) runs only iterations that load; the remaining ones are unrolled
    // after it and load only while a step is left, so no load is in flight
    // into the epilogue.
    constexpr int U = PF % 2 == 0 ? PF : 2 * PF;
    load_step(kb_begin, areg[0], breg[0]);
    static_for<PF - 1>([&](auto jc) {
        constexpr int J = decltype(jc)::value + 1;
        if (J < nk) load_step(kb_begin + J * KG, areg[J], breg[J]);
    });
    // Epilogue row table: element offset of each tile row in the output (or in
    // this split's partial slab) and in the residual; -1 past the last row.
    // Built while the first steps' loads are in flight, read after the
    // pipeline's barriers.
    int64_t* s_yoff = reinterpret_cast<int64_t*>(reinterpret_cast<char*>(smem) + lds_stage_bytes<BM, BN, KG>());
    int64_t* s_roff = s_yoff + BM;
    int64_t* s_uoff = s_roff + BM;
    if (tid < BM) {
        const int m = m0 + tid;
        int64_t yo = -1, ro = 0, uo = 0;
        if (m < M) {
            if (a.splits > 1) {
                yo = ((static_cast<int64_t>(grp) * a.splits + bz) * M + m) * a.Cout;
            } else {
                const int n = fdiv(m, a.fd_howo);
                const int rem = m - n * HoWo;
                const int ho = fdiv(rem, a.fd_wo);
                const int wo = rem - ho * a.Wo;
                yo = static_cast<int64_t>(n) * a.y_sn + static_cast<int64_t>(ho) * a.y_sh +
                     static_cast<int64_t>(wo) * a.y_sw + g_out;
                if (a.res)
                    ro = static_cast<int64_t>(n) * a.r_sn + static_cast<int64_t>(ho) * a.r_sh +
                         static_cast<int64_t>(wo) * a.r_sw + g_out;
                if (a.up)
                    uo = static_cast<int64_t>(n) * a.u_sn + static_cast<int64_t>(2 * ho) * a.u_sh +
                         static_cast<int64_t>(2 * wo) * a.u_sw + g_out;
            }
        }
        s_yoff[tid] = yo;
        s_roff[tid] = ro;
        s_uoff[tid] = uo;
    }

    // between a stage's LDS writes and its reads, and its reads and its next
    // writes: a workgroup barrier, or with one wave per slice only a
    // compiler fence (the wave's LDS operations stay in issue order)
    auto stage_sync = [&] {
        if constexpr (WP) {
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
        } else {
            __syncthreads();
        }
    };
    store_step(0, areg[0], breg[0]);
    stage_sync();
    // In the main loop both the load and the store happen unconditionally, so
    // each iteration is one basic block and the scheduler can interleave the
    // loads' address arithmetic and the LDS stores with the MFMA chain.
    auto iteration = [&](int it, auto jc, bool load, bool store) {
        constexpr int J = decltype(jc)::value;
        constexpr int R = J % PF;  // register stage of step it
        constexpr int L = J % 2;   // LDS stage of step it
        if (load) load_step(kb_begin + (it + PF) * KG, areg[R], breg[R]);
        compute_step(L);
        if (store) store_step(L ^ 1, areg[(R + 1) % PF], breg[(R + 1) % PF]);
        stage_sync();
    };
    int it = 0;
    for (; it + U + PF <= nk; it += U)
        static_for<U>([&](auto jc) { iteration(it + decltype(jc)::value, jc, true, true); });
    static_for<U + PF - 1>([&](auto jc) {
        constexpr int J = decltype(jc)::value;
        if (it + J < nk) iteration(it + J, jc, it + J + PF < nk, it + J + 1 < nk);
    });

    // ---- output.  The row table was written before the prologue barrier
    // (every split has at least one step, checked by the launcher).  A tile
    // element's raw sum becomes a split-K partial (splits > 1) or bias +
    // activation + residual.  The activation, residual and partial choices are
    // hoisted into template arguments so each lane's elements are straight-line
    // code: all row offsets (LDS) first, then all residual loads, then all
    // stores, every load or store of the tile in flight together.
    auto epilogue = [&](auto act_c, auto res_c, auto part_c, auto up_c, auto fix_c) {
        constexpr int ACT = decltype(act_c)::value;
        constexpr bool RES = decltype(res_c)::value;
        constexpr bool PART = decltype(part_c)::value;
        constexpr bool UP = decltype(up_c)::value;
        float* dst = PART ? a.ws : a.y;
        // the four upsampled copies of an element at row offset uo, column co
        auto store_up = [&](int64_t uo, int co, float v) {
            float* u = a.up + uo + co;
            u[0] = v;
            u[a.u_sw] = v;
            u[a.u_sh] = v;
            u[a.u_sh + a.u_sw] = v;
        };
        // compat SiLU: outputs whose pre-activation lies next to one of its
        // jumps are flagged, left out of the stores and written afterwards
        // from a float64 recomputation (jump_fix.hpp); the output row offsets
        // stay in LDS
        constexpr bool FIX = decltype(fix_c)::value && ACT == kActSiluWinogradForm && !PART;
        auto rewrite = [&](int row, int c, float pre) {
            float v = act_fixed<ACT>(pre, a.act, a.slope);
            if constexpr (RES) v += a.res[s_roff[row] + c];
            dst[s_yoff[row] + c] = v;
            if constexpr (UP) store_up(s_uoff[row], c, v);
        };
        auto coord_of_row = [&](int row, int& n, int& oh, int& ow) {
            const int m = m0 + row;
            n = fdiv(m, a.fd_howo);
            const int rem = m - n * HoWo;
            oh = fdiv(rem, a.fd_wo);
            ow = rem - oh * a.Wo;
        };
        if constexpr (KG == 1) {
            // block register e of lane l holds row acc_row(e), column l % MB
            using Bits = std::conditional_t<(TM * TN * NE > 32), uint64_t, uint32_t>;
            Bits bits = 0;
            int co[TN];
            bool cok[TN];
            float bias_v[TN];
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                co[tn] = n0 + wave_n * WN + tn * MB + lcol;
                cok[tn] = co[tn] < a.Cout;
                bias_v[tn] = PART ? 0.0f : bias_lane[tn];
            }
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
                int64_t yo[NE], ro[NE], uo[NE];
#pragma unroll
                for (int e = 0; e < NE; ++e) {
                    const int row = wave_m * WM + tm * MB + acc_row(e);
                    yo[e] = s_yoff[row];
                    if (RES) ro[e] = s_roff[row];
                    if (UP) uo[e] = s_uoff[row];
                }
                float rv[NE][TN];
                if constexpr (RES) {
#pragma unroll
                    for (int e = 0; e < NE; ++e)
#pragma unroll
                        for (int tn = 0; tn < TN; ++tn) {
                            const bool ok = yo[e] >= 0 && cok[tn];
                            const float r = a.res[ok ? ro[e] + co[tn] : 0];
                            rv[e][tn] = ok ? r : 0.0f;
                        }
                }
#pragma unroll
                for (int e = 0; e < NE; ++e)
#pragma unroll
                    for (int tn = 0; tn < TN; ++tn) {
                        float v = acc[tm][tn][e];
                        bool flagged = false;
                        if (!PART) {
                            const float pre = v + bias_v[tn];
                            if constexpr (FIX) {
                                v = silu_winograd_form(pre, a.jump_window, &flagged);
                                flagged = flagged & (yo[e] >= 0) & cok[tn];
                                bits |= static_cast<Bits>(flagged) << ((tm * TN + tn) * NE + e);
                            } else {
                                v = act_fixed<ACT>(pre, a.act, a.slope);
                            }
                        }
                        if (RES) v += rv[e][tn];
                        const bool ok = yo[e] >= 0 && cok[tn] && !flagged;
                        __builtin_nontemporal_store(v, ok ? &dst[yo[e] + co[tn]] : &g_epilogue_discard[tid]);
                        if constexpr (UP) {
                            if (ok) store_up(uo[e], co[tn], v);
                        }
                    }
            }
            if constexpr (FIX) {
                // element (tm * TN + tn) * NE + e
                if (a.w_kmaj)
                    fix_near_jumps(
                        a, bits, grp,
                        [&](int el, int& n, int& oh, int& ow, int& c) {
                            const int tm = el / (TN * NE), e = el % NE;
                            coord_of_row(wave_m * WM + tm * MB + acc_row(e), n, oh, ow);
                            c = n0 + wave_n * WN + ((el / NE) % TN) * MB + lcol;
                        },
                        [&](int el, float pre) {
                            const int tm = el / (TN * NE), e = el % NE;
                            rewrite(wave_m * WM + tm * MB + acc_row(e), n0 + wave_n * WN + ((el / NE) % TN) * MB + lcol,
                                    pre);
                        });
            }
        } else {
            // Slice partials -> LDS (after a barrier that retires every LDS
            // read of the stages: the pipeline's last one, or with one wave
            // per slice this one), then each lane sums its elements (fixed
            // column, rows tid/BN + i*256/BN) in slice order.
            if constexpr (WP) __syncthreads();
            float* red = smem;  // [KG][BM][BN]
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int e = 0; e < NE; ++e)
#pragma unroll
                    for (int tn = 0; tn < TN; ++tn) {
                        const int row = wave_m * WM + tm * MB + acc_row(e);
                        const int col = wave_n * WN + tn * MB + lcol;
                        red[(wg * BM + row) * BN + col] = acc[tm][tn][e];
                    }
            __syncthreads();
            constexpr int E = BM * BN / NT;
            constexpr int RSTEP = NT / BN;
            const int col = tid % BN;
            const int co = n0 + col;
            const bool cok = co < a.Cout;
            const float bias_v = PART ? 0.0f : bias_lane[0];
            float v[E];
            int64_t yo[E], ro[E], uo[E];
#pragma unroll
            for (int i = 0; i < E; ++i) {
                const int row = tid / BN + i * RSTEP;
                float sum = red[row * BN + col];
#pragma unroll
                for (int g = 1; g < KG; ++g) sum += red[(g * BM + row) * BN + col];
                v[i] = sum;
                yo[i] = s_yoff[row];
                if (RES) ro[i] = s_roff[row];
                if (UP) uo[i] = s_uoff[row];
            }
            float rv[E];
            if constexpr (RES) {
#pragma unroll
                for (int i = 0; i < E; ++i) {
                    const bool ok = yo[i] >= 0 && cok;
                    const float r = a.res[ok ? ro[i] + co : 0];
                    rv[i] = ok ? r : 0.0f;
                }
            }
            using Bits = std::conditional_t<(E > 32), uint64_t, uint32_t>;
            Bits bits = 0;
#pragma unroll
            for (int i = 0; i < E; ++i) {
                float r = v[i];
                bool flagged = false;
                if (!PART) {
                    const float pre = r + bias_v;
                    if constexpr (FIX) {
                        r = silu_winograd_form(pre, a.jump_window, &flagged);
                        flagged = flagged & (yo[i] >= 0) & cok;
                        bits |= static_cast<Bits>(flagged) << i;
                    } else {
                        r = act_fixed<ACT>(pre, a.act, a.slope);
                    }
                }
                if (RES) r += rv[i];
                const bool ok = yo[i] >= 0 && cok && !flagged;
                __builtin_nontemporal_store(r, ok ? &dst[yo[i] + co] : &g_epilogue_discard[tid]);
                if constexpr (UP) {
                    if (ok) store_up(uo[i], co, r);
                }
            }
            if constexpr (FIX) {
                // element i: row tid / BN + i * RSTEP, column co
                if (a.w_kmaj)
                    fix_near_jumps(
                        a, bits, grp,
                        [&](int i, int& n, int& oh, int& ow, int& c) {
                            coord_of_row(tid / BN + i * RSTEP, n, oh, ow);
                            c = co;
                        },
                        [&](int i, float pre) { rewrite(tid / BN + i * RSTEP, co, pre); });
            }
        }
    };
    using YES = std::true_type;
    using NO = std::false_type;
    using SILU = std::integral_constant<int, kActSilu>;
    using COMPAT = std::integral_constant<int, kActSiluWinogradForm>;
    using GENERIC = std::integral_constant<int, kActGeneric>;
    using NONE = std::integral_constant<int, kActNone>;
    if constexpr (EPI == kEpiFixOnly) {  // a compat-SiLU conv with the second pass (checked by the launcher)
        if (a.res) epilogue(COMPAT{}, YES{}, NO{}, NO{}, YES{});
        else epilogue(COMPAT{}, NO{}, NO{}, NO{}, YES{});
    } else if (a.splits > 1) {
        epilogue(NONE{}, NO{}, YES{}, NO{}, NO{});
    } else if (EPI == kEpiUp && a.up) {  // upsampled copy (the FPN's Resize inputs: SiLU, no residual)
        if constexpr (EPI == kEpiUp) {
            if (a.act == kActSilu && !a.res) epilogue(SILU{}, NO{}, NO{}, YES{}, NO{});
            else if (a.res) epilogue(GENERIC{}, YES{}, NO{}, YES{}, NO{});
            else epilogue(GENERIC{}, NO{}, NO{}, YES{}, NO{});
        }
    } else if (a.act == kActSilu) {
        if (a.res) epilogue(SILU{}, YES{}, NO{}, NO{}, NO{});
        else epilogue(SILU{}, NO{}, NO{}, NO{}, NO{});
    } else if (a.act == kActSiluWinogradForm) {
        if (EPI == kEpiFix && a.w_kmaj) {
            if constexpr (EPI == kEpiFix) {
                if (a.res) epilogue(COMPAT{}, YES{}, NO{}, NO{}, YES{});
                else epilogue(COMPAT{}, NO{}, NO{}, NO{}, YES{});
            }
        } else {
            if (a.res) epilogue(COMPAT{}, YES{}, NO{}, NO{}, NO{});
            else epilogue(COMPAT{}, NO{}, NO{}, NO{}, NO{});
        }
    } else if (a.act == kActNone) {
        if (a.res) epilogue(NONE{}, YES{}, NO{}, NO{}, NO{});
        else epilogue(NONE{}, NO{}, NO{}, NO{}, NO{});
    } else {
        if (a.res) epilogue(GENERIC{}, YES{}, NO{}, NO{}, NO{});
        else epilogue(GENERIC{}, NO{}, NO{}, NO{}, NO{});
    }
}

// One problem; grid (m tiles, n tiles, K splits), tiles in XCD order with the
// m tile fastest (neighbouring output rows share input rows, all tiles of one
// n block share weights).
template <int BM, int BN, int WM, int WN, int KG, int PF, bool VEC, int EPI>
__global__ __launch_bounds__((tile_threads<BM, BN, WM, WN, KG>())) void conv_mfma_kernel(ConvArgs a) {
    const int gx = gridDim.x, gxy = gridDim.x * gridDim.y;
    const int tile_id = xcd_tile(blockIdx.x + gx * blockIdx.y + gxy * blockIdx.z, gxy * gridDim.z);
    const int bz = fdiv(tile_id, a.fd_gxy);  // group * splits + split
    const int bxy = tile_id - bz * gxy;
    const int by = fdiv(bxy, a.fd_gx);
    const int grp = fdiv(bz, a.fd_splits);
    conv_tile<BM, BN, WM, WN, KG, PF, VEC, EPI>(a, bxy - by * gx, by, bz - grp * a.splits, grp);
}

// Several independent problems in one launch (no split-K): a 1-D grid over
// the concatenated tile lists, problem p owning tiles
// [tile_begin[p], tile_begin[p + 1]) with its m tile fastest.
template <int BM, int BN, int WM, int WN, int KG, int PF, bool VEC, int EPI>
__global__ __launch_bounds__((tile_threads<BM, BN, WM, WN, KG>())) void conv_mfma_group_kernel(ConvGroupArgs g) {
    const int tile_id = xcd_tile(blockIdx.x, gridDim.x);
    int p = 0;
    while (p + 1 < g.count && tile_id >= g.tile_begin[p + 1]) ++p;
    const int local = tile_id - g.tile_begin[p];
    const int by = fdiv(local, g.p[p].fd_gx);
    conv_tile<BM, BN, WM, WN, KG, PF, VEC, EPI>(g.p[p], local - by * g.m_tiles[p], by, 0, 0);
}

namespace {

template <int BM, int BN, int WM, int WN, int KG, int PF, bool VEC, int EPI>
void launch_one(const ConvArgs& a, dim3 grid, hipStream_t s) {
    constexpr size_t bytes = lds_bytes<BM, BN, KG>();
    static_assert(lds_stage_bytes<BM, BN, KG>() >= sizeof(float) * KG * BM * BN,
                  "slice reduction fits in the stage buffers");
    static std::once_flag once;
    std::call_once(once, [] {
        if (bytes > 65536)
            (void)hipFuncSetAttribute(
                reinterpret_cast<const void*>(&conv_mfma_kernel<BM, BN, WM, WN, KG, PF, VEC, EPI>),
                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    });
    hipLaunchKernelGGL((conv_mfma_kernel<BM, BN, WM, WN, KG, PF, VEC, EPI>), grid,
                       dim3(tile_threads<BM, BN, WM, WN, KG>()), bytes, s, a);
}

template <int BM, int BN, int WM, int WN, int KG, int PF, int EPI>
void launch_group_epi(const ConvGroupArgs& g, hipStream_t s) {
    constexpr size_t bytes = lds_bytes<BM, BN, KG>();
    static std::once_flag once;
    std::call_once(once, [] {
        if (bytes > 65536)
            (void)hipFuncSetAttribute(
                reinterpret_cast<const void*>(&conv_mfma_group_kernel<BM, BN, WM, WN, KG, PF, true, EPI>),
                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    });
    hipLaunchKernelGGL((conv_mfma_group_kernel<BM, BN, WM, WN, KG, PF, true, EPI>),
                       dim3(static_cast<unsigned>(g.tile_begin[g.count])), dim3(tile_threads<BM, BN, WM, WN, KG>()),
                       bytes, s, g);
}

void fail(const std::string& m) { throw std::runtime_error("conv_mfma: " + m); }

// The build a problem needs: an upsampled copy, the compat SiLU's float64
// second pass, or neither.
int epi_of(const ConvArgs& a) {
    const bool fix = a.act == kActSiluWinogradForm && a.w_kmaj && a.splits == 1;
    if (a.up && fix) fail("a compat-SiLU conv with the float64 second pass cannot write an upsampled copy");
    return a.up ? kEpiUp : (fix ? kEpiFix : kEpiPlain);
}

template <int BM, int BN, int WM, int WN, int KG, int PF>
void launch_group(const ConvGroupArgs& g, hipStream_t s) {
    bool up = false, fix = false;
    for (int i = 0; i < g.count; ++i) {
        const int e = epi_of(g.p[i]);
        up = up || e == kEpiUp;
        fix = fix || e == kEpiFix;
    }
    if (up && fix) fail("a grouped launch mixes an upsampled copy and the compat SiLU's float64 second pass");
    const int epi = up ? kEpiUp : (fix ? kEpiFix : kEpiPlain);
    if (epi == kEpiUp)
        launch_group_epi<BM, BN, WM, WN, KG, PF, kEpiUp>(g, s);
    else if (epi == kEpiFix)
        launch_group_epi<BM, BN, WM, WN, KG, PF, kEpiFix>(g, s);
    else
        launch_group_epi<BM, BN, WM, WN, KG, PF, kEpiPlain>(g, s);
}

constexpr int kPrefetch = 2;  // register stages: loads run two steps ahead

template <int BM, int BN, int WM, int WN, int KG>
void launch_tile(const ConvArgs& a, bool vec, dim3 grid, hipStream_t s) {
    const int epi = epi_of(a);
    if (epi == kEpiUp) {
        if (!vec) fail("an upsampled output needs vector loads");
        launch_one<BM, BN, WM, WN, KG, kPrefetch, true, kEpiUp>(a, grid, s);
    } else if (epi == kEpiFix) {
        if (vec)
            launch_one<BM, BN, WM, WN, KG, kPrefetch, true, kEpiFixOnly>(a, grid, s);
        else
            launch_one<BM, BN, WM, WN, KG, kPrefetch, false, kEpiFixOnly>(a, grid, s);
    } else if (vec) {
        launch_one<BM, BN, WM, WN, KG, kPrefetch, true, kEpiPlain>(a, grid, s);
    } else {
        launch_one<BM, BN, WM, WN, KG, kPrefetch, false, kEpiPlain>(a, grid, s);
    }
}

}  // namespace

}  // namespace k
}  // namespace pdefa
