// YOLO head decode + per-class greedy NMS on the device: the reference's
// decode_yolo / _iou / _nms (pdefa/python/src/pdefa/_bindings.py:1095-1212)
// with its Python float (IEEE double) arithmetic, operation for operation
// (contraction into fused multiply-adds is off in these kernels).
//
// 1. candidates: one lane per anchor scans the class rows with a strict '>'
//    (first maximum wins), drops best < conf, forms the xyxy box
//    (cx - w*0.5, ...), maps it through the letterbox ((x - pad) * (1/ratio),
//    clamped to the original image) and appends a sort key
//    (class, score descending, anchor) to the image's candidate list.
// 2. one workgroup per image sorts the keys (bitonic, in LDS), so each class
//    is a contiguous run in the reference's visiting order (score descending,
//    anchor ascending on ties: its stable sort of an anchor-ordered list);
//    each wave takes whole classes and runs the greedy loop on them, the 64
//    lanes testing the later boxes of the class against the kept one
//    (suppress when IoU > iou_thres, IoU = inter / (area_a + area_b - inter
//    + 1e-9));
// 3. the kept boxes are sorted by (score descending, first anchor of their
//    class, anchor) -- the reference's stable sort of its keep list, which it
//    builds class by class in order of each class's first candidate -- and
//    the first max_det are written out.
#include "../kernels.hpp"

#include <algorithm>
#include <mutex>
#include <stdexcept>

namespace pdefa {
namespace k {

namespace {

constexpr int kDecodeThreads = 1024;
constexpr unsigned long long kKeyPad = ~0ull;

// Order-preserving map of a float to uint32 (ascending float -> ascending int).
__device__ __forceinline__ uint32_t ordered_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_ordered_bits(uint32_t o) {
    const uint32_t u = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
    return __uint_as_float(u);
}

// Candidate key: class (16 bits) | descending score (32 bits) | anchor (16 bits).
__device__ __forceinline__ unsigned long long cand_key(uint32_t cls, float score, uint32_t anchor) {
    return (static_cast<unsigned long long>(cls) << 48) |
           (static_cast<unsigned long long>(~ordered_bits(score)) << 16) | anchor;
}

// Bitonic sort of s[0, P) ascending, P a power of two, all threads of the block.
__device__ void block_sort(unsigned long long* s, int P) {
    for (int k = 2; k <= P; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < P; i += blockDim.x) {
                const int l = i ^ j;
                if (l > i) {
                    const unsigned long long a = s[i], b = s[l];
                    const bool up = (i & k) == 0;
                    if ((a > b) == up) {
                        s[i] = b;
                        s[l] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
}

__device__ __forceinline__ double clampd(double v, double hi) { return v < 0 ? 0.0 : (v > hi ? hi : v); }

}  // namespace

__global__ __launch_bounds__(256) void yolo_zero_counts_kernel(int32_t* counts, int32_t* ndet, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) {
        counts[i] = 0;
        ndet[i] = 0;
    }
}

__global__ __launch_bounds__(256) void yolo_candidates_kernel(YoloDecodeArgs a) {
#pragma clang fp contract(off)
    const int an = blockIdx.x * 256 + threadIdx.x;
    const int img = blockIdx.y;
    if (an >= a.A) return;
    const float* col = a.out + img * a.sn + an * a.sa;
    const int nc = a.C - 4;
    int best_c = 0;
    float best_s = col[4 * a.sc];
    for (int c = 1; c < nc; ++c) {
        const float s = col[(4 + c) * a.sc];
        if (s > best_s) {
            best_s = s;
            best_c = c;
        }
    }
    if (static_cast<double>(best_s) < a.conf) return;
    const double cx = col[0], cy = col[a.sc], w = col[2 * a.sc], h = col[3 * a.sc];
    double x1 = cx - w * 0.5, y1 = cy - h * 0.5, x2 = cx + w * 0.5, y2 = cy + h * 0.5;
    if (a.meta) {
        const double* m = a.meta + 5 * img;  // ratio, pad_x, pad_y, orig_w, orig_h
        const double scale = 1.0 / m[0];
        x1 = clampd((x1 - m[1]) * scale, m[3]);
        y1 = clampd((y1 - m[2]) * scale, m[4]);
        x2 = clampd((x2 - m[1]) * scale, m[3]);
        y2 = clampd((y2 - m[2]) * scale, m[4]);
    }
    double* b = a.boxes + (static_cast<int64_t>(img) * a.A + an) * 4;
    b[0] = x1;
    b[1] = y1;
    b[2] = x2;
    b[3] = y2;
    a.cls[static_cast<int64_t>(img) * a.A + an] = best_c;
    const int slot = atomicAdd(a.counts + img, 1);
    a.keys[static_cast<int64_t>(img) * a.A + slot] = cand_key(best_c, best_s, an);
}

__global__ __launch_bounds__(kDecodeThreads) void yolo_nms_kernel(YoloDecodeArgs a) {
#pragma clang fp contract(off)
    extern __shared__ unsigned long long sk[];
    const int img = blockIdx.x;
    const int n = a.counts[img];
    if (n > a.max_cand) {  // reported to the host as an error
        if (threadIdx.x == 0) a.ndet[img] = -1;
        return;
    }
    if (n == 0) return;
    int P = 1;
    while (P < n) P <<= 1;
    unsigned long long* gkeys = a.keys + static_cast<int64_t>(img) * a.A;
    const double* boxes = a.boxes + static_cast<int64_t>(img) * a.A * 4;
    const int32_t* cls_of = a.cls + static_cast<int64_t>(img) * a.A;
    int32_t* seg_first = a.seg + static_cast<int64_t>(img) * a.A;  // per sorted candidate: first anchor of its class
    // per sorted candidate, in LDS after the keys: bit 0 suppressed, bit 1 kept
    volatile uint8_t* flags = reinterpret_cast<volatile uint8_t*>(sk + a.max_cand_pow2);

    for (int i = threadIdx.x; i < P; i += blockDim.x) sk[i] = i < n ? gkeys[i] : kKeyPad;
    __syncthreads();
    block_sort(sk, P);
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        gkeys[i] = sk[i];
        flags[i] = 0;
    }
    __syncthreads();

    // greedy NMS, one class run per wave at a time; a run starts where the
    // class changes.  Runs are dealt to waves by their start index.
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nwaves = blockDim.x >> 6;
    volatile uint8_t* vf = flags;  // LDS: a wave's accesses complete in order
    int run = 0;  // running count of class runs seen by this wave's scan
    for (int s = 0; s < n;) {
        const uint32_t c = static_cast<uint32_t>(gkeys[s] >> 48);
        int e = s + 1;
        while (e < n && static_cast<uint32_t>(gkeys[e] >> 48) == c) ++e;
        if (run % nwaves == wave) {
            // first anchor of the class = smallest anchor in the run
            uint32_t first = 0xffffffffu;
            for (int j = s + lane; j < e; j += 64) first = min(first, static_cast<uint32_t>(gkeys[j] & 0xffffu));
            for (int off = 32; off > 0; off >>= 1) first = min(first, static_cast<uint32_t>(__shfl_xor(first, off)));
            for (int j = s + lane; j < e; j += 64) seg_first[j] = static_cast<int32_t>(first);
            for (int i = s; i < e; ++i) {
                if (vf[i] & 1) continue;
                if (lane == 0) vf[i] = 2;
                const int ai = static_cast<int>(gkeys[i] & 0xffffu);
                const double* bi = boxes + static_cast<int64_t>(ai) * 4;
                const double ax1 = bi[0], ay1 = bi[1], ax2 = bi[2], ay2 = bi[3];
                for (int j = i + 1 + lane; j < e; j += 64) {
                    if (vf[j] & 1) continue;
                    const double* bj = boxes + static_cast<int64_t>(gkeys[j] & 0xffffu) * 4;
                    const double bx1 = bj[0], by1 = bj[1], bx2 = bj[2], by2 = bj[3];
                    const double x1 = ax1 > bx1 ? ax1 : bx1;
                    const double y1 = ay1 > by1 ? ay1 : by1;
                    const double x2 = ax2 < bx2 ? ax2 : bx2;
                    const double y2 = ay2 < by2 ? ay2 : by2;
                    const double w = x2 - x1, h = y2 - y1;
                    if (w <= 0 || h <= 0) continue;
                    const double inter = w * h;
                    const double area_a = (ax2 - ax1) * (ay2 - ay1);
                    const double area_b = (bx2 - bx1) * (by2 - by1);
                    const double iou = inter / (area_a + area_b - inter + 1e-9);
                    if (iou > a.iou) vf[j] = 1;
                }
                __builtin_amdgcn_wave_barrier();
            }
        }
        ++run;
        s = e;
    }
    __syncthreads();

    // kept boxes in the reference's output order
    __shared__ int m_kept;
    if (threadIdx.x == 0) m_kept = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        if (!(flags[i] & 2)) continue;
        const uint32_t score_desc = static_cast<uint32_t>(gkeys[i] >> 16);
        const int slot = atomicAdd(&m_kept, 1);
        sk[slot] = (static_cast<unsigned long long>(score_desc) << 32) |
                   (static_cast<unsigned long long>(seg_first[i]) << 16) | (gkeys[i] & 0xffffu);
    }
    __syncthreads();
    const int m = m_kept;
    int Q = 1;
    while (Q < m) Q <<= 1;
    for (int i = m + threadIdx.x; i < Q; i += blockDim.x) sk[i] = kKeyPad;
    __syncthreads();
    block_sort(sk, Q);
    const int out_n = min(m, a.max_det);
    for (int i = threadIdx.x; i < out_n; i += blockDim.x) {
        const unsigned long long k2 = sk[i];
        const int an = static_cast<int>(k2 & 0xffffu);
        const double* b = boxes + static_cast<int64_t>(an) * 4;
        YoloDetection d;
        d.x1 = b[0];
        d.y1 = b[1];
        d.x2 = b[2];
        d.y2 = b[3];
        d.conf = static_cast<double>(from_ordered_bits(~static_cast<uint32_t>(k2 >> 32)));
        d.cls = cls_of[an];
        d.anchor = an;
        a.dets[static_cast<int64_t>(img) * a.max_det + i] = d;
    }
    if (threadIdx.x == 0) a.ndet[img] = out_n;
}

// keys (8 bytes) + flags (1 byte) per candidate slot, capacity rounded up to
// a power of two
size_t yolo_decode_lds_bytes(int max_cand_pow2) {
    return (sizeof(unsigned long long) + 1) * static_cast<size_t>(max_cand_pow2);
}

void launch_yolo_decode(const YoloDecodeArgs& a, hipStream_t s) {
    if (!a.out || !a.boxes || !a.keys || !a.cls || !a.seg || !a.counts || !a.dets || !a.ndet)
        throw std::runtime_error("yolo_decode: null pointer");
    if (a.N <= 0 || a.A <= 0 || a.C < 5) throw std::runtime_error("yolo_decode: head must be [N, 4 + classes, A]");
    if (a.A > 65535 || a.C - 4 > 65535) throw std::runtime_error("yolo_decode: more than 65535 anchors or classes");
    if (a.max_det < 0 || a.max_cand < 1 || a.max_cand > a.max_cand_pow2 || a.max_cand_pow2 > kYoloMaxCandidates ||
        (a.max_cand_pow2 & (a.max_cand_pow2 - 1)) != 0)
        throw std::runtime_error("yolo_decode: max_det / candidate capacity");
    if (a.N > 65535) throw std::runtime_error("yolo_decode: batch too large");
    hipLaunchKernelGGL(yolo_zero_counts_kernel, dim3((a.N + 255) / 256), dim3(256), 0, s, a.counts, a.ndet, a.N);
    hipLaunchKernelGGL(yolo_candidates_kernel, dim3((a.A + 255) / 256, a.N), dim3(256), 0, s, a);
    const size_t lds = yolo_decode_lds_bytes(a.max_cand_pow2);
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&yolo_nms_kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  static_cast<int>(yolo_decode_lds_bytes(kYoloMaxCandidates)));
    });
    hipLaunchKernelGGL(yolo_nms_kernel, dim3(a.N), dim3(kDecodeThreads), lds, s, a);
}

}  // namespace k
}  // namespace pdefa
