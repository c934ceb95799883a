// Host-side engine_ops_* helpers (everything except ops_matmul).  They are not
// on the GPU hot path; their semantics follow PDEFA1.0/src/api/engine_api.cpp
// (cited per function) so the Python layer's tensor helpers behave the same.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <random>
#include <vector>

#include "api_internal.hpp"

using pdefa::HostTensor;
using pdefa::api::clear_error;
using pdefa::api::guarded;
using pdefa::api::set_error;
using pdefa::api::valid;
using pdefa::api::wrap;

namespace {

enum class Bin { Add, Sub, Mul, Div };

HostTensor new_f32(const int64_t* dims, int32_t rank) { return HostTensor::empty(dims, rank, pdefa::kF32); }

// engine_api.cpp:89-240 (broadcast shape + elementwise evaluation)
EngineStatus binary(const EngineTensor* a, const EngineTensor* b, EngineTensor** out, Bin op) {
    if (!valid(a) || !valid(b)) return ENGINE_ERR_INVALID_HANDLE;
    if (!out) return ENGINE_ERR_NULL_PTR;
    *out = nullptr;
    return guarded([&] {
        clear_error();
        const HostTensor& A = *a->ptr();
        const HostTensor& B = *b->ptr();
        const int32_t ro = std::max(A.rank, B.rank);
        if (ro > 8) {
            set_error("broadcast shape mismatch");
            return ENGINE_ERR_INVALID_SHAPE;
        }
        int64_t od[8];
        for (int32_t d = 0; d < ro; ++d) {
            const int64_t da = d < ro - A.rank ? 1 : A.dims[d - (ro - A.rank)];
            const int64_t db = d < ro - B.rank ? 1 : B.dims[d - (ro - B.rank)];
            if (da != db && da != 1 && db != 1) {
                set_error("broadcast shape mismatch");
                return ENGINE_ERR_INVALID_SHAPE;
            }
            od[d] = std::max(da, db);
        }
        HostTensor O = new_f32(od, ro);
        const int64_t n = O.numel();
        const float* ap = A.f32();
        const float* bp = B.f32();
        float* dst = O.f32();
        int64_t idx[8];
        for (int64_t i = 0; i < n; ++i) {
            int64_t t = i;
            for (int32_t d = ro - 1; d >= 0; --d) {
                idx[d] = t % od[d];
                t /= od[d];
            }
            int64_t ai = 0, bi = 0;
            for (int32_t d = 0; d < A.rank; ++d) ai = ai * A.dims[d] + (A.dims[d] == 1 ? 0 : idx[ro - A.rank + d]);
            for (int32_t d = 0; d < B.rank; ++d) bi = bi * B.dims[d] + (B.dims[d] == 1 ? 0 : idx[ro - B.rank + d]);
            const float x = ap[ai], y = bp[bi];
            switch (op) {
                case Bin::Add: dst[i] = x + y; break;
                case Bin::Sub: dst[i] = x - y; break;
                case Bin::Mul: dst[i] = x * y; break;
                case Bin::Div: dst[i] = x / y; break;
            }
        }
        *out = wrap(std::move(O));
        return ENGINE_OK;
    });
}

// engine_api.cpp:309-322: unary ops refuse borrowed tensors and non-F32 data
EngineStatus unary_check(EngineTensor* t) {
    if (!valid(t)) return ENGINE_ERR_INVALID_HANDLE;
    if (t->is_borrowed()) {
        set_error("cannot modify borrowed tensor");
        return ENGINE_ERR_INVALID_ARG;
    }
    if (t->ptr()->dtype != pdefa::kF32) {
        set_error("only F32 supported");
        return ENGINE_ERR_INVALID_ARG;
    }
    return ENGINE_OK;
}

template <typename F>
EngineStatus unary(EngineTensor* t, F f) {
    const EngineStatus s = unary_check(t);
    if (s != ENGINE_OK) return s;
    return guarded([&] {
        clear_error();
        float* p = t->ptr()->f32();
        const int64_t n = t->ptr()->numel();
        for (int64_t i = 0; i < n; ++i) p[i] = f(p[i]);
        return ENGINE_OK;
    });
}

bool axis_split(const HostTensor& t, int32_t axis, int32_t* ax, int64_t* outer, int64_t* len, int64_t* inner) {
    int32_t a = axis < 0 ? axis + t.rank : axis;
    if (a < 0 || a >= t.rank) return false;
    *ax = a;
    *outer = 1;
    for (int32_t d = 0; d < a; ++d) *outer *= t.dims[d];
    *len = t.dims[a];
    *inner = 1;
    for (int32_t d = a + 1; d < t.rank; ++d) *inner *= t.dims[d];
    return true;
}

// engine_api.cpp:1161-1241 (mode 0 max, 1 sum, 2 mean)
EngineStatus reduce(const EngineTensor* a, int32_t axis, int32_t keepdims, EngineTensor** out, int mode) {
    if (!valid(a)) return ENGINE_ERR_INVALID_HANDLE;
    if (!out) return ENGINE_ERR_NULL_PTR;
    *out = nullptr;
    return guarded([&] {
        clear_error();
        const HostTensor& in = *a->ptr();
        if (in.dtype != pdefa::kF32) {
            set_error("reduce: only F32 supported");
            return ENGINE_ERR_INVALID_ARG;
        }
        int32_t ax;
        int64_t outer, len, inner;
        if (!axis_split(in, axis, &ax, &outer, &len, &inner)) {
            set_error("reduce: axis out of range");
            return ENGINE_ERR_INVALID_ARG;
        }
        int64_t od[8];
        int32_t orank = 0;
        for (int32_t d = 0; d < in.rank; ++d) {
            if (d == ax) {
                if (keepdims) od[orank++] = 1;
            } else {
                od[orank++] = in.dims[d];
            }
        }
        if (orank == 0) od[orank++] = 1;
        HostTensor O = new_f32(od, orank);
        const float* ip = in.f32();
        float* op = O.f32();
        for (int64_t o = 0; o < outer; ++o)
            for (int64_t i = 0; i < inner; ++i) {
                const float* base = ip + o * len * inner + i;
                float r;
                if (mode == 0) {
                    r = -3.4e38f;
                    for (int64_t k = 0; k < len; ++k) r = base[k * inner] > r ? base[k * inner] : r;
                } else {
                    r = 0.0f;
                    for (int64_t k = 0; k < len; ++k) r += base[k * inner];
                    if (mode == 2) r /= static_cast<float>(len);
                }
                op[o * inner + i] = r;
            }
        *out = wrap(std::move(O));
        return ENGINE_OK;
    });
}

}  // namespace

extern "C" {

PDEFA_EXPORT EngineStatus engine_ops_add(const EngineTensor* a, const EngineTensor* b, EngineTensor** out) {
    return binary(a, b, out, Bin::Add);
}
PDEFA_EXPORT EngineStatus engine_ops_sub(const EngineTensor* a, const EngineTensor* b, EngineTensor** out) {
    return binary(a, b, out, Bin::Sub);
}
PDEFA_EXPORT EngineStatus engine_ops_mul(const EngineTensor* a, const EngineTensor* b, EngineTensor** out) {
    return binary(a, b, out, Bin::Mul);
}
PDEFA_EXPORT EngineStatus engine_ops_div(const EngineTensor* a, const EngineTensor* b, EngineTensor** out) {
    return binary(a, b, out, Bin::Div);
}

// engine_api.cpp:916-934: relu/silu check only the handle and borrow state
PDEFA_EXPORT EngineStatus engine_ops_relu(EngineTensor* t) {
    if (!valid(t)) return ENGINE_ERR_INVALID_HANDLE;
    if (t->is_borrowed()) return ENGINE_ERR_INVALID_ARG;
    if (t->ptr()->dtype != pdefa::kF32) return ENGINE_OK;
    return unary(t, [](float x) { return x > 0.0f ? x : 0.0f; });
}
PDEFA_EXPORT EngineStatus engine_ops_silu(EngineTensor* t) {
    if (!valid(t)) return ENGINE_ERR_INVALID_HANDLE;
    if (t->is_borrowed()) return ENGINE_ERR_INVALID_ARG;
    if (t->ptr()->dtype != pdefa::kF32) return ENGINE_OK;
    return unary(t, [](float x) { return x / (1.0f + std::exp(-x)); });
}
PDEFA_EXPORT EngineStatus engine_ops_sigmoid(EngineTensor* t) {
    return unary(t, [](float x) { return 1.0f / (1.0f + std::exp(-x)); });
}
PDEFA_EXPORT EngineStatus engine_ops_tanh(EngineTensor* t) {
    return unary(t, [](float x) { return std::tanh(x); });
}
// tanh-form GELU, as ops::gelu_ (PDEFA1.0/src/ops/activation.cpp gelu_ref)
PDEFA_EXPORT EngineStatus engine_ops_gelu(EngineTensor* t) {
    return unary(t, [](float x) {
        const float inner = 0.7978845608f * (x + 0.044715f * x * x * x);
        return 0.5f * x * (1.0f + std::tanh(inner));
    });
}
PDEFA_EXPORT EngineStatus engine_ops_clip(EngineTensor* t, float lo, float hi) {
    const EngineStatus s = unary_check(t);
    if (s != ENGINE_OK) return s;
    if (lo > hi) {
        set_error("clip: lo > hi");
        return ENGINE_ERR_INVALID_ARG;
    }
    return unary(t, [lo, hi](float x) { return x < lo ? lo : (x > hi ? hi : x); });
}

// engine_api.cpp:1040-1087
PDEFA_EXPORT EngineStatus engine_ops_softmax(EngineTensor* t, int32_t axis) {
    const EngineStatus s = unary_check(t);
    if (s != ENGINE_OK) return s;
    return guarded([&] {
        clear_error();
        HostTensor& x = *t->ptr();
        int32_t ax;
        int64_t outer, len, inner;
        if (!axis_split(x, axis, &ax, &outer, &len, &inner)) {
            set_error("softmax: axis out of range");
            return ENGINE_ERR_INVALID_ARG;
        }
        float* p = x.f32();
        for (int64_t o = 0; o < outer; ++o)
            for (int64_t i = 0; i < inner; ++i) {
                float* base = p + o * len * inner + i;
                float mx = -1e30f;
                for (int64_t k = 0; k < len; ++k) mx = base[k * inner] > mx ? base[k * inner] : mx;
                float sum = 0.0f;
                for (int64_t k = 0; k < len; ++k) {
                    const float e = std::exp(base[k * inner] - mx);
                    base[k * inner] = e;
                    sum += e;
                }
                const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
                for (int64_t k = 0; k < len; ++k) base[k * inner] *= inv;
            }
        return ENGINE_OK;
    });
}

PDEFA_EXPORT EngineStatus engine_ops_reduce_max(const EngineTensor* a, int32_t axis, int32_t keepdims, EngineTensor** out) {
    return reduce(a, axis, keepdims, out, 0);
}
PDEFA_EXPORT EngineStatus engine_ops_reduce_sum(const EngineTensor* a, int32_t axis, int32_t keepdims, EngineTensor** out) {
    return reduce(a, axis, keepdims, out, 1);
}
PDEFA_EXPORT EngineStatus engine_ops_reduce_mean(const EngineTensor* a, int32_t axis, int32_t keepdims, EngineTensor** out) {
    return reduce(a, axis, keepdims, out, 2);
}

// engine_api.cpp:1243-1309: I32 indices, first maximum wins
PDEFA_EXPORT EngineStatus engine_ops_argmax(const EngineTensor* a, int32_t axis, int32_t keepdims, EngineTensor** out) {
    if (!valid(a)) return ENGINE_ERR_INVALID_HANDLE;
    if (!out) return ENGINE_ERR_NULL_PTR;
    *out = nullptr;
    return guarded([&] {
        clear_error();
        const HostTensor& in = *a->ptr();
        if (in.dtype != pdefa::kF32) {
            set_error("argmax: only F32 supported");
            return ENGINE_ERR_INVALID_ARG;
        }
        int32_t ax;
        int64_t outer, len, inner;
        if (!axis_split(in, axis, &ax, &outer, &len, &inner)) {
            set_error("argmax: axis out of range");
            return ENGINE_ERR_INVALID_ARG;
        }
        int64_t od[8];
        int32_t orank = 0;
        for (int32_t d = 0; d < in.rank; ++d) {
            if (d == ax) {
                if (keepdims) od[orank++] = 1;
            } else {
                od[orank++] = in.dims[d];
            }
        }
        if (orank == 0) od[orank++] = 1;
        HostTensor O = HostTensor::empty(od, orank, pdefa::kI32);
        const float* ip = in.f32();
        int32_t* op = static_cast<int32_t*>(O.data);
        for (int64_t o = 0; o < outer; ++o)
            for (int64_t i = 0; i < inner; ++i) {
                const float* base = ip + o * len * inner + i;
                float best = base[0];
                int32_t bi = 0;
                for (int64_t k = 1; k < len; ++k)
                    if (base[k * inner] > best) {
                        best = base[k * inner];
                        bi = static_cast<int32_t>(k);
                    }
                op[o * inner + i] = bi;
            }
        *out = wrap(std::move(O));
        return ENGINE_OK;
    });
}

// engine_api.cpp:1576-1640: out-of-range indices read index 0
PDEFA_EXPORT EngineStatus engine_ops_gather(const EngineTensor* a, const EngineTensor* indices, int32_t axis,
                                            EngineTensor** out) {
    if (!valid(a) || !valid(indices)) return ENGINE_ERR_INVALID_HANDLE;
    if (!out) return ENGINE_ERR_NULL_PTR;
    *out = nullptr;
    return guarded([&] {
        clear_error();
        const HostTensor& data = *a->ptr();
        const HostTensor& idx = *indices->ptr();
        if (data.dtype != pdefa::kF32) {
            set_error("gather: only F32 data supported");
            return ENGINE_ERR_INVALID_ARG;
        }
        int32_t ax;
        int64_t outer, len, inner;
        if (!axis_split(data, axis, &ax, &outer, &len, &inner)) {
            set_error("gather: axis out of range");
            return ENGINE_ERR_INVALID_ARG;
        }
        const int64_t ni = idx.numel();
        int64_t od[8];
        int32_t orank = 0;
        for (int32_t d = 0; d < ax; ++d) od[orank++] = data.dims[d];
        od[orank++] = ni;
        for (int32_t d = ax + 1; d < data.rank; ++d) od[orank++] = data.dims[d];
        HostTensor O = new_f32(od, orank);
        auto get = [&](int64_t i) -> int64_t {
            switch (idx.dtype) {
                case pdefa::kI64: return static_cast<const int64_t*>(idx.data)[i];
                case pdefa::kI32: return static_cast<const int32_t*>(idx.data)[i];
                default: return static_cast<int64_t>(static_cast<const float*>(idx.data)[i]);
            }
        };
        for (int64_t o = 0; o < outer; ++o)
            for (int64_t j = 0; j < ni; ++j) {
                int64_t g = get(j);
                if (g < 0) g += len;
                if (g < 0 || g >= len) g = 0;
                std::memcpy(O.f32() + (o * ni + j) * inner, data.f32() + (o * len + g) * inner,
                            static_cast<size_t>(inner) * sizeof(float));
            }
        *out = wrap(std::move(O));
        return ENGINE_OK;
    });
}

// engine_api.cpp:1311-1364
PDEFA_EXPORT EngineStatus engine_ops_reshape(const EngineTensor* a, const int64_t* shape, int32_t rank, EngineTensor** out) {
    if (!valid(a)) return ENGINE_ERR_INVALID_HANDLE;
    if (!shape || !out) return ENGINE_ERR_NULL_PTR;
    if (rank < 0 || rank > 8) return ENGINE_ERR_INVALID_SHAPE;
    *out = nullptr;
    return guarded([&] {
        clear_error();
        const HostTensor& in = *a->ptr();
        if (in.dtype != pdefa::kF32) {
            set_error("reshape: only F32 supported");
            return ENGINE_ERR_INVALID_ARG;
        }
        int64_t d[8];
        int64_t known = 1;
        int32_t neg = -1;
        for (int32_t i = 0; i < rank; ++i) {
            d[i] = shape[i];
            if (d[i] == -1) neg = i;
            else if (d[i] > 0) known *= d[i];
        }
        if (neg >= 0) d[neg] = known > 0 ? in.numel() / known : 0;
        int64_t total = 1;
        for (int32_t i = 0; i < rank; ++i) total *= d[i];
        if (total != in.numel()) {
            set_error("reshape: numel mismatch");
            return ENGINE_ERR_INVALID_SHAPE;
        }
        HostTensor O = new_f32(d, rank);
        if (in.nbytes) std::memcpy(O.data, in.data, in.nbytes);
        *out = wrap(std::move(O));
        return ENGINE_OK;
    });
}

// engine_api.cpp:1366-1430
PDEFA_EXPORT EngineStatus engine_ops_transpose(const EngineTensor* a, const int32_t* perm, int32_t rank,
                                               EngineTensor** out) {
    if (!valid(a)) return ENGINE_ERR_INVALID_HANDLE;
    if (!perm || !out) return ENGINE_ERR_NULL_PTR;
    *out = nullptr;
    return guarded([&] {
        clear_error();
        const HostTensor& in = *a->ptr();
        if (in.dtype != pdefa::kF32) {
            set_error("transpose: only F32 supported");
            return ENGINE_ERR_INVALID_ARG;
        }
        if (rank != in.rank) {
            set_error("transpose: perm rank mismatch");
            return ENGINE_ERR_INVALID_SHAPE;
        }
        int32_t pv[8];
        for (int32_t i = 0; i < rank; ++i) {
            int32_t p = perm[i] < 0 ? perm[i] + rank : perm[i];
            if (p < 0 || p >= rank) {
                set_error("transpose: invalid perm");
                return ENGINE_ERR_INVALID_ARG;
            }
            pv[i] = p;
        }
        int64_t od[8], istr[8];
        for (int32_t i = 0; i < rank; ++i) od[i] = in.dims[pv[i]];
        if (rank > 0) {
            istr[rank - 1] = 1;
            for (int32_t d = rank - 2; d >= 0; --d) istr[d] = istr[d + 1] * in.dims[d + 1];
        }
        HostTensor O = new_f32(od, rank);
        const int64_t n = O.numel();
        int64_t idx[8];
        for (int64_t i = 0; i < n; ++i) {
            int64_t t = i;
            for (int32_t d = rank - 1; d >= 0; --d) {
                idx[d] = t % od[d];
                t /= od[d];
            }
            int64_t src = 0;
            for (int32_t d = 0; d < rank; ++d) src += idx[d] * istr[pv[d]];
            O.f32()[i] = in.f32()[src];
        }
        *out = wrap(std::move(O));
        return ENGINE_OK;
    });
}

// engine_api.cpp:1432-1500
PDEFA_EXPORT EngineStatus engine_ops_concat(const EngineTensor* const* inputs, int32_t n, int32_t axis, EngineTensor** out) {
    if (!inputs || n < 1 || !out) return ENGINE_ERR_NULL_PTR;
    *out = nullptr;
    return guarded([&] {
        clear_error();
        for (int32_t i = 0; i < n; ++i)
            if (!valid(inputs[i])) return ENGINE_ERR_INVALID_HANDLE;
        const HostTensor& t0 = *inputs[0]->ptr();
        const int32_t rank = t0.rank;
        const int32_t ax = axis < 0 ? axis + rank : axis;
        if (ax < 0 || ax >= rank) {
            set_error("concat: axis out of range");
            return ENGINE_ERR_INVALID_ARG;
        }
        int64_t od[8];
        for (int32_t d = 0; d < rank; ++d) od[d] = t0.dims[d];
        od[ax] = 0;
        for (int32_t i = 0; i < n; ++i) {
            const HostTensor& ti = *inputs[i]->ptr();
            if (ti.rank != rank) {
                set_error("concat: rank mismatch");
                return ENGINE_ERR_INVALID_SHAPE;
            }
            for (int32_t d = 0; d < rank; ++d)
                if (d != ax && ti.dims[d] != od[d]) {
                    set_error("concat: non-axis dim mismatch");
                    return ENGINE_ERR_INVALID_SHAPE;
                }
            od[ax] += ti.dims[ax];
        }
        HostTensor O = new_f32(od, rank);
        int64_t outer = 1, inner = 1;
        for (int32_t d = 0; d < ax; ++d) outer *= od[d];
        for (int32_t d = ax + 1; d < rank; ++d) inner *= od[d];
        for (int64_t o = 0; o < outer; ++o) {
            int64_t dst = o * od[ax] * inner;
            for (int32_t i = 0; i < n; ++i) {
                const HostTensor& ti = *inputs[i]->ptr();
                const int64_t len = ti.dims[ax] * inner;
                std::memcpy(O.f32() + dst, ti.f32() + o * len, static_cast<size_t>(len) * sizeof(float));
                dst += len;
            }
        }
        *out = wrap(std::move(O));
        return ENGINE_OK;
    });
}

// engine_api.cpp:1502-1574
PDEFA_EXPORT EngineStatus engine_ops_stack(const EngineTensor* const* inputs, int32_t n, int32_t axis, EngineTensor** out) {
    if (!inputs || n < 1 || !out) return ENGINE_ERR_NULL_PTR;
    *out = nullptr;
    return guarded([&] {
        clear_error();
        for (int32_t i = 0; i < n; ++i)
            if (!valid(inputs[i])) return ENGINE_ERR_INVALID_HANDLE;
        const HostTensor& t0 = *inputs[0]->ptr();
        const int32_t rank = t0.rank, nr = rank + 1;
        const int32_t ax = axis < 0 ? axis + nr : axis;
        if (ax < 0 || ax >= nr || nr > 8) {
            set_error("stack: axis out of range");
            return ENGINE_ERR_INVALID_ARG;
        }
        for (int32_t i = 1; i < n; ++i) {
            const HostTensor& ti = *inputs[i]->ptr();
            if (ti.rank != rank) {
                set_error("stack: rank mismatch");
                return ENGINE_ERR_INVALID_SHAPE;
            }
            for (int32_t d = 0; d < rank; ++d)
                if (ti.dims[d] != t0.dims[d]) {
                    set_error("stack: shape mismatch");
                    return ENGINE_ERR_INVALID_SHAPE;
                }
        }
        int64_t od[8];
        for (int32_t d = 0, j = 0; d < nr; ++d) od[d] = d == ax ? n : t0.dims[j++];
        HostTensor O = new_f32(od, nr);
        int64_t outer = 1;
        for (int32_t d = 0; d < ax; ++d) outer *= od[d];
        const int64_t inner = outer > 0 ? t0.numel() / outer : t0.numel();
        for (int64_t o = 0; o < outer; ++o)
            for (int32_t i = 0; i < n; ++i)
                std::memcpy(O.f32() + (o * n + i) * inner, inputs[i]->ptr()->f32() + o * inner,
                            static_cast<size_t>(inner) * sizeof(float));
        *out = wrap(std::move(O));
        return ENGINE_OK;
    });
}

// engine_api.cpp:1093-1140
static EngineStatus random_impl(const int64_t* shape, int32_t rank, uint64_t seed, EngineTensor** out, bool normal) {
    if (!shape || !out) return ENGINE_ERR_NULL_PTR;
    if (rank < 0 || rank > 8) return ENGINE_ERR_INVALID_SHAPE;
    *out = nullptr;
    return guarded([&] {
        clear_error();
        HostTensor O = new_f32(shape, rank);
        std::mt19937_64 rng(seed);
        const int64_t n = O.numel();
        if (normal) {
            std::normal_distribution<float> dist(0.0f, 1.0f);
            for (int64_t i = 0; i < n; ++i) O.f32()[i] = dist(rng);
        } else {
            std::uniform_real_distribution<float> dist(0.0f, 1.0f);
            for (int64_t i = 0; i < n; ++i) O.f32()[i] = dist(rng);
        }
        *out = wrap(std::move(O));
        return ENGINE_OK;
    });
}

PDEFA_EXPORT EngineStatus engine_random_randn(const int64_t* shape, int32_t rank, uint64_t seed, EngineTensor** out) {
    return random_impl(shape, rank, seed, out, true);
}
PDEFA_EXPORT EngineStatus engine_random_rand(const int64_t* shape, int32_t rank, uint64_t seed, EngineTensor** out) {
    return random_impl(shape, rank, seed, out, false);
}

}  // extern "C"
