// Handle structs behind the opaque C types, the thread-local error string and
// the exception barrier shared by the engine_* and pdefa_* entry points.
#pragma once

#include <memory>
#include <new>
#include <string>

#include "../../include/engine_c_api.h"
#include "host_tensor.hpp"
#include "model.hpp"
#include "runtime.hpp"

// Magic tags distinguish live handles from stale or foreign pointers
// (engine_api.cpp:36-39 uses the same idea).
constexpr uint32_t kMagicContext = 0x50444301u;
constexpr uint32_t kMagicModel = 0x50444302u;
constexpr uint32_t kMagicSession = 0x50444303u;
constexpr uint32_t kMagicTensor = 0x50444304u;

struct EngineTensor {
    uint32_t magic = kMagicTensor;
    std::unique_ptr<pdefa::HostTensor> owned;
    pdefa::HostTensor* borrowed = nullptr;  // session outputs: never freed by the caller
    pdefa::HostTensor* ptr() { return owned ? owned.get() : borrowed; }
    const pdefa::HostTensor* ptr() const { return owned ? owned.get() : borrowed; }
    bool is_borrowed() const { return !owned && borrowed != nullptr; }
};

struct EngineContext {
    uint32_t magic = kMagicContext;
    int32_t num_threads = 1;
};

struct EngineModel {
    uint32_t magic = kMagicModel;
    std::unique_ptr<pdefa::Model> inner;
};

struct EngineSession {
    uint32_t magic = kMagicSession;
    std::unique_ptr<pdefa::Session> inner;
};

namespace pdefa {
namespace api {

void set_error(const std::string& msg) noexcept;
void clear_error() noexcept;
const char* last_error() noexcept;

inline bool valid(const EngineTensor* t) { return t && t->magic == kMagicTensor && t->ptr(); }

// Runs fn, mapping exceptions to status codes with the message recorded.
template <typename Fn>
EngineStatus guarded(Fn&& fn) noexcept {
    try {
        return fn();
    } catch (const std::bad_alloc&) {
        set_error("out of memory");
        return ENGINE_ERR_OUT_OF_MEMORY;
    } catch (const HipError& e) {
        set_error(e.what());
        return e.code == hipErrorOutOfMemory ? ENGINE_ERR_OUT_OF_MEMORY : ENGINE_ERR_RUNTIME;
    } catch (const std::invalid_argument& e) {
        set_error(e.what());
        return ENGINE_ERR_INVALID_ARG;
    } catch (const std::exception& e) {
        set_error(e.what());
        return ENGINE_ERR_RUNTIME;
    } catch (...) {
        set_error("unknown exception");
        return ENGINE_ERR_UNKNOWN;
    }
}

// Wraps a new host tensor in a caller-owned handle.
EngineTensor* wrap(HostTensor&& t);

}  // namespace api
}  // namespace pdefa
