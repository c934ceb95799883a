// Static device scratch for the entry points that allocate nothing
// (pdefa_amd_ops_matmul_noalloc): one 32 MiB array per GPU, held from the
// library's load until the process ends.  The array's name is a host-side
// stand-in in host code; its device address is looked up once per device
// with hipGetSymbolAddress and that address is what kernels, copies and
// memsets receive.
#include <hip/hip_runtime.h>

#include <mutex>
#include <sstream>
#include <stdexcept>

namespace pdefa {
float* noalloc_scratch(size_t& floats);
}

namespace {

constexpr size_t kScratchFloats = size_t{8} << 20;  // 32 MiB
constexpr int kMaxDevices = 64;

}  // namespace

static __device__ __align__(256) float scratch[kScratchFloats];

namespace pdefa {

float* noalloc_scratch(size_t& floats) {
    static std::mutex mu;
    static float* ptr[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) throw std::runtime_error(std::string("hipGetDevice: ") + hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) throw std::runtime_error("noalloc scratch: device index out of range");
    std::lock_guard<std::mutex> g(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            std::ostringstream os;
            os << "hipGetSymbolAddress(scratch) on device " << dev << ": " << hipGetErrorString(e);
            throw std::runtime_error(os.str());
        }
        ptr[dev] = static_cast<float*>(p);
    }
    floats = kScratchFloats;
    return ptr[dev];
}

}  // namespace pdefa
