// Ctools.cpp -- Storage / Tensor of the host stand-in types, with a small
// caching pool for HIP device buffers (so the per-call output allocation the
// reference's CompiledKernel::execute contract implies does not hit
// hipMalloc on every dispatch).
#include "C3/Ctools.h"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <map>
#include <mutex>

namespace ct {
namespace {

// Size-class pool: blocks are rounded up to 256 B (small) or 2 MiB (large)
// and reused by exact rounded size.  Work is issued on one stream per
// process, so a block freed after its last use may be handed out again
// immediately (stream order keeps the old and new uses apart).
std::mutex g_pool_mu;
std::multimap<size_t, void*> g_pool;

size_t roundSize(size_t n) {
    if (n <= (1u << 20)) return (n + 255) & ~size_t(255);
    const size_t two_mb = size_t(2) << 20;
    return (n + two_mb - 1) / two_mb * two_mb;
}

void* poolAlloc(size_t n, size_t* cap) {
    *cap = roundSize(n == 0 ? 1 : n);
    {
        std::lock_guard<std::mutex> lk(g_pool_mu);
        auto it = g_pool.find(*cap);
        if (it != g_pool.end()) {
            void* p = it->second;
            g_pool.erase(it);
            return p;
        }
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, *cap);
    if (e != hipSuccess) {
        releaseCachedDeviceMemory();
        e = hipMalloc(&p, *cap);
    }
    if (e != hipSuccess) throw std::runtime_error(std::string("hipMalloc failed: ") + hipGetErrorString(e));
    return p;
}

void poolFree(void* p, size_t cap) {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    g_pool.emplace(cap, p);
}

}  // namespace

void releaseCachedDeviceMemory() {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    if (!g_pool.empty()) (void)hipDeviceSynchronize();
    for (auto& kv : g_pool) (void)hipFree(kv.second);
    g_pool.clear();
}

Storage::Storage(size_t nbytes, DeviceType dev) : nbytes_(nbytes), dev_(dev), owned_(true) {
    if (dev == DeviceType::kHIP) {
        ptr_ = poolAlloc(nbytes, &capacity_);
    } else {
        capacity_ = nbytes;
        ptr_ = std::malloc(nbytes == 0 ? 1 : nbytes);
        if (!ptr_) throw std::bad_alloc();
    }
}

Storage::~Storage() {
    if (!owned_ || !ptr_) return;
    if (dev_ == DeviceType::kHIP)
        poolFree(ptr_, capacity_);
    else
        std::free(ptr_);
}

Tensor::Tensor(ShapeTag, std::vector<size_t> shape, DType dt, DeviceType dev)
    : shape_(std::move(shape)), dtype_(dt), dev_(dev), defined_(true) {
    storage_ = std::make_shared<Storage>(numel() * dtypeSize(dt), dev);
}

Tensor Tensor::fromBlob(void* data, std::vector<size_t> shape, DType dt, DeviceType dev) {
    Tensor t;
    t.shape_ = std::move(shape);
    t.dtype_ = dt;
    t.dev_ = dev;
    t.defined_ = true;
    t.storage_ = std::make_shared<Storage>(data, t.numel() * dtypeSize(dt), dev);
    return t;
}

size_t Tensor::numel() const {
    size_t n = 1;
    for (size_t s : shape_) n *= s;
    return n;
}

void c3log(ErrorLevel lvl, const std::string& msg) {
    static const bool verbose = [] {
        const char* v = std::getenv("C3_VERBOSE");
        return v && *v && *v != '0';
    }();
    if (lvl == ErrorLevel::DEBUG && !verbose) return;
    if (lvl == ErrorLevel::INFO && !verbose) return;
    const char* tag = lvl == ErrorLevel::WARN ? "WARN" : lvl == ErrorLevel::ERROR ? "ERROR" : lvl == ErrorLevel::INFO ? "INFO" : "DEBUG";
    std::fprintf(stderr, "[C3 %s] %s\n", tag, msg.c_str());
}

}  // namespace ct
