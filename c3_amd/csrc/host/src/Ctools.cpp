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
#include <stdexcept>
#include <string>
#include <vector>

namespace ct {
namespace c3 {
void* getCurrentStream();
}
namespace {

// Size-class pool: blocks are rounded up to 256 B (small) or 2 MiB (large)
// and reused by exact rounded size.  A block remembers the stream it was
// allocated on (the calling thread's current stream), whose work may still
// use it after it is freed:
//  - on that same stream a freed block is handed out again at once (stream
//    order keeps the old and new uses apart);
//  - once the process has allocated on more than one stream, freeing a block
//    records an event on its stream, and a request from another stream makes
//    that stream wait for the event (hipStreamWaitEvent) before taking it;
//  - a block freed before a second stream appeared (no event) is handed to
//    another stream only after the device has drained (hipDeviceSynchronize).
// Nothing is recorded on or waited for by a stream that is being captured
// into a HIP graph: such a stream reuses only its own blocks.
struct Block {
    void* ptr = nullptr;
    hipStream_t stream = nullptr;
    hipEvent_t ready = nullptr;
};

std::mutex g_pool_mu;
std::multimap<size_t, Block> g_pool;
std::vector<hipEvent_t> g_spare_events;
bool g_any_stream = false, g_multi_stream = false;
hipStream_t g_first_stream = nullptr;

bool capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) {
        (void)hipGetLastError();
        return true;  // cannot tell: treat as capturing (no events, no waits)
    }
    return st != hipStreamCaptureStatusNone;
}

void recycleEvent(hipEvent_t e) {
    if (e) g_spare_events.push_back(e);
}

hipEvent_t takeEvent() {
    if (!g_spare_events.empty()) {
        hipEvent_t e = g_spare_events.back();
        g_spare_events.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return e;
}

size_t roundSize(size_t n) {
    if (n <= (1u << 20)) return (n + 255) & ~size_t(255);
    const size_t two_mb = size_t(2) << 20;
    return (n + two_mb - 1) / two_mb * two_mb;
}

// A cached block of `cap` bytes usable on `stream`, or nullptr (g_pool_mu held).
void* takeCached(size_t cap, hipStream_t stream) {
    auto range = g_pool.equal_range(cap);
    for (auto it = range.first; it != range.second; ++it) {
        if (it->second.stream == stream) {
            void* p = it->second.ptr;
            recycleEvent(it->second.ready);
            g_pool.erase(it);
            return p;
        }
    }
    if (range.first == range.second || capturing(stream)) return nullptr;
    for (auto it = range.first; it != range.second; ++it) {
        Block& b = it->second;
        if (b.ready) {
            if (hipStreamWaitEvent(stream, b.ready, 0) != hipSuccess) {
                (void)hipGetLastError();
                continue;
            }
        } else {
            if (capturing(b.stream)) continue;
            if (hipDeviceSynchronize() != hipSuccess) {
                (void)hipGetLastError();
                continue;
            }
        }
        void* p = b.ptr;
        recycleEvent(b.ready);
        g_pool.erase(it);
        return p;
    }
    return nullptr;
}

void* poolAlloc(size_t n, size_t* cap, hipStream_t stream) {
    *cap = roundSize(n == 0 ? 1 : n);
    {
        std::lock_guard<std::mutex> lk(g_pool_mu);
        if (!g_any_stream) {
            g_any_stream = true;
            g_first_stream = stream;
        } else if (stream != g_first_stream) {
            g_multi_stream = true;
        }
        if (void* p = takeCached(*cap, stream)) return p;
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

void poolFree(void* p, size_t cap, hipStream_t stream) {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    Block b;
    b.ptr = p;
    b.stream = stream;
    if (g_multi_stream && !capturing(stream)) {
        b.ready = takeEvent();
        if (b.ready && hipEventRecord(b.ready, stream) != hipSuccess) {
            (void)hipGetLastError();
            recycleEvent(b.ready);
            b.ready = nullptr;
        }
    }
    g_pool.emplace(cap, b);
}

}  // namespace

void releaseCachedDeviceMemory() {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    if (!g_pool.empty()) (void)hipDeviceSynchronize();
    for (auto& kv : g_pool) {
        (void)hipFree(kv.second.ptr);
        recycleEvent(kv.second.ready);
    }
    g_pool.clear();
    for (hipEvent_t e : g_spare_events) (void)hipEventDestroy(e);
    g_spare_events.clear();
}

Storage::Storage(size_t nbytes, DeviceType dev) : nbytes_(nbytes), dev_(dev), owned_(true) {
    if (dev == DeviceType::kHIP) {
        stream_ = c3::getCurrentStream();
        ptr_ = poolAlloc(nbytes, &capacity_, (hipStream_t)stream_);
    } else {
        capacity_ = nbytes;
        ptr_ = std::malloc(nbytes == 0 ? 1 : nbytes);
        if (!ptr_) throw std::bad_alloc();
    }
}

Storage::~Storage() {
    if (!owned_ || !ptr_) return;
    if (dev_ == DeviceType::kHIP)
        poolFree(ptr_, capacity_, (hipStream_t)stream_);
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
