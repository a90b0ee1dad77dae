// c3hip_noalloc.hip -- c3hip_linear_fwd_noalloc: the fused Linear forward of
// c3hip_linear_fwd with every workspace taken from a static device array
// instead of the stream-ordered pool, for callers that cannot allocate
// (code under HIP graph capture, tight serving loops).
//
// The only workspace the forward uses is the fp32 split-K partial product
// [S, M, N] of a GEMM whose grid is too small to fill the chip.  The size
// heuristic bounds it: bf16 splits 128x128-tile grids of T < 256 tiles into
// S parts with S * T <= 512, and M * N <= T * 128 * 128, so S * M * N <=
// 512 * 16384 fp32 = 32 MiB; fp32 splits 64x64-tile grids of T < 32 tiles
// with S <= 256 / T, i.e. at most 256 * 4096 fp32 = 4 MiB.  kScratchBytes
// is therefore 32 MiB, enough for every forward the size heuristic plans;
// only a forced split tile (c3hip_set_gemm_tile) can ask for more, and such a
// call is rejected with C3HIP_ERR_TOO_LARGE before anything is launched.
// Every split block writes all of its partial tile and the reduction reads
// only what was written, so nothing in the scratch has to start at zero.
//
// Each device holds its own copy of the array (at its own address) until
// the process ends.  Calls on one device share it: two calls whose work
// overlaps in time on that device (two streams, or two host threads) race
// on it; calls on one stream are ordered and safe.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>
#include <unordered_map>

#include "c3hip.h"
#include "c3hip_internal.h"

namespace {

constexpr size_t kScratchBytes = C3HIP_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0, "scratch is a whole number of 256-byte blocks");

// In host code `scratch` names a host-side stand-in, not device memory: its
// device address comes from hipGetSymbolAddress (per device) and only that
// address is ever passed to a kernel.
__attribute__((used)) static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct DeviceScratch {
    void* ptr = nullptr;
    int status = C3HIP_OK;
    std::string error;
};

std::mutex g_mu;
std::unordered_map<int, DeviceScratch> g_scratch;

// Device address of `scratch` on `device`, the current device; looked up
// once per device and kept (including a failure, which is reported again).
int scratch_for(int device, void** out) {
    std::lock_guard<std::mutex> lock(g_mu);
    auto it = g_scratch.find(device);
    if (it == g_scratch.end()) {
        DeviceScratch ds;
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            (void)hipGetLastError();
            ds.status = C3HIP_ERR_HIP;
            ds.error = std::string("hipGetSymbolAddress(scratch) failed on device ") + std::to_string(device) + ": " +
                       hipGetErrorString(e);
        } else {
            ds.ptr = p;
        }
        it = g_scratch.emplace(device, ds).first;
    }
    if (it->second.status != C3HIP_OK) return c3hip::set_error(it->second.status, it->second.error);
    *out = it->second.ptr;
    return C3HIP_OK;
}

}  // namespace

namespace c3hip {

int noalloc_setup(int device) {
    void* p = nullptr;
    return scratch_for(device, &p);
}

}  // namespace c3hip

extern "C" int c3hip_linear_fwd_noalloc(int dtype, const void* X, const void* W, const float* b, void* Y, int64_t M,
                                        int64_t K, int64_t N, int act, void* stream) {
    c3hip::clear_error();
    int dev = 0;
    int rc = c3hip::current_device(&dev);
    if (rc) return rc;
    c3hip::Workspace ws;
    rc = scratch_for(dev, &ws.base);
    if (rc) return rc;
    ws.bytes = kScratchBytes;
    return c3hip::linear_fwd(dtype, X, W, b, Y, M, K, N, act, (hipStream_t)stream, &ws);
}
