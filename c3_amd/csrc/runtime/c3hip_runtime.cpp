// c3hip_runtime.cpp -- host side of the C ABI in include/c3hip.h.
//
// Loads the prebuilt gfx950 code objects (elementwise.hsaco, gemm_f32.hsaco,
// gemm_bf16.hsaco, reduce.hsaco, loss.hsaco) with hipModuleLoadData, resolves kernels by
// name, validates arguments, picks the kernel variant (tile shape, vector or
// scalar loads) and launches it with hipModuleLaunchKernel on the caller's
// stream.  Device buffers are the caller's; nothing is copied host<->device.
//
// The reference's GPU attempt (src/C3/DCUCompiledKernel.cpp:127-209) copied
// every input host->device and the output back per call and launched one
// 64-thread block; none of that is repeated here.
#include "c3hip.h"
#include "c3hip_internal.h"

#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <string>
#include <unordered_map>
#include <vector>

namespace c3hip {

namespace {

thread_local std::string t_error;

// Launch timing (c3hip_set_launch_timing): each launch of the thread between
// two events on its stream.
struct TimedLaunch {
    std::string name;
    hipEvent_t start = nullptr, stop = nullptr;
};
thread_local bool t_timing = false;
thread_local std::vector<TimedLaunch> t_launches;

void drop_timings() {
    for (auto& t : t_launches) {
        if (t.start) (void)hipEventDestroy(t.start);
        if (t.stop) (void)hipEventDestroy(t.stop);
    }
    t_launches.clear();
}

struct DeviceState {
    int device = -1;
    std::vector<hipModule_t> modules;
    std::vector<std::string> module_names;
    std::vector<uint64_t> module_hashes;  // image_hash() of each loaded image
    std::vector<size_t> module_sizes;
    std::unordered_map<std::string, hipFunction_t> fns;
    bool dir_scanned = false;
};

// 64-bit FNV-1a over the image bytes: identifies which image a loaded module
// came from, so that a second registration of a module can be checked.
uint64_t image_hash(const void* data, size_t n) {
    const unsigned char* p = static_cast<const unsigned char*>(data);
    uint64_t h = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= 0x100000001b3ull;
    }
    return h;
}

bool read_file(const std::string& path, std::vector<char>* out) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    bool ok = std::fseek(f, 0, SEEK_END) == 0;
    const long n = ok ? std::ftell(f) : -1;
    ok = ok && n > 0 && std::fseek(f, 0, SEEK_SET) == 0;
    if (ok) {
        out->resize((size_t)n);
        ok = std::fread(out->data(), 1, (size_t)n, f) == (size_t)n;
    }
    std::fclose(f);
    return ok;
}

// Load `image` as module `name` on the current device (the caller holds g_mu).
int add_module(DeviceState* ds, const std::string& name, const void* image, size_t nbytes, const std::string& what) {
    hipModule_t m = nullptr;
    const hipError_t e = hipModuleLoadData(&m, image);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return set_error(C3HIP_ERR_HIP, "hipModuleLoadData(" + what + ") failed: " + hipGetErrorString(e));
    }
    ds->modules.push_back(m);
    ds->module_names.push_back(name);
    ds->module_hashes.push_back(image_hash(image, nbytes));
    ds->module_sizes.push_back(nbytes);
    return C3HIP_OK;
}

std::mutex g_mu;
std::unordered_map<int, std::unique_ptr<DeviceState>> g_devices;

const char* const kModuleNames[] = {"elementwise", "gemm_f32", "gemm_bf16", "reduce", "loss"};

bool known_module(const std::string& name) {
    for (const char* m : kModuleNames)
        if (name == m) return true;
    return false;
}

int module_index(const DeviceState& ds, const std::string& name) {
    for (size_t i = 0; i < ds.module_names.size(); ++i)
        if (ds.module_names[i] == name) return (int)i;
    return -1;
}

bool has_module(const DeviceState& ds, const std::string& name) { return module_index(ds, name) >= 0; }

std::string library_dir() {
    Dl_info info;
    if (dladdr((void*)&library_dir, &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        const size_t slash = p.rfind('/');
        if (slash != std::string::npos) return p.substr(0, slash);
    }
    return ".";
}

std::string code_object_dir() {
    const char* env = std::getenv("C3_HIP_CODE_OBJECT_DIR");
    if (env && *env) return env;
    return library_dir();
}

DeviceState* device_state(int device) {
    auto it = g_devices.find(device);
    if (it != g_devices.end()) return it->second.get();
    auto ds = std::make_unique<DeviceState>();
    ds->device = device;
    DeviceState* p = ds.get();
    g_devices.emplace(device, std::move(ds));
    return p;
}

// Load, on first use per device, every prebuilt module not already
// registered through c3hip_load_code_object.  The caller holds g_mu and has
// made `device` current.
int load_device(int device, DeviceState** out) {
    DeviceState* ds = device_state(device);
    if (!ds->dir_scanned) {
        const std::string dir = code_object_dir();
        for (const char* name : kModuleNames) {
            if (has_module(*ds, name)) continue;
            const std::string path = dir + "/" + name + ".hsaco";
            std::vector<char> image;
            if (!read_file(path, &image)) return set_error(C3HIP_ERR_NOT_FOUND, "cannot read code object " + path);
            const int rc = add_module(ds, name, image.data(), image.size(), path);
            if (rc) return rc;
        }
        ds->dir_scanned = true;
        // Workspaces (split-K partials, backward pre-pass buffers) come from
        // the device's default stream-ordered pool; keep freed blocks in the
        // pool across synchronizations instead of returning them to the
        // driver, so a repeated call reuses its workspace without remapping.
        hipMemPool_t pool = nullptr;
        if (hipDeviceGetDefaultMemPool(&pool, device) == hipSuccess && pool != nullptr) {
            uint64_t keep = UINT64_MAX;
            if (hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep) != hipSuccess)
                (void)hipGetLastError();
        } else {
            (void)hipGetLastError();
        }
    }
    *out = ds;
    return C3HIP_OK;
}

}  // namespace

int set_error(int code, const std::string& msg) {
    t_error = msg;
    return code;
}

void clear_error() { t_error.clear(); }

const char* last_error() { return t_error.c_str(); }

int current_device(int* dev) {
    hipError_t e = hipGetDevice(dev);
    if (e != hipSuccess) return set_error(C3HIP_ERR_HIP, std::string("hipGetDevice failed: ") + hipGetErrorString(e));
    return C3HIP_OK;
}

int get_function(const char* name, hipFunction_t* fn) {
    int dev = 0;
    int rc = current_device(&dev);
    if (rc) return rc;
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceState* ds = nullptr;
    rc = load_device(dev, &ds);
    if (rc) return rc;
    auto it = ds->fns.find(name);
    if (it != ds->fns.end()) {
        *fn = it->second;
        return C3HIP_OK;
    }
    for (hipModule_t m : ds->modules) {
        hipFunction_t f = nullptr;
        const hipError_t e = hipModuleGetFunction(&f, m, name);
        if (e == hipSuccess && f) {
            ds->fns.emplace(name, f);
            *fn = f;
            return C3HIP_OK;
        }
        // A miss in one module records hipErrorNotFound as the thread's last
        // HIP error; clear it so it is not reported by an unrelated later call.
        (void)hipGetLastError();
    }
    return set_error(C3HIP_ERR_NOT_FOUND, std::string("kernel not found in code objects: ") + name);
}

int launch(const char* name, dim3 grid, dim3 block, void** args, hipStream_t stream) {
    hipFunction_t fn = nullptr;
    int rc = get_function(name, &fn);
    if (rc) return rc;
    TimedLaunch tl;
    if (t_timing) {
        if (hipEventCreate(&tl.start) != hipSuccess || hipEventCreate(&tl.stop) != hipSuccess ||
            hipEventRecord(tl.start, stream) != hipSuccess) {
            (void)hipGetLastError();
            if (tl.start) (void)hipEventDestroy(tl.start);
            if (tl.stop) (void)hipEventDestroy(tl.stop);
            return set_error(C3HIP_ERR_HIP, std::string("launch timing: event set-up failed for ") + name);
        }
    }
    hipError_t e = hipModuleLaunchKernel(fn, grid.x, grid.y, grid.z, block.x, block.y, block.z, 0, stream, args,
                                         nullptr);
    if (t_timing) {
        if (e == hipSuccess && hipEventRecord(tl.stop, stream) == hipSuccess) {
            tl.name = name;
            t_launches.push_back(tl);
        } else {
            (void)hipEventDestroy(tl.start);
            (void)hipEventDestroy(tl.stop);
        }
    }
    if (e != hipSuccess)
        return set_error(C3HIP_ERR_HIP, std::string("hipModuleLaunchKernel(") + name + ") failed: " + hipGetErrorString(e));
    return C3HIP_OK;
}

int set_launch_timing(int enable) {
    if (!enable) drop_timings();
    t_timing = enable != 0;
    return C3HIP_OK;
}

int launch_timings(char* names, size_t name_len, float* ms, int max, int* count) {
    if (!count || max < 0 || (max > 0 && (!ms || (names && name_len == 0))))
        return set_error(C3HIP_ERR_INVALID, "launch_timings: bad output buffers");
    int n = 0;
    int rc = C3HIP_OK;
    for (auto& t : t_launches) {
        if (n >= max) break;
        float v = -1.0f;
        if (hipEventSynchronize(t.stop) != hipSuccess || hipEventElapsedTime(&v, t.start, t.stop) != hipSuccess) {
            (void)hipGetLastError();
            rc = set_error(C3HIP_ERR_HIP, "launch timing: reading the events of " + t.name + " failed");
            v = -1.0f;
        }
        ms[n] = v;
        if (names) {
            const size_t k = std::min(name_len - 1, t.name.size());
            std::memcpy(names + (size_t)n * name_len, t.name.data(), k);
            names[(size_t)n * name_len + k] = 0;
        }
        ++n;
    }
    drop_timings();
    *count = n;
    return rc;
}

int init_device(int device) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return set_error(C3HIP_ERR_HIP, std::string("hipGetDeviceCount failed: ") + hipGetErrorString(e));
    if (device < 0 || device >= count)
        return set_error(C3HIP_ERR_INVALID, "device " + std::to_string(device) + " out of range (count " +
                                                std::to_string(count) + ")");
    e = hipSetDevice(device);
    if (e != hipSuccess) return set_error(C3HIP_ERR_HIP, std::string("hipSetDevice failed: ") + hipGetErrorString(e));
    {
        std::lock_guard<std::mutex> lock(g_mu);
        DeviceState* ds = nullptr;
        const int rc = load_device(device, &ds);
        if (rc) return rc;
    }
    // Set-up of c3hip_linear_fwd_noalloc's static scratch on this device.  A
    // failure is kept and reported by that entry point; the other entry
    // points do not depend on it.
    if (noalloc_setup(device) != C3HIP_OK) clear_error();
    return C3HIP_OK;
}

int load_code_object(const char* module_name, const void* image, size_t nbytes) {
    if (!module_name || !image || nbytes == 0) return set_error(C3HIP_ERR_INVALID, "null module name or image");
    if (!known_module(module_name)) return set_error(C3HIP_ERR_INVALID, std::string("unknown module ") + module_name);
    int dev = 0;
    int rc = current_device(&dev);
    if (rc) return rc;
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceState* ds = device_state(dev);
    const int idx = module_index(*ds, module_name);
    if (idx >= 0) {
        // Already loaded: accept only the same image (kernel lookups keep
        // using the loaded module, so a different image would not take effect).
        if (ds->module_sizes[idx] == nbytes && ds->module_hashes[idx] == image_hash(image, nbytes)) return C3HIP_OK;
        return set_error(C3HIP_ERR_INVALID, std::string("code object for module ") + module_name +
                                                " differs from the image already loaded on device " +
                                                std::to_string(dev));
    }
    return add_module(ds, module_name, image, nbytes, module_name);
}

int code_object_path(const char* module_name, char* buf, size_t buflen) {
    if (!module_name || !known_module(module_name)) return set_error(C3HIP_ERR_INVALID, "unknown module");
    const std::string p = code_object_dir() + "/" + module_name + ".hsaco";
    if (!buf || buflen < p.size() + 1) return set_error(C3HIP_ERR_INVALID, "buffer too small for " + p);
    std::memcpy(buf, p.c_str(), p.size() + 1);
    return C3HIP_OK;
}

// ---- workspace arenas ----------------------------------------------------
// One device buffer per (device, stream) for the workspaces of the library's
// calls.  hipMallocAsync / hipFreeAsync on every call held the calling thread
// until the stream had caught up (measured on MI355X: a small bf16 layer
// backward, 58 us of GPU work, returned to the host after 57 us instead of a
// few), so consecutive calls could not queue ahead of the GPU.  Calls on one
// stream run in stream order, so each call can reuse the arena from offset 0;
// a call on another thread that finds the arena in use, and every call under
// stream capture (whose graph must own its memory), takes the stream-ordered
// allocator instead.  A call that needed more than the arena held sets the
// size for the next one: the arena grows when that call's last workspace is
// freed, after the stream has drained.  Freed by c3hip_shutdown.
namespace {
struct Arena {
    void* base = nullptr;
    size_t cap = 0, used = 0, want = 0;
    int live = 0;
    std::thread::id owner;
    uint64_t last_use = 0;
};
std::mutex g_arena_mu;
std::map<std::pair<int, hipStream_t>, Arena> g_arenas;
uint64_t g_arena_clock = 0;
constexpr size_t kArenaAlign = 256;
// Arenas kept per device: a process that cycles through many streams (one
// per request, say) would otherwise keep one per stream it ever used.  The
// least recently used idle arena beyond this is freed after a device
// synchronisation (its stream may no longer exist).
constexpr int kMaxArenasPerDevice = 8;

// The arena for (dev, stream), made if new; evicts as above.  The caller
// holds g_arena_mu.
Arena& arena_for(int dev, hipStream_t stream) {
    auto it = g_arenas.find({dev, stream});
    if (it == g_arenas.end()) {
        int n = 0;
        auto lru = g_arenas.end();
        for (auto j = g_arenas.begin(); j != g_arenas.end(); ++j) {
            if (j->first.first != dev) continue;
            ++n;
            if (j->second.live == 0 && (lru == g_arenas.end() || j->second.last_use < lru->second.last_use)) lru = j;
        }
        if (n >= kMaxArenasPerDevice && lru != g_arenas.end()) {
            if (!lru->second.base)
                g_arenas.erase(lru);
            else if (hipDeviceSynchronize() == hipSuccess && hipFree(lru->second.base) == hipSuccess)
                g_arenas.erase(lru);
            else
                (void)hipGetLastError();
        }
        it = g_arenas.emplace(std::make_pair(dev, stream), Arena{}).first;
    }
    it->second.last_use = ++g_arena_clock;
    return it->second;
}
}  // namespace

int ws_alloc(size_t bytes, hipStream_t stream, void** p, bool* arena, const char* what) {
    *arena = false;
    *p = nullptr;
    if (bytes == 0) bytes = 1;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess) {
        (void)hipGetLastError();
        cs = hipStreamCaptureStatusActive;  // unknown: take the stream-ordered allocator
    }
    const char* off = std::getenv("C3_HIP_WORKSPACE_ARENA");
    if (off && off[0] == '0') cs = hipStreamCaptureStatusActive;  // arena switched off: stream-ordered allocator
    int dev = 0;
    if (cs == hipStreamCaptureStatusNone && hipGetDevice(&dev) == hipSuccess) {
        std::lock_guard<std::mutex> lock(g_arena_mu);
        Arena& a = arena_for(dev, stream);
        if (a.live == 0 || a.owner == std::this_thread::get_id()) {
            const size_t off = (a.used + kArenaAlign - 1) / kArenaAlign * kArenaAlign;
            if (off + bytes <= a.cap) {
                *p = static_cast<char*>(a.base) + off;
                a.used = off + bytes;
                a.live++;
                a.owner = std::this_thread::get_id();
                *arena = true;
                return C3HIP_OK;
            }
            a.want = std::max(a.want, off + bytes);
        }
    } else if (cs == hipStreamCaptureStatusNone) {
        (void)hipGetLastError();
    }
    hipError_t e = hipMallocAsync(p, bytes, stream);
    if (e != hipSuccess) return set_error(C3HIP_ERR_HIP, std::string("hipMallocAsync(") + what + "): " + hipGetErrorString(e));
    return C3HIP_OK;
}

namespace {
// With the arena idle and a call having needed more than it holds, replace it
// by one of that size (+25%, whole MiB) once the stream's queued kernels are
// done with the old one.  No arena on failure: calls then take the
// stream-ordered allocator.  The caller holds g_arena_mu.
int grow_arena(Arena& a, hipStream_t stream) {
    if (a.live > 0 || a.want <= a.cap) return C3HIP_OK;
    const size_t cap = (a.want + a.want / 4 + (1u << 20) - 1) / (1u << 20) * (1u << 20);
    a.want = 0;
    hipError_t e = hipStreamSynchronize(stream);
    if (e == hipSuccess && a.base) e = hipFree(a.base);
    if (e != hipSuccess) return set_error(C3HIP_ERR_HIP, std::string("workspace arena: ") + hipGetErrorString(e));
    a.base = nullptr;
    a.cap = 0;
    if (hipMalloc(&a.base, cap) != hipSuccess) {
        (void)hipGetLastError();
        a.base = nullptr;
        return C3HIP_OK;
    }
    a.cap = cap;
    return C3HIP_OK;
}
}  // namespace

int ws_free(void* p, bool arena, hipStream_t stream, const char* what) {
    if (!arena) {
        hipError_t e = hipFreeAsync(p, stream);
        if (e != hipSuccess) return set_error(C3HIP_ERR_HIP, std::string("hipFreeAsync(") + what + "): " + hipGetErrorString(e));
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return arena ? set_error(C3HIP_ERR_HIP, "hipGetDevice failed") : C3HIP_OK;
    }
    std::lock_guard<std::mutex> lock(g_arena_mu);
    auto it = g_arenas.find({dev, stream});
    if (it == g_arenas.end()) return arena ? set_error(C3HIP_ERR_INVALID, "workspace arena not found") : C3HIP_OK;
    Arena& a = it->second;
    if (arena) {
        if (--a.live > 0) return C3HIP_OK;
        a.used = 0;
    }
    return grow_arena(a, stream);
}

int shutdown_all() {
    std::lock_guard<std::mutex> lock(g_mu);
    int rc = C3HIP_OK;
    int prev = -1;
    (void)hipGetDevice(&prev);
    for (auto& kv : g_devices) {
        (void)hipSetDevice(kv.first);
        for (hipModule_t m : kv.second->modules) {
            hipError_t e = hipModuleUnload(m);
            if (e != hipSuccess && rc == C3HIP_OK)
                rc = set_error(C3HIP_ERR_HIP, std::string("hipModuleUnload failed: ") + hipGetErrorString(e));
        }
    }
    g_devices.clear();
    {
        std::lock_guard<std::mutex> alock(g_arena_mu);
        for (auto& kv : g_arenas) {
            if (!kv.second.base) continue;
            (void)hipSetDevice(kv.first.first);
            hipError_t e = hipDeviceSynchronize();
            if (e == hipSuccess) e = hipFree(kv.second.base);
            if (e != hipSuccess && rc == C3HIP_OK)
                rc = set_error(C3HIP_ERR_HIP, std::string("workspace arena free failed: ") + hipGetErrorString(e));
        }
        g_arenas.clear();
    }
    if (prev >= 0) (void)hipSetDevice(prev);
    return rc;
}

}  // namespace c3hip

extern "C" {

int c3hip_abi_version(void) { return C3HIP_ABI_VERSION; }

const char* c3hip_last_error(void) { return c3hip::last_error(); }

int c3hip_init(int device) {
    c3hip::clear_error();
    return c3hip::init_device(device);
}

int c3hip_shutdown(void) {
    c3hip::clear_error();
    return c3hip::shutdown_all();
}

int c3hip_load_code_object(const char* module_name, const void* image, size_t nbytes) {
    c3hip::clear_error();
    return c3hip::load_code_object(module_name, image, nbytes);
}

int c3hip_code_object_path(const char* module_name, char* buf, size_t buflen) {
    c3hip::clear_error();
    return c3hip::code_object_path(module_name, buf, buflen);
}

int c3hip_set_launch_timing(int enable) {
    c3hip::clear_error();
    return c3hip::set_launch_timing(enable);
}

int c3hip_launch_timings(char* names, size_t name_len, float* ms, int max, int* count) {
    c3hip::clear_error();
    return c3hip::launch_timings(names, name_len, ms, max, count);
}

}  // extern "C"
