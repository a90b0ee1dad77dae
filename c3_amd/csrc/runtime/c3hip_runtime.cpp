// c3hip_runtime.cpp -- host side of the C ABI in include/c3hip.h.
//
// Loads the prebuilt gfx950 code objects (elementwise.hsaco, gemm_f32.hsaco,
// gemm_bf16.hsaco, reduce.hsaco) with hipModuleLoad, resolves kernels by
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
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace c3hip {

namespace {

thread_local std::string t_error;

struct DeviceState {
    int device = -1;
    std::vector<hipModule_t> modules;
    std::vector<std::string> module_names;
    std::unordered_map<std::string, hipFunction_t> fns;
    bool dir_scanned = false;
};

std::mutex g_mu;
std::unordered_map<int, std::unique_ptr<DeviceState>> g_devices;

const char* const kModuleNames[] = {"elementwise", "gemm_f32", "gemm_bf16", "reduce", "loss"};

bool known_module(const std::string& name) {
    for (const char* m : kModuleNames)
        if (name == m) return true;
    return false;
}

bool has_module(const DeviceState& ds, const std::string& name) {
    for (const auto& n : ds.module_names)
        if (n == name) return true;
    return false;
}

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
            hipModule_t m = nullptr;
            hipError_t e = hipModuleLoad(&m, path.c_str());
            if (e != hipSuccess) {
                (void)hipGetLastError();
                return set_error(e == hipErrorFileNotFound ? C3HIP_ERR_NOT_FOUND : C3HIP_ERR_HIP,
                                 "hipModuleLoad(" + path + ") failed: " + hipGetErrorString(e));
            }
            ds->modules.push_back(m);
            ds->module_names.push_back(name);
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
    hipError_t e = hipModuleLaunchKernel(fn, grid.x, grid.y, grid.z, block.x, block.y, block.z, 0, stream, args,
                                         nullptr);
    if (e != hipSuccess)
        return set_error(C3HIP_ERR_HIP, std::string("hipModuleLaunchKernel(") + name + ") failed: " + hipGetErrorString(e));
    return C3HIP_OK;
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
    if (has_module(*ds, module_name)) return C3HIP_OK;
    hipModule_t m = nullptr;
    hipError_t e = hipModuleLoadData(&m, image);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return set_error(C3HIP_ERR_HIP, std::string("hipModuleLoadData(") + module_name + ") failed: " +
                                            hipGetErrorString(e));
    }
    ds->modules.push_back(m);
    ds->module_names.push_back(module_name);
    return C3HIP_OK;
}

int code_object_path(const char* module_name, char* buf, size_t buflen) {
    if (!module_name || !known_module(module_name)) return set_error(C3HIP_ERR_INVALID, "unknown module");
    const std::string p = code_object_dir() + "/" + module_name + ".hsaco";
    if (!buf || buflen < p.size() + 1) return set_error(C3HIP_ERR_INVALID, "buffer too small for " + p);
    std::memcpy(buf, p.c_str(), p.size() + 1);
    return C3HIP_OK;
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

}  // extern "C"
