// c3hip_internal.h -- shared helpers of the C-ABI implementation files.
#pragma once
#include <hip/hip_runtime.h>

#include "c3hip.h"
#include <stdint.h>

#include <string>

namespace c3hip {

// Record `msg` as the calling thread's last error and return `code`.
int set_error(int code, const std::string& msg);
void clear_error();
const char* last_error();

int current_device(int* dev);
int init_device(int device);
int shutdown_all();
int load_code_object(const char* module_name, const void* image, size_t nbytes);
int code_object_path(const char* module_name, char* buf, size_t buflen);

// Resolve `name` in the current device's code objects (loading them on first use).
int get_function(const char* name, hipFunction_t* fn);

// hipModuleLaunchKernel of kernel `name` with the kernelParams array `args`
// (bracketed by two events on `stream` while launch timing is on).
int launch(const char* name, dim3 grid, dim3 block, void** args, hipStream_t stream);
int set_launch_timing(int enable);
int launch_timings(char* names, size_t name_len, float* ms, int max, int* count);

// Workspace of one call (split-K partials, dZ, column-sum partials, W^T):
// carved from the library's arena for (current device, stream) when the
// stream is not being captured and no other thread is using that arena,
// else hipMallocAsync on the stream.  *arena says which; ws_free takes it
// back.  The arena is reset when the last workspace of the call is freed
// (the stream orders the next call's kernels after this one's) and grown,
// after synchronizing the stream, when a call needed more than it held.
int ws_alloc(size_t bytes, hipStream_t stream, void** p, bool* arena, const char* what);
int ws_free(void* p, bool arena, hipStream_t stream, const char* what);

// Kernel argument block of every GEMM code object (mirrors GemmArgs in
// c3_amd/csrc/kernels/gemm_common.h; both sides are plain C layout).
struct GemmArgs {
    const void* A;
    const void* Amask;
    const void* B;
    const void* Bmask;
    void* C;
    const float* bias;
    float* db;
    int64_t M, N, K;
    int64_t lda, ldb, ldc;
    int act;
    int _pad;
    int64_t split_k;
    int64_t c_split;
    void* dz;
};

// Argument block of c3_gemm_f32_bwd[_mask]_t64x64_* (mirrors BwdPairArgs in
// gemm_f32.hip): blocks [0, nx) run dx, the rest dw.
struct BwdPairArgs {
    GemmArgs dx;
    GemmArgs dw;
    int nx;
    int _pad;
};

// Argument block of c3_sgd_multi_* (mirrors SgdMultiArgs in
// c3_amd/csrc/kernels/loss.hip).
struct SgdMultiArgs {
    void* w[C3HIP_SGD_MAX_TENSORS];
    const float* g[C3HIP_SGD_MAX_TENSORS];
    int64_t n[C3HIP_SGD_MAX_TENSORS];
    int64_t first[C3HIP_SGD_MAX_TENSORS + 1];
    int count;
    float lr;
};

// Argument block of c3_splitk_reduce (mirrors SplitReduceArgs in
// c3_amd/csrc/kernels/gemm_bf16.hip).
struct SplitReduceArgs {
    const float* ws;
    void* C;
    const float* bias;
    int64_t M, N, ldc, slice;
    int S, act, out_bf16, _pad;
};

// Kernel argument block of the fused backward chain (mirrors ChainArgs in
// c3_amd/csrc/kernels/elementwise.hip).
constexpr int kChainMaxNodes = 4;
struct ChainArgs {
    const float* g;
    const float* x[kChainMaxNodes];
    float* out[kChainMaxNodes];
    int node[kChainMaxNodes];
    int w;
    int64_t n;
};

inline bool aligned16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Device workspace given to a GEMM plan.  base == nullptr: the plan takes its
// workspace from the stream-ordered pool (hipMallocAsync / hipFreeAsync);
// otherwise it uses [base, base + bytes) and fails with C3HIP_ERR_TOO_LARGE,
// before launching anything, when it needs more.
struct Workspace {
    void* base = nullptr;
    size_t bytes = 0;
};

// Fused Linear forward (c3hip_linear_fwd) with its workspace from ws (NULL:
// the stream-ordered pool).  With a caller workspace it never takes the
// transposed-W forward, which needs a second workspace (same bits either way).
int linear_fwd(int dtype, const void* X, const void* W, const float* b, void* Y, int64_t M, int64_t K, int64_t N,
               int act, hipStream_t stream, const Workspace* ws);

// Set-up of the static scratch of c3hip_linear_fwd_noalloc on `device` (the
// current device): records its device address.  Called by c3hip_init and by
// the entry point's first call on a device.
int noalloc_setup(int device);

}  // namespace c3hip
