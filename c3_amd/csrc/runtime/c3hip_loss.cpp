// c3hip_loss.cpp -- entry points of the train-step helpers around the fused
// layers: softmax cross-entropy, dtype casts and the SGD update (kernels in
// c3_amd/csrc/kernels/loss.hip).
#include <hip/hip_runtime.h>

#include <string>

#include "c3hip.h"
#include "c3hip_internal.h"

using namespace c3hip;

namespace {

constexpr int kThreads = 256;     // loss.hip kThreads
constexpr int64_t kMaxClasses = 2048;  // loss.hip: 64 lanes x kMaxPerLane

int grid_for(int64_t n, int64_t per_block, unsigned* blocks) {
    const int64_t b = (n + per_block - 1) / per_block;
    if (b > 0x7fffffff) return set_error(C3HIP_ERR_TOO_LARGE, "grid too large");
    *blocks = (unsigned)b;
    return C3HIP_OK;
}

}  // namespace

extern "C" {

int c3hip_softmax_ce(int dtype, const void* logits, const int32_t* labels, float* loss_rows, void* dlogits,
                     int64_t M, int64_t C, void* stream) {
    clear_error();
    if (dtype != C3HIP_F32 && dtype != C3HIP_BF16) return set_error(C3HIP_ERR_INVALID, "unknown dtype");
    if (M < 0 || C < 0) return set_error(C3HIP_ERR_INVALID, "negative dimension");
    if (M > 0 && C == 0) return set_error(C3HIP_ERR_INVALID, "no classes");
    if (C > kMaxClasses) return set_error(C3HIP_ERR_UNSUPPORTED, "more than 2048 classes");
    if (M == 0 || (!loss_rows && !dlogits)) return C3HIP_OK;
    if (!logits || !labels) return set_error(C3HIP_ERR_INVALID, "null pointer");
    unsigned blocks;
    int rc = grid_for(M, kThreads / 64, &blocks);  // one wave per row
    if (rc) return rc;
    void* args[] = {(void*)&logits, (void*)&labels, &loss_rows, &dlogits, &M, &C};
    return launch(dtype == C3HIP_BF16 ? "c3_softmax_ce_bf16" : "c3_softmax_ce_f32", dim3(blocks), dim3(kThreads),
                  args, (hipStream_t)stream);
}

int c3hip_cast(int src_dtype, int dst_dtype, const void* in, void* out, int64_t n, void* stream) {
    clear_error();
    auto ok = [](int d) { return d == C3HIP_F32 || d == C3HIP_BF16; };
    if (!ok(src_dtype) || !ok(dst_dtype)) return set_error(C3HIP_ERR_INVALID, "unknown dtype");
    if (n < 0) return set_error(C3HIP_ERR_INVALID, "n < 0");
    if (n == 0) return C3HIP_OK;
    if (!in || !out) return set_error(C3HIP_ERR_INVALID, "null pointer");
    if (src_dtype == dst_dtype) {
        const size_t bytes = (size_t)n * (src_dtype == C3HIP_BF16 ? 2 : 4);
        if (hipMemcpyAsync(out, in, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream) != hipSuccess)
            return set_error(C3HIP_ERR_HIP, "hipMemcpyAsync failed");
        return C3HIP_OK;
    }
    unsigned blocks;
    int rc = grid_for(n, 4 * kThreads, &blocks);
    if (rc) return rc;
    void* args[] = {(void*)&in, &out, &n};
    return launch(src_dtype == C3HIP_F32 ? "c3_cast_f32_bf16" : "c3_cast_bf16_f32", dim3(blocks), dim3(kThreads),
                  args, (hipStream_t)stream);
}

int c3hip_sgd_update(int dtype, void* w, const float* g, float lr, int64_t n, void* stream) {
    clear_error();
    if (dtype != C3HIP_F32 && dtype != C3HIP_BF16) return set_error(C3HIP_ERR_INVALID, "unknown dtype");
    if (n < 0) return set_error(C3HIP_ERR_INVALID, "n < 0");
    if (n == 0) return C3HIP_OK;
    if (!w || !g) return set_error(C3HIP_ERR_INVALID, "null pointer");
    unsigned blocks;
    int rc = grid_for(n, 4 * kThreads, &blocks);
    if (rc) return rc;
    void* args[] = {&w, (void*)&g, &lr, &n};
    return launch(dtype == C3HIP_BF16 ? "c3_sgd_bf16" : "c3_sgd_f32", dim3(blocks), dim3(kThreads), args,
                  (hipStream_t)stream);
}

int c3hip_sgd_update_multi(int dtype, int count, void* const* w, const float* const* g, const int64_t* n, float lr,
                           void* stream) {
    clear_error();
    if (dtype != C3HIP_F32 && dtype != C3HIP_BF16) return set_error(C3HIP_ERR_INVALID, "unknown dtype");
    if (count < 0 || count > C3HIP_SGD_MAX_TENSORS)
        return set_error(C3HIP_ERR_INVALID, "count must be in 0.." + std::to_string(C3HIP_SGD_MAX_TENSORS));
    if (count == 0) return C3HIP_OK;
    if (!w || !g || !n) return set_error(C3HIP_ERR_INVALID, "null array");
    SgdMultiArgs a{};
    int64_t blocks = 0;
    int k = 0;
    for (int t = 0; t < count; ++t) {
        if (n[t] < 0) return set_error(C3HIP_ERR_INVALID, "n < 0");
        if (n[t] == 0) continue;
        if (!w[t] || !g[t]) return set_error(C3HIP_ERR_INVALID, "null pointer");
        a.w[k] = w[t];
        a.g[k] = g[t];
        a.n[k] = n[t];
        a.first[k] = blocks;
        blocks += (n[t] + 4 * kThreads - 1) / (4 * kThreads);
        ++k;
    }
    if (k == 0) return C3HIP_OK;
    if (blocks > 0x7fffffff) return set_error(C3HIP_ERR_TOO_LARGE, "sgd grid too large");
    a.first[k] = blocks;
    a.count = k;
    a.lr = lr;
    void* args[] = {&a};
    return launch(dtype == C3HIP_BF16 ? "c3_sgd_multi_bf16" : "c3_sgd_multi_f32", dim3((unsigned)blocks),
                  dim3(kThreads), args, (hipStream_t)stream);
}

}  // extern "C"
