// loss.hip -- softmax cross-entropy over the rows of a logits matrix, and its
// gradient, for the train step that follows the fused layers.
//
// The reference leaves this step to the host framework's CE op (op code 79,
// src/C3/RollingHash.cpp:66); it is here so a whole train step stays on the
// GPU.  For row i with label y:  m = max_j x_j,  s = sum_j exp(x_j - m),
//   loss_i = m + log(s) - x_y,   dx_j = (exp(x_j - m) / s - [j == y]) / M.
// One wave per row; each lane holds up to kMaxPerLane columns in registers,
// so C <= 64 * kMaxPerLane.  Reductions are butterfly shuffles (every lane
// ends with the same value, so the result does not depend on lane order).
// exp/log are the device library's expf/logf.  A label outside [0, C) makes
// that row's loss and gradient NaN (nothing is read out of bounds).
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxPerLane = 32;  // C <= 2048

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float load_logit(const void* p, int64_t i, bool bf16) {
    if (bf16) return __uint_as_float(((uint32_t)((const unsigned short*)p)[i]) << 16);
    return ((const float*)p)[i];
}

__device__ __forceinline__ unsigned short to_bf16(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (unsigned short)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (unsigned short)(u >> 16);
}

template <bool BF16>
__device__ __forceinline__ void softmax_ce_body(const void* __restrict__ logits, const int32_t* __restrict__ labels,
                                                float* __restrict__ loss_rows, void* __restrict__ dlogits, int64_t M,
                                                int64_t C) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (row >= M) return;
    const int64_t base = row * C;
    float x[kMaxPerLane];
    float mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < kMaxPerLane; ++q) {
        const int64_t j = lane + 64 * q;
        x[q] = j < C ? load_logit(logits, base + j, BF16) : -INFINITY;
        mx = fmaxf(mx, x[q]);
    }
    mx = wave_max(mx);
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < kMaxPerLane; ++q) {
        const int64_t j = lane + 64 * q;
        x[q] = j < C ? expf(x[q] - mx) : 0.0f;  // x now holds exp(x - m)
        s += x[q];
    }
    s = wave_sum(s);
    const int32_t y = labels[row];
    const bool y_ok = y >= 0 && (int64_t)y < C;
    const float xy = y_ok ? load_logit(logits, base + y, BF16) : __builtin_nanf("");
    if (lane == 0 && loss_rows) loss_rows[row] = (mx + logf(s)) - xy;
    if (dlogits) {
        const float inv_s = 1.0f / s, inv_m = 1.0f / (float)M;
#pragma unroll
        for (int q = 0; q < kMaxPerLane; ++q) {
            const int64_t j = lane + 64 * q;
            if (j < C) {
                float g = (x[q] * inv_s - (j == y ? 1.0f : 0.0f)) * inv_m;
                if (!y_ok) g = __builtin_nanf("");
                if (BF16)
                    ((unsigned short*)dlogits)[base + j] = to_bf16(g);
                else
                    ((float*)dlogits)[base + j] = g;
            }
        }
    }
}

extern "C" __global__ __launch_bounds__(kThreads) void c3_softmax_ce_f32(const void* logits, const int32_t* labels,
                                                                       float* loss_rows, void* dlogits, int64_t M,
                                                                       int64_t C) {
    softmax_ce_body<false>(logits, labels, loss_rows, dlogits, M, C);
}

extern "C" __global__ __launch_bounds__(kThreads) void c3_softmax_ce_bf16(const void* logits, const int32_t* labels,
                                                                        float* loss_rows, void* dlogits, int64_t M,
                                                                        int64_t C) {
    softmax_ce_body<true>(logits, labels, loss_rows, dlogits, M, C);
}

// fp32 -> bf16 (round to nearest even, NaN kept quiet), 4 elements per thread.
extern "C" __global__ __launch_bounds__(kThreads) void c3_cast_f32_bf16(const float* __restrict__ in,
                                                                      unsigned short* __restrict__ out, int64_t n) {
    const int64_t i = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (i + e < n) out[i + e] = to_bf16(in[i + e]);
}

// bf16 -> fp32 (exact).
extern "C" __global__ __launch_bounds__(kThreads) void c3_cast_bf16_f32(const unsigned short* __restrict__ in,
                                                                      float* __restrict__ out, int64_t n) {
    const int64_t i = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (i + e < n) out[i + e] = __uint_as_float(((uint32_t)in[i + e]) << 16);
}

// Plain SGD step on a parameter: w = w - lr * g, g fp32.  The product is
// rounded before the subtraction (no fused multiply-add), so the result is
// the same on any IEEE machine.  bf16 parameters are widened, updated in
// fp32 and rounded back to nearest-even.
template <bool BF16>
__device__ __forceinline__ void sgd_body(void* __restrict__ w, const float* __restrict__ g, float lr, int64_t n,
                                         int64_t block) {
#pragma clang fp contract(off)
    const int64_t i0 = (block * kThreads + threadIdx.x) * 4;
    // Four elements per thread: one 16-byte gradient load and one 8-byte
    // (bf16) or 16-byte (fp32) weight load and store when aligned and whole.
    const bool vec = i0 + 4 <= n && ((uintptr_t)g & 15) == 0 && ((uintptr_t)w & (BF16 ? 7 : 15)) == 0;
    if (vec) {
        const f32x4 gv = *(const f32x4*)(g + i0);
        if (BF16) {
            unsigned short* p = (unsigned short*)w + i0;
            const uint2 wv = *(const uint2*)p;
            const uint32_t h[4] = {wv.x & 0xffffu, wv.x >> 16, wv.y & 0xffffu, wv.y >> 16};
            uint32_t o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float step = lr * gv[e];
                o[e] = to_bf16(__uint_as_float(h[e] << 16) - step);
            }
            *(uint2*)p = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
        } else {
            f32x4* p = (f32x4*)((float*)w + i0);
            f32x4 wv = *p;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float step = lr * gv[e];
                wv[e] = wv[e] - step;
            }
            *p = wv;
        }
        return;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int64_t i = i0 + e;
        if (i < n) {
            const float step = lr * g[i];
            if (BF16) {
                unsigned short* p = (unsigned short*)w;
                p[i] = to_bf16(__uint_as_float(((uint32_t)p[i]) << 16) - step);
            } else {
                float* p = (float*)w;
                p[i] = p[i] - step;
            }
        }
    }
}

extern "C" __global__ __launch_bounds__(kThreads) void c3_sgd_f32(void* w, const float* g, float lr, int64_t n) {
    sgd_body<false>(w, g, lr, n, blockIdx.x);
}

extern "C" __global__ __launch_bounds__(kThreads) void c3_sgd_bf16(void* w, const float* g, float lr, int64_t n) {
    sgd_body<true>(w, g, lr, n, blockIdx.x);
}

// The same step on up to kSgdMaxTensors parameters in one launch: tensor t
// owns blocks first[t] .. first[t + 1] - 1 (a uniform scan per block).
constexpr int kSgdMaxTensors = 16;
struct SgdMultiArgs {
    void* w[kSgdMaxTensors];
    const float* g[kSgdMaxTensors];
    int64_t n[kSgdMaxTensors];
    int64_t first[kSgdMaxTensors + 1];
    int count;
    float lr;
};

template <bool BF16>
__device__ __forceinline__ void sgd_multi_body(const SgdMultiArgs& a) {
    const int64_t b = blockIdx.x;
    int t = 0;
    while (t + 1 < a.count && b >= a.first[t + 1]) ++t;
    sgd_body<BF16>(a.w[t], a.g[t], a.lr, a.n[t], b - a.first[t]);
}

extern "C" __global__ __launch_bounds__(kThreads) void c3_sgd_multi_f32(SgdMultiArgs a) { sgd_multi_body<false>(a); }
extern "C" __global__ __launch_bounds__(kThreads) void c3_sgd_multi_bf16(SgdMultiArgs a) { sgd_multi_body<true>(a); }
