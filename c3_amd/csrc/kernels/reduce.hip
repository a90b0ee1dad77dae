// reduce.hip -- SumReduce of a row-major [M, N] fp32 matrix.
//
// Reference: SumReduceOpLowering, src/C3/C3DialectLowering.cpp:382-465.
//   axis 0: out[j] = sum_i in[i*N + j]   (the bias gradient db, Add backward
//           input 1, src/C3/C3BackwardCapture.cpp:618-644, axis from :1641-1700)
//   axis 1: out[i] = sum_j in[i*N + j]
// The reference sums sequentially from 0.0f; here the sum is split into row
// chunks (axis 0) or lane strides (axis 1) and combined in a fixed order, so
// the result is deterministic run to run and within fp32 rounding of the
// sequential sum.
//
// axis 0 is two passes: pass 1 writes one partial row per chunk of rows into
// a workspace [nchunks, N]; pass 2 adds the partials in chunk order.  Each
// thread owns one column, so every row access of a wave is 256 contiguous
// bytes.
#include <hip/hip_runtime.h>
#include <stdint.h>

constexpr int kThreads = 256;

// mask (nullable, same layout as in): sums (mask > 0 ? 1 : 0) * in, the bias
// gradient of a ReLU layer computed from its forward output Y and dY.
extern "C" __global__ __launch_bounds__(kThreads) void c3_colsum_partial_f32(
    const float* __restrict__ in, const float* __restrict__ mask, float* __restrict__ part, int64_t M, int64_t N,
    int64_t rows_per_chunk) {
    const int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t chunk = blockIdx.y;
    if (j >= N) return;
    const int64_t r0 = chunk * rows_per_chunk;
    const int64_t r1 = min(M, r0 + rows_per_chunk);
    // Four independent partial sums for memory-level parallelism, combined in
    // a fixed order.
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int64_t i = r0;
    if (mask) {
        for (; i + 4 <= r1; i += 4)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t o = (i + q) * N + j;
                s[q] += (mask[o] > 0.0f ? 1.0f : 0.0f) * in[o];
            }
        for (; i < r1; ++i) s[0] += (mask[i * N + j] > 0.0f ? 1.0f : 0.0f) * in[i * N + j];
    } else {
        for (; i + 4 <= r1; i += 4)
#pragma unroll
            for (int q = 0; q < 4; ++q) s[q] += in[(i + q) * N + j];
        for (; i < r1; ++i) s[0] += in[i * N + j];
    }
    part[chunk * N + j] = (s[0] + s[1]) + (s[2] + s[3]);
}

extern "C" __global__ __launch_bounds__(kThreads) void c3_colsum_final_f32(
    const float* __restrict__ part, float* __restrict__ out, int64_t nchunks, int64_t N) {
    const int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (j >= N) return;
    float s = 0.0f;
    for (int64_t c = 0; c < nchunks; ++c) s += part[c * N + j];
    out[j] = s;
}

// One wave per row.
extern "C" __global__ __launch_bounds__(kThreads) void c3_rowsum_f32(
    const float* __restrict__ in, float* __restrict__ out, int64_t M, int64_t N) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (row >= M) return;
    const float* p = in + row * N;
    float s = 0.0f;
    for (int64_t j = lane; j < N; j += 64) s += p[j];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) out[row] = s;
}

// ---- backward pre-passes ---------------------------------------------------
// dZ = act'(Y) * dY, the gradient at the pre-activation, from the layer's
// output Y (act 1: (Y > 0 ? 1 : 0) * dY; act 2: dY * (Y * (1 - Y)); act 3:
// dY * (1 - Y * Y); act 0: dY), written to dZ when non-null, and per-chunk
// column sums of dZ in fp32 into part [nchunks, N] when non-null (the bias
// gradient, finished by c3_colsum_final_f32).  Each step is one IEEE
// operation in the order written (no multiply-add contraction).
#include "gemm_common.h"

__device__ __forceinline__ float act_grad(float y, float d, int act) {
#pragma clang fp contract(off)
    if (act == 1) return (y > 0.0f ? 1.0f : 0.0f) * d;
    if (act == 2) {
        const float t = y * (1.0f - y);
        return d * t;
    }
    if (act == 3) {
        const float sq = y * y;
        return d * (1.0f - sq);
    }
    return d;
}

// fp32: one thread per column of a chunk of rows (consecutive threads read
// consecutive columns of a row).
extern "C" __global__ __launch_bounds__(kThreads) void c3_dz_colsum_f32(
    const float* __restrict__ Y, const float* __restrict__ dY, float* __restrict__ dZ, float* __restrict__ part,
    int64_t M, int64_t N, int64_t rows_per_chunk, int act) {
    const int64_t n = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (n >= N) return;
    const int64_t chunk = blockIdx.y;
    const int64_t r0 = chunk * rows_per_chunk;
    const int64_t r1 = min(M, r0 + rows_per_chunk);
    float s = 0.0f;
    for (int64_t i = r0; i < r1; ++i) {
        const int64_t off = i * N + n;
        const float d = act_grad(act ? Y[off] : 0.0f, dY[off], act);
        if (dZ) dZ[off] = d;
        s += d;
    }
    if (part) part[chunk * N + n] = s;
}

// bf16: one thread owns 8 consecutive columns (a 16-byte vector) of a chunk
// of rows; consecutive threads cover consecutive vectors of a row.  ReLU
// works on the bit patterns (exact); sigmoid and tanh compute in fp32 and
// round dZ to bf16 once (nearest even); the column sums add the rounded
// values the GEMMs then read.  Requires N % 8 == 0 and 16-byte aligned rows.
extern "C" __global__ __launch_bounds__(kThreads) void c3_dz_colsum_bf16(
    const unsigned short* __restrict__ Y, const unsigned short* __restrict__ dY, unsigned short* __restrict__ dZ,
    float* __restrict__ part, int64_t M, int64_t N, int64_t rows_per_chunk, int act) {
    const int64_t v = (int64_t)blockIdx.x * kThreads + threadIdx.x;  // vector index within a row
    if (8 * v >= N) return;
    const int64_t chunk = blockIdx.y;
    const int64_t r0 = chunk * rows_per_chunk;
    const int64_t r1 = min(M, r0 + rows_per_chunk);
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int64_t i = r0; i < r1; ++i) {
        const int64_t off = i * N + 8 * v;
        u32x4 d = *(const u32x4*)(dY + off);
        if (act == 1) {
            d = mask_mul8(*(const u32x4*)(Y + off), d);
        } else if (act == 2 || act == 3) {
            const u32x4 y = *(const u32x4*)(Y + off);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float lo = act_grad(bf16_to_f32((unsigned short)(y[e] & 0xffff)),
                                          bf16_to_f32((unsigned short)(d[e] & 0xffff)), act);
                const float hi = act_grad(bf16_to_f32((unsigned short)(y[e] >> 16)),
                                          bf16_to_f32((unsigned short)(d[e] >> 16)), act);
                d[e] = (uint32_t)f32_to_bf16_rne(lo) | ((uint32_t)f32_to_bf16_rne(hi) << 16);
            }
        }
        if (dZ) *(u32x4*)(dZ + off) = d;
        if (part) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s[2 * e] += __uint_as_float(d[e] << 16);
                s[2 * e + 1] += __uint_as_float(d[e] & 0xffff0000u);
            }
        }
    }
    if (part) {
#pragma unroll
        for (int e = 0; e < 8; ++e) part[chunk * N + 8 * v + e] = s[e];
    }
}
