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
// axis 0 is two passes.  Pass 1 (c3_colsum_partial_f32 and the backward
// pre-passes) writes one partial row per chunk of rows into a workspace
// [nchunks, N]; pass 2 (c3_colsum_final_f32) adds the partials.  A pass-1
// block is `vb` column units (a column, or 8 columns for bf16) by 256 / vb
// row lanes: a narrow matrix still gives every block 256 busy threads.  Row
// lane r of a chunk sums rows r, r + 256/vb, ... in order; the lanes are then
// added in lane order through LDS, so each partial has one fixed order.
// Consecutive threads read consecutive column units of a row (contiguous
// bytes per wave).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemm_common.h"

constexpr int kThreads = 256;

// mask (nullable, same layout as in): sums (mask > 0 ? 1 : 0) * in, the bias
// gradient of a ReLU layer computed from its forward output Y and dY.
// Grid: (ceil(N / vb), nchunks); block 256 = vb columns x (256 / vb) row lanes.
extern "C" __global__ __launch_bounds__(kThreads) void c3_colsum_partial_f32(
    const float* __restrict__ in, const float* __restrict__ mask, float* __restrict__ part, int64_t M, int64_t N,
    int64_t rows_per_chunk, int vb) {
    __shared__ float red[kThreads];
    const int rb = kThreads / vb;
    const int u = threadIdx.x % vb, rl = threadIdx.x / vb;
    const int64_t j = (int64_t)blockIdx.x * vb + u;
    const int64_t chunk = blockIdx.y;
    const int64_t r0 = chunk * rows_per_chunk;
    const int64_t r1 = min(M, r0 + rows_per_chunk);
    float s = 0.0f;
    if (j < N) {
        for (int64_t i = r0 + rl; i < r1; i += rb) {
            const int64_t o = i * N + j;
            s += mask ? (mask[o] > 0.0f ? 1.0f : 0.0f) * in[o] : in[o];
        }
    }
    if (rb > 1) {
        red[threadIdx.x] = s;
        __syncthreads();
        if (rl == 0)
            for (int k = 1; k < rb; ++k) s += red[threadIdx.x + k * vb];
    }
    if (rl == 0 && j < N) part[chunk * N + j] = s;
}

// Pass 2: out[j] = sum over chunks of part[c][j].  Block: 64 columns x 8
// waves; wave w adds chunks w, w + 8, ... into four interleaved sums, and the
// eight wave sums are added in wave order (colsum_final_block, which the bf16
// layer-backward launch also runs).  Grid: ceil(N / 64).
extern "C" __global__ __launch_bounds__(512) void c3_colsum_final_f32(
    const float* __restrict__ part, float* __restrict__ out, int64_t nchunks, int64_t N) {
    __shared__ float red[8][64];
    colsum_final_block<8>(part, out, nchunks, N, blockIdx.x, red);
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

// fp32: one column per thread, block = vb columns x (256 / vb) row lanes,
// grid (ceil(N / vb), nchunks).
extern "C" __global__ __launch_bounds__(kThreads) void c3_dz_colsum_f32(
    const float* __restrict__ Y, const float* __restrict__ dY, float* __restrict__ dZ, float* __restrict__ part,
    int64_t M, int64_t N, int64_t rows_per_chunk, int act, int vb) {
    __shared__ float red[kThreads];
    const int rb = kThreads / vb;
    const int u = threadIdx.x % vb, rl = threadIdx.x / vb;
    const int64_t n = (int64_t)blockIdx.x * vb + u;
    const int64_t chunk = blockIdx.y;
    const int64_t r0 = chunk * rows_per_chunk;
    const int64_t r1 = min(M, r0 + rows_per_chunk);
    float s = 0.0f;
    if (n < N) {
        for (int64_t i = r0 + rl; i < r1; i += rb) {
            const int64_t off = i * N + n;
            const float d = act_grad(act ? Y[off] : 0.0f, dY[off], act);
            if (dZ) dZ[off] = d;
            s += d;
        }
    }
    if (part) {
        if (rb > 1) {
            red[threadIdx.x] = s;
            __syncthreads();
            if (rl == 0)
                for (int k = 1; k < rb; ++k) s += red[threadIdx.x + k * vb];
        }
        if (rl == 0 && n < N) part[chunk * N + n] = s;
    }
}

// fp32, vectorised: one thread owns 4 consecutive columns (a 16-byte vector);
// block = vb vectors x (256 / vb) row lanes, grid (ceil(N / 4 / vb), nchunks).
// Each column's rows are summed in the same order as in c3_dz_colsum_f32 run
// on the same row geometry.  Requires N % 4 == 0 and 16-byte aligned rows.
extern "C" __global__ __launch_bounds__(kThreads) void c3_dz_colsum_f32_v(
    const float* __restrict__ Y, const float* __restrict__ dY, float* __restrict__ dZ, float* __restrict__ part,
    int64_t M, int64_t N, int64_t rows_per_chunk, int act, int vb) {
    __shared__ float red[kThreads][5];
    const int rb = kThreads / vb;
    const int u = threadIdx.x % vb, rl = threadIdx.x / vb;
    const int64_t v = (int64_t)blockIdx.x * vb + u;  // vector index within a row
    const bool active = 4 * v < N;
    const int64_t chunk = blockIdx.y;
    const int64_t r0 = chunk * rows_per_chunk;
    const int64_t r1 = min(M, r0 + rows_per_chunk);
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    auto grad = [&](f32x4 y, f32x4 d) {
        return f32x4{act_grad(y[0], d[0], act), act_grad(y[1], d[1], act), act_grad(y[2], d[2], act),
                     act_grad(y[3], d[3], act)};
    };
    if (active) {
        // Four rows per iteration, their loads issued before the first use;
        // rows are still summed in row order.
        const bool need_y = act != 0;
        int64_t i = r0 + rl;
        for (; i + 3 * rb < r1; i += 4 * rb) {
            f32x4 d[4], y[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t off = (i + q * rb) * N + 4 * v;
                d[q] = __builtin_nontemporal_load((const f32x4*)(dY + off));
                y[q] = need_y ? __builtin_nontemporal_load((const f32x4*)(Y + off)) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t off = (i + q * rb) * N + 4 * v;
                const f32x4 g = grad(y[q], d[q]);
                if (dZ) *(f32x4*)(dZ + off) = g;
                if (part) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) s[e] += g[e];
                }
            }
        }
        for (; i < r1; i += rb) {
            const int64_t off = i * N + 4 * v;
            const f32x4 d = __builtin_nontemporal_load((const f32x4*)(dY + off));
            const f32x4 y = need_y ? __builtin_nontemporal_load((const f32x4*)(Y + off)) : f32x4{0.f, 0.f, 0.f, 0.f};
            const f32x4 g = grad(y, d);
            if (dZ) *(f32x4*)(dZ + off) = g;
            if (part) {
#pragma unroll
                for (int e = 0; e < 4; ++e) s[e] += g[e];
            }
        }
    }
    if (part) {
        if (rb > 1) {
#pragma unroll
            for (int e = 0; e < 4; ++e) red[threadIdx.x][e] = s[e];
            __syncthreads();
            if (rl == 0)
                for (int k = 1; k < rb; ++k)
#pragma unroll
                    for (int e = 0; e < 4; ++e) s[e] += red[threadIdx.x + k * vb][e];
        }
        if (rl == 0 && active) {
#pragma unroll
            for (int e = 0; e < 4; ++e) part[chunk * N + 4 * v + e] = s[e];
        }
    }
}

// bf16: one thread owns 8 consecutive columns (a 16-byte vector); block = vb
// vectors x (256 / vb) row lanes, grid (ceil(N / 8 / vb), nchunks).  ReLU
// works on the bit patterns (exact); sigmoid and tanh compute in fp32 and
// round dZ to bf16 once (nearest even); the column sums add the rounded
// values the GEMMs then read.  Requires N % 8 == 0 and 16-byte aligned rows.
extern "C" __global__ __launch_bounds__(kThreads) void c3_dz_colsum_bf16(
    const unsigned short* __restrict__ Y, const unsigned short* __restrict__ dY, unsigned short* __restrict__ dZ,
    float* __restrict__ part, int64_t M, int64_t N, int64_t rows_per_chunk, int act, int vb) {
    __shared__ float red[kThreads][9];
    const int rb = kThreads / vb;
    const int u = threadIdx.x % vb, rl = threadIdx.x / vb;
    const int64_t v = (int64_t)blockIdx.x * vb + u;  // vector index within a row
    const bool active = 8 * v < N;
    const int64_t chunk = blockIdx.y;
    const int64_t r0 = chunk * rows_per_chunk;
    const int64_t r1 = min(M, r0 + rows_per_chunk);
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    // dZ of one 16-byte vector from its Y and dY vectors.
    auto grad = [&](u32x4 y, u32x4 d) {
        if (act == 1) return mask_mul8(y, d);
        if (act == 2 || act == 3) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float lo = act_grad(bf16_to_f32((unsigned short)(y[e] & 0xffff)),
                                          bf16_to_f32((unsigned short)(d[e] & 0xffff)), act);
                const float hi = act_grad(bf16_to_f32((unsigned short)(y[e] >> 16)),
                                          bf16_to_f32((unsigned short)(d[e] >> 16)), act);
                d[e] = (uint32_t)f32_to_bf16_rne(lo) | ((uint32_t)f32_to_bf16_rne(hi) << 16);
            }
        }
        return d;
    };
    auto sum = [&](u32x4 d) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            s[2 * e] += __uint_as_float(d[e] << 16);
            s[2 * e + 1] += __uint_as_float(d[e] & 0xffff0000u);
        }
    };
    if (active) {
        // Four rows per iteration: their eight loads are issued before the
        // first use (a thread walks 4..64 rows; one row at a time leaves the
        // stream latency-bound).  Rows are still summed in row order.
        const bool need_y = act != 0;
        int64_t i = r0 + rl;
        for (; i + 3 * rb < r1; i += 4 * rb) {
            u32x4 d[4], y[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t off = (i + q * rb) * N + 8 * v;
                d[q] = __builtin_nontemporal_load((const u32x4*)(dY + off));
                y[q] = need_y ? __builtin_nontemporal_load((const u32x4*)(Y + off)) : u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t off = (i + q * rb) * N + 8 * v;
                const u32x4 g = grad(y[q], d[q]);
                if (dZ) *(u32x4*)(dZ + off) = g;
                if (part) sum(g);
            }
        }
        for (; i < r1; i += rb) {
            const int64_t off = i * N + 8 * v;
            const u32x4 d = __builtin_nontemporal_load((const u32x4*)(dY + off));
            const u32x4 y = need_y ? __builtin_nontemporal_load((const u32x4*)(Y + off)) : u32x4{0u, 0u, 0u, 0u};
            const u32x4 g = grad(y, d);
            if (dZ) *(u32x4*)(dZ + off) = g;
            if (part) sum(g);
        }
    }
    if (part) {
        if (rb > 1) {
#pragma unroll
            for (int e = 0; e < 8; ++e) red[threadIdx.x][e] = s[e];
            __syncthreads();
            if (rl == 0)
                for (int k = 1; k < rb; ++k)
#pragma unroll
                    for (int e = 0; e < 8; ++e) s[e] += red[threadIdx.x + k * vb][e];
        }
        if (rl == 0 && active) {
#pragma unroll
            for (int e = 0; e < 8; ++e) part[chunk * N + 8 * v + e] = s[e];
        }
    }
}
