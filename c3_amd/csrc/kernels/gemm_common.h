// gemm_common.h -- shared definitions for the gfx950 GEMM code objects.
//
// Logical problem: C[M,N] = sum_k A(m,k) * B(k,n), fp32 accumulation.
//   A(m,k) lives at A[m*lda + k] when the operand is "k-contiguous" (AK),
//   else at A[k*lda + m].  B(k,n) lives at B[n*ldb + k] when k-contiguous
//   (BKC), else at B[k*ldb + n].
// The three GEMMs of one Linear layer map onto this as
//   forward  Y  = X . W      : A = X  (AK),      B = W (row-major [K,N], !BKC)
//   backward dX = dZ . W^T   : A = dZ (AK),      B = W (BKC: B(k=n, j) = W[j*N+n])
//   backward dW = X^T . dZ   : A = X  (!AK),     B = dZ (!BKC)
// where dZ = (Y > 0 ? 1 : 0) * dY is formed while the tile is loaded
// (mask prologue), never materialised in HBM.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

struct GemmArgs {
    const void* A;      // operand A (fp32 or bf16)
    const void* Amask;  // mask source with A's layout (Y of the forward), or null
    const void* B;
    const void* Bmask;
    void* C;            // output [M, ldc]
    const float* bias;  // per-column bias (fp32), or null
    float* db;          // column sums of the masked B operand over k (fp32), or null
    int64_t M, N, K;
    int64_t lda, ldb, ldc;
    int act;            // 0: none, 1: ReLU (maxnum(x, 0))
    int _pad;
    int64_t split_k;    // split-K: k extent of one split (blockIdx.y = split), 0 = none
    int64_t c_split;    // split-K: elements between the fp32 outputs of consecutive splits
    void* dz;           // dx_mask_dz kinds: the masked A operand (dZ) is also written here (A's layout), or null
};

// Blocks are handed to the 8 XCDs round-robin (block i runs on XCD i % 8).
// Renumber so that consecutive logical tiles land on the same XCD and share
// its L2, then walk tiles in groups of GROUP_M row-tiles so that a group's
// A rows and B columns stay L2-resident.
// bid: the block's index among this GEMM's blocks (blockIdx.x, or less an
// offset when one launch runs the blocks of two GEMMs).
template <int GROUP_M>
__device__ __forceinline__ void tile_coords(int64_t M, int64_t N, int BM, int BN, int& tm, int& tn,
                                            int bid = -1) {
    const int nbm = (int)((M + BM - 1) / BM);
    const int nbn = (int)((N + BN - 1) / BN);
    const int nblk = nbm * nbn;
    if (bid < 0) bid = blockIdx.x;
    int id = bid;
    if ((nblk & 7) == 0) id = (bid & 7) * (nblk >> 3) + (bid >> 3);
    const int per_group = GROUP_M * nbn;
    const int g = id / per_group;
    const int first_m = g * GROUP_M;
    const int gsz = min(nbm - first_m, GROUP_M);
    const int r = id - g * per_group;
    tm = first_m + r % gsz;
    tn = r / gsz;
}

__device__ __forceinline__ float relu_mask(float y) { return y > 0.0f ? 1.0f : 0.0f; }

// act 1: maxnum(x, 0) (NaN -> 0, llvm.maxnum semantics, v_max_f32);
// act 2: 1 / (1 + expf(-x)); act 3: tanhf(x) (device library expf/tanhf).
__device__ __forceinline__ float act_apply(float v, int act) {
    if (act == 1) return fmaxf(v, 0.0f);
    if (act == 2) return 1.0f / (1.0f + expf(-v));
    if (act == 3) return tanhf(v);
    return v;
}

// The same activations with ACT fixed at compile time.  Epilogues dispatch on
// the runtime act once (with_act) and run an element loop compiled for that
// activation alone: a loop calling act_apply per element carries the sigmoid
// and tanh code at every element (tens of KiB of instructions fetched by every
// block even for ReLU).
template <int ACT>
__device__ __forceinline__ float act_c(float v) {
    if (ACT == 1) return fmaxf(v, 0.0f);
    if (ACT == 2) return 1.0f / (1.0f + expf(-v));
    if (ACT == 3) return tanhf(v);
    return v;
}

template <int V>
struct ActTag {
    static constexpr int value = V;
};

template <class F>
__device__ __forceinline__ void with_act(int act, F&& f) {
    switch (act) {
        case 1: f(ActTag<1>{}); break;
        case 2: f(ActTag<2>{}); break;
        case 3: f(ActTag<3>{}); break;
        default: f(ActTag<0>{}); break;
    }
}

__device__ __forceinline__ unsigned short f32_to_bf16_rne(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (unsigned short)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (unsigned short)(u >> 16);
}

__device__ __forceinline__ float bf16_to_f32(unsigned short h) { return __uint_as_float(((uint32_t)h) << 16); }

// ---- bf16 bit-pattern helpers ----
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// bf16 bits: Y > 0 <=> sign clear, nonzero, not NaN (+inf counts as > 0).
__device__ __forceinline__ bool bf16_gt0(unsigned short y) { return (short)y > 0 && y <= 0x7f80u; }

// (Y > 0 ? 1 : 0) * dY on bf16 bit patterns: dY when Y > 0, else a zero with
// dY's sign, or NaN when dY is Inf/NaN (0 * Inf = NaN).
__device__ __forceinline__ unsigned short bf16_mask_mul(unsigned short y, unsigned short d) {
    if (bf16_gt0(y)) return d;
    if ((d & 0x7f80u) == 0x7f80u) return 0x7fc0u;
    return d & 0x8000u;
}

__device__ __forceinline__ uint32_t mask_mul2(uint32_t y, uint32_t d) {
    return (uint32_t)bf16_mask_mul((unsigned short)(y & 0xffff), (unsigned short)(d & 0xffff)) |
           ((uint32_t)bf16_mask_mul((unsigned short)(y >> 16), (unsigned short)(d >> 16)) << 16);
}

__device__ __forceinline__ u32x4 mask_mul8(u32x4 y, u32x4 d) {
    return u32x4{mask_mul2(y[0], d[0]), mask_mul2(y[1], d[1]), mask_mul2(y[2], d[2]), mask_mul2(y[3], d[3])};
}

// ---- column-sum final pass ----
// out[j] = sum over chunks c of part[c * N + j] for the 64 columns
// j = 64 b .. 64 b + 63: virtual wave w (of 8) adds chunks w, w + 8, ...
// into four interleaved sums (chunks c, c + 8, c + 16, c + 24 per step of
// 32), and the eight wave sums are added in wave order.  A block of NW waves
// runs 8 / NW virtual waves per wave, so every NW gives the same bits.
// Eight steps of 32 issue their 32 loads before the first add (the same adds
// in the same order): the loads of one step alone left each wave waiting a
// full memory latency per four loads.
// red: 8 x 64 floats of LDS.
template <int NW>
__device__ __forceinline__ void colsum_final_block(const float* __restrict__ part, float* __restrict__ out,
                                                   int64_t nchunks, int64_t N, int64_t b, float (*red)[64]) {
    static_assert(NW == 1 || NW == 2 || NW == 4 || NW == 8, "8 virtual waves over NW waves");
    const int lane = threadIdx.x & 63, w0 = threadIdx.x >> 6;
    const int64_t j = b * 64 + lane;
#pragma unroll
    for (int v = 0; v < 8 / NW; ++v) {
        const int w = w0 + NW * v;
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
        if (j < N) {
            int64_t c = w;
            for (; c + 248 < nchunks; c += 256) {
                float v[32];
#pragma unroll
                for (int u = 0; u < 32; ++u) v[u] = part[(c + 8 * u) * N + j];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    s0 += v[4 * u];
                    s1 += v[4 * u + 1];
                    s2 += v[4 * u + 2];
                    s3 += v[4 * u + 3];
                }
            }
            for (; c + 24 < nchunks; c += 32) {
                s0 += part[c * N + j];
                s1 += part[(c + 8) * N + j];
                s2 += part[(c + 16) * N + j];
                s3 += part[(c + 24) * N + j];
            }
            for (; c < nchunks; c += 8) s0 += part[c * N + j];
        }
        red[w][lane] = (s0 + s1) + (s2 + s3);
    }
    __syncthreads();
    if (w0 == 0 && j < N) {
        float t = red[0][lane];
#pragma unroll
        for (int k = 1; k < 8; ++k) t += red[k][lane];
        out[j] = t;
    }
}
