// elementwise.hip -- the eight single-node elementwise ops as HBM streams.
//
// Reference ops (fp32, one IEEE operation per element):
//   add/sub/mul/div : BinaryOpLowering, src/C3/C3DialectLowering.cpp:246-291
//                     (bmod > 0: rhs index = idx mod bmod)
//   neg             : UnaryOpLowering<NegOp> (arith.negf), :294-317
//   relu            : ReLUOpLowering, maxnumf(x, 0), :319-350
//   scale           : Mul by a scalar (LinalgElementwiseGen rhs_mod = 1,
//                     src/C3/LinalgElementwiseGen.cpp:168-186)
//   relu_bwd        : Gt(z, 0) then Mul(mask, grad),
//                     src/C3/C3BackwardCapture.cpp:501-528 + src/C3/MLIRKernelGen.cpp:173-211
//   sigmoid         : 1 / (1 + exp(-x)), SigmoidOpLowering, src/C3/C3DialectLowering.cpp:352-380
//   tanh, exp, log  : math.tanh / math.exp / math.log, UnaryOpLowering :321-323
//   sigmoid_bwd     : s = 1/(1+exp(-x)); grad * (s * (1 - s)), src/C3/C3BackwardCapture.cpp:530-567
//   tanh_bwd        : t = (e^x - e^-x) / (e^x + e^-x); grad * (1 - t*t), :569-616 (the
//                     reference recomputes tanh through exp here, so |x| > ~88.7 gives
//                     inf/inf = NaN; kept)
//   exp_bwd         : exp(x) * grad, :823-849
//   div_bwd_b (3-in): -((a / (b*b)) * grad), buildDivBackwardGraph
// exp, log and tanh are the device library's expf, logf, tanhf.
//
// Layout: flat contiguous fp32 arrays.  Fast path: one 16-byte vector per
// operand per thread and one wave (64 threads) per block, non-temporal hints
// on loads and stores (the data is touched once).  Measured on MI355X,
// variants timed alternately in one process on random data: add at 2^28,
// 64-thread blocks 6.62 TB/s, 128 6.43-6.49, 256 5.99; scale at 2^24 with
// rotating operand sets 6.19 against 5.84 (128 and 256) and 5.94 (512); two
// or four vectors per thread, grid-stride loops and plain (cached) loads
// were all slower.  The host picks the scalar kernel when n or a base
// address is not 16-byte friendly.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f32x4 __attribute__((ext_vector_type(4)));

enum {
    EW_ADD = 0, EW_SUB = 1, EW_MUL = 2, EW_DIV = 3, EW_RELU = 4, EW_RELU_BWD = 5, EW_NEG = 6, EW_SCALE = 7,
    EW_SIGMOID = 8, EW_TANH = 9, EW_EXP = 10, EW_LOG = 11, EW_SIGMOID_BWD = 12, EW_TANH_BWD = 13, EW_EXP_BWD = 14
};

// Each step below is one IEEE operation of the reference's graph, rounded to
// fp32 in the same order (no multiply-add contraction: see the pragma).
template <int OP>
__device__ __forceinline__ float ew_apply(float a, float b, float alpha) {
#pragma clang fp contract(off)
    if (OP == EW_ADD) return a + b;
    if (OP == EW_SUB) return a - b;
    if (OP == EW_MUL) return a * b;
    if (OP == EW_DIV) return a / b;              // IEEE correctly rounded division
    if (OP == EW_RELU) return fmaxf(a, 0.0f);    // maxnum: NaN -> 0
    if (OP == EW_RELU_BWD) return (a > 0.0f ? 1.0f : 0.0f) * b;
    if (OP == EW_NEG) return -a;
    if (OP == EW_SIGMOID) return 1.0f / (1.0f + expf(-a));
    if (OP == EW_TANH) return tanhf(a);
    if (OP == EW_EXP) return expf(a);
    if (OP == EW_LOG) return logf(a);
    if (OP == EW_SIGMOID_BWD) {
        const float s = 1.0f / (1.0f + expf(-a));
        const float t = s * (1.0f - s);
        return b * t;
    }
    if (OP == EW_TANH_BWD) {
        const float e = expf(a), en = expf(-a);
        const float t = (e - en) / (e + en);
        const float sq = t * t;
        return b * (1.0f - sq);
    }
    if (OP == EW_EXP_BWD) return expf(a) * b;
    return a * alpha;                            // EW_SCALE
}

template <int OP>
constexpr bool ew_binary() {
    return OP == EW_ADD || OP == EW_SUB || OP == EW_MUL || OP == EW_DIV || OP == EW_RELU_BWD ||
           OP == EW_SIGMOID_BWD || OP == EW_TANH_BWD || OP == EW_EXP_BWD;
}

constexpr int kThreads = 256;     // scalar (grid-stride) kernels
constexpr int kVecThreads = 64;   // vector kernels: one float4 per thread (must match the host grid)
constexpr int kUnroll = 1;        // vectors per thread (must match the host grid)

__device__ __forceinline__ f32x4 ld_nt(const f32x4* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st_nt(f32x4 v, f32x4* p) { __builtin_nontemporal_store(v, p); }

// Vector kernel: n4 = number of float4 vectors; bmod4 = bmod / 4 (0 = no broadcast).
template <int OP>
__device__ __forceinline__ void ew_vec_body(const f32x4* __restrict__ a, const f32x4* __restrict__ b,
                                            float alpha, f32x4* __restrict__ out, int64_t n4, int64_t bmod4) {
    const int64_t base = (int64_t)blockIdx.x * (kVecThreads * kUnroll) + threadIdx.x;
    f32x4 va[kUnroll], vb[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t i = base + (int64_t)u * kVecThreads;
        if (i < n4) {
            va[u] = ld_nt(a + i);
            if (ew_binary<OP>()) vb[u] = bmod4 > 0 ? b[i % bmod4] : ld_nt(b + i);
        }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t i = base + (int64_t)u * kVecThreads;
        if (i < n4) {
            f32x4 r;
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = ew_apply<OP>(va[u][e], ew_binary<OP>() ? vb[u][e] : 0.0f, alpha);
            st_nt(r, out + i);
        }
    }
}

// Scalar kernel: any n, any alignment, bmod > 0 broadcasts rhs, bmod < 0 broadcasts lhs.
template <int OP>
__device__ __forceinline__ void ew_scalar_body(const float* __restrict__ a, const float* __restrict__ b,
                                               float alpha, float* __restrict__ out, int64_t n, int64_t bmod) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        int64_t li = i, ri = i;
        if (bmod > 0) ri = i % bmod;
        else if (bmod < 0) li = i % (-bmod);
        const float x = a[li];
        const float y = ew_binary<OP>() ? b[ri] : 0.0f;
        out[i] = ew_apply<OP>(x, y, alpha);
    }
}

#define C3_EW(NAME, OP)                                                                                  \
    extern "C" __global__ __launch_bounds__(kVecThreads) void c3_ew_##NAME##_f32_v(                    \
        const f32x4* a, const f32x4* b, float alpha, f32x4* out, int64_t n4, int64_t bmod4) {          \
        ew_vec_body<OP>(a, b, alpha, out, n4, bmod4);                                                   \
    }                                                                                                   \
    extern "C" __global__ __launch_bounds__(kThreads) void c3_ew_##NAME##_f32_s(                       \
        const float* a, const float* b, float alpha, float* out, int64_t n, int64_t bmod) {            \
        ew_scalar_body<OP>(a, b, alpha, out, n, bmod);                                                  \
    }

C3_EW(add, EW_ADD)
C3_EW(sub, EW_SUB)
C3_EW(mul, EW_MUL)
C3_EW(div, EW_DIV)
C3_EW(relu, EW_RELU)
C3_EW(relu_bwd, EW_RELU_BWD)
C3_EW(neg, EW_NEG)
C3_EW(scale, EW_SCALE)
C3_EW(sigmoid, EW_SIGMOID)
C3_EW(tanh, EW_TANH)
C3_EW(exp, EW_EXP)
C3_EW(log, EW_LOG)
C3_EW(sigmoid_bwd, EW_SIGMOID_BWD)
C3_EW(tanh_bwd, EW_TANH_BWD)
C3_EW(exp_bwd, EW_EXP_BWD)

// ---- fused backward chain of single-input nodes ----------------------------
// g_0 = grad; node k (k = 0 most downstream) maps g_k to g_{k+1} with its
// per-node rule from its forward input x_k, and out_k = g_{k+1} is stored (the
// upstream grad of every node, as the reference's multi-output fused graph
// returns them: src/C3/C3BackwardCapture.cpp:1140-1210).  Each rule is the
// same ew_apply step as the single-node kernel, so the chain is bit-identical
// to running the nodes one by one; only the intermediate re-reads go away.
enum { CH_RELU = 0, CH_SIGMOID = 1, CH_TANH = 2, CH_EXP = 3, CH_LOG = 4, CH_NEG = 5 };
constexpr int kChainMax = 4;

struct ChainArgs {
    const float* g;
    const float* x[kChainMax];  // x[k] unused (may be null) for a Neg node
    float* out[kChainMax];      // null: g_{k+1} is not stored
    int node[kChainMax];
    int w;
    int64_t n;                  // elements (vector kernel: the count of float4)
};

__device__ __forceinline__ float chain_step(int node, float g, float x) {
    switch (node) {
        case CH_RELU: return ew_apply<EW_RELU_BWD>(x, g, 0.0f);
        case CH_SIGMOID: return ew_apply<EW_SIGMOID_BWD>(x, g, 0.0f);
        case CH_TANH: return ew_apply<EW_TANH_BWD>(x, g, 0.0f);
        case CH_EXP: return ew_apply<EW_EXP_BWD>(x, g, 0.0f);
        case CH_LOG: return ew_apply<EW_DIV>(g, x, 0.0f);
        default: return ew_apply<EW_NEG>(g, 0.0f, 0.0f);
    }
}

// One float4 per thread.  Every load of the element is issued before the
// first store, so an output may alias an input at the same offsets.
extern "C" __global__ __launch_bounds__(kVecThreads) void c3_bwd_chain_f32_v(ChainArgs p) {
    const int64_t i = (int64_t)blockIdx.x * kVecThreads + threadIdx.x;
    if (i >= p.n) return;
    f32x4 g = ld_nt((const f32x4*)p.g + i);
    f32x4 x[kChainMax];
#pragma unroll
    for (int k = 0; k < kChainMax; ++k)
        if (k < p.w && p.node[k] != CH_NEG) x[k] = ld_nt((const f32x4*)p.x[k] + i);
#pragma unroll
    for (int k = 0; k < kChainMax; ++k) {
        if (k < p.w) {
            const int node = p.node[k];
#pragma unroll
            for (int e = 0; e < 4; ++e) g[e] = chain_step(node, g[e], node == CH_NEG ? 0.0f : x[k][e]);
            if (p.out[k]) st_nt(g, (f32x4*)p.out[k] + i);
        }
    }
}

// Any n and alignment: grid-stride over elements.
extern "C" __global__ __launch_bounds__(kThreads) void c3_bwd_chain_f32_s(ChainArgs p) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < p.n; i += stride) {
        float g = p.g[i];
        float x[kChainMax];
#pragma unroll
        for (int k = 0; k < kChainMax; ++k) x[k] = (k < p.w && p.node[k] != CH_NEG) ? p.x[k][i] : 0.0f;
#pragma unroll
        for (int k = 0; k < kChainMax; ++k) {
            if (k < p.w) {
                g = chain_step(p.node[k], g, x[k]);
                if (p.out[k]) p.out[k][i] = g;
            }
        }
    }
}

// Three-input ops: out = op(a, b, c), no broadcast, any n and alignment.
extern "C" __global__ __launch_bounds__(kThreads) void c3_ew3_div_bwd_b_f32(const float* __restrict__ a,
                                                                          const float* __restrict__ b,
                                                                          const float* __restrict__ c,
                                                                          float* __restrict__ out, int64_t n) {
#pragma clang fp contract(off)
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        const float bb = b[i] * b[i];
        const float q = a[i] / bb;
        const float m = q * c[i];
        out[i] = -m;
    }
}
