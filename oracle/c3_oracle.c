/*
 * c3_oracle.c -- CPU restatement of the reference's arithmetic for the fused
 * Linear+bias+ReLU hot path.  TEST INFRASTRUCTURE ONLY (see c3_oracle.h): the
 * product never links or calls this file.
 *
 * Build: gcc -O2 -ffp-contract=off -fno-fast-math -fPIC -shared (oracle/Makefile).
 * Every float operation below is a single IEEE-754 binary32 operation rounded
 * to nearest-even; no FMA contraction, no reassociation.  That is what the
 * reference's MLIR lowering emits: arith.mulf / arith.addf without fastmath
 * flags, carried through scf.for iter_args (src/C3/C3DialectLowering.cpp:540-572),
 * JIT-compiled with default TargetOptions (src/C3/MLIRKernelGen.cpp:1618-1646).
 */
#pragma STDC FP_CONTRACT OFF

#include "c3_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Seeded inputs.  SplitMix64 (Steele, Lea, Flood 2014; the published        */
/* constants of java.util.SplittableRandom).  Not part of the reference: it   */
/* only produces reproducible synthetic inputs.                              */
/* ------------------------------------------------------------------------ */
uint64_t oracle_splitmix64_next(uint64_t* state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* 24 random bits -> [0,1) exactly representable in fp32. */
static float u01(uint64_t* s) { return (float)(oracle_splitmix64_next(s) >> 40) * (1.0f / 16777216.0f); }

void oracle_fill_uniform(uint64_t seed, float* out, int64_t n, float lo, float hi) {
    uint64_t s = seed;
    float w = hi - lo;
    for (int64_t i = 0; i < n; ++i) out[i] = lo + w * u01(&s);
}

/* Box-Muller in double, rounded once to fp32. */
void oracle_fill_normal(uint64_t seed, float* out, int64_t n, float mean, float stddev) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        double u1 = ((double)(oracle_splitmix64_next(&s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(oracle_splitmix64_next(&s) >> 11) * (1.0 / 9007199254740992.0);
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(mean + stddev * r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(mean + stddev * r * sin(two_pi * u2));
    }
}

void oracle_fill_labels(uint64_t seed, int32_t* out, int64_t n, int32_t num_classes) {
    uint64_t s = seed;
    for (int64_t i = 0; i < n; ++i)
        out[i] = (int32_t)(oracle_splitmix64_next(&s) % (uint64_t)num_classes);
}

/* ------------------------------------------------------------------------ */
/* bf16.  The reference has no bf16 (TensorDesc defaults to kFloat,          */
/* include/C3/Graph.h:43); the bf16 path is checked by applying this fp32    */
/* restatement to inputs rounded to bf16 (round to nearest, ties to even).   */
/* ------------------------------------------------------------------------ */
uint16_t oracle_f32_to_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void oracle_round_bf16(const float* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_bf16_to_f32(oracle_f32_to_bf16(in[i]));
}

void oracle_pack_bf16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_bf16(in[i]);
}

/* arith.maxnumf / llvm.maxnum: a NaN operand yields the other operand.  The
 * sign of the result for maxnum(-0, +0) is unspecified by LLVM; this
 * restatement returns the second operand there (relu(-0) = +0).            */
float oracle_maxnum(float a, float b) {
    if (a != a) return b;
    if (b != b) return a;
    if (a == b) return b;
    return a > b ? a : b;
}

/* ------------------------------------------------------------------------ */
/* MatMul.  src/C3/C3DialectLowering.cpp:467-610 (tiled i/j loops with the   */
/* k loop innermost, accumulator starts at 0.0f) and :82-177 (small path,    */
/* same per-element k order).  transA == 112 reads A as [K][M]              */
/* (a_idx = k*M + i, :546-553); transB == 112 reads B as [N][K]             */
/* (b_idx = j*K + k, :555-562).  Any nonzero trans flag means "transposed"   */
/* here.  The tile only changes the i/j visiting order, never a result bit;  */
/* it exists so the CPU baseline walks memory the way the reference does.    */
/* Unlike the reference (tile loops unclamped, :505-521), tails are clamped.  */
/* ------------------------------------------------------------------------ */
void oracle_matmul(const float* A, const float* B, float* C, int64_t M, int64_t K, int64_t N,
                   int transA, int transB, int64_t tile) {
    if (tile <= 0) tile = 64;
    for (int64_t it = 0; it < M; it += tile) {
        int64_t ie = it + tile < M ? it + tile : M;
        for (int64_t jt = 0; jt < N; jt += tile) {
            int64_t je = jt + tile < N ? jt + tile : N;
            for (int64_t i = it; i < ie; ++i) {
                for (int64_t j = jt; j < je; ++j) {
                    float acc = 0.0f;
                    for (int64_t k = 0; k < K; ++k) {
                        float a = transA ? A[k * M + i] : A[i * K + k];
                        float b = transB ? B[j * K + k] : B[k * N + j];
                        float p = a * b;
                        acc = acc + p;
                    }
                    C[i * N + j] = acc;
                }
            }
        }
    }
}

/* Epilogue pass of the fused region: y = maxnum(t + b[idx mod N], 0).
 * src/C3/MLIRKernelGen.cpp:660-767 (broadcast by remui when numel < n,
 * :663-684; AddNode :729-731; ReLUNode maxnumf :707-710).  The bias is added
 * after the k accumulation, not used as its initial value (Graph::fuse folds
 * Add->ReLU into a FusedNode, src/C3/Graph.cpp:587-772, so the c3.matmul
 * epilogue detection at src/C3/MLIRKernelGen.cpp:1124-1198 never fires).
 * act: 0 = bias only, 1 = bias + ReLU.                                     */
/* act 2: the fused epilogue's sigmoid, 1 / (1 + expf(-z)) (NegF, expf call,
 * AddF, DivF; src/C3/MLIRKernelGen.cpp:711-718); act 3: tanhf(z) (math.tanh,
 * the c3.matmul act = 3 epilogue, src/C3/C3DialectLowering.cpp:588). */
static float act_fwd(float z, int act) {
    if (act == 1) return oracle_maxnum(z, 0.0f);
    if (act == 2) {
        float e = expf(-z);
        float d = 1.0f + e;
        return 1.0f / d;
    }
    if (act == 3) return tanhf(z);
    return z;
}

void oracle_bias_act(const float* t, const float* bias, float* y, int64_t M, int64_t N, int act) {
    for (int64_t i = 0; i < M; ++i) {
        for (int64_t j = 0; j < N; ++j) {
            float z = t[i * N + j] + bias[j];
            y[i * N + j] = act_fwd(z, act);
        }
    }
}

/* MatMul -> scratch, then the FusedNode epilogue: the two passes the
 * reference's multi-node kernel runs (src/C3/MLIRKernelGen.cpp:783-1253;
 * inputs in graph order [X, W, b], include/C3/C3HotPathManager.h:730-744). */
void oracle_linear_fwd(const float* X, const float* W, const float* b, float* Y, int64_t M,
                       int64_t K, int64_t N, int act) {
    float* t = (float*)malloc((size_t)(M * N) * sizeof(float));
    oracle_matmul(X, W, t, M, K, N, 0, 0, 64);
    oracle_bias_act(t, b, Y, M, N, act);
    free(t);
}

/* ReLU backward: Gt(z, 0) then Mul(mask, grad).
 * buildReLUBackwardGraph, src/C3/C3BackwardCapture.cpp:501-528;
 * buildGt (OGT compare, select 1.0/0.0), src/C3/MLIRKernelGen.cpp:173-211;
 * c3.mul, src/C3/C3DialectLowering.cpp:246-291.  The mask is multiplied,
 * not selected: 0 * dY keeps dY's sign (+-0) and propagates NaN/Inf.      */
void oracle_relu_mask_mul(const float* z, const float* g, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        float m = (z[i] > 0.0f) ? 1.0f : 0.0f;
        out[i] = m * g[i];
    }
}

/* SumReduce, src/C3/C3DialectLowering.cpp:382-465.  axis 0: out[j] = sum_i
 * in[i*N+j], i ascending from 0.0f (the bias gradient, axis chosen by
 * computeReduceAxis, src/C3/C3BackwardCapture.cpp:1641-1700).  axis 1:
 * out[i] = sum_j in[i*N+j].                                                 */
void oracle_sum_reduce(const float* in, float* out, int64_t M, int64_t N, int axis) {
    if (axis == 0) {
        for (int64_t j = 0; j < N; ++j) {
            float s = 0.0f;
            for (int64_t i = 0; i < M; ++i) s = s + in[i * N + j];
            out[j] = s;
        }
    } else {
        for (int64_t i = 0; i < M; ++i) {
            float s = 0.0f;
            for (int64_t j = 0; j < N; ++j) s = s + in[i * N + j];
            out[i] = s;
        }
    }
}

/* Backward of one Linear+bias(+ReLU) layer, per-node as the reference
 * captures it:
 *   ReLU  : dZ = (Z > 0 ? 1 : 0) * dY   (src/C3/C3BackwardCapture.cpp:501-528)
 *           Y > 0 <=> Z > 0 for every fp32 Z (Y = maxnum(Z, 0)), so Y serves as
 *           the mask source.
 *   MatMul: dX = dZ . W^T  (in:0, transB; src/C3/C3BackwardCapture.cpp:681-708)
 *           dW = X^T . dZ  (in:1, transA; src/C3/C3BackwardCapture.cpp:709-723)
 *   Add   : db = SumReduce(dZ, axis 0)  (src/C3/C3BackwardCapture.cpp:618-644)
 * act == 0: no ReLU node, dZ = dY.  Any of dX, dW, db may be NULL.          */
void oracle_linear_bwd(const float* X, const float* W, const float* Y, const float* dY, float* dX,
                       float* dW, float* db, int64_t M, int64_t K, int64_t N, int act) {
    float* dz = (float*)malloc((size_t)(M * N) * sizeof(float));
    if (act == 1)
        oracle_relu_mask_mul(Y, dY, dz, M * N);
    else if (act == 2 || act == 3)
        oracle_act_grad(Y, dY, dz, M * N, act);
    else
        memcpy(dz, dY, (size_t)(M * N) * sizeof(float));
    /* dX[M,K] = dZ[M,N] . W[K,N]^T : matmul with M'=M, K'=N, N'=K, transB.  */
    if (dX) oracle_matmul(dz, W, dX, M, N, K, 0, 1, 64);
    /* dW[K,N] = X[M,K]^T . dZ[M,N] : matmul with M'=K, K'=M, N'=N, transA.  */
    if (dW) oracle_matmul(X, dz, dW, K, M, N, 1, 0, 64);
    if (db) oracle_sum_reduce(dz, db, M, N, 0);
    free(dz);
}

/* Single-node elementwise ops.
 * BinaryOpLowering<Add/Sub/Mul/Div>, src/C3/C3DialectLowering.cpp:246-291
 * (bmod > 0: r_idx = idx mod bmod; bmod < 0: l_idx = idx mod -bmod);
 * NegOp (arith.negf, sign flip), :317; ReLUOpLowering (maxnumf(x, 0)), :325-350;
 * scale = Mul with a scalar rhs (LinalgElementwiseGen rhs_mod = 1,
 * src/C3/LinalgElementwiseGen.cpp:168-186), here x * alpha;
 * relu-backward mask-mul = oracle_relu_mask_mul with (a = z, b = grad).     */
void oracle_elementwise(int op, const float* a, const float* b, float alpha, float* out,
                        int64_t n, int64_t bmod) {
    for (int64_t i = 0; i < n; ++i) {
        int64_t li = i, ri = i;
        if (bmod > 0) ri = i % bmod;
        else if (bmod < 0) li = i % (-bmod);
        float x = a[li];
        float r;
        switch (op) {
            case ORACLE_EW_ADD: r = x + b[ri]; break;
            case ORACLE_EW_SUB: r = x - b[ri]; break;
            case ORACLE_EW_MUL: r = x * b[ri]; break;
            case ORACLE_EW_DIV: r = x / b[ri]; break;
            case ORACLE_EW_RELU: r = oracle_maxnum(x, 0.0f); break;
            case ORACLE_EW_RELU_BWD: r = ((x > 0.0f) ? 1.0f : 0.0f) * b[ri]; break;
            case ORACLE_EW_NEG: r = -x; break;
            case ORACLE_EW_SCALE: r = x * alpha; break;
            /* SigmoidOpLowering (src/C3/C3DialectLowering.cpp:352-380): NegF, math.exp,
             * AddF(1, e), DivF(1, d); Tanh/Exp/Log: math.tanh/exp/log (:321-323). */
            case ORACLE_EW_SIGMOID: {
                float e = expf(-x);
                float d = 1.0f + e;
                r = 1.0f / d;
                break;
            }
            case ORACLE_EW_TANH: r = tanhf(x); break;
            case ORACLE_EW_EXP: r = expf(x); break;
            case ORACLE_EW_LOG: r = logf(x); break;
            /* buildSigmoidBackwardGraph (src/C3/C3BackwardCapture.cpp:530-567):
             * s = 1/(1+exp(-x)), one_minus = 1 - s, t = s * one_minus, grad * t. */
            case ORACLE_EW_SIGMOID_BWD: {
                float e = expf(-x);
                float d = 1.0f + e;
                float s = 1.0f / d;
                float om = 1.0f - s;
                float t = s * om;
                r = b[ri] * t;
                break;
            }
            /* buildTanhBackwardGraph (:569-616): tanh through exp,
             * (e^x - e^-x) / (e^x + e^-x), then grad * (1 - t*t). */
            case ORACLE_EW_TANH_BWD: {
                float e = expf(x);
                float en = expf(-x);
                float num = e - en;
                float den = e + en;
                float t = num / den;
                float sq = t * t;
                float om = 1.0f - sq;
                r = b[ri] * om;
                break;
            }
            /* buildExpBackwardGraph (:823-849): exp(x) * grad. */
            case ORACLE_EW_EXP_BWD: r = expf(x) * b[ri]; break;
            default: r = NAN; break;
        }
        out[i] = r;
    }
}

/* buildDivBackwardGraph, input 1: b_sq = B * B, q = A / b_sq, m = q * grad, -m. */
void oracle_elementwise3(int op, const float* a, const float* b, const float* c, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        float r = NAN;
        if (op == ORACLE_EW3_DIV_BWD_B) {
            float bb = b[i] * b[i];
            float q = a[i] / bb;
            float m = q * c[i];
            r = -m;
        }
        out[i] = r;
    }
}

/* The activation's derivative applied to the incoming gradient, from the
 * activation's output y: ReLU (y > 0 ? 1 : 0) * g (buildReLUBackwardGraph with
 * z > 0 <=> y > 0); sigmoid g * (y * (1 - y)) (buildSigmoidBackwardGraph: its
 * recomputed s from the pre-activation equals y); tanh g * (1 - y * y). */
void oracle_act_grad(const float* y, const float* g, float* out, int64_t n, int act) {
    for (int64_t i = 0; i < n; ++i) {
        float r;
        if (act == 1) {
            r = ((y[i] > 0.0f) ? 1.0f : 0.0f) * g[i];
        } else if (act == 2) {
            float om = 1.0f - y[i];
            float t = y[i] * om;
            r = g[i] * t;
        } else if (act == 3) {
            float sq = y[i] * y[i];
            float om = 1.0f - sq;
            r = g[i] * om;
        } else {
            r = g[i];
        }
        out[i] = r;
    }
}

/* Mean softmax cross-entropy over M rows of C logits, its per-row terms
 * loss_rows[i] = logsumexp(row i) - row_i[label_i] (nullable) and its gradient
 * dlogits = (softmax - onehot) / M (nullable).  The reference leaves this
 * step to the host framework's CE op (op code 79 in src/C3/RollingHash.cpp:66);
 * it is here so train-step tests have a checker.  exp/log come from libm.  */
float oracle_softmax_ce(const float* logits, const int32_t* labels, float* loss_rows, float* dlogits,
                        int64_t M, int64_t C) {
    double loss = 0.0;
    float inv_m = 1.0f / (float)M;
    for (int64_t i = 0; i < M; ++i) {
        const float* row = logits + i * C;
        float mx = row[0];
        for (int64_t j = 1; j < C; ++j) mx = row[j] > mx ? row[j] : mx;
        float s = 0.0f;
        for (int64_t j = 0; j < C; ++j) s = s + expf(row[j] - mx);
        float lse = mx + logf(s);
        float li = lse - row[labels[i]];
        if (loss_rows) loss_rows[i] = li;
        loss += (double)li;
        if (dlogits) {
            for (int64_t j = 0; j < C; ++j) {
                float p = expf(row[j] - mx) / s;
                float t = (j == labels[i]) ? 1.0f : 0.0f;
                dlogits[i * C + j] = (p - t) * inv_m;
            }
        }
    }
    return (float)(loss / (double)M);
}

/* SGD step w = w - lr * g with the product rounded first (no FMA; this file
 * is built with -ffp-contract=off).  The optimizer is the host framework's in
 * the reference; this is the checker of the device update.  */
void oracle_sgd_update(float* w, const float* g, float lr, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        float step = lr * g[i];
        w[i] = w[i] - step;
    }
}

/* The same on bf16 bit patterns: widen, update in fp32, round to nearest-even. */
void oracle_sgd_update_bf16(uint16_t* w, const float* g, float lr, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        uint32_t u = (uint32_t)w[i] << 16;
        float x;
        memcpy(&x, &u, 4);
        float step = lr * g[i];
        w[i] = oracle_f32_to_bf16(x - step);
    }
}
