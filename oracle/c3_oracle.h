/*
 * c3_oracle.h -- CPU restatement of the reference's fused Linear+bias+ReLU
 * forward/backward and elementwise arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: it may be loaded by
 * tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg, and by
 * nothing else.  The product path (libc3hip.so + the gfx950 code objects) never
 * links, loads or calls it.
 *
 * All arithmetic is IEEE fp32, one rounding per operation, no fused
 * multiply-add (the file is compiled with -ffp-contract=off, without
 * -ffast-math), loops in the reference's order.  Matrices are row-major.
 *
 * How it is pinned (the reference holds no golden vectors and cannot be built
 * here; tests/test_oracle.py and tests/test_golden.py): integer-valued inputs
 * against exact arithmetic (all transpose cases, bias, mask, db, SumReduce);
 * known-answer fixtures in tests/golden/ made by numpy alone (exact integer
 * layers, single IEEE operations over special values, softmax-CE closed
 * forms); float64 brute force within the gamma_K bound; hand-built cases
 * that change if the summation order, FMA contraction, bias placement, mask
 * sign or maxnum NaN rule change; closed forms and central differences for
 * softmax-CE and SGD.  Parity unpinned: the exact bits of the reference's
 * LLVM-JIT output, i.e. that LLVM neither reassociated nor contracted the
 * sequential k-loop; this file follows the reference's source, and no check
 * available here can observe its compiled code.
 */
#ifndef C3_ORACLE_H
#define C3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Elementwise op codes (shared with include/c3hip.h). */
enum {
    ORACLE_EW_ADD = 0,
    ORACLE_EW_SUB = 1,
    ORACLE_EW_MUL = 2,
    ORACLE_EW_DIV = 3,
    ORACLE_EW_RELU = 4,
    ORACLE_EW_RELU_BWD = 5,
    ORACLE_EW_NEG = 6,
    ORACLE_EW_SCALE = 7,
    ORACLE_EW_SIGMOID = 8,
    ORACLE_EW_TANH = 9,
    ORACLE_EW_EXP = 10,
    ORACLE_EW_LOG = 11,
    ORACLE_EW_SIGMOID_BWD = 12,
    ORACLE_EW_TANH_BWD = 13,
    ORACLE_EW_EXP_BWD = 14
};
enum { ORACLE_EW3_DIV_BWD_B = 0 };

/* ---- seeded synthetic inputs (SplitMix64) ---- */
uint64_t oracle_splitmix64_next(uint64_t* state);
void oracle_fill_uniform(uint64_t seed, float* out, int64_t n, float lo, float hi);
void oracle_fill_normal(uint64_t seed, float* out, int64_t n, float mean, float stddev);
void oracle_fill_labels(uint64_t seed, int32_t* out, int64_t n, int32_t num_classes);

/* ---- bf16 helpers (round-to-nearest-even, NaN kept quiet) ---- */
uint16_t oracle_f32_to_bf16(float x);
float oracle_bf16_to_f32(uint16_t h);
void oracle_round_bf16(const float* in, float* out, int64_t n);
void oracle_pack_bf16(const float* in, uint16_t* out, int64_t n);

/* ---- scalar semantics ---- */
float oracle_maxnum(float a, float b);

/* ---- kernels ---- */
void oracle_matmul(const float* A, const float* B, float* C, int64_t M, int64_t K, int64_t N,
                   int transA, int transB, int64_t tile);
void oracle_bias_act(const float* t, const float* bias, float* y, int64_t M, int64_t N, int act);
void oracle_linear_fwd(const float* X, const float* W, const float* b, float* Y, int64_t M,
                       int64_t K, int64_t N, int act);
void oracle_relu_mask_mul(const float* z, const float* g, float* out, int64_t n);
void oracle_sum_reduce(const float* in, float* out, int64_t M, int64_t N, int axis);
void oracle_linear_bwd(const float* X, const float* W, const float* Y, const float* dY, float* dX,
                       float* dW, float* db, int64_t M, int64_t K, int64_t N, int act);
void oracle_elementwise(int op, const float* a, const float* b, float alpha, float* out,
                        int64_t n, int64_t bmod);
void oracle_elementwise3(int op, const float* a, const float* b, const float* c, float* out, int64_t n);
/* act'(y) * g from the activation's output y (act 0..3), elementwise. */
void oracle_act_grad(const float* y, const float* g, float* out, int64_t n, int act);

/* ---- softmax cross-entropy for the MLP train step (host-side step of the caller) ---- */
float oracle_softmax_ce(const float* logits, const int32_t* labels, float* loss_rows, float* dlogits,
                        int64_t M, int64_t C);
void oracle_sgd_update(float* w, const float* g, float lr, int64_t n);
void oracle_sgd_update_bf16(uint16_t* w, const float* g, float lr, int64_t n);

#ifdef __cplusplus
}
#endif
#endif
