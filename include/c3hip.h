/*
 * c3hip.h -- C ABI of the MI355X (gfx950) backend for C3's fused
 * Linear+bias+ReLU hot path and its elementwise ops.
 *
 * Plain pointers and sizes only.  Every data pointer is a DEVICE pointer on
 * the current HIP device; `stream` is a hipStream_t passed as void* (NULL =
 * the default stream).  Matrices are row-major and contiguous.  Calls are
 * asynchronous on `stream`; they return 0 on success and a nonzero
 * C3HIP_ERR_* code otherwise, with a message from c3hip_last_error() (per
 * thread).  No exception crosses this boundary.
 *
 * In the reference the same work is done by JIT-compiled CPU functions that
 * the registry calls through three raw ABIs (include/C3/C3KernelRegistry.h:61-80):
 *   C3KernelFunc        (a, b, out, n, M, K, N)              single-node ops
 *   MultiNodeKernelFunc (inputs[], out, n, M, K, N, scratch) fused regions
 *   FusedKernelFunc     (inputs[], out, n)                   elementwise chains
 * Each entry point below names the reference function it replaces.
 */
#ifndef C3HIP_H
#define C3HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define C3HIP_ABI_VERSION 1

/* Status codes. */
#define C3HIP_OK 0
#define C3HIP_ERR_INVALID 1      /* bad argument (null pointer, negative size, unknown op/dtype) */
#define C3HIP_ERR_UNSUPPORTED 2  /* valid request this build does not implement (e.g. bf16 elementwise) */
#define C3HIP_ERR_HIP 3          /* a HIP runtime call failed */
#define C3HIP_ERR_NOT_FOUND 4    /* code object or kernel symbol missing */
#define C3HIP_ERR_TOO_LARGE 5    /* operand beyond the kernels' 32-bit element addressing */

/* Element types. */
#define C3HIP_F32 0
#define C3HIP_BF16 1  /* storage bf16 (uint16 bit patterns), fp32 accumulation */

/* Activations (the reference's c3.matmul `act` attribute, include/C3/C3Ops.td:43-87;
 * src/C3/C3DialectLowering.cpp:577-589). */
#define C3HIP_ACT_NONE 0
#define C3HIP_ACT_RELU 1
#define C3HIP_ACT_SIGMOID 2 /* 1 / (1 + expf(-z)) */
#define C3HIP_ACT_TANH 3    /* tanhf(z) */

/* Elementwise ops. */
#define C3HIP_EW_ADD 0
#define C3HIP_EW_SUB 1
#define C3HIP_EW_MUL 2
#define C3HIP_EW_DIV 3
#define C3HIP_EW_RELU 4
#define C3HIP_EW_RELU_BWD 5 /* out = (a > 0 ? 1 : 0) * b  (a = forward input, b = grad) */
#define C3HIP_EW_NEG 6
#define C3HIP_EW_SCALE 7    /* out = a * alpha */
#define C3HIP_EW_SIGMOID 8  /* 1 / (1 + expf(-a))      (SigmoidOpLowering, src/C3/C3DialectLowering.cpp:352-380) */
#define C3HIP_EW_TANH 9     /* tanhf(a)                (UnaryOpLowering<TanhOp>, :321) */
#define C3HIP_EW_EXP 10     /* expf(a)                 (:322) */
#define C3HIP_EW_LOG 11     /* logf(a)                 (:323) */
/* Backward of a single-input node from its forward input a = x and b = grad: */
#define C3HIP_EW_SIGMOID_BWD 12 /* s = 1/(1+expf(-x)); grad * (s * (1 - s))   (src/C3/C3BackwardCapture.cpp:530-567) */
#define C3HIP_EW_TANH_BWD 13    /* t = (e^x - e^-x)/(e^x + e^-x); grad * (1 - t*t)   (:569-616) */
#define C3HIP_EW_EXP_BWD 14     /* expf(x) * grad                            (:823-849) */

/* Three-input elementwise ops (c3hip_elementwise3). */
#define C3HIP_EW3_DIV_BWD_B 0   /* -((a / (b * b)) * c): Div's gradient for its divisor,
                                   a = dividend, b = divisor, c = grad (buildDivBackwardGraph) */

/* Node types of a fused backward chain (c3hip_backward_chain): the rule maps
 * the node's downstream grad g to its upstream grad from its forward input x. */
#define C3HIP_CHAIN_RELU 0     /* (x > 0 ? 1 : 0) * g                  (src/C3/C3BackwardCapture.cpp:501-528) */
#define C3HIP_CHAIN_SIGMOID 1  /* s = 1/(1+expf(-x)); g * (s * (1 - s))           (:530-567) */
#define C3HIP_CHAIN_TANH 2     /* t = (e^x - e^-x)/(e^x + e^-x); g * (1 - t*t)     (:569-616) */
#define C3HIP_CHAIN_EXP 3      /* expf(x) * g                                      (:823-849) */
#define C3HIP_CHAIN_LOG 4      /* g / x                                            (:851-872) */
#define C3HIP_CHAIN_NEG 5      /* -g; x unused (may be NULL)                       (:725-741) */
#define C3HIP_CHAIN_MAX_NODES 4 /* kFusionWindowSize, include/C3/C3BackwardCapture.h:390 */

/* ABI version of the loaded library (C3HIP_ABI_VERSION). */
int c3hip_abi_version(void);

/* Last error message of the calling thread ("" if none). */
const char* c3hip_last_error(void);

/*
 * Load the gfx950 code objects for `device` and make it current.  Looks in
 * $C3_HIP_CODE_OBJECT_DIR, else beside libc3hip.so.  Idempotent; every
 * compute entry point below also initialises the current device on first
 * use.  Replaces the JIT step the reference performs per kernel
 * (mlir::ExecutionEngine::create + lookup("c3_kernel"),
 * src/C3/MLIRKernelGen.cpp:1676-1682): here the code is prebuilt and only
 * loaded (hipModuleLoad / hipModuleGetFunction).
 */
int c3hip_init(int device);

/* Unload every module and free library-owned device memory (the last step of
 * shutdownAll, include/C3/C3Cleanup.h:34-40).  Device memory handed out to
 * callers is not touched. */
int c3hip_shutdown(void);

/*
 * Register a code object image for module `module_name` ("elementwise",
 * "gemm_f32", "gemm_bf16", "reduce" or "loss") on the current device, e.g. one read
 * back from the on-disk JIT cache.  If the module is not loaded yet, the
 * image is loaded.  If it is, the call returns 0 when `image` is the loaded
 * image (same bytes) and C3HIP_ERR_INVALID otherwise, since kernel lookups
 * keep using the loaded module.
 * Replaces the reference's JITCache read path, which reloads cached LLVM
 * bitcode into an ExecutionEngine (src/C3/LinalgElementwiseGen.cpp:403-439).
 */
int c3hip_load_code_object(const char* module_name, const void* image, size_t nbytes);

/* Write into buf (NUL-terminated, at most buflen bytes) the path of the
 * prebuilt code object file for `module_name`.  Returns 0, or
 * C3HIP_ERR_INVALID when buf is too small or the name is unknown. */
int c3hip_code_object_path(const char* module_name, char* buf, size_t buflen);

/*
 * Per-launch timing, for measurement.  While enabled (enable != 0) on the
 * calling thread, every kernel this library launches for that thread is
 * bracketed by two HIP events recorded on the launch's stream; enable == 0
 * stops it and drops unread records.  c3hip_launch_timings waits for the
 * recorded launches and writes, in launch order, up to `max` records: the
 * kernel name into names + i * name_len (NUL-terminated, truncated to
 * name_len - 1; names may be NULL) and its duration between the two events
 * in ms into ms[i]; *count receives the number written and all records are
 * cleared.  The reference times its host-side calls with the host clock
 * (C3KernelRegistry::recordPerf*, include/C3/C3KernelRegistry.h:256-275);
 * device kernels are timed on the device here.
 */
int c3hip_set_launch_timing(int enable);
int c3hip_launch_timings(char* names, size_t name_len, float* ms, int max, int* count);

/*
 * Elementwise op over n contiguous elements: out[i] = op(a[li], b[ri]).
 * bmod > 0: ri = i mod bmod (rhs broadcast, e.g. a bias row); bmod < 0:
 * li = i mod -bmod (lhs broadcast); 0: no broadcast.  b is ignored (may be
 * NULL) for the unary ops (relu, neg, scale, sigmoid, tanh, exp, log);
 * alpha is used by scale only.  dtype: C3HIP_F32.  exp/log/tanh are the
 * device library's expf/logf/tanhf (not bit-identical to a host libm; within
 * a few ulp of it).
 * Replaces the single-node C3KernelFunc kernels: BinaryOpLowering /
 * UnaryOpLowering / ReLUOpLowering (src/C3/C3DialectLowering.cpp:246-350)
 * dispatched by ConcreteCompiledKernel::execute (src/C3/C3Engine.cpp:457-522),
 * the LinalgElementwiseKernel ops (src/C3/LinalgElementwiseGen.cpp:142-244),
 * and the ReLU backward graph Gt+Mul (src/C3/C3BackwardCapture.cpp:501-528).
 */
int c3hip_elementwise(int op, int dtype, const void* a, const void* b, float alpha, void* out,
                      int64_t n, int64_t bmod, void* stream);

/*
 * Three-input elementwise op over n contiguous elements (no broadcast):
 * out[i] = op(a[i], b[i], c[i]).  dtype: C3HIP_F32.  Replaces the
 * multi-input backward graphs that need both forward inputs and the grad
 * (Div in:1, src/C3/C3BackwardCapture.cpp buildDivBackwardGraph).
 */
int c3hip_elementwise3(int op, int dtype, const void* a, const void* b, const void* c, void* out, int64_t n,
                       void* stream);

/*
 * Force the GEMM tile of dtype's GEMMs launched by the calling thread (every
 * c3hip_matmul / c3hip_linear_fwd / c3hip_linear_bwd call that follows), by
 * one of the names c3hip_gemm_tile_names lists; NULL or "" restores the size
 * heuristic.  A forced direct-to-LDS bf16 tile (d*) that cannot run a
 * problem makes that call fail with C3HIP_ERR_UNSUPPORTED (no silent
 * fallback); with a forced tile the bf16 layer backward runs dX, dW and the
 * bias gradient's final pass as separate launches (the size heuristic may
 * put them in one; the bits are the same).  The fp32 direct-to-LDS tiles
 * (t256x128d, t128x256d, t256x256d, t64x64d) run the plain forward
 * (t256x256d: dX and dW only), dX and dW with K a multiple of 16 on 16-byte
 * aligned operands; any other GEMM forced onto them runs on their
 * register-staged twin (t256x128, t128x256, t64x64; t256x128 for t256x256d),
 * which multiplies in the same order, so the result is the same.  Replaces the optimisation-level choice of the reference's PGO
 * tiers (PGOCompiledKernel::compileO2 / compileOfast,
 * src/C3/PGOManager.cpp:292-366): here a tier differs by launch configuration,
 * which the tuner picks by timing the candidates on the caller's stream.
 */
int c3hip_set_gemm_tile(int dtype, const char* name);

/* Comma-separated GEMM tile names of dtype into buf (NUL-terminated). */
int c3hip_gemm_tile_names(int dtype, char* buf, size_t buflen);

/*
 * Fused backward of a chain of num_nodes (1..C3HIP_CHAIN_MAX_NODES)
 * single-input elementwise nodes over n contiguous elements, node 0 the most
 * downstream: g_0 = grad, g_{k+1} = rule(nodes[k], g_k, x[k]) and
 * outs[k] = g_{k+1} (the upstream grad of node k; a NULL outs[k] is not
 * stored).  Every rule is evaluated with the same IEEE operations as the
 * single-node backward kernels, so the outputs are bit-identical to running
 * the nodes one by one.  An output may alias an input at the same offsets.
 * dtype: C3HIP_F32.  Replaces the multi-output fused graph that
 * C3BackwardCapture::compileFusedBackwardAsync builds by merging the nodes'
 * backward graphs (src/C3/C3BackwardCapture.cpp:1140-1210) and the kernel
 * tryExecuteFusedBackward runs (:1344-1637).
 */
int c3hip_backward_chain(int dtype, const void* grad, const void* const* x, const int* nodes, int num_nodes,
                         void* const* outs, int64_t n, void* stream);

/*
 * C[M,N] = op(A) . op(B), fp32 accumulation.  transA != 0: A is stored
 * [K,M]; transB != 0: B is stored [N,K]; otherwise A is [M,K], B is [K,N].
 * fp32 in/out for C3HIP_F32; bf16 A, B and C for C3HIP_BF16.
 * Replaces the single-node c3.matmul kernel (MatMulOpLowering,
 * src/C3/C3DialectLowering.cpp:467-610; transA/transB == 112 paths :546-562),
 * including the MatMul backward kernels dX = grad.B^T and dW = A^T.grad
 * (buildMatMulBackwardGraph, src/C3/C3BackwardCapture.cpp:681-723).
 */
int c3hip_matmul(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t K, int64_t N,
                 int transA, int transB, void* stream);

/*
 * Fused Linear forward: Y[M,N] = act(X[M,K] . W[K,N] + b[N]).
 * b is fp32 (may be NULL: no bias).  C3HIP_F32: X, W, Y fp32.  C3HIP_BF16:
 * X, W, Y bf16, fp32 accumulation, bias and activation applied in fp32, Y
 * rounded to nearest-even once.
 * act: C3HIP_ACT_NONE, _RELU (maxnum(z, 0)), _SIGMOID (1 / (1 + expf(-z)),
 * the fused epilogue's formula, src/C3/MLIRKernelGen.cpp:711-718) or _TANH
 * (tanhf(z), the c3.matmul act = 3 epilogue, src/C3/C3DialectLowering.cpp:588).
 * Replaces the MultiNodeKernelFunc of the MatMul+Add+ReLU and
 * MatMul+Add+Sigmoid regions (inputs [X, W, b], buildMultiNodeMLIR +
 * buildFusedMultiNode, src/C3/MLIRKernelGen.cpp:610-768, :783-1253; executed
 * by MultiNodeCompiledKernel::execute, src/C3/C3Engine.cpp:145-235).
 */
int c3hip_linear_fwd(int dtype, const void* X, const void* W, const float* b, void* Y, int64_t M,
                     int64_t K, int64_t N, int act, void* stream);

/* Bytes of the per-device static scratch of c3hip_linear_fwd_noalloc. */
#define C3HIP_NOALLOC_SCRATCH_BYTES (32u << 20)

/*
 * c3hip_linear_fwd that allocates no device memory: same arguments, kernels,
 * launch plan and results (bit for bit) as c3hip_linear_fwd, with its only
 * workspace (the fp32 split-K partials of a grid too small to fill the chip)
 * in a static per-device array of C3HIP_NOALLOC_SCRATCH_BYTES (32 MiB),
 * which each device that runs it holds until the process ends.  Every
 * forward the size heuristic plans fits; a larger need (only possible with a
 * tile forced by c3hip_set_gemm_tile) fails with C3HIP_ERR_TOO_LARGE before
 * anything is launched.  Call c3hip_init(device) first: it loads the code
 * objects and looks up the scratch, so the entry point itself calls no
 * hipMalloc / hipFree.  Calls on one device share the scratch: calls whose
 * work overlaps in time on that device (different streams or host threads)
 * race; calls on one stream are ordered and safe.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).
 */
int c3hip_linear_fwd_noalloc(int dtype, const void* X, const void* W, const float* b, void* Y, int64_t M,
                             int64_t K, int64_t N, int act, void* stream);

/*
 * Fused Linear backward.  With dZ = (Y > 0 ? 1 : 0) * dY when act ==
 * C3HIP_ACT_RELU, dY * (Y * (1 - Y)) for C3HIP_ACT_SIGMOID, dY * (1 - Y * Y)
 * for C3HIP_ACT_TANH (the activation's derivative from its output) and
 * dZ = dY for C3HIP_ACT_NONE:
 * (The inputs hold no pre-activation Z.  For ReLU the mask from Y equals the
 * reference's Gt(Z, 0) and sigmoid's s from Y equals its recomputation from
 * Z; the reference's Tanh node instead recomputes t = (e^z - e^-z)/(e^z +
 * e^-z) from Z, so tanh layers differ from it in the last bits (within 16 ulp
 * of |dY|) and, for |z| > ~88.7 where its e^z overflows to NaN, give 0.)
 *   dX[M,K] = dZ . W^T,  dW[K,N] = X^T . dZ,  db[N] = sum over rows of dZ.
 * dX, dW and db are each optional (NULL skips it).  dZ is formed inside the
 * GEMM operand loads and never written.  C3HIP_F32: all fp32.  C3HIP_BF16:
 * X, W, Y, dY and dX bf16; dW and db fp32.  Outputs must not overlap the
 * inputs or each other: dX, dW and db may be computed by one launch (small
 * fp32 layers), so no output is ordered before another's reads.
 * Replaces the per-node backward kernels the reference installs for one
 * layer: ReLU (Gt + Mul, src/C3/C3BackwardCapture.cpp:501-528), MatMul in:0
 * and in:1 (:681-723) and Add in:1 SumReduce (:618-644), looked up through
 * C3KernelRegistry::tryExecuteBackward (src/C3/C3KernelRegistry.cpp:230-322).
 */
int c3hip_linear_bwd(int dtype, const void* X, const void* W, const void* Y, const void* dY, void* dX,
                     float* dW, float* db, int64_t M, int64_t K, int64_t N, int act, void* stream);

/*
 * SumReduce of a row-major fp32 [M,N]: axis 0 -> out[N] (column sums),
 * axis 1 -> out[M] (row sums).  Replaces SumReduceOpLowering
 * (src/C3/C3DialectLowering.cpp:382-465), the Add backward in:1 kernel
 * (src/C3/C3BackwardCapture.cpp:618-644).  Uses a library-owned workspace
 * for axis 0 (grown on demand, freed by c3hip_shutdown).
 */
int c3hip_sum_reduce(const float* in, float* out, int64_t M, int64_t N, int axis, void* stream);

/*
 * Softmax cross-entropy over the M rows of logits[M,C] (C3HIP_F32: fp32;
 * C3HIP_BF16: bf16) with int32 labels in [0, C):
 *   loss_rows[i]  = logsumexp(logits[i,:]) - logits[i, labels[i]]   (fp32)
 *   dlogits[i,j]  = (softmax(logits[i,:])_j - [j == labels[i]]) / M  (logits' dtype)
 * loss_rows or dlogits may be NULL.  C <= 2048.  A label outside [0, C)
 * gives NaN in that row.  The mean loss is the row sum of loss_rows over M
 * (c3hip_sum_reduce with axis 1 on a [1, M] view).
 * The reference has no kernel for this step: the host framework's CE op
 * (op code 79, src/C3/RollingHash.cpp:66) runs between the fused forward and
 * the backward of the MLP train step; it is here so the whole step stays on
 * the device.
 */
int c3hip_softmax_ce(int dtype, const void* logits, const int32_t* labels, float* loss_rows, void* dlogits,
                     int64_t M, int64_t C, void* stream);

/*
 * Element type conversion of n contiguous elements: C3HIP_F32 -> C3HIP_BF16
 * (round to nearest-even, NaN stays NaN) or C3HIP_BF16 -> C3HIP_F32 (exact).
 * The same dtype on both sides is a device copy.  No reference counterpart
 * (the reference is fp32 only); it prepares bf16 operands on the device.
 */
int c3hip_cast(int src_dtype, int dst_dtype, const void* in, void* out, int64_t n, void* stream);

/*
 * SGD step on a parameter of n elements: w = w - lr * g, with g fp32 and the
 * product rounded before the subtraction (no fused multiply-add).
 * dtype C3HIP_BF16: w is bf16, updated in fp32 and rounded back.  The
 * optimizer belongs to the host framework in the reference (not part of C3);
 * it closes the train step on the device.
 */
int c3hip_sgd_update(int dtype, void* w, const float* g, float lr, int64_t n, void* stream);

/* Most tensors c3hip_sgd_update_multi takes in one call. */
#define C3HIP_SGD_MAX_TENSORS 16

/*
 * c3hip_sgd_update on `count` parameters of one dtype (w[t], g[t], n[t]) in a
 * single launch, each element updated exactly as c3hip_sgd_update does (the
 * same bits).  count <= C3HIP_SGD_MAX_TENSORS; w, g and n are host arrays of
 * device pointers and sizes.  No reference counterpart (the optimizer belongs
 * to the host framework); it replaces one launch per weight and bias in a
 * train step.
 */
int c3hip_sgd_update_multi(int dtype, int count, void* const* w, const float* const* g, const int64_t* n, float lr,
                           void* stream);

#ifdef __cplusplus
}
#endif
#endif /* C3HIP_H */
