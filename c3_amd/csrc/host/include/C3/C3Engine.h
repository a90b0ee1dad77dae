// C3Engine.h -- the CompiledKernel plugin contract and the engine that
// produces gfx950 kernels for it.
//
// CompiledKernel keeps the reference's interface (include/C3/C3Engine.h:153-206):
// execute() takes the graph's inputs in order and returns its outputs
// (callee-allocated), throwing std::runtime_error on bad inputs.
//
// The reference's engine lowers a Graph through MLIR/LLVM and JIT-compiles
// CPU code (src/C3/C3Engine.cpp:712-920).  Here "compile" resolves a
// KernelSpec (the op pattern, shapes and dtype the graph would describe) to
// a prebuilt gfx950 kernel: the code object comes from the on-disk JITCache
// when present (key derived from the RollingHash of the op sequence, the
// shapes and the dtype), else from the package's prebuilt objects, which are
// then stored in the cache; the result is a HipCompiledKernel that launches
// through the C ABI (include/c3hip.h).  compileAsync keeps the reference's
// watchdog semantics: past the timeout the future yields nullptr and the
// last error says so (src/C3/C3Engine.cpp:1077-1132).
#pragma once

#include <atomic>
#include <cstdint>
#include <functional>
#include <future>
#include <memory>
#include <mutex>
#include <optional>
#include <string>
#include <unordered_map>
#include <vector>

#include "C3/C3KernelRegistry.h"
#include "C3/Ctools.h"

namespace ct {
namespace c3 {

class CompiledKernel {
public:
    virtual ~CompiledKernel() = default;
    virtual std::vector<Tensor> execute(const std::vector<Tensor>& inputs) = 0;
    [[nodiscard]] virtual const std::string& cacheKey() const = 0;
    [[nodiscard]] virtual DeviceType targetDevice() const = 0;
    [[nodiscard]] virtual size_t workspaceBytes() const = 0;
    [[nodiscard]] virtual std::optional<std::vector<size_t>> outShape() const { return std::nullopt; }
    virtual bool installIntoRegistry(op op_type, const KernelShapeInfo& shapes) {
        (void)op_type;
        (void)shapes;
        return false;
    }
    [[nodiscard]] virtual int optLevel() const { return opt_level_; }

protected:
    int opt_level_ = 3;
};

enum class C3Backend { MLIR, Handwritten, HIP };

struct CompileOptions {
    int opt_level = 3;
    C3Backend backend = C3Backend::HIP;
    bool use_cache = true;
};

// What a compile produces: one kernel family entry of the C ABI.
enum class KernelKind {
    Elementwise,   // single-node add/sub/mul/div/relu/neg/scale/sigmoid/tanh/exp/log (+ relu-bwd mask-mul),
                   // inputs in operand order
    MatMul,        // single-node c3.matmul with transA/transB
    LinearFwd,     // region MatMul(+Add)(+act): inputs [X, W(, b)]
    ReLUBackward,  // ReLU node backward: inputs [grad, x] -> (x > 0 ? 1 : 0) * grad
    UnaryBackward, // Sigmoid/Tanh/Exp node backward: inputs [grad, x] -> ew_op(x, grad)
    DivBackwardB,  // Div node backward, input 1: inputs [grad, A, B] -> -((A / (B*B)) * grad)
    AddBackwardLhs,// Add node backward, input 0: identity on grad
    SumReduce,     // Add node backward, input 1 (bias): column sums of grad
    MatMulBackwardA, // MatMul node backward, input 0: grad . B^T, inputs [grad, B]
    MatMulBackwardB, // MatMul node backward, input 1: A^T . grad, inputs [grad, A]
    LinearBwd,     // fused layer backward: inputs [dY, X, W, Y] -> [dX, dW, db]
    BackwardChain  // fused backward of single-input nodes: inputs [grad, x_0..x_{w-1}] ->
                   // [g_1..g_w], the upstream grad of each node (c3hip_backward_chain)
};

struct KernelSpec {
    KernelKind kind = KernelKind::Elementwise;
    std::vector<op> op_seq;                       // ops the kernel covers, in execution order
    int ew_op = 0;                                // C3HIP_EW_* for Elementwise
    float alpha = 1.0f;                           // scale factor of EW_SCALE
    int act = 0;                                  // C3HIP_ACT_* for LinearFwd / LinearBwd
    bool transA = false, transB = false;          // MatMul
    int axis = 0;                                 // SumReduce
    std::vector<int> chain;                       // C3HIP_CHAIN_* per node, BackwardChain
    std::vector<std::vector<size_t>> input_shapes;
    std::vector<size_t> out_shape;
    DType dtype = DType::kFloat;
    // Canonical text of the spec (the cache-key material, like Graph::toString).
    std::string toString() const;
    // C ABI module the kernel lives in ("elementwise", "gemm_f32", "gemm_bf16", "reduce").
    std::string moduleName() const;
};

struct C3CacheStats {
    size_t hits = 0;
    size_t misses = 0;
    size_t entries = 0;
    size_t compile_count = 0;
    size_t async_timeouts = 0;
};

class C3Engine {
public:
    using CompileFuture = std::shared_future<std::shared_ptr<CompiledKernel>>;

    static C3Engine& getInstance();

    std::shared_ptr<CompiledKernel> compile(const KernelSpec& spec, const CompileOptions& opts = {});
    CompileFuture compileAsync(const KernelSpec& spec, const CompileOptions& opts = {});

    void setCompileTimeoutMs(uint32_t ms) { compile_timeout_ms_.store(ms); }
    uint32_t getCompileTimeoutMs() const { return compile_timeout_ms_.load(); }
    std::string getLastCompileError() const;
    C3CacheStats getCacheStats() const;
    void clearCache();
    void shutdown();

    // Test hook: replaces the kernel factory (the "backend") used by compile.
    using Factory = std::function<std::shared_ptr<CompiledKernel>(const KernelSpec&, const CompileOptions&)>;
    void setFactoryForTest(Factory f);
    bool hasFactoryForTest() const;

private:
    C3Engine() = default;
    void setLastError(const std::string& e);

    mutable std::mutex mu_;
    std::unordered_map<std::string, std::shared_ptr<CompiledKernel>> cache_;  // key: opt|spec
    std::vector<std::future<void>> workers_;
    std::string last_error_;
    Factory factory_;
    std::atomic<uint32_t> compile_timeout_ms_{30000};
    std::atomic<size_t> hits_{0}, misses_{0}, compiles_{0}, timeouts_{0};
    std::atomic<bool> shutting_down_{false};
};

// Stream used by HipCompiledKernel launches on this thread (hipStream_t as
// void*; nullptr = the default stream).
void setCurrentStream(void* stream);
void* getCurrentStream();

}  // namespace c3
}  // namespace ct
