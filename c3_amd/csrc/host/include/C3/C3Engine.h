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
    // compile() returns a tiered PGOCompiledKernel (include/C3/C3Engine.h:80,
    // src/C3/C3Engine.cpp:838-861 of the reference).
    bool pgo_mode = false;
};

// Execution-time statistics of one kernel (include/C3/C3Engine.h:109-150 of
// the reference).  Times are host wall times of execute(); for a HIP kernel
// that is the launch, not the device run.
struct ProfileData {
    std::atomic<uint64_t> call_count{0};
    std::atomic<uint64_t> total_time_ns{0};
    std::atomic<uint64_t> min_time_ns{UINT64_MAX};
    std::atomic<uint64_t> max_time_ns{0};
    std::atomic<uint64_t> last_time_ns{0};

    void record(uint64_t ns) {
        call_count.fetch_add(1, std::memory_order_relaxed);
        total_time_ns.fetch_add(ns, std::memory_order_relaxed);
        last_time_ns.store(ns, std::memory_order_relaxed);
        uint64_t lo = min_time_ns.load(std::memory_order_relaxed);
        while (ns < lo && !min_time_ns.compare_exchange_weak(lo, ns, std::memory_order_relaxed)) {}
        uint64_t hi = max_time_ns.load(std::memory_order_relaxed);
        while (ns > hi && !max_time_ns.compare_exchange_weak(hi, ns, std::memory_order_relaxed)) {}
    }
    uint64_t avgTimeNs() const {
        const uint64_t n = call_count.load(std::memory_order_relaxed);
        return n ? total_time_ns.load(std::memory_order_relaxed) / n : 0;
    }
};

// How sub-kernel outputs feed the next sub-kernel (include/C3/GraphMerger.h:46-62
// of the reference): links[i] connects output from_output of sub i to input
// to_input of sub i + 1 (SIZE_MAX: not connected).
struct MergeLink {
    size_t from_output;
    size_t to_input;
};
struct MergeSpec {
    std::vector<MergeLink> links;  // sub count - 1 entries
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
    bool input_grad = true;                       // LinearBwd: compute dX (false: the layer input needs no gradient)
    bool transA = false, transB = false;          // MatMul
    int axis = 0;                                 // SumReduce
    std::vector<int> chain;                       // C3HIP_CHAIN_* per node, BackwardChain
    std::string tile;                             // forced GEMM tile (c3hip_set_gemm_tile); "" = size heuristic
    std::vector<std::vector<size_t>> input_shapes;
    std::vector<size_t> out_shape;
    DType dtype = DType::kFloat;
    // Canonical text of the spec (the cache-key material, like Graph::toString).
    std::string toString() const;
    // C ABI module the kernel lives in ("elementwise", "gemm_f32", "gemm_bf16", "reduce").
    std::string moduleName() const;
    // Shapes and element types of the kernel's outputs, in execute() order.
    std::vector<std::pair<std::vector<size_t>, DType>> outputDescs() const;
    // Element type expected of input j.
    DType inputDtype(size_t j) const;
    // Whether the kernel runs a GEMM whose tile a tuner may choose.
    bool hasGemm() const;
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

    // Several kernels chained by a MergeSpec into one CompiledKernel whose
    // inputs are the unlinked inputs of every sub-kernel in (sub, input)
    // order and whose outputs are the last sub-kernel's (src/C3/C3Engine.cpp
    // compileMerged*, src/C3/GraphMerger.cpp:75-245).  The sub-kernels launch
    // back to back on the current stream; linked tensors stay on the device.
    // Throws std::invalid_argument for a spec that does not validate and
    // std::runtime_error when a sub-kernel does not compile.
    std::shared_ptr<CompiledKernel> compileMerged(const std::vector<KernelSpec>& subs, const MergeSpec& spec,
                                                  const CompileOptions& opts = {});
    std::shared_ptr<CompiledKernel> compileMergedSequential(const std::vector<KernelSpec>& subs,
                                                            const CompileOptions& opts = {});
    // Background compileMerged; calls for one (subs, spec, opts) share one future.
    CompileFuture compileMergedAsync(const std::vector<KernelSpec>& subs, const MergeSpec& spec,
                                     const CompileOptions& opts = {});
    // compileMerged behind the PGO tiers (opts.pgo_mode forced on).
    std::shared_ptr<CompiledKernel> compileMergedPGO(const std::vector<KernelSpec>& subs, const MergeSpec& spec,
                                                     const CompileOptions& opts = {});
    std::shared_ptr<CompiledKernel> compileMergedPGOSequential(const std::vector<KernelSpec>& subs,
                                                               const CompileOptions& opts = {});
    // Profile data of a pgo_mode cache key (created on first use).
    std::shared_ptr<ProfileData> profileData(const std::string& key);
    // A PGO tier's compile failure, also kept as the engine's last error (ADR-010 of the reference).
    void recordCompileError(const std::string& tier, const std::string& reason);

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
    std::unordered_map<std::string, std::shared_ptr<ProfileData>> profiles_;
    std::unordered_map<std::string, CompileFuture> merged_async_;
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
