// C3KernelRegistry.h -- install / dispatch / fallback of compiled kernels.
//
// Same API, keys and semantics as the reference registry
// (include/C3/C3KernelRegistry.h:106-418, src/C3/C3KernelRegistry.cpp):
//   * single-op entries keyed (op, device, FNV-1a(lhs shape, rhs shape));
//     dispatch requires exact lhs/rhs shape equality and validates the
//     output shape (a mismatch uninstalls the kernel);
//   * fused entries keyed "pattern|op:lhs..." (makeFusedKey);
//   * backward entries keyed by the capture string, fed [grad] + the
//     forward inputs listed in fwd_input_map;
//   * install keeps an existing entry whose kernel has an opt level >= the
//     new one's;
//   * dispatch never throws: a miss, a shape mismatch or an exception from
//     the kernel returns std::nullopt so the host runs eager.
// Kernels run outside the lock on a copied entry.
#pragma once

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <optional>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "C3/Ctools.h"

namespace ct {
namespace c3 {

class CompiledKernel;

// Raw kernel ABIs of the reference's JIT output (include/C3/C3KernelRegistry.h:61-80).
// Kept for API compatibility; kernels of this backend are reached through
// CompiledKernel::execute and the C ABI of include/c3hip.h.
using C3KernelFunc = void (*)(const float*, const float*, float*, size_t, size_t, size_t, size_t);
using FusedKernelFunc = void (*)(const float* const*, float*, size_t);
using MultiNodeKernelFunc = void (*)(const float* const*, float*, size_t, size_t, size_t, size_t, float*);

struct KernelShapeInfo {
    std::vector<size_t> lhs_shape;
    std::vector<size_t> rhs_shape;
    std::vector<size_t> out_shape;
    bool is_matmul = false;
    size_t M = 0, K = 0, N = 0;
    std::string fused_pattern;  // e.g. "MatMul+Add+ReLU"; empty for single ops
};

class C3KernelRegistry {
public:
    static C3KernelRegistry& getInstance();

    // ---- install / uninstall ----
    void install(op op_type, DeviceType dev, std::shared_ptr<CompiledKernel> kernel, const KernelShapeInfo& shapes);
    void uninstall(op op_type, DeviceType dev);
    void uninstallAll();

    // ---- execution ----
    std::optional<Tensor> tryExecute(op op_type, const Tensor& a, const Tensor& b);
    std::optional<Tensor> tryExecuteUnary(op op_type, const Tensor& a);

    // ---- fused (region) kernels ----
    void installFused(std::shared_ptr<CompiledKernel> kernel, op op_type, const KernelShapeInfo& shapes);
    // Looks up the fused entry keyed by (op_type, pattern of a matching entry,
    // inputs[0] shape) and runs it; nullopt on miss.  (The reference leaves
    // this entry point a stub, src/C3/C3KernelRegistry.cpp:70-75.)
    std::optional<Tensor> tryExecuteFused(op op_type, const std::vector<Tensor>& inputs);
    Tensor executeFusedWithInputs(std::shared_ptr<CompiledKernel> kernel, const std::vector<Tensor>& inputs,
                                  const KernelShapeInfo& shapes);
    void uninstallFused(op op_type, const KernelShapeInfo& shapes);
    size_t fusedEntryCount() const;
    std::optional<std::pair<std::shared_ptr<CompiledKernel>, KernelShapeInfo>> findFusedKernelForSequence(
        const std::vector<op>& op_seq, DeviceType dev, const std::vector<size_t>& first_input_shape = {});
    std::optional<std::pair<std::shared_ptr<CompiledKernel>, KernelShapeInfo>> findFusedKernelForFirstOp(
        op op_type, const std::vector<size_t>& input_shape, DeviceType dev);

    // ---- backward kernels ----
    void installBackward(const std::string& backward_key, std::shared_ptr<CompiledKernel> kernel,
                         const std::vector<size_t>& grad_shape, const std::vector<size_t>& out_shape,
                         const std::vector<size_t>& fwd_input_map, size_t num_inputs = 1);
    std::optional<std::vector<Tensor>> tryExecuteBackward(const std::string& backward_key, const Tensor& grad,
                                                          const std::vector<Tensor>& forward_inputs = {});
    bool hasBackwardKey(const std::string& backward_key);

    // ---- statistics ----
    struct Stats {
        size_t install_count = 0;
        size_t uninstall_count = 0;
        size_t hit_count = 0;
        size_t miss_count = 0;
        size_t bypass_count = 0;
        size_t active_entries = 0;
        size_t fused_entries = 0;
        size_t backward_entries = 0;
        size_t fused_hit_count = 0;
        size_t backward_hit_count = 0;
        uint64_t region_dispatch_ns = 0;
        uint64_t region_match_ns = 0;
        uint64_t c3_single_invoke_ns = 0;
        uint64_t eager_invoke_ns = 0;
        uint64_t region_dispatch_count = 0;
        uint64_t region_match_count = 0;
        uint64_t c3_single_invoke_count = 0;
        uint64_t eager_invoke_count = 0;
        uint64_t region_cost_rejected_count = 0;
    };
    Stats getStats() const;
    void recordBypass() { bypass_count_.fetch_add(1, std::memory_order_relaxed); }
    void recordPerfRegionDispatch(uint64_t ns);
    void recordPerfRegionMatch(uint64_t ns);
    void recordPerfC3SingleInvoke(uint64_t ns);
    void recordPerfEagerInvoke(uint64_t ns);
    void recordPerfRegionCostRejected() { region_cost_rejected_count_.fetch_add(1, std::memory_order_relaxed); }

    // Key helpers (public so tests can pin them against closed forms).
    static size_t hashShapes(const std::vector<size_t>& lhs, const std::vector<size_t>& rhs);
    static std::string makeFusedKey(op op_type, const KernelShapeInfo& shapes);

private:
    C3KernelRegistry() = default;

    struct C3Entry {
        std::shared_ptr<CompiledKernel> kernel;
        KernelShapeInfo shapes;
        bool active = false;
    };
    struct FusedEntry {
        std::shared_ptr<CompiledKernel> kernel;
        KernelShapeInfo shapes;
        bool active = false;
    };
    struct BackwardEntry {
        std::shared_ptr<CompiledKernel> kernel;
        std::vector<size_t> grad_shape;
        std::vector<size_t> out_shape;
        std::vector<size_t> fwd_input_map;
        size_t num_inputs = 1;
        bool active = false;
    };
    struct KeyType {
        size_t first, second, third;
        bool operator==(const KeyType& o) const { return first == o.first && second == o.second && third == o.third; }
    };
    struct KeyHash {
        size_t operator()(const KeyType& k) const {
            size_t h = k.first;
            h ^= (k.second << 16) + 0x9e3779b9 + (h << 6) + (h >> 2);
            h ^= (k.third << 24) + 0x9e3779b9 + (h << 6) + (h >> 2);
            return h;
        }
    };
    static KeyType makeKey(op op_type, DeviceType dev, const std::vector<size_t>& lhs, const std::vector<size_t>& rhs) {
        return {static_cast<size_t>(op_type), static_cast<size_t>(dev), hashShapes(lhs, rhs)};
    }
    bool validateOutputShape(op op_type, DeviceType dev, const Tensor& out, const std::vector<size_t>& expected);

    mutable std::mutex mutex_;
    std::unordered_map<KeyType, C3Entry, KeyHash> entries_;
    std::unordered_map<std::string, FusedEntry> fused_entries_;
    std::unordered_map<std::string, BackwardEntry> backward_entries_;

    std::atomic<size_t> install_count_{0};
    std::atomic<size_t> uninstall_count_{0};
    std::atomic<size_t> hit_count_{0};
    std::atomic<size_t> miss_count_{0};
    std::atomic<size_t> bypass_count_{0};
    std::atomic<size_t> fused_hit_count_{0};
    std::atomic<size_t> backward_hit_count_{0};
    std::atomic<uint64_t> region_dispatch_ns_{0};
    std::atomic<uint64_t> region_match_ns_{0};
    std::atomic<uint64_t> c3_single_invoke_ns_{0};
    std::atomic<uint64_t> eager_invoke_ns_{0};
    std::atomic<uint64_t> region_dispatch_count_{0};
    std::atomic<uint64_t> region_match_count_{0};
    std::atomic<uint64_t> c3_single_invoke_count_{0};
    std::atomic<uint64_t> eager_invoke_count_{0};
    std::atomic<uint64_t> region_cost_rejected_count_{0};
};

std::string shapeToString(const std::vector<size_t>& shape);

}  // namespace c3
}  // namespace ct
