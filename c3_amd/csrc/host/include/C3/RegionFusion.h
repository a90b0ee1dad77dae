// RegionFusion.h -- registry of fused op-sequence ("region") kernels.
//
// Entries are keyed by regionKey(opHash, first input shape) =
// opHash ^ (shapeHash << 32) with shapeHash = fold(h * 31 + d + 1) over the
// first input's dims (src/C3/RegionFusionRegistry.cpp:85-97).
// installWithCost activates an entry only when the cost model calls the
// fusion worthwhile; mayMatchAsLastOp is an O(1) lock-free bit test on the
// last op of every installed sequence (:171-176).
//
// matchFromPosition walks the dispatch trace's prefix hashes from the longest
// candidate (<= 32 ops) down to 2, as the reference does (:138-164).  The
// reference looks the candidate up by its op hash alone, while installWithCost
// stores it under the shape-mixed key, so a shape-keyed entry can only be
// reached through find(); here the caller passes the first input's shape and
// the lookup uses the same shape-mixed key as the install.
//
// Two regions with the same op sequence and the same first-input shape (two
// Linear layers reading [M, K] with different W widths) share that key; the
// reference keeps the last one installed and the other layer's calls fail
// its shape check and run eagerly.  Here installWithCost also files every
// entry under a second key that mixes all of its input shapes, and a caller
// that passes its input shapes to matchFromPosition gets the entry compiled
// for them (falling back to the shared key, as the reference does).
#pragma once

#include <atomic>
#include <cstdint>
#include <memory>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "C3/C3KernelRegistry.h"
#include "C3/FusionCostModel.h"

namespace ct {
namespace c3 {

struct RegionEntry {
    uint64_t hash = 0;
    std::vector<op> op_seq;
    std::vector<size_t> input_shapes;
    std::vector<std::vector<size_t>> first_input_shapes;
    std::shared_ptr<CompiledKernel> kernel;
    FusedKernelFunc fused_func_ptr = nullptr;
    size_t num_external_inputs = 0;
    size_t len = 0;
    bool active = false;
    FusionCost cost;
};

class RegionFusionRegistry {
public:
    static RegionFusionRegistry& getInstance();

    static uint64_t shapeHash(const std::vector<size_t>& first_input_shape);
    static uint64_t regionKey(uint64_t op_hash, const std::vector<size_t>& first_input_shape) {
        return op_hash ^ (shapeHash(first_input_shape) << 32);
    }

    void install(uint64_t hash, const std::vector<op>& op_seq, std::shared_ptr<CompiledKernel> kernel,
                 const std::vector<size_t>& input_shapes);
    void installFromCompiledKernel(const std::vector<op>& op_seq, std::shared_ptr<CompiledKernel> kernel);
    void installWithCost(const std::vector<op>& op_seq, std::shared_ptr<CompiledKernel> kernel,
                         const std::vector<size_t>& out_numels,
                         const std::vector<std::vector<size_t>>& first_input_shapes = {});

    // Returned entries are copies (safe to use after concurrent installs).
    std::optional<RegionEntry> find(uint64_t hash);
    std::optional<RegionEntry> matchFromPosition(const std::vector<uint64_t>& prefix_hashes, size_t current_pos,
                                                 const std::vector<size_t>& first_input_shape = {},
                                                 const std::vector<std::vector<size_t>>& input_shapes = {});
    // Key of an entry under all of its input shapes (the second index above).
    static uint64_t variantKey(uint64_t region_key, const std::vector<std::vector<size_t>>& input_shapes);
    size_t entryCount() const;
    size_t installedCountNoLock() const { return installed_count_.load(std::memory_order_acquire); }
    bool mayMatchAsLastOp(op last_op) const {
        return (installed_last_ops_.load(std::memory_order_acquire) & (uint64_t(1) << static_cast<size_t>(last_op))) != 0;
    }
    void clear();
    void uninstallAll();

private:
    RegionFusionRegistry() = default;
    void setLastOpBit(const std::vector<op>& op_seq);

    mutable std::mutex mutex_;
    std::unordered_map<uint64_t, RegionEntry> entries_;
    std::unordered_map<uint64_t, RegionEntry> variants_;  // keyed by variantKey
    std::atomic<size_t> installed_count_{0};
    static_assert(static_cast<size_t>(op::kCount) <= 64, "op::kCount exceeds the last-op bitmask");
    std::atomic<uint64_t> installed_last_ops_{0};
};

}  // namespace c3
}  // namespace ct
