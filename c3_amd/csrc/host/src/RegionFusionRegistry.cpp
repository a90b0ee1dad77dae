// RegionFusionRegistry.cpp -- see include/C3/RegionFusion.h.
#include "C3/RegionFusion.h"

#include "C3/RollingHash.h"

namespace ct {
namespace c3 {

RegionFusionRegistry& RegionFusionRegistry::getInstance() {
    static RegionFusionRegistry r;
    return r;
}

uint64_t RegionFusionRegistry::shapeHash(const std::vector<size_t>& first_input_shape) {
    uint64_t h = 0;
    for (size_t d : first_input_shape) h = h * 31 + d + 1;
    return h;
}

uint64_t RegionFusionRegistry::variantKey(uint64_t region_key, const std::vector<std::vector<size_t>>& input_shapes) {
    // FNV-1a over (rank, dims...) of every input, folded into the region key.
    uint64_t h = 0xcbf29ce484222325ull;
    auto mix = [&](uint64_t v) {
        for (int i = 0; i < 8; ++i) {
            h ^= (v >> (8 * i)) & 0xff;
            h *= 0x100000001b3ull;
        }
    };
    for (const auto& s : input_shapes) {
        mix(s.size());
        for (size_t d : s) mix(d);
    }
    return region_key ^ h;
}

void RegionFusionRegistry::setLastOpBit(const std::vector<op>& op_seq) {
    if (!op_seq.empty())
        installed_last_ops_.fetch_or(uint64_t(1) << static_cast<size_t>(op_seq.back()), std::memory_order_release);
}

void RegionFusionRegistry::install(uint64_t hash, const std::vector<op>& op_seq, std::shared_ptr<CompiledKernel> kernel,
                                   const std::vector<size_t>& input_shapes) {
    std::lock_guard<std::mutex> lk(mutex_);
    RegionEntry e;
    e.hash = hash;
    e.op_seq = op_seq;
    e.kernel = std::move(kernel);
    e.input_shapes = input_shapes;
    e.len = op_seq.size();
    e.active = true;
    entries_[hash] = std::move(e);
    setLastOpBit(op_seq);
    installed_count_.fetch_add(1, std::memory_order_release);
}

void RegionFusionRegistry::installFromCompiledKernel(const std::vector<op>& op_seq,
                                                     std::shared_ptr<CompiledKernel> kernel) {
    if (op_seq.empty()) return;
    install(RollingHash::hashSequence(op_seq), op_seq, std::move(kernel), {});
}

void RegionFusionRegistry::installWithCost(const std::vector<op>& op_seq, std::shared_ptr<CompiledKernel> kernel,
                                           const std::vector<size_t>& out_numels,
                                           const std::vector<std::vector<size_t>>& first_input_shapes) {
    if (op_seq.empty() || !kernel) return;
    const FusionCost cost = FusionCostModel::estimate(op_seq, out_numels);
    const uint64_t op_hash = RollingHash::hashSequence(op_seq);
    const uint64_t hash =
        regionKey(op_hash, first_input_shapes.empty() ? std::vector<size_t>{} : first_input_shapes.front());
    std::lock_guard<std::mutex> lk(mutex_);
    RegionEntry e;
    e.hash = hash;
    e.op_seq = op_seq;
    e.kernel = std::move(kernel);
    e.len = op_seq.size();
    e.cost = cost;
    e.first_input_shapes = first_input_shapes;
    e.active = out_numels.size() == op_seq.size() && cost.worthwhile;
    if (!first_input_shapes.empty()) variants_[variantKey(hash, first_input_shapes)] = e;
    entries_[hash] = std::move(e);
    setLastOpBit(op_seq);
    installed_count_.fetch_add(1, std::memory_order_release);
}

std::optional<RegionEntry> RegionFusionRegistry::find(uint64_t hash) {
    std::lock_guard<std::mutex> lk(mutex_);
    auto it = entries_.find(hash);
    if (it != entries_.end() && it->second.active) return it->second;
    return std::nullopt;
}

std::optional<RegionEntry> RegionFusionRegistry::matchFromPosition(const std::vector<uint64_t>& prefix_hashes,
                                                                   size_t current_pos,
                                                                   const std::vector<size_t>& first_input_shape,
                                                                   const std::vector<std::vector<size_t>>& input_shapes) {
    if (prefix_hashes.empty() || current_pos >= prefix_hashes.size() - 1) return std::nullopt;
    size_t max_len = prefix_hashes.size() - 1 - current_pos;
    if (max_len > 32) max_len = 32;
    std::lock_guard<std::mutex> lk(mutex_);
    for (size_t len = max_len; len >= 2; --len) {
        const uint64_t sub = RollingHash::getSubHash(prefix_hashes, current_pos, current_pos + len - 1);
        const uint64_t key = regionKey(sub, first_input_shape);
        if (!input_shapes.empty()) {
            auto v = variants_.find(variantKey(key, input_shapes));
            if (v != variants_.end() && v->second.active && v->second.len == len) return v->second;
        }
        auto it = entries_.find(key);
        if (it != entries_.end() && it->second.active && it->second.len == len) return it->second;
    }
    return std::nullopt;
}

size_t RegionFusionRegistry::entryCount() const {
    std::lock_guard<std::mutex> lk(mutex_);
    return entries_.size();
}

void RegionFusionRegistry::clear() {
    std::lock_guard<std::mutex> lk(mutex_);
    entries_.clear();
    variants_.clear();
    installed_last_ops_.store(0, std::memory_order_release);
    installed_count_.store(0, std::memory_order_release);
}

void RegionFusionRegistry::uninstallAll() { clear(); }

}  // namespace c3
}  // namespace ct
