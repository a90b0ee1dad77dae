// C3KernelRegistry.cpp -- see include/C3/C3KernelRegistry.h.
#include "C3/C3KernelRegistry.h"

#include <chrono>

#include "C3/C3Engine.h"

namespace ct {
namespace c3 {

std::string shapeToString(const std::vector<size_t>& shape) {
    std::string s = "[";
    for (size_t i = 0; i < shape.size(); ++i) {
        if (i) s += ",";
        s += std::to_string(shape[i]);
    }
    return s + "]";
}

C3KernelRegistry& C3KernelRegistry::getInstance() {
    static C3KernelRegistry instance;
    return instance;
}

// FNV-1a over (rank, dims...) of lhs then rhs (include/C3/C3KernelRegistry.h:485-497).
size_t C3KernelRegistry::hashShapes(const std::vector<size_t>& lhs, const std::vector<size_t>& rhs) {
    size_t h = 1469598103934665603ull;
    auto mix = [&h](size_t v) {
        h ^= v;
        h *= 1099511628211ull;
    };
    mix(lhs.size());
    for (size_t s : lhs) mix(s);
    mix(rhs.size());
    for (size_t s : rhs) mix(s);
    return h;
}

// "pattern|op:d0:d1..." over the lhs shape (include/C3/C3KernelRegistry.h:516-522).
std::string C3KernelRegistry::makeFusedKey(op op_type, const KernelShapeInfo& shapes) {
    std::string key = shapes.fused_pattern;
    key += "|";
    key += std::to_string(static_cast<size_t>(op_type));
    for (size_t s : shapes.lhs_shape) key += ":" + std::to_string(s);
    return key;
}

void C3KernelRegistry::install(op op_type, DeviceType dev, std::shared_ptr<CompiledKernel> kernel,
                               const KernelShapeInfo& shapes) {
    if (!kernel) return;
    std::lock_guard<std::mutex> lock(mutex_);
    const KeyType key = makeKey(op_type, dev, shapes.lhs_shape, shapes.rhs_shape);
    auto it = entries_.find(key);
    if (it != entries_.end() && it->second.active && it->second.kernel &&
        kernel->optLevel() <= it->second.kernel->optLevel())
        return;  // a kernel of equal or higher opt level stays
    entries_[key] = C3Entry{std::move(kernel), shapes, true};
    install_count_.fetch_add(1, std::memory_order_release);
}

void C3KernelRegistry::uninstall(op op_type, DeviceType dev) {
    std::lock_guard<std::mutex> lock(mutex_);
    size_t removed = 0;
    for (auto it = entries_.begin(); it != entries_.end();) {
        if (it->first.first == static_cast<size_t>(op_type) && it->first.second == static_cast<size_t>(dev)) {
            it = entries_.erase(it);
            ++removed;
        } else {
            ++it;
        }
    }
    if (removed) uninstall_count_.fetch_add(removed, std::memory_order_release);
}

void C3KernelRegistry::uninstallAll() {
    std::lock_guard<std::mutex> lock(mutex_);
    uninstall_count_.fetch_add(entries_.size(), std::memory_order_release);
    entries_.clear();
    fused_entries_.clear();
    backward_entries_.clear();
}

bool C3KernelRegistry::validateOutputShape(op op_type, DeviceType dev, const Tensor& out,
                                           const std::vector<size_t>& expected) {
    if (expected.empty() || out.shape() == expected) return true;
    c3log(ErrorLevel::WARN, "[C3-SHAPE-CHECK] op=" + std::to_string(static_cast<int>(op_type)) +
                                " expected=" + shapeToString(expected) + " actual=" + shapeToString(out.shape()) +
                                " -- uninstalling defective kernel");
    uninstall(op_type, dev);
    return false;
}

std::optional<Tensor> C3KernelRegistry::tryExecute(op op_type, const Tensor& a, const Tensor& b) {
    const KeyType key = makeKey(op_type, a.device(), a.shape(), b.shape());
    C3Entry entry;
    {
        std::lock_guard<std::mutex> lock(mutex_);
        auto it = entries_.find(key);
        if (it == entries_.end() || !it->second.active) return std::nullopt;
        entry = it->second;
    }
    if (a.shape() != entry.shapes.lhs_shape || b.shape() != entry.shapes.rhs_shape || !entry.kernel)
        return std::nullopt;
    try {
        const auto t0 = std::chrono::steady_clock::now();
        auto outputs = entry.kernel->execute({a, b});
        if (outputs.empty()) return std::nullopt;
        recordPerfC3SingleInvoke(
            (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t0).count());
        hit_count_.fetch_add(1, std::memory_order_relaxed);
        if (!validateOutputShape(op_type, a.device(), outputs[0], entry.shapes.out_shape)) return std::nullopt;
        return outputs[0];
    } catch (...) {
        miss_count_.fetch_add(1, std::memory_order_relaxed);
        return std::nullopt;
    }
}

std::optional<Tensor> C3KernelRegistry::tryExecuteUnary(op op_type, const Tensor& a) {
    const KeyType key = makeKey(op_type, a.device(), a.shape(), {});
    C3Entry entry;
    {
        std::lock_guard<std::mutex> lock(mutex_);
        auto it = entries_.find(key);
        if (it == entries_.end() || !it->second.active) return std::nullopt;
        entry = it->second;
    }
    if (a.shape() != entry.shapes.lhs_shape || !entry.kernel) return std::nullopt;
    try {
        auto outputs = entry.kernel->execute({a});
        if (outputs.empty()) return std::nullopt;
        hit_count_.fetch_add(1, std::memory_order_relaxed);
        if (!validateOutputShape(op_type, a.device(), outputs[0], entry.shapes.out_shape)) return std::nullopt;
        return outputs[0];
    } catch (...) {
        miss_count_.fetch_add(1, std::memory_order_relaxed);
        return std::nullopt;
    }
}

void C3KernelRegistry::installFused(std::shared_ptr<CompiledKernel> kernel, op op_type, const KernelShapeInfo& shapes) {
    if (!kernel) return;
    std::lock_guard<std::mutex> lock(mutex_);
    const std::string key = makeFusedKey(op_type, shapes);
    auto it = fused_entries_.find(key);
    if (it != fused_entries_.end() && it->second.active && it->second.kernel &&
        kernel->optLevel() <= it->second.kernel->optLevel())
        return;
    fused_entries_[key] = FusedEntry{std::move(kernel), shapes, true};
    install_count_.fetch_add(1, std::memory_order_release);
}

std::optional<Tensor> C3KernelRegistry::tryExecuteFused(op op_type, const std::vector<Tensor>& inputs) {
    if (inputs.empty()) return std::nullopt;
    FusedEntry entry;
    bool found = false;
    {
        std::lock_guard<std::mutex> lock(mutex_);
        for (auto& kv : fused_entries_) {
            const FusedEntry& e = kv.second;
            if (!e.active || e.shapes.lhs_shape != inputs[0].shape()) continue;
            if (kv.first != makeFusedKey(op_type, e.shapes)) continue;
            entry = e;
            found = true;
            break;
        }
    }
    if (!found) return std::nullopt;
    Tensor out = executeFusedWithInputs(entry.kernel, inputs, entry.shapes);
    if (!out.defined()) return std::nullopt;
    return out;
}

Tensor C3KernelRegistry::executeFusedWithInputs(std::shared_ptr<CompiledKernel> kernel,
                                                const std::vector<Tensor>& inputs, const KernelShapeInfo& shapes) {
    (void)shapes;
    if (!kernel || inputs.empty()) return Tensor();
    try {
        const auto t0 = std::chrono::steady_clock::now();
        auto outputs = kernel->execute(inputs);
        recordPerfRegionMatch(
            (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t0).count());
        if (outputs.empty()) return Tensor();
        fused_hit_count_.fetch_add(1, std::memory_order_relaxed);
        return outputs[0];
    } catch (const std::exception& e) {
        c3log(ErrorLevel::WARN, std::string("C3KernelRegistry::executeFusedWithInputs: kernel execute failed: ") +
                                    e.what() + ", falling back to eager.");
        return Tensor();
    }
}

void C3KernelRegistry::uninstallFused(op op_type, const KernelShapeInfo& shapes) {
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = fused_entries_.find(makeFusedKey(op_type, shapes));
    if (it != fused_entries_.end()) {
        fused_entries_.erase(it);
        uninstall_count_.fetch_add(1, std::memory_order_release);
    }
}

size_t C3KernelRegistry::fusedEntryCount() const {
    std::lock_guard<std::mutex> lock(mutex_);
    return fused_entries_.size();
}

std::optional<std::pair<std::shared_ptr<CompiledKernel>, KernelShapeInfo>> C3KernelRegistry::findFusedKernelForSequence(
    const std::vector<op>& op_seq, DeviceType dev, const std::vector<size_t>& first_input_shape) {
    (void)dev;
    if (op_seq.empty()) return std::nullopt;
    std::string pattern;
    static const char* kNames[] = {"Add", "Sub", "Neg", "Mul", "Div", "MatMul", "Dot", "Cos", "Sin", "ReLU",
                                   "Tanh", "Sigmoid", "GELU", "LReLU", "Log", "Exp", "Abs", "Softmax", "Min",
                                   "Max", "MSE", "CE", "MAE", "Conv", "Pool"};
    for (size_t i = 0; i < op_seq.size(); ++i) {
        const int o = static_cast<int>(op_seq[i]);
        if (o < 0 || o >= static_cast<int>(op::kCount)) return std::nullopt;
        if (i) pattern += "+";
        pattern += kNames[o];
    }
    std::lock_guard<std::mutex> lock(mutex_);
    for (auto& kv : fused_entries_) {
        const FusedEntry& e = kv.second;
        if (!e.active || e.shapes.fused_pattern != pattern) continue;
        if (!first_input_shape.empty() && e.shapes.lhs_shape != first_input_shape) continue;
        return std::make_pair(e.kernel, e.shapes);
    }
    return std::nullopt;
}

std::optional<std::pair<std::shared_ptr<CompiledKernel>, KernelShapeInfo>> C3KernelRegistry::findFusedKernelForFirstOp(
    op op_type, const std::vector<size_t>& input_shape, DeviceType dev) {
    (void)dev;
    static const char* kNames[] = {"Add", "Sub", "Neg", "Mul", "Div", "MatMul", "Dot", "Cos", "Sin", "ReLU",
                                   "Tanh", "Sigmoid", "GELU", "LReLU", "Log", "Exp", "Abs", "Softmax", "Min",
                                   "Max", "MSE", "CE", "MAE", "Conv", "Pool"};
    const int o = static_cast<int>(op_type);
    if (o < 0 || o >= static_cast<int>(op::kCount)) return std::nullopt;
    const std::string prefix = std::string(kNames[o]) + "+";
    std::lock_guard<std::mutex> lock(mutex_);
    for (auto& kv : fused_entries_) {
        const FusedEntry& e = kv.second;
        if (!e.active || e.shapes.fused_pattern.rfind(prefix, 0) != 0) continue;
        if (e.shapes.lhs_shape != input_shape) continue;
        return std::make_pair(e.kernel, e.shapes);
    }
    return std::nullopt;
}

void C3KernelRegistry::installBackward(const std::string& backward_key, std::shared_ptr<CompiledKernel> kernel,
                                       const std::vector<size_t>& grad_shape, const std::vector<size_t>& out_shape,
                                       const std::vector<size_t>& fwd_input_map, size_t num_inputs) {
    if (!kernel) return;
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = backward_entries_.find(backward_key);
    if (it != backward_entries_.end() && it->second.active && it->second.kernel &&
        kernel->optLevel() <= it->second.kernel->optLevel())
        return;
    BackwardEntry e;
    e.kernel = std::move(kernel);
    e.grad_shape = grad_shape;
    e.out_shape = out_shape;
    e.fwd_input_map = fwd_input_map;
    e.num_inputs = num_inputs;
    e.active = true;
    backward_entries_[backward_key] = std::move(e);
    install_count_.fetch_add(1, std::memory_order_release);
}

std::optional<std::vector<Tensor>> C3KernelRegistry::tryExecuteBackward(const std::string& backward_key,
                                                                        const Tensor& grad,
                                                                        const std::vector<Tensor>& forward_inputs) {
    BackwardEntry entry;
    {
        std::lock_guard<std::mutex> lock(mutex_);
        auto it = backward_entries_.find(backward_key);
        if (it == backward_entries_.end() || !it->second.active) return std::nullopt;
        entry = it->second;
    }
    if (grad.shape() != entry.grad_shape) return std::nullopt;
    try {
        std::vector<Tensor> inputs;
        inputs.reserve(1 + entry.fwd_input_map.size());
        inputs.push_back(grad);
        for (size_t idx : entry.fwd_input_map) {
            if (idx >= forward_inputs.size()) return std::nullopt;
            inputs.push_back(forward_inputs[idx]);
        }
        if (inputs.size() != entry.num_inputs) return std::nullopt;
        auto outputs = entry.kernel->execute(inputs);
        if (outputs.empty()) return std::nullopt;
        backward_hit_count_.fetch_add(1, std::memory_order_relaxed);
        return outputs;
    } catch (...) {
        return std::nullopt;
    }
}

bool C3KernelRegistry::hasBackwardKey(const std::string& backward_key) {
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = backward_entries_.find(backward_key);
    return it != backward_entries_.end() && it->second.active;
}

void C3KernelRegistry::recordPerfRegionDispatch(uint64_t ns) {
    region_dispatch_ns_.fetch_add(ns, std::memory_order_relaxed);
    region_dispatch_count_.fetch_add(1, std::memory_order_relaxed);
}
void C3KernelRegistry::recordPerfRegionMatch(uint64_t ns) {
    region_match_ns_.fetch_add(ns, std::memory_order_relaxed);
    region_match_count_.fetch_add(1, std::memory_order_relaxed);
}
void C3KernelRegistry::recordPerfC3SingleInvoke(uint64_t ns) {
    c3_single_invoke_ns_.fetch_add(ns, std::memory_order_relaxed);
    c3_single_invoke_count_.fetch_add(1, std::memory_order_relaxed);
}
void C3KernelRegistry::recordPerfEagerInvoke(uint64_t ns) {
    eager_invoke_ns_.fetch_add(ns, std::memory_order_relaxed);
    eager_invoke_count_.fetch_add(1, std::memory_order_relaxed);
}

C3KernelRegistry::Stats C3KernelRegistry::getStats() const {
    Stats s;
    s.install_count = install_count_.load(std::memory_order_acquire);
    s.uninstall_count = uninstall_count_.load(std::memory_order_acquire);
    s.hit_count = hit_count_.load(std::memory_order_acquire);
    s.miss_count = miss_count_.load(std::memory_order_acquire);
    s.bypass_count = bypass_count_.load(std::memory_order_acquire);
    s.fused_hit_count = fused_hit_count_.load(std::memory_order_acquire);
    s.backward_hit_count = backward_hit_count_.load(std::memory_order_acquire);
    s.region_dispatch_ns = region_dispatch_ns_.load(std::memory_order_relaxed);
    s.region_match_ns = region_match_ns_.load(std::memory_order_relaxed);
    s.c3_single_invoke_ns = c3_single_invoke_ns_.load(std::memory_order_relaxed);
    s.eager_invoke_ns = eager_invoke_ns_.load(std::memory_order_relaxed);
    s.region_dispatch_count = region_dispatch_count_.load(std::memory_order_relaxed);
    s.region_match_count = region_match_count_.load(std::memory_order_relaxed);
    s.c3_single_invoke_count = c3_single_invoke_count_.load(std::memory_order_relaxed);
    s.eager_invoke_count = eager_invoke_count_.load(std::memory_order_relaxed);
    s.region_cost_rejected_count = region_cost_rejected_count_.load(std::memory_order_relaxed);
    std::lock_guard<std::mutex> lock(mutex_);
    s.active_entries = entries_.size();
    s.fused_entries = fused_entries_.size();
    s.backward_entries = backward_entries_.size();
    return s;
}

}  // namespace c3
}  // namespace ct
