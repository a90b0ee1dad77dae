// GraphMerger.cpp -- see include/C3/GraphMerger.h.
#include "C3/GraphMerger.h"

#include <sstream>
#include <stdexcept>

namespace ct {
namespace c3 {

namespace {

std::string descString(const std::vector<size_t>& shape, DType dt) {
    return shapeToString(shape) + " dtype=" + std::to_string(static_cast<int>(dt));
}

}  // namespace

std::string GraphMerger::validate(const std::vector<KernelSpec>& subs, const MergeSpec& spec) {
    if (subs.empty()) return "GraphMerger: no sub-kernels";
    if (spec.links.size() != subs.size() - 1) {
        std::ostringstream ss;
        ss << "GraphMerger: links count (" << spec.links.size() << ") must be sub count - 1 (" << subs.size() - 1
           << ")";
        return ss.str();
    }
    for (size_t i = 0; i + 1 < subs.size(); ++i) {
        const MergeLink& l = spec.links[i];
        const auto outs = subs[i].outputDescs();
        if (l.from_output >= outs.size()) {
            std::ostringstream ss;
            ss << "GraphMerger: link[" << i << "].from_output (" << l.from_output << ") out of range (sub " << i
               << " has " << outs.size() << " outputs)";
            return ss.str();
        }
        if (l.to_input == SIZE_MAX) continue;
        if (l.to_input >= subs[i + 1].input_shapes.size()) {
            std::ostringstream ss;
            ss << "GraphMerger: link[" << i << "].to_input (" << l.to_input << ") out of range (sub " << i + 1
               << " has " << subs[i + 1].input_shapes.size() << " inputs)";
            return ss.str();
        }
        const auto& out = outs[l.from_output];
        const auto& in_shape = subs[i + 1].input_shapes[l.to_input];
        const DType in_dt = subs[i + 1].inputDtype(l.to_input);
        if (out.first != in_shape || out.second != in_dt) {
            std::ostringstream ss;
            ss << "GraphMerger: link[" << i << "] desc mismatch: out=" << descString(out.first, out.second)
               << " vs in=" << descString(in_shape, in_dt);
            return ss.str();
        }
    }
    return "";
}

MergedSpecInfo GraphMerger::merge(const std::vector<KernelSpec>& subs, const MergeSpec& spec) {
    const std::string err = validate(subs, spec);
    if (!err.empty()) throw std::invalid_argument(err);
    MergedSpecInfo info;
    info.input_source.resize(subs.size());
    for (size_t i = 0; i < subs.size(); ++i) info.input_source[i].assign(subs[i].input_shapes.size(), SIZE_MAX);
    for (size_t i = 0; i + 1 < subs.size(); ++i)
        if (spec.links[i].to_input != SIZE_MAX) info.input_source[i + 1][spec.links[i].to_input] = spec.links[i].from_output;
    for (size_t i = 0; i < subs.size(); ++i)
        for (size_t j = 0; j < subs[i].input_shapes.size(); ++j)
            if (info.input_source[i][j] == SIZE_MAX) info.external_inputs.push_back({i, j});
    return info;
}

MergeSpec GraphMerger::makeSequentialSpec(const std::vector<KernelSpec>& subs) {
    MergeSpec spec;
    for (size_t i = 0; i + 1 < subs.size(); ++i) spec.links.push_back({0, 0});
    return spec;
}

std::string GraphMerger::mergedCacheKey(const std::vector<KernelSpec>& subs, const MergeSpec& spec) {
    if (spec.links.size() != (subs.empty() ? 0 : subs.size() - 1)) return std::string(kMergedCacheKeyPrefix) + "invalid";
    std::ostringstream ss;
    ss << kMergedCacheKeyPrefix << subs.size();
    for (size_t i = 0; i < subs.size(); ++i) {
        ss << "|G" << i << "{" << subs[i].toString() << "}";
        if (i + 1 < subs.size()) {
            const MergeLink& l = spec.links[i];
            ss << "|L" << l.from_output << ">";
            if (l.to_input == SIZE_MAX)
                ss << "out";
            else
                ss << l.to_input;
        }
    }
    return ss.str();
}

MergedCompiledKernel::MergedCompiledKernel(std::vector<std::shared_ptr<CompiledKernel>> subs,
                                           std::vector<KernelSpec> specs, MergeSpec spec, std::string cache_key,
                                           int opt_level)
    : subs_(std::move(subs)), specs_(std::move(specs)), key_(std::move(cache_key)) {
    opt_level_ = opt_level;
    info_ = GraphMerger::merge(specs_, spec);
    if (subs_.size() != specs_.size()) throw std::invalid_argument("MergedCompiledKernel: kernel / spec count differ");
}

DeviceType MergedCompiledKernel::targetDevice() const {
    return subs_.empty() ? DeviceType::kHIP : subs_.front()->targetDevice();
}

std::vector<Tensor> MergedCompiledKernel::run(
    const std::vector<KernelSpec>& specs, const MergedSpecInfo& info, const std::vector<Tensor>& inputs,
    const std::function<std::vector<Tensor>(size_t, const std::vector<Tensor>&)>& exec) {
    if (inputs.size() != info.external_inputs.size())
        throw std::runtime_error("merged kernel: expected " + std::to_string(info.external_inputs.size()) +
                                 " inputs, got " + std::to_string(inputs.size()));
    std::vector<Tensor> prev;
    size_t next_in = 0;
    for (size_t i = 0; i < specs.size(); ++i) {
        std::vector<Tensor> in(specs[i].input_shapes.size());
        for (size_t j = 0; j < in.size(); ++j) {
            const size_t src = info.input_source[i][j];
            if (src == SIZE_MAX) {
                in[j] = inputs[next_in++];
            } else {
                if (src >= prev.size()) throw std::runtime_error("merged kernel: sub-kernel output missing");
                in[j] = prev[src];
            }
        }
        prev = exec(i, in);
    }
    return prev;
}

std::vector<Tensor> MergedCompiledKernel::execute(const std::vector<Tensor>& inputs) {
    return run(specs_, info_, inputs,
               [this](size_t i, const std::vector<Tensor>& in) { return subs_[i]->execute(in); });
}

}  // namespace c3
}  // namespace ct
