// GraphMerger.h -- chaining kernels into one merged kernel (the
// "compile layer by layer, then the whole network in the background" mode of
// the reference, include/C3/GraphMerger.h:81-136, src/C3/GraphMerger.cpp).
//
// The reference merges sub-graphs into one Graph and compiles it to one CPU
// function.  Here a sub-graph is a KernelSpec (the pattern a prebuilt gfx950
// kernel covers), and the merged kernel launches the sub-kernels back to back
// on the current stream, feeding each linked output to the next sub-kernel's
// input on the device; no host round trip and no extra copies.  The merge
// rules are the reference's: links[i] joins output from_output of sub i to
// input to_input of sub i + 1 (SIZE_MAX: unconnected); the merged inputs are
// every unlinked sub input in (sub, input) order; the merged outputs are the
// last sub's outputs; a link must join equal shapes and element types.
#pragma once

#include <cstddef>
#include <memory>
#include <string>
#include <vector>

#include "C3/C3Engine.h"

namespace ct {
namespace c3 {

// Version prefix of merged cache keys (include/C3/GraphMerger.h:38).
inline constexpr const char* kMergedCacheKeyPrefix = "merged_v4_";

struct MergedSpecInfo {
    // (sub, input) of every merged input, in merged-input order.
    std::vector<std::pair<size_t, size_t>> external_inputs;
    // input_source[i][j]: SIZE_MAX if sub i's input j is a merged input, else
    // the output index of sub i - 1 that feeds it.
    std::vector<std::vector<size_t>> input_source;
};

class GraphMerger {
public:
    // "" when (subs, spec) can be merged, else the reason
    // (src/C3/GraphMerger.cpp:30-73).
    static std::string validate(const std::vector<KernelSpec>& subs, const MergeSpec& spec);
    // Input wiring of the merged kernel; throws std::invalid_argument when
    // validate fails.
    static MergedSpecInfo merge(const std::vector<KernelSpec>& subs, const MergeSpec& spec);
    // Output 0 of each sub feeds input 0 of the next.
    static MergeSpec makeSequentialSpec(const std::vector<KernelSpec>& subs);
    // Stable identity of (subs, spec) for cache keys.
    static std::string mergedCacheKey(const std::vector<KernelSpec>& subs, const MergeSpec& spec);
};

// Sub-kernels run in order with the wiring of a MergedSpecInfo.
class MergedCompiledKernel : public CompiledKernel {
public:
    MergedCompiledKernel(std::vector<std::shared_ptr<CompiledKernel>> subs, std::vector<KernelSpec> specs,
                         MergeSpec spec, std::string cache_key, int opt_level);
    std::vector<Tensor> execute(const std::vector<Tensor>& inputs) override;
    const std::string& cacheKey() const override { return key_; }
    DeviceType targetDevice() const override;
    size_t workspaceBytes() const override { return 0; }
    size_t subCount() const { return subs_.size(); }
    const std::shared_ptr<CompiledKernel>& sub(size_t i) const { return subs_[i]; }

    // Runs subs with the wiring of info (shared by the PGO interpreter tier).
    static std::vector<Tensor> run(const std::vector<KernelSpec>& specs, const MergedSpecInfo& info,
                                   const std::vector<Tensor>& inputs,
                                   const std::function<std::vector<Tensor>(size_t, const std::vector<Tensor>&)>& exec);

private:
    std::vector<std::shared_ptr<CompiledKernel>> subs_;
    std::vector<KernelSpec> specs_;
    MergedSpecInfo info_;
    std::string key_;
};

}  // namespace c3
}  // namespace ct
