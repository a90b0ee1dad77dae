// HipCompiledKernel.h -- the CompiledKernel of this backend: one KernelSpec,
// executed on HIP device tensors through the C ABI of include/c3hip.h.
#pragma once

#include "C3/C3Engine.h"

namespace ct {
namespace c3 {

class HipCompiledKernel : public CompiledKernel {
public:
    HipCompiledKernel(KernelSpec spec, int opt_level, std::string cache_key);
    std::vector<Tensor> execute(const std::vector<Tensor>& inputs) override;
    const std::string& cacheKey() const override { return key_; }
    DeviceType targetDevice() const override { return DeviceType::kHIP; }
    size_t workspaceBytes() const override { return 0; }
    std::optional<std::vector<size_t>> outShape() const override;
    const KernelSpec& spec() const { return spec_; }

private:
    KernelSpec spec_;
    std::string key_;
};

}  // namespace c3
}  // namespace ct
