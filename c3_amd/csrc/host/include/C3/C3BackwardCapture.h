// C3BackwardCapture.h -- per-node backward kernels looked up in the registry.
//
// Follows the reference (src/C3/C3BackwardCapture.cpp:47-132, :248-363):
// for a node of type T with forward inputs x_0..x_{n-1} and upstream grad,
// input i's gradient kernel is keyed
//   "T|grad:d0,d1,|inputs:a0,a1,b0,|in:i"
// and dispatched through C3KernelRegistry::tryExecuteBackward; if any input
// misses, its kernel is compiled in the background and the whole node falls
// back to eager this time.  Rules (graph inputs after grad in brackets):
//   ReLU   in:0  (x > 0 ? 1 : 0) * grad          [x]     (:501-528)
//   Add    in:i  grad, or grad summed over the broadcast rows when x_i is a
//                bias row (SumReduce axis 0)      []      (:618-644, :1641-1700)
//   MatMul in:0  grad . B^T                       [B]     (:681-708)
//          in:1  A^T . grad                       [A]     (:709-723)
//   Sigmoid in:0 s = 1/(1+exp(-x)); grad*(s*(1-s)) [x]    (:530-567)
//   Tanh   in:0  t via exp; grad * (1 - t*t)      [x]     (:569-616)
//   Exp    in:0  exp(x) * grad                    [x]     (:823-849)
//   Log    in:0  grad / x                         [x]     (:851-872)
//   Neg    in:0  -grad                            []      (:725-741)
//   Sub    in:0  grad; in:1 -grad                 []      (:743-770)
//   Mul    in:0  grad * B [B]; in:1 A * grad [A]  (buildMulBackwardGraph)
//   Div    in:0  grad / B [B]; in:1 -((A/(B*B))*grad) [A, B] (buildDivBackwardGraph)
// Mul/Sub/Div with broadcast operands are not compiled (the host runs eager).
// The reference never compiles Add's identity input (so Add backward, db
// included, always falls back to eager) and respawns a compile on every
// miss; here the identity is an installed no-copy kernel and a key is
// compiled at most once at a time.  The node type is passed as a string
// (the host framework's autograd Node is not part of this build).
//
// tryExecuteLinearBackward is the fused backward of a whole MatMul+Add(+act)
// layer -- the activation's derivative from Y, dX, dW and db in
// c3hip_linear_bwd -- keyed "Linear[+ReLU|+Sigmoid|+Tanh]|grad:...|inputs:...|fused".
#pragma once

#include <atomic>
#include <future>
#include <mutex>
#include <optional>
#include <set>
#include <string>
#include <vector>

#include "C3/C3Engine.h"
#include "C3/Ctools.h"

namespace ct {
namespace c3 {

class C3BackwardCapture {
public:
    static C3BackwardCapture& getInstance();

    void clear();
    void clearCallScopedState() {}

    std::optional<std::vector<Tensor>> tryExecuteBackward(const std::string& node_type, const Tensor& grad,
                                                          const std::vector<Tensor>& forward_inputs);
    // forward_inputs = {X, W, Y}; returns {dX, dW, db}.  act: C3HIP_ACT_* of
    // the layer (relu = true is C3HIP_ACT_RELU, false no activation).
    std::optional<std::vector<Tensor>> tryExecuteLinearBackward(const Tensor& grad,
                                                                const std::vector<Tensor>& forward_inputs, int act);
    std::optional<std::vector<Tensor>> tryExecuteLinearBackward(const Tensor& grad,
                                                                const std::vector<Tensor>& forward_inputs, bool relu) {
        return tryExecuteLinearBackward(grad, forward_inputs, relu ? 1 : 0);
    }

    static bool supportsNodeType(const std::string& node_type);
    static std::string makeBaseKey(const std::string& node_type, const Tensor& grad,
                                   const std::vector<Tensor>& forward_inputs);
    // Spec + registry metadata of the kernel for input i (false: no rule).
    static bool buildBackwardSpecForInput(const std::string& node_type, const std::vector<size_t>& grad_shape,
                                          const std::vector<std::vector<size_t>>& input_shapes, DType dt, size_t i,
                                          KernelSpec* spec, std::vector<size_t>* fwd_input_map, size_t* num_inputs);

    void waitForPendingCompiles();

    struct Stats {
        size_t cache_hit_count = 0;
        size_t cache_miss_count = 0;
        size_t compiles_submitted = 0;
        size_t compiles_failed = 0;
        size_t unsupported = 0;
    };
    Stats getStats() const;

private:
    C3BackwardCapture() = default;
    bool deviceSupported(DeviceType dev) const;
    void submit(const std::string& key, const KernelSpec& spec, const std::vector<size_t>& grad_shape,
                const std::vector<size_t>& fwd_input_map, size_t num_inputs);

    mutable std::mutex mu_;
    std::set<std::string> in_flight_;
    std::vector<std::future<void>> futures_;
    std::atomic<size_t> hits_{0}, misses_{0}, submitted_{0}, failed_{0}, unsupported_{0};
};

}  // namespace c3
}  // namespace ct
