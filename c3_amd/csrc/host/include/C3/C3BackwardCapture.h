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
//
// Fused backward chains (src/C3/C3BackwardCapture.cpp:874-1637): the host
// framework reports every backward node it runs (recordBackwardNode); runs of
// 2..kFusionWindowSize single-input elementwise nodes with one grad shape are
// compiled, from their first sighting, into one multi-output kernel keyed
//   "backward_fused_<ReLU+Sigmoid...>|g:<grad shape>|i:<upstream input shape>"
// (c3hip_backward_chain).  When the host reaches the chain's most downstream
// node N0, tryExecuteFusedBackward walks N0's upstream links (through up to
// three single-upstream wrapper nodes per hop), takes the longest compiled
// window, runs it once, returns N0's upstream grad and keeps the other nodes'
// grads until the host reaches those nodes (the intercept map).  The window
// bookkeeping follows the reference, including its reset of the window after
// two recorded nodes.  One deliberate difference: every node of the chain
// gets its own forward input; the reference's merged graph has no input for
// a Neg node, so a node upstream of a Neg there reads the wrong tensor.  And
// the short name of an LReLU node is "Other" here; the reference's substring
// match names it "ReLU", so an LReLU chain there can run a ReLU chain's kernel.
#pragma once

#include <atomic>
#include <deque>
#include <future>
#include <memory>
#include <mutex>
#include <optional>
#include <set>
#include <shared_mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "C3/C3Engine.h"
#include "C3/Ctools.h"

namespace ct {
namespace c3 {

// The host framework's autograd node as the chain traversal sees it: the
// reference reads ::Node through typeid(*node).name(), getUpStreamNodes() and
// getInputs() (src/C3/C3BackwardCapture.cpp:1344-1505).  typeName() is the
// short node type ("ReLU", "Sigmoid", ...; wrapper nodes any other name).
class BackwardNode {
public:
    virtual ~BackwardNode() = default;
    virtual std::string typeName() const = 0;
    virtual std::vector<std::shared_ptr<BackwardNode>> getUpStreamNodes() const = 0;
    virtual std::vector<Tensor> getInputs() const = 0;
};

class C3BackwardCapture {
public:
    static constexpr size_t kFusionWindowSize = 4;  // include/C3/C3BackwardCapture.h:390
    static constexpr int kFusionThreshold = 1;      // :391 (compile on the first sighting)
    static constexpr size_t kSkipMax = 4;           // wrapper skip bound, src/C3/C3BackwardCapture.cpp:1439

    static C3BackwardCapture& getInstance();

    void clear();
    // End of one backward pass: drops the window, the intercepted grads and
    // the miss markers (src/C3/C3BackwardCapture.cpp:1718-1730).
    void clearCallScopedState();

    // Node-level entry (src/C3/C3BackwardCapture.cpp:47-132): a single-input
    // node first tries a fused chain (as its most downstream node, or as an
    // upstream node whose grad a chain already produced), then the per-input
    // kernels below.  forward_inputs empty: node->getInputs().
    std::optional<std::vector<Tensor>> tryExecuteBackward(const BackwardNode* node, const Tensor& grad,
                                                          const std::vector<Tensor>& forward_inputs = {});
    void recordBackwardNode(const std::string& node_type, const std::vector<size_t>& grad_shape,
                            const std::vector<size_t>& input_shape, const std::vector<Tensor>& forward_inputs);
    std::optional<Tensor> tryExecuteFusedBackward(const BackwardNode* node, const Tensor& grad,
                                                  const std::vector<Tensor>& forward_inputs);
    bool tryLookupFusedBackwardKey(const Tensor& grad, const std::vector<size_t>& first_forward_input_shape,
                                   std::string& out_key);
    bool getLatestSequenceTail(std::vector<std::string>& out_types, size_t len) const;

    static bool isElementWiseBackward(const std::string& node_type);
    static std::string makeSequenceKey(const std::vector<std::string>& types);
    static bool isFusableSequence(const std::vector<std::string>& types);
    static std::string makeFusedBackwardKey(const std::string& seq_key, const std::vector<size_t>& grad_shape,
                                            const std::vector<size_t>& input_shape);
    // Spec of the fused kernel of a chain (node 0 downstream); false when a
    // node has no backward rule here (GELU, Sin, ...), dt is not fp32 or the
    // grad / input shapes are not all one shape.
    static bool buildChainSpec(const std::vector<std::string>& types,
                               const std::vector<std::vector<size_t>>& grad_shapes,
                               const std::vector<std::vector<size_t>>& input_shapes, DType dt, KernelSpec* spec);

    std::optional<std::vector<Tensor>> tryExecuteBackward(const std::string& node_type, const Tensor& grad,
                                                          const std::vector<Tensor>& forward_inputs);
    // forward_inputs = {X, W, Y}; returns {dX, dW, db}.  act: C3HIP_ACT_* of
    // the layer (relu = true is C3HIP_ACT_RELU, false no activation).
    // input_grad = false: the layer's input needs no gradient (autograd asks
    // only for dW and db, e.g. the first layer of a network on data); dX is
    // then not computed and comes back as an empty tensor, under its own key
    // ("...|fused|nodx").
    std::optional<std::vector<Tensor>> tryExecuteLinearBackward(const Tensor& grad,
                                                                const std::vector<Tensor>& forward_inputs, int act,
                                                                bool input_grad = true);
    std::optional<std::vector<Tensor>> tryExecuteLinearBackward(const Tensor& grad,
                                                                const std::vector<Tensor>& forward_inputs, bool relu,
                                                                bool input_grad = true) {
        return tryExecuteLinearBackward(grad, forward_inputs, relu ? 1 : 0, input_grad);
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
        size_t fusion_compile_count = 0;  // chain kernels submitted
        size_t fusion_hit_count = 0;      // nodes served by a chain kernel (both paths)
        size_t fusion_miss_count = 0;
    };
    Stats getStats() const;

private:
    C3BackwardCapture() = default;
    bool deviceSupported(DeviceType dev) const;
    void submit(const std::string& key, const KernelSpec& spec, const std::vector<size_t>& grad_shape,
                const std::vector<size_t>& fwd_input_map, size_t num_inputs);

    struct BackwardSequence {
        std::vector<std::string> node_types;
        std::vector<std::vector<size_t>> grad_shapes, input_shapes;
        DType dtype = DType::kFloat;
        int frequency = 0;
        bool compiling = false;
    };
    // Counts a window under its full key; compiles it at kFusionThreshold.
    void countSequence(std::vector<std::string> types, std::vector<std::vector<size_t>> gs,
                       std::vector<std::vector<size_t>> is, DType dt);
    void compileFusedBackwardAsync(const BackwardSequence& seq, const std::string& key);

    mutable std::mutex fusion_mu_;
    std::deque<std::string> recent_sequence_;
    std::deque<std::vector<size_t>> recent_grad_shapes_, recent_input_shapes_;
    std::deque<std::vector<Tensor>> recent_forward_inputs_;
    std::unordered_map<std::string, BackwardSequence> sequence_counts_;
    std::shared_mutex intercepted_mu_;
    std::unordered_map<const BackwardNode*, std::pair<std::string, Tensor>> pending_intercepted_;
    std::mutex miss_mu_;
    std::unordered_set<const BackwardNode*> miss_marker_nodes_;
    std::atomic<size_t> fusion_compiles_{0}, fusion_hits_{0}, fusion_misses_{0};

    mutable std::mutex mu_;
    std::set<std::string> in_flight_;
    std::vector<std::future<void>> futures_;
    std::atomic<size_t> hits_{0}, misses_{0}, submitted_{0}, failed_{0}, unsupported_{0};
};

}  // namespace c3
}  // namespace ct
