// MlpTrainer.h -- the host framework's side of an MLP train step, run through
// C3's dispatch flow on HIP device tensors.
//
// In the reference this role belongs to the CTorch scheduler and autograd
// engine (not part of the repository; their calls into C3 are evidenced at
// include/C3/C3KernelRegistry.h:241-252, include/C3/RegionFusion.h:91-105,
// include/C3/C3BackwardCapture.h:197-203).  One step of a stack of Linear
// layers (ReLU after every layer but the last) is:
//   forward   the op trace [MatMul, Add, ReLU]* [MatMul, Add] is walked with
//             RollingHash prefix hashes; at each position the longest
//             installed region (RegionFusionRegistry::matchFromPosition, keyed
//             with the first input's shape) runs as one fused kernel, else the
//             single op runs through C3KernelRegistry::tryExecute, else
//             eagerly.  Every op dispatched is reported to C3HotPathManager in
//             autograd scope, which compiles and installs the region kernels
//             and hot single ops in the background;
//   loss      softmax cross-entropy of the logits (the host framework's CE op);
//   backward  last layer first, C3BackwardCapture::tryExecuteLinearBackward
//             (ReLU mask, dX, dW, db fused), else the eager layer backward;
//   update    SGD on every W and b (W in the step's dtype, b fp32).
// Eager ops are the backend's plain kernels (what the host framework would
// run itself).  bf16 has no single elementwise kernels, so an unmatched bf16
// layer runs eagerly as one Linear (matmul + bias + act) call.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "C3/Ctools.h"

namespace ct {
namespace c3 {

struct MlpStepStats {
    size_t steps = 0;
    size_t region_hits = 0;       // layers run by an installed region kernel
    size_t single_op_hits = 0;    // single ops run by an installed registry kernel
    size_t eager_ops = 0;         // forward ops (or bf16 layers) run eagerly
    size_t backward_hits = 0;     // layer backwards run by an installed fused kernel
    size_t backward_misses = 0;   // layer backwards run eagerly
    size_t graph_replays = 0;     // steps run by replaying the captured graph
};

class MlpTrainer {
public:
    // dims = {in, h1, ..., out}; batch rows per step.  Parameters are
    // allocated on the current HIP device; W[l] is [dims[l], dims[l+1]]
    // (row-major, [in, out]) in dt, b[l] is fp32 [dims[l+1]].
    MlpTrainer(std::vector<size_t> dims, size_t batch, DType dt);
    ~MlpTrainer();
    MlpTrainer(const MlpTrainer&) = delete;
    MlpTrainer& operator=(const MlpTrainer&) = delete;

    size_t numLayers() const { return W_.size(); }
    Tensor& weight(size_t l) { return W_.at(l); }
    Tensor& bias(size_t l) { return b_.at(l); }
    DType dtype() const { return dt_; }
    size_t batch() const { return batch_; }
    size_t inFeatures() const { return dims_.front(); }

    // Forward through the dispatch flow; returns the logits [batch, out].
    Tensor forward(const Tensor& X);
    // One train step.  labels: int32 device buffer of `batch` entries.
    // Returns the mean loss when want_loss (synchronises the stream), else NaN.
    float step(const Tensor& X, const void* labels, float lr, bool want_loss);
    // Run steps until every layer's forward region (where the cost model
    // activates one) and fused backward are installed, waiting for the
    // background compiles between steps.  Returns the number of steps run.
    size_t warmUp(const Tensor& X, const void* labels, float lr, size_t max_steps = 16);
    // True when the last step dispatched every ReLU layer as a region and
    // every layer backward as a fused kernel.
    bool lastStepFullyDispatched() const { return last_fully_dispatched_; }

    // Record one train step (with learning rate lr, inputs X and labels at
    // their current addresses) as a HIP graph on the current stream, which
    // must not be the default stream; replay() then runs that step again with
    // one launch: the same kernels the dispatch flow chose, on the same
    // buffers (the captured step's intermediates stay allocated).  Call after
    // warmUp so that every dispatch hits an installed kernel and no compile
    // or allocation happens during the capture.  The caller refreshes X and
    // the labels in place between replays.
    void captureStep(const Tensor& X, const void* labels, float lr);
    void replay();
    bool hasGraph() const { return graph_exec_ != nullptr; }

    const MlpStepStats& stats() const { return stats_; }

    // Keep the last step's gradients for inspection (off by default: holding
    // them keeps their memory out of the pool between steps).
    void setKeepGradients(bool keep) { keep_grads_ = keep; }
    // acts(0) = X, acts(l + 1) = layer l's output (ReLU applied) of the last forward.
    const Tensor& activation(size_t l) const { return acts_.at(l); }
    // With setKeepGradients(true): the gradient arriving at layer l's output
    // (for the last layer, dlogits), and layer l's dW and db.
    const Tensor& outputGrad(size_t l) const { return kept_g_.at(l); }
    const Tensor& weightGrad(size_t l) const { return kept_dW_.at(l); }
    const Tensor& biasGrad(size_t l) const { return kept_db_.at(l); }

private:
    Tensor layerForwardEager(size_t l, const Tensor& A, bool relu);
    Tensor make(std::vector<size_t> shape, DType dt);  // device tensor, held while retaining
    Tensor hold(Tensor t);                              // keep t alive while retaining
    void releaseGraph();

    std::vector<size_t> dims_;
    size_t batch_;
    DType dt_;
    std::vector<Tensor> W_, b_;
    std::vector<op> trace_;
    std::vector<uint64_t> prefix_;
    std::vector<Tensor> acts_;  // acts_[0] = X, acts_[l + 1] = layer l output
    MlpStepStats stats_;
    bool last_fully_dispatched_ = false;
    bool keep_grads_ = false;
    bool retain_ = false;
    std::vector<Tensor> retained_;
    void* graph_ = nullptr;       // hipGraph_t
    void* graph_exec_ = nullptr;  // hipGraphExec_t
    bool graph_dispatched_ = false;
    std::vector<Tensor> kept_g_, kept_dW_, kept_db_;
    size_t step_region_hits_ = 0, step_bwd_hits_ = 0;
};

}  // namespace c3
}  // namespace ct

// C entry points over MlpTrainer for non-C++ callers (Python via ctypes).
// Return 0 on success, nonzero with c3mlp_last_error() otherwise.
extern "C" {
typedef struct c3mlp c3mlp;
const char* c3mlp_last_error(void);
// dtype 0 = fp32, 1 = bf16; dims has ndims entries (>= 2).
int c3mlp_create(int dtype, const int64_t* dims, int ndims, int64_t batch, c3mlp** out);
void c3mlp_destroy(c3mlp* m);
// Device pointers of layer l's parameters (owned by the trainer).
int c3mlp_params(c3mlp* m, int layer, void** W, float** b);
// Launches go on `stream` (NULL = default stream).
int c3mlp_forward(c3mlp* m, const void* X, void* logits_out, void* stream);
int c3mlp_step(c3mlp* m, const void* X, const int32_t* labels, float lr, float* loss_out, void* stream);
int c3mlp_warm_up(c3mlp* m, const void* X, const int32_t* labels, float lr, int max_steps, int* steps_run,
                  void* stream);
// out[0..7] = steps, region_hits, single_op_hits, eager_ops, backward_hits,
// backward_misses, last step fully dispatched (0/1), graph replays.
int c3mlp_stats(c3mlp* m, int64_t* out8);
// Capture one step as a HIP graph on `stream` (not NULL), then replay it.
int c3mlp_capture(c3mlp* m, const void* X, const int32_t* labels, float lr, void* stream);
int c3mlp_replay(c3mlp* m, void* stream);
int c3mlp_set_keep_gradients(c3mlp* m, int keep);
// Device pointer of a tensor of the last step: which = 0 activation(layer)
// (layer 0..L), 1 outputGrad(layer), 2 weightGrad(layer), 3 biasGrad(layer).
int c3mlp_tensor(c3mlp* m, int which, int layer, void** ptr);
}
