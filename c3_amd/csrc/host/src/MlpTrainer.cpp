// MlpTrainer.cpp -- MLP train step over C3's dispatch flow (the host
// framework's role: op trace, region dispatch, autograd order, CE, SGD).
#include "C3/MlpTrainer.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <stdexcept>
#include <string>

#include "C3/C3BackwardCapture.h"
#include "C3/C3Config.h"
#include "C3/C3Engine.h"
#include "C3/C3HotPathManager.h"
#include "C3/C3KernelRegistry.h"
#include "C3/RegionFusion.h"
#include "C3/RollingHash.h"
#include "c3hip.h"

namespace ct {
namespace c3 {
namespace {

int hipDtype(DType t) { return t == DType::kBFloat16 ? C3HIP_BF16 : C3HIP_F32; }

void check(int rc, const char* what) {
    if (rc != C3HIP_OK) throw std::runtime_error(std::string(what) + ": " + c3hip_last_error());
}

Tensor devTensor(std::vector<size_t> shape, DType dt) { return Tensor(ShapeTag{}, std::move(shape), dt, DeviceType::kHIP); }

void hipCheck(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace

MlpTrainer::MlpTrainer(std::vector<size_t> dims, size_t batch, DType dt) : dims_(std::move(dims)), batch_(batch), dt_(dt) {
    if (dims_.size() < 2) throw std::invalid_argument("MlpTrainer: need at least one layer");
    if (batch_ == 0) throw std::invalid_argument("MlpTrainer: batch must be positive");
    for (size_t d : dims_)
        if (d == 0) throw std::invalid_argument("MlpTrainer: zero-width layer");
    const size_t L = dims_.size() - 1;
    for (size_t l = 0; l < L; ++l) {
        W_.push_back(devTensor({dims_[l], dims_[l + 1]}, dt_));
        b_.push_back(devTensor({dims_[l + 1]}, DType::kFloat));
        // Zero until the caller writes its initial values (c3mlp_params).
        if (hipMemset(W_.back().data(), 0, W_.back().nbytes()) != hipSuccess ||
            hipMemset(b_.back().data(), 0, b_.back().nbytes()) != hipSuccess)
            throw std::runtime_error("MlpTrainer: hipMemset of the parameters failed");
        trace_.push_back(op::MatMul);
        trace_.push_back(op::Add);
        if (l + 1 < L) trace_.push_back(op::ReLU);
    }
    prefix_ = RollingHash::computePrefixHashes(trace_);
    acts_.resize(L + 1);
}

Tensor MlpTrainer::layerForwardEager(size_t l, const Tensor& A, bool relu) {
    const size_t M = A.shape()[0], K = dims_[l], N = dims_[l + 1];
    void* st = getCurrentStream();
    auto& H = C3HotPathManager::instance();
    auto& R = C3KernelRegistry::getInstance();
    const Tensor& W = W_[l];
    const Tensor& b = b_[l];
    auto record = [&] {
        H.recordCall(op::MatMul, DeviceType::kHIP, A.shape(), W.shape(), true, dt_);
        H.recordCall(op::Add, DeviceType::kHIP, {M, N}, b.shape(), true, dt_);
        if (relu) H.recordCall(op::ReLU, DeviceType::kHIP, {M, N}, {}, true, dt_);
    };
    if (dt_ == DType::kBFloat16) {
        // No bf16 single elementwise kernels: the layer runs as one eager Linear.
        Tensor Y = make({M, N}, dt_);
        check(c3hip_linear_fwd(C3HIP_BF16, A.data(), W.data(), b.data_ptr<float>(), Y.data(), (int64_t)M, (int64_t)K,
                               (int64_t)N, relu ? C3HIP_ACT_RELU : C3HIP_ACT_NONE, st),
              "eager linear");
        stats_.eager_ops++;
        record();
        return Y;
    }
    // MatMul, Add (bias row broadcast), ReLU: registry first, eager on a miss.
    Tensor T;
    if (auto r = singleKernelEnabled() ? R.tryExecute(op::MatMul, A, W) : std::nullopt) {
        T = *r;
        stats_.single_op_hits++;
    } else {
        T = make({M, N}, dt_);
        check(c3hip_matmul(C3HIP_F32, A.data(), W.data(), T.data(), (int64_t)M, (int64_t)K, (int64_t)N, 0, 0, st),
              "eager matmul");
        stats_.eager_ops++;
    }
    Tensor Z;
    if (auto r = singleKernelEnabled() ? R.tryExecute(op::Add, T, b) : std::nullopt) {
        Z = *r;
        stats_.single_op_hits++;
    } else {
        Z = make({M, N}, dt_);
        check(c3hip_elementwise(C3HIP_EW_ADD, C3HIP_F32, T.data(), b.data(), 0.f, Z.data(), (int64_t)(M * N),
                                (int64_t)N, st),
              "eager add");
        stats_.eager_ops++;
    }
    if (!relu) {
        record();
        return Z;
    }
    Tensor Y;
    if (auto r = singleKernelEnabled() ? R.tryExecuteUnary(op::ReLU, Z) : std::nullopt) {
        Y = *r;
        stats_.single_op_hits++;
    } else {
        Y = make({M, N}, dt_);
        check(c3hip_elementwise(C3HIP_EW_RELU, C3HIP_F32, Z.data(), nullptr, 0.f, Y.data(), (int64_t)(M * N), 0, st),
              "eager relu");
        stats_.eager_ops++;
    }
    record();
    return Y;
}

Tensor MlpTrainer::forward(const Tensor& X) {
    if (X.shape() != std::vector<size_t>{batch_, dims_[0]} || X.dtype() != dt_ || X.device() != DeviceType::kHIP)
        throw std::invalid_argument("MlpTrainer::forward: X must be a HIP tensor [batch, in] of the trainer's dtype");
    const size_t L = numLayers();
    acts_[0] = X;
    step_region_hits_ = 0;
    auto& RF = RegionFusionRegistry::getInstance();
    size_t pos = 0;
    for (size_t l = 0; l < L; ++l) {
        const bool relu = l + 1 < L;
        const size_t layer_ops = relu ? 3 : 2;
        const Tensor& A = acts_[l];
        bool done = false;
        // Longest installed region starting at this layer's MatMul; only one
        // that covers exactly this layer's ops has known external inputs.
        if (regionFusionEnabled() && RF.installedCountNoLock() > 0 && RF.mayMatchAsLastOp(trace_[pos + layer_ops - 1])) {
            auto m = RF.matchFromPosition(prefix_, pos, A.shape(), {A.shape(), W_[l].shape()});
            if (m && m->len == layer_ops && m->kernel) {
                try {
                    acts_[l + 1] = hold(C3KernelRegistry::getInstance().executeFusedWithInputs(
                        m->kernel, {A, W_[l], b_[l]}, KernelShapeInfo{}));
                    done = acts_[l + 1].defined();
                } catch (const std::exception& e) {
                    c3log(ErrorLevel::WARN, std::string("region kernel failed, running eagerly: ") + e.what());
                }
                if (done) {
                    stats_.region_hits++;
                    step_region_hits_++;
                }
            }
        }
        if (!done) acts_[l + 1] = layerForwardEager(l, A, relu);
        pos += layer_ops;
    }
    return acts_[L];
}

float MlpTrainer::step(const Tensor& X, const void* labels, float lr, bool want_loss) {
    if (!labels) throw std::invalid_argument("MlpTrainer::step: labels is null");
    void* st = getCurrentStream();
    const size_t L = numLayers();
    const size_t C = dims_.back();
    Tensor logits = forward(X);
    Tensor rows = make({batch_}, DType::kFloat);
    Tensor g = make({batch_, C}, dt_);
    check(c3hip_softmax_ce(hipDtype(dt_), logits.data(), static_cast<const int32_t*>(labels), rows.data_ptr<float>(),
                           g.data(), (int64_t)batch_, (int64_t)C, st),
          "softmax_ce");
    step_bwd_hits_ = 0;
    if (keep_grads_) {
        kept_g_.assign(L, Tensor());
        kept_dW_.assign(L, Tensor());
        kept_db_.assign(L, Tensor());
    } else {
        kept_g_.clear();
        kept_dW_.clear();
        kept_db_.clear();
    }
    auto& B = C3BackwardCapture::getInstance();
    // Gradients of every layer; the SGD step runs once after the backward
    // (every dA is formed from the old weights either way, so the result is
    // the same as updating each layer as soon as its gradients exist).
    std::vector<Tensor> dWs(L), dbs(L);
    for (size_t i = L; i-- > 0;) {
        const bool relu = i + 1 < L;
        // The first layer's input is the data batch: no gradient for it.
        const bool input_grad = i > 0;
        const Tensor& A = acts_[i];
        const Tensor& Y = acts_[i + 1];
        Tensor dA, dW, db;
        auto r = B.tryExecuteLinearBackward(g, {A, W_[i], Y}, relu, input_grad);
        if (r && r->size() == 3) {
            dA = hold((*r)[0]);
            dW = hold((*r)[1]);
            db = hold((*r)[2]);
            stats_.backward_hits++;
            step_bwd_hits_++;
        } else {
            const size_t M = A.shape()[0], K = dims_[i], N = dims_[i + 1];
            if (input_grad) dA = make({M, K}, dt_);
            dW = make({K, N}, DType::kFloat);
            db = make({N}, DType::kFloat);
            check(c3hip_linear_bwd(hipDtype(dt_), A.data(), W_[i].data(), Y.data(), g.data(),
                                   input_grad ? dA.data() : nullptr, dW.data_ptr<float>(), db.data_ptr<float>(),
                                   (int64_t)M, (int64_t)K, (int64_t)N, relu ? C3HIP_ACT_RELU : C3HIP_ACT_NONE, st),
                  "eager linear backward");
            stats_.backward_misses++;
        }
        if (keep_grads_) {
            kept_g_[i] = g;
            kept_dW_[i] = dW;
            kept_db_[i] = db;
        }
        dWs[i] = dW;
        dbs[i] = db;
        g = dA;
    }
    // fp32 weights: weights and biases share one launch (up to 16 tensors);
    // bf16 weights: one launch for the weights, one for the fp32 biases.
    // The same per-element update either way.
    std::vector<void*> sw, sb;
    std::vector<const float*> sgw, sgb;
    std::vector<int64_t> snw, snb;
    for (size_t i = 0; i < L; ++i) {
        sw.push_back(W_[i].data());
        sgw.push_back(dWs[i].data_ptr<float>());
        snw.push_back((int64_t)W_[i].numel());
        auto& bp = dt_ == DType::kFloat ? sw : sb;
        auto& bg = dt_ == DType::kFloat ? sgw : sgb;
        auto& bn = dt_ == DType::kFloat ? snw : snb;
        bp.push_back(b_[i].data());
        bg.push_back(dbs[i].data_ptr<float>());
        bn.push_back((int64_t)b_[i].numel());
    }
    auto sgd = [&](int dtype, std::vector<void*>& w, std::vector<const float*>& g, std::vector<int64_t>& n,
                   const char* what) {
        for (size_t i0 = 0; i0 < w.size(); i0 += C3HIP_SGD_MAX_TENSORS) {
            const size_t k = std::min<size_t>(C3HIP_SGD_MAX_TENSORS, w.size() - i0);
            check(c3hip_sgd_update_multi(dtype, (int)k, w.data() + i0, g.data() + i0, n.data() + i0, lr, st), what);
        }
    };
    sgd(hipDtype(dt_), sw, sgw, snw, "sgd W");
    if (!sb.empty()) sgd(C3HIP_F32, sb, sgb, snb, "sgd b");
    stats_.steps++;
    // Every ReLU layer as a region (MatMul+Add alone is below the cost
    // model's threshold and stays unfused) and every backward fused.
    last_fully_dispatched_ = step_region_hits_ == L - 1 && step_bwd_hits_ == L;
    if (!want_loss) return std::nanf("");
    Tensor sum = make({1}, DType::kFloat);
    check(c3hip_sum_reduce(rows.data_ptr<float>(), sum.data_ptr<float>(), 1, (int64_t)batch_, 1, st), "sum_reduce");
    float h = 0.f;
    if (hipMemcpyAsync(&h, sum.data(), 4, hipMemcpyDeviceToHost, (hipStream_t)st) != hipSuccess ||
        hipStreamSynchronize((hipStream_t)st) != hipSuccess)
        throw std::runtime_error("loss readback failed");
    return h / (float)batch_;
}

Tensor MlpTrainer::make(std::vector<size_t> shape, DType dt) { return hold(devTensor(std::move(shape), dt)); }

Tensor MlpTrainer::hold(Tensor t) {
    if (retain_ && t.defined()) retained_.push_back(t);
    return t;
}

void MlpTrainer::captureStep(const Tensor& X, const void* labels, float lr) {
    hipStream_t st = (hipStream_t)getCurrentStream();
    if (st == nullptr) throw std::invalid_argument("MlpTrainer::captureStep: the default stream cannot be captured");
    releaseGraph();
    // One step with every buffer held grows the device pool to what a step
    // needs with nothing freed, so the captured step allocates nothing new
    // (no hipMalloc may run while the stream is capturing).
    retain_ = true;
    try {
        step(X, labels, lr, false);
        hipCheck(hipStreamSynchronize(st), "hipStreamSynchronize");
        retained_.clear();
        hipCheck(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        try {
            step(X, labels, lr, false);
        } catch (...) {
            hipGraph_t g = nullptr;
            (void)hipStreamEndCapture(st, &g);
            if (g) (void)hipGraphDestroy(g);
            throw;
        }
        hipGraph_t g = nullptr;
        hipCheck(hipStreamEndCapture(st, &g), "hipStreamEndCapture");
        graph_ = g;
        hipGraphExec_t ex = nullptr;
        hipCheck(hipGraphInstantiate(&ex, g, nullptr, nullptr, 0), "hipGraphInstantiate");
        graph_exec_ = ex;
    } catch (...) {
        retain_ = false;
        retained_.clear();
        releaseGraph();
        throw;
    }
    // The captured step's buffers stay held for the graph's lifetime.
    retain_ = false;
    graph_dispatched_ = last_fully_dispatched_;
}

void MlpTrainer::replay() {
    if (!graph_exec_) throw std::logic_error("MlpTrainer::replay: no captured step");
    hipCheck(hipGraphLaunch((hipGraphExec_t)graph_exec_, (hipStream_t)getCurrentStream()), "hipGraphLaunch");
    stats_.steps++;
    stats_.graph_replays++;
}

void MlpTrainer::releaseGraph() {
    if (graph_exec_) (void)hipGraphExecDestroy((hipGraphExec_t)graph_exec_);
    if (graph_) (void)hipGraphDestroy((hipGraph_t)graph_);
    graph_exec_ = nullptr;
    graph_ = nullptr;
    retained_.clear();
}

MlpTrainer::~MlpTrainer() {
    if (graph_exec_ || graph_) {
        (void)hipDeviceSynchronize();
        releaseGraph();
    }
}

size_t MlpTrainer::warmUp(const Tensor& X, const void* labels, float lr, size_t max_steps) {
    for (size_t s = 0; s < max_steps; ++s) {
        step(X, labels, lr, false);
        if (last_fully_dispatched_) return s + 1;
        if (hipStreamSynchronize((hipStream_t)getCurrentStream()) != hipSuccess)
            throw std::runtime_error("warmUp: stream synchronisation failed");
        C3HotPathManager::instance().waitForPendingCompiles();
        C3BackwardCapture::getInstance().waitForPendingCompiles();
    }
    return max_steps;
}

}  // namespace c3
}  // namespace ct

// ---- C entry points --------------------------------------------------------

struct c3mlp {
    ct::c3::MlpTrainer trainer;
};

namespace {
thread_local std::string t_mlp_error;

template <typename F>
int guarded(F&& f) {
    t_mlp_error.clear();
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        t_mlp_error = e.what();
    } catch (...) {
        t_mlp_error = "unknown exception";
    }
    return 1;
}

ct::DType toDtype(int d) {
    if (d == C3HIP_F32) return ct::DType::kFloat;
    if (d == C3HIP_BF16) return ct::DType::kBFloat16;
    throw std::invalid_argument("unknown dtype " + std::to_string(d));
}

struct StreamScope {
    explicit StreamScope(void* s) : prev(ct::c3::getCurrentStream()) { ct::c3::setCurrentStream(s); }
    ~StreamScope() { ct::c3::setCurrentStream(prev); }
    void* prev;
};

ct::Tensor borrow(const void* p, std::vector<size_t> shape, ct::DType dt, const char* what) {
    if (!p) throw std::invalid_argument(std::string(what) + " is null");
    return ct::Tensor::fromBlob(const_cast<void*>(p), std::move(shape), dt, ct::DeviceType::kHIP);
}
}  // namespace

extern "C" {

const char* c3mlp_last_error(void) { return t_mlp_error.c_str(); }

int c3mlp_create(int dtype, const int64_t* dims, int ndims, int64_t batch, c3mlp** out) {
    return guarded([&] {
        if (!out || !dims || ndims < 2 || batch <= 0) throw std::invalid_argument("bad arguments");
        std::vector<size_t> d;
        for (int i = 0; i < ndims; ++i) {
            if (dims[i] <= 0) throw std::invalid_argument("dims must be positive");
            d.push_back((size_t)dims[i]);
        }
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) throw std::runtime_error("hipGetDevice failed");
        if (c3hip_init(dev) != C3HIP_OK) throw std::runtime_error(std::string("c3hip_init: ") + c3hip_last_error());
        *out = new c3mlp{ct::c3::MlpTrainer(d, (size_t)batch, toDtype(dtype))};
    });
}

void c3mlp_destroy(c3mlp* m) { delete m; }

int c3mlp_params(c3mlp* m, int layer, void** W, float** b) {
    return guarded([&] {
        if (!m || layer < 0 || (size_t)layer >= m->trainer.numLayers()) throw std::invalid_argument("bad layer");
        if (W) *W = m->trainer.weight(layer).data();
        if (b) *b = m->trainer.bias(layer).data_ptr<float>();
    });
}

int c3mlp_forward(c3mlp* m, const void* X, void* logits_out, void* stream) {
    return guarded([&] {
        if (!m || !logits_out) throw std::invalid_argument("null argument");
        auto& t = m->trainer;
        StreamScope ss(stream);
        ct::Tensor logits = t.forward(borrow(X, {t.batch(), t.inFeatures()}, t.dtype(), "X"));
        if (hipMemcpyAsync(logits_out, logits.data(), logits.nbytes(), hipMemcpyDeviceToDevice, (hipStream_t)stream) !=
            hipSuccess)
            throw std::runtime_error("logits copy failed");
    });
}

int c3mlp_step(c3mlp* m, const void* X, const int32_t* labels, float lr, float* loss_out, void* stream) {
    return guarded([&] {
        if (!m) throw std::invalid_argument("null trainer");
        auto& t = m->trainer;
        StreamScope ss(stream);
        const float loss = t.step(borrow(X, {t.batch(), t.inFeatures()}, t.dtype(), "X"), labels, lr, loss_out != nullptr);
        if (loss_out) *loss_out = loss;
    });
}

int c3mlp_warm_up(c3mlp* m, const void* X, const int32_t* labels, float lr, int max_steps, int* steps_run,
                  void* stream) {
    return guarded([&] {
        if (!m || max_steps < 0) throw std::invalid_argument("bad arguments");
        auto& t = m->trainer;
        StreamScope ss(stream);
        const size_t n = t.warmUp(borrow(X, {t.batch(), t.inFeatures()}, t.dtype(), "X"), labels, lr, (size_t)max_steps);
        if (steps_run) *steps_run = (int)n;
    });
}

int c3mlp_stats(c3mlp* m, int64_t* out) {
    return guarded([&] {
        if (!m || !out) throw std::invalid_argument("null argument");
        const auto& s = m->trainer.stats();
        out[0] = (int64_t)s.steps;
        out[1] = (int64_t)s.region_hits;
        out[2] = (int64_t)s.single_op_hits;
        out[3] = (int64_t)s.eager_ops;
        out[4] = (int64_t)s.backward_hits;
        out[5] = (int64_t)s.backward_misses;
        out[6] = m->trainer.lastStepFullyDispatched() ? 1 : 0;
        out[7] = (int64_t)s.graph_replays;
    });
}

int c3mlp_capture(c3mlp* m, const void* X, const int32_t* labels, float lr, void* stream) {
    return guarded([&] {
        if (!m || !labels) throw std::invalid_argument("null argument");
        if (!stream) throw std::invalid_argument("capture needs a non-default stream");
        auto& t = m->trainer;
        StreamScope ss(stream);
        t.captureStep(borrow(X, {t.batch(), t.inFeatures()}, t.dtype(), "X"), labels, lr);
    });
}

int c3mlp_replay(c3mlp* m, void* stream) {
    return guarded([&] {
        if (!m) throw std::invalid_argument("null trainer");
        StreamScope ss(stream);
        m->trainer.replay();
    });
}

int c3mlp_set_keep_gradients(c3mlp* m, int keep) {
    return guarded([&] {
        if (!m) throw std::invalid_argument("null trainer");
        m->trainer.setKeepGradients(keep != 0);
    });
}

int c3mlp_tensor(c3mlp* m, int which, int layer, void** ptr) {
    return guarded([&] {
        if (!m || !ptr || layer < 0) throw std::invalid_argument("bad arguments");
        auto& t = m->trainer;
        const size_t l = (size_t)layer;
        const ct::Tensor* x = nullptr;
        if (which == 0 && l <= t.numLayers()) x = &t.activation(l);
        else if (which >= 1 && which <= 3 && l < t.numLayers()) {
            try {
                x = which == 1 ? &t.outputGrad(l) : which == 2 ? &t.weightGrad(l) : &t.biasGrad(l);
            } catch (const std::out_of_range&) {
                throw std::invalid_argument("gradients were not kept (c3mlp_set_keep_gradients)");
            }
        } else {
            throw std::invalid_argument("bad tensor selector or layer");
        }
        if (!x->defined()) throw std::invalid_argument("tensor not computed yet");
        *ptr = x->data();
    });
}

}  // extern "C"
