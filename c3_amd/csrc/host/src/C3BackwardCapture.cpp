// C3BackwardCapture.cpp -- see include/C3/C3BackwardCapture.h.
#include "C3/C3BackwardCapture.h"

#include <sstream>

#include "C3/C3Config.h"
#include "C3/C3KernelRegistry.h"
#include "c3hip.h"

namespace ct {
namespace c3 {

C3BackwardCapture& C3BackwardCapture::getInstance() {
    static C3BackwardCapture c;
    return c;
}

bool C3BackwardCapture::supportsNodeType(const std::string& t) {
    return t == "ReLU" || t == "Add" || t == "MatMul" || t == "Sigmoid" || t == "Tanh" || t == "Exp" || t == "Log" ||
           t == "Neg" || t == "Sub" || t == "Mul" || t == "Div";
}

bool C3BackwardCapture::deviceSupported(DeviceType dev) const {
    return dev == DeviceType::kHIP || C3Engine::getInstance().hasFactoryForTest();
}

std::string C3BackwardCapture::makeBaseKey(const std::string& node_type, const Tensor& grad,
                                           const std::vector<Tensor>& forward_inputs) {
    std::ostringstream ss;
    ss << node_type << "|grad:";
    for (size_t s : grad.sizes()) ss << s << ",";
    ss << "|inputs:";
    for (const auto& t : forward_inputs)
        for (size_t s : t.sizes()) ss << s << ",";
    return ss.str();
}

bool C3BackwardCapture::buildBackwardSpecForInput(const std::string& node_type, const std::vector<size_t>& g,
                                                  const std::vector<std::vector<size_t>>& in, DType dt, size_t i,
                                                  KernelSpec* spec, std::vector<size_t>* map, size_t* num_inputs) {
    KernelSpec s;
    s.dtype = dt;
    map->clear();
    if (node_type == "ReLU") {
        if (i != 0 || in.size() != 1 || in[0] != g || dt != DType::kFloat) return false;
        s.kind = KernelKind::ReLUBackward;
        s.op_seq = {op::ReLU};
        s.input_shapes = {g, in[0]};
        s.out_shape = g;
        *map = {0};
        *num_inputs = 2;
    } else if (node_type == "Add") {
        if (i >= in.size() || in.size() != 2) return false;
        s.op_seq = {op::Add};
        s.input_shapes = {g};
        *num_inputs = 1;
        if (in[i] == g) {
            s.kind = KernelKind::AddBackwardLhs;
            s.out_shape = g;
        } else if (g.size() == 2 && in[i].size() == 1 && in[i][0] == g[1] && dt == DType::kFloat) {
            s.kind = KernelKind::SumReduce;  // bias row broadcast over the rows: reduce axis 0
            s.axis = 0;
            s.out_shape = in[i];
        } else {
            return false;
        }
    } else if (node_type == "MatMul") {
        if (in.size() != 2 || g.size() != 2 || in[0].size() != 2 || in[1].size() != 2) return false;
        s.op_seq = {op::MatMul};
        if (i == 0) {
            s.kind = KernelKind::MatMulBackwardA;  // grad . B^T
            s.input_shapes = {g, in[1]};
            s.out_shape = in[0];
            *map = {1};
        } else if (i == 1) {
            s.kind = KernelKind::MatMulBackwardB;  // A^T . grad
            s.input_shapes = {g, in[0]};
            s.out_shape = in[1];
            *map = {0};
        } else {
            return false;
        }
        *num_inputs = 2;
    } else if (node_type == "Sigmoid" || node_type == "Tanh" || node_type == "Exp") {
        // [grad, x] -> f'(x) * grad with the reference's graph (x = forward_inputs[0]).
        if (i != 0 || in.size() != 1 || in[0] != g || dt != DType::kFloat) return false;
        s.kind = KernelKind::UnaryBackward;
        s.op_seq = {node_type == "Sigmoid" ? op::Sigmoid : node_type == "Tanh" ? op::Tanh : op::Exp};
        s.ew_op = node_type == "Sigmoid" ? C3HIP_EW_SIGMOID_BWD : node_type == "Tanh" ? C3HIP_EW_TANH_BWD : C3HIP_EW_EXP_BWD;
        s.input_shapes = {g, in[0]};
        s.out_shape = g;
        *map = {0};
        *num_inputs = 2;
    } else if (node_type == "Log") {
        // grad / x  [grad, x]  (buildLogBackwardGraph)
        if (i != 0 || in.size() != 1 || in[0] != g || dt != DType::kFloat) return false;
        s.kind = KernelKind::Elementwise;
        s.op_seq = {op::Log};
        s.ew_op = C3HIP_EW_DIV;
        s.input_shapes = {g, in[0]};
        s.out_shape = g;
        *map = {0};
        *num_inputs = 2;
    } else if (node_type == "Neg" || node_type == "Sub") {
        // Neg: -grad; Sub: in:0 grad, in:1 -grad  [grad]  (buildNegBackwardGraph, buildSubBackwardGraph)
        if (dt != DType::kFloat) return false;
        if (node_type == "Neg" ? (i != 0 || in.size() != 1 || in[0] != g)
                               : (in.size() != 2 || i >= 2 || in[i] != g))
            return false;
        s.op_seq = {node_type == "Neg" ? op::Neg : op::Sub};
        s.input_shapes = {g};
        s.out_shape = g;
        *num_inputs = 1;
        if (node_type == "Sub" && i == 0) {
            s.kind = KernelKind::AddBackwardLhs;
        } else {
            s.kind = KernelKind::Elementwise;
            s.ew_op = C3HIP_EW_NEG;
        }
    } else if (node_type == "Mul" || node_type == "Div") {
        // Mul: in:0 grad * B [grad, B], in:1 A * grad [grad, A]; Div: in:0 grad / B [grad, B],
        // in:1 -((A / (B*B)) * grad) [grad, A, B]  (buildMulBackwardGraph, buildDivBackwardGraph).
        // Broadcast operands would need a reduction: not compiled (eager).
        if (in.size() != 2 || i >= 2 || in[0] != g || in[1] != g || dt != DType::kFloat) return false;
        const bool div = node_type == "Div";
        s.op_seq = {div ? op::Div : op::Mul};
        s.out_shape = g;
        if (div && i == 1) {
            s.kind = KernelKind::DivBackwardB;
            s.input_shapes = {g, in[0], in[1]};
            *map = {0, 1};
            *num_inputs = 3;
        } else {
            s.kind = KernelKind::Elementwise;
            s.ew_op = div ? C3HIP_EW_DIV : C3HIP_EW_MUL;
            s.input_shapes = {g, in[1 - i]};
            *map = {1 - i};
            *num_inputs = 2;
        }
    } else {
        return false;
    }
    *spec = s;
    return true;
}

void C3BackwardCapture::submit(const std::string& key, const KernelSpec& spec, const std::vector<size_t>& grad_shape,
                               const std::vector<size_t>& fwd_input_map, size_t num_inputs) {
    {
        std::lock_guard<std::mutex> lk(mu_);
        if (!in_flight_.insert(key).second) return;  // already compiling
    }
    submitted_++;
    auto fut = std::async(std::launch::async, [this, key, spec, grad_shape, fwd_input_map, num_inputs]() {
        CompileOptions opts;
        opts.opt_level = 3;
        auto kernel = C3Engine::getInstance().compile(spec, opts);
        if (kernel)
            C3KernelRegistry::getInstance().installBackward(key, kernel, grad_shape, spec.out_shape, fwd_input_map,
                                                            num_inputs);
        else
            failed_++;
        std::lock_guard<std::mutex> lk(mu_);
        in_flight_.erase(key);
    });
    std::lock_guard<std::mutex> lk(mu_);
    futures_.push_back(std::move(fut));
}

std::optional<std::vector<Tensor>> C3BackwardCapture::tryExecuteBackward(const std::string& node_type,
                                                                         const Tensor& grad,
                                                                         const std::vector<Tensor>& forward_inputs) {
    if (!backwardFusionEnabled()) return std::nullopt;
    if (!supportsNodeType(node_type) || !deviceSupported(grad.device())) {
        unsupported_++;
        return std::nullopt;
    }
    const size_t n_inputs = forward_inputs.empty() ? 1 : forward_inputs.size();
    const std::string base = makeBaseKey(node_type, grad, forward_inputs);
    std::vector<std::vector<size_t>> shapes;
    for (const auto& t : forward_inputs) shapes.push_back(t.shape());
    std::vector<Tensor> out;
    out.reserve(n_inputs);
    bool missed = false;
    for (size_t i = 0; i < n_inputs; ++i) {
        const std::string key = base + "|in:" + std::to_string(i);
        auto r = C3KernelRegistry::getInstance().tryExecuteBackward(key, grad, forward_inputs);
        if (r && !r->empty()) {
            out.push_back(std::move(r->at(0)));
            continue;
        }
        missed = true;
        KernelSpec spec;
        std::vector<size_t> map;
        size_t num = 1;
        if (buildBackwardSpecForInput(node_type, grad.shape(), shapes, grad.dtype(), i, &spec, &map, &num))
            submit(key, spec, grad.shape(), map, num);
        else
            unsupported_++;
    }
    if (missed) {
        misses_++;
        return std::nullopt;
    }
    hits_++;
    return out;
}

std::optional<std::vector<Tensor>> C3BackwardCapture::tryExecuteLinearBackward(const Tensor& grad,
                                                                               const std::vector<Tensor>& fwd,
                                                                               int act) {
    if (!backwardFusionEnabled()) return std::nullopt;
    if (fwd.size() != 3 || !deviceSupported(grad.device())) {
        unsupported_++;
        return std::nullopt;
    }
    if (act < C3HIP_ACT_NONE || act > C3HIP_ACT_TANH) {
        unsupported_++;
        return std::nullopt;
    }
    static const char* const kNames[] = {"Linear", "Linear+ReLU", "Linear+Sigmoid", "Linear+Tanh"};
    const std::string key = makeBaseKey(kNames[act], grad, fwd) + "|fused";
    // Graph inputs [dY, X, W, Y]: forward_inputs {X, W, Y} in order.
    auto r = C3KernelRegistry::getInstance().tryExecuteBackward(key, grad, fwd);
    if (r && r->size() == 3) {
        hits_++;
        return r;
    }
    misses_++;
    const Tensor &X = fwd[0], &W = fwd[1];
    if (X.shape().size() != 2 || W.shape().size() != 2 || grad.shape().size() != 2) {
        unsupported_++;
        return std::nullopt;
    }
    KernelSpec s;
    s.kind = KernelKind::LinearBwd;
    s.op_seq = {op::MatMul, op::Add};
    if (act == C3HIP_ACT_RELU) s.op_seq.push_back(op::ReLU);
    if (act == C3HIP_ACT_SIGMOID) s.op_seq.push_back(op::Sigmoid);
    if (act == C3HIP_ACT_TANH) s.op_seq.push_back(op::Tanh);
    s.act = act;
    s.dtype = X.dtype();
    s.input_shapes = {grad.shape(), X.shape(), W.shape(), fwd[2].shape()};
    s.out_shape = X.shape();
    submit(key, s, grad.shape(), {0, 1, 2}, 4);
    return std::nullopt;
}

void C3BackwardCapture::waitForPendingCompiles() {
    std::vector<std::future<void>> fs;
    {
        std::lock_guard<std::mutex> lk(mu_);
        fs.swap(futures_);
    }
    for (auto& f : fs)
        if (f.valid()) f.wait();
}

void C3BackwardCapture::clear() {
    waitForPendingCompiles();
    hits_ = misses_ = submitted_ = failed_ = unsupported_ = 0;
}

C3BackwardCapture::Stats C3BackwardCapture::getStats() const {
    Stats s;
    s.cache_hit_count = hits_.load();
    s.cache_miss_count = misses_.load();
    s.compiles_submitted = submitted_.load();
    s.compiles_failed = failed_.load();
    s.unsupported = unsupported_.load();
    return s;
}

}  // namespace c3
}  // namespace ct
