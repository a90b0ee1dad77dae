// C3BackwardCapture.cpp -- see include/C3/C3BackwardCapture.h.
#include "C3/C3BackwardCapture.h"

#include <numeric>
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
                                                                               int act, bool input_grad) {
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
    // Without the input gradient (a layer whose input is the data) the
    // kernel is a different one: its own key, output 0 empty.
    const std::string key = makeBaseKey(kNames[act], grad, fwd) + (input_grad ? "|fused" : "|fused|nodx");
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
    s.input_grad = input_grad;
    s.dtype = X.dtype();
    s.input_shapes = {grad.shape(), X.shape(), W.shape(), fwd[2].shape()};
    s.out_shape = X.shape();
    submit(key, s, grad.shape(), {0, 1, 2}, 4);
    return std::nullopt;
}

// ------------------------------------------------- fused backward chains --

bool C3BackwardCapture::isElementWiseBackward(const std::string& t) {
    // The single-input node types the reference admits into chains
    // (supportsNodeType there, src/C3/C3BackwardCapture.cpp:463-483).
    static const std::set<std::string> kTypes = {"ReLU", "Sigmoid", "Tanh", "Neg", "GELU", "LReLU", "Sin",
                                                 "Cos",  "Abs",     "Exp",  "Log", "Min",  "Max"};
    return kTypes.count(t) != 0;
}

std::string C3BackwardCapture::makeSequenceKey(const std::vector<std::string>& types) {
    static const std::set<std::string> kNamed = {"ReLU", "Sigmoid", "Tanh", "Neg", "Add",
                                                 "Sub",  "Mul",     "Div",  "Exp", "Log"};
    std::string key;
    for (const auto& t : types) {
        if (!key.empty()) key += "+";
        key += kNamed.count(t) ? t : std::string("Other");
    }
    return key;
}

bool C3BackwardCapture::isFusableSequence(const std::vector<std::string>& types) {
    if (types.size() < 2) return false;
    for (const auto& t : types)
        if (!isElementWiseBackward(t)) return false;
    return true;
}

std::string C3BackwardCapture::makeFusedBackwardKey(const std::string& seq_key, const std::vector<size_t>& grad_shape,
                                                    const std::vector<size_t>& input_shape) {
    std::ostringstream ss;
    ss << "backward_fused_" << seq_key << "|g:";
    for (size_t d : grad_shape) ss << d << ",";
    ss << "|i:";
    for (size_t d : input_shape) ss << d << ",";
    return ss.str();
}

bool C3BackwardCapture::buildChainSpec(const std::vector<std::string>& types,
                                       const std::vector<std::vector<size_t>>& gs,
                                       const std::vector<std::vector<size_t>>& is, DType dt, KernelSpec* spec) {
    if (types.empty() || types.size() > kFusionWindowSize || gs.size() != types.size() ||
        is.size() != types.size() || dt != DType::kFloat)
        return false;
    KernelSpec s;
    s.kind = KernelKind::BackwardChain;
    s.dtype = dt;
    const std::vector<size_t>& g = gs.front();
    for (size_t k = 0; k < types.size(); ++k) {
        if (gs[k] != g || is[k] != g) return false;  // one flat index space for every tensor
        const std::string& t = types[k];
        if (t == "ReLU") {
            s.chain.push_back(C3HIP_CHAIN_RELU);
            s.op_seq.push_back(op::ReLU);
        } else if (t == "Sigmoid") {
            s.chain.push_back(C3HIP_CHAIN_SIGMOID);
            s.op_seq.push_back(op::Sigmoid);
        } else if (t == "Tanh") {
            s.chain.push_back(C3HIP_CHAIN_TANH);
            s.op_seq.push_back(op::Tanh);
        } else if (t == "Exp") {
            s.chain.push_back(C3HIP_CHAIN_EXP);
            s.op_seq.push_back(op::Exp);
        } else if (t == "Log") {
            s.chain.push_back(C3HIP_CHAIN_LOG);
            s.op_seq.push_back(op::Log);
        } else if (t == "Neg") {
            s.chain.push_back(C3HIP_CHAIN_NEG);
            s.op_seq.push_back(op::Neg);
        } else {
            return false;  // no backward rule for this node type
        }
    }
    s.input_shapes.assign(1 + types.size(), g);
    s.out_shape = g;
    *spec = std::move(s);
    return true;
}

void C3BackwardCapture::countSequence(std::vector<std::string> types, std::vector<std::vector<size_t>> gs,
                                      std::vector<std::vector<size_t>> is, DType dt) {
    // Caller holds fusion_mu_.  Counted per (types, grad shape, upstream input
    // shape) so every shape gets its own kernel (src/C3/C3BackwardCapture.cpp:959-1004).
    const std::string key = makeFusedBackwardKey(makeSequenceKey(types), gs.front(), is.back());
    BackwardSequence& e = sequence_counts_[key];
    if (e.node_types.empty()) {
        e.node_types = std::move(types);
        e.grad_shapes = std::move(gs);
        e.input_shapes = std::move(is);
        e.dtype = dt;
    }
    e.frequency++;
    if (e.frequency >= kFusionThreshold && !e.compiling) {
        e.compiling = true;
        compileFusedBackwardAsync(e, key);
    }
}

void C3BackwardCapture::compileFusedBackwardAsync(const BackwardSequence& seq, const std::string& key) {
    KernelSpec spec;
    if (!buildChainSpec(seq.node_types, seq.grad_shapes, seq.input_shapes, seq.dtype, &spec)) {
        unsupported_++;
        return;  // as in the reference, the entry stays marked and is not retried
    }
    // Graph inputs [grad, x_0 .. x_{w-1}]: forward_inputs[k] is node k's input.
    std::vector<size_t> map(seq.node_types.size());
    std::iota(map.begin(), map.end(), size_t{0});
    fusion_compiles_++;
    submit(key, spec, seq.grad_shapes.front(), map, 1 + map.size());
}

void C3BackwardCapture::recordBackwardNode(const std::string& node_type, const std::vector<size_t>& grad_shape,
                                           const std::vector<size_t>& input_shape,
                                           const std::vector<Tensor>& forward_inputs) {
    if (!isElementWiseBackward(node_type)) return;
    if (!forward_inputs.empty() && !deviceSupported(forward_inputs[0].device())) return;
    const DType dt = forward_inputs.empty() ? DType::kFloat : forward_inputs[0].dtype();
    std::lock_guard<std::mutex> lk(fusion_mu_);
    // A full pair is counted once more (if its grad shapes agree) and the
    // window restarts, so pairs of consecutive passes do not mix
    // (src/C3/C3BackwardCapture.cpp:888-923).
    if (recent_sequence_.size() == 2) {
        std::vector<std::string> chain(recent_sequence_.begin(), recent_sequence_.end());
        std::vector<std::vector<size_t>> gs(recent_grad_shapes_.begin(), recent_grad_shapes_.end());
        std::vector<std::vector<size_t>> is(recent_input_shapes_.begin(), recent_input_shapes_.end());
        bool same = true;
        for (size_t k = 1; k < gs.size(); ++k) same = same && gs[k] == gs[0];
        if (same && isFusableSequence(chain)) countSequence(std::move(chain), std::move(gs), std::move(is), dt);
        recent_sequence_.clear();
        recent_grad_shapes_.clear();
        recent_input_shapes_.clear();
        recent_forward_inputs_.clear();
    }
    recent_sequence_.push_back(node_type);
    recent_grad_shapes_.push_back(grad_shape);
    recent_input_shapes_.push_back(input_shape);
    recent_forward_inputs_.push_back(forward_inputs);
    if (recent_sequence_.size() > kFusionWindowSize) {
        recent_sequence_.pop_front();
        recent_grad_shapes_.pop_front();
        recent_input_shapes_.pop_front();
        recent_forward_inputs_.pop_front();
    }
    // Every fusable tail window of length 2..kFusionWindowSize.
    const size_t L = recent_sequence_.size();
    for (size_t w = 2; w <= kFusionWindowSize && w <= L; ++w) {
        const size_t start = L - w;
        std::vector<std::string> types(recent_sequence_.begin() + start, recent_sequence_.end());
        if (!isFusableSequence(types)) continue;
        std::vector<std::vector<size_t>> gs(recent_grad_shapes_.begin() + start, recent_grad_shapes_.end());
        std::vector<std::vector<size_t>> is(recent_input_shapes_.begin() + start, recent_input_shapes_.end());
        countSequence(std::move(types), std::move(gs), std::move(is), dt);
    }
}

bool C3BackwardCapture::getLatestSequenceTail(std::vector<std::string>& out_types, size_t len) const {
    std::lock_guard<std::mutex> lk(fusion_mu_);
    if (recent_sequence_.size() < len) return false;
    out_types.assign(recent_sequence_.end() - (std::ptrdiff_t)len, recent_sequence_.end());
    return true;
}

bool C3BackwardCapture::tryLookupFusedBackwardKey(const Tensor& grad,
                                                  const std::vector<size_t>& first_forward_input_shape,
                                                  std::string& out_key) {
    for (size_t w = kFusionWindowSize; w >= 2; --w) {
        std::vector<std::string> types;
        if (!getLatestSequenceTail(types, w) || !isFusableSequence(types)) continue;
        const std::string key = makeFusedBackwardKey(makeSequenceKey(types), grad.sizes(), first_forward_input_shape);
        if (C3KernelRegistry::getInstance().hasBackwardKey(key)) {
            out_key = key;
            return true;
        }
    }
    return false;
}

std::optional<Tensor> C3BackwardCapture::tryExecuteFusedBackward(const BackwardNode* node, const Tensor& grad,
                                                                 const std::vector<Tensor>& forward_inputs) {
    if (!node) return std::nullopt;
    const std::string cur_type = node->typeName();
    // Path A: a chain run at a downstream node already produced this node's
    // upstream grad (src/C3/C3BackwardCapture.cpp:1349-1398).
    bool present = false;
    {
        std::shared_lock<std::shared_mutex> rl(intercepted_mu_);
        present = pending_intercepted_.count(node) != 0;
    }
    if (present) {
        std::unique_lock<std::shared_mutex> wl(intercepted_mu_);
        auto it = pending_intercepted_.find(node);
        if (it != pending_intercepted_.end()) {
            if (it->second.first == cur_type) {
                Tensor t = std::move(it->second.second);
                pending_intercepted_.erase(it);
                fusion_hits_++;
                return t;
            }
            pending_intercepted_.erase(it);  // same address, another node: stale
        }
    }
    // A node that already missed in this pass is not walked again (:1400-1410).
    {
        std::lock_guard<std::mutex> ml(miss_mu_);
        if (miss_marker_nodes_.count(node)) {
            fusion_misses_++;
            return std::nullopt;
        }
    }
    // Path B: this node is the chain's most downstream node N0 (:1412-1637).
    if (!isElementWiseBackward(cur_type)) return std::nullopt;
    std::vector<std::shared_ptr<BackwardNode>> chain_nodes{nullptr};
    std::vector<std::string> chain_types{cur_type};
    std::vector<std::vector<Tensor>> chain_inputs{forward_inputs};
    const BackwardNode* cur = node;
    for (size_t step = 1; step < kFusionWindowSize; ++step) {
        // Next elementwise node up the single-upstream links, skipping at
        // most kSkipMax - 1 wrapper nodes.
        std::shared_ptr<BackwardNode> cand;
        const BackwardNode* c = cur;
        for (size_t skips = 0; skips < kSkipMax; ++skips) {
            auto ups = c->getUpStreamNodes();
            if (ups.size() != 1 || !ups[0]) break;
            if (isElementWiseBackward(ups[0]->typeName())) {
                cand = ups[0];
                break;
            }
            c = ups[0].get();
        }
        if (!cand) break;
        auto cand_ups = cand->getUpStreamNodes();
        if (cand_ups.size() != 1 || !cand_ups[0]) break;
        auto in = cand->getInputs();
        if (in.empty() || in[0].sizes() != grad.sizes()) break;  // one shape along the whole chain
        chain_nodes.push_back(cand);
        chain_types.push_back(cand->typeName());
        chain_inputs.push_back(std::move(in));
        cur = cand.get();
    }
    // Longest compiled window first.
    std::vector<Tensor> best_inputs;
    std::string best_key;
    size_t best_w = 0;
    for (size_t w = kFusionWindowSize; w >= 2; --w) {
        if (w > chain_types.size()) continue;
        std::vector<std::string> types(chain_types.begin(), chain_types.begin() + (std::ptrdiff_t)w);
        if (!isFusableSequence(types)) continue;
        const std::vector<size_t>& up_shape = chain_inputs[w - 1].empty() ? grad.sizes() : chain_inputs[w - 1][0].sizes();
        std::string key = makeFusedBackwardKey(makeSequenceKey(types), grad.sizes(), up_shape);
        if (C3KernelRegistry::getInstance().hasBackwardKey(key)) {
            best_inputs.clear();
            for (size_t k = 0; k < w; ++k)
                if (!chain_inputs[k].empty()) best_inputs.push_back(chain_inputs[k][0]);
            best_key = std::move(key);
            best_w = w;
            break;
        }
    }
    if (best_w < 2 || best_inputs.size() != best_w) {
        std::lock_guard<std::mutex> ml(miss_mu_);
        miss_marker_nodes_.insert(node);
        if (miss_marker_nodes_.size() > 10000) miss_marker_nodes_.clear();
        fusion_misses_++;
        return std::nullopt;
    }
    auto outs = C3KernelRegistry::getInstance().tryExecuteBackward(best_key, grad, best_inputs);
    if (!outs || outs->size() != best_w) {
        fusion_misses_++;
        return std::nullopt;
    }
    {
        std::unique_lock<std::shared_mutex> wl(intercepted_mu_);
        for (size_t k = 1; k < best_w; ++k)
            pending_intercepted_[chain_nodes[k].get()] = std::make_pair(chain_types[k], (*outs)[k]);
    }
    fusion_hits_++;
    return (*outs)[0];
}

std::optional<std::vector<Tensor>> C3BackwardCapture::tryExecuteBackward(const BackwardNode* node,
                                                                         const Tensor& grad,
                                                                         const std::vector<Tensor>& forward_inputs) {
    if (!backwardFusionEnabled() || !node) return std::nullopt;
    size_t n_inputs = forward_inputs.empty() ? node->getInputs().size() : forward_inputs.size();
    if (n_inputs == 0) n_inputs = 1;
    if (n_inputs == 1) {
        auto fused = tryExecuteFusedBackward(node, grad, forward_inputs);
        if (fused) {
            hits_++;
            return std::vector<Tensor>{std::move(*fused)};
        }
    }
    return tryExecuteBackward(node->typeName(), grad, forward_inputs);
}

void C3BackwardCapture::clearCallScopedState() {
    {
        std::lock_guard<std::mutex> lk(fusion_mu_);
        recent_sequence_.clear();
        recent_grad_shapes_.clear();
        recent_input_shapes_.clear();
        recent_forward_inputs_.clear();
    }
    {
        std::unique_lock<std::shared_mutex> wl(intercepted_mu_);
        pending_intercepted_.clear();
    }
    std::lock_guard<std::mutex> ml(miss_mu_);
    miss_marker_nodes_.clear();
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
    clearCallScopedState();
    {
        std::lock_guard<std::mutex> lk(fusion_mu_);
        sequence_counts_.clear();
    }
    hits_ = misses_ = submitted_ = failed_ = unsupported_ = 0;
    fusion_compiles_ = fusion_hits_ = fusion_misses_ = 0;
}

C3BackwardCapture::Stats C3BackwardCapture::getStats() const {
    Stats s;
    s.cache_hit_count = hits_.load();
    s.cache_miss_count = misses_.load();
    s.compiles_submitted = submitted_.load();
    s.compiles_failed = failed_.load();
    s.unsupported = unsupported_.load();
    s.fusion_compile_count = fusion_compiles_.load();
    s.fusion_hit_count = fusion_hits_.load();
    s.fusion_miss_count = fusion_misses_.load();
    return s;
}

}  // namespace c3
}  // namespace ct
