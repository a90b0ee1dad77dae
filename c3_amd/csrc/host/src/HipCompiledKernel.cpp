// HipCompiledKernel.cpp -- CompiledKernel whose execute() launches the gfx950
// kernels through the C ABI (include/c3hip.h) on device-resident tensors.
//
// Replaces the reference's CPU wrappers ConcreteCompiledKernel::execute
// (src/C3/C3Engine.cpp:457-522, single ops) and
// MultiNodeCompiledKernel::execute (:145-235, fused regions): inputs are
// borrowed, outputs are allocated here (callee-allocated, as in the
// reference) from the device caching pool, and no host copies are made.
#include "C3/HipCompiledKernel.h"

#include <initializer_list>

#include <stdexcept>

#include "c3hip.h"

namespace ct {
namespace c3 {
namespace {

thread_local void* t_stream = nullptr;

int hipDtype(DType t) { return t == DType::kBFloat16 ? C3HIP_BF16 : C3HIP_F32; }

void check(int rc, const char* what) {
    if (rc != C3HIP_OK) throw std::runtime_error(std::string(what) + ": " + c3hip_last_error());
}

void requireDevice(const Tensor& t, const char* what) {
    if (!t.defined()) throw std::runtime_error(std::string(what) + ": undefined tensor");
    if (t.device() != DeviceType::kHIP) throw std::runtime_error(std::string(what) + ": tensor is not on a HIP device");
}

// Forces the spec's GEMM tile on this thread for the duration of one launch.
struct TileGuard {
    explicit TileGuard(const KernelSpec& s) : dt(hipDtype(s.dtype)), on(!s.tile.empty()) {
        if (on) check(c3hip_set_gemm_tile(dt, s.tile.c_str()), "c3hip_set_gemm_tile");
    }
    ~TileGuard() {
        if (on) (void)c3hip_set_gemm_tile(dt, nullptr);
    }
    int dt;
    bool on;
};

}  // namespace

void setCurrentStream(void* stream) { t_stream = stream; }
void* getCurrentStream() { return t_stream; }

HipCompiledKernel::HipCompiledKernel(KernelSpec spec, int opt_level, std::string cache_key)
    : spec_(std::move(spec)), key_(std::move(cache_key)) {
    opt_level_ = opt_level;
}

std::optional<std::vector<size_t>> HipCompiledKernel::outShape() const {
    if (spec_.out_shape.empty()) return std::nullopt;
    return spec_.out_shape;
}

std::vector<Tensor> HipCompiledKernel::execute(const std::vector<Tensor>& in) {
    const KernelSpec& s = spec_;
    auto need = [&](size_t n) {
        if (in.size() != n)
            throw std::runtime_error("HipCompiledKernel: expected " + std::to_string(n) + " inputs, got " +
                                     std::to_string(in.size()));
        for (size_t i = 0; i < n; ++i) requireDevice(in[i], "HipCompiledKernel input");
        if (!s.input_shapes.empty()) {
            for (size_t i = 0; i < n && i < s.input_shapes.size(); ++i)
                if (!s.input_shapes[i].empty() && in[i].shape() != s.input_shapes[i])
                    throw std::runtime_error("HipCompiledKernel: input " + std::to_string(i) + " shape " +
                                             shapeToString(in[i].shape()) + " != compiled " +
                                             shapeToString(s.input_shapes[i]));
        }
    };
    // GEMM kinds read every operand with the spec's element type (registry
    // keys do not carry the dtype, so a kernel can be reached with other
    // operands): a mismatch throws, and the registry falls back to eager.
    auto sameDtype = [&](std::initializer_list<size_t> idx, const char* what) {
        for (size_t i : idx) {
            if (in[i].dtype() != s.dtype)
                throw std::runtime_error(std::string(what) + ": input " + std::to_string(i) + " is " +
                                         (in[i].dtype() == DType::kBFloat16 ? "bf16" : "fp32") + ", kernel compiled for " +
                                         (s.dtype == DType::kBFloat16 ? "bf16" : "fp32"));
            if (in[i].shape().size() != 2) throw std::runtime_error(std::string(what) + ": operands must be 2-D");
        }
    };
    void* st = t_stream;
    TileGuard tile_guard(s);
    switch (s.kind) {
        case KernelKind::Elementwise: {
            const bool binary = s.ew_op == C3HIP_EW_ADD || s.ew_op == C3HIP_EW_SUB || s.ew_op == C3HIP_EW_MUL ||
                                s.ew_op == C3HIP_EW_DIV || s.ew_op == C3HIP_EW_RELU_BWD ||
                                s.ew_op == C3HIP_EW_SIGMOID_BWD || s.ew_op == C3HIP_EW_TANH_BWD ||
                                s.ew_op == C3HIP_EW_EXP_BWD;
            need(binary ? 2 : 1);
            const Tensor& a = in[0];
            if (a.dtype() != DType::kFloat) throw std::runtime_error("elementwise ops take fp32");
            int64_t bmod = 0;
            const void* bp = nullptr;
            if (binary) {
                const Tensor& b = in[1];
                if (b.dtype() != DType::kFloat) throw std::runtime_error("elementwise ops take fp32");
                if (b.numel() != a.numel()) {
                    if (b.numel() == 0 || a.numel() % b.numel() != 0)
                        throw std::runtime_error("elementwise: rhs of " + shapeToString(b.shape()) +
                                                 " does not broadcast to " + shapeToString(a.shape()));
                    bmod = (int64_t)b.numel();
                }
                bp = b.data();
            }
            Tensor out(ShapeTag{}, a.shape(), DType::kFloat, DeviceType::kHIP);
            check(c3hip_elementwise(s.ew_op, C3HIP_F32, a.data(), bp, s.alpha, out.data(), (int64_t)a.numel(), bmod,
                                    st),
                  "c3hip_elementwise");
            return {out};
        }
        case KernelKind::MatMul: {
            need(2);
            sameDtype({0, 1}, "matmul");
            const Tensor &A = in[0], &B = in[1];
            const size_t M = s.transA ? A.shape()[1] : A.shape()[0], K = s.transA ? A.shape()[0] : A.shape()[1];
            const size_t KB = s.transB ? B.shape()[1] : B.shape()[0], N = s.transB ? B.shape()[0] : B.shape()[1];
            if (K != KB) throw std::runtime_error("matmul: inner dimensions differ");
            Tensor C(ShapeTag{}, {M, N}, A.dtype(), DeviceType::kHIP);
            check(c3hip_matmul(hipDtype(A.dtype()), A.data(), B.data(), C.data(), (int64_t)M, (int64_t)K, (int64_t)N,
                               s.transA, s.transB, st),
                  "c3hip_matmul");
            return {C};
        }
        case KernelKind::LinearFwd: {
            // [X, W, b] for MatMul+Add+act, [X, W] for MatMul+act.
            const bool has_bias = s.input_shapes.size() != 2;
            need(has_bias ? 3 : 2);
            sameDtype({0, 1}, "linear");
            const Tensor &X = in[0], &W = in[1];
            const size_t M = X.shape()[0], K = X.shape()[1], N = W.shape()[1];
            if (W.shape()[0] != K || (has_bias && (in[2].numel() != N || in[2].dtype() != DType::kFloat)))
                throw std::runtime_error("linear: shapes of X, W, b do not agree");
            Tensor Y(ShapeTag{}, {M, N}, X.dtype(), DeviceType::kHIP);
            check(c3hip_linear_fwd(hipDtype(X.dtype()), X.data(), W.data(), has_bias ? in[2].data_ptr<float>() : nullptr,
                                   Y.data(), (int64_t)M, (int64_t)K, (int64_t)N, s.act, st),
                  "c3hip_linear_fwd");
            return {Y};
        }
        case KernelKind::ReLUBackward: {
            need(2);  // [grad, x]
            const Tensor &g = in[0], &x = in[1];
            if (g.shape() != x.shape() || g.dtype() != DType::kFloat || x.dtype() != DType::kFloat)
                throw std::runtime_error("relu backward: grad and input differ in shape or are not fp32");
            Tensor out(ShapeTag{}, g.shape(), DType::kFloat, DeviceType::kHIP);
            check(c3hip_elementwise(C3HIP_EW_RELU_BWD, C3HIP_F32, x.data(), g.data(), 0.0f, out.data(),
                                    (int64_t)g.numel(), 0, st),
                  "c3hip_elementwise(relu_bwd)");
            return {out};
        }
        case KernelKind::UnaryBackward: {
            need(2);  // [grad, x] -> ew_op(x, grad)
            const Tensor &g = in[0], &x = in[1];
            if (g.shape() != x.shape() || g.dtype() != DType::kFloat || x.dtype() != DType::kFloat)
                throw std::runtime_error("unary backward: grad and input differ in shape or are not fp32");
            Tensor out(ShapeTag{}, g.shape(), DType::kFloat, DeviceType::kHIP);
            check(c3hip_elementwise(s.ew_op, C3HIP_F32, x.data(), g.data(), 0.0f, out.data(), (int64_t)g.numel(), 0, st),
                  "c3hip_elementwise(backward)");
            return {out};
        }
        case KernelKind::DivBackwardB: {
            need(3);  // [grad, A, B] -> -((A / (B*B)) * grad)
            const Tensor &g = in[0], &a = in[1], &b = in[2];
            if (g.shape() != a.shape() || g.shape() != b.shape() || g.dtype() != DType::kFloat ||
                a.dtype() != DType::kFloat || b.dtype() != DType::kFloat)
                throw std::runtime_error("div backward: operands differ in shape or are not fp32");
            Tensor out(ShapeTag{}, g.shape(), DType::kFloat, DeviceType::kHIP);
            check(c3hip_elementwise3(C3HIP_EW3_DIV_BWD_B, C3HIP_F32, a.data(), b.data(), g.data(), out.data(),
                                     (int64_t)g.numel(), st),
                  "c3hip_elementwise3");
            return {out};
        }
        case KernelKind::AddBackwardLhs: {
            need(1);
            return {in[0]};
        }
        case KernelKind::SumReduce: {
            need(1);
            const Tensor& g = in[0];
            if (g.dtype() != DType::kFloat || g.shape().size() != 2) throw std::runtime_error("sum_reduce takes fp32 2-D");
            const size_t M = g.shape()[0], N = g.shape()[1];
            Tensor out(ShapeTag{}, {s.axis == 0 ? N : M}, DType::kFloat, DeviceType::kHIP);
            check(c3hip_sum_reduce(g.data_ptr<float>(), out.data_ptr<float>(), (int64_t)M, (int64_t)N, s.axis, st),
                  "c3hip_sum_reduce");
            return {out};
        }
        case KernelKind::MatMulBackwardA: {
            need(2);  // [grad(M,N), B(K,N)] -> grad . B^T (M,K)
            sameDtype({0, 1}, "matmul backward A");
            const Tensor &g = in[0], &B = in[1];
            const size_t M = g.shape()[0], N = g.shape()[1], K = B.shape()[0];
            if (B.shape()[1] != N) throw std::runtime_error("matmul backward A: shapes do not agree");
            Tensor out(ShapeTag{}, {M, K}, g.dtype(), DeviceType::kHIP);
            check(c3hip_matmul(hipDtype(g.dtype()), g.data(), B.data(), out.data(), (int64_t)M, (int64_t)N, (int64_t)K,
                               0, 1, st),
                  "c3hip_matmul(grad.B^T)");
            return {out};
        }
        case KernelKind::MatMulBackwardB: {
            need(2);  // [grad(M,N), A(M,K)] -> A^T . grad (K,N)
            sameDtype({0, 1}, "matmul backward B");
            const Tensor &g = in[0], &A = in[1];
            const size_t M = g.shape()[0], N = g.shape()[1], K = A.shape()[1];
            if (A.shape()[0] != M) throw std::runtime_error("matmul backward B: shapes do not agree");
            Tensor out(ShapeTag{}, {K, N}, g.dtype(), DeviceType::kHIP);
            check(c3hip_matmul(hipDtype(g.dtype()), A.data(), g.data(), out.data(), (int64_t)K, (int64_t)M, (int64_t)N,
                               1, 0, st),
                  "c3hip_matmul(A^T.grad)");
            return {out};
        }
        case KernelKind::LinearBwd: {
            need(4);  // [dY, X, W, Y] -> [dX, dW, db]; dX empty when the spec asks for no input gradient
            sameDtype({0, 1, 2, 3}, "linear backward");
            const Tensor &dY = in[0], &X = in[1], &W = in[2], &Y = in[3];
            const size_t M = X.shape()[0], K = X.shape()[1], N = W.shape()[1];
            if (W.shape()[0] != K || dY.shape() != std::vector<size_t>{M, N} || Y.shape() != dY.shape())
                throw std::runtime_error("linear backward: shapes of dY, X, W, Y do not agree");
            Tensor dX = s.input_grad ? Tensor(ShapeTag{}, {M, K}, X.dtype(), DeviceType::kHIP) : Tensor();
            Tensor dW(ShapeTag{}, {K, N}, DType::kFloat, DeviceType::kHIP);
            Tensor db(ShapeTag{}, {N}, DType::kFloat, DeviceType::kHIP);
            check(c3hip_linear_bwd(hipDtype(X.dtype()), X.data(), W.data(), Y.data(), dY.data(),
                                   s.input_grad ? dX.data() : nullptr, dW.data_ptr<float>(), db.data_ptr<float>(),
                                   (int64_t)M, (int64_t)K, (int64_t)N, s.act, st),
                  "c3hip_linear_bwd");
            return {dX, dW, db};
        }
        case KernelKind::BackwardChain: {
            // [grad, x_0..x_{w-1}] -> [g_1..g_w], every tensor of grad's shape.
            const size_t w = s.chain.size();
            if (w == 0 || w > C3HIP_CHAIN_MAX_NODES) throw std::runtime_error("backward chain: bad node count");
            need(1 + w);
            const Tensor& g = in[0];
            std::vector<const void*> xs(w);
            std::vector<void*> outs(w);
            std::vector<Tensor> res;
            res.reserve(w);
            for (size_t k = 0; k < w; ++k) {
                const Tensor& x = in[1 + k];
                if (x.shape() != g.shape() || x.dtype() != DType::kFloat || g.dtype() != DType::kFloat)
                    throw std::runtime_error("backward chain: inputs differ in shape from grad or are not fp32");
                xs[k] = x.data();
                res.emplace_back(ShapeTag{}, g.shape(), DType::kFloat, DeviceType::kHIP);
                outs[k] = res.back().data();
            }
            check(c3hip_backward_chain(C3HIP_F32, g.data(), xs.data(), s.chain.data(), (int)w, outs.data(),
                                       (int64_t)g.numel(), st),
                  "c3hip_backward_chain");
            return res;
        }
    }
    throw std::runtime_error("HipCompiledKernel: unknown kernel kind");
}

}  // namespace c3
}  // namespace ct
