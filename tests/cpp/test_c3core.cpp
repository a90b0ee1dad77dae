// test_c3core.cpp -- unit tests of the C++ dispatch layer (libc3core.so).
//
// CPU tests use host tensors and a test kernel factory (no GPU, no HIP
// calls): they pin the hash / key formulas against their closed forms and
// check the registry, region registry, cost model, JIT cache, hot-path
// manager, engine watchdog and backward capture behaviour.  Tests named gpu_*
// run the same flow on HIP device tensors and are invoked by the GPU pytest.
#include <dirent.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <thread>

#include "C3/C3BackwardCapture.h"
#include "C3/C3Cleanup.h"
#include "C3/C3Config.h"
#include "C3/C3Engine.h"
#include "C3/C3HotPathManager.h"
#include "C3/C3KernelRegistry.h"
#include "C3/FusionCostModel.h"
#include "C3/GraphMerger.h"
#include "C3/HipCompiledKernel.h"
#include "C3/PGOManager.h"
#include "C3/JITCache.h"
#include "C3/RegionFusion.h"
#include "C3/RollingHash.h"
#include "c3hip.h"
#include "testing.h"

using namespace ct;
using namespace ct::c3;

namespace {

Tensor host(std::vector<size_t> shape, std::vector<float> v) {
    Tensor t(ShapeTag{}, shape, DType::kFloat, DeviceType::kCPU);
    CHECK_EQ(t.numel(), v.size());
    std::memcpy(t.data(), v.data(), v.size() * 4);
    return t;
}

std::vector<float> vals(const Tensor& t) {
    const float* p = t.data_ptr<float>();
    return std::vector<float>(p, p + t.numel());
}

// Host implementation of a KernelSpec, used as the engine's backend in CPU
// tests.  Also counts how many kernels were built.
std::atomic<int> g_built{0};

class HostKernel : public CompiledKernel {
public:
    HostKernel(KernelSpec s, int opt) : s_(std::move(s)), key_(s_.toString()) { opt_level_ = opt; }
    const std::string& cacheKey() const override { return key_; }
    DeviceType targetDevice() const override { return DeviceType::kCPU; }
    size_t workspaceBytes() const override { return 0; }
    std::vector<Tensor> execute(const std::vector<Tensor>& in) override {
        switch (s_.kind) {
            case KernelKind::Elementwise: {
                Tensor o(ShapeTag{}, in[0].shape(), DType::kFloat, DeviceType::kCPU);
                const float* a = in[0].data_ptr<float>();
                const float* b = in.size() > 1 ? in[1].data_ptr<float>() : nullptr;
                const size_t bn = in.size() > 1 ? in[1].numel() : 1;
                float* y = o.data_ptr<float>();
                for (size_t i = 0; i < o.numel(); ++i) {
                    const float x = a[i], r = b ? b[i % bn] : 0.f;
                    switch (s_.ew_op) {
                        case C3HIP_EW_ADD: y[i] = x + r; break;
                        case C3HIP_EW_SUB: y[i] = x - r; break;
                        case C3HIP_EW_MUL: y[i] = x * r; break;
                        case C3HIP_EW_DIV: y[i] = x / r; break;
                        case C3HIP_EW_RELU: y[i] = x > 0 ? x : 0.f; break;
                        case C3HIP_EW_NEG: y[i] = -x; break;
                        default: throw std::runtime_error("op");
                    }
                }
                return {o};
            }
            case KernelKind::ReLUBackward: {
                Tensor o(ShapeTag{}, in[0].shape(), DType::kFloat, DeviceType::kCPU);
                for (size_t i = 0; i < o.numel(); ++i)
                    o.data_ptr<float>()[i] = (in[1].data_ptr<float>()[i] > 0 ? 1.f : 0.f) * in[0].data_ptr<float>()[i];
                return {o};
            }
            case KernelKind::AddBackwardLhs: return {in[0]};
            case KernelKind::BackwardChain: {
                // [grad, x_0..] -> [g_1..]: the exact rules (relu mask, log g/x, neg).
                std::vector<Tensor> outs;
                std::vector<float> g = vals(in[0]);
                for (size_t k = 0; k < s_.chain.size(); ++k) {
                    const float* x = in[1 + k].data_ptr<float>();
                    for (size_t i = 0; i < g.size(); ++i) {
                        switch (s_.chain[k]) {
                            case C3HIP_CHAIN_RELU: g[i] = (x[i] > 0 ? 1.f : 0.f) * g[i]; break;
                            case C3HIP_CHAIN_LOG: g[i] = g[i] / x[i]; break;
                            case C3HIP_CHAIN_NEG: g[i] = -g[i]; break;
                            default: throw std::runtime_error("HostKernel: chain node not implemented");
                        }
                    }
                    outs.push_back(host(in[0].shape(), g));
                }
                return outs;
            }
            case KernelKind::SumReduce: {
                const size_t M = in[0].shape()[0], N = in[0].shape()[1];
                Tensor o(ShapeTag{}, {N}, DType::kFloat, DeviceType::kCPU);
                for (size_t j = 0; j < N; ++j) {
                    float s = 0;
                    for (size_t i = 0; i < M; ++i) s += in[0].data_ptr<float>()[i * N + j];
                    o.data_ptr<float>()[j] = s;
                }
                return {o};
            }
            case KernelKind::MatMulBackwardA:
            case KernelKind::MatMulBackwardB:
            case KernelKind::MatMul:
            case KernelKind::LinearFwd: {
                // C = op(A) op(B) on small host matrices.
                const bool bwA = s_.kind == KernelKind::MatMulBackwardA, bwB = s_.kind == KernelKind::MatMulBackwardB;
                const Tensor& A = bwB ? in[1] : in[0];
                const Tensor& B = bwB ? in[0] : in[1];
                const bool tA = bwB || (s_.kind == KernelKind::MatMul && s_.transA);
                const bool tB = bwA || (s_.kind == KernelKind::MatMul && s_.transB);
                const size_t M = tA ? A.shape()[1] : A.shape()[0], K = tA ? A.shape()[0] : A.shape()[1];
                const size_t N = tB ? B.shape()[0] : B.shape()[1];
                Tensor o(ShapeTag{}, {M, N}, DType::kFloat, DeviceType::kCPU);
                for (size_t i = 0; i < M; ++i)
                    for (size_t j = 0; j < N; ++j) {
                        float acc = 0;
                        for (size_t k = 0; k < K; ++k) {
                            const float a = tA ? A.data_ptr<float>()[k * M + i] : A.data_ptr<float>()[i * K + k];
                            const float b = tB ? B.data_ptr<float>()[j * K + k] : B.data_ptr<float>()[k * N + j];
                            acc += a * b;
                        }
                        if (s_.kind == KernelKind::LinearFwd) {
                            if (in.size() > 2) acc += in[2].data_ptr<float>()[j];
                            if (s_.act == 1) acc = acc > 0 ? acc : 0.f;
                        }
                        o.data_ptr<float>()[i * N + j] = acc;
                    }
                return {o};
            }
            default: throw std::runtime_error("HostKernel: kind not implemented");
        }
    }

private:
    KernelSpec s_;
    std::string key_;
};

struct HostBackend {
    HostBackend() {
        C3Engine::getInstance().setFactoryForTest([](const KernelSpec& s, const CompileOptions& o) {
            g_built++;
            return std::make_shared<HostKernel>(s, o.opt_level);
        });
        reset();
    }
    ~HostBackend() {
        reset();
        C3Engine::getInstance().setFactoryForTest(nullptr);
    }
    static void reset() {
        C3HotPathManager::instance().waitForPendingCompiles();
        C3BackwardCapture::getInstance().clear();
        C3HotPathManager::instance().clear();
        C3KernelRegistry::getInstance().uninstallAll();
        RegionFusionRegistry::getInstance().clear();
        C3Engine::getInstance().clearCache();
        HotPathConfig cfg;
        C3HotPathManager::instance().configure(cfg);
        g_built = 0;
    }
};

// A kernel returning a fixed list (or throwing), for registry failure paths.
class ScriptedKernel : public CompiledKernel {
public:
    explicit ScriptedKernel(int opt, std::function<std::vector<Tensor>(const std::vector<Tensor>&)> f)
        : f_(std::move(f)) {
        opt_level_ = opt;
    }
    const std::string& cacheKey() const override { return key_; }
    DeviceType targetDevice() const override { return DeviceType::kCPU; }
    size_t workspaceBytes() const override { return 0; }
    std::vector<Tensor> execute(const std::vector<Tensor>& in) override { return f_(in); }

private:
    std::function<std::vector<Tensor>(const std::vector<Tensor>&)> f_;
    std::string key_ = "scripted";
};

std::string tmpdir() {
    char tmpl[] = "/tmp/c3core_test_XXXXXX";
    const char* d = mkdtemp(tmpl);
    CHECK(d != nullptr);
    return d;
}

}  // namespace

// ------------------------------------------------------------------ hashes --
TEST(rolling_hash_closed_forms) {
    auto p = RollingHash::computePrefixHashes({op::MatMul, op::Add, op::ReLU});
    CHECK(p == (std::vector<uint64_t>{0, 13, 1705, 223384}));
    CHECK_EQ(RollingHash::hashSequence({op::MatMul, op::Add, op::Sigmoid}), 223392ull);
    CHECK_EQ(RollingHash::hashSequence({op::MatMul, op::ReLU}), 1732ull);
    CHECK_EQ(RollingHash::hashSequence({op::MatMul, op::Sigmoid}), 1740ull);
    CHECK_EQ(RollingHash::hashSequence({op::Add, op::ReLU}), 291ull);
    // Sub-range hash equals the hash of the sub-sequence.
    auto q = RollingHash::computePrefixHashes({op::Neg, op::MatMul, op::Add, op::ReLU, op::Mul});
    CHECK_EQ(RollingHash::getSubHash(q, 1, 3), 223384ull);
    CHECK_EQ(RollingHash::getSubHash(q, 0, 0), 5ull);
    CHECK_EQ(RollingHash::getOpCode(op::CE), 79ull);
    CHECK_EQ(RollingHash::getOpCode(op::kCount), 101ull);
}

TEST(rolling_hash_wraps_mod_2_64) {
    // 40 MatMuls: the polynomial exceeds 2^64; sub-hashes of equal windows agree.
    std::vector<op> seq(40, op::MatMul);
    auto p = RollingHash::computePrefixHashes(seq);
    CHECK_EQ(RollingHash::getSubHash(p, 3, 30), RollingHash::getSubHash(p, 10, 37));
    CHECK(RollingHash::getSubHash(p, 3, 30) != RollingHash::getSubHash(p, 3, 29));
}

TEST(region_key_closed_forms) {
    CHECK_EQ(RegionFusionRegistry::shapeHash({128, 784}), 4784ull);
    CHECK_EQ(RegionFusionRegistry::shapeHash({128, 256}), 4256ull);
    CHECK_EQ(RegionFusionRegistry::shapeHash({8192, 4096}), 258080ull);
    CHECK_EQ(RegionFusionRegistry::regionKey(223384, {128, 784}), 0x12b000036898ull);
    CHECK_EQ(RegionFusionRegistry::regionKey(223384, {128, 256}), 0x10a000036898ull);
    CHECK_EQ(RegionFusionRegistry::regionKey(223384, {8192, 4096}), 0x3f02000036898ull);
}

TEST(registry_fnv_closed_forms) {
    CHECK_EQ(C3KernelRegistry::hashShapes({128, 784}, {784, 256}), (size_t)0xd3cd56bc81bd4363ull);
    CHECK_EQ(C3KernelRegistry::hashShapes({1u << 24}, {1u << 24}), (size_t)0x9158189b386f57cbull);
    KernelShapeInfo s;
    s.fused_pattern = "MatMul+Add+ReLU";
    s.lhs_shape = {128, 784};
    CHECK_EQ(C3KernelRegistry::makeFusedKey(op::ReLU, s), std::string("MatMul+Add+ReLU|9:128:784"));
}

TEST(cost_model_closed_forms) {
    const size_t mn = 128 * 256;
    auto c = FusionCostModel::estimate({op::MatMul, op::Add, op::ReLU}, {mn, mn, mn});
    CHECK_EQ(c.eager_accesses, 5 * mn);
    CHECK_EQ(c.saved_accesses, 2 * mn);
    CHECK(std::fabs(c.gain_ratio - 0.4) < 1e-12);
    CHECK(c.worthwhile);
    auto d = FusionCostModel::estimate({op::MatMul, op::ReLU}, {mn, mn});
    CHECK_EQ(d.saved_accesses, (size_t)0);
    CHECK(!d.worthwhile);
    // Elementwise chain Add->ReLU->Neg: eager 5n, saved 4n -> 0.8.
    auto e = FusionCostModel::estimate({op::Add, op::ReLU, op::Neg}, {10, 10, 10});
    CHECK(std::fabs(e.gain_ratio - 0.8) < 1e-12);
    CHECK(FusionCostModel::estimate({}, {}).eager_accesses == 0);
    CHECK_EQ(c.fused_accesses, 3 * mn);
    // Lengths differ: only the common prefix counts (MatMul, Add over [mn] -> eager 3mn, saved 0).
    auto f = FusionCostModel::estimate({op::MatMul, op::Add, op::ReLU}, {mn, mn});
    CHECK_EQ(f.eager_accesses, 3 * mn);
    CHECK_EQ(f.saved_accesses, (size_t)0);
    CHECK(!f.worthwhile);
    // Empty outputs: no accesses, ratio 0, not worthwhile.
    auto z = FusionCostModel::estimate({op::Add, op::ReLU}, {0, 0});
    CHECK(z.eager_accesses == 0 && z.gain_ratio == 0.0 && !z.worthwhile);
}

TEST(sha256_fips_vectors) {
    CHECK_EQ(sha256_hex("abc"), std::string("ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"));
    CHECK_EQ(sha256_hex(""), std::string("e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"));
    CHECK_EQ(sha256_hex("abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq"),
             std::string("248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"));
    CHECK_EQ(sha256_hex(std::string(1000000, 'a')),
             std::string("cdc76e5c9914fb9281a1c7e284d73e67f1809a48a497200e046d39ccc7112cd0"));
    // Lengths 55/56/63/64 straddle the padding boundary.
    CHECK_EQ(sha256_hex(std::string(64, 'a')),
             std::string("ffe054fe7ae0cb6dc65c3af9b61d5209f439851db43d0ba5997337df154668eb"));
}

// --------------------------------------------------------------- JITCache --
TEST(jit_cache_layout_and_versioning) {
    const std::string dir = tmpdir();
    setenv("C3_AOT_CACHE_DIR", dir.c_str(), 1);
    unsetenv("C3_JIT_CACHE_DISABLE");
    JITCache& c = JITCache::getInstance();
    CHECK_EQ(c.cacheDir(), dir);
    const std::string key = JITCache::makeKey("rh=36898|kind=linear_fwd", 3);
    CHECK_EQ(key, sha256_hex(std::string("c3_jit_") + JITCache::currentJITVersion() + "_3_rh=36898|kind=linear_fwd"));
    const uint64_t m0 = c.misses(), h0 = c.hits(), s0 = c.stores();
    CHECK(c.lookup(key).empty());
    CHECK_EQ(c.misses(), m0 + 1);
    std::vector<char> img = {'\x7f', 'E', 'L', 'F', 1, 2, 3};
    const std::string sha = sha256_hex(img.data(), img.size());
    const std::string path = c.store(key, img, {"module=gemm_f32"});
    CHECK_EQ(path, dir + "/c3_jit_obj_" + sha + ".hsaco");
    CHECK_EQ(c.stores(), s0 + 1);
    CHECK_EQ(c.lookup(key), path);
    CHECK_EQ(c.lookup(key, sha), path);
    CHECK_EQ(c.hits(), h0 + 2);
    std::vector<char> back;
    CHECK(JITCache::readFile(path, &back) && back == img);
    {
        std::ifstream meta(dir + "/c3_jit_" + key + ".meta");
        std::string line;
        std::getline(meta, line);
        CHECK_EQ(line, std::string(JITCache::currentJITVersion()));
        std::getline(meta, line);
        CHECK_EQ(line, "image=" + sha);
        std::getline(meta, line);
        CHECK_EQ(line, std::string("module=gemm_f32"));
    }
    // A stale version evicts the entry.
    { std::ofstream m(dir + "/c3_jit_" + key + ".meta"); m << "jit_v2\nimage=" << sha << "\n"; }
    CHECK(c.lookup(key).empty());
    CHECK(access((dir + "/c3_jit_" + key + ".meta").c_str(), F_OK) != 0);
    // No temporary files are left behind; evict removes entries and objects.
    CHECK(!c.store(key, img).empty());
    c.evict();
    CHECK(c.lookup(key).empty());
    CHECK(access(path.c_str(), F_OK) != 0);
    setenv("C3_JIT_CACHE_DISABLE", "1", 1);
    CHECK(!JITCache::isEnabled());
    unsetenv("C3_JIT_CACHE_DISABLE");
    CHECK(JITCache::isEnabled());
    unsetenv("C3_AOT_CACHE_DIR");
}

TEST(jit_cache_one_object_per_image) {
    // Many spec keys naming the same code object store it once.
    const std::string dir = tmpdir();
    setenv("C3_AOT_CACHE_DIR", dir.c_str(), 1);
    JITCache& c = JITCache::getInstance();
    std::vector<char> a(100000, 'a'), b(5000, 'b');
    for (int i = 0; i < 20; ++i) CHECK(!c.store(JITCache::makeKey("spec" + std::to_string(i), 2), i % 2 ? a : b).empty());
    int objects = 0, metas = 0;
    DIR* d = opendir(dir.c_str());
    while (dirent* e = readdir(d)) {
        const std::string n = e->d_name;
        if (n.rfind("c3_jit_obj_", 0) == 0) objects++;
        else if (n.rfind("c3_jit_", 0) == 0 && n.size() > 5 && n.substr(n.size() - 5) == ".meta") metas++;
        CHECK(n.find(".tmp") == std::string::npos);
    }
    closedir(d);
    CHECK_EQ(objects, 2);
    CHECK_EQ(metas, 20);
    for (int i = 0; i < 20; ++i)
        CHECK_EQ(c.lookup(JITCache::makeKey("spec" + std::to_string(i), 2)),
                 dir + "/c3_jit_obj_" + sha256_hex(i % 2 ? a.data() : b.data(), i % 2 ? a.size() : b.size()) + ".hsaco");
    c.evict();
    unsetenv("C3_AOT_CACHE_DIR");
}

TEST(jit_cache_rejects_damaged_and_stale_images) {
    const std::string dir = tmpdir();
    setenv("C3_AOT_CACHE_DIR", dir.c_str(), 1);
    JITCache& c = JITCache::getInstance();
    std::vector<char> img(4096);
    for (size_t i = 0; i < img.size(); ++i) img[i] = (char)(i * 7);
    const std::string key = JITCache::makeKey("rh=1|kind=matmul", 2), key2 = JITCache::makeKey("rh=2|kind=matmul", 2);
    const std::string path = c.store(key, img);
    CHECK(!c.store(key2, img).empty());
    const std::string sha = sha256_hex(img.data(), img.size());
    // An entry recorded for another image (an older build's) is rejected and
    // evicted; the shared object stays for the other key.
    const uint64_t r0 = c.rejected();
    CHECK(c.lookup(key, std::string(64, '0')).empty());
    CHECK_EQ(c.rejected(), r0 + 1);
    CHECK(access((dir + "/c3_jit_" + key + ".meta").c_str(), F_OK) != 0);
    CHECK_EQ(c.lookup(key2, sha), path);
    // A damaged object (one byte changed, same size) is rejected and removed.
    {
        std::fstream f(path, std::ios::in | std::ios::out | std::ios::binary);
        f.seekp(1000);
        f.put((char)(img[1000] ^ 0x5a));
    }
    struct timespec ts[2] = {{0, UTIME_NOW}, {0, UTIME_NOW}};
    utimensat(AT_FDCWD, path.c_str(), ts, 0);
    CHECK(c.lookup(key2, sha).empty());
    CHECK_EQ(c.rejected(), r0 + 2);
    CHECK(access(path.c_str(), F_OK) != 0);
    // Storing again restores a good entry.
    CHECK_EQ(c.store(key2, img), path);
    CHECK_EQ(c.lookup(key2, sha), path);
    c.evict();
    unsetenv("C3_AOT_CACHE_DIR");
}

// ------------------------------------------------------ HipCompiledKernel --
// Borrowed kHIP tensors over host memory (never dereferenced): execute()
// must refuse operands whose element type differs from the spec's before any
// HIP call, so a registry hit with mixed operands falls back to eager.
TEST(hip_kernel_rejects_mixed_dtypes) {
    std::vector<float> buf(4096);
    auto hip = [&](std::vector<size_t> shape, DType dt) { return Tensor::fromBlob(buf.data(), std::move(shape), dt, DeviceType::kHIP); };
    auto throws = [](HipCompiledKernel& k, const std::vector<Tensor>& in, const char* needle) {
        try {
            k.execute(in);
        } catch (const std::runtime_error& e) {
            return std::string(e.what()).find(needle) != std::string::npos;
        }
        return false;
    };
    KernelSpec f;
    f.kind = KernelKind::LinearFwd;
    f.dtype = DType::kBFloat16;
    f.act = C3HIP_ACT_RELU;
    f.input_shapes = {{8, 16}, {16, 8}, {8}};
    HipCompiledKernel kf(f, 2, "t");
    CHECK(throws(kf, {hip({8, 16}, DType::kFloat), hip({16, 8}, DType::kBFloat16), hip({8}, DType::kFloat)},
                 "compiled for bf16"));
    CHECK(throws(kf, {hip({8, 16}, DType::kBFloat16), hip({16, 8}, DType::kFloat), hip({8}, DType::kFloat)},
                 "input 1 is fp32"));
    KernelSpec b;
    b.kind = KernelKind::LinearBwd;
    b.dtype = DType::kFloat;
    b.act = C3HIP_ACT_RELU;
    b.input_shapes = {{8, 8}, {8, 16}, {16, 8}, {8, 8}};
    HipCompiledKernel kb(b, 2, "t");
    CHECK(throws(kb, {hip({8, 8}, DType::kFloat), hip({8, 16}, DType::kFloat), hip({16, 8}, DType::kFloat),
                      hip({8, 8}, DType::kBFloat16)},
                 "input 3 is bf16"));
    KernelSpec m;
    m.kind = KernelKind::MatMul;
    m.dtype = DType::kFloat;
    HipCompiledKernel km(m, 2, "t");
    CHECK(throws(km, {hip({8, 16}, DType::kFloat), hip({16, 8}, DType::kBFloat16)}, "compiled for fp32"));
    CHECK(throws(km, {hip({128}, DType::kFloat), hip({16, 8}, DType::kFloat)}, "2-D"));
}

// ---------------------------------------------------------------- registry --
TEST(registry_install_dispatch_and_precedence) {
    HostBackend hb;
    auto& R = C3KernelRegistry::getInstance();
    KernelSpec add;
    add.kind = KernelKind::Elementwise;
    add.ew_op = C3HIP_EW_ADD;
    KernelShapeInfo info;
    info.lhs_shape = {2, 3};
    info.rhs_shape = {2, 3};
    info.out_shape = {2, 3};
    auto k4 = std::make_shared<HostKernel>(add, 4);
    R.install(op::Add, DeviceType::kCPU, k4, info);
    Tensor a = host({2, 3}, {1, 2, 3, 4, 5, 6}), b = host({2, 3}, {10, 20, 30, 40, 50, 60});
    auto r = R.tryExecute(op::Add, a, b);
    CHECK(r.has_value());
    CHECK(vals(*r) == (std::vector<float>{11, 22, 33, 44, 55, 66}));
    // Other shapes / devices / ops miss.
    CHECK(!R.tryExecute(op::Add, host({3, 2}, {1, 2, 3, 4, 5, 6}), host({3, 2}, {1, 2, 3, 4, 5, 6})).has_value());
    CHECK(!R.tryExecute(op::Sub, a, b).has_value());
    // A lower or equal opt level does not replace; a higher one does.
    KernelSpec sub = add;
    sub.ew_op = C3HIP_EW_SUB;
    const size_t inst0 = R.getStats().install_count;
    R.install(op::Add, DeviceType::kCPU, std::make_shared<HostKernel>(sub, 2), info);
    R.install(op::Add, DeviceType::kCPU, std::make_shared<HostKernel>(sub, 4), info);
    CHECK_EQ(R.getStats().install_count, inst0);
    CHECK(vals(*R.tryExecute(op::Add, a, b))[0] == 11.f);
    R.install(op::Add, DeviceType::kCPU, std::make_shared<HostKernel>(sub, 5), info);
    CHECK(vals(*R.tryExecute(op::Add, a, b))[0] == -9.f);
    const auto st = R.getStats();
    CHECK_EQ(st.active_entries, (size_t)1);
    CHECK(st.hit_count >= 3);
    R.uninstall(op::Add, DeviceType::kCPU);
    CHECK(!R.tryExecute(op::Add, a, b).has_value());
}

TEST(registry_failures_fall_back) {
    HostBackend hb;
    auto& R = C3KernelRegistry::getInstance();
    KernelShapeInfo info;
    info.lhs_shape = {4};
    info.out_shape = {4};
    // A throwing kernel: nullopt and a counted miss, the entry stays.
    R.install(op::ReLU, DeviceType::kCPU,
              std::make_shared<ScriptedKernel>(3, [](const std::vector<Tensor>&) -> std::vector<Tensor> {
                  throw std::runtime_error("boom");
              }),
              info);
    const size_t miss0 = R.getStats().miss_count;
    CHECK(!R.tryExecuteUnary(op::ReLU, host({4}, {1, -1, 2, -2})).has_value());
    CHECK_EQ(R.getStats().miss_count, miss0 + 1);
    CHECK_EQ(R.getStats().active_entries, (size_t)1);
    // A kernel producing the wrong output shape is uninstalled.
    R.uninstallAll();
    R.install(op::Neg, DeviceType::kCPU,
              std::make_shared<ScriptedKernel>(3, [](const std::vector<Tensor>&) {
                  return std::vector<Tensor>{host({2}, {0, 0})};
              }),
              info);
    CHECK(!R.tryExecuteUnary(op::Neg, host({4}, {1, 2, 3, 4})).has_value());
    CHECK_EQ(R.getStats().active_entries, (size_t)0);
    // An empty result is a miss too.
    R.install(op::Neg, DeviceType::kCPU,
              std::make_shared<ScriptedKernel>(3, [](const std::vector<Tensor>&) { return std::vector<Tensor>{}; }),
              info);
    CHECK(!R.tryExecuteUnary(op::Neg, host({4}, {1, 2, 3, 4})).has_value());
    // Fused execution failure returns an undefined tensor.
    auto bad = std::make_shared<ScriptedKernel>(3, [](const std::vector<Tensor>&) -> std::vector<Tensor> {
        throw std::runtime_error("bad");
    });
    CHECK(!R.executeFusedWithInputs(bad, {host({1}, {1})}, KernelShapeInfo{}).defined());
}

TEST(registry_backward_entries) {
    HostBackend hb;
    auto& R = C3KernelRegistry::getInstance();
    // Kernel returning its inputs so the feed order is visible.
    auto echo = std::make_shared<ScriptedKernel>(3, [](const std::vector<Tensor>& in) { return in; });
    R.installBackward("MatMul|k|in:0", echo, {2, 2}, {2, 3}, {1}, 2);
    Tensor g = host({2, 2}, {1, 2, 3, 4}), A = host({2, 3}, {0, 0, 0, 0, 0, 0}), B = host({3, 2}, {7, 7, 7, 7, 7, 7});
    auto r = R.tryExecuteBackward("MatMul|k|in:0", g, {A, B});
    CHECK(r.has_value() && r->size() == 2);
    CHECK(vals((*r)[0]) == vals(g));
    CHECK(vals((*r)[1]) == vals(B));  // fwd_input_map {1} feeds B, not A
    CHECK(R.hasBackwardKey("MatMul|k|in:0"));
    CHECK(!R.hasBackwardKey("MatMul|k|in:1"));
    CHECK(!R.tryExecuteBackward("MatMul|k|in:0", host({4}, {1, 2, 3, 4}), {A, B}).has_value());  // grad shape
    CHECK(!R.tryExecuteBackward("MatMul|k|in:0", g, {A}).has_value());                          // map out of range
    R.installBackward("X|in:0", echo, {2, 2}, {2, 2}, {0}, 3);                                  // num_inputs 3
    CHECK(!R.tryExecuteBackward("X|in:0", g, {A}).has_value());
}

TEST(registry_fused_entries) {
    HostBackend hb;
    auto& R = C3KernelRegistry::getInstance();
    KernelSpec lin;
    lin.kind = KernelKind::LinearFwd;
    lin.act = 1;
    KernelShapeInfo info;
    info.lhs_shape = {2, 2};
    info.rhs_shape = {2, 2};
    info.out_shape = {2, 2};
    info.fused_pattern = "MatMul+Add+ReLU";
    R.installFused(std::make_shared<HostKernel>(lin, 3), op::ReLU, info);
    CHECK_EQ(R.fusedEntryCount(), (size_t)1);
    Tensor X = host({2, 2}, {1, 2, 3, 4}), W = host({2, 2}, {1, 0, 0, -1}), b = host({2}, {0.5f, 1});
    auto y = R.tryExecuteFused(op::ReLU, {X, W, b});
    CHECK(y.has_value());
    CHECK(vals(*y) == (std::vector<float>{1.5f, 0, 3.5f, 0}));
    CHECK(!R.tryExecuteFused(op::Sigmoid, {X, W, b}).has_value());
    auto f = R.findFusedKernelForSequence({op::MatMul, op::Add, op::ReLU}, DeviceType::kCPU, {2, 2});
    CHECK(f.has_value() && f->second.fused_pattern == "MatMul+Add+ReLU");
    CHECK(!R.findFusedKernelForSequence({op::MatMul, op::ReLU}, DeviceType::kCPU).has_value());
    CHECK(R.findFusedKernelForFirstOp(op::MatMul, {2, 2}, DeviceType::kCPU).has_value());
    CHECK(R.getStats().fused_hit_count >= 1);
    R.uninstallFused(op::ReLU, info);
    CHECK_EQ(R.fusedEntryCount(), (size_t)0);
}

// ---------------------------------------------------------- region fusion --
TEST(region_registry_install_and_match) {
    HostBackend hb;
    auto& RF = RegionFusionRegistry::getInstance();
    KernelSpec lin;
    lin.kind = KernelKind::LinearFwd;
    auto k = std::make_shared<HostKernel>(lin, 3);
    const size_t mn = 128 * 256;
    RF.installWithCost({op::MatMul, op::Add, op::ReLU}, k, {mn, mn, mn}, {{128, 784}, {784, 256}});
    RF.installWithCost({op::MatMul, op::ReLU}, k, {mn, mn}, {{128, 784}, {784, 256}});
    CHECK_EQ(RF.entryCount(), (size_t)2);
    CHECK(RF.mayMatchAsLastOp(op::ReLU));
    CHECK(!RF.mayMatchAsLastOp(op::Sigmoid));
    auto e = RF.find(0x12b000036898ull);
    CHECK(e.has_value() && e->len == 3 && e->cost.worthwhile);
    CHECK(!RF.find(RegionFusionRegistry::regionKey(1732, {128, 784})).has_value());  // MatMul+ReLU: inactive
    // Longest match from a position of a dispatch trace.
    auto p = RollingHash::computePrefixHashes({op::Neg, op::MatMul, op::Add, op::ReLU, op::Mul});
    auto m = RF.matchFromPosition(p, 1, {128, 784});
    CHECK(m.has_value() && m->len == 3);
    CHECK(!RF.matchFromPosition(p, 1, {128, 256}).has_value());  // other first-input shape
    CHECK(!RF.matchFromPosition(p, 0, {128, 784}).has_value());
    CHECK(!RF.matchFromPosition(p, 4, {128, 784}).has_value());
    // Same op sequence and first-input shape, another W width: the shared key
    // keeps the last install (reference behaviour), the full input shapes
    // reach each kernel.
    auto k2 = std::make_shared<HostKernel>(lin, 3);
    RF.installWithCost({op::MatMul, op::Add, op::ReLU}, k2, {mn, mn, mn}, {{128, 784}, {784, 512}});
    auto shared = RF.matchFromPosition(p, 1, {128, 784});
    CHECK(shared.has_value() && shared->kernel == k2);
    auto v1 = RF.matchFromPosition(p, 1, {128, 784}, {{128, 784}, {784, 256}});
    auto v2 = RF.matchFromPosition(p, 1, {128, 784}, {{128, 784}, {784, 512}});
    CHECK(v1.has_value() && v1->kernel == k);
    CHECK(v2.has_value() && v2->kernel == k2);
    auto v3 = RF.matchFromPosition(p, 1, {128, 784}, {{128, 784}, {784, 999}});  // unknown: shared key
    CHECK(v3.has_value() && v3->kernel == k2);
    CHECK(RegionFusionRegistry::variantKey(1, {{2, 3}}) != RegionFusionRegistry::variantKey(1, {{3, 2}}));
    CHECK(RegionFusionRegistry::variantKey(1, {{2}, {3}}) != RegionFusionRegistry::variantKey(1, {{2, 3}}));
    // Inconsistent out_numels leave the entry inactive.
    RF.installWithCost({op::MatMul, op::Add, op::ReLU}, k, {mn, mn}, {{64, 64}, {64, 64}});
    CHECK(!RF.find(RegionFusionRegistry::regionKey(223384, {64, 64})).has_value());
    RF.clear();
    CHECK(!RF.mayMatchAsLastOp(op::ReLU));
}

// ------------------------------------------------ activation specs ------
TEST(sigmoid_tanh_exp_log_specs) {
    KernelSpec s;
    using R = C3HotPathManager::DispatchRecord;
    CHECK(C3HotPathManager::buildFusedSpec({R{op::MatMul, {8, 4, 4, 6}, {8, 4}, {4, 6}, DType::kFloat, {}},
                                            R{op::Add, {8, 6, 6}, {8, 6}, {6}, DType::kFloat, {}},
                                            R{op::Sigmoid, {8, 6}, {8, 6}, {}, DType::kFloat, {}}},
                                           "MatMul+Add+Sigmoid", &s));
    CHECK(s.kind == KernelKind::LinearFwd && s.act == C3HIP_ACT_SIGMOID && s.input_shapes.size() == 3);
    CHECK(C3HotPathManager::buildFusedSpec({R{op::MatMul, {8, 4, 4, 6}, {8, 4}, {4, 6}, DType::kFloat, {}},
                                            R{op::Sigmoid, {8, 6}, {8, 6}, {}, DType::kFloat, {}}},
                                           "MatMul+Sigmoid", &s));
    CHECK(s.act == C3HIP_ACT_SIGMOID && s.input_shapes.size() == 2);  // no bias
    const std::pair<op, int> unary[] = {{op::Sigmoid, C3HIP_EW_SIGMOID}, {op::Tanh, C3HIP_EW_TANH},
                                        {op::Exp, C3HIP_EW_EXP}, {op::Log, C3HIP_EW_LOG}};
    for (auto [o, code] : unary) {
        CHECK(C3HotPathManager::isSupportedOp(o));
        CHECK(C3HotPathManager::buildSingleOpSpec(o, {4, 5}, {}, DType::kFloat, &s));
        CHECK(s.kind == KernelKind::Elementwise && s.ew_op == code && s.input_shapes.size() == 1);
    }
    CHECK(!C3HotPathManager::isSupportedOp(op::Cos));
}

TEST(backward_rules_of_elementwise_nodes) {
    KernelSpec s;
    std::vector<size_t> map;
    size_t n = 0;
    const std::vector<size_t> g = {4, 6};
    auto build = [&](const char* t, std::vector<std::vector<size_t>> in, size_t i) {
        return C3BackwardCapture::buildBackwardSpecForInput(t, g, in, DType::kFloat, i, &s, &map, &n);
    };
    CHECK(build("Sigmoid", {g}, 0) && s.kind == KernelKind::UnaryBackward && s.ew_op == C3HIP_EW_SIGMOID_BWD &&
          map == std::vector<size_t>{0} && n == 2);
    CHECK(build("Tanh", {g}, 0) && s.ew_op == C3HIP_EW_TANH_BWD);
    CHECK(build("Exp", {g}, 0) && s.ew_op == C3HIP_EW_EXP_BWD);
    CHECK(!build("Exp", {g}, 1));
    CHECK(build("Log", {g}, 0) && s.kind == KernelKind::Elementwise && s.ew_op == C3HIP_EW_DIV && n == 2);
    CHECK(build("Neg", {g}, 0) && s.ew_op == C3HIP_EW_NEG && map.empty() && n == 1);
    CHECK(build("Sub", {g, g}, 0) && s.kind == KernelKind::AddBackwardLhs);
    CHECK(build("Sub", {g, g}, 1) && s.kind == KernelKind::Elementwise && s.ew_op == C3HIP_EW_NEG);
    CHECK(build("Mul", {g, g}, 0) && s.ew_op == C3HIP_EW_MUL && map == std::vector<size_t>{1});
    CHECK(build("Mul", {g, g}, 1) && s.ew_op == C3HIP_EW_MUL && map == std::vector<size_t>{0});
    CHECK(build("Div", {g, g}, 0) && s.ew_op == C3HIP_EW_DIV && map == std::vector<size_t>{1});
    CHECK(build("Div", {g, g}, 1) && s.kind == KernelKind::DivBackwardB && map == (std::vector<size_t>{0, 1}) &&
          n == 3);
    CHECK(!build("Mul", {g, {6}}, 0));  // broadcast operand: not compiled
    CHECK(!build("Cos", {g}, 0));
    for (const char* t : {"Sigmoid", "Tanh", "Exp", "Log", "Neg", "Sub", "Mul", "Div"})
        CHECK(C3BackwardCapture::supportsNodeType(t));
}

// ---------------------------------------------------------------- engine ---
TEST(engine_cache_and_watchdog) {
    HostBackend hb;
    auto& E = C3Engine::getInstance();
    KernelSpec s;
    s.kind = KernelKind::Elementwise;
    s.ew_op = C3HIP_EW_NEG;
    s.input_shapes = {{8}};
    auto k1 = E.compile(s, {});
    auto k2 = E.compile(s, {});
    CHECK(k1 && k1 == k2);
    CHECK_EQ(g_built.load(), 1);
    CompileOptions o4;
    o4.opt_level = 4;
    CHECK(E.compile(s, o4) != k1);
    // Watchdog: a backend slower than the timeout yields nullptr + the error.
    E.setFactoryForTest([](const KernelSpec& sp, const CompileOptions& o) {
        std::this_thread::sleep_for(std::chrono::milliseconds(300));
        return std::make_shared<HostKernel>(sp, o.opt_level);
    });
    const uint32_t old = E.getCompileTimeoutMs();
    E.setCompileTimeoutMs(20);
    const size_t t0 = E.getCacheStats().async_timeouts;
    auto f = E.compileAsync(s, {});
    CHECK(f.get() == nullptr);
    CHECK(E.getLastCompileError().find("[async-timeout]") != std::string::npos);
    CHECK_EQ(E.getCacheStats().async_timeouts, t0 + 1);
    E.setCompileTimeoutMs(old);
    // A failing backend leaves an error and no kernel.
    E.setFactoryForTest([](const KernelSpec&, const CompileOptions&) -> std::shared_ptr<CompiledKernel> {
        throw std::runtime_error("no kernel for this spec");
    });
    CHECK(E.compile(s, {}) == nullptr);
    CHECK(E.getLastCompileError().find("no kernel for this spec") != std::string::npos);
}

// ---------------------------------------------------------------- hot path -
TEST(hotpath_threshold_dual_tier_install) {
    HostBackend hb;
    auto& H = C3HotPathManager::instance();
    auto& R = C3KernelRegistry::getInstance();
    for (int i = 0; i < 4; ++i) H.recordCall(op::Add, DeviceType::kCPU, {2, 3}, {2, 3});
    H.waitForPendingCompiles();
    CHECK_EQ(H.getStats().compilations_triggered, (size_t)0);
    H.recordCall(op::Add, DeviceType::kCPU, {2, 3}, {2, 3});
    H.waitForPendingCompiles();
    CHECK_EQ(H.getStats().compilations_triggered, (size_t)1);
    CHECK_EQ(g_built.load(), 2);  // O2 and O4 tiers
    auto r = R.tryExecute(op::Add, host({2, 3}, {1, 1, 1, 1, 1, 1}), host({2, 3}, {1, 2, 3, 4, 5, 6}));
    CHECK(r.has_value() && vals(*r)[5] == 7.f);
    // Within the cooldown further hot calls do not recompile.
    for (int i = 0; i < 10; ++i) H.recordCall(op::Add, DeviceType::kCPU, {2, 3}, {2, 3});
    H.waitForPendingCompiles();
    CHECK_EQ(H.getStats().compilations_triggered, (size_t)1);
    CHECK(H.getStats().cooldown_hits >= 1);
    // MPS calls are ignored; unsupported ops trigger but build nothing.
    H.recordCall(op::Add, DeviceType::kMPS, {9}, {9});
    for (int i = 0; i < 5; ++i) H.recordCall(op::Cos, DeviceType::kCPU, {4});
    H.waitForPendingCompiles();
    CHECK_EQ(g_built.load(), 2);
}

TEST(hotpath_backpressure) {
    HostBackend hb;
    auto& H = C3HotPathManager::instance();
    HotPathConfig cfg;
    cfg.max_pending = 0;
    H.configure(cfg);
    for (int i = 0; i < 6; ++i) H.recordCall(op::Mul, DeviceType::kCPU, {4}, {4});
    CHECK(H.getStats().backpressure_hits >= 6);
    CHECK_EQ(H.getStats().compilations_triggered, (size_t)0);
}

TEST(hotpath_fused_pattern_installs_region) {
    HostBackend hb;
    auto& H = C3HotPathManager::instance();
    // Autograd-scope calls: MatMul [3,4]x[4,2], Add [3,2]+[2], ReLU [3,2].
    H.recordCall(op::MatMul, DeviceType::kCPU, {3, 4}, {4, 2}, true);
    H.recordCall(op::Add, DeviceType::kCPU, {3, 2}, {2}, true);
    H.recordCall(op::ReLU, DeviceType::kCPU, {3, 2}, {}, true);
    H.waitForPendingCompiles();
    CHECK_EQ(C3KernelRegistry::getInstance().fusedEntryCount(), (size_t)1);
    auto e = RegionFusionRegistry::getInstance().find(RegionFusionRegistry::regionKey(223384, {3, 4}));
    CHECK(e.has_value() && e->cost.worthwhile);
    // The region kernel computes relu(X W + b).
    Tensor X = host({3, 4}, {1, 0, 0, 0, 0, 1, 0, 0, 0, 0, 1, 1});
    Tensor W = host({4, 2}, {1, -1, 2, -2, 3, -3, 4, -4});
    Tensor b = host({2}, {0.5f, 0.5f});
    Tensor y = C3KernelRegistry::getInstance().executeFusedWithInputs(e->kernel, {X, W, b}, KernelShapeInfo{});
    CHECK(vals(y) == (std::vector<float>{1.5f, 0, 2.5f, 0, 7.5f, 0}));
    // Repeated detections (every training step) do not rebuild.
    const int built = g_built.load();
    for (int i = 0; i < 3; ++i) {
        H.recordCall(op::MatMul, DeviceType::kCPU, {3, 4}, {4, 2}, true);
        H.recordCall(op::Add, DeviceType::kCPU, {3, 2}, {2}, true);
        H.recordCall(op::ReLU, DeviceType::kCPU, {3, 2}, {}, true);
    }
    H.waitForPendingCompiles();
    CHECK_EQ(g_built.load(), built);
    // Sigmoid epilogue: a region kernel too.
    H.recordCall(op::MatMul, DeviceType::kCPU, {5, 4}, {4, 2}, true);
    H.recordCall(op::Add, DeviceType::kCPU, {5, 2}, {2}, true);
    H.recordCall(op::Sigmoid, DeviceType::kCPU, {5, 2}, {}, true);
    H.waitForPendingCompiles();
    CHECK_EQ(g_built.load(), built + 1);
    // A full-tensor Add (not a bias row) is detected but has no fused kernel.
    H.recordCall(op::MatMul, DeviceType::kCPU, {6, 4}, {4, 2}, true);
    H.recordCall(op::Add, DeviceType::kCPU, {6, 2}, {6, 2}, true);
    H.recordCall(op::Sigmoid, DeviceType::kCPU, {6, 2}, {}, true);
    H.waitForPendingCompiles();
    CHECK(H.getStats().patterns_unsupported >= 1);
    CHECK_EQ(g_built.load(), built + 1);
}

TEST(hotpath_spec_builders) {
    KernelSpec s;
    CHECK(C3HotPathManager::buildSingleOpSpec(op::Div, {7}, {7}, DType::kFloat, &s));
    CHECK(s.kind == KernelKind::Elementwise && s.ew_op == C3HIP_EW_DIV && s.input_shapes.size() == 2);
    CHECK(C3HotPathManager::buildSingleOpSpec(op::MatMul, {8, 4}, {4, 2}, DType::kBFloat16, &s));
    CHECK(s.kind == KernelKind::MatMul && s.out_shape == (std::vector<size_t>{8, 2}) && s.moduleName() == "gemm_bf16");
    CHECK(!C3HotPathManager::buildSingleOpSpec(op::MatMul, {8, 4}, {3, 2}, DType::kFloat, &s));
    CHECK(!C3HotPathManager::buildSingleOpSpec(op::Cos, {8}, {}, DType::kFloat, &s));
    CHECK(!C3HotPathManager::buildSingleOpSpec(op::Sigmoid, {8}, {}, DType::kBFloat16, &s));
    using R = C3HotPathManager::DispatchRecord;
    std::vector<R> recs = {R{op::MatMul, {8, 4, 4, 2}, {8, 4}, {4, 2}, DType::kFloat, {}},
                           R{op::Add, {8, 2, 2}, {8, 2}, {2}, DType::kFloat, {}},
                           R{op::ReLU, {8, 2}, {8, 2}, {}, DType::kFloat, {}}};
    CHECK(C3HotPathManager::buildFusedSpec(recs, "MatMul+Add+ReLU", &s));
    CHECK(s.kind == KernelKind::LinearFwd && s.act == 1 && s.input_shapes[2] == (std::vector<size_t>{2}));
    CHECK(s.op_seq == (std::vector<op>{op::MatMul, op::Add, op::ReLU}) && s.moduleName() == "gemm_f32");
    recs[1].rhs_shape = {8, 2};  // not a bias row: no fused kernel
    CHECK(!C3HotPathManager::buildFusedSpec(recs, "MatMul+Add+ReLU", &s));
    CHECK(!C3HotPathManager::buildFusedSpec(recs, "MatMul+Add+Sigmoid", &s));
}

// -------------------------------------------------------- backward capture -
TEST(backward_capture_rules_and_keys) {
    HostBackend hb;
    auto& B = C3BackwardCapture::getInstance();
    Tensor g = host({2, 2}, {1, -2, 3, -4});
    Tensor x = host({2, 2}, {-1, 0, 2, 5});
    CHECK_EQ(C3BackwardCapture::makeBaseKey("ReLU", g, {x}), std::string("ReLU|grad:2,2,|inputs:2,2,"));
    CHECK(!B.tryExecuteBackward("ReLU", g, {x}).has_value());  // miss: compiles in the background
    B.waitForPendingCompiles();
    auto r = B.tryExecuteBackward("ReLU", g, {x});
    CHECK(r.has_value() && vals((*r)[0]) == (std::vector<float>{0, -0.f, 3, -4}));
    // Add with a bias row: in:0 identity, in:1 column sums.
    Tensor t = host({2, 2}, {0, 0, 0, 0}), bias = host({2}, {0, 0});
    CHECK(!B.tryExecuteBackward("Add", g, {t, bias}).has_value());
    B.waitForPendingCompiles();
    auto ra = B.tryExecuteBackward("Add", g, {t, bias});
    CHECK(ra.has_value() && ra->size() == 2);
    CHECK(vals((*ra)[0]) == vals(g));
    CHECK(vals((*ra)[1]) == (std::vector<float>{4, -6}));
    // MatMul: dA = g B^T, dB = A^T g.
    Tensor A = host({2, 3}, {1, 0, 2, 0, 1, 0}), Bm = host({3, 2}, {1, 2, 3, 4, 5, 6});
    CHECK(!B.tryExecuteBackward("MatMul", g, {A, Bm}).has_value());
    B.waitForPendingCompiles();
    auto rm = B.tryExecuteBackward("MatMul", g, {A, Bm});
    CHECK(rm.has_value() && rm->size() == 2);
    CHECK(vals((*rm)[0]) == (std::vector<float>{-3, -5, -7, -5, -7, -9}));
    CHECK(vals((*rm)[1]) == (std::vector<float>{1, -2, 3, -4, 2, -4}));
    // Unknown node types are refused; a key compiles once even on repeated misses.
    CHECK(!B.tryExecuteBackward("Softmax", g, {x}).has_value());
    const auto st = B.getStats();
    CHECK(st.cache_hit_count == 3 && st.cache_miss_count == 3 && st.compiles_submitted == 5);
}

// A layer whose input needs no gradient (the first layer on a data batch):
// its fused backward is a different kernel (spec input_grad = false, "|nodx"
// in the cache text and the registry key) whose output 0 is empty.
TEST(linear_backward_without_input_grad) {
    HostBackend hb;
    KernelSpec seen;
    int built_bwd = 0;
    C3Engine::getInstance().setFactoryForTest([&](const KernelSpec& s, const CompileOptions& o) {
        if (s.kind == KernelKind::LinearBwd) {
            seen = s;
            built_bwd++;
        }
        return std::make_shared<HostKernel>(s, o.opt_level);
    });
    auto& B = C3BackwardCapture::getInstance();
    Tensor g = host({2, 2}, {1, -2, 3, -4});
    Tensor X = host({2, 3}, {1, 0, 2, 0, 1, 0}), W = host({3, 2}, {1, 2, 3, 4, 5, 6}), Y = host({2, 2}, {1, 0, 2, 3});
    CHECK(!B.tryExecuteLinearBackward(g, {X, W, Y}, true, false).has_value());
    B.waitForPendingCompiles();
    CHECK_EQ(built_bwd, 1);
    CHECK(!seen.input_grad && seen.act == C3HIP_ACT_RELU);
    CHECK(seen.toString().find("|nodx") != std::string::npos);
    KernelSpec with = seen;
    with.input_grad = true;
    CHECK(with.toString().find("|nodx") == std::string::npos);
    const auto d = seen.outputDescs();
    CHECK(d.size() == 3 && d[0].first == std::vector<size_t>{0} && d[1].first == (std::vector<size_t>{3, 2}) &&
          d[2].first == std::vector<size_t>{2});
    CHECK(with.outputDescs()[0].first == (std::vector<size_t>{2, 3}));
    const std::string base = C3BackwardCapture::makeBaseKey("Linear+ReLU", g, {X, W, Y});
    CHECK(C3KernelRegistry::getInstance().hasBackwardKey(base + "|fused|nodx"));
    CHECK(!C3KernelRegistry::getInstance().hasBackwardKey(base + "|fused"));
}

// ---------------------------------------------------- merged kernels, PGO --
namespace {
KernelSpec linearSpec(size_t M, size_t K, size_t N, int act) {
    KernelSpec s;
    s.kind = KernelKind::LinearFwd;
    s.op_seq = {op::MatMul, op::Add};
    if (act == 1) s.op_seq.push_back(op::ReLU);
    s.act = act;
    s.input_shapes = {{M, K}, {K, N}, {N}};
    s.out_shape = {M, N};
    return s;
}

// relu(X W + b) on the host, in the kernel's order.
std::vector<float> hostLinear(const std::vector<float>& X, const std::vector<float>& W, const std::vector<float>& b,
                              size_t M, size_t K, size_t N, bool relu) {
    std::vector<float> Y(M * N);
    for (size_t i = 0; i < M; ++i)
        for (size_t j = 0; j < N; ++j) {
            float acc = 0;
            for (size_t k = 0; k < K; ++k) acc += X[i * K + k] * W[k * N + j];
            acc += b[j];
            Y[i * N + j] = relu ? (acc > 0 ? acc : 0.f) : acc;
        }
    return Y;
}

// PGO test rig: host kernels, synchronous compile chains, a counting interpreter.
struct PgoRig {
    HostBackend hb;
    std::atomic<int> interpreted{0};
    PgoRig() {
        auto& P = PGOManager::getInstance();
        P.config() = PGOConfig{};
        P.config().async_compilation = false;
        P.setInterpreterForTest([this](const KernelSpec& s, const std::vector<Tensor>& in) {
            interpreted++;
            return HostKernel(s, 0).execute(in);
        });
    }
    ~PgoRig() {
        PGOManager::getInstance().setInterpreterForTest(nullptr);
        PGOManager::getInstance().config() = PGOConfig{};
        PGOManager::getInstance().clear();
    }
};
}  // namespace

TEST(graph_merger_validate_and_wiring) {
    const auto a = linearSpec(8, 12, 6, 1), b = linearSpec(8, 6, 4, 1), c = linearSpec(8, 4, 3, 0);
    CHECK_EQ(GraphMerger::validate({a, b, c}, GraphMerger::makeSequentialSpec({a, b, c})), std::string());
    CHECK(GraphMerger::validate({}, {}).find("no sub-kernels") != std::string::npos);
    CHECK(GraphMerger::validate({a, b}, {}).find("links count") != std::string::npos);
    CHECK(GraphMerger::validate({a, b}, MergeSpec{{{1, 0}}}).find("from_output") != std::string::npos);
    CHECK(GraphMerger::validate({a, b}, MergeSpec{{{0, 3}}}).find("to_input") != std::string::npos);
    CHECK(GraphMerger::validate({a, c}, MergeSpec{{{0, 0}}}).find("desc mismatch") != std::string::npos);
    CHECK(GraphMerger::validate({a, b}, MergeSpec{{{0, 1}}}).find("desc mismatch") != std::string::npos);
    auto info = GraphMerger::merge({a, b, c}, GraphMerger::makeSequentialSpec({a, b, c}));
    const std::vector<std::pair<size_t, size_t>> ext = {{0, 0}, {0, 1}, {0, 2}, {1, 1}, {1, 2}, {2, 1}, {2, 2}};
    CHECK(info.external_inputs == ext);
    CHECK(info.input_source[1][0] == 0 && info.input_source[1][1] == SIZE_MAX);
    // An unconnected link leaves the next sub's input external.
    auto open = GraphMerger::merge({a, a}, MergeSpec{{{0, SIZE_MAX}}});
    CHECK_EQ(open.external_inputs.size(), size_t(6));
    const std::string key = GraphMerger::mergedCacheKey({a, b}, GraphMerger::makeSequentialSpec({a, b}));
    CHECK(key.rfind("merged_v4_2|G0{", 0) == 0 && key.find("|L0>0|G1{") != std::string::npos);
    CHECK(key != GraphMerger::mergedCacheKey({a, b}, MergeSpec{{{0, SIZE_MAX}}}));
    bool threw = false;
    try {
        GraphMerger::merge({a, c}, MergeSpec{{{0, 0}}});
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    CHECK(threw);
}

TEST(merged_kernel_runs_layers_in_order) {
    HostBackend hb;
    auto& E = C3Engine::getInstance();
    const size_t M = 2, K = 3, H = 2, N = 2;
    const std::vector<float> X = {1, -2, 3, 0, 1, -1}, W1 = {1, 0, -1, 2, 1, 1}, b1 = {0.5f, -1},
                             W2 = {1, -1, 2, 1}, b2 = {0, 1};
    const auto s1 = linearSpec(M, K, H, 1), s2 = linearSpec(M, H, N, 0);
    auto k = E.compileMergedSequential({s1, s2});
    CHECK(k && k == E.compileMergedSequential({s1, s2}));  // cached
    auto out = k->execute({host({M, K}, X), host({K, H}, W1), host({H}, b1), host({H, N}, W2), host({N}, b2)});
    CHECK_EQ(out.size(), size_t(1));
    CHECK(vals(out[0]) == hostLinear(hostLinear(X, W1, b1, M, K, H, true), W2, b2, M, H, N, false));
    auto f = E.compileMergedAsync({s1, s2}, GraphMerger::makeSequentialSpec({s1, s2}));
    CHECK(f.get() != nullptr && f.get().get() == E.compileMergedAsync({s1, s2}, GraphMerger::makeSequentialSpec({s1, s2})).get().get());
    bool threw = false;
    try {
        E.compileMerged({s1, s1}, GraphMerger::makeSequentialSpec({s1, s1}));
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    CHECK(threw);
    // Wrong input count.
    threw = false;
    try {
        k->execute({host({M, K}, X)});
    } catch (const std::runtime_error&) {
        threw = true;
    }
    CHECK(threw);
}

// A PGO kernel: eager first (the interpreter) and the compile chain; then
// the Ofast tuner times the eight fp32 tiles on real calls (the host kernels
// sleep per tile, t128x128 fastest) and keeps the fastest; results are the
// same on every tier.
TEST(pgo_tiers_tune_and_deopt) {
    PgoRig rig;
    auto& E = C3Engine::getInstance();
    auto& P = PGOManager::getInstance();
    E.setFactoryForTest([](const KernelSpec& sp, const CompileOptions& o) -> std::shared_ptr<CompiledKernel> {
        g_built++;
        auto inner = std::make_shared<HostKernel>(sp, o.opt_level);
        const int ms = sp.tile == "t64x64"      ? 4
                       : sp.tile == "t256x128"  ? 8
                       : sp.tile == "t128x256"  ? 6
                       : sp.tile == "t256x128d" ? 7
                       : sp.tile == "t128x256d" ? 5
                       : sp.tile == "t256x256d" ? 3
                       : sp.tile == "t64x64d"   ? 2
                                                : 0;
        return std::make_shared<ScriptedKernel>(o.opt_level, [inner, ms](const std::vector<Tensor>& in) {
            if (ms) std::this_thread::sleep_for(std::chrono::milliseconds(ms));
            return inner->execute(in);
        });
    });
    const size_t M = 3, K = 4, N = 2;
    const std::vector<float> X = {1, 2, 0, -1, 3, -2, 1, 1, 0, 0, 2, -3}, W = {1, -1, 0, 2, 1, 1, -2, 0}, b = {0.25f, -0.5f};
    const auto want = hostLinear(X, W, b, M, K, N, true);
    const std::vector<Tensor> in = {host({M, K}, X), host({K, N}, W), host({N}, b)};
    CompileOptions po;
    po.pgo_mode = true;
    auto k = std::dynamic_pointer_cast<PGOCompiledKernel>(E.compile(linearSpec(M, K, N, 1), po));
    CHECK(k && k == std::dynamic_pointer_cast<PGOCompiledKernel>(E.compile(linearSpec(M, K, N, 1), po)));
    CHECK(P.isEnabled() && !k->isPromoted());
    CHECK(vals(k->execute(in)[0]) == want);  // eager, and the chain compiles (synchronously here)
    CHECK_EQ(rig.interpreted.load(), 1);
    CHECK(k->isPromoted() && k->o2Kernel() && k->ofastKernel());
    auto tuners = k->tuners();
    CHECK(tuners.size() == 1 && tuners[0] && tuners[0]->candidateCount() == 8);
    int calls = 1;
    while (!tuners[0]->tuned() && calls < 40) {
        CHECK(vals(k->execute(in)[0]) == want);
        ++calls;
    }
    CHECK(tuners[0]->tuned());
    CHECK_EQ(calls, 1 + 8 * (1 + P.config().tune_samples));
    CHECK_EQ(tuners[0]->chosen(), std::string("t128x128"));
    CHECK(vals(k->execute(in)[0]) == want);
    CHECK_EQ(rig.interpreted.load(), 1);
    CHECK_EQ(k->profileData().call_count.load(), (uint64_t)calls + 1);
    // Heat score closed form.
    const double n = (double)k->profileData().call_count.load(), t = (double)k->profileData().total_time_ns.load();
    const double want_heat = 0.4 * std::min(1.0, std::log2(1.0 + n) / std::log2(1001.0)) + 0.6 * std::min(1.0, t / 1e9);
    CHECK(std::fabs(k->computeHeatScore() - want_heat) < 1e-12);
    auto st = P.getStats();
    CHECK(st.total_registered == 1 && st.o2_ready == 1 && st.ofast_ready == 1 && st.pending == 0);

    // Deopt: every Ofast candidate throws -> Ofast disabled, O2 serves.
    E.setFactoryForTest([](const KernelSpec& sp, const CompileOptions& o) -> std::shared_ptr<CompiledKernel> {
        auto inner = std::make_shared<HostKernel>(sp, o.opt_level);
        const bool bad = !sp.tile.empty();
        return std::make_shared<ScriptedKernel>(o.opt_level, [inner, bad](const std::vector<Tensor>& x) {
            if (bad) throw std::runtime_error("tile cannot run");
            return inner->execute(x);
        });
    });
    auto k2 = std::dynamic_pointer_cast<PGOCompiledKernel>(E.compile(linearSpec(M, K, N, 0), po));
    const auto want2 = hostLinear(X, W, b, M, K, N, false);
    CHECK(vals(k2->execute(in)[0]) == want2);  // eager + chain
    CHECK(vals(k2->execute(in)[0]) == want2);  // Ofast fails over every candidate -> O2
    CHECK(k2->isOfastDisabled() && !k2->isO2Disabled() && k2->deoptCount() == 1);
    CHECK(k2->lastDeoptReason().rfind("ofast:", 0) == 0);
    CHECK(vals(k2->execute(in)[0]) == want2);
    CHECK_EQ(k2->deoptCount(), uint64_t(1));
}

TEST(pgo_backpressure_queue_and_merged_plan) {
    PgoRig rig;
    auto& E = C3Engine::getInstance();
    auto& P = PGOManager::getInstance();
    P.config().max_concurrent_compilations = 0;  // every chain waits in the queue
    CompileOptions po;
    po.pgo_mode = true;
    const size_t M = 2, K = 3, H = 2, N = 2;
    const std::vector<float> X = {1, -2, 3, 0, 1, -1}, W1 = {1, 0, -1, 2, 1, 1}, b1 = {0.5f, -1},
                             W2 = {1, -1, 2, 1}, b2 = {0, 1};
    const std::vector<Tensor> in = {host({M, K}, X), host({K, H}, W1), host({H}, b1), host({H, N}, W2), host({N}, b2)};
    const auto want = hostLinear(hostLinear(X, W1, b1, M, K, H, true), W2, b2, M, H, N, false);
    auto k = std::dynamic_pointer_cast<PGOCompiledKernel>(
        E.compileMergedPGOSequential({linearSpec(M, K, H, 1), linearSpec(M, H, N, 0)}));
    CHECK(k != nullptr);
    CHECK(vals(k->execute(in)[0]) == want);  // eager over both layers
    CHECK_EQ(rig.interpreted.load(), 2);
    auto st = P.getStats();
    CHECK(st.queued == 1 && st.queue_rejections == 1 && st.pending == 1 && !k->isPromoted());
    P.config().max_concurrent_compilations = 4;
    P.processQueue();  // runs the queued chain
    CHECK(k->isPromoted() && P.getStats().queued == 0);
    CHECK(vals(k->execute(in)[0]) == want);  // Ofast merged: both layers' tuners
    auto tuners = k->tuners();
    CHECK(tuners.size() == 2 && tuners[0] && tuners[1]);
    const int n_tiles = (int)tuners[0]->candidateCount();
    for (int i = 0; i < n_tiles * (1 + P.config().tune_samples) + 1; ++i) CHECK(vals(k->execute(in)[0]) == want);
    CHECK(tuners[0]->tuned() && tuners[1]->tuned());
    CHECK_EQ(rig.interpreted.load(), 2);
    // promoteAll on a fresh kernel compiles it in the calling thread.
    auto k3 = std::dynamic_pointer_cast<PGOCompiledKernel>(E.compile(linearSpec(M, K, H, 1), po));
    CHECK(!k3->isPromoted());
    P.promoteAll();
    CHECK(k3->isPromoted());
    CHECK(vals(k3->execute({in[0], in[1], in[2]})[0]) == hostLinear(X, W1, b1, M, K, H, true));
    CHECK_EQ(rig.interpreted.load(), 2);
}

// ------------------------------------------------- fused backward chains --
namespace {
// A host-framework autograd node: its type, upstream links and forward inputs.
struct FakeNode : BackwardNode {
    FakeNode(std::string t, std::vector<Tensor> in) : type(std::move(t)), inputs(std::move(in)) {}
    std::string typeName() const override { return type; }
    std::vector<std::shared_ptr<BackwardNode>> getUpStreamNodes() const override { return ups; }
    std::vector<Tensor> getInputs() const override { return inputs; }
    std::string type;
    std::vector<Tensor> inputs;
    std::vector<std::shared_ptr<BackwardNode>> ups;
};

std::shared_ptr<FakeNode> node(std::string t, std::vector<Tensor> in, std::shared_ptr<BackwardNode> up) {
    auto n = std::make_shared<FakeNode>(std::move(t), std::move(in));
    if (up) n->ups.push_back(std::move(up));
    return n;
}
}  // namespace

TEST(backward_chain_keys_and_window) {
    HostBackend hb;
    using B = C3BackwardCapture;
    CHECK_EQ(B::makeSequenceKey({"ReLU", "Sigmoid"}), std::string("ReLU+Sigmoid"));
    CHECK_EQ(B::makeSequenceKey({"LReLU", "GELU", "Tanh"}), std::string("Other+Other+Tanh"));
    CHECK_EQ(B::makeFusedBackwardKey("ReLU+Sigmoid", {32, 64}, {32, 64}),
             std::string("backward_fused_ReLU+Sigmoid|g:32,64,|i:32,64,"));
    CHECK(!B::isFusableSequence({"ReLU"}));
    CHECK(!B::isFusableSequence({"ReLU", "Add"}));
    CHECK(B::isFusableSequence({"ReLU", "Sin", "Neg"}));
    KernelSpec sp;
    const std::vector<size_t> g = {4, 6};
    CHECK(B::buildChainSpec({"ReLU", "Log", "Neg"}, {g, g, g}, {g, g, g}, DType::kFloat, &sp));
    CHECK(sp.kind == KernelKind::BackwardChain &&
          sp.chain == (std::vector<int>{C3HIP_CHAIN_RELU, C3HIP_CHAIN_LOG, C3HIP_CHAIN_NEG}) &&
          sp.input_shapes.size() == 4 && sp.out_shape == g && sp.moduleName() == "elementwise");
    CHECK(!B::buildChainSpec({"ReLU", "GELU"}, {g, g}, {g, g}, DType::kFloat, &sp));       // no rule
    CHECK(!B::buildChainSpec({"ReLU", "Log"}, {g, g}, {g, {6}}, DType::kFloat, &sp));       // shapes differ
    CHECK(!B::buildChainSpec({"ReLU", "Log"}, {g, g}, {g, g}, DType::kBFloat16, &sp));      // fp32 only
    CHECK(!B::buildChainSpec({"ReLU", "Log", "Neg", "Exp", "Tanh"}, std::vector<std::vector<size_t>>(5, g),
                             std::vector<std::vector<size_t>>(5, g), DType::kFloat, &sp));  // > window
    // The window: a pair compiles on its first sighting, then the window restarts.
    auto& C = B::getInstance();
    Tensor x = host(g, std::vector<float>(24, 1.f));
    C.recordBackwardNode("Add", g, g, {x});  // not a chain node: ignored
    C.recordBackwardNode("ReLU", g, g, {x});
    C.recordBackwardNode("Log", g, g, {x});
    C.waitForPendingCompiles();
    CHECK(C3KernelRegistry::getInstance().hasBackwardKey("backward_fused_ReLU+Log|g:4,6,|i:4,6,"));
    C.recordBackwardNode("Neg", g, g, {x});  // counts ReLU+Log again, restarts at [Neg]
    std::vector<std::string> tail;
    CHECK(C.getLatestSequenceTail(tail, 1) && tail == std::vector<std::string>{"Neg"});
    CHECK(!C.getLatestSequenceTail(tail, 2));
    C.recordBackwardNode("ReLU", g, g, {x});
    C.waitForPendingCompiles();
    CHECK(C3KernelRegistry::getInstance().hasBackwardKey("backward_fused_Neg+ReLU|g:4,6,|i:4,6,"));
    std::string key;
    Tensor gt = host(g, std::vector<float>(24, 0.f));
    CHECK(C.tryLookupFusedBackwardKey(gt, g, key) && key == "backward_fused_Neg+ReLU|g:4,6,|i:4,6,");
    // Mixed grad shapes along a pair: counted (the tail windows do not check
    // shapes) but never compiled; a GELU pair has no rule.
    C.clearCallScopedState();
    C.recordBackwardNode("ReLU", g, g, {x});
    C.recordBackwardNode("Log", {24}, {24}, {x});
    C.clearCallScopedState();
    C.recordBackwardNode("GELU", g, g, {x});
    C.recordBackwardNode("ReLU", g, g, {x});
    C.waitForPendingCompiles();
    const auto st = C.getStats();
    CHECK(st.fusion_compile_count == 2);
    CHECK(!C3KernelRegistry::getInstance().hasBackwardKey("backward_fused_ReLU+Log|g:4,6,|i:24,"));
    CHECK(!C3KernelRegistry::getInstance().hasBackwardKey("backward_fused_Other+ReLU|g:4,6,|i:4,6,"));
}

// y = relu(wrap(log(x2))): backward runs ReLU (N0), then Log (N1).  The first
// pass runs the nodes one by one and records them; the chain compiles; the
// second pass runs it once at N0 and hands N1 its grad from the intercept map.
TEST(backward_chain_fused_execution) {
    HostBackend hb;
    auto& C = C3BackwardCapture::getInstance();
    const std::vector<size_t> s = {2, 3};
    Tensor x2 = host(s, {0.5f, 2.f, 4.f, 8.f, 0.25f, 1.f});
    Tensor x1 = host(s, {-1.f, 0.f, 2.f, 3.f, -0.5f, 7.f});  // the ReLU's input (log's output, say)
    Tensor gy = host(s, {1.f, 2.f, 3.f, -4.f, 5.f, -6.f});
    auto leaf = node("AccumulateGrad", {}, nullptr);
    auto nlog = node("Log", {x2}, leaf);
    auto wrap = node("Factor", {x1}, nlog);
    auto nrelu = node("ReLU", {x1}, wrap);
    const std::vector<float> want1 = {0.f, 0.f, 3.f, -4.f, 0.f, -6.f};               // (x1 > 0) * gy
    const std::vector<float> want2 = {0.f, 0.f, 0.75f, -0.5f, 0.f, -6.f};            // want1 / x2
    // Pass 1: nothing compiled yet.
    CHECK(!C.tryExecuteBackward(nrelu.get(), gy, {x1}).has_value());
    C.recordBackwardNode("ReLU", s, s, {x1});
    Tensor g1 = host(s, want1);
    CHECK(!C.tryExecuteBackward(nlog.get(), g1, {x2}).has_value());
    C.recordBackwardNode("Log", s, s, {x2});
    C.clearCallScopedState();
    C.waitForPendingCompiles();
    // Pass 2: one chain launch serves both nodes.
    auto r0 = C.tryExecuteBackward(nrelu.get(), gy, {x1});
    CHECK(r0.has_value() && r0->size() == 1 && vals((*r0)[0]) == want1);
    auto r1 = C.tryExecuteBackward(nlog.get(), (*r0)[0], {x2});
    CHECK(r1.has_value() && vals((*r1)[0]) == want2);
    auto st = C.getStats();
    CHECK(st.fusion_hit_count == 2);
    // The intercepted grad is consumed once: a third call runs the Log node's
    // own kernel (compiled in pass 1) from the grad it is given.
    auto r2 = C.tryExecuteBackward(nlog.get(), (*r0)[0], {x2});
    CHECK(r2.has_value() && vals((*r2)[0]) == want2);
    CHECK(C.getStats().fusion_hit_count == 2);
    C.clearCallScopedState();
    // Four wrappers between the nodes: beyond the skip bound, no chain.
    auto w4 = node("Factor", {x1}, node("Factor", {x1}, node("Factor", {x1}, node("Factor", {x1}, nlog))));
    auto far = node("ReLU", {x1}, w4);
    const size_t misses = C.getStats().fusion_miss_count;
    auto rf = C.tryExecuteBackward(far.get(), gy, {x1});
    CHECK(rf.has_value() && vals((*rf)[0]) == want1);  // the ReLU node's own kernel
    CHECK(C.getStats().fusion_miss_count == misses + 1);
    CHECK(C.getStats().fusion_hit_count == 2);
    // Three wrappers: within the bound, the chain runs.
    auto w3 = node("Factor", {x1}, node("Factor", {x1}, node("Factor", {x1}, nlog)));
    auto near = node("ReLU", {x1}, w3);
    auto rn = C.tryExecuteBackward(near.get(), gy, {x1});
    CHECK(rn.has_value() && vals((*rn)[0]) == want1 && C.getStats().fusion_hit_count == 3);
    C.clearCallScopedState();
    // An upstream node whose input has another shape ends the chain.
    Tensor x2b = host({6}, {0.5f, 2.f, 4.f, 8.f, 0.25f, 1.f});
    auto nlogb = node("Log", {x2b}, leaf);
    auto nrelub = node("ReLU", {x1}, nlogb);
    const size_t hits = C.getStats().fusion_hit_count;
    auto rb = C.tryExecuteBackward(nrelub.get(), gy, {x1});
    CHECK(rb.has_value() && C.getStats().fusion_hit_count == hits);
    // Without an upstream of its own the Log node cannot close the chain.
    auto orphan = node("Log", {x2}, nullptr);
    auto nrelu_o = node("ReLU", {x1}, orphan);
    C.clearCallScopedState();
    auto ro = C.tryExecuteBackward(nrelu_o.get(), gy, {x1});
    CHECK(ro.has_value() && C.getStats().fusion_hit_count == hits);
}

TEST(config_kill_switches) {
    HostBackend hb;
    setenv("C3_DISABLE_BACKWARD", "1", 1);
    reloadConfig();
    CHECK(!backwardFusionEnabled());
    Tensor g = host({2}, {1, 2});
    CHECK(!C3BackwardCapture::getInstance().tryExecuteBackward("ReLU", g, {g}).has_value());
    CHECK_EQ(C3BackwardCapture::getInstance().getStats().compiles_submitted, (size_t)0);
    unsetenv("C3_DISABLE_BACKWARD");
    setenv("C3_DISABLE_HOTPATH", "1", 1);
    reloadConfig();
    const size_t c0 = C3HotPathManager::instance().getStats().calls_tracked;
    C3HotPathManager::instance().recordCall(op::Add, DeviceType::kCPU, {2}, {2});
    CHECK_EQ(C3HotPathManager::instance().getStats().calls_tracked, c0);
    unsetenv("C3_DISABLE_HOTPATH");
    reloadConfig();
    CHECK(backwardFusionEnabled() && hotPathTrackingEnabled() && regionFusionEnabled() && singleKernelEnabled());
}

TEST(shutdown_all_clears_state) {
    HostBackend hb;
    auto& H = C3HotPathManager::instance();
    for (int i = 0; i < 5; ++i) H.recordCall(op::Neg, DeviceType::kCPU, {3});
    shutdownAll();
    CHECK_EQ(C3KernelRegistry::getInstance().getStats().active_entries, (size_t)0);
    CHECK_EQ(RegionFusionRegistry::getInstance().entryCount(), (size_t)0);
    CHECK_EQ(C3Engine::getInstance().getCacheStats().entries, (size_t)0);
    // The manager accepts work again after shutdown.
    H.recordCall(op::Neg, DeviceType::kCPU, {3});
    CHECK(H.getStats().calls_tracked >= 1);
}

#include "test_c3core_gpu.inc"

int main(int argc, char** argv) { return run_tests(argc, argv); }
