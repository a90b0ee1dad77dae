// C3Engine.cpp -- see include/C3/C3Engine.h.
#include "C3/C3Engine.h"

#include <chrono>
#include <cstdio>
#include <sstream>

#include "C3/GraphMerger.h"
#include "C3/HipCompiledKernel.h"
#include "C3/JITCache.h"
#include "C3/PGOManager.h"
#include "C3/RollingHash.h"
#include "c3hip.h"

namespace ct {
namespace c3 {

namespace {

const char* kindName(KernelKind k) {
    switch (k) {
        case KernelKind::Elementwise: return "elementwise";
        case KernelKind::MatMul: return "matmul";
        case KernelKind::LinearFwd: return "linear_fwd";
        case KernelKind::ReLUBackward: return "relu_bwd";
        case KernelKind::UnaryBackward: return "unary_bwd";
        case KernelKind::DivBackwardB: return "div_bwd_b";
        case KernelKind::AddBackwardLhs: return "add_bwd_lhs";
        case KernelKind::SumReduce: return "sum_reduce";
        case KernelKind::MatMulBackwardA: return "matmul_bwd_a";
        case KernelKind::MatMulBackwardB: return "matmul_bwd_b";
        case KernelKind::LinearBwd: return "linear_bwd";
        case KernelKind::BackwardChain: return "bwd_chain";
    }
    return "?";
}

// The default backend: resolve the spec's code object through the JIT cache
// and wrap the spec in a HipCompiledKernel.  The authoritative image is the
// prebuilt code object the library ships beside itself; a cache entry is used
// only when it holds that same image (same SHA-256; entries from another
// build or with a damaged object are evicted by the lookup), otherwise the
// prebuilt image is read and cached.  Either way the image is handed to
// c3hip_load_code_object, which loads it or, when the module is already
// loaded on the device, checks that it is the loaded image.
std::shared_ptr<CompiledKernel> hipFactory(const KernelSpec& spec, const CompileOptions& opts, std::string* err) {
    const std::string spec_str = spec.toString();
    const std::string key = JITCache::makeKey(spec_str, opts.opt_level);
    const std::string module = spec.moduleName();
    if (!module.empty() && opts.use_cache && JITCache::isEnabled()) {
        JITCache& cache = JITCache::getInstance();
        char path[4096];
        if (c3hip_code_object_path(module.c_str(), path, sizeof(path)) != C3HIP_OK) {
            *err = "no code object path for module " + module;
            return nullptr;
        }
        const std::string prebuilt_sha = cache.fileSha(path);
        if (prebuilt_sha.empty()) {
            *err = std::string("prebuilt code object ") + path + " not found";
            return nullptr;
        }
        std::vector<char> image;
        const std::string hit = cache.lookup(key, prebuilt_sha);
        if (!hit.empty()) {
            if (!JITCache::readFile(hit, &image) || image.empty()) {
                *err = "JITCache: cannot read " + hit;
                return nullptr;
            }
        } else {
            if (!JITCache::readFile(path, &image) || image.empty()) {
                *err = std::string("cannot read prebuilt code object ") + path;
                return nullptr;
            }
            (void)cache.store(key, image, {"module=" + module, "spec=" + spec_str});
        }
        if (c3hip_load_code_object(module.c_str(), image.data(), image.size()) != C3HIP_OK) {
            *err = std::string("loading code object failed: ") + c3hip_last_error();
            return nullptr;
        }
    }
    return std::make_shared<HipCompiledKernel>(spec, opts.opt_level, key);
}

}  // namespace

std::string KernelSpec::toString() const {
    std::ostringstream ss;
    ss << "rh=" << std::hex << RollingHash::hashSequence(op_seq) << std::dec << "|kind=" << kindName(kind)
       << "|ew=" << ew_op << "|alpha=" << alpha << "|act=" << act << "|t=" << transA << transB << "|axis=" << axis
       << "|dtype=" << static_cast<int>(dtype);
    if (!chain.empty()) {
        ss << "|chain=";
        for (int c : chain) ss << c << ",";
    }
    if (!tile.empty()) ss << "|tile=" << tile;
    if (kind == KernelKind::LinearBwd && !input_grad) ss << "|nodx";
    ss << "|in=";
    for (const auto& s : input_shapes) ss << shapeToString(s) << ";";
    ss << "|out=" << shapeToString(out_shape);
    return ss.str();
}

std::string KernelSpec::moduleName() const {
    switch (kind) {
        case KernelKind::Elementwise:
        case KernelKind::ReLUBackward:
        case KernelKind::UnaryBackward:
        case KernelKind::DivBackwardB:
        case KernelKind::BackwardChain: return "elementwise";
        case KernelKind::SumReduce: return "reduce";
        case KernelKind::AddBackwardLhs: return "";
        default: return dtype == DType::kBFloat16 ? "gemm_bf16" : "gemm_f32";
    }
}

std::vector<std::pair<std::vector<size_t>, DType>> KernelSpec::outputDescs() const {
    switch (kind) {
        case KernelKind::LinearBwd: {
            // [dY, X, W, Y] -> dX (X's type), dW and db (fp32)
            if (input_shapes.size() != 4) return {};
            const auto& X = input_shapes[1];
            const auto& W = input_shapes[2];
            if (X.size() != 2 || W.size() != 2) return {};
            // Without the input gradient output 0 is an empty tensor (shape {0}).
            return {{input_grad ? X : std::vector<size_t>{0}, dtype}, {{X[1], W[1]}, DType::kFloat},
                    {{W[1]}, DType::kFloat}};
        }
        case KernelKind::BackwardChain: {
            std::vector<std::pair<std::vector<size_t>, DType>> o;
            for (size_t k = 0; k < chain.size(); ++k) o.push_back({out_shape, DType::kFloat});
            return o;
        }
        case KernelKind::MatMul:
        case KernelKind::LinearFwd:
        case KernelKind::MatMulBackwardA:
        case KernelKind::MatMulBackwardB: return {{out_shape, dtype}};
        default: return {{out_shape, DType::kFloat}};
    }
}

DType KernelSpec::inputDtype(size_t j) const {
    if (kind == KernelKind::LinearFwd && j == 2) return DType::kFloat;  // the bias row
    return dtype;
}

bool KernelSpec::hasGemm() const {
    switch (kind) {
        case KernelKind::MatMul:
        case KernelKind::LinearFwd:
        case KernelKind::LinearBwd:
        case KernelKind::MatMulBackwardA:
        case KernelKind::MatMulBackwardB: return true;
        default: return false;
    }
}

C3Engine& C3Engine::getInstance() {
    static C3Engine e;
    return e;
}

void C3Engine::setLastError(const std::string& e) {
    std::lock_guard<std::mutex> lk(mu_);
    last_error_ = e.size() > 1024 ? e.substr(0, 1024) : e;
}

std::string C3Engine::getLastCompileError() const {
    std::lock_guard<std::mutex> lk(mu_);
    return last_error_;
}

void C3Engine::setFactoryForTest(Factory f) {
    std::lock_guard<std::mutex> lk(mu_);
    factory_ = std::move(f);
    cache_.clear();
}

bool C3Engine::hasFactoryForTest() const {
    std::lock_guard<std::mutex> lk(mu_);
    return static_cast<bool>(factory_);
}

std::shared_ptr<ProfileData> C3Engine::profileData(const std::string& key) {
    std::lock_guard<std::mutex> lk(mu_);
    auto& p = profiles_[key];
    if (!p) p = std::make_shared<ProfileData>();
    return p;
}

void C3Engine::recordCompileError(const std::string& tier, const std::string& reason) {
    setLastError("[" + tier + "] " + reason);
}

std::shared_ptr<CompiledKernel> C3Engine::compile(const KernelSpec& spec, const CompileOptions& opts) {
    if (shutting_down_.load()) return nullptr;
    if (opts.pgo_mode) {
        // Tiered kernel, one per (options, spec) (src/C3/C3Engine.cpp:838-861).
        auto& pgo = PGOManager::getInstance();
        if (!pgo.isEnabled()) pgo.setEnabled(true);
        const std::string key = "pgo|" + std::to_string(opts.opt_level) + "|" + spec.toString();
        return pgo.registerKernel(PGOPlan{{spec}, {}}, opts, key, profileData(key), *this);
    }
    const std::string ckey = std::to_string(opts.opt_level) + "|" + spec.toString();
    Factory factory;
    {
        std::lock_guard<std::mutex> lk(mu_);
        auto it = cache_.find(ckey);
        if (it != cache_.end()) {
            hits_++;
            return it->second;
        }
        factory = factory_;
    }
    misses_++;
    compiles_++;
    std::shared_ptr<CompiledKernel> k;
    std::string err;
    try {
        k = factory ? factory(spec, opts) : hipFactory(spec, opts, &err);
    } catch (const std::exception& e) {
        err = e.what();
        k = nullptr;
    }
    if (!k) {
        setLastError("[O" + std::to_string(opts.opt_level) + "] " + (err.empty() ? "compile failed" : err));
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(mu_);
    if (cache_.size() >= 256) cache_.erase(cache_.begin());
    cache_.emplace(ckey, k);
    return k;
}

C3Engine::CompileFuture C3Engine::compileAsync(const KernelSpec& spec, const CompileOptions& opts) {
    auto work = std::async(std::launch::async, [this, spec, opts] { return compile(spec, opts); }).share();
    const uint32_t tmo = compile_timeout_ms_.load();
    auto watch = std::async(std::launch::async, [this, work, tmo]() -> std::shared_ptr<CompiledKernel> {
                     if (work.wait_for(std::chrono::milliseconds(tmo)) != std::future_status::ready) {
                         timeouts_++;
                         setLastError("[async-timeout] compile exceeded " + std::to_string(tmo) + " ms");
                         return nullptr;
                     }
                     try {
                         return work.get();
                     } catch (...) {
                         return nullptr;
                     }
                 }).share();
    {
        std::lock_guard<std::mutex> lk(mu_);
        workers_.push_back(std::async(std::launch::async, [work, watch] {
            work.wait();
            watch.wait();
        }));
    }
    return watch;
}

std::shared_ptr<CompiledKernel> C3Engine::compileMerged(const std::vector<KernelSpec>& subs, const MergeSpec& spec,
                                                        const CompileOptions& opts) {
    const std::string err = GraphMerger::validate(subs, spec);
    if (!err.empty()) throw std::invalid_argument("C3Engine::compileMerged: " + err);
    const std::string key = std::to_string(opts.opt_level) + "|" + GraphMerger::mergedCacheKey(subs, spec);
    {
        std::lock_guard<std::mutex> lk(mu_);
        auto it = cache_.find(key);
        if (it != cache_.end()) {
            hits_++;
            return it->second;
        }
    }
    CompileOptions sub_opts = opts;
    sub_opts.pgo_mode = false;
    std::vector<std::shared_ptr<CompiledKernel>> ks;
    for (size_t i = 0; i < subs.size(); ++i) {
        auto k = compile(subs[i], sub_opts);
        if (!k)
            throw std::runtime_error("C3Engine::compileMerged: sub-kernel " + std::to_string(i) +
                                     " did not compile: " + getLastCompileError());
        ks.push_back(std::move(k));
    }
    auto merged = std::make_shared<MergedCompiledKernel>(std::move(ks), subs, spec, key, opts.opt_level);
    std::lock_guard<std::mutex> lk(mu_);
    if (cache_.size() >= 256) cache_.erase(cache_.begin());
    cache_.emplace(key, merged);
    return merged;
}

std::shared_ptr<CompiledKernel> C3Engine::compileMergedSequential(const std::vector<KernelSpec>& subs,
                                                                  const CompileOptions& opts) {
    return compileMerged(subs, GraphMerger::makeSequentialSpec(subs), opts);
}

C3Engine::CompileFuture C3Engine::compileMergedAsync(const std::vector<KernelSpec>& subs, const MergeSpec& spec,
                                                     const CompileOptions& opts) {
    const std::string key = std::to_string(opts.opt_level) + "|" + std::to_string(opts.pgo_mode) + "|" +
                            GraphMerger::mergedCacheKey(subs, spec);
    std::lock_guard<std::mutex> lk(mu_);
    auto it = merged_async_.find(key);
    if (it != merged_async_.end()) return it->second;
    auto fut = std::async(std::launch::async, [this, subs, spec, opts]() -> std::shared_ptr<CompiledKernel> {
                   return opts.pgo_mode ? compileMergedPGO(subs, spec, opts) : compileMerged(subs, spec, opts);
               }).share();
    merged_async_.emplace(key, fut);
    workers_.push_back(std::async(std::launch::async, [fut] { fut.wait(); }));
    return fut;
}

std::shared_ptr<CompiledKernel> C3Engine::compileMergedPGO(const std::vector<KernelSpec>& subs, const MergeSpec& spec,
                                                           const CompileOptions& opts) {
    const std::string err = GraphMerger::validate(subs, spec);
    if (!err.empty()) throw std::invalid_argument("C3Engine::compileMergedPGO: " + err);
    CompileOptions pgo_opts = opts;
    pgo_opts.pgo_mode = true;
    auto& pgo = PGOManager::getInstance();
    if (!pgo.isEnabled()) pgo.setEnabled(true);
    const std::string key = "pgo|" + std::to_string(opts.opt_level) + "|" + GraphMerger::mergedCacheKey(subs, spec);
    return pgo.registerKernel(PGOPlan{subs, spec}, pgo_opts, key, profileData(key), *this);
}

std::shared_ptr<CompiledKernel> C3Engine::compileMergedPGOSequential(const std::vector<KernelSpec>& subs,
                                                                     const CompileOptions& opts) {
    return compileMergedPGO(subs, GraphMerger::makeSequentialSpec(subs), opts);
}

C3CacheStats C3Engine::getCacheStats() const {
    C3CacheStats s;
    s.hits = hits_.load();
    s.misses = misses_.load();
    s.compile_count = compiles_.load();
    s.async_timeouts = timeouts_.load();
    std::lock_guard<std::mutex> lk(mu_);
    s.entries = cache_.size();
    return s;
}

void C3Engine::clearCache() {
    {
        std::lock_guard<std::mutex> lk(mu_);
        cache_.clear();
        profiles_.clear();
        merged_async_.clear();
    }
    // The tiered kernels go with the cache (src/C3/C3Engine.cpp:1572-1574).
    PGOManager::getInstance().clear();
}

void C3Engine::shutdown() {
    PGOManager::getInstance().shutdown();  // background compile chains first
    shutting_down_.store(true);
    std::vector<std::future<void>> ws;
    {
        std::lock_guard<std::mutex> lk(mu_);
        ws.swap(workers_);
    }
    for (auto& w : ws)
        if (w.valid() && w.wait_for(std::chrono::seconds(30)) != std::future_status::ready)
            c3log(ErrorLevel::WARN, "C3Engine::shutdown: a background compile did not finish in 30 s");
    clearCache();
    shutting_down_.store(false);
}

}  // namespace c3
}  // namespace ct
