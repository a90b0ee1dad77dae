// PGOManager.cpp -- see include/C3/PGOManager.h.
#include "C3/PGOManager.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <sstream>

#include "C3/HipCompiledKernel.h"
#include "c3hip.h"

namespace ct {
namespace c3 {

namespace {

uint64_t nowNs() {
    return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

double median(std::vector<double> v) {
    if (v.empty()) return -1.0;
    std::sort(v.begin(), v.end());
    return v[v.size() / 2];
}

std::vector<std::string> tileNames(DType dt) {
    char buf[512];
    if (c3hip_gemm_tile_names(dt == DType::kBFloat16 ? C3HIP_BF16 : C3HIP_F32, buf, sizeof(buf)) != C3HIP_OK) return {};
    std::vector<std::string> names;
    std::stringstream ss(buf);
    std::string item;
    while (std::getline(ss, item, ','))
        if (!item.empty()) names.push_back(item);
    return names;
}

// Tier 1: the pattern op by op through single-op kernels (each a node of the
// reference's interpreted graph); patterns with no op-by-op form at their
// element type (bf16 has no single elementwise kernels) run as one call.
std::vector<Tensor> interpretOnDevice(const KernelSpec& s, const std::vector<Tensor>& in) {
    auto single = [](KernelSpec t, const std::vector<Tensor>& x) {
        HipCompiledKernel k(std::move(t), 0, "");
        return k.execute(x);
    };
    auto ew = [&](int code, const std::vector<Tensor>& x) {
        KernelSpec t;
        t.kind = KernelKind::Elementwise;
        t.ew_op = code;
        return single(t, x)[0];
    };
    if (s.kind == KernelKind::LinearFwd && s.dtype == DType::kFloat && s.act >= C3HIP_ACT_NONE &&
        s.act <= C3HIP_ACT_TANH && in.size() >= 2) {
        KernelSpec mm;
        mm.kind = KernelKind::MatMul;
        Tensor t = single(mm, {in[0], in[1]})[0];
        if (in.size() == 3) t = ew(C3HIP_EW_ADD, {t, in[2]});
        static const int kAct[] = {-1, C3HIP_EW_RELU, C3HIP_EW_SIGMOID, C3HIP_EW_TANH};
        if (s.act != C3HIP_ACT_NONE) t = ew(kAct[s.act], {t});
        return {t};
    }
    if (s.kind == KernelKind::LinearBwd && s.dtype == DType::kFloat && s.act <= C3HIP_ACT_RELU && in.size() == 4) {
        // [dY, X, W, Y]: dZ = relu mask(Y) * dY; dX = dZ W^T; dW = X^T dZ; db = colsum dZ.
        Tensor dZ = in[0];
        if (s.act == C3HIP_ACT_RELU) {
            KernelSpec r;
            r.kind = KernelKind::ReLUBackward;
            dZ = single(r, {in[0], in[3]})[0];
        }
        KernelSpec a, b, c;
        a.kind = KernelKind::MatMulBackwardA;
        b.kind = KernelKind::MatMulBackwardB;
        c.kind = KernelKind::SumReduce;
        c.axis = 0;
        return {single(a, {dZ, in[2]})[0], single(b, {dZ, in[1]})[0], single(c, {dZ})[0]};
    }
    if (s.kind == KernelKind::BackwardChain && in.size() == s.chain.size() + 1) {
        std::vector<Tensor> outs;
        Tensor g = in[0];
        for (size_t k = 0; k < s.chain.size(); ++k) {
            const Tensor& x = in[1 + k];
            KernelSpec t;
            switch (s.chain[k]) {
                case C3HIP_CHAIN_RELU: t.kind = KernelKind::ReLUBackward; g = single(t, {g, x})[0]; break;
                case C3HIP_CHAIN_SIGMOID:
                case C3HIP_CHAIN_TANH:
                case C3HIP_CHAIN_EXP:
                    t.kind = KernelKind::UnaryBackward;
                    t.ew_op = s.chain[k] == C3HIP_CHAIN_SIGMOID ? C3HIP_EW_SIGMOID_BWD
                              : s.chain[k] == C3HIP_CHAIN_TANH  ? C3HIP_EW_TANH_BWD
                                                                : C3HIP_EW_EXP_BWD;
                    g = single(t, {g, x})[0];
                    break;
                case C3HIP_CHAIN_LOG: g = ew(C3HIP_EW_DIV, {g, x}); break;
                default: g = ew(C3HIP_EW_NEG, {g}); break;
            }
            outs.push_back(g);
        }
        return outs;
    }
    KernelSpec t = s;
    t.tile.clear();
    return single(t, in);
}

}  // namespace

// ------------------------------------------------------------- TunedKernel --

TunedKernel::TunedKernel(std::vector<Candidate> candidates, int samples, std::string cache_key)
    : samples_(std::max(1, samples)), key_(std::move(cache_key)) {
    for (auto& c : candidates) cands_.push_back(Slot{std::move(c), {}, 0, false});
    opt_level_ = 3;
}

TunedKernel::~TunedKernel() {
    std::lock_guard<std::mutex> lk(mu_);
    for (auto& p : pending_) {
        (void)hipEventDestroy((hipEvent_t)p.start);
        (void)hipEventDestroy((hipEvent_t)p.stop);
    }
    pending_.clear();
}

DeviceType TunedKernel::targetDevice() const {
    return cands_.empty() ? DeviceType::kHIP : cands_.front().c.kernel->targetDevice();
}

void TunedKernel::pollLocked(bool wait) {
    for (size_t i = 0; i < pending_.size();) {
        Pending& p = pending_[i];
        hipError_t e = wait ? hipEventSynchronize((hipEvent_t)p.stop) : hipEventQuery((hipEvent_t)p.stop);
        if (e == hipErrorNotReady) {
            ++i;
            continue;
        }
        float ms = -1.0f;
        if (e == hipSuccess && hipEventElapsedTime(&ms, (hipEvent_t)p.start, (hipEvent_t)p.stop) == hipSuccess)
            cands_[p.cand].ms.push_back(ms);
        (void)hipEventDestroy((hipEvent_t)p.start);
        (void)hipEventDestroy((hipEvent_t)p.stop);
        pending_.erase(pending_.begin() + (std::ptrdiff_t)i);
    }
}

void TunedKernel::finishIfDoneLocked() {
    if (best_ >= 0) return;
    double best_ms = 0.0;
    long best = -1;
    for (size_t i = 0; i < cands_.size(); ++i) {
        const Slot& s = cands_[i];
        if (s.dropped) continue;
        if ((int)s.ms.size() < samples_) return;  // still measuring
        const double m = median(s.ms);
        if (best < 0 || m < best_ms) {
            best = (long)i;
            best_ms = m;
        }
    }
    best_ = best;
}

std::vector<Tensor> TunedKernel::execute(const std::vector<Tensor>& inputs) {
    std::unique_lock<std::mutex> lk(mu_);
    pollLocked(false);
    finishIfDoneLocked();
    if (best_ >= 0) {
        auto k = cands_[(size_t)best_].c.kernel;
        lk.unlock();
        return k->execute(inputs);
    }
    const bool hip = targetDevice() == DeviceType::kHIP;
    void* stream = getCurrentStream();
    bool capturing = false;
    if (hip) {
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        capturing = hipStreamIsCapturing((hipStream_t)stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
    }
    for (;;) {
        // Next candidate still owed a launch (one warm-up + samples_ timed), round robin.
        long pick = -1;
        if (!capturing) {
            for (size_t n = 0; n < cands_.size(); ++n) {
                const size_t i = (next_ + n) % cands_.size();
                if (!cands_[i].dropped && cands_[i].launched < samples_ + 1) {
                    pick = (long)i;
                    break;
                }
            }
        }
        bool timed = false;
        const bool owed = pick >= 0;
        if (owed) {
            next_ = (size_t)pick + 1;
            timed = cands_[(size_t)pick].launched >= 1;
        } else {
            // Every candidate has been launched (timings in flight) or the
            // stream is capturing: the first candidate still standing, untimed.
            for (size_t i = 0; i < cands_.size() && pick < 0; ++i)
                if (!cands_[i].dropped) pick = (long)i;
            if (pick < 0) throw std::runtime_error("TunedKernel: every candidate failed");
        }
        Slot& s = cands_[(size_t)pick];
        hipEvent_t e0 = nullptr, e1 = nullptr;
        if (timed && hip) {
            if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess ||
                hipEventRecord(e0, (hipStream_t)stream) != hipSuccess) {
                if (e0) (void)hipEventDestroy(e0);
                if (e1) (void)hipEventDestroy(e1);
                e0 = e1 = nullptr;
                timed = false;
            }
        }
        const uint64_t t0 = nowNs();
        std::vector<Tensor> out;
        try {
            out = s.c.kernel->execute(inputs);
        } catch (...) {
            // This launch configuration cannot run the call: drop it and serve
            // the call with the next candidate.
            s.dropped = true;
            if (e0) (void)hipEventDestroy(e0);
            if (e1) (void)hipEventDestroy(e1);
            finishIfDoneLocked();
            if (best_ >= 0) {
                auto k = cands_[(size_t)best_].c.kernel;
                lk.unlock();
                return k->execute(inputs);
            }
            continue;
        }
        if (owed) s.launched++;
        if (timed) {
            if (hip) {
                if (hipEventRecord(e1, (hipStream_t)stream) == hipSuccess) {
                    pending_.push_back(Pending{(size_t)pick, (void*)e0, (void*)e1});
                } else {
                    (void)hipEventDestroy(e0);
                    (void)hipEventDestroy(e1);
                    s.launched--;  // measure it again
                }
            } else {
                s.ms.push_back((double)(nowNs() - t0) * 1e-6);
            }
        }
        finishIfDoneLocked();
        return out;
    }
}

bool TunedKernel::tuned() const {
    std::lock_guard<std::mutex> lk(mu_);
    return best_ >= 0;
}

std::string TunedKernel::chosen() const {
    std::lock_guard<std::mutex> lk(mu_);
    return best_ >= 0 ? cands_[(size_t)best_].c.name : std::string();
}

std::vector<std::pair<std::string, double>> TunedKernel::timings() const {
    std::lock_guard<std::mutex> lk(mu_);
    std::vector<std::pair<std::string, double>> r;
    for (const auto& s : cands_) r.push_back({s.c.name, s.dropped ? -1.0 : median(s.ms)});
    return r;
}

// ------------------------------------------------------- PGOCompiledKernel --

PGOCompiledKernel::PGOCompiledKernel(PGOPlan plan, CompileOptions options, std::string cache_key,
                                     std::shared_ptr<ProfileData> profile, C3Engine& engine)
    : plan_(std::move(plan)), options_(options), key_(std::move(cache_key)), profile_(std::move(profile)),
      engine_(engine) {
    info_ = GraphMerger::merge(plan_.subs, plan_.links);
    opt_level_ = options_.opt_level;
}

std::vector<Tensor> PGOCompiledKernel::execute(const std::vector<Tensor>& inputs) {
    // Ofast, then O2, then eager; a tier that throws is disabled for good
    // (src/C3/PGOManager.cpp:109-166).
    std::shared_ptr<CompiledKernel> k;
    {
        std::lock_guard<std::mutex> lk(mu_);
        k = ofast_;
    }
    if (k && !ofast_disabled_.load()) {
        try {
            const uint64_t t0 = nowNs();
            auto r = k->execute(inputs);
            profile_->record(nowNs() - t0);
            return r;
        } catch (const std::exception& e) {
            recordDeopt("ofast", e.what());
        } catch (...) {
            recordDeopt("ofast", "unknown exception");
        }
        ofast_disabled_.store(true);
    }
    {
        std::lock_guard<std::mutex> lk(mu_);
        k = o2_;
    }
    if (k && !o2_disabled_.load()) {
        try {
            const uint64_t t0 = nowNs();
            auto r = k->execute(inputs);
            profile_->record(nowNs() - t0);
            return r;
        } catch (const std::exception& e) {
            recordDeopt("o2", e.what());
        } catch (...) {
            recordDeopt("o2", "unknown exception");
        }
        o2_disabled_.store(true);
    }
    const uint64_t t0 = nowNs();
    auto r = executeInterpreted(inputs);
    profile_->record(nowNs() - t0);
    if (!triggered_.exchange(true)) triggerCompilationChain();
    return r;
}

std::vector<Tensor> PGOCompiledKernel::executeInterpreted(const std::vector<Tensor>& inputs) {
    auto& pgo = PGOManager::getInstance();
    return MergedCompiledKernel::run(plan_.subs, info_, inputs, [&](size_t i, const std::vector<Tensor>& in) {
        return pgo.interpret(plan_.subs[i], in);
    });
}

void PGOCompiledKernel::recordDeopt(const char* tier, const std::string& reason) {
    deopts_++;
    {
        std::lock_guard<std::mutex> lk(err_mu_);
        last_deopt_ = std::string(tier) + ": " + reason;
    }
    c3log(ErrorLevel::WARN, "PGO: deopt " + std::string(tier) + " kernel for " + key_ + " -- " + reason);
}

void PGOCompiledKernel::recordCompileError(const char* tier, const std::string& reason) {
    std::string r = reason;
    if (r.size() > 1024) r = r.substr(0, 1024) + "... [truncated, original=" + std::to_string(reason.size()) + " bytes]";
    {
        std::lock_guard<std::mutex> lk(err_mu_);
        last_compile_error_ = std::string(tier) + ": " + r;
    }
    c3log(ErrorLevel::WARN, "PGO: compile error " + std::string(tier) + " for " + key_ + " -- " + r);
    try {
        engine_.recordCompileError(tier, r);
    } catch (...) {
    }
}

std::string PGOCompiledKernel::lastDeoptReason() const {
    std::lock_guard<std::mutex> lk(err_mu_);
    return last_deopt_;
}

std::string PGOCompiledKernel::lastCompileError() const {
    std::lock_guard<std::mutex> lk(err_mu_);
    return last_compile_error_;
}

void PGOCompiledKernel::clearLastCompileError() {
    std::lock_guard<std::mutex> lk(err_mu_);
    last_compile_error_.clear();
}

bool PGOCompiledKernel::isPromoted() const {
    std::lock_guard<std::mutex> lk(mu_);
    return o2_ || ofast_;
}

std::shared_ptr<CompiledKernel> PGOCompiledKernel::o2Kernel() const {
    std::lock_guard<std::mutex> lk(mu_);
    return o2_;
}

std::shared_ptr<CompiledKernel> PGOCompiledKernel::ofastKernel() const {
    std::lock_guard<std::mutex> lk(mu_);
    return ofast_;
}

std::vector<std::shared_ptr<TunedKernel>> PGOCompiledKernel::tuners() const {
    std::lock_guard<std::mutex> lk(mu_);
    return tuners_;
}

void PGOCompiledKernel::triggerCompilationChain() {
    auto& pgo = PGOManager::getInstance();
    auto self = shared_from_this();
    if (!pgo.canAcceptCompilation()) {
        // Back-pressure: queue the chain by heat and stay on eager; the next
        // call may trigger again (src/C3/PGOManager.cpp:215-246).
        const double heat = computeHeatScore();
        auto task = [self, &pgo]() {
            pgo.notifyCompilationStarted();
            self->compileO2();
            self->compileOfast();
            pgo.notifyCompilationCompleted();
        };
        {
            std::lock_guard<std::mutex> lk(pgo.queue_mutex());
            pgo.task_queue().push(CompilationTask{heat, std::move(task), std::chrono::steady_clock::now(), "PGO: " + key_});
        }
        pgo.recordQueueRejection();
        triggered_.store(false);
        return;
    }
    pgo.notifyCompilationStarted();
    if (pgo.config().async_compilation) {
        pgo.addFuture(std::async(std::launch::async, [self]() {
            try {
                self->compileO2();
                self->compileOfast();
            } catch (const std::exception& e) {
                c3log(ErrorLevel::WARN, "PGO: compile chain exception for " + self->key_ + ": " + e.what());
            } catch (...) {
                c3log(ErrorLevel::WARN, "PGO: compile chain exception for " + self->key_);
            }
            PGOManager::getInstance().notifyCompilationCompleted();
        }));
    } else {
        compileO2();
        compileOfast();
        pgo.notifyCompilationCompleted();
    }
}

void PGOCompiledKernel::compileO2() {
    try {
        CompileOptions o = options_;
        o.opt_level = 2;
        o.pgo_mode = false;
        std::shared_ptr<CompiledKernel> k = plan_.subs.size() == 1 ? engine_.compile(plan_.subs[0], o)
                                                                   : engine_.compileMerged(plan_.subs, plan_.links, o);
        if (!k) {
            recordCompileError("o2", "compile returned nullptr: " + engine_.getLastCompileError());
            return;
        }
        std::lock_guard<std::mutex> lk(mu_);
        o2_ = std::move(k);
    } catch (const std::exception& e) {
        recordCompileError("o2", e.what());
    } catch (...) {
        recordCompileError("o2", "unknown exception");
    }
}

void PGOCompiledKernel::compileOfast() {
    try {
        CompileOptions o = options_;
        o.opt_level = 3;
        o.pgo_mode = false;
        CompileOptions cand_opts = o;
        cand_opts.use_cache = false;  // transient candidates: not written to the JIT cache
        std::vector<std::shared_ptr<CompiledKernel>> ks;
        std::vector<std::shared_ptr<TunedKernel>> tuners;
        for (size_t i = 0; i < plan_.subs.size(); ++i) {
            const KernelSpec& s = plan_.subs[i];
            std::shared_ptr<CompiledKernel> k;
            std::shared_ptr<TunedKernel> tuner;
            if (s.hasGemm() && s.tile.empty()) {
                std::vector<TunedKernel::Candidate> cands;
                for (const std::string& name : tileNames(s.dtype)) {
                    KernelSpec c = s;
                    c.tile = name;
                    if (auto ck = engine_.compile(c, cand_opts)) cands.push_back({name, ck});
                }
                if (cands.size() == 1) k = cands[0].kernel;
                if (cands.size() > 1) {
                    tuner = std::make_shared<TunedKernel>(std::move(cands), PGOManager::getInstance().config().tune_samples,
                                                          key_ + "|ofast|" + std::to_string(i));
                    k = tuner;
                }
            } else {
                k = engine_.compile(s, o);
            }
            if (!k) {
                recordCompileError("ofast", "sub-kernel " + std::to_string(i) + " did not compile: " +
                                                engine_.getLastCompileError());
                return;
            }
            ks.push_back(std::move(k));
            tuners.push_back(std::move(tuner));
        }
        std::shared_ptr<CompiledKernel> k =
            ks.size() == 1 ? ks[0]
                           : std::make_shared<MergedCompiledKernel>(std::move(ks), plan_.subs, plan_.links,
                                                                    key_ + "|ofast", 3);
        std::lock_guard<std::mutex> lk(mu_);
        ofast_ = std::move(k);
        tuners_ = std::move(tuners);
    } catch (const std::exception& e) {
        recordCompileError("ofast", e.what());
    } catch (...) {
        recordCompileError("ofast", "unknown exception");
    }
}

void PGOCompiledKernel::promote() {
    if (triggered_.exchange(true)) {
        if (!isPromoted()) {
            compileO2();
            compileOfast();
        }
        return;
    }
    compileO2();
    compileOfast();
}

double PGOCompiledKernel::computeHeatScore() const {
    // 0.4 x log-saturating call count + 0.6 x accumulated time against 1 s
    // (src/C3/PGOManager.cpp:368-384).
    const uint64_t calls = profile_->call_count.load();
    if (calls == 0) return 0.0;
    const double window = (double)PGOManager::getInstance().config().heat_score_window_calls;
    const double call_score = std::min(1.0, std::log2(1.0 + (double)calls) / std::log2(1.0 + window));
    const double time_score = std::min(1.0, (double)profile_->total_time_ns.load() / 1e9);
    return 0.4 * call_score + 0.6 * time_score;
}

// --------------------------------------------------------------- PGOManager --

PGOManager& PGOManager::getInstance() {
    static PGOManager m;
    return m;
}

std::shared_ptr<PGOCompiledKernel> PGOManager::registerKernel(PGOPlan plan, const CompileOptions& options,
                                                              std::string cache_key,
                                                              std::shared_ptr<ProfileData> profile,
                                                              C3Engine& engine) {
    std::lock_guard<std::mutex> lk(mu_);
    auto it = cache_.find(cache_key);
    if (it != cache_.end() && it->second) return it->second;
    auto k = std::make_shared<PGOCompiledKernel>(std::move(plan), options, cache_key, std::move(profile), engine);
    entries_.push_back(k);
    cache_[cache_key] = k;
    return k;
}

bool PGOManager::canAcceptCompilation() const {
    if (active_.load() >= config_.max_concurrent_compilations) return false;
    std::lock_guard<std::mutex> lk(queue_mu_);
    return queue_.size() < config_.queue_backpressure_threshold;
}

void PGOManager::notifyCompilationStarted() { active_++; }

void PGOManager::notifyCompilationCompleted() {
    active_--;
    processQueue();
}

void PGOManager::recordQueueRejection() { rejections_++; }

void PGOManager::processQueue() {
    CompilationTask task;
    {
        std::lock_guard<std::mutex> lk(queue_mu_);
        if (queue_.empty()) return;
        task = queue_.top();
        queue_.pop();
    }
    try {
        if (task.task) task.task();
    } catch (...) {
    }
}

void PGOManager::clear() {
    std::lock_guard<std::mutex> lk(mu_);
    entries_.clear();
    cache_.clear();
    active_.store(0);
    rejections_.store(0);
    std::lock_guard<std::mutex> qk(queue_mu_);
    std::priority_queue<CompilationTask> empty;
    std::swap(queue_, empty);
}

PGOManager::Stats PGOManager::getStats() const {
    Stats s;
    std::lock_guard<std::mutex> lk(mu_);
    s.total_registered = entries_.size();
    s.active_compilations = active_.load();
    s.queue_rejections = rejections_.load();
    for (const auto& e : entries_) {
        const bool o2 = e->o2Kernel() != nullptr, of = e->ofastKernel() != nullptr;
        if (of) s.ofast_ready++;
        if (o2) s.o2_ready++;
        if (!o2 && !of) s.pending++;
    }
    std::lock_guard<std::mutex> qk(queue_mu_);
    s.queued = queue_.size();
    return s;
}

void PGOManager::promoteAll() {
    std::vector<std::shared_ptr<PGOCompiledKernel>> es;
    {
        std::lock_guard<std::mutex> lk(mu_);
        es = entries_;
    }
    for (auto& e : es) e->promote();
}

void PGOManager::addFuture(std::future<void> f) {
    std::lock_guard<std::mutex> lk(futures_mu_);
    futures_.push_back(std::move(f));
}

void PGOManager::shutdown() {
    std::vector<std::future<void>> fs;
    {
        std::lock_guard<std::mutex> lk(futures_mu_);
        fs.swap(futures_);
    }
    for (auto& f : fs) {
        if (!f.valid()) continue;
        if (f.wait_for(std::chrono::seconds(30)) == std::future_status::ready) {
            try {
                f.get();
            } catch (...) {
            }
        } else {
            c3log(ErrorLevel::WARN, "PGOManager::shutdown: a background compile chain did not finish in 30 s");
        }
    }
}

void PGOManager::setInterpreterForTest(Interpreter f) {
    std::lock_guard<std::mutex> lk(interp_mu_);
    interp_ = std::move(f);
}

std::vector<Tensor> PGOManager::interpret(const KernelSpec& spec, const std::vector<Tensor>& inputs) {
    Interpreter f;
    {
        std::lock_guard<std::mutex> lk(interp_mu_);
        f = interp_;
    }
    return f ? f(spec, inputs) : interpretOnDevice(spec, inputs);
}

}  // namespace c3
}  // namespace ct
