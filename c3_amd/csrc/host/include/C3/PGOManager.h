// PGOManager.h -- tiered kernels (include/C3/PGOManager.h:1-336 and
// src/C3/PGOManager.cpp of the reference, re-designed for a GPU backend).
//
// A PGOCompiledKernel stands for one kernel or one merged chain of kernels
// and serves every call from the best tier available:
//   Tier 1 "eager":  the pattern op by op through the single-op kernels (the
//                    reference interprets the graph node by node); the first
//                    call also starts the compile chain.
//   Tier 2 "O2":     the prebuilt fused kernel with the size heuristic's tile.
//   Tier 3 "Ofast":  profile-guided.  The reference recompiles with -Ofast;
//                    on the GPU the choice that pays is the launch
//                    configuration, so Ofast holds every candidate GEMM tile
//                    of the pattern and times them on the caller's own calls
//                    (HIP events on the current stream; each call runs one
//                    candidate, so every call still computes its result),
//                    then keeps the fastest.  Patterns without a GEMM have one
//                    candidate and Ofast is that kernel.
// A tier whose execute() throws is disabled for good and the call falls back
// to the next tier (deoptimisation, ADR-006 of the reference); compile
// failures are recorded per tier and in the engine (ADR-007/-010).  Compile
// chains run asynchronously, at most max_concurrent_compilations at a time;
// beyond that, or with queue_backpressure_threshold chains queued, a chain
// waits in a priority queue ordered by heat score (0.4 * call score + 0.6 *
// time score, src/C3/PGOManager.cpp:368-384) and the kernel stays on eager.
//
// Different tiles sum in different orders, so the tiers agree to the fp32 /
// bf16 tolerance of the GEMM, not bit for bit.
#pragma once

#include <atomic>
#include <chrono>
#include <functional>
#include <future>
#include <memory>
#include <mutex>
#include <queue>
#include <string>
#include <unordered_map>
#include <vector>

#include "C3/C3Engine.h"
#include "C3/GraphMerger.h"

namespace ct {
namespace c3 {

struct PGOConfig {
    uint64_t max_concurrent_compilations = 4;
    uint64_t queue_backpressure_threshold = 32;
    uint64_t heat_score_window_calls = 1000;
    bool async_compilation = true;
    // Ofast tuning: timed calls per candidate (after one untimed warm-up call).
    int tune_samples = 3;
};

struct CompilationTask {
    double priority;
    std::function<void()> task;
    std::chrono::steady_clock::time_point created_at;
    std::string description;
    bool operator<(const CompilationTask& o) const { return priority < o.priority; }
};

// Ofast tier of one kernel: candidate launch configurations timed on real
// calls, then the fastest.  Timings of HIP kernels are HIP events recorded on
// the current stream and read once they complete (no synchronisation); host
// kernels are timed by the clock.  No timing while the stream is capturing a
// graph (the current best candidate runs).
// Bit reproducibility: while tuning, calls are served by the candidates in
// turn, and candidates need not add the k range in the same order (a tile
// forced for tuning never splits an fp32 GEMM over k, while the size
// heuristic splits small-grid ones; a forced bf16 direct tile splits by its
// own plan).  So on real-valued data, results may differ in the last bits
// between calls until the tuner has chosen; from then on one candidate
// serves every call.  Integer-valued (exactly summed) results never differ.
class TunedKernel : public CompiledKernel {
public:
    struct Candidate {
        std::string name;
        std::shared_ptr<CompiledKernel> kernel;
    };
    TunedKernel(std::vector<Candidate> candidates, int samples, std::string cache_key);
    ~TunedKernel() override;
    std::vector<Tensor> execute(const std::vector<Tensor>& inputs) override;
    const std::string& cacheKey() const override { return key_; }
    DeviceType targetDevice() const override;
    size_t workspaceBytes() const override { return 0; }

    bool tuned() const;
    // The chosen candidate's name ("" while tuning).
    std::string chosen() const;
    // Median time (ms) measured per candidate, negative when not measured or dropped.
    std::vector<std::pair<std::string, double>> timings() const;
    size_t candidateCount() const { return cands_.size(); }

private:
    struct Pending {
        size_t cand;
        void* start;
        void* stop;
    };
    void pollLocked(bool wait);
    void finishIfDoneLocked();

    struct Slot {
        Candidate c;
        std::vector<double> ms;
        int launched = 0;
        bool dropped = false;
    };
    std::vector<Slot> cands_;
    int samples_;
    std::string key_;
    mutable std::mutex mu_;
    std::vector<Pending> pending_;
    size_t next_ = 0;
    long best_ = -1;
};

// What a PGO kernel executes: one spec, or specs chained by a MergeSpec.
struct PGOPlan {
    std::vector<KernelSpec> subs;
    MergeSpec links;
};

class PGOCompiledKernel : public CompiledKernel, public std::enable_shared_from_this<PGOCompiledKernel> {
public:
    PGOCompiledKernel(PGOPlan plan, CompileOptions options, std::string cache_key,
                      std::shared_ptr<ProfileData> profile, C3Engine& engine);
    std::vector<Tensor> execute(const std::vector<Tensor>& inputs) override;
    const std::string& cacheKey() const override { return key_; }
    DeviceType targetDevice() const override { return DeviceType::kHIP; }
    size_t workspaceBytes() const override { return 0; }

    bool isPromoted() const;
    std::shared_ptr<CompiledKernel> o2Kernel() const;
    std::shared_ptr<CompiledKernel> ofastKernel() const;
    const ProfileData& profileData() const { return *profile_; }
    uint64_t deoptCount() const { return deopts_.load(); }
    std::string lastDeoptReason() const;
    bool isOfastDisabled() const { return ofast_disabled_.load(); }
    bool isO2Disabled() const { return o2_disabled_.load(); }
    std::string lastCompileError() const;
    void clearLastCompileError();
    void promote();
    double computeHeatScore() const;
    // The tuner of each sub-kernel's Ofast tier (null where there is one candidate).
    std::vector<std::shared_ptr<TunedKernel>> tuners() const;

private:
    friend class PGOManager;
    std::vector<Tensor> executeInterpreted(const std::vector<Tensor>& inputs);
    void triggerCompilationChain();
    void compileO2();
    void compileOfast();
    void recordDeopt(const char* tier, const std::string& reason);
    void recordCompileError(const char* tier, const std::string& reason);

    PGOPlan plan_;
    MergedSpecInfo info_;
    CompileOptions options_;
    std::string key_;
    std::shared_ptr<ProfileData> profile_;
    C3Engine& engine_;

    mutable std::mutex mu_;
    std::shared_ptr<CompiledKernel> o2_, ofast_;
    std::vector<std::shared_ptr<TunedKernel>> tuners_;
    std::atomic<bool> triggered_{false};
    std::atomic<bool> ofast_disabled_{false}, o2_disabled_{false};
    std::atomic<uint64_t> deopts_{0};
    mutable std::mutex err_mu_;
    std::string last_deopt_, last_compile_error_;
};

class PGOManager {
public:
    static PGOManager& getInstance();

    std::shared_ptr<PGOCompiledKernel> registerKernel(PGOPlan plan, const CompileOptions& options,
                                                      std::string cache_key, std::shared_ptr<ProfileData> profile,
                                                      C3Engine& engine);
    PGOConfig& config() { return config_; }
    const PGOConfig& config() const { return config_; }
    void setEnabled(bool on) { enabled_.store(on); }
    bool isEnabled() const { return enabled_.load(); }

    bool canAcceptCompilation() const;
    void notifyCompilationStarted();
    void notifyCompilationCompleted();
    void recordQueueRejection();
    void processQueue();
    void clear();

    struct Stats {
        size_t total_registered = 0;
        size_t o2_ready = 0;
        size_t ofast_ready = 0;
        size_t pending = 0;
        uint64_t active_compilations = 0;
        uint64_t queue_rejections = 0;
        size_t queued = 0;
    };
    Stats getStats() const;
    void promoteAll();
    // Waits for every background chain (30 s each at most).
    void shutdown();

    // Tier-1 executor of one spec: by default the pattern op by op through
    // the single-op C ABI kernels.  Tests replace it.
    using Interpreter = std::function<std::vector<Tensor>(const KernelSpec&, const std::vector<Tensor>&)>;
    void setInterpreterForTest(Interpreter f);
    std::vector<Tensor> interpret(const KernelSpec& spec, const std::vector<Tensor>& inputs);

    std::mutex& queue_mutex() { return queue_mu_; }
    std::priority_queue<CompilationTask>& task_queue() { return queue_; }
    void addFuture(std::future<void> f);

private:
    PGOManager() = default;
    ~PGOManager() { shutdown(); }

    mutable std::mutex mu_;
    std::vector<std::shared_ptr<PGOCompiledKernel>> entries_;
    std::unordered_map<std::string, std::shared_ptr<PGOCompiledKernel>> cache_;
    PGOConfig config_;
    std::atomic<bool> enabled_{false};
    mutable std::mutex queue_mu_;
    std::priority_queue<CompilationTask> queue_;
    std::atomic<uint64_t> active_{0};
    std::atomic<uint64_t> rejections_{0};
    std::mutex futures_mu_;
    std::vector<std::future<void>> futures_;
    std::mutex interp_mu_;
    Interpreter interp_;
};

}  // namespace c3
}  // namespace ct
