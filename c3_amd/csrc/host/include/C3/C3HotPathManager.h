// C3HotPathManager.h -- hot-call detection and asynchronous kernel install.
//
// Same flow as the reference (include/C3/C3HotPathManager.h:60-1046):
//   * recordCall counts calls per (op, shape, device) key; at hot_threshold
//     (5) it submits a compile, honouring the per-key cooldown (60 s after a
//     compile) and backpressure (at most max_pending compiles in flight);
//   * every call is also appended to a 32-deep ring of recent dispatches; in
//     autograd scope the ring is checked at once for a fusable pattern
//     (MatMul+Add+ReLU, MatMul+Add+Sigmoid, MatMul+ReLU, MatMul+Sigmoid);
//   * single-op compiles run two tiers in parallel (O2 and O4), each
//     installed when ready; the registry keeps the higher opt level;
//   * a fused compile installs the region kernel into the registry
//     (installFused) and the region registry (installWithCost);
//   * shutdown waits for in-flight compiles (30 s per future).
// "Compile" resolves a gfx950 kernel through C3Engine (JITCache + prebuilt
// code objects).  Kernels are installed for the device the calls were
// recorded on (the reference hard-codes kCPU, :1007).  Patterns whose
// epilogue has no gfx950 kernel yet (Sigmoid) are detected and counted but
// not compiled.
#pragma once

#include <atomic>
#include <chrono>
#include <deque>
#include <future>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "C3/C3Engine.h"
#include "C3/Ctools.h"

namespace ct {
namespace c3 {

struct HotPathConfig {
    size_t hot_threshold = 5;
    size_t cooldown_sec = 60;
    size_t max_pending = 16;
    uint32_t compile_timeout_ms = 30000;
    bool verbose = false;
};

class C3HotPathManager {
public:
    static C3HotPathManager& instance();

    void configure(const HotPathConfig& cfg);
    HotPathConfig getConfig() const;

    struct Stats {
        size_t calls_tracked = 0;
        size_t compilations_triggered = 0;
        size_t pending_compiles = 0;
        size_t cooldown_hits = 0;
        size_t backpressure_hits = 0;
        size_t patterns_detected = 0;
        size_t patterns_unsupported = 0;
    };
    Stats getStats() const;

    struct DispatchRecord {
        op op_type;
        std::vector<size_t> shape;      // lhs ++ rhs (pattern detection)
        std::vector<size_t> lhs_shape;
        std::vector<size_t> rhs_shape;
        DType dtype = DType::kFloat;
        std::chrono::steady_clock::time_point timestamp;
    };

    // dt: element type of the call's tensors (the reference is fp32-only).
    void recordCall(op op_type, DeviceType dev, const std::vector<size_t>& lhs_shape,
                    const std::vector<size_t>& rhs_shape = {}, bool in_autograd = false, DType dt = DType::kFloat);

    void clear();
    void shutdown();
    bool isShuttingDown() const { return shutting_down_.load(std::memory_order_acquire); }
    void resetAfterShutdown() { shutting_down_.store(false, std::memory_order_release); }
    void waitForPendingCompiles();

    // The kernel spec a fused pattern compiles to (test hook, like the
    // reference's buildFusedGraphForTest, :658-662).  Returns false for a
    // pattern without a gfx950 kernel.
    static bool buildFusedSpec(const std::vector<DispatchRecord>& records, const std::string& pattern, KernelSpec* out);
    static bool buildSingleOpSpec(op op_type, const std::vector<size_t>& lhs, const std::vector<size_t>& rhs, DType dt,
                                  KernelSpec* out);
    static size_t hashShapeKey(const std::vector<size_t>& shape, op op_type, DeviceType dev);
    static bool isSupportedOp(op op_type);

private:
    C3HotPathManager() = default;

    struct HotEntry {
        size_t call_count = 0;
        bool compiling = false;
        std::chrono::steady_clock::time_point last_compile_time{};
    };

    void tryFuseRecentDispatches(DeviceType dev, const HotPathConfig& cfg);
    void submitFusedCompileAsync(const std::vector<DispatchRecord>& records, DeviceType dev, const HotPathConfig& cfg,
                                 const std::string& pattern_name);
    void submitCompileAsync(const DispatchRecord& rec, DeviceType dev, size_t key, const HotPathConfig& cfg);
    void finishCompile(size_t key);

    static constexpr size_t kMaxRingBufferSize = 32;

    mutable std::mutex mutex_, cfg_mutex_, rb_mutex_, futures_mutex_;
    HotPathConfig config_;
    std::unordered_map<size_t, HotEntry> entries_;
    std::deque<DispatchRecord> recent_dispatches_;
    std::vector<std::future<void>> pending_futures_;
    std::atomic<size_t> calls_tracked_{0}, compilations_triggered_{0}, pending_compiles_{0};
    std::atomic<size_t> patterns_detected_{0}, patterns_unsupported_{0};
    std::atomic<bool> shutting_down_{false};
    size_t cooldown_hits_ = 0, backpressure_hits_ = 0;
};

}  // namespace c3
}  // namespace ct
