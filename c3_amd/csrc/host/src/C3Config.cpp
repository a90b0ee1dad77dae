// C3Config.cpp -- see include/C3/C3Config.h.
#include "C3/C3Config.h"

#include <atomic>
#include <cstdlib>
#include <cstring>

namespace ct {
namespace c3 {
namespace {

bool envOne(const char* name) {
    const char* v = std::getenv(name);
    return v && std::strcmp(v, "1") == 0;
}

struct Flags {
    std::atomic<bool> loaded{false};
    std::atomic<bool> single{true}, region{true}, backward{true}, hotpath{true};
};
Flags g_flags;

void load() {
    g_flags.single = !envOne("C3_DISABLE_SINGLE_KERNEL");
    g_flags.region = !envOne("C3_DISABLE_REGION_FUSION");
    g_flags.backward = !envOne("C3_DISABLE_BACKWARD") && !envOne("CTORCH_DISABLE_C3_BACKWARD");
    g_flags.hotpath = !envOne("C3_DISABLE_HOTPATH");
    g_flags.loaded = true;
}

inline void ensure() {
    if (!g_flags.loaded.load(std::memory_order_acquire)) load();
}

}  // namespace

bool singleKernelEnabled() { ensure(); return g_flags.single; }
bool regionFusionEnabled() { ensure(); return g_flags.region; }
bool backwardFusionEnabled() { ensure(); return g_flags.backward; }
bool hotPathTrackingEnabled() { ensure(); return g_flags.hotpath; }
void reloadConfig() { load(); }

}  // namespace c3
}  // namespace ct
