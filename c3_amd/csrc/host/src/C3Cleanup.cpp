// C3Cleanup.cpp -- see include/C3/C3Cleanup.h.
#include "C3/C3Cleanup.h"

#include "C3/C3BackwardCapture.h"
#include "C3/C3Engine.h"
#include "C3/C3HotPathManager.h"
#include "C3/C3KernelRegistry.h"
#include "C3/RegionFusion.h"
#include "c3hip.h"

namespace ct {
namespace c3 {

void shutdownAll() {
    C3HotPathManager::instance().shutdown();
    C3BackwardCapture::getInstance().waitForPendingCompiles();
    C3Engine::getInstance().shutdown();
    C3Engine::getInstance().clearCache();
    RegionFusionRegistry::getInstance().clear();
    C3KernelRegistry::getInstance().uninstallAll();
    releaseCachedDeviceMemory();
    (void)c3hip_shutdown();
    C3HotPathManager::instance().resetAfterShutdown();
}

}  // namespace c3
}  // namespace ct
