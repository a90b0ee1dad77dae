// C3Config.h -- runtime kill switches (include/C3/C3Config.h:34-87 of the
// reference): an environment variable set to "1" disables the feature.
//   C3_DISABLE_SINGLE_KERNEL   single-op registry dispatch
//   C3_DISABLE_REGION_FUSION   fused-region dispatch
//   C3_DISABLE_BACKWARD        backward capture (also CTORCH_DISABLE_C3_BACKWARD)
//   C3_DISABLE_HOTPATH         hot-path call tracking / compilation
// Values are read once and cached; reloadConfig() re-reads them (tests).
#pragma once

namespace ct {
namespace c3 {

bool singleKernelEnabled();
bool regionFusionEnabled();
bool backwardFusionEnabled();
bool hotPathTrackingEnabled();
void reloadConfig();

}  // namespace c3
}  // namespace ct
