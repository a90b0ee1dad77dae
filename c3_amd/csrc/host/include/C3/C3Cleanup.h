// C3Cleanup.h -- ordered teardown (include/C3/C3Cleanup.h:34-40 of the
// reference): hot-path manager, backward capture, engine, engine cache,
// region registry, kernel registry, then this backend's device state
// (cached device buffers and the loaded code objects).  Call before main()
// returns; no kernel may be in flight on another thread.
#pragma once

namespace ct {
namespace c3 {

void shutdownAll();

}  // namespace c3
}  // namespace ct
