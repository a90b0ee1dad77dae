// JITCache.h -- on-disk cache of compiled kernels.
//
// Same layout and protocol as the reference's bitcode cache
// (src/C3/JITCache.cpp:214-311): files c3_jit_<key>.<ext> + c3_jit_<key>.meta
// in $C3_AOT_CACHE_DIR, else ~/.c3cache, else /tmp/.c3cache; the first line
// of .meta is the cache version and a mismatch evicts the entry; writes go to
// *.tmp and are renamed into place; C3_JIT_CACHE_DISABLE=1 turns it off.
// key = sha256_hex("c3_jit_" + version + "_" + opt + "_" + spec) (:214-220).
// What is stored here is a gfx950 code object (.hsaco) instead of LLVM
// bitcode, and the spec text starts with the RollingHash of the kernel's op
// sequence, so entries are keyed by that hash plus shapes and dtype.
#pragma once

#include <atomic>
#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

namespace ct {
namespace c3 {

std::string sha256_hex(const std::string& data);

class JITCache {
public:
    static JITCache& getInstance();

    static std::string makeKey(const std::string& spec_str, int opt_level);
    static const char* currentJITVersion() { return "hip_gfx950_v1"; }
    static bool isEnabled();

    // Path of the cached code object for `key`, or "" on a miss.
    std::string lookup(const std::string& key);
    // Atomically store `image` under `key` with `meta_lines` after the version line.
    std::string store(const std::string& key, const std::vector<char>& image,
                      const std::vector<std::string>& meta_lines = {});
    static bool readFile(const std::string& path, std::vector<char>* out);
    std::string cacheDir() const;
    void evict();

    uint64_t hits() const { return hits_.load(); }
    uint64_t misses() const { return misses_.load(); }
    uint64_t stores() const { return stores_.load(); }

private:
    JITCache() = default;
    static std::string resolveCacheDir();
    mutable std::mutex mutex_;
    std::atomic<uint64_t> hits_{0}, misses_{0}, stores_{0};
};

}  // namespace c3
}  // namespace ct
