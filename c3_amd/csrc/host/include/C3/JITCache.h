// JITCache.h -- on-disk cache of compiled kernels.
//
// Same directory, naming, versioning and write protocol as the reference's
// bitcode cache (src/C3/JITCache.cpp:214-311): entries c3_jit_<key>.meta in
// $C3_AOT_CACHE_DIR, else ~/.c3cache, else /tmp/.c3cache; the first line of
// .meta is the cache version and a mismatch evicts the entry; writes go to
// *.tmp<pid> and are renamed into place; C3_JIT_CACHE_DISABLE=1 turns it off;
// key = sha256_hex("c3_jit_" + version + "_" + opt + "_" + spec) (:214-220),
// the spec text starting with the RollingHash of the kernel's op sequence.
//
// What is cached here is a gfx950 code object instead of LLVM bitcode, and
// it is content-addressed: the object is stored once, as
// c3_jit_obj_<sha256 of its bytes>.hsaco, however many spec keys use it, and
// each key's .meta names it on an "image=<sha256>" line.  A lookup verifies
// the object against that hash (a damaged file is rejected) and against the
// hash of the image the library itself would load (an entry written by an
// older build is rejected), and evicts rejected entries.
#pragma once

#include <atomic>
#include <cstdint>
#include <map>
#include <mutex>
#include <string>
#include <vector>

namespace ct {
namespace c3 {

std::string sha256_hex(const std::string& data);
std::string sha256_hex(const char* data, size_t n);

class JITCache {
public:
    static JITCache& getInstance();

    static std::string makeKey(const std::string& spec_str, int opt_level);
    static const char* currentJITVersion() { return "hip_gfx950_abi1_v2"; }
    static bool isEnabled();

    // Path of the code object entry `key` names, or "" on a miss.  A hit
    // needs the current version line, the named object file, its content
    // hash equal to the recorded one and, when expected_sha is not empty,
    // the recorded hash equal to expected_sha; an entry failing any of these
    // is evicted and counted as rejected.
    std::string lookup(const std::string& key, const std::string& expected_sha = "");
    // Store `image` (once per content hash) and the entry `key` naming it,
    // with `meta_lines` after the version and image lines.  Returns the
    // object's path, or "" on failure.
    std::string store(const std::string& key, const std::vector<char>& image,
                      const std::vector<std::string>& meta_lines = {});
    // SHA-256 (hex) of the file at `path` (the prebuilt code objects, which
    // do not change under a running process), memoised by path, size and
    // modification time; "" when it cannot be read.
    std::string fileSha(const std::string& path);
    static bool readFile(const std::string& path, std::vector<char>* out);
    std::string cacheDir() const;
    // Remove every entry and object.
    void evict();

    uint64_t hits() const { return hits_.load(); }
    uint64_t misses() const { return misses_.load(); }
    uint64_t stores() const { return stores_.load(); }
    uint64_t rejected() const { return rejected_.load(); }

private:
    JITCache() = default;
    static std::string resolveCacheDir();
    std::string fileShaLocked(const std::string& path);
    mutable std::mutex mutex_;
    struct FileStamp {
        int64_t size = -1, mtime_ns = -1;
        std::string sha;
    };
    std::map<std::string, FileStamp> sha_memo_;
    std::atomic<uint64_t> hits_{0}, misses_{0}, stores_{0}, rejected_{0};
};

}  // namespace c3
}  // namespace ct
