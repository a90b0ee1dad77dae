// JITCache.cpp -- see include/C3/JITCache.h.
#include "C3/JITCache.h"

#include <dirent.h>
#include <errno.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>

namespace ct {
namespace c3 {
namespace {

// SHA-256, FIPS 180-4 section 6.2.  Round constants: first 32 bits of the
// fractional parts of the cube roots of the first 64 primes (section 4.2.2);
// initial hash: square roots of the first 8 primes (section 5.3.3).
const uint32_t kK[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

void compress(uint32_t h[8], const unsigned char* blk) {
    uint32_t w[64];
    for (int t = 0; t < 16; ++t)
        w[t] = (uint32_t)blk[4 * t] << 24 | (uint32_t)blk[4 * t + 1] << 16 | (uint32_t)blk[4 * t + 2] << 8 | blk[4 * t + 3];
    for (int t = 16; t < 64; ++t) {
        const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
        const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
        w[t] = w[t - 16] + s0 + w[t - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], k = h[7];
    for (int t = 0; t < 64; ++t) {
        const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
        const uint32_t ch = (e & f) ^ (~e & g);
        const uint32_t t1 = k + S1 + ch + kK[t] + w[t];
        const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
        const uint32_t maj = (a & b) ^ (a & c) ^ (b & c);
        const uint32_t t2 = S0 + maj;
        k = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += k;
}

bool ensureDir(const std::string& dir) {
    struct stat st;
    if (stat(dir.c_str(), &st) == 0) return S_ISDIR(st.st_mode);
    return mkdir(dir.c_str(), 0755) == 0 || errno == EEXIST;
}

}  // namespace

std::string sha256_hex(const char* data, size_t n) {
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    size_t i = 0;
    for (; i + 64 <= n; i += 64) compress(h, reinterpret_cast<const unsigned char*>(data) + i);
    unsigned char tail[128] = {0};
    const size_t rem = n - i;
    if (rem) std::memcpy(tail, data + i, rem);
    tail[rem] = 0x80;
    const size_t tail_len = rem + 1 + 8 <= 64 ? 64 : 128;
    const uint64_t bits = (uint64_t)n * 8;
    for (int b = 0; b < 8; ++b) tail[tail_len - 1 - b] = (unsigned char)(bits >> (8 * b));
    compress(h, tail);
    if (tail_len == 128) compress(h, tail + 64);
    char out[65];
    for (int b = 0; b < 8; ++b) std::snprintf(out + 8 * b, 9, "%08x", h[b]);
    return std::string(out, 64);
}

std::string sha256_hex(const std::string& data) { return sha256_hex(data.data(), data.size()); }

JITCache& JITCache::getInstance() {
    static JITCache c;
    return c;
}

bool JITCache::isEnabled() {
    const char* v = std::getenv("C3_JIT_CACHE_DISABLE");
    return !(v && v[0] == '1');
}

std::string JITCache::makeKey(const std::string& spec_str, int opt_level) {
    std::ostringstream ss;
    ss << "c3_jit_" << currentJITVersion() << "_" << opt_level << "_" << spec_str;
    return sha256_hex(ss.str());
}

std::string JITCache::resolveCacheDir() {
    if (const char* d = std::getenv("C3_AOT_CACHE_DIR"); d && *d) return d;
    if (const char* home = std::getenv("HOME"); home && *home) {
        const std::string p = std::string(home) + "/.c3cache";
        if (ensureDir(p) && access(p.c_str(), W_OK) == 0) return p;
    }
    return "/tmp/.c3cache";
}

std::string JITCache::cacheDir() const { return resolveCacheDir(); }

namespace {

std::string objectPath(const std::string& dir, const std::string& sha) { return dir + "/c3_jit_obj_" + sha + ".hsaco"; }
std::string metaPath(const std::string& dir, const std::string& key) { return dir + "/c3_jit_" + key + ".meta"; }

// Write `n` bytes to `path` through a temporary file renamed into place.
bool writeAtomically(const std::string& path, const char* data, size_t n) {
    const std::string tmp = path + ".tmp" + std::to_string(getpid());
    {
        std::ofstream o(tmp, std::ios::binary);
        if (!o.is_open()) return false;
        o.write(data, (std::streamsize)n);
        if (!o.good()) {
            o.close();
            unlink(tmp.c_str());
            return false;
        }
    }
    if (rename(tmp.c_str(), path.c_str()) != 0) {
        unlink(tmp.c_str());
        return false;
    }
    return true;
}

}  // namespace

// SHA-256 (hex) of the file's current bytes, "" when it cannot be read.
static std::string hashFile(const std::string& path) {
    std::vector<char> bytes;
    if (!JITCache::readFile(path, &bytes)) return "";
    return sha256_hex(bytes.data(), bytes.size());
}

std::string JITCache::fileShaLocked(const std::string& path) {
    struct stat st;
    if (stat(path.c_str(), &st) != 0) return "";
    const int64_t mt = (int64_t)st.st_mtim.tv_sec * 1000000000LL + st.st_mtim.tv_nsec;
    auto it = sha_memo_.find(path);
    if (it != sha_memo_.end() && it->second.size == (int64_t)st.st_size && it->second.mtime_ns == mt)
        return it->second.sha;
    std::vector<char> bytes;
    if (!readFile(path, &bytes)) return "";
    FileStamp fs;
    fs.size = (int64_t)st.st_size;
    fs.mtime_ns = mt;
    fs.sha = sha256_hex(bytes.data(), bytes.size());
    sha_memo_[path] = fs;
    return fs.sha;
}

std::string JITCache::fileSha(const std::string& path) {
    std::lock_guard<std::mutex> lk(mutex_);
    return fileShaLocked(path);
}

std::string JITCache::lookup(const std::string& key, const std::string& expected_sha) {
    std::lock_guard<std::mutex> lk(mutex_);
    const std::string dir = resolveCacheDir();
    const std::string meta = metaPath(dir, key);
    std::ifstream m(meta);
    if (!m.is_open()) {
        misses_++;
        return "";
    }
    std::string version, line, sha;
    const bool versioned = std::getline(m, version) && version == currentJITVersion();
    while (versioned && std::getline(m, line))
        if (line.rfind("image=", 0) == 0) sha = line.substr(6);
    m.close();
    const std::string obj = sha.empty() ? "" : objectPath(dir, sha);
    // The object is hashed in full on every lookup: a rewrite within the
    // file system's timestamp granularity would fool a size/mtime memo.
    const std::string obj_sha = obj.empty() || access(obj.c_str(), R_OK) != 0 ? "" : hashFile(obj);
    const bool ok = versioned && !sha.empty() && obj_sha == sha && (expected_sha.empty() || sha == expected_sha);
    if (!ok) {
        // Stale version, missing or damaged object, or built from other code:
        // drop the entry; a damaged object goes too (its name is its hash).
        unlink(meta.c_str());
        if (!obj_sha.empty() && obj_sha != sha) unlink(obj.c_str());
        if (versioned) rejected_++;
        misses_++;
        return "";
    }
    hits_++;
    return obj;
}

std::string JITCache::store(const std::string& key, const std::vector<char>& image,
                            const std::vector<std::string>& meta_lines) {
    std::lock_guard<std::mutex> lk(mutex_);
    const std::string dir = resolveCacheDir();
    if (!ensureDir(dir)) return "";
    const std::string sha = sha256_hex(image.data(), image.size());
    const std::string obj = objectPath(dir, sha);
    if (hashFile(obj) != sha && !writeAtomically(obj, image.data(), image.size())) return "";
    std::ostringstream mt;
    mt << currentJITVersion() << "\n" << "image=" << sha << "\n";
    for (const auto& l : meta_lines) mt << l << "\n";
    const std::string text = mt.str();
    if (!writeAtomically(metaPath(dir, key), text.data(), text.size())) return "";
    stores_++;
    return obj;
}

bool JITCache::readFile(const std::string& path, std::vector<char>* out) {
    std::ifstream f(path, std::ios::binary);
    if (!f.is_open()) return false;
    f.seekg(0, std::ios::end);
    const std::streamoff n = f.tellg();
    if (n < 0) return false;
    f.seekg(0);
    out->resize((size_t)n);
    f.read(out->data(), n);
    return f.good() || f.eof();
}

void JITCache::evict() {
    std::lock_guard<std::mutex> lk(mutex_);
    const std::string dir = resolveCacheDir();
    DIR* d = opendir(dir.c_str());
    if (!d) return;
    while (dirent* e = readdir(d)) {
        if (std::strncmp(e->d_name, "c3_jit_", 7) == 0) unlink((dir + "/" + e->d_name).c_str());
    }
    closedir(d);
    sha_memo_.clear();
}

}  // namespace c3
}  // namespace ct
