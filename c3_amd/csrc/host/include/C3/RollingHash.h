// RollingHash.h -- polynomial hash of op sequences with O(1) sub-range hashes.
//
// prefix[i+1] = prefix[i] * 131 + code(op_i) (mod 2^64), code = a distinct
// prime per op; sub(l, r) = prefix[r+1] - prefix[l] * 131^(r-l+1).
// Same base, codes and formulas as the reference (src/C3/RollingHash.cpp:14-72),
// so region keys and cache keys computed by either side agree.
#pragma once

#include <cstddef>
#include <cstdint>
#include <mutex>
#include <vector>

#include "C3/Ctools.h"

namespace ct {
namespace c3 {

class RollingHash {
public:
    static constexpr uint64_t kBase = 131;
    static void precompute(size_t max_len);
    static std::vector<uint64_t> computePrefixHashes(const std::vector<op>& ops);
    static uint64_t getSubHash(const std::vector<uint64_t>& prefix, size_t l, size_t r);
    static uint64_t getOpCode(op op_type);
    static size_t maxLen();
    // Hash of a whole sequence (sub-hash over [0, n-1]).
    static uint64_t hashSequence(const std::vector<op>& ops);
};

}  // namespace c3
}  // namespace ct
