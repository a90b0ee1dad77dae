// FusionCostModel.h -- read/write-count estimate of what fusing an op
// sequence saves (include/C3/FusionCostModel.h:60-106 of the reference).
//
// eager  = sum of every node's output writes + one read of every non-last node;
// saved  = 2 * numel for every non-last node that is not compute-intensive
//          (a MatMul's output is written and read either way);
// worthwhile when saved > 0 and saved / eager >= 0.20.
// MatMul+Add+ReLU over [M,N]: eager 5MN, saved 2MN -> 0.4 (active);
// MatMul+ReLU: saved 0 (never active).
#pragma once

#include <algorithm>
#include <cstddef>
#include <vector>

#include "C3/Ctools.h"

namespace ct {
namespace c3 {

struct FusionCost {
    size_t eager_accesses = 0;
    size_t fused_accesses = 0;
    size_t saved_accesses = 0;
    double gain_ratio = 0.0;
    bool worthwhile = false;
};

class FusionCostModel {
public:
    static constexpr double kMinGainRatio = 0.20;

    static bool isComputeIntensive(op op_type) { return op_type == op::MatMul; }

    // Element accesses of the sequence run op by op (every output written,
    // every output but the last read back by its consumer) and what one
    // fused kernel saves (the write and the read of each intermediate that
    // is not compute-intensive).  Only the first min(|op_seq|, |out_numels|)
    // ops count.  With I = the intermediates and L = the last output:
    //   eager = L + 2 * sum(I),  saved = 2 * sum(I that are not MatMul).
    static FusionCost estimate(const std::vector<op>& op_seq, const std::vector<size_t>& out_numels) {
        FusionCost c;
        const size_t count = std::min(op_seq.size(), out_numels.size());
        if (count == 0) return c;
        size_t intermediates = 0, removable = 0;
        for (size_t k = 0; k + 1 < count; ++k) {
            intermediates += out_numels[k];
            if (!isComputeIntensive(op_seq[k])) removable += out_numels[k];
        }
        c.eager_accesses = out_numels[count - 1] + 2 * intermediates;
        c.saved_accesses = 2 * removable;
        c.fused_accesses = c.eager_accesses - c.saved_accesses;  // saved <= eager by construction
        c.gain_ratio = c.eager_accesses ? (double)c.saved_accesses / (double)c.eager_accesses : 0.0;
        c.worthwhile = c.saved_accesses > 0 && c.gain_ratio >= kMinGainRatio;
        return c;
    }
};

}  // namespace c3
}  // namespace ct
