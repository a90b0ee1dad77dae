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

    static FusionCost estimate(const std::vector<op>& op_seq, const std::vector<size_t>& out_numels) {
        FusionCost cost;
        const size_t n = op_seq.size() < out_numels.size() ? op_seq.size() : out_numels.size();
        if (n == 0) return cost;
        size_t write_all = 0, read_intermediate = 0;
        for (size_t i = 0; i < n; ++i) {
            write_all += out_numels[i];
            if (i + 1 < n) read_intermediate += out_numels[i];
        }
        cost.eager_accesses = write_all + read_intermediate;
        for (size_t i = 0; i + 1 < n; ++i)
            if (!isComputeIntensive(op_seq[i])) cost.saved_accesses += out_numels[i] * 2;
        cost.fused_accesses =
            cost.eager_accesses > cost.saved_accesses ? cost.eager_accesses - cost.saved_accesses : 0;
        if (cost.eager_accesses > 0)
            cost.gain_ratio = static_cast<double>(cost.saved_accesses) / static_cast<double>(cost.eager_accesses);
        cost.worthwhile = cost.saved_accesses > 0 && cost.gain_ratio >= kMinGainRatio;
        return cost;
    }
};

}  // namespace c3
}  // namespace ct
