// Register-resident fast path for bf16 rows (placeholder: not enabled yet).
#pragma once

#include "dsr_general.h"

namespace dsr {

struct FastShared {
  GenShared gen;
};

static inline bool fast_path_eligible(const dsr_sample_args_t&) { return false; }

__device__ inline bool fast_sample_row(const dsr_sample_args_t&, int64_t, FastShared&) { return false; }

}  // namespace dsr
