// decode_fast.hpp -- fused batch-1 fp32 decode step (see decode_fast.hip).
#pragma once

#include "../../include/forge_hip.h"
#include "common.hpp"

namespace fh {

// Holds the device state of the fused decode path for one session.  When the
// session's shape is outside what the fused kernels were built for, `enabled`
// stays false and the generic kernels run instead.
struct FastDecode {
  bool enabled = false;
  int init(hipStream_t st, const fh_model_desc& d, int compute_units);
  int on_weights_loaded();
  int enqueue(hipStream_t st, const RowSrc& src);
  void release();
};

}  // namespace fh
