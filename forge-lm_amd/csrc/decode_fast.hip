// decode_fast.hip -- fused batch-1 fp32 decode step.
#include "decode_fast.hpp"

namespace fh {

int FastDecode::init(hipStream_t, const fh_model_desc&, int) {
  enabled = false;
  return FH_OK;
}

int FastDecode::on_weights_loaded() { return FH_OK; }

int FastDecode::enqueue(hipStream_t, const RowSrc&) { return FH_ERR_STATE; }

void FastDecode::release() {}

}  // namespace fh
