// MFMA backward (bf16 / fp16): placeholder until the kernels land.
#include "sk_common.h"
#include "sk_kernels.h"

namespace sk {
hipError_t launch_bwd_mfma(int dtype, const BwdParams& p, bool causal, hipStream_t s) {
  (void)dtype; (void)p; (void)causal; (void)s;
  return hipErrorNotSupported;
}
}  // namespace sk
