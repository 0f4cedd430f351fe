// Instantiations of the attention forward kernel for bf16 inputs.
#include "fa_fwd_launch.h"

hipError_t fa_launch_fwd_bf16(const fa::FwdParams& p, int mode, int head_dim, bool generic,
                             hipStream_t st) {
  if (mode == fa::kModePrefill)
    return fa::launch_fwd_mode<fa::BF16, fa::kModePrefill>(p, head_dim, generic, st);
  return fa::launch_fwd_mode<fa::BF16, fa::kModeKvcache>(p, head_dim, generic, st);
}
