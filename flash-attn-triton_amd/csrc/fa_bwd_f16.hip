// Instantiations of the attention backward kernels for f16 inputs.
#include "fa_bwd_launch.h"

hipError_t fa_launch_bwd_f16(const fa::BwdParams& p, int head_dim, bool generic, hipStream_t st) {
  return fa::launch_bwd<fa::F16>(p, head_dim, generic, st);
}
