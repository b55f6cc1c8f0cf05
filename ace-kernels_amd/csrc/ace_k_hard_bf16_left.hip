// Kernel instantiations: hard binning, __hip_bfloat16 logits, right=false.
#include "ace_core.hpp"

namespace ace {
ACE_DEFINE_LAUNCHERS(__hip_bfloat16, false, false)
}  // namespace ace
