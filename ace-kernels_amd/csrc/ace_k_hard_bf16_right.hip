// Kernel instantiations: hard binning, __hip_bfloat16 logits, right=true.
#include "ace_core.hpp"

namespace ace {
ACE_DEFINE_LAUNCHERS(__hip_bfloat16, false, true)
}  // namespace ace
