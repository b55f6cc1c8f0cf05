// Kernel instantiations: soft binning, __hip_bfloat16 logits, right=false.
#include "ace_core.hpp"

namespace ace {
ACE_DEFINE_LAUNCHERS(__hip_bfloat16, true, false)
}  // namespace ace
