// Kernel instantiations: hard binning, float logits, right=false.
#include "ace_core.hpp"

namespace ace {
ACE_DEFINE_LAUNCHERS(float, false, false)
}  // namespace ace
