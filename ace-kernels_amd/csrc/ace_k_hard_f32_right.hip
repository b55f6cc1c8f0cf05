// Kernel instantiations: hard binning, float logits, right=true.
#include "ace_core.hpp"

namespace ace {
ACE_DEFINE_LAUNCHERS(float, false, true)
}  // namespace ace
