// Kernel instantiations: hard binning, float logits.
#include "ace_core.hpp"

namespace ace {
ACE_DEFINE_LAUNCHERS(float, false)
}  // namespace ace
