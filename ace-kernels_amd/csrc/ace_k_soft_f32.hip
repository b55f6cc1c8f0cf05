// Kernel instantiations: soft binning, float logits.
#include "ace_core.hpp"

namespace ace {
ACE_DEFINE_LAUNCHERS(float, true)
}  // namespace ace
