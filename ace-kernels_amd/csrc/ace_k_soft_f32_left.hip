// Kernel instantiations: soft binning, float logits, right=false.
#include "ace_core.hpp"

namespace ace {
ACE_DEFINE_LAUNCHERS(float, true, false)
}  // namespace ace
