// Kernel instantiations: soft binning, float logits, right=true.
#include "ace_core.hpp"

namespace ace {
ACE_DEFINE_LAUNCHERS(float, true, true)
}  // namespace ace
