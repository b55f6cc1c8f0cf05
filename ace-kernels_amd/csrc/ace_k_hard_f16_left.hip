// Kernel instantiations: hard binning, __half logits, right=false.
#include "ace_core.hpp"

namespace ace {
ACE_DEFINE_LAUNCHERS(__half, false, false)
}  // namespace ace
