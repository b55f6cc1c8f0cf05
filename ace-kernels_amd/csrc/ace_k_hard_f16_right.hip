// Kernel instantiations: hard binning, __half logits, right=true.
#include "ace_core.hpp"

namespace ace {
ACE_DEFINE_LAUNCHERS(__half, false, true)
}  // namespace ace
