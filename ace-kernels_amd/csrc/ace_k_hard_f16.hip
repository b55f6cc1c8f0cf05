// Kernel instantiations: hard binning, __half logits.
#include "ace_core.hpp"

namespace ace {
ACE_DEFINE_LAUNCHERS(__half, false)
}  // namespace ace
