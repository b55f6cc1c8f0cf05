// Kernel instantiations: soft binning, __half logits.
#include "ace_core.hpp"

namespace ace {
ACE_DEFINE_LAUNCHERS(__half, true)
}  // namespace ace
