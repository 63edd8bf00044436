// Symmetric-contraction launchers, input lmax 3, target lmax 0.
#include "sc_launch.h"
namespace ictc {
namespace sc {
ICTC_SC_DEFINE(3, 0, 1)
ICTC_SC_DEFINE(3, 0, 2)
ICTC_SC_DEFINE(3, 0, 3)
}  // namespace sc
}  // namespace ictc
