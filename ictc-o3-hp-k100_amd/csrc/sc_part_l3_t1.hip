// Symmetric-contraction launchers, input lmax 3, target lmax 1.
#include "sc_launch.h"
namespace ictc {
namespace sc {
ICTC_SC_DEFINE(3, 1, 1)
ICTC_SC_DEFINE(3, 1, 2)
ICTC_SC_DEFINE(3, 1, 3)
}  // namespace sc
}  // namespace ictc
