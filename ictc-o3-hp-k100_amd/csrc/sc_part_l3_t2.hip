// Symmetric-contraction launchers, input lmax 3, target lmax 2.
#include "sc_launch.h"
namespace ictc {
namespace sc {
ICTC_SC_DEFINE(3, 2, 1)
ICTC_SC_DEFINE(3, 2, 2)
ICTC_SC_DEFINE(3, 2, 3)
}  // namespace sc
}  // namespace ictc
