// Symmetric-contraction launchers, input lmax 0..2.
#include "sc_launch.h"
namespace ictc {
namespace sc {
#define ICTC_SC_LOW(A, B, C) ICTC_SC_IF_LOW_##A(A, B, C)
#define ICTC_SC_IF_LOW_0(A, B, C) ICTC_SC_DEFINE(A, B, C)
#define ICTC_SC_IF_LOW_1(A, B, C) ICTC_SC_DEFINE(A, B, C)
#define ICTC_SC_IF_LOW_2(A, B, C) ICTC_SC_DEFINE(A, B, C)
#define ICTC_SC_IF_LOW_3(A, B, C)
ICTC_FOR_EACH_SC(ICTC_SC_LOW)
}  // namespace sc
}  // namespace ictc
