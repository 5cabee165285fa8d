// linear_pair.hip -- perturbed forward for large ranks (placeholder).
#include "linear_common.h"
#include "runtime.h"
namespace hses {
int launch_linear_pair(LinParams&, DeviceState*, hipStream_t) { return HSES_ERR_UNSUPPORTED; }
}  // namespace hses
