// linear.hip -- perturbed forward (placeholder until the MFMA kernel lands).
#include "runtime.h"
using namespace hses;
extern "C" int hses_perturbed_linear(const void*, int32_t, int64_t, int64_t, int32_t, const float*,
                                     int32_t, int32_t, uint64_t, int32_t, float, int32_t, int32_t,
                                     int32_t, int32_t, int32_t, float*, int64_t, int64_t, int32_t,
                                     void*) {
    return set_error(HSES_ERR_UNSUPPORTED, "hses_perturbed_linear: not built yet");
}
