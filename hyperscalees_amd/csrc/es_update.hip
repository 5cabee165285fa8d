// es_update.hip -- ES update (placeholder until the MFMA kernel lands).
#include "runtime.h"
using namespace hses;
extern "C" size_t hses_es_update_workspace(int32_t, int32_t, int32_t, int32_t) { return 0; }
extern "C" int hses_es_update(const float*, int32_t, int32_t, uint64_t, int32_t, float, int32_t,
                              int32_t, int32_t, int32_t, float, float*, void*, size_t, void*) {
    return set_error(HSES_ERR_UNSUPPORTED, "hses_es_update: not built yet");
}
