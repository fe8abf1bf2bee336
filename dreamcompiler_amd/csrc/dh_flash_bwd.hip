#include "dh_common.hpp"
using namespace dh;
extern "C" int dh_flash_bwd(int, int, int, int, float, int, const void*, const void*, const void*, const void*, const void*, const float*, float*, float*, float*, int) {
    DH_TRY(ensure_init());
    return set_error(DH_ERR_UNSUPPORTED, "dh_flash_bwd: not built yet");
}
