#include "dh_common.hpp"
using namespace dh;
extern "C" int dh_flash_fwd(int, int, int, int, float, int, const void*, const void*, const void*, void*, float*) {
    DH_TRY(ensure_init());
    return set_error(DH_ERR_UNSUPPORTED, "dh_flash_fwd: not built yet");
}
