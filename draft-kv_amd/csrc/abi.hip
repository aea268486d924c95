// Error state and version of the C ABI (include/draftkv_hip.h).
#include "dkv_common.h"

namespace dkv {

static thread_local std::string g_error;

void set_error(const std::string& msg) { g_error = msg; }

int fail(int code, const std::string& msg) {
    g_error = msg;
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(DKV_ELAUNCH, std::string(what) + ": " + hipGetErrorString(e));
    return DKV_OK;
}

}  // namespace dkv

extern "C" const char* dkv_last_error(void) { return dkv::g_error.c_str(); }

extern "C" int32_t dkv_version(void) { return 1; }
