// Status reporting shared by every C-ABI entry point of libmvme_paged.so.
#include "mvme_common.h"

namespace mvme {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& message) { g_last_error = message; }

int fail(int code, const std::string& message) {
    g_last_error = message;
    return code;
}

// Launch errors are sticky per thread in HIP; reading them with
// hipGetLastError() is legal during stream capture.
int check_launch(const char* what) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return fail(MVME_ELAUNCH, std::string(what) + " launch failed: " + hipGetErrorString(err));
    return MVME_OK;
}

}  // namespace mvme

extern "C" int mvme_abi_version(void) { return MVME_ABI_VERSION; }

extern "C" const char* mvme_last_error(void) { return mvme::g_last_error.c_str(); }
