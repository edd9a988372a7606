// et_abi.hip -- status plumbing of the C ABI (et_last_error, et_abi_version).
#include "et_common.hpp"

namespace et {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg)
{
    set_error(msg);
    return code;
}

int check_launch(const char* what)
{
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail(ET_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
    return ET_OK;
}

}  // namespace et

extern "C" int et_abi_version(void) { return ET_ABI_VERSION; }

extern "C" const char* et_last_error(void) { return et::g_last_error.c_str(); }
