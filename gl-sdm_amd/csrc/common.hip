// Status reporting shared by every entry point of libglsdm.so.
#include <cstdarg>
#include <cstdio>

#include "glsdm_internal.h"

namespace glsdm {

static thread_local char g_last_error[512] = "";

int fail(int status, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
    return status;
}

int check_launch(const char *what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(GLSDM_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return GLSDM_OK;
}

}  // namespace glsdm

extern "C" const char *glsdm_version(void) { return "glsdm-mi355x 0.1.0 (gfx950)"; }

extern "C" const char *glsdm_last_error(void) { return glsdm::g_last_error; }
