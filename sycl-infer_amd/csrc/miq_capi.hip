// Library-wide pieces of the C ABI: version, error text, row sizes.
#include <cstdarg>
#include <cstdio>

#include "miq_common.h"

namespace miq {

static thread_local char g_err[512] = "";

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

int check_launch(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: %s", what, hipGetErrorString(e));
        return MIQ_EHIP;
    }
    return MIQ_OK;
}

}  // namespace miq

extern "C" {

const char *miq_version(void) { return "miq 0.1 (gfx950)"; }

const char *miq_last_error(void) { return miq::g_err; }

size_t miq_row_bytes(uint32_t type, int K) {
    const int vb = miq::block_values(type);
    if (miq::block_bytes(type) == 0 || K <= 0 || K % vb) return 0;
    return (size_t)(K / vb) * miq::block_bytes(type);
}

}  // extern "C"
