// qwm_error.cpp -- the calling thread's last error and the exception barrier
// of the C ABI.  The message lives in a fixed thread-local buffer, so
// recording an error never allocates and cannot throw.
#include <cstdarg>
#include <cstdio>
#include <exception>
#include <new>
#include <string>

#include "qwm_internal.h"

namespace qwm {

static thread_local char g_last_error[1024];

const char * last_error() noexcept { return g_last_error; }

void set_error(const char * msg) noexcept { std::snprintf(g_last_error, sizeof g_last_error, "%s", msg); }
int fail(int code, const char * msg) noexcept {
    set_error(msg);
    return code;
}
int fail(int code, const std::string & msg) noexcept { return fail(code, msg.c_str()); }
int failf(int code, const char * fmt, ...) noexcept {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
    return code;
}
int fail_exception(const char * who) noexcept {
    try {
        throw;
    } catch (const std::bad_alloc &) {
        return failf(QWM_ERR_NOMEM, "%s: out of host memory (std::bad_alloc)", who);
    } catch (const std::exception & e) {
        return failf(QWM_ERR_INTERNAL, "%s: %s", who, e.what());
    } catch (...) {
        return failf(QWM_ERR_INTERNAL, "%s: unknown exception", who);
    }
}

}  // namespace qwm
