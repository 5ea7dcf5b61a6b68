// Status codes and the per-thread error message of the C ABI
// (midman-api/src/ffi.rs:5-32, 44-61, 99-145): every entry point runs its body
// through guard(), which turns an mmh::Error into its status and message and
// any other exception into MMH_ERR_PANIC, so nothing unwinds across the
// boundary. Host code (built with g++).
#include <exception>
#include <new>
#include <string>

#include "mmh_error.h"

namespace mmh {

namespace {
thread_local std::string g_error;
}  // namespace

void fail(int32_t status, const std::string &message) { throw Error{status, message}; }

int32_t guard_impl(const std::function<int32_t()> &body) {
    g_error.clear();
    try {
        return body();
    } catch (const Error &e) {
        g_error = e.message;
        return e.status;
    } catch (const std::bad_alloc &) {
        g_error = "out of host memory";
        return MMH_ERR_OTHER;
    } catch (const std::exception &e) {
        g_error = std::string("internal error: ") + e.what();
        return MMH_ERR_PANIC;
    } catch (...) {
        g_error = "internal error: unknown exception";
        return MMH_ERR_PANIC;
    }
}

}  // namespace mmh

extern "C" {

uint32_t mmh_abi_version(void) { return MMH_ABI_VERSION; }
const char *mmh_error_ptr(void) { return mmh::g_error.c_str(); }
uint32_t mmh_error_len(void) { return (uint32_t)mmh::g_error.size(); }

}  // extern "C"
