// Status-code errors of the C ABI, host-only (no HIP headers): shared by the
// g++-built host files and the HIP translation units.
#pragma once

#include <cstdint>
#include <functional>
#include <string>
#include <utility>

#include "../../include/midman_hip.h"

namespace mmh {

// An error that the C-ABI boundary turns into a status code + message.
struct Error {
    int32_t status;
    std::string message;
};

[[noreturn]] void fail(int32_t status, const std::string &message);

// Runs an entry point body: an Error becomes its status and the thread's
// error message; any other exception becomes MMH_ERR_PANIC.
int32_t guard_impl(const std::function<int32_t()> &body);
template <class F>
int32_t guard(F &&f) {
    return guard_impl(std::function<int32_t()>(std::forward<F>(f)));
}

}  // namespace mmh
