#pragma once

// Exception capture for every extern "C" entry point: contract violations and
// other C++ exceptions become a -1 return plus a thread-local message; nothing
// is thrown across the ABI (same policy as the reference's
// src/llama_c_api.cu:16-35).

#include <cstring>
#include <exception>
#include <new>
#include <string>

namespace opworks::capi {

inline std::string &last_error() {
    static thread_local std::string msg;
    return msg;
}

inline int capture_error(const char *what, char *err = nullptr, int err_len = 0) {
    last_error() = what ? what : "unknown error";
    if (err && err_len > 0) {
        std::strncpy(err, last_error().c_str(), static_cast<size_t>(err_len) - 1);
        err[err_len - 1] = '\0';
    }
    return -1;
}

template <typename F> int guard(F &&f, char *err = nullptr, int err_len = 0) {
    try {
        return f();
    } catch (const std::exception &e) {
        return capture_error(e.what(), err, err_len);
    } catch (...) {
        return capture_error("unknown C++ exception", err, err_len);
    }
}

} // namespace opworks::capi
