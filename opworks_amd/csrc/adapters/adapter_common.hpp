#pragma once

// Shared guard for the `solve` adapters. Each adapter is its own shared
// library exporting `extern "C" void solve(...)`, called through ctypes by the
// challenge runner (reference caller: tests/run.py:48-64). A contract
// violation leaves the outputs untouched, is written to stderr and is kept
// for opw_solve_last_error(); no C++ exception crosses the C boundary.
// Every solve synchronizes the device before returning.

#include <cstdio>
#include <exception>
#include <string>

#include <opworks>

namespace opworks_adapter {

inline std::string &last_error() {
    static thread_local std::string message;
    return message;
}

template <typename Fn> void guarded(const char *name, Fn &&fn) {
    last_error().clear();
    try {
        fn();
        opworks::synchronize();
    } catch (const std::exception &e) {
        last_error() = std::string(name) + ": " + e.what();
        std::fprintf(stderr, "opworks solve(%s)\n", last_error().c_str());
    }
}

} // namespace opworks_adapter

extern "C" const char *opw_solve_last_error() { return opworks_adapter::last_error().c_str(); }
