// runtime_error.h — the error type of the forward-pass runtime. The reference prints a message
// and exits 1 on every load/alloc/shape failure (model.cpp:16-21, 737-740, 801-816, 1563-1566);
// here the failure is thrown so the C-ABI can return it to the caller, and the CLI turns it back
// into "error: <message>" + exit(1).
#pragma once

#include <stdexcept>
#include <string>

struct gl_error : std::runtime_error {
    explicit gl_error(const std::string & msg) : std::runtime_error(msg) {}
};
