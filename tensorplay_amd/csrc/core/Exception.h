// Exception types of the host core; the Python bindings map each to the
// Python exception of the same name (as /root/reference/src/bindings/python/init.cpp:13-38).
#pragma once

#include <stdexcept>
#include <string>

namespace tensorplay {

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct RuntimeError : Error { using Error::Error; };
struct IndexError : Error { using Error::Error; };
struct TypeError : Error { using Error::Error; };
struct ValueError : Error { using Error::Error; };
struct NotImplementedError : Error { using Error::Error; };

}  // namespace tensorplay

#define TP_THROW(Type, msg) throw ::tensorplay::Type(std::string(msg))
#define TP_CHECK(cond, Type, msg) \
    do {                          \
        if (!(cond)) TP_THROW(Type, msg); \
    } while (0)
