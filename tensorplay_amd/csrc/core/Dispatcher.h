// Operator registry of the host core: kernels are registered under
// (schema name, DispatchKey) at library-load time and looked up per call.
// Same shape as TensorPlay's P10 dispatcher
// (/root/reference/p10/include/Dispatcher.h:16-96, p10/src/Dispatcher.cpp:11-27):
// the registry is keyed by the full schema name ("sum.dim_IntList"), the last
// registration for a (name, key) pair wins, and a missing kernel raises
// NotImplementedError.  It adds DispatchKey::ROCm.  Kernels must be registered
// with exactly the argument types DispatchStub calls them with (the
// reference's STUB_TYPE_MAP, tools/codegen/gen.py:38-53); the TP_LIBRARY_IMPL
// helper checks that at compile time through KernelSig.
#pragma once

#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "Device.h"
#include "Exception.h"

namespace tensorplay {

enum class DispatchKey : int { CPU = 0, ROCm = 1, Autograd = 2, EndOfKeys = 3 };

inline const char* toString(DispatchKey k) {
    switch (k) {
        case DispatchKey::CPU: return "CPU";
        case DispatchKey::ROCm: return "ROCm";
        case DispatchKey::Autograd: return "Autograd";
        default: return "Unknown";
    }
}

inline DispatchKey computeDispatchKey(const Device& d) {
    return d.is_rocm() ? DispatchKey::ROCm : DispatchKey::CPU;
}

using KernelFunction = void*;

class Dispatcher {
public:
    static Dispatcher& singleton();
    void registerKernel(const std::string& op, DispatchKey key, KernelFunction fn);
    KernelFunction getKernel(const std::string& op, DispatchKey key);
    std::vector<std::string> registeredOps(DispatchKey key);

private:
    Dispatcher() = default;
    std::unordered_map<std::string, std::unordered_map<int, KernelFunction>> ops_;
    std::mutex mu_;
};

template <typename Return, typename... Args>
struct DispatchStub {
    static Return call(const std::string& op, DispatchKey key, Args... args) {
        KernelFunction k = Dispatcher::singleton().getKernel(op, key);
        if (!k) {
            TP_THROW(NotImplementedError,
                     "Kernel not found for op: " + op + " on backend: " + toString(key));
        }
        return reinterpret_cast<Return (*)(Args...)>(k)(std::forward<Args>(args)...);
    }
};

class Library {
public:
    explicit Library(DispatchKey key) : key_(key) {}
    // The function type is spelled out by the caller, so a kernel whose
    // parameters differ from the stub's (e.g. a vector taken by value where the
    // stub passes const&) does not compile.
    template <typename Sig>
    Library& impl(const std::string& name, Sig* fn) {
        Dispatcher::singleton().registerKernel(name, key_, reinterpret_cast<KernelFunction>(fn));
        return *this;
    }

private:
    DispatchKey key_;
};

#define TP_CONCAT_INNER(a, b) a##b
#define TP_CONCAT(a, b) TP_CONCAT_INNER(a, b)
#define TENSORPLAY_LIBRARY_IMPL(KEY, NAME)                                              \
    static void TP_CONCAT(tp_library_init_, NAME)(::tensorplay::Library&);              \
    static const int TP_CONCAT(tp_library_reg_, NAME) = [] {                            \
        ::tensorplay::Library lib(::tensorplay::DispatchKey::KEY);                      \
        TP_CONCAT(tp_library_init_, NAME)(lib);                                          \
        return 0;                                                                        \
    }();                                                                                 \
    static void TP_CONCAT(tp_library_init_, NAME)(::tensorplay::Library & m)

}  // namespace tensorplay
