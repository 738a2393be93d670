#include "Dispatcher.h"

#include <algorithm>

namespace tensorplay {

Dispatcher& Dispatcher::singleton() {
    static Dispatcher* d = new Dispatcher();  // never destroyed: safe in static init/exit order
    return *d;
}

void Dispatcher::registerKernel(const std::string& op, DispatchKey key, KernelFunction fn) {
    std::lock_guard<std::mutex> g(mu_);
    ops_[op][static_cast<int>(key)] = fn;
}

KernelFunction Dispatcher::getKernel(const std::string& op, DispatchKey key) {
    std::lock_guard<std::mutex> g(mu_);
    auto it = ops_.find(op);
    if (it == ops_.end()) return nullptr;
    auto k = it->second.find(static_cast<int>(key));
    return k == it->second.end() ? nullptr : k->second;
}

std::vector<std::string> Dispatcher::registeredOps(DispatchKey key) {
    std::lock_guard<std::mutex> g(mu_);
    std::vector<std::string> out;
    for (auto& kv : ops_)
        if (kv.second.count(static_cast<int>(key))) out.push_back(kv.first);
    std::sort(out.begin(), out.end());
    return out;
}

}  // namespace tensorplay
