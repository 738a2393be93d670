// Devices of the host core: the CPU and one backend for AMD GPUs (ROCm).
// Mirrors the shape of TensorPlay's Device (/root/reference/p10/include/Device.h:11-21)
// with DeviceType::ROCm in place of CUDA.
#pragma once

#include <cstdint>
#include <string>

#include "Exception.h"

namespace tensorplay {

enum class DeviceType : int8_t { CPU = 0, ROCm = 1 };

struct Device {
    DeviceType type = DeviceType::CPU;
    int index = 0;

    Device() = default;
    Device(DeviceType t, int i = 0) : type(t), index(i) {}
    // "cpu", "rocm", "rocm:1"
    explicit Device(const std::string& s) {
        std::string name = s;
        int idx = 0;
        auto colon = s.find(':');
        if (colon != std::string::npos) {
            name = s.substr(0, colon);
            try {
                idx = std::stoi(s.substr(colon + 1));
            } catch (...) {
                TP_THROW(ValueError, "invalid device string: " + s);
            }
        }
        if (name == "cpu") type = DeviceType::CPU;
        else if (name == "rocm") type = DeviceType::ROCm;
        else TP_THROW(ValueError, "unknown device '" + s + "' (expected cpu or rocm[:N])");
        if (idx < 0) TP_THROW(ValueError, "negative device index: " + s);
        index = idx;
    }
    bool is_cpu() const { return type == DeviceType::CPU; }
    bool is_rocm() const { return type == DeviceType::ROCm; }
    bool operator==(const Device& o) const { return type == o.type && (type == DeviceType::CPU || index == o.index); }
    bool operator!=(const Device& o) const { return !(*this == o); }
    std::string str() const { return is_cpu() ? "cpu" : "rocm:" + std::to_string(index); }
};

}  // namespace tensorplay
