// Element types of the host core.  The numbering follows TensorPlay's
// ScalarType (/root/reference/p10/include/DType.h:63-79) so that values pass
// unchanged through the C-ABI (enum tpr_dtype).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

namespace tensorplay {

enum class DType : int8_t {
    UInt8 = 0, Int8, Int16, Int32, Int64, UInt16, UInt32, UInt64,
    Float32, Float64, Bool,
    Undefined = 13,
};

inline size_t elementSize(DType t) {
    switch (t) {
        case DType::UInt8: case DType::Int8: case DType::Bool: return 1;
        case DType::Int16: case DType::UInt16: return 2;
        case DType::Int32: case DType::UInt32: case DType::Float32: return 4;
        case DType::Int64: case DType::UInt64: case DType::Float64: return 8;
        default: return 0;
    }
}

inline bool isIntegralType(DType t, bool includeBool) {
    switch (t) {
        case DType::UInt8: case DType::Int8: case DType::Int16: case DType::Int32:
        case DType::Int64: case DType::UInt16: case DType::UInt32: case DType::UInt64: return true;
        case DType::Bool: return includeBool;
        default: return false;
    }
}

inline bool isFloatingType(DType t) { return t == DType::Float32 || t == DType::Float64; }

inline const char* toString(DType t) {
    switch (t) {
        case DType::UInt8: return "uint8";
        case DType::Int8: return "int8";
        case DType::Int16: return "int16";
        case DType::Int32: return "int32";
        case DType::Int64: return "int64";
        case DType::UInt16: return "uint16";
        case DType::UInt32: return "uint32";
        case DType::UInt64: return "uint64";
        case DType::Float32: return "float32";
        case DType::Float64: return "float64";
        case DType::Bool: return "bool";
        default: return "undefined";
    }
}

}  // namespace tensorplay
