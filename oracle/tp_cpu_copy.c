/*
 * TEST INFRASTRUCTURE ONLY -- see tp_cpu_reduce.h.  Never part of the product.
 *
 * CPU restatement of TensorPlay's CPU copy_ path:
 *   copy_recursive  /root/reference/p10/src/backend/cpu/CopyKernels.cpp:27-55
 *   copy_kernel     /root/reference/p10/src/backend/cpu/CopyKernels.cpp:73-127
 * Row-major walk over the destination's sizes; every element is converted with
 * a plain C cast, which for these arithmetic types is C++'s static_cast
 * (conversion to _Bool is x != 0, float -> integer truncates toward zero and
 * is undefined out of range, integer -> float rounds to nearest).
 *
 * Parity pins (tests/test_oracle.py): numpy's astype on as_strided views
 * (the same conversions), brute force on tiny shapes, broadcasting views.
 */
#include "tp_cpu_reduce.h"
#include <stdbool.h>
#include <stdint.h>

#define OR_TYPES(_) \
    _(uint8_t, 0) _(int8_t, 1) _(int16_t, 2) _(int32_t, 3) _(int64_t, 4) \
    _(uint16_t, 5) _(uint32_t, 6) _(uint64_t, 7) _(float, 8) _(double, 9) _(bool, 10)

/* The destination list again (a macro cannot expand inside its own expansion). */
#define OR_DST_TYPES(_) \
    _(uint8_t, 0) _(int8_t, 1) _(int16_t, 2) _(int32_t, 3) _(int64_t, 4) \
    _(uint16_t, 5) _(uint32_t, 6) _(uint64_t, 7) _(float, 8) _(double, 9) _(bool, 10)

/* One element: load as the source type, C-cast, store as the destination type. */
#define OR_DST_STORE(dtype, dcode) \
    case dcode: *(dtype*)d = (dtype)v; break;
#define OR_DEF_STORE(stype, scode) \
    static void or_store_##scode(void* d, int dst_dtype, stype v) { \
        switch (dst_dtype) { OR_DST_TYPES(OR_DST_STORE) default: break; } \
    }
OR_TYPES(OR_DEF_STORE)
#define OR_SRC_CASE(stype, scode) \
    case scode: or_store_##scode(d, dst_dtype, *(const stype*)s); return 0;

static int or_esize(int dt) {
    switch (dt) {
        case 0: case 1: case 10: return 1;
        case 2: case 5: return 2;
        case 3: case 6: case 8: return 4;
        case 4: case 7: case 9: return 8;
        default: return 0;
    }
}

static int or_cast_one(void* d, int dst_dtype, const void* s, int src_dtype) {
    switch (src_dtype) {
        OR_TYPES(OR_SRC_CASE)
        default: return -1;
    }
}

/* copy_recursive: dims outermost first, innermost loop over the last dim. */
static void or_copy_rec(char* dst, int dde, const int64_t* dst_strides, int dst_dtype,
                        const char* src, int sde, const int64_t* src_strides, int src_dtype,
                        const int64_t* sizes, int ndim, int dim, int64_t doff, int64_t soff) {
    if (ndim == 0) {
        or_cast_one(dst, dst_dtype, src, src_dtype);
        return;
    }
    const int64_t n = sizes[dim];
    for (int64_t i = 0; i < n; ++i) {
        const int64_t dd = doff + i * dst_strides[dim], ss = soff + i * src_strides[dim];
        if (dim == ndim - 1)
            or_cast_one(dst + dd * dde, dst_dtype, src + ss * sde, src_dtype);
        else
            or_copy_rec(dst, dde, dst_strides, dst_dtype, src, sde, src_strides, src_dtype, sizes, ndim,
                        dim + 1, dd, ss);
    }
}

int or_copy(void* dst, int dst_dtype, const int64_t* dst_strides, const void* src, int src_dtype,
            const int64_t* src_strides, int ndim, const int64_t* sizes) {
    const int dde = or_esize(dst_dtype), sde = or_esize(src_dtype);
    if (!dde || !sde || ndim < 0) return -1;
    for (int i = 0; i < ndim; ++i)
        if (sizes[i] == 0) return 0;
    or_copy_rec((char*)dst, dde, dst_strides, dst_dtype, (const char*)src, sde, src_strides, src_dtype, sizes,
                ndim, 0, 0, 0);
    return 0;
}
