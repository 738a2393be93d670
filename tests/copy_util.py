"""Shared helpers of the copy_ tests (imported only by tests).

Data for a (src dtype, dst dtype) pair stays where C's cast -- the
reference's static_cast (cpu/CopyKernels.cpp:36,44) -- is defined:
float -> unsigned in [0, 200), float -> signed in the target's range,
float64 -> float32 inside float32's range.  Integer -> integer covers the
whole source range (modular wrap on narrowing, as C and numpy do).  NaN, +-inf
and -0.0 appear where the cast is defined (float -> float, float -> bool)."""
import numpy as np

DTYPES = [np.uint8, np.int8, np.int16, np.int32, np.int64, np.uint16, np.uint32, np.uint64,
          np.float32, np.float64, np.bool_]
FLOATS = (np.float32, np.float64)


def _is_float(dt):
    return np.dtype(dt) in (np.dtype(np.float32), np.dtype(np.float64))


def src_values(rng, src, dst, shape):
    src, dst = np.dtype(src), np.dtype(dst)
    n = int(np.prod(shape)) if len(shape) else 1
    if src == np.bool_:
        v = rng.random(n) < 0.5
    elif _is_float(src):
        if dst == np.bool_ or _is_float(dst):
            v = rng.standard_normal(n) * 1e3
            if dst == np.float32 and src == np.float64:
                v = v * rng.choice([1e-30, 1.0, 1e30], n)  # inside float32's range, many rounding cases
            k = min(n, 5)
            v[:k] = [np.nan, np.inf, -np.inf, -0.0, 0.0][:k]
            rng.shuffle(v)
        elif np.issubdtype(dst, np.unsignedinteger):
            v = rng.uniform(0, 200, n)
        else:
            info = np.iinfo(dst)
            lo, hi = max(float(info.min), -1e15), min(float(info.max), 1e15)
            v = rng.uniform(lo / 2, hi / 2, n) * rng.choice([1e-6, 1e-3, 1.0], n)
        v = v.astype(src)
    else:
        info = np.iinfo(src)
        big = rng.integers(info.min, info.max, size=n, dtype=src, endpoint=True)
        small = rng.integers(max(info.min, -300), min(info.max, 300), size=n, endpoint=True).astype(src)
        v = np.where(rng.random(n) < 0.5, big, small)
    return np.asarray(v, dtype=src).reshape(shape)


def as_bytes(a):
    """Bitwise view (NaNs compare by payload) of a dense copy."""
    a = np.ascontiguousarray(a)
    return a.view(np.uint8).reshape(-1)


def expected(src_view, dst_dtype):
    """numpy's astype of the same view: the C cast, element by element."""
    with np.errstate(invalid="ignore", over="ignore"):
        return src_view.astype(dst_dtype)
