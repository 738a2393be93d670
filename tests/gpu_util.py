"""Shared helpers of the GPU parity tests (imported only by tests)."""
import numpy as np

REL_TOL = 1e-5  # float sums/means/var/std vs an fp64 host reference (north_star bound)


def device_view(torch, base_np, view_np):
    """Put base_np on the GPU and return the torch view with view_np's geometry."""
    assert view_np.base is base_np or view_np is base_np or np.shares_memory(view_np, base_np)
    t = torch.from_numpy(base_np).to("cuda")
    off = (view_np.__array_interface__["data"][0] - base_np.__array_interface__["data"][0]) // 4
    return t.as_strided(view_np.shape, [s // 4 for s in view_np.strides], off)


def fp64_reference(v, op, dims, correction=1, p=2.0):
    x = v.astype(np.float64)
    ax = None if dims is None else tuple(dims)
    if op == "sum":
        return x.sum(axis=ax)
    if op == "prod":
        return x.prod(axis=ax)
    if op == "norm":
        with np.errstate(divide="ignore", over="ignore"):
            s = (np.abs(x) ** p).sum(axis=ax)
            return s ** (1.0 / p)
    if op == "mean":
        return x.mean(axis=ax) if x.size else np.full(np.sum(x, axis=ax).shape, np.nan)
    if op in ("var", "std"):
        n = x.size if ax is None else int(np.prod([x.shape[d] for d in ax]))
        if n == 0:
            r = np.full(np.sum(x, axis=ax).shape, np.nan)
        else:
            m = x.mean(axis=ax, keepdims=True)
            ss = ((x - m) ** 2).sum(axis=ax)
            with np.errstate(divide="ignore", invalid="ignore"):
                r = ss / max(0.0, n - correction)
        return np.sqrt(r) if op == "std" else r
    raise ValueError(op)


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    both_nan = np.isnan(got) & np.isnan(ref)
    same_inf = np.isinf(ref) & (got == ref)
    denom = np.maximum(np.abs(ref), 1e-30)
    e = np.abs(got - ref) / denom
    e = np.where(both_nan | same_inf | ((got == 0) & (ref == 0)), 0.0, e)
    return float(e.max()) if e.size else 0.0


def assert_close_rel(got, ref, tol=REL_TOL):
    e = rel_err(got, ref)
    assert e <= tol, f"max relative error {e:.3e} > {tol:.1e}"
    return e


def assert_bits_equal(got, expect):
    got = np.asarray(got)
    expect = np.asarray(expect)
    assert got.shape == expect.shape, (got.shape, expect.shape)
    if got.dtype == np.float32:
        np.testing.assert_array_equal(got.view(np.uint32), expect.astype(np.float32).view(np.uint32))
    else:
        np.testing.assert_array_equal(got, expect)


def softmax_reference(x64, dim, log):
    """fp64 softmax / log_softmax of x64 along dim with the reference's NaN
    rules (max ignores NaN; a NaN, or no value above -inf, makes the slice NaN)."""
    x = np.moveaxis(np.asarray(x64, np.float64), dim, -1)
    with np.errstate(invalid="ignore", over="ignore"):
        m = np.max(np.where(np.isnan(x), -np.inf, x), axis=-1, keepdims=True)
        d = x - m
        e = np.exp(d)
        s = e.sum(-1, keepdims=True)
        lse = np.log(s)
        y = d - lse if log else e / s
    y = np.where(np.isnan(s) | (m == -np.inf), np.nan, y)
    return np.moveaxis(y, -1, dim), np.moveaxis(np.broadcast_to(lse, x.shape), -1, dim)


def softmax_error(got, x64, dim, log, log_abs_floor=0.0):
    """Max error of an fp32 softmax / log_softmax in units of its tolerance:
    softmax 1e-5 relative; log_softmax 1e-5 * (|y| + |log-sum-exp|) absolute
    (the terms it subtracts), plus log_abs_floor (0 unless a caller states
    one).  NaN / +-inf positions must match exactly.  Returns the worst ratio
    (<= 1 passes)."""
    ref, lse = softmax_reference(x64, dim, log)
    got = np.asarray(got, np.float64)
    assert got.shape == ref.shape
    nan_r = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan_r)
    inf_r = np.isinf(ref)
    np.testing.assert_array_equal(got[inf_r], ref[inf_r])
    ok = ~nan_r & ~inf_r
    if not ok.any():
        return 0.0
    if log:
        tol = 1e-5 * (np.abs(ref) + np.abs(lse)) + log_abs_floor
    else:
        tol = 1e-5 * np.abs(ref)
    with np.errstate(invalid="ignore"):
        err = np.abs(got - ref)
    ratio = np.where(ok, err / np.maximum(tol, 1e-38), 0.0)
    ratio = np.where(ok & (err == 0), 0.0, ratio)
    return float(ratio.max())
