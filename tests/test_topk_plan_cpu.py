"""Host-side checks of the top-k planner (tpr_topk_plan, no GPU): the segment
contract that the merge pass relies on.  A split row's segments each write
exactly k composites into the workspace and k_topk_merge ranks all
nseg * k of them, so every segment must hold at least k elements; the wave
kernel also needs a full first slice (1024 elements) per wave."""
import numpy as np
import pytest

from tensorplay_amd import _capi

MERGE_MAX = 8192  # candidates one merge workgroup ranks
SLICE = 1024      # elements per wave slice of the wave kernel


def _cols_grid():
    cols = set()
    for b in (4096, 8192, 16384, 32768, 65536):
        for m in range(1, 40):
            for d in (-3, -1, 0, 1, 5):
                cols.add(b * m + d)
    cols.update(int(c) for c in np.unique(np.geomspace(1, 1 << 24, 160).astype(np.int64)))
    cols.update([151936, 151937, 500000, 100000, 32769 * 3, 1 << 26])
    return sorted(c for c in cols if c >= 1)


def _check(dtype, rows, cols, k):
    kind, nseg, seg_len, nw, ws = _capi.topk_plan(dtype, rows, cols, k)
    esize = 8 if dtype in (_capi.INT64, _capi.UINT64, _capi.FLOAT64) else 4
    assert nseg >= 1 and seg_len >= 1
    if kind in ("rsel_seg", "wave", "block") and nseg > 1:
        assert nseg * k <= MERGE_MAX, (dtype, rows, cols, k, nseg)
        assert (nseg - 1) * seg_len < cols, ("empty last segment", dtype, rows, cols, k, nseg, seg_len)
        assert nseg * seg_len >= cols, ("elements past the last segment", rows, cols, k, nseg, seg_len)
        last = cols - (nseg - 1) * seg_len
        assert min(seg_len, last) >= k, ("segment shorter than k", dtype, rows, cols, k, nseg, seg_len)
        assert ws >= rows * nseg * k * 8
        if kind == "rsel_seg":
            assert (seg_len * esize) % 16 == 0  # segment starts stay 16-byte aligned
    else:
        assert nseg == 1
    if kind == "wave8":  # per-row flags in the workspace, one segment
        assert nseg == 1 and ws >= rows * 4 and esize == 8
    if kind == "wave":
        last = cols - (nseg - 1) * seg_len
        assert min(seg_len, last) >= nw * SLICE, ("wave without a full first slice", rows, cols, k, nw)
    return kind, nseg


@pytest.mark.parametrize("dtype", [_capi.FLOAT32, _capi.INT32, _capi.UINT8, _capi.INT16, _capi.FLOAT64])
def test_segments_hold_k_elements_every_k(dtype):
    """Every k <= 1024 on rows around the segment boundaries, few and many rows."""
    seen = set()
    cols_all = _cols_grid()
    for rows in (1, 3, 100, 256, 1024):
        for cols in cols_all:
            ks = range(1, min(cols, 1024) + 1) if rows in (1, 256) else range(1, min(cols, 1024) + 1, 37)
            for k in ks:
                kind, nseg = _check(dtype, rows, cols, k)
                seen.add((kind, nseg > 1))
    # the grid reaches the split plans
    if dtype in (_capi.FLOAT32, _capi.INT32):
        assert ("wave", True) in seen and ("rsel_seg", True) in seen
    else:
        assert ("rsel_seg", True) in seen or dtype == _capi.FLOAT64


def test_rsel_segment_formula_exhaustive():
    """The register radix select's segmentation (ceil(cols / nseg) rounded up to
    a multiple of 4) leaves no short or empty last segment, for every row
    length from 32769 to 2^20 and every k <= 1024 it serves."""
    cols = np.arange(32769, (1 << 20) + 1, dtype=np.int64)
    nseg = (cols + 32767) // 32768
    seg = ((cols + nseg - 1) // nseg + 3) & ~3
    last = cols - (nseg - 1) * seg
    # the shortest segment of each row; rows where nseg * k > 8192 stream instead
    shortest = np.minimum(seg, last)
    kmax = np.minimum(1024, 8192 // nseg)
    assert np.all(last >= 1)
    assert np.all(shortest >= kmax), cols[np.argmin(shortest - kmax)]


def test_plan_rejects_bad_shapes():
    with pytest.raises(_capi.TprError):
        _capi.topk_plan(_capi.FLOAT32, 4, 10, 11)
    with pytest.raises(_capi.TprError):
        _capi.topk_plan(99, 4, 10, 1)


def test_benchmark_shapes_plan():
    """The configs' shapes take the kernels the design describes."""
    assert _capi.topk_plan(_capi.FLOAT32, 1024, 32768, 64)[:2] == ("wave", 1)
    assert _capi.topk_plan(_capi.FLOAT32, 256, 151936, 50)[0] == "wave"
    assert _capi.topk_plan(_capi.FLOAT32, 16384, 1024, 32)[0] == "short"
    assert _capi.topk_plan(_capi.FLOAT32, 4096, 2048, 1000)[0] == "rsel"


def test_workspace_query_covers_every_alignment():
    """tpr_topk_workspace_bytes does not see the input pointer or stride, so it
    must cover the plan of an aligned and of an unaligned input alike (1- and
    2-byte rows take the wave kernel only when 16-byte aligned)."""
    import ctypes
    L = _capi.lib()
    rng = np.random.default_rng(5)
    for dtype in (_capi.INT8, _capi.UINT16, _capi.FLOAT32, _capi.INT32, _capi.FLOAT64):
        for _ in range(400):
            rows = int(rng.choice([1, 7, 42, 256, 1000]))
            cols = int(rng.integers(4000, 600000))
            k = int(rng.integers(1, 1025))
            k = min(k, cols)
            ws = L.tpr_topk_workspace_bytes(dtype, rows, cols, k)
            for aligned in (True, False):
                plan_ws = _capi.topk_plan(dtype, rows, cols, k, cols + (0 if aligned else 1), aligned)[4]
                assert ws >= plan_ws, (dtype, rows, cols, k, aligned, ws, plan_ws)
