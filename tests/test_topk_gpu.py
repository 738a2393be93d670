"""GPU parity of tpr_topk (via the C-ABI) against the CPU oracle: values and
indices bit-exact (ties to the lowest index, -0.0 == +0.0, NaN largest)."""
import numpy as np
import pytest

from oracle import oracle as O
from tensorplay_amd import _capi
from tests.gpu_util import assert_bits_equal, device_view

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(autouse=True)
def _reset_knobs():
    _capi.debug_get("topk_merge_clamped")  # clears the test build's merge check counter
    yield
    clamped = _capi.debug_get("topk_merge_clamped")
    for k in ("topk_fallback", "topk_variant", "topk_waves", "splits", "topk_short", "topk_radix", "topk_dyn"):
        _capi.debug_set(k, 0)
    # every split row's segments wrote their k composites: no merge output index needed clamping
    assert clamped == 0, f"{clamped} merge outputs had a row index past the row"


def check(base, v, k, largest=True):
    print(f"case topk shape={v.shape} strides={v.strides} k={k} largest={largest}", flush=True)
    t = device_view(torch, base, v)
    gv, gi = _capi.topk(t, k, largest)
    torch.cuda.synchronize()
    ev, ei = O.topk(np.ascontiguousarray(v) if v.strides[1] != 4 else v, k, largest)
    assert_bits_equal(gi.cpu().numpy(), ei)
    assert_bits_equal(gv.cpu().numpy(), ev)


@pytest.mark.parametrize("fallback", [0, 1])
def test_random_shapes(fallback):
    _capi.debug_set("topk_fallback", fallback)
    rng = np.random.default_rng(21)
    for rows, cols in [(1, 1), (3, 7), (5, 64), (4, 1000), (2, 4097), (9, 16384), (3, 40000)]:
        x = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
        for k in sorted({1, min(cols, 7), min(cols, 64), min(cols, 1024), cols if cols <= 1024 else 1024}):
            for largest in (True, False):
                check(x, x, k, largest)


def test_adversarial_rows():
    rng = np.random.default_rng(22)
    n = 20000
    rows = [np.full(n, 0.25, np.float32),                        # all equal
            np.arange(n, dtype=np.float32),                      # ascending
            np.arange(n, dtype=np.float32)[::-1].copy(),         # descending
            rng.integers(0, 3, n).astype(np.float32),            # heavy duplicates
            np.where(rng.random(n) < 0.5, -0.0, 0.0).astype(np.float32),
            rng.standard_normal(n).astype(np.float32)]
    r = rng.standard_normal(n).astype(np.float32)
    r[rng.choice(n, 100, replace=False)] = np.nan
    r[rng.choice(n, 10, replace=False)] = np.inf
    r[rng.choice(n, 10, replace=False)] = -np.inf
    rows.append(r)
    x = np.stack(rows)
    for k in (1, 50, 64, 1024):
        for largest in (True, False):
            check(x, x, k, largest)


def test_strided_and_misaligned_rows():
    rng = np.random.default_rng(23)
    b = rng.uniform(-1, 1, (6, 5003)).astype(np.float32)
    check(b, b[:, 1:], 33)            # misaligned rows, odd stride
    check(b, b[::2, :4096], 64)       # row stride 2*5003
    check(b, b[:, 3:3 + 1031], 100)
    # long misaligned rows: the wave kernel's 32-bit buffer loads
    c = rng.standard_normal((4, 40003)).astype(np.float32)
    for k in (1, 50, 128):
        check(c, c[:, 1:], k)
        check(c, c[:, 1:], k, False)
    check(c, c[:, 2:], 64)


def test_config3_uniform():
    rng = np.random.default_rng(3)
    x = rng.uniform(-1, 1, (1024, 32768)).astype(np.float32)
    # U(-1,1) fp32 rows of 32768 contain duplicate values: ties are exercised
    assert any(len(np.unique(x[r])) < x.shape[1] for r in range(64))
    check(x, x, 64)


@pytest.mark.parametrize("dyn", [0, -1])
def test_config5_peaked_logits(dyn):
    # dyn=0: the 16-wave kernel hands slices out dynamically; -1: static order
    _capi.debug_set("topk_dyn", dyn)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((256, 151936), dtype=np.float32) * np.float32(3.0)
    for r in range(256):
        x[r, rng.choice(151936, 8, replace=False)] += np.float32(15.0)
    check(x, x, 50)


@pytest.mark.parametrize("waves", [4, 8, 16])
@pytest.mark.parametrize("variant", [1, 2, 3, 5])
@pytest.mark.parametrize("splits", [0, 1, 2, 3, 5])
def test_wave_kernel_variants_and_segments(variant, splits, waves):
    # wave-kernel prefetch depths and workgroup sizes, rows cut into 1..5
    # segments (merge pass); static slice order on odd split counts
    _capi.debug_set("topk_dyn", -1 if splits % 2 else 0)
    _capi.debug_set("topk_variant", variant)
    _capi.debug_set("topk_waves", waves)
    _capi.debug_set("splits", splits)
    rng = np.random.default_rng(24 + splits)
    x = rng.standard_normal((6, 50000)).astype(np.float32)
    x[1, :] = np.round(x[1, :] * 4) / 4   # many duplicate values
    x[2, 123] = np.nan
    for k in (1, 50, 128):
        for largest in (True, False):
            check(x, x, k, largest)


@pytest.mark.parametrize("waves", [4, 8, 16])
@pytest.mark.parametrize("variant", [1, 2, 3])
def test_rising_rows_stale_candidates(variant, waves):
    # Values trend upwards along the row, so every wave keeps finding better
    # elements, compacts repeatedly and raises the shared bound while other
    # waves still hold entries admitted under older, lower bounds.
    _capi.debug_set("topk_variant", variant)
    _capi.debug_set("topk_waves", waves)
    rng = np.random.default_rng(25)
    n = 65536
    trend = np.linspace(0, 50, n, dtype=np.float32)
    x = np.stack([trend + rng.standard_normal(n).astype(np.float32) * s for s in (0.5, 2.0, 8.0)]
                 + [trend[::-1].copy() + rng.standard_normal(n).astype(np.float32)])
    for k in (1, 17, 64, 128):
        check(x, x, k, True)
        check(x, x, k, False)


@pytest.mark.parametrize("waves", [4, 8, 16])
@pytest.mark.parametrize("variant", [1, 2, 3])
def test_single_row_ragged_end(variant, waves):
    # one aligned row whose length is not a multiple of 4: the last 128-bit
    # load straddles the row end (the segment range check zeroes the rest)
    _capi.debug_set("topk_variant", variant)
    _capi.debug_set("topk_waves", waves)
    rng = np.random.default_rng(26)
    for n in (50003, 65537, 16387):
        x = rng.standard_normal((1, n)).astype(np.float32)
        x[0, n - 1] = 100.0  # the last element is the maximum
        x[0, n - 3] = 99.0
        for k in (1, 3, 64):
            check(x, x, k, True)
            check(x, x, k, False)


@pytest.mark.parametrize("waves", [4, 8, 16])
def test_denormals_signed_zeros_and_infinities(waves):
    # Thresholds that land on +-0, denormals and +-inf: the float-domain filter
    # must agree with the key order (denormals kept, -0.0 == +0.0).
    _capi.debug_set("topk_waves", waves)
    rng = np.random.default_rng(27)
    n = 40000
    tiny = np.float32(1e-45)  # smallest denormal
    pool = np.array([0.0, -0.0, tiny, -tiny, 3 * tiny, -3 * tiny, 1e-39, -1e-39,
                     np.inf, -np.inf, 1.0, -1.0], np.float32)
    x = pool[rng.integers(0, len(pool), size=(4, n))]
    x[1] = np.where(rng.random(n) < 0.5, np.float32(0.0), np.float32(-0.0))
    x[2, ::7] = np.nan
    x[3] = -np.inf
    x[3, 17] = -1e-39
    for k in (1, 5, 64, 128):
        check(x, x, k, True)
        check(x, x, k, False)


@pytest.mark.parametrize("short", [1, -1])
def test_short_rows(short):
    """Rows of <= 4096 elements with k <= 64 take the lane-group kernel (16, 32
    or 64 lanes per row, rows held in registers); -1 forces the workgroup
    kernels for the same cases.  Ragged row lengths, row counts that leave a
    workgroup partly empty, misaligned rows, ties, NaN / +-0 / +-inf."""
    _capi.debug_set("topk_short", short)
    rng = np.random.default_rng(28)
    for rows, cols in [(1, 5), (7, 16), (33, 64), (19, 255), (130, 256), (9, 1000), (5, 2049), (6, 4096),
                       (3, 4093)]:
        x = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
        for k in sorted({1, min(cols, 3), min(cols, 8), min(cols, 17), min(cols, 32), min(cols, 64), min(cols, 65),
                         min(cols, 100), min(cols, 128)}):
            check(x, x, k, True)
            check(x, x, k, False)
    b = rng.standard_normal((40, 1031)).astype(np.float32)
    check(b, b[:, 1:1025], 16)          # misaligned rows: scalar loads
    check(b, b[::3, :600], 50)
    # exact path: more than 8 lanes' worth of elements tie at or above the bound
    t = np.full((5, 3000), 2.0, np.float32)
    t[1, ::2] = 1.0
    t[2] = np.round(rng.standard_normal(3000) * 2) / 2
    t[3, 100:2100] = 7.0
    t[4] = np.where(rng.random(3000) < 0.5, -0.0, 0.0)
    for k in (1, 10, 33, 64, 100, 128):
        check(t, t, k, True)
        check(t, t, k, False)
    s = rng.standard_normal((8, 512)).astype(np.float32)
    s[0, ::5] = np.nan
    s[1, :] = -np.inf
    s[2, 7] = np.inf
    s[3, :] = np.float32(1e-45)
    s[3, 300] = -np.float32(1e-45)
    for k in (1, 7, 64, 127):
        check(s, s, k, True)
        check(s, s, k, False)


def test_short_full_rows_special_values():
    """Full float32 rows of the lane-group kernel (every lane's vectors inside
    the row: 64 .. 4096 elements) filter on the floats themselves; NaN of
    every kind (quiet, signalling, negative; whole rows of them), +-0,
    denormals and +-inf must still select exactly as the key order does."""
    rng = np.random.default_rng(31)
    snan = np.array([0x7F800001, 0xFFC00000, 0x7FFFFFFF], np.uint32).view(np.float32)
    tiny = np.float32(1e-45)
    for rows, cols in [(70, 64), (130, 256), (40, 512), (33, 1024), (9, 2048), (8, 4096)]:
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        x[0, ::5] = np.nan
        x[1, :] = np.nan
        x[2, ::3] = snan[rng.integers(0, 3, len(x[2, ::3]))]
        x[3, :] = -np.inf
        x[3, 9] = tiny
        x[4] = np.where(rng.random(cols) < 0.5, -0.0, 0.0)
        x[5] = rng.choice(np.array([tiny, -tiny, 0.0, -0.0, 1e-39, -1e-39], np.float32), cols)
        x[6, 1::2] = np.nan
        x[7, :] = np.inf
        for k in (1, 7, 32, 50, 64):
            if k <= cols:
                check(x, x, k, True)
                check(x, x, k, False)


def test_short_rows_many():
    # BASELINE-like volumes of short rows: every row and every output checked
    rng = np.random.default_rng(29)
    x = rng.uniform(-1, 1, (65536, 256)).astype(np.float32)
    check(x, x, 8)
    y = rng.standard_normal((16384, 1024)).astype(np.float32)
    check(y, y, 32)
    # 64-lane rows whose candidates (37..128 after the bound) are ranked by a
    # lane sort of one or two composites per lane instead of compares
    # k of 65..128 on >= 8 rows per CU of <= 1024 elements: exact bit search in
    # the lane groups, then the lane sort
    for rows, cols, k in ((2048, 1024, 48), (1024, 2048, 64), (4096, 512, 40), (2048, 1024, 37),
                          (4096, 1000, 100), (2048, 256, 128), (2048, 1024, 65), (2048, 2048, 90)):
        z = rng.standard_normal((rows, cols)).astype(np.float32)
        z[::5] = np.round(z[::5] * 4) / 4  # ties among the candidates
        check(z, z, k, True)
        check(z, z, k, False)


def test_few_long_rows_many_segments():
    # A few very long rows are cut into up to 4096 / k segments; the merge
    # pass radix-selects the k winners among nseg * k candidates (> 512) before
    # ranking them.  Ties across segments, NaN, and winners in the last segment.
    rng = np.random.default_rng(32)
    x = rng.standard_normal((2, 3_000_000)).astype(np.float32)
    x[1] = np.round(x[1] * 2) / 2            # heavy ties across every segment
    x[0, -5:] = 50.0                         # top values in the last segment
    x[0, 17] = np.nan
    for k in (5, 64, 128, 1000):
        check(x, x, k, True)
        check(x, x, k, False)
    y = rng.uniform(-1, 1, (8, 1_000_000)).astype(np.float32)
    check(y, y, 50)


@pytest.mark.parametrize("dt", [np.float64, np.int64])
def test_streaming_radix_many_rows_8_byte(dt):
    # >= 2 rows per CU of 8-byte elements: 256-thread streaming radix
    # workgroups; the passes stop early unless the k-th key's class needs the
    # tie order (heavy ties below)
    rng = np.random.default_rng(34)
    if dt == np.float64:
        x = rng.standard_normal((600, 3000))
        x[1::7] = np.round(x[1::7] * 2)
        x[3, ::9] = np.nan
    else:
        x = rng.integers(-(1 << 40), 1 << 40, size=(600, 3000), dtype=np.int64)
        x[1::7] %= 5
    t = torch.from_numpy(x).cuda()
    for k in (1, 50, 700):
        for largest in (True, False):
            print(f"case topk {np.dtype(dt).name} [600, 3000] k={k} largest={largest}", flush=True)
            gv, gi = _capi.topk(t, k, largest)
            torch.cuda.synchronize()
            ev, ei = O.topk_any(x, k, largest)
            np.testing.assert_array_equal(gi.cpu().numpy(), ei)
            np.testing.assert_array_equal(gv.cpu().numpy().view(np.uint8), ev.view(np.uint8))


def test_long_rows_large_k_segments():
    # rows longer than 32768 with k of 129..1024: segments of <= 32768 through
    # the register radix select, winners merged (radix select over the
    # nseg * k composites, then a bitonic sort of the k)
    rng = np.random.default_rng(33)
    x = (rng.standard_normal((5, 151936)) * 3).astype(np.float32)
    x[1] = np.round(x[1])                    # heavy ties across segments
    x[2, ::13] = np.nan
    x[3] = 1.0                               # all equal: the lowest indices
    x[4, -300:] = 40.0                       # winners in the last segment
    for k in (129, 256, 1000, 1024):
        check(x, x, k, True)
        check(x, x, k, False)
    check(x, x[:, 1:100001], 700)            # misaligned rows


def test_wave_kernel_k_129_to_256():
    # k of 129..256 in the wave kernel (512-entry wave lists) on every
    # workgroup shape: 16 waves (few rows), 8 waves (many), 4 waves (rows of
    # 4096..16383), split rows with the merge; ties, NaN, all-equal rows (exact
    # path) and rows whose values rise along the row (repeated compaction)
    rng = np.random.default_rng(36)
    n = 40000
    trend = np.linspace(0, 50, n, dtype=np.float32)
    a = rng.standard_normal((6, n)).astype(np.float32)
    a[1] = np.round(a[1] * 3) / 3
    a[2, ::11] = np.nan
    a[3] = 1.5
    a[4] = trend + rng.standard_normal(n).astype(np.float32)
    for k in (129, 200, 256):
        check(a, a, k, True)
        check(a, a, k, False)
    b = rng.uniform(-1, 1, (1100, 20000)).astype(np.float32)
    check(b, b, 256)
    c = rng.standard_normal((1100, 6000)).astype(np.float32)
    c[::9] = np.round(c[::9] * 2) / 2
    check(c, c, 150, True)
    check(c, c, 150, False)
    d = rng.standard_normal((2, 1_000_000)).astype(np.float32)
    check(d, d, 256)
    check(d, d[:, 1:], 200)                  # misaligned rows: scalar loads


def test_one_to_two_rows_per_cu():
    # between one and two long rows per CU: 16-wave workgroups, two per CU,
    # no prefetch (the default plan there); adversarial rows included
    rng = np.random.default_rng(35)
    x = rng.uniform(-1, 1, (300, 20000)).astype(np.float32)
    x[4] = 0.5                                # all equal: exact path
    x[6] = np.round(x[6] * 3) / 3
    x[8, ::17] = np.nan
    for k in (1, 50, 128):
        check(x, x, k, True)
        check(x, x, k, False)


def test_mid_rows_four_wave_workgroups():
    # >= 4 rows per CU of 4096 .. 16383 elements take 4-wave workgroups of the
    # wave kernel (k <= 128; also k of 65..128 below 8192 elements, which
    # otherwise go to the radix select); adversarial rows take its exact path
    rng = np.random.default_rng(31)
    x = rng.uniform(-1, 1, (1100, 6000)).astype(np.float32)
    x[3] = 2.0                               # all equal: list overflow -> exact path
    x[5] = np.round(x[5] * 3) / 3            # heavy ties
    x[7, ::11] = np.nan
    x[9] = np.where(rng.random(6000) < 0.5, np.float32(0.0), np.float32(-0.0))
    for k in (1, 16, 64, 100, 128):
        check(x, x, k, True)
        check(x, x, k, False)
    y = rng.standard_normal((1024, 12289)).astype(np.float32)
    check(y, y, 50)
    check(y, y[:, 1:12289], 64)              # misaligned rows: scalar loads


@pytest.mark.parametrize("force", [0, 1, 2])
def test_radix_select_large_k(force):
    """Large k: k_topk_rsel (rows of <= 32768 elements held in registers) or,
    with force=2, the streaming k_topk_radix (bitonic sort in LDS up to 4096,
    in the workspace beyond).  force=1 and 2 send small k through them too."""
    _capi.debug_set("topk_radix", force)
    rng = np.random.default_rng(30)
    x = rng.standard_normal((7, 5000)).astype(np.float32)
    x[1] = np.round(x[1] * 2) / 2            # heavy ties
    x[2] = 3.0                                # all equal
    x[3, ::3] = np.nan
    x[4] = np.where(rng.random(5000) < 0.5, -0.0, 0.0)
    for k in (1, 65, 129, 1000, 1025, 4096, 4097, 5000):
        check(x, x, k, True)
        check(x, x, k, False)
    y = rng.uniform(-1, 1, (3, 20000)).astype(np.float32)
    check(y, y, 8193)                         # workspace sort (k > 4096)
    check(y, y[:, 1:], 3000, False)           # misaligned rows


@pytest.mark.parametrize("cols", [700, 1024, 2000, 2048, 4000, 4096, 6000, 8192, 12000, 16384, 20000, 32768])
def test_register_rows_large_k(cols):
    """k_topk_rsel for every workgroup shape (256 threads x 4/8/16 keys, 512 x
    16, 1024 x 16/32) and every sort width (1..32 composites per thread, one
    to 16 waves): random rows, heavy ties (the index-ordered exact path when
    the k-th key's class is larger than the number still wanted), all-equal
    rows, NaN / +-0, rows of a strided view."""
    rng = np.random.default_rng(cols)
    x = rng.standard_normal((5, cols + 3)).astype(np.float32)
    x[1] = np.round(x[1] * 2) / 2
    x[2] = 1.5
    x[3, ::5] = np.nan
    x[4] = np.where(rng.random(cols + 3) < 0.5, -0.0, 0.0)
    v = x[:, 3:]
    ks = {1, 64, 65, 129, 255, 257, 1000, 1025, 2049, 4097, 8193, 16385, cols}
    for k in sorted(k for k in ks if k <= cols):
        check(x, v, k, True)
        if k in (65, 1025, cols):
            check(x, v, k, False)


def test_workspace_sort_paths():
    """k whose pow2 exceeds the LDS sort (the streaming kernel sorts in the
    workspace): 1024-thread workgroups (fewer rows than 2 per CU) with chunks
    of 4096 and 8192 composites in registers and up to three global stages per
    pass; 256-thread workgroups (more rows) with 4096-composite chunks in LDS;
    8-byte dtypes (128-bit composites, 2048-composite LDS chunks).  Ties, equal
    rows, NaN / +-0 and k = cols included."""
    _capi.debug_set("topk_radix", 2)  # every row through the streaming kernel
    rng = np.random.default_rng(36)
    x = rng.standard_normal((6, 70000)).astype(np.float32)
    x[1] = np.round(x[1] * 4) / 4
    x[2] = 0.5
    x[3, ::3] = np.nan
    x[4] = np.where(rng.random(70000) < 0.5, -0.0, 0.0)
    for k in (4097, 8192, 8193, 20000, 65537, 70000):  # pow2: 8192 .. 131072
        check(x, x, k, True)
    check(x, x, 8193, False)
    check(x, x, 70000, False)
    many = rng.standard_normal((600, 9000)).astype(np.float32)  # 256-thread workgroups
    many[::7] = np.round(many[::7])
    check(many, many, 5000, True)
    check(many, many, 9000, False)
    for dt in (np.float64, np.int64, np.uint64):
        if dt == np.float64:
            y = rng.standard_normal((5, 12000))
            y[0, ::5] = np.nan
            y[1] = np.round(y[1])
        else:
            info = np.iinfo(dt)
            y = rng.integers(info.min, info.max, size=(5, 12000), dtype=dt, endpoint=True)
            y[1] = y[1] % 7
        yt = torch.from_numpy(y).cuda()
        for k, largest in ((2049, True), (9000, False), (12000, True)):
            print(f"case topk dtype={np.dtype(dt).name} shape={y.shape} k={k} largest={largest}", flush=True)
            gv, gi = _capi.topk(yt, k, largest)
            torch.cuda.synchronize()
            ev, ei = O.topk_any(y, k, largest)
            np.testing.assert_array_equal(gi.cpu().numpy(), ei)
            np.testing.assert_array_equal(gv.cpu().numpy().view(np.uint8), ev.view(np.uint8))


def test_large_k_configs():
    rng = np.random.default_rng(31)
    x = rng.uniform(-1, 1, (4096, 2048)).astype(np.float32)
    check(x, x, 1000)
    c3 = rng.uniform(-1, 1, (1024, 32768)).astype(np.float32)
    check(c3, c3, 2048)
    check(c3[:256], c3[:256], 4096)


@pytest.mark.parametrize("dt", [np.float64, np.int8, np.int16, np.int32, np.int64, np.uint8, np.uint16,
                                np.uint32, np.uint64, np.bool_])
def test_other_dtypes(dt):
    """tpr_topk on every dtype (the radix-select kernel with the dtype's sortable
    key): values (bit-exact, in the input dtype) and indices against
    oracle.topk_any, with ties, extremes, NaN / +-0 for float64, k up to cols."""
    rng = np.random.default_rng(42)
    rows, cols = 9, 3001
    if dt == np.bool_:
        x = rng.random((rows, cols)) < 0.3
    elif dt == np.float64:
        x = rng.standard_normal((rows, cols))
        x[0, ::7] = np.nan
        x[1] = np.where(rng.random(cols) < 0.5, -0.0, 0.0)
        x[2, :50] = np.inf
        x[3] = np.round(x[3] * 3)
    else:
        info = np.iinfo(dt)
        x = rng.integers(info.min, info.max, size=(rows, cols), dtype=dt, endpoint=True)
        x[0, 100:300] = info.max
        x[1, 100:300] = info.min
        x[2] = x[2] % 5
    t = torch.from_numpy(x).cuda()
    cases = [(t, x, k) for k in (1, 10, 64, 1000, cols)]
    if np.dtype(dt).itemsize <= 4:  # longer rows: 1024-thread workgroups (and the streaming kernel beyond 32768)
        for n in (20000, 40000, 100000):
            y = np.concatenate([x[:3]] * (n // cols + 1), axis=1)[:, :n].copy()
            cases += [(torch.from_numpy(y).cuda(), y, k) for k in ((100, 300, 5000) if n == 100000 else (100, 5000))]
    for t, x, k in cases:
        for largest in (True, False):
            print(f"case topk dtype={np.dtype(dt).name} shape={x.shape} k={k} largest={largest}", flush=True)
            gv, gi = _capi.topk(t, k, largest)
            torch.cuda.synchronize()
            ev, ei = O.topk_any(x, k, largest)
            np.testing.assert_array_equal(gi.cpu().numpy(), ei)
            g = gv.cpu().numpy()
            assert g.dtype == ev.dtype
            np.testing.assert_array_equal(g.view(np.uint8), ev.view(np.uint8))


@pytest.mark.parametrize("dt", [np.int32, np.uint32])
def test_short_rows_32bit_integers(dt):
    """int32 / uint32 rows of <= 4096 through the lane-group kernel: key 0
    (INT_MIN / 0 for largest, INT_MAX / UINT_MAX for smallest) is a real
    element here, so rows with fewer than k other keys take the exact search;
    also all-extreme rows, heavy ties, k = cols and a strided view."""
    rng = np.random.default_rng(77)
    info = np.iinfo(dt)
    cases = []
    for rows, cols, ks in [(37, 5, (1, 5)), (300, 100, (1, 7, 64, 100)), (700, 1000, (8, 33, 64)),
                           (300, 4096, (1, 16, 64)), (2600, 1024, (65, 100, 128)), (2600, 2048, (80, 128))]:
        x = rng.integers(info.min, info.max, size=(rows, cols), dtype=dt, endpoint=True)
        x[0] = info.min
        x[1] = info.max
        x[2] = np.where(rng.random(cols) < 0.9, info.min, x[2])
        x[3] = np.where(rng.random(cols) < 0.9, info.max, x[3])
        x[4] = x[4] % 3
        x[5, : cols // 2] = info.min
        x[5, cols // 2:] = info.max
        cases.append((x, ks))
    for x, ks in cases:
        t = torch.from_numpy(x).cuda()
        for k in ks:
            for largest in (True, False):
                print(f"case topk dtype={np.dtype(dt).name} shape={x.shape} k={k} largest={largest}", flush=True)
                gv, gi = _capi.topk(t, k, largest)
                torch.cuda.synchronize()
                ev, ei = O.topk_any(x, k, largest)
                np.testing.assert_array_equal(gi.cpu().numpy(), ei)
                np.testing.assert_array_equal(gv.cpu().numpy(), ev)
    # strided rows (scalar loads): every other row of a wider buffer
    x = rng.integers(info.min, info.max, size=(64, 3001), dtype=dt, endpoint=True)
    x[::5, ::2] = info.min
    t = torch.from_numpy(x).cuda()[:, :2999]
    for k in (1, 30, 64):
        for largest in (True, False):
            print(f"case topk dtype={np.dtype(dt).name} strided k={k} largest={largest}", flush=True)
            gv, gi = _capi.topk(t, k, largest)
            torch.cuda.synchronize()
            ev, ei = O.topk_any(np.ascontiguousarray(x[:, :2999]), k, largest)
            np.testing.assert_array_equal(gi.cpu().numpy(), ei)
            np.testing.assert_array_equal(gv.cpu().numpy(), ev)


@pytest.mark.parametrize("dt", [np.int32, np.uint32])
@pytest.mark.parametrize("knob", [("topk_short", 0), ("topk_short", -1), ("topk_fallback", 1)])
def test_long_rows_32bit_integers(dt, knob):
    """int32 / uint32 through the wave and workgroup kernels (and the merge of
    split rows): rows where fewer than k elements have a non-zero key take the
    exact select; topk_short = -1 sends short rows to the workgroup kernels,
    topk_fallback = 1 forces the exact select everywhere."""
    _capi.debug_set(*knob)
    rng = np.random.default_rng(78)
    info = np.iinfo(dt)
    shapes = [(600, 1000, (8, 64)), (1100, 8192, (1, 50, 128)), (300, 20000, (16, 100, 256)),
              (5, 70000, (10, 200)), (1100, 5000, (64, 200))]
    for rows, cols, ks in shapes:
        x = rng.integers(info.min, info.max, size=(rows, cols), dtype=dt, endpoint=True)
        x[0] = info.min
        x[1] = info.max
        x[2] = np.where(rng.random(cols) < 0.995, info.min, x[2])
        x[3] = np.where(rng.random(cols) < 0.995, info.max, x[3])
        x[4] = x[4] % 3
        t = torch.from_numpy(x).cuda()
        for k in ks:
            for largest in (True, False):
                print(f"case topk dtype={np.dtype(dt).name} {knob} shape={x.shape} k={k} largest={largest}",
                      flush=True)
                gv, gi = _capi.topk(t, k, largest)
                torch.cuda.synchronize()
                ev, ei = O.topk_any(x, k, largest)
                np.testing.assert_array_equal(gi.cpu().numpy(), ei)
                np.testing.assert_array_equal(gv.cpu().numpy(), ev)


@pytest.mark.parametrize("dt", [np.int8, np.uint8, np.int16, np.uint16, np.bool_])
@pytest.mark.parametrize("short", [0, -1])
def test_small_integer_rows(dt, short):
    """1- and 2-byte elements, ties everywhere (few distinct values).  With
    short=0 aligned rows of <= 4096 elements and k <= 64 take the lane-group
    kernel and the rest the register radix select; with short=-1 (the lane-group
    kernel off) every row takes the radix select: one / two radix passes,
    grouped loads on aligned rows (cols a multiple of 4 or 8 here) and element
    loads on the others."""
    _capi.debug_set("topk_short", short)
    rng = np.random.default_rng(79)
    for rows, cols, ks in [(2000, 1024, (1, 8, 100)), (300, 4096, (16, 64, 1000)), (77, 1003, (5, 50)),
                           (40, 32768, (300,)), (3, 100000, (256,))]:
        if dt == np.bool_:
            x = rng.random((rows, cols)) < 0.1
        else:
            info = np.iinfo(dt)
            x = rng.integers(info.min, info.max, size=(rows, cols), dtype=dt, endpoint=True)
            x[0] = info.min
            x[1] = info.max
        t = torch.from_numpy(x).cuda()
        for k in ks:
            for largest in (True, False):
                print(f"case topk dtype={np.dtype(dt).name} shape={x.shape} k={k} largest={largest}", flush=True)
                gv, gi = _capi.topk(t, k, largest)
                torch.cuda.synchronize()
                ev, ei = O.topk_any(x, k, largest)
                np.testing.assert_array_equal(gi.cpu().numpy(), ei)
                np.testing.assert_array_equal(gv.cpu().numpy().view(np.uint8), ev.view(np.uint8))


@pytest.mark.parametrize("dt", [np.int8, np.uint8, np.int16, np.uint16, np.bool_])
def test_small_integer_short_rows(dt):
    """1- and 2-byte rows of <= 4096 with 16-byte aligned rows through the
    lane-group kernel (16 or 8 elements per lane vector): views of a wider
    buffer give odd column counts (a row's last dword partly past its end),
    k = cols, extreme-value rows (keys of 0) and heavy ties."""
    rng = np.random.default_rng(80)
    for rows, width, cols, ks in [(300, 1024, 1024, (1, 8, 32, 64)), (300, 1024, 1001, (1, 37, 64)),
                                  (97, 16, 5, (1, 5)), (64, 64, 63, (63,)), (200, 4096, 4096, (1, 16, 64)),
                                  (500, 256, 200, (8, 50)), (3000, 2048, 2047, (65, 128))]:
        if dt == np.bool_:
            x = rng.random((rows, width)) < 0.2
        else:
            info = np.iinfo(dt)
            x = rng.integers(info.min, info.max, size=(rows, width), dtype=dt, endpoint=True)
            x[0] = info.min
            x[1] = info.max
            x[2] = np.where(rng.random(width) < 0.95, info.min, x[2])
            x[3] = np.where(rng.random(width) < 0.95, info.max, x[3])
            x[4] = x[4] % 3
        t = torch.from_numpy(x).cuda()[:, :cols]
        xc = np.ascontiguousarray(x[:, :cols])
        for k in ks:
            for largest in (True, False):
                print(f"case topk dtype={np.dtype(dt).name} rows={rows} width={width} cols={cols} k={k} "
                      f"largest={largest}", flush=True)
                gv, gi = _capi.topk(t, k, largest)
                torch.cuda.synchronize()
                ev, ei = O.topk_any(xc, k, largest)
                np.testing.assert_array_equal(gi.cpu().numpy(), ei)
                np.testing.assert_array_equal(gv.cpu().numpy().view(np.uint8), ev.view(np.uint8))


@pytest.mark.parametrize("dt", [np.int8, np.uint8, np.int16, np.uint16, np.bool_])
@pytest.mark.parametrize("fallback", [0, 1])
def test_small_integer_long_rows_wave_kernel(dt, fallback):
    """1- and 2-byte rows longer than the lane-group kernel takes, 16-byte
    aligned, k <= 128: the wave kernel on their integer keys (one or two
    16-byte vectors per lane per slice), with 8 / 16 / 4-wave workgroups, split
    rows merged, heavy ties (few distinct values: most rows take the exact
    path at some point), and the forced exact path (fallback=1)."""
    _capi.debug_set("topk_fallback", fallback)
    rng = np.random.default_rng(97)
    esz = np.dtype(dt).itemsize
    for rows, cols, ks in [(1024, 16384, (64,)), (128, 151936, (50,)), (2048, 12288, (100,)),
                           (16, 500000, (128, 1)), (300, 40000, (33,))]:
        if dt == np.bool_:
            x = rng.random((rows, cols)) < 0.01
        else:
            info = np.iinfo(dt)
            x = rng.integers(info.min, info.max, size=(rows, cols), dtype=dt, endpoint=True)
            x[0] = info.min
            x[1, ::3] = info.max
        t = torch.from_numpy(x).cuda()
        for k in ks:
            kind = _capi.topk_plan(_capi._torch_dtypes()[t.dtype], rows, cols, k)[0]
            assert kind == "wave", (dt, rows, cols, k, kind)
            for largest in (True, False):
                print(f"case topk-wave dtype={np.dtype(dt).name} shape={x.shape} k={k} largest={largest} "
                      f"fallback={fallback}", flush=True)
                gv, gi = _capi.topk(t, k, largest)
                torch.cuda.synchronize()
                ev, ei = O.topk_any(x, k, largest)
                np.testing.assert_array_equal(gi.cpu().numpy(), ei)
                np.testing.assert_array_equal(gv.cpu().numpy().view(np.uint8), ev.view(np.uint8))
        del t
    assert esz in (1, 2)


@pytest.mark.parametrize("dt", [np.float64, np.int64, np.uint64])
@pytest.mark.parametrize("fallback", [0, 1])
def test_eight_byte_rows_wave_kernel(dt, fallback):
    """8-byte rows (16-byte aligned, k <= 128) through the wave kernel: the
    filter on the high 32 bits of each 64-bit key, the ranking with the low
    halves read back; rows it cannot finish are flagged and finished by the
    streaming radix select (forced for every row by fallback=1; taken
    naturally by int64 rows of small values, whose high halves all tie).
    Values and indices bit-exact against the oracle, NaN / +-0 / inf and
    high-half ties included."""
    _capi.debug_set("topk_fallback", fallback)
    rng = np.random.default_rng(98 + fallback)
    for rows, cols, ks in [(256, 151936, (50,)), (1024, 16384, (64, 1)), (2048, 12288, (100,)), (300, 40000, (128,))]:
        if dt == np.float64:
            x = rng.standard_normal((rows, cols)) * 3
            x[0, ::7] = np.nan
            x[1, ::5] = -0.0
            x[1, 1::5] = 0.0
            x[2, :100] = np.inf
            # equal high halves, different low halves (ties of the filter key)
            x[3] = 1.0 + rng.integers(0, 1 << 20, size=cols) * 2.0 ** -52
        elif dt == np.int64:
            x = rng.integers(-(1 << 62), 1 << 62, size=(rows, cols), dtype=np.int64)
            x[0] = rng.integers(-50, 50, size=cols)           # all high halves equal: flagged rows
            x[1, ::3] = np.iinfo(np.int64).min
        else:
            x = rng.integers(0, np.iinfo(np.uint64).max, size=(rows, cols), dtype=np.uint64, endpoint=True)
            x[0] = rng.integers(0, 1000, size=cols).astype(np.uint64)
            x[1, ::4] = np.iinfo(np.uint64).max
        t = torch.from_numpy(x).cuda()
        for k in ks:
            kind = _capi.topk_plan(_capi._torch_dtypes()[t.dtype], rows, cols, k)[0]
            assert kind == "wave8", (dt, rows, cols, k, kind)
            for largest in (True, False):
                print(f"case topk-wave8 dtype={np.dtype(dt).name} shape={x.shape} k={k} largest={largest} "
                      f"fallback={fallback}", flush=True)
                gv, gi = _capi.topk(t, k, largest)
                torch.cuda.synchronize()
                ev, ei = O.topk_any(x, k, largest)
                np.testing.assert_array_equal(gi.cpu().numpy(), ei)
                np.testing.assert_array_equal(gv.cpu().numpy().view(np.uint8), ev.view(np.uint8))
        del t
