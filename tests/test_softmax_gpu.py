"""GPU parity of tpr_softmax (softmax / log_softmax forward and backward) and
tpr_nll_loss / tpr_nll_loss_backward through the C-ABI.

Tolerances (stated here, asserted below):
  * softmax: |y - y64| <= 1e-5 |y64| per element against fp64; log_softmax:
    <= 1e-5 (|y64| + |log-sum-exp|); NaN / inf positions exact.  The CPU path's
    own error (the oracle restatement of the reference composite) is printed
    beside it.
  * softmax gradients: <= 1e-5 of the magnitudes the formula combines
    ((|g| + sum|g*y|) * y, resp. |g| + exp(y) * sum|g|) against fp64 autograd.
  * nll_loss: per-sample losses and unit-weight totals bit-exact against the
    oracle; weighted totals, mean and sum within 1e-6 relative; the backward
    gradient bit-exact given the same total weight.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tensorplay_amd import _capi
from tests.gpu_util import assert_bits_equal, device_view, softmax_error

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(autouse=True)
def _reset_knobs():
    yield
    for k in ("smx_two_pass", "smx_split", "smx_lanes", "smx_res", "general", "nt", "smx_pieces", "smx_spin",
              "smx_fwd_pieces"):
        _capi.debug_set(k, 0)


def check_fwd(base, v, dim, log):
    print(f"case softmax shape={v.shape} strides={v.strides} dim={dim} log={log}", flush=True)
    t = device_view(torch, base, v)
    got = _capi.softmax(t, dim, log=log)
    torch.cuda.synchronize()
    r = softmax_error(got.cpu().numpy(), v.astype(np.float64), dim, log)
    assert r <= 1.0, f"error {r:.2f}x the tolerance"
    return r


ROW_NS = [1, 3, 17, 64, 100, 256, 1000, 1001, 1024, 4096, 5000, 16383, 16384, 32768, 32772, 40000, 70001]


# (two_pass, split, lanes): automatic; every row through the two-pass kernel with
# one workgroup per row; through the split (row, chunk) kernels; 512-lane rows
PLANS = [(0, 0, 0), (1, -1, 0), (1, 1, 0), (0, 0, 512)]


def set_plan(plan):
    _capi.debug_set("smx_two_pass", plan[0])
    _capi.debug_set("smx_split", plan[1])
    _capi.debug_set("smx_lanes", plan[2])


@pytest.mark.parametrize("log", [False, True])
@pytest.mark.parametrize("plan", PLANS)
def test_rows_every_variant(log, plan):
    set_plan(plan)
    rng = np.random.default_rng(11)
    for n in ROW_NS:
        rows = 5 if n > 4096 else 37
        x = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
        check_fwd(x, x, 1, log)


@pytest.mark.parametrize("log", [False, True])
@pytest.mark.parametrize("spin", [0, -1])
def test_rows_by_pieces(log, spin):
    """Forward softmax / log_softmax by row pieces (x held by 1..16 workgroups
    per row, (max, sum exp) exchanged, spin=0; or every piece recomputing the
    others from memory, spin=-1), forced onto every row the pieces can hold:
    ragged last pieces, rows of NaN / -inf / +inf, more rows than CUs."""
    _capi.debug_set("smx_fwd_pieces", 1)
    _capi.debug_set("smx_spin", spin)
    rng = np.random.default_rng(33)
    for rows, n in [(3, 16388), (2, 40964), (3, 41000), (2, 81924), (3, 151936), (2, 327680), (300, 20000)]:
        x = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
        if rows <= 3:
            x[0, n // 3] = np.nan            # a NaN row
            x[1, :] = -np.inf                # no value above -inf: NaN
            x[1, n - 1] = np.nan if n % 2 else -np.inf
            x[-1, 7] = np.inf
        check_fwd(x, x, 1, log)


@pytest.mark.parametrize("log", [False, True])
def test_long_rows_planned(log):
    """Rows longer than one CU holds (153601..655360 floats) take the row
    pieces on the default plan, any row count; longer rows keep the two-pass
    kernels.  NaN / -inf rows, ragged last pieces."""
    rng = np.random.default_rng(36)
    for rows, n in [(3, 153604), (2, 200000), (2, 500001), (2, 655360), (2, 700000)]:
        x = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
        x[0, n // 5] = np.nan
        x[1, :] = -np.inf
        x[1, 3] = 1.0
        check_fwd(x, x, 1, log)


def test_rows_by_pieces_exchange_equals_recompute():
    """The exchanged and the recomputed (max, sum exp) pairs are the same bits,
    so the output does not depend on whether the pieces met; and the planned
    route (more rows than CUs, two pieces or more per row) runs the pieces."""
    rng = np.random.default_rng(34)
    x = torch.from_numpy((rng.standard_normal((600, 65536)) * 3).astype(np.float32)).cuda()
    for log in (False, True):
        a = _capi.softmax(x, -1, log=log)
        _capi.debug_set("smx_spin", -1)
        b = _capi.softmax(x, -1, log=log)
        _capi.debug_set("smx_spin", 0)
        _capi.debug_set("smx_fwd_pieces", -1)
        c = _capi.softmax(x, -1, log=log)  # the one-row-per-CU kernel
        _capi.debug_set("smx_fwd_pieces", 0)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
        r = softmax_error(a[:6].cpu().numpy(), x[:6].double().cpu().numpy(), 1, log)
        assert r <= 1.0
        assert softmax_error(c[:6].cpu().numpy(), x[:6].double().cpu().numpy(), 1, log) <= 1.0


@pytest.mark.parametrize("log", [False, True])
def test_rows_misaligned_and_strided(log):
    rng = np.random.default_rng(12)
    b = rng.standard_normal((40, 1030)).astype(np.float32)
    check_fwd(b, b[1:, 1:], 1, log)      # rows not 16-byte aligned -> scalar loads
    check_fwd(b, b[:, 2:1026], 1, log)   # aligned start, row stride 1030 (not a multiple of 4)
    check_fwd(b, b[::3, :1024], 1, log)  # stepped rows
    check_fwd(b, b[:, ::2], 1, log)      # stepped softmax dim -> strided kernel
    check_fwd(b, b.T, 1, log)            # transposed: the dim is the outer stride-1 one
    check_fwd(b, b, 0, log)              # dim 0 of a row-major matrix


@pytest.mark.parametrize("log", [False, True])
def test_strided_dims(log):
    rng = np.random.default_rng(13)
    for shape, dim in [((4, 300, 33), 1), ((8, 512, 96), 1), ((300, 70), 0), ((2, 3, 4, 5), 2), ((7, 1, 9), 1),
                       ((3, 5, 2), 0), ((1, 2000, 64), 1), ((2, 300, 128), 1), ((3, 64, 20), 1), ((5, 7, 36), 1),
                       ((130, 1000), 0)]:
        x = (rng.standard_normal(shape) * 2).astype(np.float32)
        check_fwd(x, x, dim, log)
    b = (rng.standard_normal((3, 200, 68)) * 2).astype(np.float32)
    check_fwd(b, b[:, :, 4:], 1, log)    # inner 64 from a 16-byte aligned offset: float4 columns
    check_fwd(b, b[:, :, 1:65], 1, log)  # misaligned start: scalar columns
    _capi.debug_set("general", 1)        # the scalar strided kernel on a contiguous last dim too,
    x = rng.standard_normal((9, 700)).astype(np.float32)
    check_fwd(x, x, 1, log)
    x = (rng.standard_normal((8, 512, 96)) * 2).astype(np.float32)
    check_fwd(x, x, 1, log)              # and on a float4-eligible strided dim


@pytest.mark.parametrize("log", [False, True])
@pytest.mark.parametrize("res", [0, -1])
def test_strided_dim_held_in_registers(log, res):
    # float4 column slices of 65..1024 rows stay in registers (res=0: 64-column
    # groups, 8 or 16 waves, 4/8/16 rows per lane; res=-1: the two-pass column
    # kernel), at the edges of each variant, with ragged column groups and
    # NaN / inf columns.
    _capi.debug_set("smx_res", res)
    rng = np.random.default_rng(17)
    inf, nan = np.inf, np.nan
    for n in (65, 128, 129, 256, 257, 512, 513, 1000, 1024, 1025):
        for inner in (64, 200, 264):
            x = (rng.standard_normal((3, n, inner)) * 2).astype(np.float32)
            x[0, n // 2, 1] = nan
            x[1, :, 2] = -inf
            x[2, n - 1, 3] = inf
            x[2, : n - 1, 5] = -inf
            check_fwd(x, x, 1, log)


@pytest.mark.parametrize("log", [False, True])
@pytest.mark.parametrize("spin", [0, -1])
def test_strided_dim_row_pieces(log, spin):
    """Forward strided slices of 513..1024 rows by two row pieces per 64-column
    group (per-column (max, sum exp) exchanged, spin=0; or each piece
    recomputing the other's from memory, spin=-1): ragged column groups, a
    short second piece, NaN / -inf / +inf columns, and the pieces' results
    equal bit for bit whether they met or not."""
    _capi.debug_set("smx_spin", spin)
    rng = np.random.default_rng(35)
    for n in (513, 600, 1000, 1024):
        for inner in (64, 200, 264):
            x = (rng.standard_normal((3, n, inner)) * 2).astype(np.float32)
            x[0, n // 2, 1] = np.nan
            x[0, 3, 9] = np.nan
            x[1, :, 2] = -np.inf
            x[1, : n - 1, 6] = -np.inf
            x[2, n - 1, 3] = np.inf
            x[2, : n - 1, 5] = -np.inf
            check_fwd(x, x, 1, log)
    x = torch.from_numpy((rng.standard_normal((16, 1024, 1024)) * 2).astype(np.float32)).cuda()
    _capi.debug_set("smx_spin", 0)
    a = _capi.softmax(x, 1, log=log)
    _capi.debug_set("smx_spin", -1)
    b = _capi.softmax(x, 1, log=log)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


@pytest.mark.parametrize("log", [False, True])
def test_nontemporal_variants(log):
    """The kernels' nontemporal instantiations (chosen from 256 MiB of traffic;
    the nt knob forces them here on small shapes): rows through every plan,
    strided slices held in registers, and the gradients over rows."""
    _capi.debug_set("nt", 1)
    rng = np.random.default_rng(19)
    for plan in PLANS:
        set_plan(plan)
        for n in (100, 1024, 5000, 40000):
            x = (rng.standard_normal((4, n)) * 3).astype(np.float32)
            check_fwd(x, x, 1, log)
    set_plan((0, 0, 0))
    for n in (65, 256, 1000):
        x = (rng.standard_normal((2, n, 200)) * 2).astype(np.float32)
        x[0, n // 2, 1] = np.nan
        check_fwd(x, x, 1, log)
    for plan in PLANS[:3]:
        set_plan(plan)
        for i, n in enumerate([64, 4096, 20000]):
            check_bwd((4, n), 1, log, 500 + i)


@pytest.mark.parametrize("log", [False, True])
@pytest.mark.parametrize("plan", PLANS[:3])
def test_nan_inf_slices(log, plan):
    set_plan(plan)
    inf, nan = np.inf, np.nan
    rng = np.random.default_rng(14)
    for n in (8, 1000, 3001, 20000):
        x = rng.standard_normal((7, n)).astype(np.float32)
        x[0, n // 2] = nan
        x[1, :] = -inf
        x[2, :] = -inf
        x[2, 1::2] = nan
        x[3, n - 1] = inf
        x[4, : n // 2] = -inf        # leading -inf then finite values
        x[5, :] = 0.0
        x[6, 0] = 80.0               # one dominant value
        check_fwd(x, x, 1, log)
        check_fwd(x, x.T, 0, log)    # the same slices through the strided kernel (scalar columns)
        y = np.ascontiguousarray(x.T)
        check_fwd(y, y, 0, log)      # ... and float4 columns when n % 4 == 0


@pytest.mark.parametrize("log", [False, True])
@pytest.mark.parametrize("res", [0, -1])
def test_rows_held_in_registers_and_lds(log, res):
    # rows of 16384..153600 floats (vocabulary-sized): one 512-thread workgroup
    # per row keeps 8, 24, 40 or 56 float4 per lane in registers and the rest
    # in LDS (res=0), at the edges of each kernel's range; res=-1 sends the
    # same rows through the two-pass kernel.
    _capi.debug_set("smx_split", -1)
    _capi.debug_set("smx_res", res)
    inf, nan = np.inf, np.nan
    rng = np.random.default_rng(16)
    for n in (16384, 20000, 32768, 32772, 40000, 49152, 50260, 55296, 65536, 81920, 88064, 100000, 114688, 114692,
              128256, 131072, 151936, 153596, 153600):
        x = (rng.standard_normal((9, n)) * 3).astype(np.float32)
        x[0, n - 1] = nan            # NaN in the LDS part
        x[1, 5] = nan                # NaN in the register part
        x[2, :] = -inf
        x[3, n - 1] = inf            # +inf in the last vector
        x[4, : n - 7] = -inf         # only the tail is finite
        x[5, n // 5] = 90.0          # dominant value in the register part
        x[6, n - 3] = 90.0           # dominant value in the LDS part
        check_fwd(x, x, 1, log)
    # a row longer than the resident capacity goes to the two-pass kernel
    x = rng.standard_normal((3, 153604)).astype(np.float32)
    check_fwd(x, x, 1, log)
    # rows that are a window of wider rows (row stride 20004 > n = 20000)
    w = (rng.standard_normal((4, 20004)) * 3).astype(np.float32)
    check_fwd(w, w[:, :20000], 1, log)


@pytest.mark.parametrize("log", [False, True])
def test_float64_inputs(log):
    # float64 softmax / log_softmax and their gradients (the reference composite
    # keeps the input dtype): rows and strided dims, NaN / inf slices, against
    # numpy / torch in float64 within 1e-12 relative
    rng = np.random.default_rng(21)
    # strided dims: a workgroup per slice when there are few slices ([200000, 2] over dim 0), a thread per slice
    # otherwise ([300, 20000] over dim 0)
    for shape, dim in [((7, 1000), 1), ((3, 40000), 1), ((4, 300, 33), 1), ((300, 70), 0), ((5, 3, 8), 2),
                       ((200000, 2), 0), ((3000, 64), 0), ((300, 20000), 0), ((100, 5), 0)]:
        x = rng.standard_normal(shape) * 3
        if x.ndim == 2 and dim == 1:
            x[0, 5] = np.nan
            x[1, :] = -np.inf
            x[2, 3] = np.inf
        t = torch.from_numpy(x).cuda()
        print(f"case softmax f64 shape={shape} dim={dim} log={log}", flush=True)
        got = _capi.softmax(t, dim, log=log).cpu().numpy()
        ref = (torch.log_softmax if log else torch.softmax)(torch.from_numpy(x), dim).numpy()
        np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
        ok = np.isfinite(ref)
        np.testing.assert_allclose(got[ok], ref[ok], rtol=1e-12, atol=1e-300 if not log else 1e-12)
        # gradient against torch autograd in float64
        xf = np.where(np.isfinite(x), x, 0.0)
        tx = torch.from_numpy(xf).requires_grad_(True)
        ty = (torch.log_softmax if log else torch.softmax)(tx, dim)
        g = rng.standard_normal(shape)
        ty.backward(torch.from_numpy(g))
        y = ty.detach()
        gi = _capi.softmax(torch.from_numpy(g).cuda(), dim, log=log, grad_of=y.cuda()).cpu().numpy()
        np.testing.assert_allclose(gi, tx.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_large_logits_c5_shape():
    # BASELINE configs[4]-shaped logits: [256, 151936] ~ N(0, 3) + 8 boosted positions per row
    rng = np.random.default_rng(15)
    x = (rng.standard_normal((256, 151936)) * 3).astype(np.float32)
    for r in range(256):
        x[r, rng.choice(151936, 8, replace=False)] += 15.0
    t = torch.from_numpy(x).cuda()
    for log, split in ((False, 0), (True, 0), (False, -1)):
        _capi.debug_set("smx_split", split)
        got = _capi.softmax(t, -1, log=log).cpu().numpy()
        r = softmax_error(got[:32], x[:32].astype(np.float64), 1, log)
        assert r <= 1.0
        # size-independent property on every row: softmax rows sum to 1
        if not log:
            s = got.astype(np.float64).sum(1)
            assert np.all(np.abs(s - 1.0) <= 1e-4)


def test_cpu_path_error_is_reported():
    # The reference composite's own error on the same input (fp32 sequential sum)
    rng = np.random.default_rng(16)
    x = (rng.standard_normal((64, 4096)) * 3).astype(np.float32)
    t = torch.from_numpy(x).cuda()
    for log in (False, True):
        g = softmax_error(_capi.softmax(t, 1, log=log).cpu().numpy(), x.astype(np.float64), 1, log)
        c = softmax_error(O.softmax(x, 1, log=log), x.astype(np.float64), 1, log)
        print(f"softmax log={log}: GPU error {g:.3f}x tolerance, CPU path {c:.3f}x")
        assert g <= 1.0


def test_empty_and_scalar():
    for shape, dim in [((0, 5), 1), ((5, 0), 1), ((3, 0, 4), 0)]:
        t = torch.empty(shape, dtype=torch.float32, device="cuda")
        assert tuple(_capi.softmax(t, dim).shape) == shape
    t = torch.tensor(2.5, device="cuda")
    assert float(_capi.softmax(t, 0).cpu()) == 1.0
    assert float(_capi.softmax(t, 0, log=True).cpu()) == 0.0


# ---- backward -------------------------------------------------------------------------------
def check_bwd(shape, dim, log, seed, view=None):
    rng = np.random.default_rng(seed)
    x64 = rng.standard_normal(shape) * 2
    g64 = rng.standard_normal(shape)
    tx = torch.from_numpy(x64).requires_grad_(True)
    ty = torch.log_softmax(tx, dim) if log else torch.softmax(tx, dim)
    ty.backward(torch.from_numpy(g64))
    ref = tx.grad.numpy()
    y = ty.detach().numpy().astype(np.float32)
    g = g64.astype(np.float32)
    print(f"case softmax_bwd shape={shape} dim={dim} log={log}", flush=True)
    tg, tyy = torch.from_numpy(g).cuda(), torch.from_numpy(y).cuda()
    if view == "T":
        tg, tyy = tg.t().contiguous().t(), tyy.t().contiguous().t()  # same values, column-major storage
    got = _capi.softmax(tg, dim, log=log, grad_of=tyy).cpu().numpy().astype(np.float64)
    y64, gg = y.astype(np.float64), g.astype(np.float64)
    if log:
        tol = 1e-5 * (np.abs(gg) + np.exp(y64) * np.abs(gg).sum(dim, keepdims=True))
    else:
        tol = 1e-5 * (np.abs(gg) + np.abs(gg * y64).sum(dim, keepdims=True)) * np.abs(y64) + 1e-30
    assert np.all(np.abs(got - ref) <= tol)
    # against the oracle's restatement of the autograd composite, same tolerance
    assert np.all(np.abs(got - O.softmax_backward(g, y, dim, log=log)) <= 2 * tol)


@pytest.mark.parametrize("log", [False, True])
@pytest.mark.parametrize("plan", PLANS[:3])
def test_backward_rows(log, plan):
    set_plan(plan)
    for i, n in enumerate([3, 64, 1000, 1001, 4096, 16384, 20000]):
        check_bwd((6, n), 1, log, 100 + i)


@pytest.mark.parametrize("log", [False, True])
@pytest.mark.parametrize("res", [0, -1])
@pytest.mark.parametrize("pieces", [0, -1])
def test_backward_long_rows(log, res, pieces):
    # softmax / log_softmax gradients over rows of 16384..153600: by row
    # pieces holding g and y (pieces=0), else g held in registers + LDS
    # while y streams (res=0; once for log_softmax, twice for softmax), or the
    # two-pass kernel (res=-1)
    _capi.debug_set("smx_split", -1)
    _capi.debug_set("smx_res", res)
    _capi.debug_set("smx_pieces", pieces)
    for i, n in enumerate([16384, 20000, 32772, 49152, 49156, 50260, 114688, 151936, 153600]):
        check_bwd((3, n), 1, log, 400 + i)


@pytest.mark.parametrize("log", [False, True])
@pytest.mark.parametrize("spin", [0, -1])
def test_backward_row_pieces(spin, log):
    """Softmax / log_softmax gradients by row pieces (g and y held, partial
    sums (g . y, or sum g) exchanged
    between the pieces' workgroups), with the exchange (spin=0) and with every
    piece recomputing the others' partials from memory (spin=-1, the path a
    piece takes when a partner is not resident in time): rows of 1..8 pieces,
    ragged last pieces, more rows than CUs."""
    _capi.debug_set("smx_spin", spin)
    for i, (rows, n) in enumerate([(3, 49152), (2, 49156), (5, 98308), (3, 151936), (2, 200000), (2, 393216),
                                   (300, 20000)]):
        check_bwd((rows, n), 1, log, 600 + i)


def test_backward_row_pieces_exchange_equals_recompute():
    """The exchanged partial dots and the recomputed ones are the same bits, so
    the gradient does not depend on whether the pieces met: C5-shaped rows."""
    rng = np.random.default_rng(31)
    g = torch.from_numpy(rng.standard_normal((256, 151936)).astype(np.float32)).cuda()
    y = torch.softmax(torch.from_numpy((rng.standard_normal((256, 151936)) * 3).astype(np.float32)), -1).cuda()
    a = _capi.softmax(g, -1, grad_of=y)
    _capi.debug_set("smx_spin", -1)
    b = _capi.softmax(g, -1, grad_of=y)
    _capi.debug_set("smx_spin", 0)
    c = _capi.softmax(g, -1, grad_of=y)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    assert torch.equal(a.view(torch.int32), c.view(torch.int32))
    # against fp64 on a sample of rows
    g64, y64 = g[:8].double().cpu().numpy(), y[:8].double().cpu().numpy()
    ref = (g64 - (g64 * y64).sum(1, keepdims=True)) * y64
    tol = 1e-5 * (np.abs(g64) + np.abs(g64 * y64).sum(1, keepdims=True)) * np.abs(y64) + 1e-30
    assert np.all(np.abs(a[:8].double().cpu().numpy() - ref) <= tol)
    # log_softmax gradient: the exchanged and recomputed sums of g agree too
    yl = torch.log_softmax(torch.from_numpy((rng.standard_normal((256, 151936)) * 3).astype(np.float32)), -1).cuda()
    a = _capi.softmax(g, -1, log=True, grad_of=yl)
    _capi.debug_set("smx_spin", -1)
    b = _capi.softmax(g, -1, log=True, grad_of=yl)
    _capi.debug_set("smx_spin", 0)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


@pytest.mark.parametrize("log", [False, True])
def test_backward_strided(log):
    check_bwd((4, 300, 33), 1, log, 200)
    check_bwd((4, 300, 64), 1, log, 203)
    check_bwd((3, 50, 20), 1, log, 204)
    check_bwd((300, 70), 0, log, 201)
    check_bwd((50, 80), 1, log, 202, view="T")
    check_bwd((2, 129, 68), 1, log, 205)   # column slices held in registers
    check_bwd((2, 256, 64), 1, log, 206)
    check_bwd((2, 200, 300), 1, log, 208)  # 32-column groups
    check_bwd((2, 257, 64), 1, log, 207)   # two-pass column kernel


# ---- nll_loss ------------------------------------------------------------------------------
def nll_case(N, C, reduction, weighted, seed, x_step=1, t_step=1, ignore=-100):
    rng = np.random.default_rng(seed)
    xb = rng.standard_normal((N, C * x_step)).astype(np.float32)
    x = xb[:, ::x_step]
    tb = rng.integers(0, C, N * t_step).astype(np.int64)
    if N > 4:
        tb[::7] = ignore
    t = tb[::t_step]
    w = rng.uniform(0.1, 2.0, C).astype(np.float32) if weighted else None
    print(f"case nll N={N} C={C} reduction={reduction} weighted={weighted} steps={x_step},{t_step}", flush=True)
    tx = device_view(torch, xb, x)
    tt = torch.from_numpy(tb).cuda()[::t_step]
    tw_ = None if w is None else torch.from_numpy(w).cuda()
    out, tw, status = _capi.nll_loss(tx, tt, tw_, reduction, ignore)
    torch.cuda.synchronize()
    assert int(status.cpu()) == 0
    eo, etw = O.nll_loss(np.ascontiguousarray(x), t, w, reduction, ignore)
    got_tw = tw.cpu().numpy()
    keep = (t != ignore)
    wt = np.ones(C, np.float32) if w is None else w
    losses = np.zeros(N, np.float32)
    losses[keep] = -x[keep, t[keep]] * wt[t[keep]]     # float32, as the reference
    tw64 = wt[t[keep]].astype(np.float64).sum()
    if weighted:
        # fp64 accumulation of the weights; the reference's fp32 running sum is printed beside it
        assert abs(float(got_tw[0]) - tw64) <= 1e-6 * tw64
        print(f"  total_weight rel. error: GPU {abs(float(got_tw[0]) - tw64) / tw64:.2e}, "
              f"CPU path {abs(float(etw[0]) - tw64) / tw64:.2e}")
    else:
        assert_bits_equal(got_tw, etw)
    if reduction == 0:
        assert_bits_equal(out.cpu().numpy(), eo)
    else:
        ref = losses.astype(np.float64).sum()
        if reduction == 1 and tw64 > 0:
            ref /= tw64
        assert abs(float(out.cpu()) - ref) <= 1e-6 * abs(ref)
        if not weighted:
            assert abs(float(out.cpu()) - float(eo)) <= 1e-6 * abs(float(eo))
    # backward: same total weight on both sides -> bit-exact
    g = rng.standard_normal(N if reduction == 0 else ()).astype(np.float32)
    gi = _capi.nll_loss_backward(torch.from_numpy(g).cuda(), tt, N, C, tw_, reduction, ignore, tw)
    egi = O.nll_loss_backward(g, t, C, w, reduction, ignore, got_tw)
    assert_bits_equal(gi.cpu().numpy(), egi)


@pytest.mark.parametrize("reduction", [0, 1, 2])
@pytest.mark.parametrize("weighted", [False, True])
def test_nll_loss_shapes(reduction, weighted):
    for i, (N, C) in enumerate([(1, 1), (37, 10), (5000, 3), (300000, 5), (64, 1000), (16, 1024), (8, 4097),
                                (4, 151936)]):
        nll_case(N, C, reduction, weighted, 300 + i)


def test_nll_loss_strided_and_ignore_index():
    nll_case(100, 33, 1, True, 400, x_step=3, t_step=2)
    nll_case(100, 2048, 0, False, 401, x_step=2)
    nll_case(50, 9, 2, False, 402, ignore=4)      # ignore_index inside [0, C)


def test_nll_loss_status_flag():
    x = torch.zeros((3, 4), device="cuda")
    for bad in (4, -1):
        t = torch.tensor([0, bad, 2], dtype=torch.int64, device="cuda")
        _, _, status = _capi.nll_loss(x, t, None, 1, -100)
        assert int(status.cpu()) == 1
    t = torch.tensor([0, -100, 2], dtype=torch.int64, device="cuda")
    _, tw, status = _capi.nll_loss(x, t, None, 1, -100)
    assert int(status.cpu()) == 0 and float(tw.cpu()) == 2.0


def test_nll_loss_empty_batch():
    x = torch.zeros((0, 4), device="cuda")
    t = torch.zeros((0,), dtype=torch.int64, device="cuda")
    out, tw, status = _capi.nll_loss(x, t, None, 1, -100)
    assert float(out.cpu()) == 0.0 and float(tw.cpu()) == 0.0 and int(status.cpu()) == 0
