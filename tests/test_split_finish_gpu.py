"""Split reductions that finish in their own launch (the last workgroup of an
output combines the partial states, no finalize kernel) against the same plans
with the separate finalize launch (test build knob split_fin = -1): bit-exact,
since both combine the partials in the same fixed order.  Also repeated and
alternating calls (the ticket counters must return to 0 after every launch) and
two streams at once (each stream has its own counters)."""
import numpy as np
import pytest

from tensorplay_amd import _capi

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

OPS_F32 = ["sum", "mean", "amax", "amin", "argmax", "argmin", "var", "std", "prod", "norm", "all", "any"]


@pytest.fixture(autouse=True)
def _reset_knobs():
    yield
    _capi.debug_set("split_fin", 0)
    _capi.debug_set("splits", 0)


def _both(t, op, dims, **kw):
    _capi.debug_set("split_fin", 0)
    a = _capi.reduce(t, op, dims, **kw)
    _capi.debug_set("split_fin", -1)
    b = _capi.reduce(t, op, dims, **kw)
    _capi.debug_set("split_fin", 0)
    torch.cuda.synchronize()
    return a.cpu().numpy(), b.cpu().numpy()


def _eq(a, b, what):
    assert a.shape == b.shape, what
    assert np.array_equal(np.atleast_1d(a).view(np.uint8), np.atleast_1d(b).view(np.uint8)), (what, a, b)


@pytest.mark.parametrize("op", OPS_F32)
@pytest.mark.parametrize("n", [1 << 20, 3_000_017, 1 << 24])
def test_full_reduction_fused_equals_finalize(op, n):
    print(f"case op={op} n={n}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(n % 1000)
    x = torch.randn(n, device="cuda", generator=g) * 2 + 0.5
    if op == "prod":
        x = 1 + x * 1e-7
    a, b = _both(x, op, None)
    _eq(a, b, op)


@pytest.mark.parametrize("dtype", [torch.float64, torch.int32, torch.int8, torch.int64])
@pytest.mark.parametrize("op", ["sum", "amax", "argmin"])
def test_full_reduction_other_dtypes(dtype, op):
    print(f"case dtype={dtype} op={op}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(7)
    if dtype.is_floating_point:
        x = torch.randn(5_000_011, device="cuda", dtype=dtype, generator=g)
    else:
        x = torch.randint(-100, 100, (5_000_011,), device="cuda", dtype=dtype, generator=g)
    a, b = _both(x, op, None)
    _eq(a, b, (dtype, op))


@pytest.mark.parametrize("rows,cols", [(2, 1 << 22), (7, 999_999), (64, 1 << 18)])
@pytest.mark.parametrize("op", ["sum", "argmax", "var"])
def test_few_long_rows(rows, cols, op):
    print(f"case rows={rows} cols={cols} op={op}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows)
    x = torch.randn(rows, cols, device="cuda", generator=g)
    a, b = _both(x, op, [1])
    _eq(a, b, op)


@pytest.mark.parametrize("splits", [2, 3, 64, 1000])
def test_forced_split_counts(splits):
    print(f"case splits={splits}", flush=True)
    x = torch.randn(1 << 22, device="cuda")
    _capi.debug_set("splits", splits)
    for op in ("sum", "argmax", "var"):
        a, b = _both(x, op, None)
        _eq(a, b, (splits, op))


def test_repeated_calls_reset_the_counters():
    """Many split launches in a row on one stream, of different split counts and
    ops: every one must see its counter at 0."""
    xs = [torch.randn(n, device="cuda") for n in (1 << 24, 1 << 20, 5_000_000)]
    exp = [float(x.double().sum()) for x in xs]
    amax = [int(torch.argmax(x)) for x in xs]
    outs = []
    for it in range(40):
        i = it % 3
        outs.append((i, _capi.reduce(xs[i], "sum", None), _capi.reduce(xs[i], "argmax", None)))
    torch.cuda.synchronize()
    for i, s, am in outs:
        assert abs(float(s) - exp[i]) <= 1e-5 * max(1.0, abs(exp[i])) + 1e-3
        assert int(am) == amax[i]


def test_two_streams_at_once():
    """Split reductions on two streams concurrently use separate counters."""
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    xs = [torch.randn(1 << 23, device="cuda") for _ in range(2)]
    torch.cuda.synchronize()
    ref = [int(torch.argmax(x)) for x in xs]
    res = [[], []]
    for _ in range(20):
        for j, s in enumerate((s1, s2)):
            with torch.cuda.stream(s):
                res[j].append(_capi.reduce(xs[j], "argmax", None))
    torch.cuda.synchronize()
    for j in range(2):
        assert all(int(r) == ref[j] for r in res[j])


def test_graph_capture_takes_the_finalize_launch():
    """Under HIP graph capture a split reduction takes the separate finalize
    launch (a captured launch may replay on another stream, so it does not use
    the capturing stream's ticket counters).  The graph is replayed several
    times with eager work between the replays; every replay must equal the
    eager result."""
    x = torch.randn(1 << 22, device="cuda")
    eager = {op: _capi.reduce(x, op, None).clone() for op in ("sum", "argmax", "var")}
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        _capi.reduce(x, "sum", None)  # warm the allocator on the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            outs = {op: _capi.reduce(x, op, None) for op in ("sum", "argmax", "var")}
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(4):
        for o in outs.values():
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for op in outs:
            assert torch.equal(outs[op], eager[op]), (rep, op, outs[op], eager[op])
        # eager split reductions between the replays (they use the ticket counters)
        y = _capi.reduce(x, "sum", None)
        torch.cuda.synchronize()
        assert torch.equal(y, eager["sum"])
