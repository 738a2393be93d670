"""tpr_reduce_noalloc (fixed per-device scratch instead of a workspace) against
tpr_reduce on the same inputs: bit-identical outputs, on two calls in a row
where the second input is smaller, for plans that use the scratch (split rows,
split columns, chunk partials are not needed at these sizes) and for the median
histograms."""
import numpy as np
import pytest

from tensorplay_amd import _capi

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

CASES = [
    # (op, shape of the first call, shape of the second call, dims)
    ("sum", (1 << 24,), (1 << 20,), None),            # full: split row + finalize
    ("argmax", (1 << 24,), (3 << 18,), None),
    ("var", (1 << 24,), (1 << 20,), None),
    ("amax", (4, 1 << 21), (2, 1 << 19), [1]),        # few long rows: splits
    ("mean", (2, 8192, 64), (2, 4096, 64), [1]),      # columns with a split reduced dim
    ("argmin", (1, 65536, 32), (1, 16384, 32), [1]),
    ("median", (1 << 22,), (1 << 18,), None),         # radix-select histograms
    ("sum", (4096, 4096), (512, 4096), [1]),           # no scratch needed
]


def _workspace_bytes(x, op, dims):
    import ctypes
    nd = x.dim()
    rd = list(range(nd)) if dims is None else sorted(d % nd for d in dims)
    desc = _capi.make_desc(op, list(x.shape), list(x.stride()), rd, _capi.default_out_dtype(op))
    return _capi.lib().tpr_reduce_workspace_bytes(ctypes.byref(desc))


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-{c[1]}" for c in CASES])
def test_noalloc_matches_tpr_reduce(case):
    op, s1, s2, dims = case
    g = torch.Generator(device="cuda")
    g.manual_seed(77)
    for j, shape in enumerate((s1, s2)):
        print(f"case noalloc op={op} shape={shape} dims={dims}", flush=True)
        x = torch.randn(shape, generator=g, device="cuda")
        if j == 0 and op != "sum" or shape == (1 << 24,):
            need = _workspace_bytes(x, op, dims)
            assert 0 < need <= _capi.REDUCE_SCRATCH_BYTES, need  # the plan really uses the scratch
        if op == "argmax":
            x.view(-1)[x.numel() // 3] = 50.0
            x.view(-1)[x.numel() - 1] = 50.0   # tie: the lower index wins
        ref = _capi.reduce(x, op, dims)
        got = _capi.reduce_noalloc(x, op, dims)
        torch.cuda.synchronize()
        a, b = ref.cpu().numpy().reshape(-1), got.cpu().numpy().reshape(-1)
        assert a.shape == b.shape
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), (op, shape)


def test_noalloc_out_of_capacity_is_reported():
    x = torch.zeros((1,), device="cuda")
    n = (1 << 31) + 5
    d = _capi.make_desc("var", [1 << 20, n], [n, 1], [1], _capi.FLOAT32)
    import ctypes
    L = _capi.lib()
    assert L.tpr_reduce_noalloc(ctypes.byref(d), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                None) == _capi.ERR_WORKSPACE
