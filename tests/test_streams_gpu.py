"""Reductions through the Tensor API on two HIP streams at once.

The caching allocator keeps each freed block on the stream it was allocated on
(csrc/core/CachingAllocatorCore.h): a block freed while stream A may still use
it is never handed to an allocation on stream B.  Here C2-sized reductions
([64, 1024, 1024] fp32) run back to back on two streams,
with outputs and workspaces freed and re-allocated while both streams are
busy, and every result is checked against the oracle (bit-exact for amax /
argmax) or fp64 (mean / var, <= 1e-5 relative).
"""
import numpy as np
import pytest

import tensorplay_amd as tp
from oracle import oracle as O
from tests.gpu_util import assert_bits_equal, assert_close_rel

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture
def streams():
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()  # default priority
    yield s1, s2
    tp.rocm.set_stream(0)
    torch.cuda.synchronize()


def _c2(seed):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((64, 1024, 1024), dtype=np.float32)


def test_two_streams_c2_reductions(streams):
    s1, s2 = streams
    xs = [_c2(31), _c2(32)]
    ts = [tp.from_torch(torch.from_numpy(x).cuda()) for x in xs]
    torch.cuda.synchronize()
    results = [{}, {}]
    for rep in range(2):  # the second round reuses cached blocks on each stream
        for i, s in enumerate((s1, s2)):
            print(f"case streams rep={rep} stream={i}", flush=True)
            tp.rocm.set_stream(s.cuda_stream)
            t = ts[i]
            results[i] = {"mean1": t.mean([1]), "amax0": t.max([0]), "argmax0": t.argmax(0),
                          "var2": t.var([2], 1), "std2": t.std([2], 1)}
    torch.cuda.synchronize()
    for i, x in enumerate(xs):
        r = results[i]
        x64 = x.astype(np.float64)
        assert_close_rel(r["mean1"].numpy(), x64.mean(1))
        assert_bits_equal(r["amax0"].numpy(), O.amax(x, [0]))
        assert_bits_equal(r["argmax0"].numpy(), O.argmax(x, 0))
        v = x64.var(2, ddof=1)
        assert_close_rel(r["var2"].numpy(), v)
        assert_close_rel(r["std2"].numpy(), np.sqrt(v))


def test_block_freed_on_one_stream_is_not_reused_on_another(streams):
    s1, s2 = streams
    x = tp.from_torch(torch.randn((4096, 4096), device="cuda"))
    torch.cuda.synchronize()
    tp.rocm.set_stream(s1.cuda_stream)
    a = x.sum([1])             # output block owned by s1
    pa = a.data_ptr()
    del a                      # freed while s1 may still be writing it
    tp.rocm.set_stream(s2.cuda_stream)
    b = x.sum([1])
    assert b.data_ptr() != pa  # s2 never takes s1's block
    tp.rocm.set_stream(s1.cuda_stream)
    c = x.sum([1])
    assert c.data_ptr() == pa  # s1 reuses its own block in stream order
    torch.cuda.synchronize()
    ref = x.sum([1]).numpy()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(b.numpy(), ref)
    np.testing.assert_array_equal(c.numpy(), ref)


def test_record_stream_defers_reuse(streams):
    s1, s2 = streams
    x = tp.from_torch(torch.randn((2048, 4096), device="cuda"))
    torch.cuda.synchronize()
    tp.rocm.set_stream(s1.cuda_stream)
    y = x.sum([1])             # allocated on s1
    torch.cuda.synchronize()
    tp.rocm.set_stream(s2.cuda_stream)
    z = y.max()                # y read on s2
    y.record_stream(s2.cuda_stream)
    py = y.data_ptr()
    before = tp.rocm.memory_stats()["pending_bytes"]
    del y                      # waits for s2's work before any reuse
    after = tp.rocm.memory_stats()["pending_bytes"]
    assert after > before
    torch.cuda.synchronize()
    tp.rocm.set_stream(s1.cuda_stream)
    w = x.sum([1])             # s2's event has completed: s1 may reuse the block
    assert w.data_ptr() == py
    assert tp.rocm.memory_stats()["pending_bytes"] == before
    torch.cuda.synchronize()
    assert z.item() == w.numpy().max()
