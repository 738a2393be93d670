"""Writes reference_known_answers.json: the known answers that TensorPlay's own
reduction tests assert, as data (inputs + expected outputs), one record per
assertion, each citing the test line it comes from.  Nothing here imports or
runs the reference; the values are transcribed from its test files:
  test/test_cuda_reductions.py:19-98, test/test_reduction.py:5-57
"""
import json
import math
import os

CASES = [
    # test_cuda_reductions.py
    dict(src="test/test_cuda_reductions.py:22-24", op="sum", x=[1.0] * 10, shape=[10], dims=None, expect=10.0),
    dict(src="test/test_cuda_reductions.py:27-33", op="sum", x=[1.0] * 12, shape=[3, 4], dims=[0],
         expect=[3.0, 3.0, 3.0, 3.0], expect_shape=[4]),
    dict(src="test/test_cuda_reductions.py:35-37", op="sum", x=[1.0] * 12, shape=[3, 4], dims=[1], keepdim=True,
         expect=[4.0, 4.0, 4.0], expect_shape=[3, 1]),
    dict(src="test/test_cuda_reductions.py:41-43", op="mean", x=[1.0] * 12, shape=[3, 4], dims=None, expect=1.0),
    dict(src="test/test_cuda_reductions.py:45-48", op="mean", x=[2.0] * 12, shape=[3, 4], dims=[0],
         expect=[2.0, 2.0, 2.0, 2.0], expect_shape=[4]),
    dict(src="test/test_cuda_reductions.py:55-56", op="amax", x=[1.0, 2.0, 3.0, 4.0], shape=[2, 2], dims=None, expect=4.0),
    dict(src="test/test_cuda_reductions.py:57", op="amin", x=[1.0, 2.0, 3.0, 4.0], shape=[2, 2], dims=None, expect=1.0),
    dict(src="test/test_cuda_reductions.py:59-63", op="amax", x=[1.0, 2.0, 3.0, 4.0], shape=[2, 2], dims=[0],
         expect=[3.0, 4.0], expect_shape=[2]),
    dict(src="test/test_cuda_reductions.py:79-89", op="var", x=[1.0, 2.0, 3.0, 4.0], shape=[4], dims=None,
         expect=5.0 / 3.0, places=7),
    dict(src="test/test_cuda_reductions.py:90", op="std", x=[1.0, 2.0, 3.0, 4.0], shape=[4], dims=None,
         expect=math.sqrt(5.0 / 3.0), places=7),
    dict(src="test/test_cuda_reductions.py:96", op="argmax", x=[1.0, 5.0, 2.0, 8.0], shape=[4], dims=None, expect=3),
    dict(src="test/test_cuda_reductions.py:97", op="argmin", x=[1.0, 5.0, 2.0, 8.0], shape=[4], dims=None, expect=0),
    # test_reduction.py
    dict(src="test/test_reduction.py:39-40", op="argmax", x=[1.0, 5.0, 2.0, 4.0, 3.0, 6.0], shape=[2, 3], dims=None, expect=5),
    dict(src="test/test_reduction.py:41-42", op="argmin", x=[1.0, 5.0, 2.0, 4.0, 3.0, 6.0], shape=[2, 3], dims=None, expect=0),
    dict(src="test/test_reduction.py:44-48", op="argmax", x=[1.0, 5.0, 2.0, 4.0, 3.0, 6.0], shape=[2, 3], dims=[0],
         expect=[1, 0, 1], expect_shape=[3]),
    dict(src="test/test_reduction.py:50-52", op="argmax", x=[1.0, 5.0, 2.0, 4.0, 3.0, 6.0], shape=[2, 3], dims=[1],
         expect=[1, 2], expect_shape=[2]),
    dict(src="test/test_cuda_reductions.py:66-69", op="prod", x=[1.0, 2.0, 3.0, 4.0], shape=[4], dims=None, expect=24.0),
    dict(src="test/test_cuda_reductions.py:71-75", op="norm", x=[3.0, 4.0], shape=[2], dims=None, expect=5.0),
    dict(src="test/test_reduction.py:5-8", op="prod", x=[1.0, 2.0, 3.0, 4.0], shape=[2, 2], dims=None, expect=24.0),
    dict(src="test/test_reduction.py:11-13", op="prod", x=[1.0, 2.0, 3.0, 4.0], shape=[2, 2], dims=[0],
         expect=[3.0, 8.0], expect_shape=[2]),
    dict(src="test/test_reduction.py:15-17", op="prod", x=[1.0, 2.0, 3.0, 4.0], shape=[2, 2], dims=[1],
         expect=[2.0, 12.0], expect_shape=[2]),
    dict(src="test/test_reduction.py:20-21", op="any", x=[1.0, 0.0, 1.0, 1.0], shape=[2, 2], dims=None, expect=True),
    dict(src="test/test_reduction.py:20-22", op="all", x=[1.0, 0.0, 1.0, 1.0], shape=[2, 2], dims=None, expect=False),
    dict(src="test/test_reduction.py:24-25", op="all", x=[1.0, 1.0], shape=[2], dims=None, expect=True),
    dict(src="test/test_reduction.py:27-28", op="any", x=[0.0, 0.0], shape=[2], dims=None, expect=False),
    dict(src="test/test_reduction.py:31-33", op="all", x=[1.0, 0.0, 1.0, 1.0], shape=[2, 2], dims=[0],
         expect=[True, False], expect_shape=[2]),
    dict(src="test/test_reduction.py:55", op="sum", x=[1.0, 2.0, 3.0, 4.0], shape=[2, 2], dims=None, expect=10.0),
    dict(src="test/test_reduction.py:56", op="mean", x=[1.0, 2.0, 3.0, 4.0], shape=[2, 2], dims=None, expect=2.5),
]

_E = [math.exp(1.0), math.exp(2.0), math.exp(3.0)]
_T = sum(_E)

# Softmax-family known answers (test/test_pointwise.py:154-174): softmax of
# [[1, 2, 3], [1, 2, 3]] along dim 1 is e^i / (e + e^2 + e^3) per row (places=5),
# and every row sums to 1 (places=5).
SOFTMAX_CASES = [
    dict(src="test/test_pointwise.py:155-174", op="softmax", x=[1.0, 2.0, 3.0, 1.0, 2.0, 3.0], shape=[2, 3],
         dim=1, expect=[e / _T for e in _E] * 2, expect_shape=[2, 3], places=5),
    dict(src="test/test_pointwise.py:159-162", op="softmax_rowsum", x=[1.0, 2.0, 3.0, 1.0, 2.0, 3.0], shape=[2, 3],
         dim=1, expect=[1.0, 1.0], expect_shape=[2], places=5),
]

if __name__ == "__main__":
    here = os.path.dirname(os.path.abspath(__file__))
    for name, cases in (("reference_known_answers.json", CASES),
                        ("reference_known_answers_softmax.json", SOFTMAX_CASES)):
        out = os.path.join(here, name)
        with open(out, "w") as f:
            json.dump(cases, f, indent=1)
        print("wrote", out, len(cases), "cases")
