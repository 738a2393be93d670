import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# The ctypes binding loads the test build of the launch library (the same
# kernels plus tpr_debug_set, which the forced-plan tests need); the host core
# tensorplay_amd._C links the shipped libtpr_rocm.so either way.
os.environ.setdefault("TPR_ROCM_DEV", "1")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs on the GPU box)")
