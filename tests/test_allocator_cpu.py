"""The caching allocator's stream rules (csrc/core/CachingAllocatorCore.h),
checked on the CPU with mock streams and events: a block freed on stream A is
never handed to a request on stream B, and a block recorded on another stream
is not reused until that stream's event completes.  The test program is
compiled from tests/native/alloc_mock_test.cpp with g++ and run."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CORE = os.path.join(os.path.dirname(HERE), "tensorplay_amd", "csrc", "core")


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not installed")
def test_stream_rules_with_mock_events(tmp_path):
    exe = str(tmp_path / "alloc_mock_test")
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-fsanitize=address,undefined", "-I", CORE,
                    os.path.join(HERE, "native", "alloc_mock_test.cpp"), "-o", exe, "-lpthread"], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and "OK" in r.stdout
