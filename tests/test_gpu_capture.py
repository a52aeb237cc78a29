"""The library's calls are capture-safe once the workspaces are attached: a fresh process makes
its first ffn8 (tiled records), prefill GEMM (split tiles) and Q6_K GEMV calls under stream
capture, and every graph replay equals the eager calls bit for bit (tests/capture_first_calls.py).
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def test_first_calls_under_capture(gpu):
    print("[case] first library calls under stream capture (subprocess)", flush=True)
    r = subprocess.run([sys.executable, "-u", os.path.join(HERE, "capture_first_calls.py")],
                       capture_output=True, text=True, timeout=110)
    print(r.stdout[-4000:], r.stderr[-2000:])
    assert r.returncode == 0 and "[capture] OK" in r.stdout
