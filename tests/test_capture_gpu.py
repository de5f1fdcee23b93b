"""hipgemm_gemm_noalloc under stream capture and its memory footprint, each in
a fresh child process (tests/noalloc_capture_child.py) so that the entry
point's first use on the GPU happens where the test needs it:

* inside a CUDA graph capture: the first noalloc calls of the process are
  captured for shapes whose schedules use its static scratch (the strip
  schedule's K-slices, the 128 x 128 schedule's K-slices), and every replay
  of the graph, and an eager call after them, equals the oracle bit for bit;
* after other GEMMs have run: device memory in use grows by at least the
  scratch array at the first noalloc call that needs it, and not before
  (the array sits in a code object of its own, loaded at that first use).
"""
import os
import subprocess
import sys

import pytest

from util import say

pytestmark = pytest.mark.gpu

CHILD = os.path.join(os.path.dirname(os.path.abspath(__file__)),
                     "noalloc_capture_child.py")


@pytest.mark.parametrize("mode", ["capture", "footprint"])
def test_noalloc_first_use_in_fresh_process(gpu, mode):
    say(f"case noalloc child process: {mode}")
    r = subprocess.run([sys.executable, "-u", CHILD, mode],
                       capture_output=True, text=True, timeout=240)
    for line in (r.stdout + r.stderr).splitlines()[-20:]:
        say("    | " + line)
    assert r.returncode == 0 and r.stdout.strip().endswith("OK")
