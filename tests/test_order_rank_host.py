"""CPU check of the longest-piece-first rank (``ragged_piece_rank``).

``tests/order_rank_check.cpp`` includes the kernel header, builds as a host
program with hipcc (no GPU needed) and compares every piece's rank with its
position in a brute-force sort over ~300k pieces of random ragged batches.
The GPU side of the same order is checked in ``test_gpu_dispatch_order.py``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    return None


def test_rank_matches_a_sort_of_the_pieces():
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "order_rank_check")
        subprocess.run([hipcc, "-O1", "-std=c++17", "--offload-arch=gfx950",
                        os.path.join(HERE, "order_rank_check.cpp"), "-o", exe],
                       check=True, capture_output=True, timeout=300)
        r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    cases, bad = (int(x) for x in r.stdout.split()[1::2])
    assert cases > 100000 and bad == 0
