"""CPU checks of bench.py's contract pieces that need no GPU.

- More than one GPU is refused with a message and a non-zero exit status,
  before anything touches a device.
- Every committed traffic summary the benchmark legs read parses to a byte
  count. The count lies between the leg's unique algorithmic bytes and
  4x them: the kernel-trace summaries document those bytes, and gathered rows
  that miss L2 add to the fetches.
"""
from __future__ import annotations

import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402

# traffic summary -> the leg's unique algorithmic bytes per launch
LEGS = {
    "dsa_mla_fwd_fp8_c3_traffic.txt": 417_464_320,
    "dsa_mla_fwd_mxfp8_mx_traffic.txt": 228_196_352,
    "dsa_mla_fwd_bf16_c5_traffic.txt": 2_362_441_728,
    "dsa_mla_fwd_v4_traffic.txt": None,
    "dsa_mla_fwd_v4fp8_traffic.txt": None,
    "dsa_topk_traffic.txt": 69_205_504,
}


def test_multi_gpu_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


@pytest.mark.parametrize("name", sorted(LEGS))
def test_profiled_traffic_parses(name):
    t = bench.profiled_traffic(name)
    assert isinstance(t, int) and t > 0, name
    # the summary's own FETCH / WRITE lines add up to the recorded total
    text = open(os.path.join(ROOT, "profiles", name)).read()
    parts = [int(m.replace(",", "")) for m in re.findall(r"= ([\d,]+) B", text)]
    assert len(parts) == 2 and abs(sum(parts) - t) <= 2, (name, parts, t)
    alg = LEGS[name]
    if alg is not None:
        assert alg <= t <= 4 * alg, (name, t, alg)
