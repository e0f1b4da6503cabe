"""The issue probe (libdsa_issue_probe.so, bench.py --issue-probe): argument checks on the
CPU, and on the GPU that every mode launches and writes its results (the probe measures;
it asserts no hardware rate)."""
from __future__ import annotations

import ctypes
import os

import pytest

from opfoundry_amd.abi import bind_torch_hip_runtime
from opfoundry_amd.build import ISSUE_PROBE_LIB_PATH


def probe():
    if not os.path.exists(ISSUE_PROBE_LIB_PATH):
        pytest.fail(f"{ISSUE_PROBE_LIB_PATH} not built (python -m opfoundry_amd.build)")
    bind_torch_hip_runtime()
    lib = ctypes.CDLL(ISSUE_PROBE_LIB_PATH)
    lib.dsa_issue_probe.restype = ctypes.c_int
    lib.dsa_issue_probe.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    return lib


def test_rejects_bad_arguments():
    lib = probe()
    p = ctypes.c_void_p(16)          # never dereferenced: every call below fails its checks
    for mode, iters, out in ((-1, 10, p), (9, 10, p), (0, 0, p), (0, -3, p), (0, 10, None)):
        assert lib.dsa_issue_probe(mode, iters, out, None) == -2, (mode, iters, out)


@pytest.mark.gpu
def test_every_mode_runs():
    import torch
    lib = probe()
    out = torch.empty(256 * 256, dtype=torch.float32, device="cuda:0")
    st = torch.cuda.current_stream().cuda_stream
    for mode in range(9):
        print(f"[case] issue probe mode {mode}", flush=True)
        out.fill_(12345.0)
        assert lib.dsa_issue_probe(mode, 8, out.data_ptr(), st) == 0
        torch.cuda.synchronize()
        # every thread wrote its result over the sentinel
        assert int((out == 12345.0).sum()) == 0
