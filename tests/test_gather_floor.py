"""The gather-floor probe (libdsa_gather_floor.so, bench.py --gather-floor): argument checks
on the CPU, and on the GPU that every gathered word lands (per-token word sums against
numpy's) for both row widths and every slot count it accepts."""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from opfoundry_amd.abi import bind_torch_hip_runtime
from opfoundry_amd.build import PROBE_LIB_PATH


def probe():
    if not os.path.exists(PROBE_LIB_PATH):
        pytest.fail(f"{PROBE_LIB_PATH} not built (python -m opfoundry_amd.build)")
    bind_torch_hip_runtime()
    lib = ctypes.CDLL(PROBE_LIB_PATH)
    lib.dsa_gather_floor.restype = ctypes.c_int
    lib.dsa_gather_floor.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    return lib


def test_rejects_bad_arguments():
    lib = probe()
    p = ctypes.c_void_p(16)          # never dereferenced: every call below fails its checks
    for ntok, nrows, rb, slots in ((1, 48, 656, 3), (1, 4096, 656, 3), (0, 32, 656, 3),
                                   (1, 32, 640, 3), (1, 32, 656, 5), (1, 32, 1152, 4)):
        assert lib.dsa_gather_floor(p, p, ntok, nrows, rb, slots, p, None) == -1
    assert lib.dsa_gather_floor(None, p, 1, 32, 656, 3, p, None) == -1


@pytest.mark.gpu
@pytest.mark.parametrize("row_bytes,slots", [(656, 2), (656, 3), (656, 4), (1152, 2), (1152, 3)])
def test_sums_match(dev, row_bytes, slots):
    import torch
    lib = probe()
    rng = np.random.default_rng(row_bytes + slots)
    nkv, ntok, nrows = 5000, 12, 2048 if slots == 3 else 320
    kv = rng.integers(0, 256, (nkv, row_bytes), dtype=np.uint8)
    rows = rng.integers(0, nkv, (ntok, nrows)).astype(np.int32)
    words = kv.view(np.uint32).astype(np.uint64)
    want = (words.sum(1)[rows].sum(1) & 0xFFFFFFFF).astype(np.uint32)
    kv_t, rows_t = torch.from_numpy(kv).to(dev), torch.from_numpy(rows).to(dev)
    sums = torch.zeros(ntok, dtype=torch.int32, device=dev)
    print(f"[case] gather floor: row_bytes {row_bytes}, slots {slots}, {ntok} x {nrows} rows", flush=True)
    rc = lib.dsa_gather_floor(kv_t.data_ptr(), rows_t.data_ptr(), ntok, nrows, row_bytes, slots,
                              sums.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert np.array_equal(sums.cpu().numpy().view(np.uint32), want)
