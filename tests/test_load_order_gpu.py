"""Loading libdsa_mla.so before torch is imported: the loader binds torch's HIP runtime
first (opfoundry_amd.abi.bind_torch_hip_runtime), so a decode on torch tensors still runs.
Without that, the library's libamdhip64.so.7 dependency resolved to /opt/rocm's runtime,
torch then loaded its own, and the decode returned DSA_ERR_HIP.

Runs in a fresh child process, since the parent has imported torch already."""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r"""
import sys
sys.path[:0] = [ROOT, ROOT + "/tests"]
assert "torch" not in sys.modules
from opfoundry_amd.abi import load_library
load_library()
import numpy as np
import torch
from _cases import assert_parity, paged_case
from opfoundry_amd import dsa
dev = torch.device("cuda:0")
c = paged_case(seed=5, B=2, s_q=1, seq_len=1024, topk=256)
t16 = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(dev)
out, lse = dsa.mla_decode(t16(c.q), t16(c.kv), torch.from_numpy(c.indices).to(dev), c.sm_scale,
                          seq_lens=torch.from_numpy(c.seq_lens).to(dev),
                          block_table=torch.from_numpy(c.block_table).to(dev),
                          block_size=c.block_size, num_splits=2)
torch.cuda.synchronize()
o_ref, l_ref = c.oracle()
assert_parity(out.cpu().view(torch.int16).numpy().view(np.uint16), lse.cpu().numpy(), o_ref, l_ref,
              "library loaded before torch")
print("load-order decode ok", flush=True)
"""


def test_library_loaded_before_torch():
    print("[case] child process: load_library() before import torch, then a decode", flush=True)
    res = subprocess.run([sys.executable, "-c", CHILD.replace("ROOT", repr(ROOT))],
                         capture_output=True, text=True, timeout=100)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-2000:]
    assert "load-order decode ok" in res.stdout
