"""GPU check of dsa_mla_decode_noalloc, the entry point that allocates nothing: its split
partials live in the library's per-device scratch instead of a caller workspace.  Called
through the C ABI (ctypes), it must give exactly dsa_mla_decode's bits on the same
arguments, on two calls in a row (the second with a smaller input, so stale scratch
contents from the first call would show), and run unsplit calls without the scratch."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from _cases import paged_case
from opfoundry_amd import abi, dsa

pytestmark = pytest.mark.gpu


def t16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)


def kv_tensor(kv, dev):
    return t16(kv, dev) if kv.dtype == np.uint16 else torch.from_numpy(kv).to(dev)


def both(case, dev, num_splits):
    """(reference entry with a workspace, no-allocation entry) outputs on the same case."""
    lib = abi.load_library()
    q, kv = t16(case.q, dev), kv_tensor(case.kv, dev)
    idx = torch.from_numpy(case.indices).to(dev)
    sl = torch.from_numpy(case.seq_lens).to(dev)
    bt = torch.from_numpy(case.block_table).to(dev)
    res = []
    for noalloc in (False, True):
        B, s_q, H = case.q.shape[:3]
        out = torch.full((B, s_q, H, 512), float("nan"), dtype=torch.bfloat16, device=dev)
        lse = torch.full((B, s_q, H), float("nan"), dtype=torch.float32, device=dev)
        a = dsa.make_decode_args(q, kv, idx, case.sm_scale, out, lse, seq_lens=sl, block_table=bt,
                                 block_size=case.block_size, causal=case.causal, num_splits=num_splits)
        stream = torch.cuda.current_stream().cuda_stream
        if noalloc:
            rc = lib.dsa_mla_decode_noalloc(ctypes.byref(a), ctypes.c_void_p(stream))
        else:
            ws_bytes = dsa.decode_workspace_size(a)
            ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
            rc = lib.dsa_mla_decode(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), ws_bytes,
                                    ctypes.c_void_p(stream))
        assert rc == 0, abi.ERRORS.get(rc, rc)
        torch.cuda.synchronize()
        res.append((out.cpu().view(torch.int16).numpy(), lse.cpu().numpy()))
    return res


@pytest.mark.parametrize("fp8", [False, True])
def test_noalloc_matches_workspace_entry(dev, fp8):
    # first call: 4 tokens x 8 splits (8.4 MB of partials); second: smaller, 2 x 3 splits
    big = paged_case(seed=71 + fp8, B=4, s_q=1, seq_len=8192, topk=2048, fp8=fp8, varlen=True)
    small = paged_case(seed=73 + fp8, B=2, s_q=1, seq_len=1024, topk=300, fp8=fp8)
    for case, ns in ((big, 8), (small, 3), (small, 1)):
        print(f"[case] noalloc fp8={fp8} shape={case.shape} splits={ns}", flush=True)
        (o_ws, l_ws), (o_na, l_na) = both(case, dev, ns)
        assert np.array_equal(o_ws, o_na), f"O differs at {(o_ws != o_na).sum()} elements"
        assert np.array_equal(l_ws, l_na, equal_nan=True)
        assert not np.isnan(l_na).all()


def test_noalloc_scratch_limit(dev):
    """A call whose partials exceed the scratch is refused before any launch; the outputs
    are left untouched."""
    c = paged_case(seed=75, B=2, s_q=1, seq_len=4096, topk=2048)
    q, kv = t16(c.q, dev), kv_tensor(c.kv, dev)
    out = torch.zeros((2, 1, 128, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.zeros((2, 1, 128), dtype=torch.float32, device=dev)
    a = dsa.make_decode_args(q, kv, torch.from_numpy(c.indices).to(dev), c.sm_scale, out, lse,
                             seq_lens=torch.from_numpy(c.seq_lens).to(dev),
                             block_table=torch.from_numpy(c.block_table).to(dev), block_size=64,
                             num_splits=64)
    assert abi.load_library().dsa_mla_decode_noalloc(ctypes.byref(a), None) == -9
    torch.cuda.synchronize()
    assert (lse == 0).all() and (out == 0).all()
