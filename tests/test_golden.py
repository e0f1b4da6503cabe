"""Golden fixtures (tests/golden/*.npz): regenerated inputs match the recorded
digest, the CPU oracle reproduces the recorded outputs bit for bit, and (GPU)
the HIP decode path matches them within the parity bar (bf16 O max-abs
<= 2e-2, LSE within 1e-3 * (1 + |LSE|))."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden  # noqa: E402

from _cases import assert_parity  # noqa: E402


@pytest.fixture(scope="module", params=sorted(make_golden.CASES))
def golden(request):
    name = request.param
    d = make_golden.CASES[name]()
    return name, d, make_golden.load(name)


def test_inputs_regenerate(golden):
    name, d, g = golden
    assert make_golden.input_digest(d) == str(g["input_sha256"]), name


def test_oracle_reproduces_fixture(golden):
    name, d, g = golden
    o, lse = make_golden.run_oracle(d)
    assert np.array_equal(o, g["o"]), name
    assert np.array_equal(lse, g["lse"]), name


def test_generator_statistics():
    """The counter-based N(0,1) generator has the right moments and the distinct sampler
    returns distinct in-range positions."""
    z = make_golden.normal(1, 1, 200000).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    s = make_golden.distinct(5, 7, 1000, 300)
    assert len(np.unique(s)) == 300 and s.min() >= 0 and s.max() < 1000


@pytest.mark.gpu
def test_hip_matches_fixture(golden, dev):
    import torch
    from opfoundry_amd import dsa
    name, d, g = golden
    print(f"[case] golden {name}", flush=True)
    t16 = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)  # noqa: E731
    kv = t16(d["kv"]) if d["kv"].dtype == np.uint16 else torch.from_numpy(d["kv"]).to(dev)
    bt = None if d["block_table"] is None else torch.from_numpy(d["block_table"]).to(dev)
    for splits in (1, 0, 4):
        out, lse = dsa.mla_decode(t16(d["q"]), kv, torch.from_numpy(d["indices"]).to(dev),
                                  float(g["sm_scale"]), seq_lens=torch.from_numpy(d["seq_lens"]).to(dev),
                                  block_table=bt, block_size=d["block_size"], causal=d["causal"],
                                  num_splits=splits, kv_batch_stride=d["kv_batch_stride"])
        torch.cuda.synchronize()
        o = out.cpu().view(torch.int16).numpy().view(np.uint16)
        e = assert_parity(o, lse.cpu().numpy(), g["o"], g["lse"], f"{name} splits={splits}")
        print(f"[case] golden {name} splits={splits}: max|dO|={e[0]:.3e} rel dLSE={e[1]:.3e}",
              flush=True)
