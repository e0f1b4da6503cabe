"""Seeded sweep of decode shapes on the GPU against the CPU oracle.

Each case draws, from its seed:
- batch 1..5 and MTP length 1..2;
- sequence lengths up to 6000, varlen or fixed;
- top-k 1..2048, with -1 padding to a wider index tensor (at most 2048 wide);
- block size 1, 16 or 64;
- causal or not;
- bf16 or fp8 (656-B) rows;
- a split count of 0 (planned), 1, 2, 4 or 8.

It covers list lengths around tile boundaries (1, 31, 32, 33, ... rows), the
pipelined bf16 loop's one-, two- and many-tile paths, and the split / combine
path.  The bar is that of every parity test: bf16 O max-abs <= 2e-2, LSE
within 1e-3 * (1 + |LSE|).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from _cases import assert_parity, paged_case
from opfoundry_amd import dsa

pytestmark = pytest.mark.gpu


def t16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)


def draw(seed: int) -> dict:
    rng = np.random.default_rng(1000 + seed)
    edge = [1, 2, 31, 32, 33, 63, 64, 65, 2047, 2048]
    topk = int(rng.choice(edge)) if rng.random() < 0.5 else int(rng.integers(1, 2049))
    seq_len = int(rng.integers(max(1, topk // 2), 6001))
    return dict(seed=seed, B=int(rng.integers(1, 6)), s_q=int(rng.integers(1, 3)), seq_len=seq_len,
                block_size=int(rng.choice([1, 16, 64])), topk=topk, fp8=bool(rng.random() < 0.5),
                causal=bool(rng.random() < 0.5), varlen=bool(rng.random() < 0.5),
                pad=int(rng.integers(0, 64)), splits=int(rng.choice([0, 1, 2, 4, 8])))


@pytest.mark.parametrize("seed", range(16))
def test_decode_sweep(dev, seed):
    p = draw(seed)
    print(f"[case] sweep {p}", flush=True)
    c = paged_case(seed=p["seed"], B=p["B"], s_q=p["s_q"], seq_len=p["seq_len"], block_size=p["block_size"],
                   topk=p["topk"], fp8=p["fp8"], causal=p["causal"], varlen=p["varlen"],
                   pad_to=min(p["topk"] + p["pad"], 2048))   # one workgroup takes <= 2048 entries
    o_ref, l_ref = c.oracle()
    kv = t16(c.kv, dev) if c.kv.dtype == np.uint16 else torch.from_numpy(c.kv).to(dev)
    out, lse = dsa.mla_decode(t16(c.q, dev), kv, torch.from_numpy(c.indices).to(dev), c.sm_scale,
                              seq_lens=torch.from_numpy(c.seq_lens).to(dev),
                              block_table=torch.from_numpy(c.block_table).to(dev), block_size=c.block_size,
                              causal=c.causal, num_splits=p["splits"])
    torch.cuda.synchronize()
    o = out.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    e = assert_parity(o, lse.cpu().numpy(), o_ref, l_ref, f"sweep seed={seed}")
    print(f"[case] max|dO|={e[0]:.3e} max rel dLSE={e[1]:.3e}", flush=True)
